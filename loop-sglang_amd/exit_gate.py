"""Continuous Depth Batching exit gates on the HIP kernels of libloopsgl_tok.so.

Drop-ins for the gate half of the decode token path:
  ``cumulative_exit_probability`` / ``relative_state_change``
      python/loopsgl/models/looped/exit_gates.py:6-24
  ``OuroExitGate.init_exit_state`` / ``exit_signal``
      models/looped/ouro.py:107-155 (gate linear, layers/linear.py:32-33)
  ``HuginnExitGate.init_exit_state`` / ``exit_signal``
      models/looped/huginn.py:180-194
plus ``exit_signal_compact``, which also returns the stable compaction of the
exited rows (``exit_idx``, ``keep_idx``, ``n_exit``) that the reference computes
on the host in CDBScheduler._consume_gate (managers/cdb_scheduler.py:215-228).

Contract kept from models/looped/base.py:126-143: the signal is bool[B] on the
states' device, the updated Ouro state keeps its float32 [B] shape, nothing
synchronises with the host (every call is capturable in a HIP graph as long as
its output tensors come from the graph pool).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple

import torch

from . import _lib


def _ls_args(loop_step, B: int, device: torch.device):
    """(per-row int32 tensor or None, scalar step) without any host sync."""
    if isinstance(loop_step, torch.Tensor):
        if loop_step.device != device:
            raise ValueError("loop_step tensor must be on the hidden states' device")
        if loop_step.dim() == 0:
            return loop_step.to(torch.int32).expand(B).contiguous(), 0
        if loop_step.shape != (B,):
            raise ValueError(f"loop_step must be a scalar or shape ({B},)")
        return loop_step.to(torch.int32).contiguous(), 0
    return None, int(loop_step)


def cumulative_exit_probability(
    logits: torch.Tensor, previous_probability: torch.Tensor
) -> torch.Tensor:
    """F' = F + (1 - F) * sigmoid(float(logits)) in float32 (exit_gates.py:6-15)."""
    _lib.require_gpu(logits, "logits")
    if logits.shape != previous_probability.shape:
        raise ValueError("logits and previous_probability must have matching shapes")
    z = logits.contiguous().reshape(-1)
    F = previous_probability.float().contiguous().reshape(-1)
    out = torch.empty_like(F)
    rc = _lib.load().lsg_cumulative_exit_probability(
        _lib.ptr(z), _lib.dtype_code(z), _lib.ptr(F), _lib.ptr(out), z.numel(), _lib.stream_of(z))
    _lib.check(rc, "lsg_cumulative_exit_probability")
    return out.reshape(previous_probability.shape)


class GateResult(NamedTuple):
    signal: torch.Tensor  # bool[B]
    state: torch.Tensor  # Ouro: float32[B] cumulative exit probability; Huginn: hidden
    exit_idx: torch.Tensor  # int32[B]; first n_exit entries valid, ascending
    keep_idx: torch.Tensor  # int32[B]; first B - n_exit entries valid, ascending
    n_exit: torch.Tensor  # int32[1] on the device


class RouteResult(NamedTuple):
    signal: torch.Tensor  # bool[B] this step's gate signal (ouro.py:154)
    route: torch.Tensor  # bool[B] rows routed to the coda in this step
    state: torch.Tensor  # float32 exit state (or the state pool when slots are given)
    exit_idx: torch.Tensor  # int32[B]; first n_exit entries valid, ascending
    keep_idx: torch.Tensor  # int32[B]; first B - n_exit entries valid, ascending
    n_exit: torch.Tensor  # int32[1] on the device


class _Workspace:
    """Device workspace of the exit compaction, sized for ``max_batch`` rows and
    zero-filled once when the gate is built on a device, so that no call
    allocates (the first call may be inside a graph capture).  The library keeps
    a call serial number in it, so one workspace serves one sequence of calls."""

    def __init__(self, op: int, max_batch: int, device: torch.device | None):
        if max_batch < 1:
            raise ValueError("max_batch must be positive")
        self.op = op
        self.max_batch = int(max_batch)
        self.buf: torch.Tensor | None = None
        if device is not None and torch.device(device).type == "cuda":
            self._allocate(torch.device(device))

    def _allocate(self, device: torch.device) -> None:
        need = int(_lib.load().lsg_workspace_bytes(self.op, self.max_batch))
        self.buf = torch.zeros(need, dtype=torch.uint8, device=device)

    def get(self, B: int, device: torch.device) -> torch.Tensor:
        if B > self.max_batch:
            raise ValueError(f"batch of {B} rows exceeds the gate's max_batch={self.max_batch}")
        if self.buf is None:
            self._allocate(device)  # a gate built without a device: first call allocates
        elif self.buf.device != device:
            raise ValueError(f"gate workspace lives on {self.buf.device}, hidden states on {device}")
        return self.buf


def relative_state_change(
    current: torch.Tensor, previous: torch.Tensor, *, eps: float = 1e-9
) -> torch.Tensor:
    """||current - previous||_2 / max(||current||_2, eps) per row in float32 (exit_gates.py:18-24)."""
    ratio, _ = _rel_change(current, previous, float("nan"), eps, None)
    return ratio


def _rel_change(current, previous, tau, eps, ws: _Workspace | None):
    _lib.require_gpu(current, "current")
    if current.shape != previous.shape or current.dim() != 2:
        raise ValueError("current and previous must both be [B, H]")
    h = current if current.stride(1) == 1 else current.contiguous()
    hp = previous if previous.stride(1) == 1 else previous.contiguous()
    if hp.dtype != h.dtype:
        hp = hp.to(h.dtype)
    B, H = h.shape
    dev = h.device
    ratio = torch.empty(B, dtype=torch.float32, device=dev)
    mask = torch.empty(B, dtype=torch.bool, device=dev)
    compact = None
    wsb, wsn = None, 0
    if ws is not None:
        compact = (torch.empty(B, dtype=torch.int32, device=dev), torch.empty(B, dtype=torch.int32, device=dev),
                   torch.empty(1, dtype=torch.int32, device=dev))
        wsb = ws.get(B, dev)
        wsn = wsb.numel()
    rc = _lib.load().lsg_relative_state_change(
        _lib.ptr(h), _lib.ptr(hp), _lib.dtype_code(h), B, H, h.stride(0), hp.stride(0), float(tau),
        float(eps), _lib.ptr(ratio), _lib.ptr(mask),
        _lib.ptr(compact[0]) if compact else None, _lib.ptr(compact[1]) if compact else None,
        _lib.ptr(compact[2]) if compact else None, _lib.ptr(wsb), wsn, _lib.stream_of(h))
    _lib.check(rc, "lsg_relative_state_change")
    if compact is not None:
        return ratio, (mask, *compact)
    return ratio, mask


def ouro_exit_signal(hidden_states: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                     exit_state: torch.Tensor, loop_step: int | torch.Tensor, *, exit_threshold: float,
                     min_loop_steps: int = 1,
                     exit_gate_type: str = "early_exit") -> tuple[torch.Tensor, torch.Tensor]:
    """OuroModel.exit_signal (ouro.py:142-155) on given gate parameters: one
    launch computes z = round(h . w + b), the cumulative exit probability and
    the signal.  Allocates only the two outputs (mask bool[B], state f32[B]);
    ``weight`` ([1, H] or [H]) and ``bias`` ([1] or None) must already be in the
    hidden states' dtype and on their device."""
    _lib.require_gpu(hidden_states, "hidden_states")
    h = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
    if h.dim() != 2:
        raise ValueError("hidden_states must be [B, H]")
    B, H = h.shape
    dev = h.device
    w = weight.reshape(-1)
    if w.numel() != H or w.dtype != h.dtype or w.device != dev or not w.is_contiguous():
        raise ValueError(f"gate weight must be {H} contiguous {h.dtype} values on {dev}")
    b = None
    if bias is not None:
        b = bias.reshape(-1)
        if b.numel() < 1 or b.dtype != h.dtype or b.device != dev:
            raise ValueError(f"gate bias must be a {h.dtype} value on {dev}")
    F_prev = None
    if exit_state is not None:
        if exit_state.dtype != torch.float32 or exit_state.device != dev or exit_state.shape != (B,):
            raise ValueError("exit_state must be float32[B] on the hidden states' device")
        F_prev = exit_state.contiguous()
    ls_tensor, ls_scalar = _ls_args(loop_step, B, dev)
    mask = torch.empty(B, dtype=torch.bool, device=dev)
    state = torch.empty(B, dtype=torch.float32, device=dev)
    rc = _lib.load().lsg_exit_gate(
        _lib.ptr(h), _lib.dtype_code(h), B, H, h.stride(0), _lib.ptr(w), _lib.ptr(b), _lib.ptr(F_prev),
        _lib.ptr(state), None, _lib.ptr(ls_tensor), ls_scalar, float(exit_threshold), int(min_loop_steps),
        int(exit_gate_type == "lookahead"), 0, _lib.ptr(mask), None, None, None, None, None, 0,
        _lib.stream_of(h))
    _lib.check(rc, "lsg_exit_gate")
    return mask, state


@dataclass
class OuroExitGate:
    """Ouro's early-exit gate (ouro.py:63-72,84-87,107-155).

    ``weight``: [1, H] or [H] in the model dtype; ``bias``: [1] or None.
    """

    weight: torch.Tensor
    bias: torch.Tensor | None
    exit_threshold: float
    min_loop_steps: int = 1
    exit_gate_type: str = "early_exit"
    loop_steps: int | None = None
    max_batch: int = 65536

    def __post_init__(self) -> None:
        if not 0 < self.exit_threshold <= 1:
            raise ValueError("Ouro exit_threshold must be in (0, 1]")
        upper = self.loop_steps if self.loop_steps is not None else self.min_loop_steps
        if (
            isinstance(self.min_loop_steps, bool)
            or not isinstance(self.min_loop_steps, int)
            or not 1 <= self.min_loop_steps <= upper
        ):
            raise ValueError("Ouro min_loop_steps must be an integer in [1, loop_steps]")
        if self.exit_gate_type not in ("early_exit", "lookahead"):
            raise ValueError("Ouro exit_gate_type must be 'early_exit' or 'lookahead'")
        self.weight = self.weight.reshape(-1).contiguous()
        if self.bias is not None:
            self.bias = self.bias.reshape(-1)[:1].to(self.weight.dtype).contiguous()
        dev = self.weight.device if self.weight.is_cuda else None
        self._ws = _Workspace(_lib.OP_EXIT_GATE, self.max_batch, dev)
        self._route_ws = _Workspace(_lib.OP_EXIT_GATE, self.max_batch, dev)

    def cdb_state_spec(self, hidden_size: int, dtype: torch.dtype):
        """Shapes/dtypes of the per-token CDB states (ouro.py:107-111)."""
        return {"hidden": ((hidden_size,), dtype), "exit": ((), torch.float32)}

    def init_exit_state(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """Cumulative exit probability starts at zero in float32 (ouro.py:138-140)."""
        return torch.zeros(hidden_states.shape[0], dtype=torch.float32, device=hidden_states.device)

    def _run(self, hidden_states, exit_state, loop_step, *, compact: bool, slots=None,
             out_state=None, max_depth: int = 0, z_out=None, routing=None):
        _lib.require_gpu(hidden_states, "hidden_states")
        h = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
        if h.dim() != 2:
            raise ValueError("hidden_states must be [B, H]")
        B, H = h.shape
        dev = h.device
        if self.weight.numel() != H:
            raise ValueError(f"gate weight has {self.weight.numel()} inputs, hidden size is {H}")
        w = self.weight if self.weight.dtype == h.dtype else self.weight.to(h.dtype)
        b = None if self.bias is None else (self.bias if self.bias.dtype == h.dtype else self.bias.to(h.dtype))
        if w.device != dev:
            raise ValueError("gate weight must be on the hidden states' device")
        F_prev = None
        if exit_state is not None:
            if exit_state.dtype != torch.float32 or exit_state.device != dev:
                raise ValueError("exit_state must be float32 on the hidden states' device")
            F_prev = exit_state.contiguous()
        if slots is not None:
            if slots.dtype != torch.int32 or slots.shape != (B,):
                raise ValueError("slots must be int32[B]")
            if out_state is None:
                raise ValueError("slots need out_state (the state pool to update)")
        if out_state is None:
            out_state = torch.empty(B, dtype=torch.float32, device=dev)
        ls_tensor, ls_scalar = _ls_args(loop_step, B, dev)
        mask = torch.empty(B, dtype=torch.bool, device=dev)
        exit_idx = keep_idx = n_exit = None
        wsb, wsn = None, 0
        if compact:
            exit_idx = torch.empty(B, dtype=torch.int32, device=dev)
            keep_idx = torch.empty(B, dtype=torch.int32, device=dev)
            n_exit = torch.empty(1, dtype=torch.int32, device=dev)
            wsb = (self._route_ws if routing is not None else self._ws).get(B, dev)
            wsn = wsb.numel()
        args = (_lib.ptr(h), _lib.dtype_code(h), B, H, h.stride(0), _lib.ptr(w), _lib.ptr(b),
                _lib.ptr(F_prev), _lib.ptr(out_state), _lib.ptr(slots), _lib.ptr(ls_tensor), ls_scalar,
                float(self.exit_threshold), int(self.min_loop_steps),
                int(self.exit_gate_type == "lookahead"), int(max_depth))
        if routing is None:
            rc = _lib.load().lsg_exit_gate(
                *args, _lib.ptr(mask), _lib.ptr(exit_idx), _lib.ptr(keep_idx), _lib.ptr(n_exit),
                _lib.ptr(z_out), _lib.ptr(wsb), wsn, _lib.stream_of(h))
            _lib.check(rc, "lsg_exit_gate")
            return mask, out_state, exit_idx, keep_idx, n_exit
        direct, pending, replay = routing
        route = torch.empty(B, dtype=torch.bool, device=dev)
        rc = _lib.load().lsg_exit_gate_route(
            *args, int(bool(direct)), _lib.ptr(pending), _lib.ptr(replay), _lib.ptr(mask), _lib.ptr(route),
            _lib.ptr(exit_idx), _lib.ptr(keep_idx), _lib.ptr(n_exit), _lib.ptr(z_out), _lib.ptr(wsb), wsn,
            _lib.stream_of(h))
        _lib.check(rc, "lsg_exit_gate_route")
        return mask, route, out_state, exit_idx, keep_idx, n_exit

    def exit_signal(self, hidden_states: torch.Tensor, exit_state: torch.Tensor,
                    loop_step: int | torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(exit requested bool[B], updated cumulative exit probability f32[B])
        (ouro.py:142-155); ``loop_step`` is the zero-based step just executed."""
        return ouro_exit_signal(hidden_states, self.weight, self.bias, exit_state, loop_step,
                                exit_threshold=self.exit_threshold, min_loop_steps=self.min_loop_steps,
                                exit_gate_type=self.exit_gate_type)

    def exit_signal_compact(self, hidden_states: torch.Tensor, exit_state: torch.Tensor | None,
                            loop_step: int | torch.Tensor, *, slots: torch.Tensor | None = None,
                            state_pool: torch.Tensor | None = None, max_depth: int = 0,
                            z_out: torch.Tensor | None = None) -> GateResult:
        """exit_signal plus the on-device stable exit compaction.

        With ``slots`` the exit state is read from and written back to
        ``state_pool[slots]`` in place (cdb_model_runner.py:94-109); ``max_depth``
        > 0 also exits rows whose depth reaches it (cdb_scheduler.py:262-266).
        """
        if slots is not None:
            if state_pool is None:
                raise ValueError("slots need state_pool")
            exit_state = state_pool
        mask, state, exit_idx, keep_idx, n_exit = self._run(
            hidden_states, exit_state, loop_step, compact=True, slots=slots,
            out_state=state_pool if slots is not None else None, max_depth=max_depth, z_out=z_out)
        return GateResult(mask, state, exit_idx, keep_idx, n_exit)

    def init_pending_pool(self, n_slots: int, device: torch.device | None = None) -> torch.Tensor:
        """Pending-gate pool of ``exit_route``: one opaque int64 per state slot, 0 = none."""
        return torch.zeros(n_slots, dtype=torch.int64, device=device or self.weight.device)

    def exit_route(self, hidden_states: torch.Tensor, exit_state: torch.Tensor | None,
                   loop_step: int | torch.Tensor, *, pending: torch.Tensor | None,
                   disable_lookahead_exit: bool = False, slots: torch.Tensor | None = None,
                   state_pool: torch.Tensor | None = None, max_depth: int = 0,
                   replay_depth: torch.Tensor | None = None,
                   z_out: torch.Tensor | None = None) -> RouteResult:
        """exit_signal plus the scheduler's routing of one core step, on the device.

        The default timing follows CDBScheduler._run_core / _consume_gate
        (cdb_scheduler.py:207-222,254-266): the request recorded for a row's state
        slot (``pending``, see ``init_pending_pool``) by the previous call routes
        the row now, and this step's request is recorded for the next call.  With
        ``disable_lookahead_exit`` a row's own request routes it at once.
        ``replay_depth`` (int32[B], > 0 where set) replaces the request by
        ``depth >= replay - delay``; ``max_depth`` > 0 routes rows whose depth
        (``loop_step + 1``) reaches it.  Successive calls on one gate are
        successive core steps of one scheduler: the pending pool is tagged with
        the gate's call count.  A caller that puts a new token into a slot other
        than by routing the old one out (cancellation) zeroes ``pending[slot]``.
        """
        if slots is not None:
            if state_pool is None:
                raise ValueError("slots need state_pool")
            exit_state = state_pool
        if pending is not None and (pending.dtype != torch.int64 or pending.device != hidden_states.device
                                    or not pending.is_contiguous()):
            raise ValueError("pending must be a contiguous int64 pool on the hidden states' device")
        if not disable_lookahead_exit and pending is None:
            raise ValueError("lookahead routing needs the pending-gate pool")
        n = hidden_states.shape[0]
        if replay_depth is not None:
            if replay_depth.dtype != torch.int32 or replay_depth.shape != (n,):
                raise ValueError("replay_depth must be int32[B]")
            replay_depth = replay_depth.contiguous()
        mask, route, state, exit_idx, keep_idx, n_exit = self._run(
            hidden_states, exit_state, loop_step, compact=True, slots=slots,
            out_state=state_pool if slots is not None else None, max_depth=max_depth, z_out=z_out,
            routing=(disable_lookahead_exit, pending, replay_depth))
        return RouteResult(mask, route, state, exit_idx, keep_idx, n_exit)


@dataclass
class HuginnExitGate:
    """Huginn's relative-state-change gate (huginn.py:96-98,180-194)."""

    exit_threshold: float
    eps: float = 1e-9
    max_batch: int = 65536
    device: torch.device | str | None = None  # where the compaction workspace is built

    def __post_init__(self) -> None:
        if not (self.exit_threshold == self.exit_threshold) or self.exit_threshold < 0 or \
                self.exit_threshold == float("inf"):
            raise ValueError("Huginn exit_threshold must be finite and nonnegative")
        self._ws = _Workspace(_lib.OP_REL_CHANGE, self.max_batch, self.device)

    def init_exit_state(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """The initial recurrent state is the first comparison's previous state."""
        return hidden_states

    def exit_signal(self, hidden_states: torch.Tensor, exit_state: torch.Tensor,
                    loop_step: int | torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(relative change < threshold, hidden_states) -- equality does not exit."""
        _, mask = _rel_change(hidden_states, exit_state, self.exit_threshold, self.eps, None)
        return mask, hidden_states

    def exit_signal_compact(self, hidden_states: torch.Tensor, exit_state: torch.Tensor,
                            loop_step: int | torch.Tensor) -> GateResult:
        _, (mask, exit_idx, keep_idx, n_exit) = _rel_change(
            hidden_states, exit_state, self.exit_threshold, self.eps, self._ws)
        return GateResult(mask, hidden_states, exit_idx, keep_idx, n_exit)
