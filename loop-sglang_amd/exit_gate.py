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


class _Workspace:
    """Zero-filled device workspace for the in-kernel compaction (one per device)."""

    def __init__(self, op: int):
        self.op = op
        self.buf: dict[torch.device, torch.Tensor] = {}

    def get(self, B: int, device: torch.device) -> torch.Tensor:
        need = int(_lib.load().lsg_workspace_bytes(self.op, B))
        buf = self.buf.get(device)
        if buf is None or buf.numel() < need:
            # allocated once and left zero-filled by every call
            buf = torch.zeros(max(need, 4096), dtype=torch.uint8, device=device)
            self.buf[device] = buf
        return buf


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
        self._ws = _Workspace(_lib.OP_EXIT_GATE)

    def cdb_state_spec(self, hidden_size: int, dtype: torch.dtype):
        """Shapes/dtypes of the per-token CDB states (ouro.py:107-111)."""
        return {"hidden": ((hidden_size,), dtype), "exit": ((), torch.float32)}

    def init_exit_state(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """Cumulative exit probability starts at zero in float32 (ouro.py:138-140)."""
        return torch.zeros(hidden_states.shape[0], dtype=torch.float32, device=hidden_states.device)

    def _run(self, hidden_states, exit_state, loop_step, *, compact: bool, slots=None,
             out_state=None, max_depth: int = 0, z_out=None):
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
            wsb = self._ws.get(B, dev)
            wsn = wsb.numel()
        rc = _lib.load().lsg_exit_gate(
            _lib.ptr(h), _lib.dtype_code(h), B, H, h.stride(0), _lib.ptr(w), _lib.ptr(b),
            _lib.ptr(F_prev), _lib.ptr(out_state), _lib.ptr(slots), _lib.ptr(ls_tensor), ls_scalar,
            float(self.exit_threshold), int(self.min_loop_steps),
            int(self.exit_gate_type == "lookahead"), int(max_depth), _lib.ptr(mask),
            _lib.ptr(exit_idx), _lib.ptr(keep_idx), _lib.ptr(n_exit), _lib.ptr(z_out),
            _lib.ptr(wsb), wsn, _lib.stream_of(h))
        _lib.check(rc, "lsg_exit_gate")
        return mask, out_state, exit_idx, keep_idx, n_exit

    def exit_signal(self, hidden_states: torch.Tensor, exit_state: torch.Tensor,
                    loop_step: int | torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(exit requested bool[B], updated cumulative exit probability f32[B])
        (ouro.py:142-155); ``loop_step`` is the zero-based step just executed."""
        mask, state, *_ = self._run(hidden_states, exit_state, loop_step, compact=False)
        return mask, state

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


@dataclass
class HuginnExitGate:
    """Huginn's relative-state-change gate (huginn.py:96-98,180-194)."""

    exit_threshold: float
    eps: float = 1e-9

    def __post_init__(self) -> None:
        if not (self.exit_threshold == self.exit_threshold) or self.exit_threshold < 0 or \
                self.exit_threshold == float("inf"):
            raise ValueError("Huginn exit_threshold must be finite and nonnegative")
        self._ws = _Workspace(_lib.OP_REL_CHANGE)

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
