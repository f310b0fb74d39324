"""CPU oracle for the decode token path (sampler + CDB exit gate).

TEST INFRASTRUCTURE ONLY.  This package is the checker: ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product package never does.

The arithmetic lives in ``oracle.c`` (plain C, float64), compiled with gcc into
``liboracle.so`` next to this file.  The functions here only marshal numpy
arrays across ctypes.  Reference citations for every rule are in ``oracle.c``.

Arrays holding bf16 or fp16 data are passed as ``numpy.uint16`` bit patterns;
fp32 data as ``numpy.float32``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
SRC_PATH = os.path.join(HERE, "oracle.c")

F32, BF16, F16 = 0, 1, 2
# Rows whose decision lies within this relative distance of a boundary are
# reported as ambiguous (the CDF-versus-uniform rule and the top-p mass rule).
AMB_TOL = 1e-6

_lib = None


def build(force: bool = True) -> str:
    """Compile oracle.c with gcc (OpenMP for the row loop, no FP contraction)."""
    if not force and os.path.exists(LIB_PATH):
        return LIB_PATH
    cmd = [
        "gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC",
        SRC_PATH, "-o", LIB_PATH + ".tmp", "-lm",
    ]
    subprocess.run(cmd, check=True)
    os.replace(LIB_PATH + ".tmp", LIB_PATH)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I32, F, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_double
        L.orc_argmax.argtypes = [P, ctypes.c_int, I64, I64, I64, P, ctypes.c_int]
        L.orc_sample.argtypes = [P, ctypes.c_int, I64, I64, I64, P, P, P, P, P, P, D, ctypes.c_int, P]
        L.orc_exit_gate.argtypes = [P, ctypes.c_int, I64, I64, I64, P, P, P, P, I32, F, I32, I32,
                                    I32, P, P, P, P, P, P, P]
        L.orc_cumulative_exit_probability.argtypes = [P, P, I64, P]
        L.orc_rel_change.argtypes = [P, P, ctypes.c_int, I64, I64, I64, I64, F, D, P, P, P]
        for fn in ("orc_argmax", "orc_sample", "orc_exit_gate", "orc_cumulative_exit_probability",
                   "orc_rel_change"):
            getattr(L, fn).restype = None
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dtype_code(a: np.ndarray, dtype: int | None) -> int:
    if dtype is not None:
        return dtype
    if a.dtype == np.float32:
        return F32
    raise ValueError("uint16 arrays need an explicit dtype (BF16 or F16)")


def _rows(a: np.ndarray):
    assert a.ndim == 2 and a.strides[1] == a.itemsize, "rows must be contiguous"
    return a.shape[0], a.shape[1], a.strides[0] // a.itemsize


def argmax(logits: np.ndarray, dtype: int | None = None, nthreads: int = 0) -> np.ndarray:
    """torch.argmax(logits, dim=-1).to(int32) restated (sample.py:110-111)."""
    B, V, ld = _rows(logits)
    out = np.empty(B, np.int32)
    lib().orc_argmax(_ptr(logits), _dtype_code(logits, dtype), B, V, ld, _ptr(out), nthreads)
    return out


def sample(logits: np.ndarray, temperatures, top_k, top_p, uniforms, dtype: int | None = None,
           tol: float = AMB_TOL, nthreads: int = 0, with_alt: bool = False):
    """Non-greedy sampling (S2-S5). Returns (ids int32[B], amb uint8[B]), and with
    ``with_alt`` also alt int32[B]: for rows whose top-p mass is ambiguous (amb
    bit 1), the draw from the other kept set a float evaluation can produce
    (amb bit 2: that draw's CDF is itself within tol of u); elsewhere alt = ids.

    ``temperatures is None`` selects the all-greedy branch (argmax), matching
    ``Sampler.sample`` (sample.py:110).  ``top_k``/``top_p``/``uniforms`` may be None.
    """
    B, V, ld = _rows(logits)
    f = lambda a, t: None if a is None else np.ascontiguousarray(a, dtype=t)
    T, K, Pp, U = f(temperatures, np.float32), f(top_k, np.int32), f(top_p, np.float32), f(uniforms, np.float32)
    out = np.empty(B, np.int32)
    amb = np.zeros(B, np.uint8)
    alt = np.empty(B, np.int32)
    lib().orc_sample(_ptr(logits), _dtype_code(logits, dtype), B, V, ld, _ptr(T), _ptr(K), _ptr(Pp),
                     _ptr(U), _ptr(out), _ptr(amb), tol, nthreads, _ptr(alt))
    return (out, amb, alt) if with_alt else (out, amb)


def exit_gate(h: np.ndarray, w: np.ndarray, bias, F_prev, loop_step, tau: float,
              min_loop_steps: int = 1, lookahead: bool = False, max_depth: int = 0,
              dtype: int | None = None):
    """Ouro gate G1-G5 (ouro.py:142-155). Returns a dict of outputs.

    ``loop_step`` is an int (scalar step for all rows) or an int32 array.
    """
    B, H, ld = _rows(h)
    code = _dtype_code(h, dtype)
    w = np.ascontiguousarray(w)
    b = None if bias is None else np.ascontiguousarray(np.atleast_1d(bias), dtype=w.dtype)
    F = None if F_prev is None else np.ascontiguousarray(F_prev, dtype=np.float32)
    if isinstance(loop_step, (int, np.integer)):
        ls_arr, ls_scalar = None, int(loop_step)
    else:
        ls_arr, ls_scalar = np.ascontiguousarray(loop_step, dtype=np.int32), 0
    out = dict(
        F_next=np.empty(B, np.float32), mask=np.empty(B, np.uint8), exit_idx=np.empty(B, np.int32),
        keep_idx=np.empty(B, np.int32), n_exit=np.zeros(1, np.int32), z=np.empty(B, np.float32),
        amb=np.zeros(B, np.uint8),
    )
    lib().orc_exit_gate(_ptr(h), code, B, H, ld, _ptr(w), _ptr(b), _ptr(F), _ptr(ls_arr), ls_scalar,
                        float(tau), int(min_loop_steps), int(bool(lookahead)), int(max_depth),
                        _ptr(out["F_next"]), _ptr(out["mask"]), _ptr(out["exit_idx"]),
                        _ptr(out["keep_idx"]), _ptr(out["n_exit"]), _ptr(out["z"]), _ptr(out["amb"]))
    n = int(out["n_exit"][0])
    out["exit_idx"] = out["exit_idx"][:n]
    out["keep_idx"] = out["keep_idx"][: B - n]
    return out


def cumulative_exit_probability(z: np.ndarray, F_prev: np.ndarray) -> np.ndarray:
    """exit_gates.py:6-15 on given fp32 gate logits."""
    z = np.ascontiguousarray(z, np.float32)
    F = np.ascontiguousarray(F_prev, np.float32)
    out = np.empty_like(F)
    lib().orc_cumulative_exit_probability(_ptr(z), _ptr(F), z.shape[0], _ptr(out))
    return out


def relative_state_change(h: np.ndarray, h_prev: np.ndarray, tau: float, dtype: int | None = None,
                          tol: float = 1e-5):
    """Huginn G6 (huginn.py:184-194). Returns (ratio f32[B], mask u8[B], amb u8[B])."""
    B, H, ld = _rows(h)
    _, _, ldp = _rows(h_prev)
    ratio = np.empty(B, np.float32)
    mask = np.empty(B, np.uint8)
    amb = np.zeros(B, np.uint8)
    lib().orc_rel_change(_ptr(h), _ptr(h_prev), _dtype_code(h, dtype), B, H, ld, ldp, float(tau), tol,
                         _ptr(ratio), _ptr(mask), _ptr(amb))
    return ratio, mask, amb


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of a torch bf16/fp16 tensor (on CPU)."""
    import torch

    t = x.detach().cpu().contiguous()
    return t.view(torch.int16).numpy().view(np.uint16)


class Token:
    """A decode position in flight: identity (request, slot, position), depth and
    an optional replay exit depth (CDBDecodeToken, managers/cdb_scheduler.py:39-60)."""

    __slots__ = ("ident", "slot", "depth", "replay", "live")

    def __init__(self, ident, slot: int, depth: int = 0, replay: int | None = None):
        self.ident, self.slot, self.depth, self.replay, self.live = ident, slot, depth, replay, True

    def advanced(self) -> "Token":
        t = Token(self.ident, self.slot, self.depth + 1, self.replay)
        t.live = self.live
        return t


class CdbRouter:
    """CPU restatement of the CDB scheduler's exit routing for core steps.

    ``core_step`` follows CDBScheduler._run_core (cdb_scheduler.py:232-267):
    the batch's tokens advance one depth, this step's gate decisions become the
    current gate, and the previous gate (lookahead timing) or the current one
    (``disable_lookahead_exit``) is consumed by ``_consume`` (the rules of
    _consume_gate, cdb_scheduler.py:189-229): replay depths replace decisions
    (``token.depth >= replay - delay``), a token leaves when
    ``current.depth >= max_depth or (requested and exit_ready)`` with
    ``exit_ready = disable_lookahead_exit or current.depth > token.depth``, and
    the depth cap routes every remaining core token at ``max_depth``.
    Returns the identities routed to the coda in this step, in routing order.
    """

    def __init__(self, max_depth: int, disable_lookahead_exit: bool):
        self.max_depth = max_depth
        self.direct = disable_lookahead_exit
        self.core: list[Token] = []
        self.pending = None

    def add(self, token: Token) -> None:
        self.core.append(token)

    def cancel(self, ident) -> None:
        for t in self.core:
            if t.ident == ident:
                t.live = False
        self.core = [t for t in self.core if t.ident != ident]

    def _consume(self, gate) -> list:
        if gate is None:
            return []
        tokens, decisions = gate
        current = {t.ident: t for t in self.core}
        decisions = list(decisions)
        for i, t in enumerate(tokens):
            if t.replay is not None:
                decisions[i] = t.depth >= t.replay - (0 if self.direct else 1)
        exited = []
        for t, req in zip(tokens, decisions):
            cur = current.get(t.ident)
            if cur is None or not cur.live:
                continue
            ready = self.direct or cur.depth > t.depth
            if cur.depth >= self.max_depth or (req and ready):
                exited.append(cur)
        ids = {t.ident for t in exited}
        self.core = [t for t in self.core if t.ident not in ids]
        return [t.ident for t in exited]

    def core_step(self, batch_idents: list, decisions: list) -> list:
        """``decisions[i]``: the gate's signal for ``batch_idents[i]`` this step."""
        advanced = {}
        for i, t in enumerate(self.core):
            if t.ident in batch_idents:
                self.core[i] = advanced[t.ident] = t.advanced()
        gate_tokens = [advanced[i] for i in batch_idents]
        current = (gate_tokens, list(decisions))
        if self.direct:
            out = self._consume(current)
        else:
            previous, self.pending = self.pending, current
            out = self._consume(previous)
        capped = [t for t in self.core if t.depth >= self.max_depth]
        self.core = [t for t in self.core if t.depth < self.max_depth]
        return out + [t.ident for t in capped]
