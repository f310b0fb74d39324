"""The fused coda tail: vocabulary projection and token step without an fp32
logits buffer.

Replaces, for the decode step of the reference:
  ParallelLMHead.forward (python/loopsgl/layers/embedding.py:88-111, tp_size 1)
  -> the copy into GraphCaptureBuffer.logits (model_executor/graph.py:34,
     model_executor/cdb_graph.py:80-82)
  -> Sampler.sample (model_executor/sample.py:107-112).

``lm_head`` returns the bf16 logits the reference's F.linear produces (MFMA,
fp32 accumulation).  ``coda_sample`` runs the projection and the token step in
one call: all-greedy batches finish from per-tile row maxima written by the
projection's epilogue (the logits are not read back); sampling batches run the
sampler on the bf16 logits once.
"""
from __future__ import annotations

import torch

from . import _lib
from .sampler import BatchSamplingArgs, _per_row


def _check_operands(hidden: torch.Tensor, weight: torch.Tensor):
    _lib.require_gpu(hidden, "hidden")
    _lib.require_gpu(weight, "weight")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("hidden and weight must be bfloat16 (the model dtype of the LM head)")
    if hidden.dim() != 2 or weight.dim() != 2 or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"hidden [B, H] and weight [V, H] expected, got {tuple(hidden.shape)}, {tuple(weight.shape)}")
    if hidden.device != weight.device:
        raise ValueError("hidden and weight must be on the same device")
    if hidden.stride(1) != 1 or hidden.stride(0) % 8 or hidden.data_ptr() % 16:
        hidden = hidden.contiguous()
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        weight = weight.contiguous()
    return hidden, weight


def lm_head(hidden: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16 logits [B, V] = hidden [B, H] @ weight [V, H]^T (H a multiple of 64)."""
    hidden, weight = _check_operands(hidden, weight)
    B, H = hidden.shape
    V = weight.shape[0]
    if out is None:
        out = torch.empty(B, V, dtype=torch.bfloat16, device=hidden.device)
    elif out.dtype != torch.bfloat16 or out.shape != (B, V) or out.stride(1) != 1:
        raise ValueError(f"out must be bfloat16[{B}, {V}] with unit column stride")
    rc = _lib.load().lsg_lm_head(_lib.ptr(hidden), B, H, hidden.stride(0), _lib.ptr(weight), V, weight.stride(0),
                                 _lib.ptr(out), out.stride(0), _lib.stream_of(hidden))
    _lib.check(rc, "lsg_lm_head")
    return out


def workspace_bytes(B: int, V: int) -> int:
    return int(_lib.load().lsg_lm_head_workspace_bytes(B, V))


def coda_sample(hidden: torch.Tensor, weight: torch.Tensor, args: BatchSamplingArgs,
                workspace: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Projection + token step: int32 ids [B].  ``args.temperatures is None``
    selects argmax for every row; otherwise ``args.uniforms`` is required.
    ``workspace`` (uint8, >= workspace_bytes(B, V)) may be passed in to keep
    the call free of allocations (e.g. under graph capture)."""
    hidden, weight = _check_operands(hidden, weight)
    B, H = hidden.shape
    V = weight.shape[0]
    dev = hidden.device
    T = _per_row(args.temperatures, B, torch.float32, dev, "temperatures")
    K = _per_row(args.top_k, B, torch.int32, dev, "top_k")
    P = _per_row(args.top_p, B, torch.float32, dev, "top_p")
    U = _per_row(args.uniforms, B, torch.float32, dev, "uniforms")
    if T is not None and U is None:
        raise ValueError("non-greedy sampling needs uniforms")
    need = workspace_bytes(B, V)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    elif workspace.dtype != torch.uint8 or workspace.numel() < need or workspace.device != dev:
        raise ValueError(f"workspace must be uint8 with >= {need} elements on {dev}")
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=dev)
    rc = _lib.load().lsg_lm_head_sample(
        _lib.ptr(hidden), B, H, hidden.stride(0), _lib.ptr(weight), V, weight.stride(0),
        _lib.ptr(T), _lib.ptr(K), _lib.ptr(P), _lib.ptr(U),
        _lib.ptr(workspace), workspace.numel(), _lib.ptr(out), _lib.stream_of(hidden))
    _lib.check(rc, "lsg_lm_head_sample")
    return out


def workspace_logits(workspace: torch.Tensor, B: int, V: int) -> torch.Tensor:
    """The bf16 logits coda_sample left in its workspace (a view, row stride V
    rounded up to a multiple of 8)."""
    ld = (V + 7) // 8 * 8
    return workspace[: B * ld * 2].view(torch.bfloat16).view(B, ld)[:, :V]
