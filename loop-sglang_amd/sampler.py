"""Token sampler for the decode step, on the HIP kernels of libloopsgl_tok.so.

Drop-in for python/loopsgl/model_executor/sample.py: the same
``BatchSamplingArgs`` (with ``filter_batch``/``merge_batch``), ``Sampler``
(``prepare``/``sample``), ``make_device_tensor`` and ``sample_impl`` names and
argument meanings.  One deliberate extension: ``BatchSamplingArgs.uniforms``
(float32[B] in [0, 1)), the explicit per-row random draw.  When it is absent,
``Sampler.sample`` draws it from its own generator (seeded like the reference's
``torch.manual_seed(42)``, model_executor/model_runner.py:46), so callers written
for the reference keep working.

Returned ids are int32 (the reference returns int64 for greedy and casts to
int32 in ``ModelRunner._sample_logits``, model_runner.py:279-280).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, List

import torch

from . import _lib

@dataclass
class BatchSamplingArgs:
    """Per-row sampling arguments (sample.py:14-53); ``None`` means "off for every row"."""

    temperatures: torch.Tensor | None
    top_k: torch.Tensor | None = None
    top_p: torch.Tensor | None = None
    uniforms: torch.Tensor | None = None

    def filter_batch(
        self, indices: torch.Tensor, all_greedy: bool, *, need_top_k: bool, need_top_p: bool
    ) -> BatchSamplingArgs:
        """Keep rows ``indices`` (sample.py:20-31); uniforms follow their rows."""
        return BatchSamplingArgs(
            (
                self.temperatures[indices]
                if self.temperatures is not None and not all_greedy
                else None
            ),
            self.top_k[indices] if self.top_k is not None and need_top_k else None,
            self.top_p[indices] if self.top_p is not None and need_top_p else None,
            self.uniforms[indices] if self.uniforms is not None else None,
        )

    def merge_batch(
        self, other: BatchSamplingArgs, size: int, other_size: int, vocab_size: int
    ) -> BatchSamplingArgs:
        """Concatenate two batches, filling absent fields with the neutral
        defaults T=1e-6, k=V, p=1.0 (sample.py:33-53).  Uniforms are kept only
        when both sides carry them (otherwise they are drawn at sample time)."""

        def merge(
            left: torch.Tensor | None, right: torch.Tensor | None, default: int | float
        ) -> torch.Tensor | None:
            if left is None and right is None:
                return None
            template = left if left is not None else right
            assert template is not None
            if left is None:
                left = template.new_full((size,), default)
            if right is None:
                right = template.new_full((other_size,), default)
            return torch.cat([left, right])

        uniforms = (
            torch.cat([self.uniforms, other.uniforms])
            if self.uniforms is not None and other.uniforms is not None
            else None
        )
        return BatchSamplingArgs(
            merge(self.temperatures, other.temperatures, 1e-6),
            merge(self.top_k, other.top_k, vocab_size),
            merge(self.top_p, other.top_p, 1.0),
            uniforms,
        )


def make_device_tensor(data: List, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """Pinned host tensor copied asynchronously to ``device`` (sample.py:56-57)."""
    return torch.tensor(data, dtype=dtype, pin_memory=True).to(device, non_blocking=True)


def _per_row(x: Any, B: int, dtype: torch.dtype, device: torch.device, name: str):
    if x is None:
        return None
    if not isinstance(x, torch.Tensor):
        return torch.full((B,), x, dtype=dtype, device=device)
    if x.dim() == 0:
        return x.to(device=device, dtype=dtype).expand(B).contiguous()
    if x.shape != (B,):
        raise ValueError(f"{name} must have shape ({B},), got {tuple(x.shape)}")
    if x.device != device:
        raise ValueError(f"{name} is on {x.device}, logits on {device}")
    return x.to(dtype).contiguous()


def sample_rows(
    logits: torch.Tensor,
    temperatures: torch.Tensor | None,
    top_k: torch.Tensor | int | None,
    top_p: torch.Tensor | float | None,
    uniforms: torch.Tensor | None,
    *,
    row_idx: torch.Tensor | None = None,
    n_rows: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Run lsg_sample.  ``temperatures is None`` selects argmax for every row.

    ``row_idx`` (int32[B_out]) gathers logits rows (per-row arguments are read
    at the gathered row); ``n_rows`` (int32[1] on the device) limits the rows
    written without a host sync.
    """
    _lib.require_gpu(logits, "logits")
    if logits.dim() != 2:
        raise ValueError(f"logits must be 2-D [B, V], got shape {tuple(logits.shape)}")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    B, V = logits.shape
    dev = logits.device
    T = _per_row(temperatures, B, torch.float32, dev, "temperatures")
    K = _per_row(top_k, B, torch.int32, dev, "top_k")
    P = _per_row(top_p, B, torch.float32, dev, "top_p")
    U = _per_row(uniforms, B, torch.float32, dev, "uniforms")
    if T is not None and U is None:
        raise ValueError("non-greedy sampling needs uniforms")
    if row_idx is not None:
        if row_idx.dtype != torch.int32 or row_idx.dim() != 1 or row_idx.device != dev:
            raise ValueError("row_idx must be int32[B_out] on the logits' device")
        row_idx = row_idx.contiguous()
        B_out = row_idx.shape[0]
    else:
        B_out = B
    if n_rows is not None and (n_rows.dtype != torch.int32 or n_rows.device != dev or n_rows.numel() < 1):
        raise ValueError("n_rows must be an int32 device tensor with one element")
    if out is None:
        out = torch.empty(B_out, dtype=torch.int32, device=dev)
    elif out.dtype != torch.int32 or out.shape != (B_out,) or not out.is_contiguous():
        raise ValueError(f"out must be contiguous int32[{B_out}]")
    L = _lib.load()
    rc = L.lsg_sample(
        _lib.ptr(logits), _lib.dtype_code(logits), B, V, logits.stride(0),
        _lib.ptr(T), _lib.ptr(K), _lib.ptr(P), _lib.ptr(U),
        _lib.ptr(row_idx), B_out, _lib.ptr(n_rows), _lib.ptr(out), _lib.stream_of(logits),
    )
    _lib.check(rc, "lsg_sample")
    return out


def sample_impl(
    logits: torch.Tensor,
    temperatures: torch.Tensor,
    top_k: torch.Tensor | int | None,
    top_p: torch.Tensor | float | None,
    uniforms: torch.Tensor | None = None,
    generator: torch.Generator | None = None,
) -> torch.Tensor:
    """Softmax with temperature, optional top-k then top-p, one draw per row
    (the four flashinfer dispatches of sample.py:60-81 in one kernel)."""
    if uniforms is None:
        uniforms = torch.rand(logits.shape[0], device=logits.device, generator=generator)
    return sample_rows(logits, temperatures, top_k, top_p, uniforms)


@dataclass
class Sampler:
    """sample.py:84-112 on the HIP sampler."""

    device: torch.device
    vocab_size: int
    seed: int = 42
    generator: torch.Generator | None = field(default=None, repr=False)

    def _gen(self) -> torch.Generator:
        if self.generator is None:
            self.generator = torch.Generator(device=self.device)
            self.generator.manual_seed(self.seed)
        return self.generator

    def prepare(self, batch) -> BatchSamplingArgs:
        """Normalise the requests' SamplingParams (sample.py:89-105): greedy rows
        get T = 1e-6 when any row samples, k < 1 means V, and each tensor is
        None when it is neutral for every row."""
        params = [r.sampling_params for r in batch.reqs]
        MIN_T = 1e-6
        ts = [max(0.0 if p.is_greedy else p.temperature, MIN_T) for p in params]
        top_ks = [p.top_k if p.top_k >= 1 else self.vocab_size for p in params]
        top_ps = [p.top_p for p in params]
        temperatures = (
            None
            if all(p.is_greedy for p in params)
            else make_device_tensor(ts, torch.float32, self.device)
        )
        top_k, top_p = None, None
        if any(k != self.vocab_size for k in top_ks):
            top_k = make_device_tensor(top_ks, torch.int32, self.device)
        if any(p < 1.0 for p in top_ps):
            top_p = make_device_tensor(top_ps, torch.float32, self.device)
        return BatchSamplingArgs(temperatures, top_k=top_k, top_p=top_p)

    def sample(self, logits: torch.Tensor, args: BatchSamplingArgs) -> torch.Tensor:
        """int32 ids: argmax when ``args.temperatures`` is None (sample.py:110-111),
        otherwise softmax(logits / T) filtered by top-k then top-p and sampled
        with ``args.uniforms`` (drawn here when absent)."""
        with torch.cuda.nvtx.range("Sampler"):
            if args.temperatures is None:  # greedy sampling
                return sample_rows(logits, None, None, None, None)
            uniforms = args.uniforms
            if uniforms is None:
                uniforms = torch.rand(logits.shape[0], device=logits.device, generator=self._gen())
            return sample_rows(logits, args.temperatures, args.top_k, args.top_p, uniforms)
