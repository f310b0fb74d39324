"""Seeded synthetic inputs of the decode-token-path workloads.

Each generator returns torch tensors on ``device`` (random-init data of the
named shapes; no checkpoints or datasets).  The same tensors are handed to the
HIP kernels and, copied to the host, to the CPU oracle.

  sample_small       B=8,    V=49152, fp32 N(0, 2^2); greedy, and T=0.7 k=50 p=0.9
  sample_ouro        B=256,  V=49152, bf16 logits = h W^T (Ouro-1.4B-shaped LM head),
                     per-row T~U[0.3,1.2], k in {1,20,50,off}, p~U[0.8,1]
  gate_cdb           B=512,  4 loop steps, H=2048 bf16 hidden ~N(0,1), gate weight
                     ~N(0, 0.02^2), bias -2.5, tau 0.2; exited rows greedy over V=49152
  sample_huginn      B=1024, V=65536, bf16 Zipf-like logits (-1.1 ln rank + N(0, 0.5^2),
                     permuted per row); T=0.6, p=0.95, k off
  cdb_mixed_depth    B=2048, V=65536, fp32 Student-t(3)*3 logits with exact top-2 ties in
                     5% of rows; depths 1-4; gate as gate_cdb; mixed greedy/top-k/top-p
"""
from __future__ import annotations

import math

import torch


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def sample_small(device="cpu", seed: int = 0):
    g = _gen(seed, "cpu")
    B, V = 8, 49152
    logits = torch.randn(B, V, generator=g) * 2.0
    u = torch.rand(B, generator=g)
    return dict(
        logits=logits.to(device),
        temperatures=torch.full((B,), 0.7, device=device),
        top_k=torch.full((B,), 50, dtype=torch.int32, device=device),
        top_p=torch.full((B,), 0.9, device=device),
        uniforms=u.to(device),
    )


def sample_ouro(device="cpu", seed: int = 1, B: int = 256, V: int = 49152, H: int = 2048):
    g = _gen(seed, device)
    h = torch.randn(B, H, generator=g, device=device)
    W = torch.randn(V, H, generator=g, device=device) * 0.02
    logits = (h @ W.t()).to(torch.bfloat16)
    del W
    T = 0.3 + 0.9 * torch.rand(B, generator=g, device=device)
    choices = torch.tensor([1, 20, 50, -1], dtype=torch.int32, device=device)
    k = choices[torch.randint(0, 4, (B,), generator=g, device=device)]
    p = 0.8 + 0.2 * torch.rand(B, generator=g, device=device)
    u = torch.rand(B, generator=g, device=device)
    # the sampler's own normalisation: k < 1 means "off" (= V)
    k = torch.where(k >= 1, k, torch.full_like(k, V))
    return dict(logits=logits, temperatures=T, top_k=k, top_p=p, uniforms=u)


def zipf_logits(B: int, V: int, device, seed: int, slope: float = 1.1, noise: float = 0.5,
                dtype=torch.bfloat16) -> torch.Tensor:
    g = _gen(seed, device)
    ranks = torch.arange(1, V + 1, device=device, dtype=torch.float32)
    vals = -slope * torch.log(ranks)[None, :] + noise * torch.randn(B, V, generator=g, device=device)
    perm = torch.argsort(torch.rand(B, V, generator=g, device=device), dim=1)
    out = torch.empty_like(vals)
    out.scatter_(1, perm, vals)
    return out.to(dtype)


def sample_huginn(device="cpu", seed: int = 3, B: int = 1024, V: int = 65536):
    logits = zipf_logits(B, V, device, seed)
    g = _gen(seed + 1000, device)
    return dict(
        logits=logits,
        temperatures=torch.full((B,), 0.6, device=device),
        top_k=None,
        top_p=torch.full((B,), 0.95, device=device),
        uniforms=torch.rand(B, generator=g, device=device),
    )


def gate_cdb(device="cpu", seed: int = 2, B: int = 512, H: int = 2048, steps: int = 4,
             V: int = 49152, bias: float = -2.5, tau: float = 0.2):
    g = _gen(seed, device)
    hidden = [torch.randn(B, H, generator=g, device=device).to(torch.bfloat16) for _ in range(steps)]
    w = (torch.randn(H, generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = torch.tensor([bias], device=device).to(torch.bfloat16)
    logits = (torch.randn(B, V, generator=g, device=device) * 2.0).to(torch.bfloat16)
    return dict(hidden=hidden, weight=w, bias=b, tau=tau, logits=logits)


def cdb_mixed_depth(device="cpu", seed: int = 4, B: int = 2048, V: int = 65536, H: int = 2048,
                    bias: float = -2.5, tau: float = 0.2):
    g = _gen(seed, device)
    # Student-t(3) * 3 via normal / sqrt(chi2_3 / 3)
    z = torch.randn(B, V, generator=g, device=device)
    chi = torch.randn(B, V, 3, generator=g, device=device).pow(2).sum(-1)
    logits = 3.0 * z / torch.sqrt(chi / 3.0)
    del z, chi
    # exact top-2 ties in 5% of rows: copy the maximum to another random index
    tie_rows = torch.rand(B, generator=g, device=device) < 0.05
    amax = logits.argmax(dim=1)
    other = torch.randint(0, V, (B,), generator=g, device=device)
    other = torch.where(other == amax, (other + 1) % V, other)
    rows = torch.nonzero(tie_rows).flatten()
    logits[rows, other[rows]] = logits[rows, amax[rows]]
    depth = torch.randint(1, 5, (B,), generator=g, device=device, dtype=torch.int32)
    hidden = torch.randn(B, H, generator=g, device=device).to(torch.bfloat16)
    w = (torch.randn(H, generator=g, device=device) * 0.02).to(torch.bfloat16)
    b = torch.tensor([bias], device=device).to(torch.bfloat16)
    # prior cumulative exit probability from depth-1 earlier steps of sigmoid hazards
    F = torch.zeros(B, device=device)
    for step in range(3):
        lam = torch.sigmoid(bias + 0.9 * torch.randn(B, generator=g, device=device))
        F = torch.where(depth > step + 1, F + (1 - F) * lam, F)
    mode = torch.randint(0, 3, (B,), generator=g, device=device)
    T = torch.where(mode == 0, torch.full((B,), 1e-6, device=device),
                    torch.where(mode == 1, torch.full((B,), 0.8, device=device),
                                torch.full((B,), 0.9, device=device)))
    k = torch.where(mode == 1, torch.full((B,), 40, dtype=torch.int32, device=device),
                    torch.full((B,), V, dtype=torch.int32, device=device))
    p = torch.where(mode == 2, torch.full((B,), 0.9, device=device), torch.ones(B, device=device))
    u = torch.rand(B, generator=g, device=device)
    return dict(logits=logits, tie_rows=tie_rows, depth=depth, hidden=hidden, weight=w, bias=b,
                F_prev=F, tau=tau, temperatures=T, top_k=k, top_p=p, uniforms=u,
                loop_step=depth - 1)


def algorithmic_bytes_sampling(B: int, V: int, elem_size: int, n_params: int) -> int:
    """One read of every logit and per-row input, one write of every id."""
    return B * V * elem_size + B * (4 * n_params + 4 + 4)


def algorithmic_bytes_gate(B: int, H: int, elem_size: int = 2) -> int:
    """Hidden rows, weight, bias, F in/out, depth, mask, one index per row, n_exit."""
    return B * H * elem_size + H * elem_size + elem_size + B * (4 + 4 + 4 + 1 + 4) + 4


LOG2E = 1.0 / math.log(2.0)
