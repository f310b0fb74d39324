"""The fused coda tail (lsg_lm_head / lsg_lm_head_sample) against exact
arithmetic, float64 and the CPU oracle.

Bars:
  * logits: bit-exact bf16 where the fp32 sums are exact (integer-valued data);
    on Gaussian data within 2^-8 relative + 2e-5 of float64 h W^T everywhere,
    equal to bf16(float64) except where the float64 value lies within 3e-5 of a
    rounding boundary (fp32 accumulation order; under 0.1 % of the entries);
  * greedy ids bit-exact against torch.argmax of the produced bf16 logits;
  * sampled ids against the oracle on the produced bf16 logits, with the
    sampler's acceptance rule (other kept set on top-p-ambiguous rows, draws
    within 1e-6 of u excused).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _exact_operands(B, H, V, seed, dev):
    g = torch.Generator(device="cpu").manual_seed(seed)
    h = torch.randint(-3, 4, (B, H), generator=g).float() * 0.25
    w = torch.randint(-3, 4, (V, H), generator=g).float() * 0.125
    return h.to(torch.bfloat16).to(dev), w.to(torch.bfloat16).to(dev), h, w


@pytest.mark.parametrize("B,H,V", [(1, 64, 1000), (37, 128, 5000), (256, 2048, 49152), (300, 192, 1234),
                                   (513, 64, 193)])
def test_lm_head_exact_arithmetic(lsg, dev, B, H, V):
    """Products are multiples of 2^-5 and every partial sum stays below 2^16:
    fp32 accumulation is exact in any order, so the bf16 logits are exact."""
    hb, wb, h, w = _exact_operands(B, H, V, B * 7 + V, dev)
    got = lsg.coda.lm_head(hb, wb)
    want = (h.double() @ w.double().T).to(torch.bfloat16)
    assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))


def test_lm_head_gaussian_vs_float64(lsg, dev):
    """Ouro-1.4B-shaped projection (h ~ N(0, 1) [256, 2048], W ~ N(0, 0.02^2)
    [49152, 2048])."""
    g = torch.Generator(device=dev).manual_seed(5)
    h = torch.randn(256, 2048, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(49152, 2048, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    got = lsg.coda.lm_head(h, w).cpu()
    ref = h.cpu().double() @ w.cpu().double().T
    # bf16 rounding of the fp32 sum (half an ulp, 2^-9 relative) plus the fp32
    # accumulation error (absolute: it is what remains of logits that cancel
    # to near zero)
    err = (got.double() - ref).abs()
    assert (err <= ref.abs() * 2.0 ** -8 + 2e-5).all(), err.max().item()
    # entries that round the other way: their float64 value lies within the
    # accumulation error of the rounding boundary between the two candidates
    want = ref.to(torch.bfloat16)
    mism = got.view(torch.int16) != want.view(torch.int16)
    mid = (got.double()[mism] + want.double()[mism]) / 2
    assert ((ref[mism] - mid).abs() <= 3e-5).all()
    assert mism.sum().item() <= got.numel() // 1000, mism.sum().item()


def _check_ids(orc, logits, T, K, P, U, ids, max_excused):
    bits = logits.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    np_ = lambda t: None if t is None else t.cpu().numpy()
    ref, amb, alt = orc.sample(bits, np_(T), np_(K), np_(P), np_(U), dtype=orc.BF16, with_alt=True)
    ids = ids.cpu().numpy()
    excused = ((amb & 1) != 0) | (((amb & 2) != 0) & ((amb & 4) != 0))
    ok = (ids == ref) | (((amb & 2) != 0) & (ids == alt)) | excused
    assert ok.all(), np.nonzero(~ok)[0][:5]
    assert excused.sum() <= max_excused


def test_coda_sample_ouro(lsg, orc, dev):
    """Ouro-shaped coda: greedy from the tile maxima, then mixed sampling."""
    g = torch.Generator(device=dev).manual_seed(9)
    B, H, V = 256, 2048, 49152
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    h[3, 5] = float("nan")  # a NaN row: argmax is 0 (the first NaN), as torch.argmax
    ws = torch.empty(lsg.coda.workspace_bytes(B, V), dtype=torch.uint8, device=dev)
    ids = lsg.coda.coda_sample(h, w, lsg.BatchSamplingArgs(None), workspace=ws)
    logits = lsg.coda.workspace_logits(ws, B, V)
    assert torch.equal(logits.view(torch.int16), lsg.coda.lm_head(h, w).view(torch.int16))  # bitwise (NaN row)
    assert torch.equal(ids.long(), torch.argmax(logits, dim=-1))
    assert ids[3].item() == 0
    T = 0.3 + 0.9 * torch.rand(B, generator=g, device=dev)
    T[::9] = 0.0  # greedy rows inside a sampling batch
    K = torch.tensor([1, 20, 50, V], dtype=torch.int32, device=dev)[torch.randint(0, 4, (B,), generator=g, device=dev)]
    P = 0.8 + 0.2 * torch.rand(B, generator=g, device=dev)
    U = torch.rand(B, generator=g, device=dev)
    args = lsg.BatchSamplingArgs(T, K.contiguous(), P, U)
    ids = lsg.coda.coda_sample(h, w, args, workspace=ws)
    logits = lsg.coda.workspace_logits(ws, B, V)
    _check_ids(orc, logits, T, K, P, U, ids, max_excused=5)


def test_coda_sample_ragged_and_large_batch(lsg, orc, dev):
    """V not a multiple of the 192-column tile and B above one 256-row tile;
    greedy ids against torch.argmax, sampled ids against the oracle."""
    g = torch.Generator(device=dev).manual_seed(13)
    B, H, V = 300, 256, 50257
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g, device=dev) * 0.1).to(torch.bfloat16)
    ws = torch.empty(lsg.coda.workspace_bytes(B, V), dtype=torch.uint8, device=dev)
    ids = lsg.coda.coda_sample(h, w, lsg.BatchSamplingArgs(None), workspace=ws)
    logits = lsg.coda.workspace_logits(ws, B, V)
    assert torch.equal(ids.long(), torch.argmax(logits, dim=-1))
    T = torch.full((B,), 0.8, device=dev)
    P = torch.full((B,), 0.9, device=dev)
    U = torch.rand(B, generator=g, device=dev)
    ids = lsg.coda.coda_sample(h, w, lsg.BatchSamplingArgs(T, None, P, U), workspace=ws)
    # near-flat rows (each token ~1/30000 of the mass): ~3 % of draws fall within 1e-6 of u
    _check_ids(orc, lsg.coda.workspace_logits(ws, B, V), T, None, P, U, ids, max_excused=15)


def test_coda_graph_replay(lsg, dev):
    """coda_sample with a preallocated workspace captured in a graph: every
    replay (with eager work between them) equals the eager call."""
    g = torch.Generator(device=dev).manual_seed(17)
    B, H, V = 64, 512, 8000
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    args = lsg.BatchSamplingArgs(torch.full((B,), 0.9, device=dev), None, torch.full((B,), 0.95, device=dev),
                                 torch.rand(B, generator=g, device=dev))
    ws = torch.empty(lsg.coda.workspace_bytes(B, V), dtype=torch.uint8, device=dev)
    out = torch.empty(B, dtype=torch.int32, device=dev)
    eager = lsg.coda.coda_sample(h, w, args, workspace=ws).clone()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        lsg.coda.coda_sample(h, w, args, workspace=ws, out=out)
    for i in range(3):
        out.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


def test_coda_argument_errors(lsg, dev):
    h = torch.zeros(4, 100, dtype=torch.bfloat16, device=dev)  # H not a multiple of 64
    w = torch.zeros(10, 100, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        lsg.coda.lm_head(h, w)
    h = torch.zeros(4, 64, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(10, 64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="workspace"):
        lsg.coda.coda_sample(h, w, lsg.BatchSamplingArgs(None), workspace=torch.empty(8, dtype=torch.uint8,
                                                                                       device=dev))
