"""Parity of the HIP sampler (lsg_sample) with the CPU oracle and torch.argmax.

Bar: greedy ids bit-exact; sampled ids equal to the oracle's, except that a row
whose top-p mass lies within 1e-6 of p may return the draw from the other kept
set (the oracle computes it), and a row whose CDF lies within 1e-6 of the
uniform (for the id drawn) is excused.  Each check caps the excused rows.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _host(orc, logits):
    x = logits.detach().cpu().contiguous()
    if x.dtype == torch.float32:
        return x.numpy(), orc.F32
    return orc.bf16_bits(x), (orc.BF16 if x.dtype == torch.bfloat16 else orc.F16)


def _np(t):
    return None if t is None else t.detach().cpu().numpy()


def check_sampling(lsg, orc, logits, T, K, P, U, max_excused=0):
    """The GPU ids against the oracle's on the same inputs.  Accepted per row:
    the oracle's id; on a top-p-ambiguous row (amb bit 1) the draw from the
    other kept set; excused (any id): a row whose draw's CDF lies within 1e-6 of
    u (bit 0, or bit 2 when the GPU took the other kept set).  At most
    max_excused rows may be excused."""
    ids = lsg.sample_rows(logits, T, K, P, U).cpu().numpy()
    arr, code = _host(orc, logits)
    ref, amb, alt = orc.sample(arr, _np(T), _np(K), _np(P), _np(U), dtype=code, with_alt=True)
    took_alt = ((amb & 2) != 0) & (ids == alt) & (ids != ref)
    excused = ((amb & 1) != 0) | (((amb & 2) != 0) & ((amb & 4) != 0))
    ok = (ids == ref) | took_alt | excused
    bad = np.nonzero(~ok)[0]
    assert bad.size == 0, f"{bad.size} mismatching rows, e.g. row {bad[:5]}: gpu {ids[bad[:5]]} oracle {ref[bad[:5]]}"
    print(f"[parity] rows {len(ids)}: top-p-ambiguous {int(((amb & 2) != 0).sum())} "
          f"(other kept set taken {int(took_alt.sum())}), excused {int(excused.sum())} "
          f"(differing {int((excused & (ids != ref)).sum())})")
    assert excused.sum() <= max_excused, f"too many excused rows: {int(excused.sum())} > {max_excused}"
    assert ((ids >= 0) & (ids < logits.shape[1])).all()
    return ids, ref, amb


# ------------------------------------------------------------------ greedy ----
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("V", [1, 7, 4096, 49152, 65536, 65537, 131072, 300001])
def test_greedy_bit_exact(lsg, orc, dev, dtype, V):
    g = torch.Generator(device=dev).manual_seed(V)
    B = 16
    x = torch.randn(B, V, generator=g, device=dev).to(dtype)
    if V > 10:
        x[0, V // 3] = float("nan")
        x[1, :] = 0.0
        x[1, V // 2] = -0.0
        x[2, V - 1] = float("inf")
        x[3, :] = float("-inf")
        x[4, :] = float("nan")
        x[5, 3] = 9.0
        x[5, V - 2] = 9.0
        x[6, :] = 1.0
        x[7, V - 1] = float("inf")
        x[7, 1] = float("nan")
    ids = lsg.sample_rows(x, None, None, None, None).cpu().numpy()
    want = torch.argmax(x, dim=-1).to(torch.int32).cpu().numpy()  # the reference's call
    assert np.array_equal(ids, want)
    arr, code = _host(orc, x)
    assert np.array_equal(ids, orc.argmax(arr, dtype=code))


def test_greedy_sampler_interface(lsg, dev):
    """Sampler.sample with temperatures None is argmax (sample.py:110-111)."""
    x = torch.randn(32, 5000, device=dev)
    s = lsg.Sampler(dev, 5000)
    ids = s.sample(x, lsg.BatchSamplingArgs(None))
    assert ids.dtype == torch.int32
    assert torch.equal(ids.long(), torch.argmax(x, -1))


# ---------------------------------------------------------------- workloads --
def test_sample_small_golden(lsg, orc, dev):
    """B=8, V=49152 fp32: greedy equals torch.argmax's committed ids; sampled
    ids (T=0.7, k=50, p=0.9) equal the committed oracle ids."""
    with open(os.path.join(HERE, "golden", "sample_small.json")) as f:
        gold = json.load(f)
    wl = lsg.workloads.sample_small(dev, seed=gold["seed"])
    assert abs(float(wl["logits"].double().sum()) - gold["logits_checksum"]) < 1e-6
    ids = lsg.sample_rows(wl["logits"], None, None, None, None).cpu().tolist()
    assert ids == gold["greedy_ids"]
    ids = lsg.sample_rows(wl["logits"], wl["temperatures"], wl["top_k"], wl["top_p"], wl["uniforms"])
    ids = ids.cpu().numpy()
    amb = np.array(gold["sampled_amb"])
    assert np.array_equal(ids[amb == 0], np.array(gold["sampled_ids"])[amb == 0])


def test_sample_ouro_mixed(lsg, orc, dev):
    """B=256, V=49152 bf16 logits = h W^T; per-row T, k in {1,20,50,off}, p~U[0.8,1]."""
    wl = lsg.workloads.sample_ouro(dev)
    # near-flat logits: each token carries ~1/40000 of the mass, so a few top-p
    # boundaries fall within the 1e-6 ambiguity band
    check_sampling(lsg, orc, wl["logits"], wl["temperatures"], wl["top_k"], wl["top_p"], wl["uniforms"],
                   max_excused=5)


def test_sample_huginn_full(lsg, orc, dev):
    """B=1024, V=65536 bf16 Zipf-like, T=0.6, p=0.95 (the headline workload)."""
    wl = lsg.workloads.sample_huginn(dev)
    check_sampling(lsg, orc, wl["logits"], wl["temperatures"], None, wl["top_p"], wl["uniforms"])


def test_sample_mixed_depth_fp32(lsg, orc, dev):
    """B=2048, V=65536 fp32 Student-t with exact top-2 ties; mixed greedy
    (T=1e-6)/top-k/top-p rows."""
    wl = lsg.workloads.cdb_mixed_depth(dev)
    ids, ref, amb = check_sampling(lsg, orc, wl["logits"], wl["temperatures"], wl["top_k"], wl["top_p"],
                                   wl["uniforms"], max_excused=2)
    # greedy rows with tied maxima split their mass: the uniform decides the tie
    tie = wl["tie_rows"].cpu().numpy() & (wl["temperatures"].cpu().numpy() < 1e-5)
    if tie.any():
        top = torch.topk(wl["logits"][torch.from_numpy(tie).to(dev)], 2, dim=1).indices.sort(dim=1).values
        top = top.cpu().numpy()
        u = wl["uniforms"].cpu().numpy()[tie]
        want = np.where(u < 0.5, top[:, 0], top[:, 1])
        assert np.array_equal(ids[tie], want)


# --------------------------------------------------------------- edge cases --
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("V", [1, 3, 100, 1000, 8191, 24576, 32768, 40000, 49152, 65536, 150001])
def test_modes_ragged(lsg, orc, dev, dtype, V):
    """Every filter combination on ragged V (partial tail chunks)."""
    g = torch.Generator(device=dev).manual_seed(1000 + V)
    B = 24
    x = (torch.randn(B, V, generator=g, device=dev) * 4).to(dtype)
    T = 0.4 + torch.rand(B, generator=g, device=dev)
    K = torch.tensor([0, 1, 5, 50, V, V + 3, -1, 2] * 3, dtype=torch.int32, device=dev)
    P = torch.tensor([1.0, 0.9, 0.5, 1.0, 0.99, 0.3, 0.95, 1.0] * 3, device=dev)
    U = torch.rand(B, generator=g, device=dev)
    for k_, p_ in ((K, P), (None, None), (K, None), (None, P)):
        check_sampling(lsg, orc, x, T, k_, p_, U, max_excused=2)


def test_flat_rows_exact_path(lsg, orc, dev):
    """Near-uniform rows make the top-p set large: the exact (bisection) path."""
    g = torch.Generator(device=dev).manual_seed(9)
    B, V = 16, 49152
    x = (torch.randn(B, V, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    T = torch.full((B,), 1.0, device=dev)
    P = torch.linspace(0.1, 0.99, B, device=dev)
    K = torch.tensor([-1] * 8 + [30000] * 8, dtype=torch.int32, device=dev)
    U = torch.rand(B, generator=g, device=dev)
    check_sampling(lsg, orc, x, T, K, P, U, max_excused=1)


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 49152), (torch.float16, 49152), (torch.float32, 24576),
                                     (torch.float32, 49152)])
def test_dense_topp_rows(lsg, orc, dev, dtype, V):
    """Top-p rows whose kept set holds thousands of elements (B=64 <= CUs:
    one row per CU, six register chunks per thread; twelve for fp32 V=49152,
    whose rows take the exact refinement instead): the mass histogram, the
    crossing bin's members and their key radix.  Rows: near-flat Gaussian at
    several T and p (0.05 .. 0.999), thresholds near x = 0 (wide key span in
    the crossing bin), NaN and -inf elements, half the row tied at one value,
    a constant row (every element in one bin: the exact refinement decides),
    and a row with a single dominant element."""
    g = torch.Generator(device=dev).manual_seed(V + 5)
    B = 64
    x = torch.randn(B, V, generator=g, device=dev) * 0.9
    x[1] -= x[1].mean() + 3.0 * x[1].std()  # most of the row far below its top
    x[2, ::7] = float("nan")
    x[3, ::5] = float("-inf")
    x[4, : V // 2] = 0.5  # half the row tied
    x[5, :] = 1.25  # constant
    x[6, 123] = 40.0  # one dominant element
    x[7] = torch.randn(V, generator=g, device=dev) * 0.01  # values packed around 0
    x = x.to(dtype)
    T = torch.tensor([0.3, 0.7, 1.0, 1.5], device=dev).repeat(B // 4)
    P = torch.tensor([0.05, 0.5, 0.8, 0.9, 0.95, 0.99, 0.999, 0.7], device=dev).repeat(B // 8)
    U = torch.rand(B, generator=g, device=dev)
    # near-flat rows: each element carries ~1/30000 of the mass, so a few
    # percent of the rows have u or p within 1e-6 of a CDF step
    check_sampling(lsg, orc, x, T, None, P, U, max_excused=12)
    K = torch.full((B,), V, dtype=torch.int32, device=dev)
    K[::9] = 1000  # top-k + top-p rows keep the previous paths
    check_sampling(lsg, orc, x, T, K, P, U, max_excused=12)


def test_closed_forms_gpu(lsg, dev):
    """Uniform row -> floor(u V); one-hot -> hot index; T <= 0 -> argmax;
    all -inf -> 0; +inf max -> first +inf (argmax rule)."""
    V = 1000
    u = torch.tensor([0.1234, 0.5001, 0.9999, 0.0], device=dev)
    x = torch.zeros(4, V, device=dev)
    ids = lsg.sample_rows(x, torch.full((4,), 0.8, device=dev), None, None, u).cpu()
    assert ids.tolist() == [123, 500, 999, 0]
    x = torch.full((4, V), -1000.0, device=dev)
    x[:, 321] = 30.0
    assert lsg.sample_rows(x, torch.ones(4, device=dev), None, None, u).cpu().tolist() == [321] * 4
    y = torch.randn(4, V, device=dev)
    y[2, :] = float("-inf")
    y[3, 7] = float("inf")
    y[3, 9] = float("inf")
    ids = lsg.sample_rows(y, torch.tensor([0.0, -1.0, 1.0, 1.0], device=dev), None, None, u).cpu()
    assert ids[0] == torch.argmax(y[0]).item() and ids[1] == torch.argmax(y[1]).item()
    assert ids[2] == 0 and ids[3] == 7


def test_nan_logits_in_sampling_rows(lsg, orc, dev):
    """NaN logits carry no mass in sampling rows (treated as -inf)."""
    g = torch.Generator(device=dev).manual_seed(4)
    x = torch.randn(8, 3000, generator=g, device=dev)
    x[:, ::7] = float("nan")
    T = torch.full((8,), 0.9, device=dev)
    U = torch.rand(8, generator=g, device=dev)
    ids, _, _ = check_sampling(lsg, orc, x, T, torch.full((8,), 20, dtype=torch.int32, device=dev),
                               torch.full((8,), 0.8, device=dev), U)
    assert (ids % 7 != 0).all()


def test_unaligned_rows(lsg, orc, dev):
    """Row stride not a multiple of 16 bytes and an odd base offset."""
    g = torch.Generator(device=dev).manual_seed(6)
    big = torch.randn(12, 50258, generator=g, device=dev).to(torch.bfloat16)
    x = big[:, 1:50258]  # V = 50257 (GPT-2 vocab), ld = 50258, base offset 2 bytes
    T = torch.full((12,), 0.8, device=dev)
    U = torch.rand(12, generator=g, device=dev)
    check_sampling(lsg, orc, x.contiguous(), T, None, torch.full((12,), 0.9, device=dev), U)
    ids_view = lsg.sample_rows(x, T, None, torch.full((12,), 0.9, device=dev), U)
    ids_cont = lsg.sample_rows(x.contiguous(), T, None, torch.full((12,), 0.9, device=dev), U)
    assert torch.equal(ids_view, ids_cont)
    assert torch.equal(lsg.sample_rows(x, None, None, None, None).long(), torch.argmax(x, -1))


def test_gather_and_device_count(lsg, dev):
    """row_idx gathers rows (invalid -> -1); n_rows limits the rows written."""
    g = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn(10, 4096, generator=g, device=dev)
    idx = torch.tensor([9, 0, 3, 42, -1, 5], dtype=torch.int32, device=dev)
    out = torch.full((6,), -7, dtype=torch.int32, device=dev)
    lsg.sample_rows(x, None, None, None, None, row_idx=idx, out=out)
    am = torch.argmax(x, -1)
    assert out.cpu().tolist() == [am[9].item(), am[0].item(), am[3].item(), -1, -1, am[5].item()]
    out.fill_(-7)
    n = torch.tensor([2], dtype=torch.int32, device=dev)
    T = torch.full((10,), 0.7, device=dev)
    U = torch.rand(10, generator=g, device=dev)
    lsg.sample_rows(x, T, None, None, U, row_idx=idx, n_rows=n, out=out)
    full = lsg.sample_rows(x, T, None, None, U)
    got = out.cpu().tolist()
    assert got[:2] == [full[9].item(), full[0].item()] and got[2:] == [-7] * 4


def test_deterministic(lsg, dev):
    wl = lsg.workloads.sample_ouro(dev)
    a = lsg.sample_rows(wl["logits"], wl["temperatures"], wl["top_k"], wl["top_p"], wl["uniforms"])
    b = lsg.sample_rows(wl["logits"], wl["temperatures"], wl["top_k"], wl["top_p"], wl["uniforms"])
    assert torch.equal(a, b)


def test_graph_replay(lsg, dev):
    """Captured in a HIP graph, every replay matches eager execution."""
    wl = lsg.workloads.sample_ouro(dev, B=64)
    args = (wl["logits"], wl["temperatures"], wl["top_k"], wl["top_p"], wl["uniforms"])
    eager = lsg.sample_rows(*args).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lsg.sample_rows(*args)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = lsg.sample_rows(*args)
    for i in range(3):
        out.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
    wl["uniforms"].copy_(torch.rand_like(wl["uniforms"]))
    graph.replay()
    assert torch.equal(out, lsg.sample_rows(*args))


def test_sampler_prepare_and_sample(lsg, orc, dev, SP):
    """Sampler.prepare normalises per-request params; sample draws with the
    given uniforms (greedy rows in a mixed batch use T=1e-6)."""
    from types import SimpleNamespace

    reqs = [SimpleNamespace(sampling_params=p) for p in
            [SP(), SP(temperature=0.8, top_k=20), SP(temperature=1.0, top_p=0.9), SP(top_k=1, temperature=2.0)]]
    s = lsg.Sampler(dev, 3000)
    args = s.prepare(SimpleNamespace(reqs=reqs))
    assert args.temperatures is not None
    g = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(4, 3000, device=dev, generator=g)
    args.uniforms = torch.rand(4, device=dev, generator=g)
    ids = s.sample(x, args)
    check_sampling(lsg, orc, x, args.temperatures, args.top_k, args.top_p, args.uniforms)
    # rows 0 and 3 are greedy: T = 1e-6 puts all mass on the argmax
    am = torch.argmax(x, -1)
    assert ids[0].item() == am[0].item() and ids[3].item() == am[3].item()
    # without uniforms the sampler draws its own (seeded) ones
    args.uniforms = None
    a = s.sample(x, args)
    assert ((a >= 0) & (a < 3000)).all()


def test_filter_merge_batches_on_device(lsg, orc, dev, SP):
    """A batch filtered to some of its rows and merged with another
    (BatchSamplingArgs.filter_batch / merge_batch, sample.py:20-53), then sampled
    on the device: ids against the oracle on the merged arguments, and the merged
    rows carry their own arguments or the neutral defaults (T=1e-6, k=V, p=1)."""
    from types import SimpleNamespace

    V = 5000
    s = lsg.Sampler(dev, V)
    mk = lambda ps: s.prepare(SimpleNamespace(reqs=[SimpleNamespace(sampling_params=p) for p in ps]))
    a = mk([SP(temperature=0.7, top_k=30), SP(), SP(temperature=1.1, top_p=0.85), SP(temperature=0.5),
            SP(temperature=0.9, top_k=5, top_p=0.9), SP(top_k=1, temperature=1.0)])
    b = mk([SP(temperature=0.8, top_p=0.9), SP(temperature=1.3, top_p=0.7), SP(temperature=0.6, top_p=0.95),
            SP(temperature=1.0, top_p=0.8)])
    g = torch.Generator(device=dev).manual_seed(41)
    a.uniforms = torch.rand(6, device=dev, generator=g)
    b.uniforms = torch.rand(4, device=dev, generator=g)
    keep = torch.tensor([4, 0, 2], device=dev)
    af = a.filter_batch(keep, False, need_top_k=True, need_top_p=True)
    assert b.top_k is None  # the second batch has no top-k rows: merge fills k = V
    m = af.merge_batch(b, 3, 4, V)
    assert torch.equal(m.temperatures[:3], a.temperatures[keep]) and torch.equal(m.temperatures[3:], b.temperatures)
    assert torch.equal(m.top_k[:3], a.top_k[keep]) and (m.top_k[3:] == V).all()
    assert torch.equal(m.top_p[:3], a.top_p[keep]) and torch.equal(m.top_p[3:], b.top_p)
    assert torch.equal(m.uniforms, torch.cat([a.uniforms[keep], b.uniforms]))
    x = torch.randn(7, V, device=dev, generator=g)
    ids = s.sample(x, m)
    got, _, _ = check_sampling(lsg, orc, x, m.temperatures, m.top_k, m.top_p, m.uniforms)
    assert torch.equal(ids.cpu(), torch.from_numpy(got))


# ------------------------------------------- large batches (B > 2 x CUs) ----
def _mixed_params(B, V, g, dev):
    """Per-row modes cycling through greedy-in-batch (T=1e-6), no filter,
    top-k, top-p, top-k + top-p, k=1 and k >= V."""
    T = 0.3 + torch.rand(B, generator=g, device=dev)
    T[0::7] = 1e-6
    K = torch.tensor([-1, -1, 20, -1, 50, 1, V + 1], dtype=torch.int32, device=dev).repeat(B // 7 + 1)[:B]
    P = torch.tensor([1.0, 1.0, 1.0, 0.9, 0.95, 1.0, 0.8], device=dev).repeat(B // 7 + 1)[:B]
    U = torch.rand(B, generator=g, device=dev)
    return T, K.contiguous(), P.contiguous(), U


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 65536), (torch.float16, 65536), (torch.bfloat16, 40000),
                                     (torch.float32, 32768), (torch.float32, 20001), (torch.bfloat16, 49152),
                                     (torch.float16, 49152), (torch.float32, 24576)])
def test_large_batches(lsg, orc, dev, dtype, V):
    """B=600 rows: more workgroups than two per CU, so rows run in successive
    waves of workgroups; mixed modes per row, ragged and full rows."""
    g = torch.Generator(device=dev).manual_seed(V + 17)
    B = 600
    x = (torch.randn(B, V, generator=g, device=dev) * 3).to(dtype)
    x[5, 100] = float("nan")
    x[9, :] = float("-inf")
    x[9, V - 1] = 2.0
    T, K, P, U = _mixed_params(B, V, g, dev)
    check_sampling(lsg, orc, x, T, K, P, U, max_excused=20)
    check_sampling(lsg, orc, x, T, None, None, U, max_excused=20)
    ids = lsg.sample_rows(x, None, None, None, None)
    assert torch.equal(ids.long(), torch.argmax(x, -1))


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 65536), (torch.float16, 49152), (torch.float32, 32768),
                                     (torch.float32, 65536)])
def test_streamed_rows_edge_cases(lsg, orc, dev, dtype, V):
    """B=320 (more rows than compute units: the streamed row kernel): the
    argmax edge cases of the small-batch test (NaN, all -inf, +inf, ties, -0,
    constant rows) in greedy and sampling modes, next to NaN-holding rows."""
    g = torch.Generator(device=dev).manual_seed(V + 31)
    B = 320
    x = (torch.randn(B, V, generator=g, device=dev) * 2).to(dtype)
    x[0, V // 3] = float("nan")
    x[1, :] = 0.0
    x[1, V // 2] = -0.0
    x[2, V - 1] = float("inf")
    x[3, :] = float("-inf")
    x[4, :] = float("nan")
    x[5, 3] = 9.0
    x[5, V - 2] = 9.0
    x[6, :] = 1.0
    x[7, V - 1] = float("inf")
    x[7, 1] = float("nan")
    x[8, ::5] = float("nan")
    x[10, :] = float("-inf")
    x[10, 12345] = -3.0
    ids = lsg.sample_rows(x, None, None, None, None).cpu().numpy()
    assert np.array_equal(ids, torch.argmax(x, dim=-1).to(torch.int32).cpu().numpy())
    T, K, P, U = _mixed_params(B, V, g, dev)
    ids, _, _ = check_sampling(lsg, orc, x, T, K, P, U, max_excused=8)
    assert ids[8] % 5 != 0 and ids[10] == 12345


@pytest.mark.parametrize("dtype,V", [(torch.bfloat16, 65536), (torch.float32, 65536), (torch.float32, 32768)])
def test_far_topk_floor(lsg, orc, dev, dtype, V):
    """B=320 top-k rows whose k-th largest logit lies far (up to thousands of
    binary orders at T=0.05) below the maximum: Student-t(3) logits at low
    temperature, k from 1 to past the lanes' pair maxima (1025, 4000), with
    and without top-p; plus ties at the k-th value far below the maximum, a
    crossing bin holding most of the row (window overflow: the exact path), a
    maximum 1e30 above the rest (beyond the binned distances) and -inf
    elements."""
    g = torch.Generator(device=dev).manual_seed(V + 77)
    B = 320
    z = torch.randn(B, V, generator=g, device=dev)
    chi = torch.randn(B, V, 3, generator=g, device=dev).pow(2).sum(-1)
    x = 3.0 * z / torch.sqrt(chi / 3.0)
    del z, chi
    x[0, :] = -1000.0  # ties at the k-th value: 10 at 0, 50 at -500
    x[0, torch.randperm(V, generator=g, device=dev)[:60]] = torch.tensor([0.0] * 10 + [-500.0] * 50, device=dev)
    x[1, :] = torch.randn(V, generator=g, device=dev) * 1e-3  # k-th inside the bulk
    x[1, 7] = 1000.0
    x[2, 100] = 1e30  # distance beyond the last bin
    x[3, ::3] = float("-inf")
    x = x.to(dtype)
    T = torch.tensor([0.8, 0.3, 0.05, 1.0], device=dev).repeat(B // 4)
    K = torch.tensor([1, 2, 5, 40, 41, 200, 512, 1024, 1025, 4000], dtype=torch.int32,
                     device=dev).repeat(B // 10)
    P = torch.tensor([1.0, 1.0, 0.9, 1.0, 0.5], device=dev).repeat(B // 5)
    T[0:4] = 0.8
    K[0:4] = torch.tensor([20, 40, 40, 40], dtype=torch.int32, device=dev)
    P[0:4] = 1.0
    U = torch.rand(B, generator=g, device=dev)
    check_sampling(lsg, orc, x, T, K, P, U, max_excused=2)


def test_large_gather_and_count(lsg, orc, dev):
    """Large batch with row_idx (invalid entries -> -1) and a device row count
    below B_out: rows past the count stay untouched."""
    g = torch.Generator(device=dev).manual_seed(23)
    Bs, V = 700, 65536
    x = (torch.randn(Bs, V, generator=g, device=dev) * 2).to(torch.bfloat16)
    T, K, P, U = _mixed_params(Bs, V, g, dev)
    perm = torch.randperm(Bs, generator=g, device=dev).to(torch.int32)[:640].contiguous()
    perm[3] = -5
    perm[300] = Bs + 1
    full = lsg.sample_rows(x, T, K, P, U)
    out = torch.full((640,), -7, dtype=torch.int32, device=dev)
    lsg.sample_rows(x, T, K, P, U, row_idx=perm, out=out)
    pi = perm.long().cpu()
    valid = (pi >= 0) & (pi < Bs)
    got = out.cpu()
    assert torch.equal(got[valid], full.cpu()[pi[valid]])
    assert (got[~valid] == -1).all()
    out.fill_(-7)
    n = torch.tensor([555], dtype=torch.int32, device=dev)
    lsg.sample_rows(x, None, None, None, None, row_idx=perm, n_rows=n, out=out)
    got = out.cpu()
    am = torch.argmax(x, -1).to(torch.int32).cpu()
    v = valid[:555]
    assert torch.equal(got[:555][v], am[pi[:555][v]])
    assert (got[:555][~v] == -1).all() and (got[555:] == -7).all()


def test_large_graph_replay(lsg, dev):
    """A 520-row top-p launch captured in a HIP graph: every replay matches eager."""
    wl = lsg.workloads.sample_huginn(dev, B=520)
    args = (wl["logits"], wl["temperatures"], None, wl["top_p"], wl["uniforms"])
    eager = lsg.sample_rows(*args).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        lsg.sample_rows(*args)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        out = lsg.sample_rows(*args)
    for i in range(3):
        out.fill_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
