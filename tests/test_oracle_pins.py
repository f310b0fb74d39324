"""Pin the CPU oracle before trusting it (CPU only).

Each check compares the oracle with something independent of its code: the
reference's own greedy call (torch.argmax), library routines (torch.softmax,
the HF transformers top-k/top-p warpers, numpy.searchsorted, scipy's expit,
numpy.nonzero), closed forms, brute force on tiny inputs, and the reference's
known-answer tests (tests/core/test_exit_gates.py).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch


def _bits(x):
    import oracle

    return oracle.bf16_bits(x)


# ---------------------------------------------------------------- greedy -----
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_argmax_matches_torch(orc, dtype):
    """sample.py:111 is torch.argmax; the oracle must agree on every row,
    including ties, NaN, +-inf and signed zeros."""
    g = torch.Generator().manual_seed(5)
    B, V = 64, 1000
    x = torch.randn(B, V, generator=g).to(dtype)
    x[0, 17] = float("nan")
    x[1, :] = 0.0
    x[1, 3] = -0.0
    x[2, 400] = float("inf")
    x[3, :] = float("-inf")
    x[4, :] = float("nan")
    x[5, 10] = x[5].max() + 1
    x[5, 20] = x[5, 10]  # tie: first wins
    x[6, :] = 1.0  # all equal
    x[7, 999] = float("inf")
    x[7, 500] = float("nan")  # NaN beats +inf
    x[8, 0] = -0.0
    x[8, 1:] = -1.0
    x[8, 5] = 0.0  # +0 == -0: first (index 0) wins
    code = {torch.float32: orc.F32, torch.bfloat16: orc.BF16, torch.float16: orc.F16}[dtype]
    arr = x.numpy() if dtype == torch.float32 else _bits(x)
    got = orc.argmax(arr, dtype=code)
    want = torch.argmax(x.float() if dtype != torch.float32 else x, dim=-1).numpy()
    want_native = torch.argmax(x, dim=-1).numpy()
    assert np.array_equal(want, want_native)
    assert np.array_equal(got, want)


# ------------------------------------------------------ sampling helpers -----
def _softmax_probs(x, T):
    return torch.softmax(torch.as_tensor(x, dtype=torch.float64) / T, dim=-1).numpy()


def _hf_kept(x, T, k, p):
    """Kept set by the HF warpers (Temperature -> TopK -> TopP), float64."""
    from transformers.generation.logits_process import TopKLogitsWarper, TopPLogitsWarper

    s = torch.as_tensor(x, dtype=torch.float64)[None, :] / T
    if k is not None:
        s = TopKLogitsWarper(top_k=int(k))(None, s)
    if p is not None and p < 1.0:
        s = TopPLogitsWarper(top_p=float(p))(None, s)
    return np.isfinite(s[0].numpy())


def _oracle_kept_and_probs(orc, x, T, k, p, n_u=257):
    """Infer the oracle's kept set from where its draws land, by sweeping u."""
    B = n_u
    xs = np.repeat(x[None, :].astype(np.float32), B, axis=0)
    us = (np.arange(B, dtype=np.float64) + 0.5) / B
    ids, amb = orc.sample(xs, np.full(B, T, np.float32), None if k is None else np.full(B, k, np.int32),
                          None if p is None else np.full(B, p, np.float32), us.astype(np.float32))
    return ids, amb, us


def test_softmax_matches_torch(orc):
    """S2: with no filter, ids follow the inverse CDF of softmax(x / T) in
    index order -- numpy.searchsorted on torch.softmax's cumulative sum."""
    rng = np.random.default_rng(0)
    for T in (0.3, 0.7, 1.0, 2.5):
        x = rng.normal(0, 2, 300).astype(np.float32)
        ids, amb, us = _oracle_kept_and_probs(orc, x, T, None, None)
        cdf = np.cumsum(_softmax_probs(x, T))
        want = np.searchsorted(cdf, us * cdf[-1], side="right")
        ok = (ids == want) | (amb != 0)
        assert ok.all(), (T, np.nonzero(~ok))


@pytest.mark.parametrize("k,p", [(1, None), (5, None), (50, None), (None, 0.5), (None, 0.9),
                                 (20, 0.8), (3, 0.99), (299, 0.7)])
def test_filters_match_hf_warpers(orc, k, p):
    """S3/S4: the kept set equals the HF TopK/TopP warpers' on tie-free rows,
    and draws follow searchsorted over the renormalised kept mass."""
    rng = np.random.default_rng(1 + (k or 0))
    for trial in range(6):
        x = rng.normal(0, 1.5, 300).astype(np.float32)
        T = 0.6 + 0.2 * trial
        kept = _hf_kept(x, T, k, p)
        probs = _softmax_probs(x, T) * kept
        cdf = np.cumsum(probs)
        ids, amb, us = _oracle_kept_and_probs(orc, x, T, k, p)
        want = np.searchsorted(cdf, us * cdf[-1], side="right")
        ok = (ids == want) | (amb != 0)
        assert ok.all(), (trial, np.nonzero(~ok))
        assert kept[ids[amb == 0]].all()


def test_closed_forms(orc):
    """Uniform row: id = floor(u * V); one-hot row: always the hot index;
    T <= 0 -> argmax; p tiny -> the argmax (ties kept, u decides among them)."""
    V = 1000
    us = np.array([0.0, 0.1234, 0.5, 0.9999], np.float32)
    B = len(us)
    x = np.zeros((B, V), np.float32)
    ids, amb = orc.sample(x, np.full(B, 0.8, np.float32), None, None, us)
    assert np.array_equal(ids[amb == 0], np.floor(us.astype(np.float64) * V).astype(np.int32)[amb == 0])
    x = np.full((B, V), -1000.0, np.float32)  # exp(-2000) is exactly 0 in float64
    x[:, 321] = 30.0
    ids, _ = orc.sample(x, np.full(B, 1.0, np.float32), None, None, us)
    assert (ids == 321).all()
    x[:, :] = -30.0  # tiny but positive mass elsewhere: u = 0 picks index 0, flagged
    x[:, 321] = 30.0
    ids, amb = orc.sample(x, np.full(B, 1.0, np.float32), None, None, us)
    assert ids[0] == 0 and amb[0] & 1 and (ids[1:] == 321).all()
    y = np.random.default_rng(3).normal(size=(B, V)).astype(np.float32)
    ids, _ = orc.sample(y, np.zeros(B, np.float32), None, None, us)
    assert np.array_equal(ids, y.argmax(1))
    y[:, 10] = 9.0
    y[:, 700] = 9.0
    ids, _ = orc.sample(y, np.full(B, 1.0, np.float32), None, np.full(B, 1e-6, np.float32), us)
    assert np.array_equal(ids, np.where(us < 0.5, 10, 700))


def test_brute_force_tiny(orc):
    """Tiny V with heavy ties: enumerate the definition directly (sort by value,
    tie groups kept whole) and compare every draw."""
    rng = np.random.default_rng(7)
    for trial in range(200):
        V = int(rng.integers(1, 9))
        x = rng.integers(-3, 3, V).astype(np.float32)
        T = float(rng.choice([0.5, 1.0, 2.0]))
        k = int(rng.integers(0, V + 2))
        p = float(rng.choice([0.3, 0.6, 0.9, 1.0]))
        u = float(rng.random())
        e = np.exp((x.astype(np.float64) - x.max()) / T)
        keep = np.ones(V, bool)
        if 1 <= k < V:
            kth = np.sort(x)[::-1][k - 1]
            keep &= x >= kth
        if p < 1.0:
            zk = e[keep].sum()
            cands = sorted(set(x[keep].tolist()), reverse=True)
            tau = max(c for c in cands if e[keep & (x >= c)].sum() >= p * zk)
            keep &= x >= tau
        cum = np.cumsum(np.where(keep, e, 0.0))
        want = int(np.argmax(cum > u * cum[-1]))
        ids, amb = orc.sample(x[None, :], np.array([T], np.float32), np.array([k], np.int32),
                              np.array([p], np.float32), np.array([u], np.float32))
        if amb[0] == 0:
            assert ids[0] == want, (x, T, k, p, u, ids[0], want)


def test_ambiguity_flag_is_tight(orc):
    """A uniform placed exactly on a CDF step is flagged; one far away is not."""
    x = np.zeros((2, 4), np.float32)  # probs 0.25 each
    ids, amb = orc.sample(x, np.ones(2, np.float32), None, None, np.array([0.5, 0.6], np.float32))
    assert amb[0] & 1 and not amb[1] & 1
    assert ids[1] == 2


def test_topp_alternative_draw(orc):
    """Rows whose top-p mass sits on p: the oracle also gives the draw from the
    other kept set.  Masses 1 : 1/2 : 1/2 (x = ln 2, 0, 0 at T = 1), u = 0.9:
    p = 1/2 puts the first element's mass on the target (kept set {0}, id 0;
    alternative {0, 1, 2}, U = 1.8 of 2 -> id 2); p just above 1/2 puts the
    tied pair's lower edge on it (kept set {0, 1, 2}, id 2; alternative {0})."""
    x = np.array([[np.log(2.0), 0.0, 0.0]] * 2, np.float32)
    p = np.array([0.5, 0.5 + 1e-8], np.float32)
    p[1] = np.nextafter(np.float32(0.5), np.float32(1.0))
    ids, amb, alt = orc.sample(x, np.ones(2, np.float32), None, p, np.full(2, 0.9, np.float32), with_alt=True)
    assert amb[0] & 2 and ids[0] == 0 and alt[0] == 2
    assert amb[1] & 2 and ids[1] == 2 and alt[1] == 0
    # far from the boundary: no flag, the alternative is the draw itself
    ids, amb, alt = orc.sample(x, np.ones(2, np.float32), None, np.array([0.3, 0.8], np.float32),
                               np.full(2, 0.9, np.float32), with_alt=True)
    assert (amb == 0).all() and (alt == ids).all() and ids.tolist() == [0, 2]


# ------------------------------------------------------------ exit gate -----
def _logit(p):
    return float(np.log(p / (1 - p)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_gate_reference_kat(orc, dtype):
    """tests/core/test_exit_gates.py:15-36: hazards 0.3 / 0.1, then reordered
    rows at step 1 give states [0.19, 0.51] and signal [F, T] at tau = 0.5."""
    hidden = torch.logit(torch.tensor([[0.3], [0.1]])).to(dtype)
    code = {torch.float32: orc.F32, torch.bfloat16: orc.BF16, torch.float16: orc.F16}[dtype]
    arr = hidden.numpy() if dtype == torch.float32 else _bits(hidden)
    one = torch.ones(1, dtype=dtype)
    w = one.numpy() if dtype == torch.float32 else _bits(one)
    r0 = orc.exit_gate(arr, w, None, np.zeros(2, np.float32), 0, 0.5, dtype=code)
    assert not r0["mask"].any()
    np.testing.assert_allclose(r0["F_next"], [0.3, 0.1], atol=1e-3)
    order = [1, 0]
    r1 = orc.exit_gate(np.ascontiguousarray(arr[order]), w, None, r0["F_next"][order], 1, 0.5, dtype=code)
    assert r1["mask"].tolist() == [0, 1]
    np.testing.assert_allclose(r1["F_next"], [0.19, 0.51], atol=1e-3)
    assert r1["exit_idx"].tolist() == [1] and r1["keep_idx"].tolist() == [0]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gate_graph_kat(orc, dtype):
    """tests/core/test_exit_gates.py:63-112: z = -0.8472978604 (lambda 0.3)
    does not exit at step 0; the state copied back and hidden * 1.02 exits."""
    hidden = torch.ones(4, 128, dtype=dtype)
    hidden[:, 0] = -0.8472978604
    w = torch.zeros(128, dtype=dtype)
    w[0] = 1
    b = torch.zeros(1, dtype=dtype)
    code = orc.BF16 if dtype == torch.bfloat16 else orc.F16
    F = np.zeros(4, np.float32)
    for step in range(2):
        r = orc.exit_gate(_bits(hidden), _bits(w), _bits(b), F, 0, 0.5, dtype=code)
        assert bool(r["mask"].all()) == (step == 1)
        F = r["F_next"]
        hidden = hidden * 1.02


def test_gate_product_form_and_expit(orc):
    """G2/G3: lambda = expit(z) (scipy) and F_t = 1 - prod(1 - lambda_s)."""
    from scipy.special import expit

    rng = np.random.default_rng(11)
    z = rng.normal(-1, 2, (5, 1000)).astype(np.float32)
    F = np.zeros(1000, np.float32)
    surv = np.ones(1000)
    for t in range(5):
        F = orc.cumulative_exit_probability(z[t], F)
        surv *= 1 - expit(z[t].astype(np.float64))
        np.testing.assert_allclose(F, 1 - surv, atol=2e-6)
    lam = orc.cumulative_exit_probability(z[0], np.zeros(1000, np.float32))
    want = expit(z[0].astype(np.float64)).astype(np.float32)
    # float32 evaluation of 1 / (1 + exp(-z)) (three roundings): within two ulps
    # of the rounded exact value
    assert np.abs(lam.view(np.int32) - want.view(np.int32)).max() <= 2


def _finite_half_values():
    """Every finite bf16 and fp16 value, as float32 (the gate logit's dtypes)."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16)
    out = []
    for dt in (torch.bfloat16, torch.float16):
        z = bits.view(dt).float()
        out.append(z[torch.isfinite(z)])
    return torch.cat(out).numpy()


def test_sigmoid_is_float32_formula(orc):
    """G2: for every finite bf16 and fp16 z, lambda is exactly
    float32(1 / float32(1 + e)) with e = exp(-z) correctly rounded to float32 --
    the float32 formula torch's sigmoid evaluates -- where e comes from a
    40-digit decimal exp and the + and / are numpy's IEEE float32 operations."""
    from decimal import Context, Decimal

    z = _finite_half_values()
    ctx = Context(prec=40)

    def exp_neg(v):
        x = -float(v)
        return float("inf") if x > 200 else 0.0 if x < -200 else float(ctx.exp(Decimal(x)))

    with np.errstate(over="ignore"):
        e = np.array([exp_neg(v) for v in z]).astype(np.float32)
        want = np.float32(1) / (np.float32(1) + e)
    lam = orc.cumulative_exit_probability(z, np.zeros(z.size, np.float32))
    assert np.array_equal(lam.view(np.int32), want.astype(np.float32).view(np.int32))


def test_sigmoid_matches_torch_float32(orc):
    """G2/G4 against torch's own CPU float32 sigmoid (exit_gates.py:13) over every
    finite bf16 and fp16 z: lambda within two ulps (torch's vectorised CPU exp is
    not correctly rounded); F' against ``prev + (1 - prev) * z.float().sigmoid()``;
    every row whose mask flips between the two at a threshold lies inside the
    flagged tau band."""
    z = _finite_half_values()
    lam = orc.cumulative_exit_probability(z, np.zeros(z.size, np.float32))
    lam_t = torch.sigmoid(torch.from_numpy(z)).numpy()
    ulp = np.abs(lam.view(np.int32).astype(np.int64) - lam_t.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2
    assert (ulp == 0).mean() > 0.99
    rng = np.random.default_rng(5)
    F = rng.random(z.size).astype(np.float32) * 0.9
    Fn = orc.cumulative_exit_probability(z, F)
    Ft = torch.from_numpy(F)
    Fn_t = (Ft + (1.0 - Ft) * torch.sigmoid(torch.from_numpy(z))).numpy()
    assert np.abs(Fn.astype(np.float64) - Fn_t).max() < 4e-7
    # identity gate (H = 1, w = 1, no bias) so z = h exactly; thresholds at the
    # values where the two F' disagree most often
    diff = np.nonzero(Fn != Fn_t)[0]
    assert diff.size > 0
    h = torch.from_numpy(z[diff]).to(torch.float32).numpy().reshape(-1, 1)
    for tau in np.unique(np.concatenate([Fn[diff][:50], Fn_t[diff][:50]])):
        r = orc.exit_gate(h, np.ones(1, np.float32), None, F[diff], 0, float(tau), dtype=orc.F32)
        ref = Fn_t[diff] >= np.float32(tau)
        flip = r["mask"].astype(bool) != ref
        assert ((r["amb"][flip] & 9) == 9).all()


def test_exp_rounding_is_safe(orc):
    """exp(-z) rounded from float64 to float32 is the correctly rounded float32
    exp for every finite bf16 and fp16 z, whichever float64 exp computes it
    (device or host) as long as its error stays under two float64 ulps: the
    exact value lies at least four float64 ulps away from every float32
    rounding boundary (the closest case is z = 2^-25, where exp(-z) sits
    z^2/2 above the midpoint 1 - 2^-25)."""
    z = _finite_half_values().astype(np.float64)
    with np.errstate(over="ignore"):
        e = np.exp(-z)
    ok = np.isfinite(e) & (e >= np.float64(np.finfo(np.float32).tiny))
    ok &= e < np.float64(np.finfo(np.float32).max)
    e = e[ok]
    f = e.astype(np.float32)
    lo = np.nextafter(f, np.float32(0)).astype(np.float64)
    hi = np.nextafter(f, np.float32(np.inf)).astype(np.float64)
    fd = f.astype(np.float64)
    gap = np.minimum(np.abs(e - (fd + lo) / 2), np.abs(e - (fd + hi) / 2))
    assert (gap / np.spacing(e)).min() >= 4


def test_router_reference_kat(orc):
    """tests/core/test_scheduler.py:65-78: a depth-two replay exits at depth two
    under either gate timing; a replacement request in the same slot is not
    routed by the old token's gate."""
    for direct in (False, True):
        r = orc.CdbRouter(max_depth=4, disable_lookahead_exit=direct)
        r.add(orc.Token(("req0", 0, 2), 0, depth=2, replay=2))
        gate_token = orc.Token(("req0", 0, 2), 0, depth=2 if direct else 1, replay=2)
        assert r._consume(([gate_token], [False])) == [("req0", 0, 2)]
        r = orc.CdbRouter(max_depth=4, disable_lookahead_exit=direct)
        r.add(orc.Token(("req0b", 0, 2), 0, depth=1))
        assert r._consume(([gate_token], [False])) == []
        assert len(r.core) == 1


def test_router_timings(orc):
    """The same replay and request sequence under both timings: direct routing
    exits in the step the gate fires; lookahead routing one core step later
    (the token advanced once more), and a gate whose token skipped the next core
    step is dropped; the depth cap routes at max_depth either way."""
    for direct in (False, True):
        r = orc.CdbRouter(max_depth=4, disable_lookahead_exit=direct)
        r.add(orc.Token("a", 0))
        r.add(orc.Token("b", 1, replay=2))
        r.add(orc.Token("c", 2))
        s1 = r.core_step(["a", "b", "c"], [True, False, False])
        assert s1 == (["a"] if direct else [])
        s2 = r.core_step(["b", "c"] if direct else ["a", "b", "c"], [False, False, True])
        assert s2 == (["b"] if direct else ["a", "b"])
        # c requested at its second step; under lookahead it skips the next step
        s3 = r.core_step([] if not direct else ["c"], [] if not direct else [False])
        assert s3 == ([] if not direct else [])
        s4 = r.core_step(["c"], [False])
        assert s4 == ([] if not direct else ["c"])
        if not direct:
            assert r.core_step(["c"], [False]) == ["c"]  # depth cap at 4


def test_gate_dot_and_compaction(orc):
    """G1: z = round_bf16(h . w + b) against a float64 dot; G5 against numpy.nonzero."""
    g = torch.Generator().manual_seed(2)
    B, H = 300, 2048
    h = torch.randn(B, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(H, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.tensor([-2.5]).to(torch.bfloat16)
    F = torch.rand(B, generator=g).numpy() * 0.3
    ls = torch.randint(0, 4, (B,), generator=g).to(torch.int32).numpy()
    r = orc.exit_gate(_bits(h), _bits(w), _bits(b), F, ls, 0.2, min_loop_steps=2, dtype=orc.BF16)
    v = h.double().numpy() @ w.double().numpy() + float(b.double())
    z_ref = torch.tensor(v).to(torch.bfloat16).double().numpy()  # torch's own RNE rounding
    clean = (r["amb"] & 4) == 0
    np.testing.assert_array_equal(r["z"][clean], z_ref[clean])
    assert np.array_equal(r["exit_idx"], np.nonzero(r["mask"])[0])
    assert np.array_equal(r["keep_idx"], np.nonzero(r["mask"] == 0)[0])
    assert int(r["n_exit"][0]) == int(r["mask"].sum())
    depth_ok = ls + 1 >= 2
    assert not r["mask"][~depth_ok].any()
    # max_depth forces exits at depth >= max_depth (cdb_scheduler.py:262-266)
    r2 = orc.exit_gate(_bits(h), _bits(w), _bits(b), F, ls, 0.2, min_loop_steps=2, max_depth=3,
                       dtype=orc.BF16)
    assert r2["mask"][ls + 1 >= 3].all()
    # lookahead shifts the depth test by one (ouro.py:152)
    r3 = orc.exit_gate(_bits(h), _bits(w), _bits(b), F, ls, 0.2, min_loop_steps=2, lookahead=True,
                       dtype=orc.BF16)
    assert np.array_equal(r3["mask"], ((r3["F_next"] >= np.float32(0.2)) & (ls + 2 >= 2)).astype(np.uint8))


def test_huginn_reference_kat(orc):
    """tests/core/test_exit_gates.py:39-60: [T, F, F, T] with strict '<'."""
    prev = np.array([[0, 0], [1, 0], [-1, -1], [1, 1]], np.float32)
    cur = np.array([[0, 0], [2, 0], [1, 1], [1, 1]], np.float32)
    ratio, mask, _ = orc.relative_state_change(cur, prev, 0.5)
    assert mask.tolist() == [1, 0, 0, 1]
    want = np.linalg.norm(cur - prev, axis=1) / np.maximum(np.linalg.norm(cur, axis=1), 1e-9)
    np.testing.assert_allclose(ratio, want, rtol=1e-6)
    _, mask2, _ = orc.relative_state_change(cur, prev, 1.0)  # ratio 0.5 at row 1 -> exits
    assert mask2.tolist() == [1, 1, 0, 1]
