"""Parity of the HIP exit gates (lsg_exit_gate, lsg_cumulative_exit_probability,
lsg_relative_state_change) with the CPU oracle and the reference's KATs.

Bar: the exit mask and the compaction indices bit-exact (except rows whose
decision the oracle flags as sensitive to fp32 accumulation of the gate logit);
the fp32 cumulative exit probability within 1e-5.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _code(orc, dtype):
    return {torch.float32: orc.F32, torch.bfloat16: orc.BF16, torch.float16: orc.F16}[dtype]


def _arr(orc, t):
    t = t.detach().cpu().contiguous()
    return t.numpy() if t.dtype == torch.float32 else orc.bf16_bits(t)


def _check_compaction(res, B):
    mask = res.signal.cpu().numpy()
    n = int(res.n_exit.item())
    assert n == int(mask.sum())
    assert np.array_equal(res.exit_idx[:n].cpu().numpy(), np.nonzero(mask)[0])
    assert np.array_equal(res.keep_idx[: B - n].cpu().numpy(), np.nonzero(~mask)[0])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_ouro_cumulative_exit_state_kat(lsg, dev, dtype):
    """Mirror of tests/core/test_exit_gates.py:15-36 on the HIP gate (identity
    gate: H = 1, weight 1, no bias)."""
    gate = lsg.OuroExitGate(torch.ones(1, 1, dtype=dtype, device=dev), None, exit_threshold=0.5,
                            min_loop_steps=1, loop_steps=4)
    hidden = torch.logit(torch.tensor([[0.3], [0.1]])).to(dtype).to(dev)
    initial = gate.init_exit_state(hidden)
    first_signal, first_state = gate.exit_signal(hidden, initial, 0)
    assert first_signal.dtype == torch.bool and not first_signal.any()
    assert first_state.dtype == torch.float32
    order = torch.tensor([1, 0], device=dev)
    signal, state = gate.exit_signal(hidden[order], first_state[order], 1)
    assert signal.tolist() == [False, True]
    torch.testing.assert_close(state.cpu(), torch.tensor([0.19, 0.51]), atol=1e-3, rtol=1e-3)
    torch.testing.assert_close(first_state.cpu(), torch.tensor([0.3, 0.1]), atol=1e-3, rtol=1e-3)
    assert not initial.any()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_exit_gate_graph_kat(lsg, dev, dtype):
    """Mirror of tests/core/test_exit_gates.py:63-112: captured gate replays
    match eager runs while hidden states and exit history change."""
    hidden = torch.ones(4, 128, device=dev, dtype=dtype)
    w = torch.zeros(1, 128, device=dev, dtype=dtype)
    w[:, 0] = 1
    gate = lsg.OuroExitGate(w, torch.zeros(1, device=dev, dtype=dtype), exit_threshold=0.5)
    hidden[:, 0] = -0.8472978604  # sigmoid 0.3
    state = gate.init_exit_state(hidden)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(3):
            gate.exit_signal(hidden, state, 0)
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        captured_signal, captured_state = gate.exit_signal(hidden, state, 0)
    for step in range(2):
        hidden_before, state_before = hidden.clone(), state.clone()
        expected_signal, expected_state = gate.exit_signal(hidden, state, 0)
        graph.replay()
        torch.testing.assert_close(captured_signal, expected_signal)
        torch.testing.assert_close(captured_state, expected_state)
        torch.testing.assert_close(hidden, hidden_before)
        torch.testing.assert_close(state, state_before)
        assert captured_signal.all().item() == (step == 1)
        state.copy_(captured_state)
        hidden.mul_(1.02)


def test_gate_cdb_four_steps(lsg, orc, dev):
    """B=512, H=2048 bf16, 4 steps, tau=0.2 (the CDB gate workload): mask,
    z, F' and compaction against the oracle at every step."""
    wl = lsg.workloads.gate_cdb(dev)
    gate = lsg.OuroExitGate(wl["weight"], wl["bias"], exit_threshold=wl["tau"], loop_steps=4)
    B = wl["hidden"][0].shape[0]
    F = gate.init_exit_state(wl["hidden"][0])
    F_host = np.zeros(B, np.float32)
    exited_any = 0
    for step, h in enumerate(wl["hidden"]):
        z = torch.empty(B, dtype=torch.float32, device=dev)
        res = gate.exit_signal_compact(h, F, step, z_out=z)
        ref = orc.exit_gate(_arr(orc, h), _arr(orc, wl["weight"]), _arr(orc, wl["bias"]), F_host, step,
                            wl["tau"], dtype=orc.BF16)
        amb = ref["amb"]
        mask = res.signal.cpu().numpy().astype(np.uint8)
        assert np.array_equal(mask[(amb & 1) == 0], ref["mask"][(amb & 1) == 0])
        zc = z.cpu().numpy()
        assert np.array_equal(zc[(amb & 4) == 0], ref["z"][(amb & 4) == 0])
        Fg = res.state.cpu().numpy()
        zok = (amb & 4) == 0  # z cannot round differently under fp32 accumulation
        np.testing.assert_allclose(Fg[zok], ref["F_next"][zok], atol=1e-5)
        # given the same z, F' is bit-exact
        same = zc == ref["z"]
        assert np.array_equal(Fg[same], ref["F_next"][same])
        _check_compaction(res, B)
        if not (amb & 1).any():
            assert np.array_equal(res.exit_idx[: int(res.n_exit.item())].cpu().numpy(), ref["exit_idx"])
        exited_any += int(mask.sum())
        F, F_host = res.state, Fg
    assert exited_any > 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H", [(1, 1), (5, 7), (64, 2048), (300, 5280), (2049, 100), (4096, 2048)])
def test_gate_shapes_and_options(lsg, orc, dev, dtype, B, H):
    """Ragged H, odd B, per-row loop steps, min_loop_steps, lookahead, max_depth."""
    g = torch.Generator(device=dev).manual_seed(B * 7 + H)
    h = torch.randn(B, H, generator=g, device=dev).to(dtype)
    w = (torch.randn(H, generator=g, device=dev) / max(1.0, H ** 0.5)).to(dtype)
    b = torch.tensor([-0.3], device=dev).to(dtype)
    F = torch.rand(B, generator=g, device=dev) * 0.5
    ls = torch.randint(0, 4, (B,), generator=g, device=dev, dtype=torch.int32)
    for lookahead in (False, True):
        for max_depth in (0, 3):
            gate = lsg.OuroExitGate(w, b, exit_threshold=0.45, min_loop_steps=2, loop_steps=4,
                                    exit_gate_type="lookahead" if lookahead else "early_exit")
            res = gate.exit_signal_compact(h, F, ls, max_depth=max_depth)
            ref = orc.exit_gate(_arr(orc, h), _arr(orc, w), _arr(orc, b), F.cpu().numpy(), ls.cpu().numpy(), 0.45,
                                min_loop_steps=2, lookahead=lookahead, max_depth=max_depth,
                                dtype=_code(orc, dtype))
            clean = (ref["amb"] & 1) == 0
            mask = res.signal.cpu().numpy().astype(np.uint8)
            assert np.array_equal(mask[clean], ref["mask"][clean])
            zok = (ref["amb"] & 4) == 0
            np.testing.assert_allclose(res.state.cpu().numpy()[zok], ref["F_next"][zok], atol=1e-5)
            _check_compaction(res, B)


def test_gate_state_pool_slots(lsg, orc, dev):
    """slots: exit state read from and written back into a pool in place
    (the index_select / index_copy_ of cdb_model_runner.py:94-109)."""
    g = torch.Generator(device=dev).manual_seed(3)
    B, H, cap = 100, 512, 300
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(H, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    pool = torch.rand(cap, generator=g, device=dev) * 0.3
    slots = torch.randperm(cap, generator=g, device=dev)[:B].to(torch.int32)
    before = pool.clone()
    gate = lsg.OuroExitGate(w, None, exit_threshold=0.3)
    res = gate.exit_signal_compact(h, None, 2, slots=slots, state_pool=pool)
    ref = orc.exit_gate(_arr(orc, h), _arr(orc, w), None, before[slots.long()].cpu().numpy(), 2, 0.3,
                        dtype=orc.BF16)
    np.testing.assert_allclose(pool[slots.long()].cpu().numpy(), ref["F_next"], atol=1e-5)
    untouched = torch.ones(cap, dtype=torch.bool, device=dev)
    untouched[slots.long()] = False
    assert torch.equal(pool[untouched], before[untouched])
    _check_compaction(res, B)


def test_workspace_reuse(lsg, dev):
    """One workspace serves back-to-back calls of any size up to max_batch
    (a smaller batch after a larger one reads no stale counts); each call
    advances the serial number kept in its first word."""
    g = torch.Generator(device=dev).manual_seed(12)
    w = (torch.randn(256, generator=g, device=dev) * 0.2).to(torch.bfloat16)
    gate = lsg.OuroExitGate(w, None, exit_threshold=0.5, max_batch=5000)
    sizes = (5000, 37, 4096, 1, 0, 300)
    for B in sizes:
        h = torch.randn(B, 256, generator=g, device=dev).to(torch.bfloat16)
        F = torch.rand(B, generator=g, device=dev)
        res = gate.exit_signal_compact(h, F, 1)
        _check_compaction(res, B)
    serial = gate._ws.buf[:4].cpu().numpy().view(np.uint32)[0]
    flags = gate._ws.buf[4:8].cpu().numpy().view(np.uint32)[0]
    assert serial == len(sizes) and flags == 0
    with pytest.raises(ValueError, match="max_batch"):
        gate.exit_signal_compact(torch.zeros(5001, 256, device=dev, dtype=torch.bfloat16), None, 1)


def test_gate_graph_replay_compact(lsg, dev):
    """exit_signal_compact captured in a HIP graph: every replay is exact."""
    g = torch.Generator(device=dev).manual_seed(13)
    B, H = 700, 2048
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn(H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    gate = lsg.OuroExitGate(w, torch.tensor([-1.0], device=dev).to(torch.bfloat16), exit_threshold=0.3)
    F = torch.rand(B, generator=g, device=dev) * 0.4
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gate.exit_signal_compact(h, F, 1)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        cap = gate.exit_signal_compact(h, F, 1)
    for i in range(4):
        eager = gate.exit_signal_compact(h, F, 1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(cap.signal, eager.signal)
        assert torch.equal(cap.n_exit, eager.n_exit)
        n = int(eager.n_exit.item())
        assert torch.equal(cap.exit_idx[:n], eager.exit_idx[:n])
        assert torch.equal(cap.keep_idx[: B - n], eager.keep_idx[: B - n])
        F.copy_(torch.rand(B, generator=g, device=dev) * 0.4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_sigmoid_exhaustive(lsg, orc, dev, dtype):
    """lambda = 1 / (1 + exp(-z)) in float32 for every finite bf16 / fp16 z, and
    the three-op recurrence: bit-exact against the oracle (which is pinned to
    the float32 formula with a correctly rounded exp)."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(dtype)
    z = bits.float()
    keep = torch.isfinite(z)
    z = bits[keep].contiguous()
    F0 = torch.zeros(z.numel())
    F1 = torch.rand(z.numel(), generator=torch.Generator().manual_seed(1))
    for F in (F0, F1):
        got = lsg.cumulative_exit_probability(z.to(dev), F.to(dev)).cpu().numpy()
        want = orc.cumulative_exit_probability(z.float().numpy(), F.numpy())
        assert np.array_equal(got, want)


def _route_trace(lsg, orc, dev, direct: bool, seed: int, steps: int = 40, n_slots: int = 24):
    """Drive exit_route through a multi-step trace and the scheduler restatement
    side by side: random batches (tokens skip core steps), random requests,
    replay depths, successors taking exited tokens' slots, cancellations."""
    rng = np.random.default_rng(seed)
    max_depth = 4
    gate = lsg.OuroExitGate(torch.ones(1, dtype=torch.bfloat16, device=dev), None, exit_threshold=0.5,
                            loop_steps=max_depth, max_batch=n_slots)
    pending = gate.init_pending_pool(n_slots)
    router = orc.CdbRouter(max_depth=max_depth, disable_lookahead_exit=direct)
    gen = [0] * n_slots
    tokens = {}

    def admit(slot):
        gen[slot] += 1
        rp = int(rng.integers(1, max_depth + 1)) if rng.random() < 0.3 else None
        t = orc.Token((slot, gen[slot]), slot, 0, rp)
        tokens[slot] = t
        router.add(t)

    for s in range(n_slots):
        admit(s)
    routed_total = 0
    for step in range(steps):
        if rng.random() < 0.1:  # cancellation: the host clears the slot's pending gate
            s = int(rng.integers(n_slots))
            router.cancel(tokens[s].ident)
            pending[s] = 0
            admit(s)
        live = {t.ident: t for t in router.core}
        batch = [t for t in router.core if rng.random() < 0.8]
        if not batch:
            continue
        rng.shuffle(batch)
        req = rng.random(len(batch)) < 0.3
        z = torch.tensor(np.where(req, 3.0, -3.0), dtype=torch.bfloat16, device=dev).reshape(-1, 1)
        slots = torch.tensor([t.slot for t in batch], dtype=torch.int32, device=dev)
        depth = torch.tensor([t.depth for t in batch], dtype=torch.int32, device=dev)
        replay = torch.tensor([t.replay or 0 for t in batch], dtype=torch.int32, device=dev)
        pool = torch.zeros(n_slots, dtype=torch.float32, device=dev)
        res = gate.exit_route(z, None, depth, pending=pending, disable_lookahead_exit=direct,
                              slots=slots, state_pool=pool, max_depth=max_depth, replay_depth=replay)
        want = router.core_step([t.ident for t in batch], list(req))
        got_rows = np.nonzero(res.route.cpu().numpy())[0]
        got = sorted(batch[i].ident for i in got_rows)
        assert got == sorted(want), (step, got, want)
        assert np.array_equal(res.signal.cpu().numpy(), req)
        n = int(res.n_exit.item())
        assert n == len(got_rows)
        assert np.array_equal(res.exit_idx[:n].cpu().numpy(), got_rows)
        assert np.array_equal(res.keep_idx[: len(batch) - n].cpu().numpy(),
                              np.nonzero(~res.route.cpu().numpy())[0])
        for ident in want:
            admit(live[ident].slot)
        routed_total += n
    return routed_total


@pytest.mark.parametrize("direct", [False, True])
def test_route_trace_matches_scheduler(lsg, orc, dev, direct):
    """f2: on-device routing under the scheduler's default (lookahead) timing
    and under --disable-lookahead-exit, against the CPU restatement of
    CDBScheduler._run_core / _consume_gate (cdb_scheduler.py:189-229,254-266)."""
    total = sum(_route_trace(lsg, orc, dev, direct, seed) for seed in range(4))
    assert total > 20


@pytest.mark.parametrize("direct", [False, True])
def test_route_replay_kat(lsg, dev, direct):
    """tests/core/test_scheduler.py:65-78 on the device: a token whose replay
    depth is two is routed at depth two under either timing, and a replacement
    token moved into the same slot (pending entry zeroed) is not routed by the
    old token's gate."""
    gate = lsg.OuroExitGate(torch.ones(1, dtype=torch.bfloat16, device=dev), None, exit_threshold=0.5,
                            loop_steps=4, max_batch=4)
    pending = gate.init_pending_pool(1)
    slots = torch.zeros(1, dtype=torch.int32, device=dev)
    pool = torch.zeros(1, dtype=torch.float32, device=dev)
    h = torch.full((1, 1), -3.0, dtype=torch.bfloat16, device=dev)  # the gate itself never asks
    replay = torch.full((1,), 2, dtype=torch.int32, device=dev)
    routed_at = None
    for depth in range(4):
        r = gate.exit_route(h, None, torch.full((1,), depth, dtype=torch.int32, device=dev),
                            pending=pending, disable_lookahead_exit=direct, slots=slots, state_pool=pool,
                            max_depth=4, replay_depth=replay)
        if r.route.item():
            routed_at = depth + 1
            break
    assert routed_at == 2
    # the old token asked for an exit at depth 1 (lookahead record); a replacement
    # takes slot 0 and the host zeroes its pending entry
    r = gate.exit_route(h, None, torch.zeros(1, dtype=torch.int32, device=dev), pending=pending,
                        disable_lookahead_exit=direct, slots=slots, state_pool=pool, max_depth=4,
                        replay_depth=replay)
    pending.zero_()
    r = gate.exit_route(h, None, torch.ones(1, dtype=torch.int32, device=dev), pending=pending,
                        disable_lookahead_exit=direct, slots=slots, state_pool=pool, max_depth=4)
    assert not r.route.item()


def test_first_gate_call_inside_capture(lsg, dev):
    """The gates build their workspaces at construction: the very first call of
    exit_signal_compact / exit_route / the Huginn compaction can be captured,
    and every replay matches an eager call made between replays."""
    g = torch.Generator(device=dev).manual_seed(31)
    B, H = 300, 512
    h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
    hp = (h.float() + 0.2 * torch.randn(B, H, generator=g, device=dev)).to(torch.bfloat16)
    w = (torch.randn(H, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    F = torch.rand(B, generator=g, device=dev) * 0.5
    ouro = lsg.OuroExitGate(w, None, exit_threshold=0.4, max_batch=B)
    router = lsg.OuroExitGate(w, None, exit_threshold=0.4, max_batch=B)
    eager_router = lsg.OuroExitGate(w, None, exit_threshold=0.4, max_batch=B)
    huginn = lsg.HuginnExitGate(exit_threshold=0.2, max_batch=B, device=dev)
    pend, pend_e = router.init_pending_pool(B), eager_router.init_pending_pool(B)
    ls = torch.full((B,), 1, dtype=torch.int32, device=dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        c1 = ouro.exit_signal_compact(h, F, 1)
        c2 = router.exit_route(h, F, ls, pending=pend, max_depth=3)
        c3 = huginn.exit_signal_compact(h, hp, 0)
    torch.cuda.synchronize()
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        e1 = ouro.exit_signal_compact(h, F, 1)
        e2 = eager_router.exit_route(h, F, ls, pending=pend_e, max_depth=3)
        e3 = huginn.exit_signal_compact(h, hp, 0)
        torch.cuda.synchronize()
        for c, e in ((c1, e1), (c2, e2), (c3, e3)):
            n = int(e.n_exit.item())
            assert torch.equal(c.signal, e.signal) and torch.equal(c.n_exit, e.n_exit)
            assert torch.equal(c.exit_idx[:n], e.exit_idx[:n])
            assert torch.equal(c.keep_idx[: B - n], e.keep_idx[: B - n])
        assert torch.equal(c2.route, e2.route) and torch.equal(pend, pend_e)
        assert i > 0 or int(e2.n_exit.item()) == 0  # lookahead: nothing pending at the first step
        ls.add_(1).clamp_(max=2)


def test_integration_binds_reference_fields(lsg, orc, dev):
    """integration.ouro_exit_signal on an object shaped like the reference's
    OuroModel (tests/core/test_exit_gates.py:18-22,76-84: early_exit_gate with
    weight/bias, loop_params.exit_threshold, _exit_gate_type, min_loop_steps),
    with a non-contiguous hidden view, against the oracle."""
    from types import SimpleNamespace

    g = torch.Generator(device=dev).manual_seed(41)
    B, H = 96, 2048
    wide = torch.randn(B, 2 * H, generator=g, device=dev).to(torch.bfloat16)
    hidden = wide[:, ::2]  # stride(1) == 2
    assert hidden.stride(1) != 1
    gate = SimpleNamespace(weight=(torch.randn(1, H, generator=g, device=dev) * 0.03).to(torch.bfloat16),
                           bias=torch.tensor([-0.5], device=dev).to(torch.bfloat16))
    for kind, min_steps in (("early_exit", 1), ("lookahead", 3)):
        model = SimpleNamespace(early_exit_gate=gate, min_loop_steps=min_steps, _exit_gate_type=kind,
                                loop_params=SimpleNamespace(loop_steps=4, exit_threshold=0.3))
        F = torch.rand(B, generator=g, device=dev) * 0.3
        signal, state = lsg.integration.ouro_exit_signal(model, hidden, F, 1)
        assert signal.dtype == torch.bool and state.dtype == torch.float32
        ref = orc.exit_gate(_arr(orc, hidden.contiguous()), _arr(orc, gate.weight.reshape(-1)),
                            _arr(orc, gate.bias), F.cpu().numpy(), 1, 0.3, min_loop_steps=min_steps,
                            lookahead=kind == "lookahead", dtype=orc.BF16)
        clean = (ref["amb"] & 1) == 0
        assert np.array_equal(signal.cpu().numpy()[clean], ref["mask"][clean].astype(bool))
        zok = (ref["amb"] & 4) == 0
        np.testing.assert_allclose(state.cpu().numpy()[zok], ref["F_next"][zok], atol=1e-5)
    # the Huginn binding reads loop_params.exit_threshold
    hmodel = SimpleNamespace(loop_params=SimpleNamespace(loop_steps=4, exit_threshold=0.5))
    prev = torch.tensor([[0, 0], [1, 0], [-1, -1], [1, 1]], dtype=torch.bfloat16, device=dev)
    cur = torch.tensor([[0, 0], [2, 0], [1, 1], [1, 1]], dtype=torch.bfloat16, device=dev)
    sig, st = lsg.integration.huginn_exit_signal(hmodel, cur, prev, 0)
    assert sig.tolist() == [True, False, False, True] and st is cur
    # a gate without a weight (the reference KAT's lambda gate) is refused loudly
    with pytest.raises(TypeError):
        lsg.integration.ouro_exit_signal(
            SimpleNamespace(early_exit_gate=SimpleNamespace(forward=lambda x: x[:, :1]), min_loop_steps=1,
                            _exit_gate_type="early_exit", loop_params=SimpleNamespace(exit_threshold=0.5)),
            hidden, F, 0)


def test_huginn_kat_and_parity(lsg, orc, dev):
    """Mirror of tests/core/test_exit_gates.py:39-60 and parity of the ratio."""
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        gate = lsg.HuginnExitGate(exit_threshold=0.5)
        previous = torch.tensor([[0, 0], [1, 0], [-1, -1], [1, 1]], dtype=dtype, device=dev)
        current = torch.tensor([[0, 0], [2, 0], [1, 1], [1, 1]], dtype=dtype, device=dev)
        initial = gate.init_exit_state(previous)
        assert initial is previous
        signal, state = gate.exit_signal(current, initial, 0)
        assert signal.dtype == torch.bool and signal.tolist() == [True, False, False, True]
        assert state is current
        res = gate.exit_signal_compact(current, previous, 0)
        assert res.exit_idx[: int(res.n_exit.item())].tolist() == [0, 3]
    g = torch.Generator(device=dev).manual_seed(21)
    h = torch.randn(256, 5280, generator=g, device=dev).to(torch.bfloat16)
    hp = (h.float() + 0.3 * torch.randn(256, 5280, generator=g, device=dev)).to(torch.bfloat16)
    ratio = lsg.relative_state_change(h, hp)
    want, _, _ = orc.relative_state_change(_arr(orc, h), _arr(orc, hp), 0.3, dtype=orc.BF16)
    np.testing.assert_allclose(ratio.cpu().numpy(), want, rtol=1e-5)
    ref_torch = (h.float() - hp.float()).norm(dim=-1) / h.float().norm(dim=-1).clamp_min(1e-9)
    np.testing.assert_allclose(ratio.cpu().numpy(), ref_torch.cpu().numpy(), rtol=1e-5)


def test_empty_batch(lsg, dev):
    gate = lsg.OuroExitGate(torch.ones(16, device=dev, dtype=torch.bfloat16), None, exit_threshold=0.5)
    h = torch.empty(0, 16, device=dev, dtype=torch.bfloat16)
    res = gate.exit_signal_compact(h, None, 0)
    assert int(res.n_exit.item()) == 0
