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
    """The compaction workspace is left zero-filled: back-to-back calls with a
    smaller batch stay exact."""
    g = torch.Generator(device=dev).manual_seed(12)
    w = (torch.randn(256, generator=g, device=dev) * 0.2).to(torch.bfloat16)
    gate = lsg.OuroExitGate(w, None, exit_threshold=0.5)
    for B in (5000, 37, 4096, 1):
        h = torch.randn(B, 256, generator=g, device=dev).to(torch.bfloat16)
        F = torch.rand(B, generator=g, device=dev)
        res = gate.exit_signal_compact(h, F, 1)
        _check_compaction(res, B)
    ws = gate._ws.buf[dev]
    torch.cuda.synchronize()
    assert int(ws.sum().item()) == 0


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


def test_sigmoid_exhaustive_bf16(lsg, orc, dev):
    """lambda = float32(sigmoid(z)) for every finite bf16 z, and the
    three-op recurrence: bit-exact against the oracle."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    z = bits.float()
    keep = torch.isfinite(z)
    z = bits[keep].contiguous()
    F0 = torch.zeros(z.numel())
    F1 = torch.rand(z.numel(), generator=torch.Generator().manual_seed(1))
    for F in (F0, F1):
        got = lsg.cumulative_exit_probability(z.to(dev), F.to(dev)).cpu().numpy()
        want = orc.cumulative_exit_probability(z.float().numpy(), F.numpy())
        assert np.array_equal(got, want)


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
