"""The fused CDB decode step (gate -> device compaction -> sampling of the
exited rows) against the oracle composed the same way."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _arr(orc, t):
    t = t.detach().cpu().contiguous()
    return t.numpy() if t.dtype == torch.float32 else orc.bf16_bits(t)


def test_mixed_depth_decode_step(lsg, orc, dev):
    """B=2048 rows at depths 1-4, fp32 logits V=65536, gate tau=0.2; exited rows
    sample with mixed greedy/top-k/top-p parameters."""
    wl = lsg.workloads.cdb_mixed_depth(dev)
    gate = lsg.OuroExitGate(wl["weight"], wl["bias"], exit_threshold=wl["tau"], loop_steps=4)
    args = lsg.BatchSamplingArgs(wl["temperatures"], wl["top_k"], wl["top_p"], wl["uniforms"])
    res = lsg.cdb_decode_step(gate, wl["hidden"], wl["F_prev"], wl["loop_step"], wl["logits"], args)
    torch.cuda.synchronize()
    B = wl["logits"].shape[0]
    ref = orc.exit_gate(_arr(orc, wl["hidden"]), _arr(orc, wl["weight"]), _arr(orc, wl["bias"]),
                        wl["F_prev"].cpu().numpy(), wl["loop_step"].cpu().numpy(), wl["tau"], dtype=orc.BF16)
    mask = res.signal.cpu().numpy()
    clean = (ref["amb"] & 1) == 0
    assert np.array_equal(mask[clean].astype(np.uint8), ref["mask"][clean])
    n = int(res.n_exit.item())
    exit_idx = res.exit_idx[:n].cpu().numpy()
    assert np.array_equal(exit_idx, np.nonzero(mask)[0])
    assert n > 0
    rows = exit_idx
    x = wl["logits"][torch.from_numpy(rows).to(dev).long()].cpu().numpy()
    sel = lambda t: t.cpu().numpy()[rows]
    want, amb, alt = orc.sample(x, sel(wl["temperatures"]), sel(wl["top_k"]), sel(wl["top_p"]),
                                sel(wl["uniforms"]), with_alt=True)
    got = res.token_ids[:n].cpu().numpy()
    # the oracle's id, the other kept set's draw on a top-p-ambiguous row, or
    # any id where the draw's CDF lies within 1e-6 of u
    excused = ((amb & 1) != 0) | (((amb & 2) != 0) & ((amb & 4) != 0))
    bad = (got != want) & ~(((amb & 2) != 0) & (got == alt)) & ~excused
    assert not bad.any(), np.nonzero(bad)
    print(f"[parity] exited rows {n}: top-p-ambiguous {int(((amb & 2) != 0).sum())}, excused {int(excused.sum())}")
    assert excused.sum() <= 3


def test_gate_then_greedy(lsg, dev):
    """The CDB gate workload: exited rows greedy-sampled from bf16 logits."""
    wl = lsg.workloads.gate_cdb(dev)
    gate = lsg.OuroExitGate(wl["weight"], wl["bias"], exit_threshold=wl["tau"], loop_steps=4)
    F = None
    for step, h in enumerate(wl["hidden"]):
        res = lsg.cdb_decode_step(gate, h, F, step, wl["logits"], lsg.BatchSamplingArgs(None))
        n = int(res.n_exit.item())
        rows = res.exit_idx[:n].long()
        want = torch.argmax(wl["logits"][rows], dim=-1).to(torch.int32)
        assert torch.equal(res.token_ids[:n], want)
        F = res.state


def test_lookahead_decode_steps(lsg, orc, dev):
    """Three core steps with the default lookahead routing: the rows sampled in
    a step are those whose previous-step request (or the depth cap) routes
    them, exactly the rows a second gate's exit_route sends out on the same
    inputs; their tokens match the oracle on those rows; nothing leaves at the
    first step (no request is pending yet)."""
    g = torch.Generator(device=dev).manual_seed(41)
    B, H, V = 384, 512, 8000
    w = (torch.randn(H, generator=g, device=dev) * 0.05).to(torch.bfloat16)
    b = torch.tensor([-0.5], device=dev).to(torch.bfloat16)
    gate = lsg.OuroExitGate(w, b, exit_threshold=0.4, loop_steps=4)
    twin = lsg.OuroExitGate(w, b, exit_threshold=0.4, loop_steps=4)
    pend, pend_t = gate.init_pending_pool(B), twin.init_pending_pool(B)
    logits = torch.randn(B, V, generator=g, device=dev) * 2
    args = lsg.BatchSamplingArgs(torch.full((B,), 0.7, device=dev), None, torch.full((B,), 0.9, device=dev),
                                 torch.rand(B, generator=g, device=dev))
    F = F_t = None
    for step in range(3):
        h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
        res = lsg.cdb_decode_step(gate, h, F, step, logits, args, max_depth=3, pending=pend)
        ref = twin.exit_route(h, F_t, step, pending=pend_t, max_depth=3)
        n = int(res.n_exit.item())
        assert n == int(ref.n_exit.item())
        assert torch.equal(res.exit_idx[:n], ref.exit_idx[:n])
        assert torch.equal(res.route, ref.route)
        if step == 0:
            assert n == 0
        if n:
            rows = res.exit_idx[:n].long()
            x = logits[rows].cpu().numpy()
            sel = lambda t: t[rows].cpu().numpy()
            want, amb, alt = orc.sample(x, sel(args.temperatures), None, sel(args.top_p), sel(args.uniforms),
                                        with_alt=True)
            got = res.token_ids[:n].cpu().numpy()
            excused = ((amb & 1) != 0) | (((amb & 2) != 0) & ((amb & 4) != 0))
            ok = (got == want) | (((amb & 2) != 0) & (got == alt)) | excused
            assert ok.all() and excused.sum() <= 2
        F, F_t = res.state, ref.state
    assert n > 0  # rows routed by the previous steps' requests or the depth cap
