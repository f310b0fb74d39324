"""lsg_exit_gate_noalloc (static device workspace) against lsg_exit_gate with a
caller-provided workspace, through the C ABI: identical outputs on two calls
in a row, the second with fewer rows."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _gate_call(lsg, fn, h, w, b, F, ls, ws):
    L = lsg._lib.load()
    B, H = h.shape
    dev = h.device
    out = dict(F_next=torch.empty(B, dtype=torch.float32, device=dev),
               mask=torch.empty(B, dtype=torch.uint8, device=dev),
               exit_idx=torch.full((B,), -7, dtype=torch.int32, device=dev),
               keep_idx=torch.full((B,), -7, dtype=torch.int32, device=dev),
               n_exit=torch.full((1,), -7, dtype=torch.int32, device=dev),
               z=torch.empty(B, dtype=torch.float32, device=dev))
    p = lsg._lib.ptr
    args = [p(h), lsg._lib.DTYPE_BF16, B, H, h.stride(0), p(w), p(b), p(F), p(out["F_next"]), None,
            p(ls), 0, 0.3, 2, 0, 4, p(out["mask"]), p(out["exit_idx"]), p(out["keep_idx"]),
            p(out["n_exit"]), p(out["z"])]
    if fn == "lsg_exit_gate":
        args += [p(ws), ws.numel()]
    rc = getattr(L, fn)(*args, lsg._lib.stream_of(h))
    lsg._lib.check(rc, fn)
    return out


def test_noalloc_matches_workspace_entry_point(lsg, dev):
    g = torch.Generator(device=dev).manual_seed(77)
    H = 2048
    w = (torch.randn(H, generator=g, device=dev) * 0.03).to(torch.bfloat16)
    b = torch.tensor([-1.0], device=dev).to(torch.bfloat16)
    L = lsg._lib.load()
    ws = torch.zeros(int(L.lsg_workspace_bytes(1, 4096)), dtype=torch.uint8, device=dev)
    for B in (3000, 700):
        print(f"lsg_exit_gate_noalloc B={B} H={H}", flush=True)
        h = torch.randn(B, H, generator=g, device=dev).to(torch.bfloat16)
        F = torch.rand(B, generator=g, device=dev) * 0.4
        ls = torch.randint(0, 4, (B,), generator=g, device=dev, dtype=torch.int32)
        want = _gate_call(lsg, "lsg_exit_gate", h, w, b, F, ls, ws)
        got = _gate_call(lsg, "lsg_exit_gate_noalloc", h, w, b, F, ls, None)
        torch.cuda.synchronize()
        n = int(want["n_exit"].item())
        assert 0 < n < B
        assert int(got["n_exit"].item()) == n
        for k in ("F_next", "mask", "z"):
            assert torch.equal(got[k], want[k]), k
        assert torch.equal(got["exit_idx"][:n], want["exit_idx"][:n])
        assert torch.equal(got["keep_idx"][: B - n], want["keep_idx"][: B - n])
        m = want["mask"].cpu().numpy().astype(bool)
        assert np.array_equal(got["exit_idx"][:n].cpu().numpy(), np.nonzero(m)[0])


def test_noalloc_rejects_oversize(lsg):
    L = lsg._lib.load()
    rc = L.lsg_exit_gate_noalloc(ctypes.c_void_p(16), 1, 65537, 16, 16, ctypes.c_void_p(16), None, None,
                                 ctypes.c_void_p(16), None, None, 0, 0.5, 1, 0, 0, ctypes.c_void_p(16),
                                 None, None, ctypes.c_void_p(16), None, None)
    assert rc == 1 and b"65536" in L.lsg_last_error()
