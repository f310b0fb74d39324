"""Host-side logic and the C ABI boundary (CPU only; no kernel launches)."""
from __future__ import annotations

import ctypes
import os
import re
from types import SimpleNamespace

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


# -------------------------------------------------------- Sampler.prepare ----
def _prepare(lsg, monkeypatch, params, vocab=100):
    import loop_sglang_amd.sampler as sampler_mod

    monkeypatch.setattr(sampler_mod, "make_device_tensor",
                        lambda data, dtype, device: torch.tensor(data, dtype=dtype))
    s = lsg.Sampler(torch.device("cpu"), vocab)
    return s.prepare(SimpleNamespace(reqs=[SimpleNamespace(sampling_params=p) for p in params]))


def test_prepare_all_greedy(lsg, monkeypatch, SP):
    args = _prepare(lsg, monkeypatch, [SP(), SP(temperature=0.5, top_k=1)])
    assert args.temperatures is None and args.top_k is not None and args.top_p is None
    assert args.top_k.tolist() == [100, 1]


def test_prepare_mixed(lsg, monkeypatch, SP):
    """sample.py:89-105: greedy rows get T = 1e-6 once any row samples; k < 1
    becomes V; tensors are None when neutral for every row."""
    args = _prepare(lsg, monkeypatch, [SP(), SP(temperature=0.8), SP(temperature=1.2, top_p=0.9),
                                       SP(temperature=0.5, top_k=7)])
    assert torch.allclose(args.temperatures, torch.tensor([1e-6, 0.8, 1.2, 0.5]))
    assert args.top_k.tolist() == [100, 100, 100, 7]
    assert torch.allclose(args.top_p, torch.tensor([1.0, 1.0, 0.9, 1.0]))
    args = _prepare(lsg, monkeypatch, [SP(temperature=0.8), SP(temperature=0.9)])
    assert args.top_k is None and args.top_p is None


def test_filter_and_merge(lsg):
    """sample.py:20-53: filter keeps rows; merge fills defaults 1e-6 / V / 1.0."""
    A = lsg.BatchSamplingArgs(torch.tensor([0.5, 0.6, 0.7]), torch.tensor([1, 2, 3], dtype=torch.int32), None,
                              torch.tensor([0.1, 0.2, 0.3]))
    f = A.filter_batch(torch.tensor([2, 0]), False, need_top_k=True, need_top_p=False)
    assert f.temperatures.tolist() == pytest.approx([0.7, 0.5]) and f.top_k.tolist() == [3, 1]
    assert f.uniforms.tolist() == pytest.approx([0.3, 0.1])
    f = A.filter_batch(torch.tensor([1]), True, need_top_k=False, need_top_p=False)
    assert f.temperatures is None and f.top_k is None
    Bb = lsg.BatchSamplingArgs(None, None, torch.tensor([0.9, 0.8]))
    m = A.merge_batch(Bb, 3, 2, 50)
    assert m.temperatures.tolist() == pytest.approx([0.5, 0.6, 0.7, 1e-6, 1e-6])
    assert m.top_k.tolist() == [1, 2, 3, 50, 50]
    assert m.top_p.tolist() == pytest.approx([1.0, 1.0, 1.0, 0.9, 0.8])
    assert m.uniforms is None  # only one side carried uniforms: drawn at sample time
    assert lsg.BatchSamplingArgs(None).merge_batch(lsg.BatchSamplingArgs(None), 1, 1, 9).temperatures is None


def test_gate_argument_validation(lsg):
    """ouro.py:63-72,85-87 / huginn.py:96-98 argument rules."""
    w = torch.ones(4)
    with pytest.raises(ValueError):
        lsg.OuroExitGate(w, None, exit_threshold=0.0)
    with pytest.raises(ValueError):
        lsg.OuroExitGate(w, None, exit_threshold=1.5)
    with pytest.raises(ValueError):
        lsg.OuroExitGate(w, None, exit_threshold=0.5, min_loop_steps=5, loop_steps=4)
    with pytest.raises(ValueError):
        lsg.OuroExitGate(w, None, exit_threshold=0.5, exit_gate_type="other")
    with pytest.raises(ValueError):
        lsg.HuginnExitGate(exit_threshold=-1.0)
    gate = lsg.OuroExitGate(w, None, exit_threshold=0.5)
    with pytest.raises(ValueError):  # CPU tensors: the product path has no CPU fallback
        gate.exit_signal(torch.zeros(2, 4), torch.zeros(2), 0)
    with pytest.raises(ValueError):
        lsg.sample_rows(torch.zeros(2, 4), None, None, None, None)


# ---------------------------------------------------------------- C ABI ------
def _header_functions():
    text = open(os.path.join(ROOT, "include", "loopsgl_tok.h")).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(lsg_\w+)\(", text, flags=re.M)))


def test_capi_exports_every_declared_symbol(lsg):
    """The shared library loads and exports every function include/ declares."""
    from loop_sglang_amd import _lib

    L = _lib.load()
    names = _header_functions()
    assert set(names) == set(_lib.SIGNATURES), names
    for name in names:
        assert hasattr(L, name), name
    assert L.lsg_version() == 1


def test_capi_argument_errors_without_gpu(lsg):
    """Invalid arguments are rejected before any HIP call, with a message."""
    from loop_sglang_amd import _lib

    L = _lib.load()
    rc = L.lsg_sample(None, 0, 1, 10, 10, None, None, None, None, None, 1, None, None, None)
    assert rc == 1 and b"null" in L.lsg_last_error()
    rc = L.lsg_sample(ctypes.c_void_p(16), 0, 4, 10, 5, None, None, None, None, None, 4, None,
                      ctypes.c_void_p(16), None)
    assert rc == 1 and b"bad shape" in L.lsg_last_error()
    rc = L.lsg_sample(ctypes.c_void_p(16), 0, 4, 10, 10, ctypes.c_void_p(16), None, None, None, None, 4,
                      None, ctypes.c_void_p(16), None)
    assert rc == 1 and b"uniforms" in L.lsg_last_error()
    rc = L.lsg_sample(ctypes.c_void_p(16), 9, 4, 10, 10, None, None, None, None, None, 4, None,
                      ctypes.c_void_p(16), None)
    assert rc == 1 and b"dtype" in L.lsg_last_error()
    # serial number page + one 64-bit word per four rows, padded to 256 B
    assert L.lsg_workspace_bytes(1, 512) == 256 + 1024
    assert L.lsg_workspace_bytes(1, 100000) == 256 + ((100000 + 3) // 4 * 8 + 255) // 256 * 256
    assert L.lsg_workspace_bytes(7, 10) == 0
    rc = L.lsg_exit_gate(ctypes.c_void_p(16), 1, 8, 16, 16, ctypes.c_void_p(16), None, None,
                         ctypes.c_void_p(16), None, None, 0, 0.5, 1, 0, 0, ctypes.c_void_p(16),
                         ctypes.c_void_p(16), None, None, None, None, 0, None)
    assert rc == 3 and b"workspace" in L.lsg_last_error()
    rc = L.lsg_exit_gate(None, 1, 8, 16, 16, None, None, None, None, None, None, 0, 0.5, 1, 0, 0,
                         None, None, None, None, None, None, 0, None)
    assert rc == 1
    # lookahead routing needs the pending-gate pool, then a workspace
    rc = L.lsg_exit_gate_route(ctypes.c_void_p(16), 1, 8, 16, 16, ctypes.c_void_p(16), None, None,
                               ctypes.c_void_p(16), None, None, 0, 0.5, 1, 0, 0, 0, None, None,
                               ctypes.c_void_p(16), None, None, None, None, None, None, 0, None)
    assert rc == 1 and b"pending" in L.lsg_last_error()
    rc = L.lsg_exit_gate_route(ctypes.c_void_p(16), 1, 8, 16, 16, ctypes.c_void_p(16), None, None,
                               ctypes.c_void_p(16), None, None, 0, 0.5, 1, 0, 0, 0, ctypes.c_void_p(16),
                               None, ctypes.c_void_p(16), None, None, None, None, None, None, 0, None)
    assert rc == 3 and b"workspace" in L.lsg_last_error()
