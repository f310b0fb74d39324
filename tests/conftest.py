"""Shared fixtures.  GPU tests are marked ``gpu``; everything else runs on CPU."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def lsg():
    """The product package (loop-sglang_amd/)."""
    return __graft_entry__.package()


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (test infrastructure)."""
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def SP():
    """Stand-in for the engine's SamplingParams: the fields Sampler.prepare reads
    (temperature, top_k, top_p) and ``is_greedy`` as python/loopsgl/core.py:83-85
    defines it."""
    from dataclasses import dataclass

    @dataclass
    class SamplingParams:
        temperature: float = 0.0
        top_k: int = -1
        top_p: float = 1.0

        @property
        def is_greedy(self) -> bool:
            return (self.temperature <= 0.0 or self.top_k == 1) and self.top_p == 1.0

    return SamplingParams
