"""Sampling and loop parameters of a request.

Mirrors the argument semantics of python/loopsgl/core.py:18-85
(``LoopParams`` and the sampling fields of ``SamplingParams``: defaults,
``verify`` and ``is_greedy``).  Request-lifecycle fields that do not reach the
token path (stop strings, detokenisation flags) are out of scope here.
"""
from __future__ import annotations

from dataclasses import dataclass
from math import isfinite
from typing import List


@dataclass(frozen=True)
class LoopParams:
    """core.py:18-29."""

    loop_steps: int | None = None
    exit_threshold: float | None = None

    def __post_init__(self) -> None:
        if self.loop_steps is not None and (
            isinstance(self.loop_steps, bool)
            or not isinstance(self.loop_steps, int)
            or self.loop_steps <= 0
        ):
            raise ValueError("loop_steps must be a positive integer")


@dataclass
class SamplingParams:
    """Sampling fields of core.py:32-85 (defaults: greedy, top-k and top-p off)."""

    temperature: float = 0.0
    top_k: int = -1
    top_p: float = 1.0
    ignore_eos: bool = False
    max_tokens: int = 1024
    replay_exit_depths: List[int] | None = None

    def verify(self) -> None:
        """Reject unsupported sampling values before dispatching model work (core.py:54-81)."""
        if (
            isinstance(self.temperature, bool)
            or not isinstance(self.temperature, (int, float))
            or not isfinite(self.temperature)
            or self.temperature < 0
        ):
            raise ValueError("temperature must be a nonnegative finite number.")
        if (
            isinstance(self.top_p, bool)
            or not isinstance(self.top_p, (int, float))
            or not isfinite(self.top_p)
            or not 0 < self.top_p <= 1
        ):
            raise ValueError("top_p must be in (0, 1].")
        if (
            isinstance(self.top_k, bool)
            or not isinstance(self.top_k, int)
            or (self.top_k != -1 and self.top_k < 1)
        ):
            raise ValueError("top_k must be -1 (disable) or a positive integer.")
        if (
            isinstance(self.max_tokens, bool)
            or not isinstance(self.max_tokens, int)
            or self.max_tokens < 1
        ):
            raise ValueError("max_tokens must be a positive integer.")

    @property
    def is_greedy(self) -> bool:
        """core.py:83-85."""
        return (self.temperature <= 0.0 or self.top_k == 1) and self.top_p == 1.0
