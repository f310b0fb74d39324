"""Bindings of the HIP decode token path to the reference's own objects.

Each function is the body a maintainer assigns over the reference method it
names; it reads that object's own attributes, so nothing else in the engine
changes:

  ouro_exit_signal    OuroModel.exit_signal    python/loopsgl/models/looped/ouro.py:142-155
      reads ``early_exit_gate.weight`` / ``.bias`` (ouro.py:84, a LinearReplicated),
      ``loop_params.exit_threshold`` (looped/base.py:32), ``_exit_gate_type``
      (ouro.py:85) and ``min_loop_steps`` (ouro.py:66)
  huginn_exit_signal  HuginnModel.exit_signal  models/looped/huginn.py:184-194
      reads ``loop_params.exit_threshold``
  sampler_sample      Sampler.sample           model_executor/sample.py:107-112
      reads ``args.temperatures`` / ``.top_k`` / ``.top_p`` (sample.py:14-18)

Hidden states whose last dimension is not contiguous are copied to a
contiguous tensor first (the kernels read rows with unit element stride).
"""
from __future__ import annotations

import torch

from . import _lib
from .exit_gate import ouro_exit_signal as _ouro_exit_signal
from .exit_gate import _rel_change
from .sampler import sample_rows


def ouro_exit_signal(model, hidden_states: torch.Tensor, exit_state: torch.Tensor,
                     loop_step: int | torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """OuroModel.exit_signal on the fused HIP gate: (signal bool[B], F' f32[B])."""
    gate = model.early_exit_gate
    weight = getattr(gate, "weight", None)
    if weight is None:
        raise TypeError("early_exit_gate has no weight: the fused gate needs the linear layer's "
                        "weight [1, H] (and bias [1])")
    h = hidden_states if hidden_states.stride(-1) == 1 else hidden_states.contiguous()
    return _ouro_exit_signal(h, weight, getattr(gate, "bias", None), exit_state, loop_step,
                             exit_threshold=model.loop_params.exit_threshold,
                             min_loop_steps=model.min_loop_steps,
                             exit_gate_type=model._exit_gate_type)


def huginn_exit_signal(model, hidden_states: torch.Tensor, exit_state: torch.Tensor,
                       loop_step: int | torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """HuginnModel.exit_signal: (relative change < threshold, hidden_states)."""
    _, mask = _rel_change(hidden_states, exit_state, float(model.loop_params.exit_threshold), 1e-9, None)
    return mask, hidden_states


def sampler_sample(sampler, logits: torch.Tensor, args,
                   generator: torch.Generator | None = None) -> torch.Tensor:
    """Sampler.sample: argmax rows when ``args.temperatures`` is None, otherwise
    softmax(logits / T) filtered by top-k then top-p and drawn with one uniform
    per row (``args.uniforms`` when the args carry them, else torch.rand).
    Returns int32 ids (the cast of model_runner.py:279-280 is folded in)."""
    if args.temperatures is None:
        return sample_rows(logits, None, None, None, None)
    uniforms = getattr(args, "uniforms", None)
    if uniforms is None:
        _lib.require_gpu(logits, "logits")
        uniforms = torch.rand(logits.shape[0], device=logits.device, generator=generator)
    return sample_rows(logits, args.temperatures, args.top_k, args.top_p, uniforms)
