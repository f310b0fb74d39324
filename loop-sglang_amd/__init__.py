"""MI355X-native (gfx950) decode token path of Loop-SGLang.

Host-side mirror of the reference interfaces for this path, driving the HIP
kernels in ``libloopsgl_tok.so`` (C ABI: include/loopsgl_tok.h):

  sampler      Sampler / BatchSamplingArgs / sample_impl  (model_executor/sample.py)
  exit_gate    OuroExitGate / HuginnExitGate / cumulative_exit_probability /
               relative_state_change                     (models/looped/*.py)
  decode_step  gate -> on-device exit compaction -> sampling of exited rows
  core         SamplingParams / LoopParams               (core.py)

The directory name contains a hyphen, so import it through
``__graft_entry__.package()`` (registers it as ``loop_sglang_amd``).
"""
from .core import LoopParams, SamplingParams
from .decode_step import DecodeStepResult, cdb_decode_step
from .exit_gate import (
    GateResult,
    HuginnExitGate,
    OuroExitGate,
    cumulative_exit_probability,
    relative_state_change,
)
from .sampler import BatchSamplingArgs, Sampler, make_device_tensor, sample_impl, sample_rows
from . import workloads

__all__ = [
    "BatchSamplingArgs", "DecodeStepResult", "GateResult", "HuginnExitGate", "LoopParams",
    "OuroExitGate", "Sampler", "SamplingParams", "cdb_decode_step", "cumulative_exit_probability",
    "make_device_tensor", "relative_state_change", "sample_impl", "sample_rows",
]
