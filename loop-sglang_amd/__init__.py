"""MI355X-native (gfx950) decode token path of Loop-SGLang.

Host-side mirror of the reference interfaces for this path, driving the HIP
kernels in ``libloopsgl_tok.so`` (C ABI: include/loopsgl_tok.h):

  sampler      Sampler / BatchSamplingArgs / sample_impl  (model_executor/sample.py)
  exit_gate    OuroExitGate / HuginnExitGate / cumulative_exit_probability /
               relative_state_change                     (models/looped/*.py)
               OuroExitGate.exit_route: the scheduler's exit routing
                                                          (managers/cdb_scheduler.py)
  integration  exit_signal / sample bindings for the reference's own model
               and sampler objects
  decode_step  gate -> on-device exit compaction -> sampling of exited rows
  coda         lm_head / coda_sample: the vocabulary projection (MFMA) and the
               token step without an fp32 logits buffer (layers/embedding.py)

The directory name contains a hyphen, so import it through
``__graft_entry__.package()`` (registers it as ``loop_sglang_amd``).
"""
from .decode_step import DecodeStepResult, cdb_decode_step
from .exit_gate import (
    GateResult,
    RouteResult,
    HuginnExitGate,
    OuroExitGate,
    cumulative_exit_probability,
    ouro_exit_signal,
    relative_state_change,
)
from .sampler import BatchSamplingArgs, Sampler, make_device_tensor, sample_impl, sample_rows
from . import coda, integration, workloads

__all__ = [
    "BatchSamplingArgs", "coda", "DecodeStepResult", "GateResult", "HuginnExitGate", "OuroExitGate",
    "RouteResult", "Sampler", "cdb_decode_step", "cumulative_exit_probability", "integration", "ouro_exit_signal",
    "make_device_tensor", "relative_state_change", "sample_impl", "sample_rows",
]
