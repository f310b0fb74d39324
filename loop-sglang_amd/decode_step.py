"""One CDB decode step on the device: exit gate -> stable exit compaction ->
sampling of the exited rows, as one launch sequence with no host sync.

In the reference this spans OuroModel.exit_signal inside the core graph
(models/looped/ouro.py:142-155), the D2H gate readback and host filter
(model_executor/cdb_model_runner.py:154-182, managers/cdb_scheduler.py:189-229)
and Sampler.sample on the coda batch (model_executor/sample.py:107-112).  Here
the exited row list never leaves the GPU: the sampler gathers the exited rows'
logits by ``exit_idx`` and reads the row count from ``n_exit`` on the device.

Routing timing: given the gate's pending-request pool (``pending``, from
``OuroExitGate.init_pending_pool``) the step routes rows as the reference
scheduler does by default (lookahead exit: the request the previous core step
recorded for a row's state slot routes it now, and this step's request is
recorded; cdb_scheduler.py:207-222,254-266).  Without it, a row's own gate
signal routes it in the same step, the reference's --disable-lookahead-exit.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from .exit_gate import OuroExitGate
from .sampler import BatchSamplingArgs, sample_rows


class DecodeStepResult(NamedTuple):
    signal: torch.Tensor  # bool[B] exit decision per row
    state: torch.Tensor  # float32[B] updated cumulative exit probability
    exit_idx: torch.Tensor  # int32[B]; first n_exit entries: exited rows, ascending
    keep_idx: torch.Tensor  # int32[B]; first B - n_exit entries: rows that keep looping
    n_exit: torch.Tensor  # int32[1] on the device
    token_ids: torch.Tensor  # int32[B]; entry b < n_exit is the token of row exit_idx[b]
    route: torch.Tensor | None = None  # bool[B] rows routed to the coda (lookahead timing)


def cdb_decode_step(
    gate: OuroExitGate,
    hidden_states: torch.Tensor,
    exit_state: torch.Tensor | None,
    loop_step: int | torch.Tensor,
    logits: torch.Tensor,
    args: BatchSamplingArgs,
    *,
    max_depth: int = 0,
    pending: torch.Tensor | None = None,
) -> DecodeStepResult:
    """Gate every row, compact the exited rows and sample them.

    ``logits`` is [B, V] (one row per gated row); ``args`` holds per-row
    parameters indexed like the gated rows (uniforms required unless greedy).
    Entries of ``token_ids`` at positions >= n_exit are left unwritten.  With
    ``pending`` the exited rows are those the lookahead routing sends to the
    coda in this core step (``route``); without it, those whose gate fires.
    """
    if pending is None:
        res = gate.exit_signal_compact(hidden_states, exit_state, loop_step, max_depth=max_depth)
        route = None
    else:
        res = gate.exit_route(hidden_states, exit_state, loop_step, pending=pending, max_depth=max_depth)
        route = res.route
    ids = torch.empty(logits.shape[0], dtype=torch.int32, device=logits.device)
    sample_rows(
        logits, args.temperatures, args.top_k, args.top_p, args.uniforms,
        row_idx=res.exit_idx, n_rows=res.n_exit, out=ids,
    )
    return DecodeStepResult(res.signal, res.state, res.exit_idx, res.keep_idx, res.n_exit, ids, route)
