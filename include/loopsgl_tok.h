/*
 * loopsgl_tok -- C ABI of the MI355X (gfx950) decode token path of Loop-SGLang:
 * token sampling (greedy / temperature / top-k / top-p with explicit uniforms)
 * and the Continuous Depth Batching exit gate with on-device exit compaction.
 *
 * Conventions
 *   - All pointers are device pointers unless stated otherwise.  Sizes and row
 *     strides (ld*) are in elements.  `stream` is a hipStream_t (NULL = the
 *     default stream); every call only enqueues work on it and never
 *     synchronises, allocates or frees memory, so calls can be captured in a
 *     HIP graph.
 *   - Return value: LSG_OK (0) or an LSG_ERR_* code; lsg_last_error() then
 *     returns a message for the calling host thread.
 *   - dtype codes: LSG_DTYPE_F32, LSG_DTYPE_BF16, LSG_DTYPE_F16.
 *   - Calls that share a workspace must not overlap in time on the device.
 */
#ifndef LOOPSGL_TOK_H
#define LOOPSGL_TOK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSG_DTYPE_F32 0
#define LSG_DTYPE_BF16 1
#define LSG_DTYPE_F16 2

#define LSG_OK 0
#define LSG_ERR_ARG 1       /* invalid argument (nothing was launched) */
#define LSG_ERR_HIP 2       /* the HIP runtime reported an error */
#define LSG_ERR_WORKSPACE 3 /* workspace missing or too small */

#define LSG_OP_EXIT_GATE 1
#define LSG_OP_REL_CHANGE 2

/*
 * Token sampling.  Replaces Sampler.sample (python/loopsgl/model_executor/
 * sample.py:107-112): torch.argmax for all-greedy batches (sample.py:110-111)
 * and flashinfer's softmax + {,top_k_,top_p_,top_k_top_p_}sampling_from_probs
 * (sample.py:60-81) otherwise; the int32 result matches the cast at
 * model_executor/model_runner.py:279-280.
 *
 *   logits        [B_src, V] rows with stride ld, dtype fp32/bf16/fp16.
 *   temperatures  f32[B_src] or NULL.  NULL: every row is argmax (torch rules:
 *                 first maximum wins, NaN counts as the maximum).  Per row,
 *                 T <= 0 or non-finite also selects argmax.
 *   top_k         i32[B_src] or NULL; k < 1 or k >= V disables top-k.
 *   top_p         f32[B_src] or NULL; p >= 1 disables top-p.  top-p is applied
 *                 after top-k (renormalised over the top-k set).
 *   uniforms      f32[B_src] in [0, 1); required when temperatures != NULL.
 *   row_idx       i32[B_out] or NULL: output row b samples logits row
 *                 row_idx[b] (a gather, e.g. the exit_idx of lsg_exit_gate);
 *                 per-row parameters are read at the same source row.  An index
 *                 outside [0, B_src) yields id -1.
 *   B_out         number of output rows (grid size).
 *   n_rows_dev    i32* (device) or NULL: when given, only rows b < *n_rows_dev
 *                 are written (rows past the count are left untouched).
 *   out_ids       i32[B_out] sampled token ids.
 */
int lsg_sample(const void* logits, int dtype, int64_t B_src, int64_t V, int64_t ld,
               const float* temperatures, const int32_t* top_k, const float* top_p,
               const float* uniforms, const int32_t* row_idx, int64_t B_out,
               const int32_t* n_rows_dev, int32_t* out_ids, void* stream);

/*
 * Ouro exit gate with stable exit compaction.  Replaces OuroModel.exit_signal
 * (python/loopsgl/models/looped/ouro.py:142-155) -- the gate linear
 * (layers/linear.py:32-33), cumulative_exit_probability (models/looped/
 * exit_gates.py:6-15) and the threshold/depth test -- plus the host-side stable
 * filter of exited rows in CDBScheduler._consume_gate (managers/
 * cdb_scheduler.py:215-228) and the state-pool gather/scatter of the exit state
 * in CDBModelRunner._execute_phase (model_executor/cdb_model_runner.py:94-109).
 *
 *   h             [B, H] hidden states, stride ldh, dtype fp32/bf16/fp16.
 *   w, bias       gate weight [H] and bias [1] in the same dtype (bias may be NULL).
 *   F_prev/F_next f32 cumulative exit probability before/after this step.  With
 *                 slots == NULL they are indexed by row; otherwise by slots[row]
 *                 (a state pool).  F_next may alias F_prev.  F_prev == NULL
 *                 means all zeros (init_exit_state, ouro.py:138-140).
 *   loop_step     i32[B] zero-based step just executed, or NULL to use
 *                 loop_step_scalar for every row.
 *   tau           exit threshold (compared as float32, inclusive).
 *   min_loop_steps, lookahead (0/1: exit_gate_type == "lookahead").
 *   max_depth     > 0: also exit rows with loop_step + 1 >= max_depth (the
 *                 scheduler's depth cap, cdb_scheduler.py:221,262-266); 0 = off.
 *   mask          u8[B] exit signal (0/1, torch.bool layout).
 *   exit_idx      i32[B] ascending rows with mask 1 (first *n_exit valid), or NULL.
 *   keep_idx      i32[B] ascending rows with mask 0 (first B - *n_exit), or NULL.
 *   n_exit        i32[1] number of exited rows, or NULL.
 *   z_out         f32[B] gate logit after rounding to dtype, or NULL.
 *   workspace     >= lsg_workspace_bytes(LSG_OP_EXIT_GATE, B) bytes, needed when
 *                 exit_idx, keep_idx or n_exit is given; zero-filled once before
 *                 its first use, then owned by the library (it keeps a call
 *                 serial number there).  B < 2^30 with compaction.
 * This is the --disable-lookahead-exit routing: a row's own gate routes it in the
 * step it fires.  lsg_exit_gate_route adds the default (lookahead) timing.
 */
int lsg_exit_gate(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh, const void* w,
                  const void* bias, const float* F_prev, float* F_next, const int32_t* slots,
                  const int32_t* loop_step, int32_t loop_step_scalar, float tau,
                  int32_t min_loop_steps, int32_t lookahead, int32_t max_depth, uint8_t* mask,
                  int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit, float* z_out,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * lsg_exit_gate for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It has
 * no counterpart in the reference.  Same arguments and results as lsg_exit_gate
 * without the workspace: the compaction uses a static device array inside the
 * library (one per GPU, about 64 KiB, held until the process ends), looked up
 * for the current device, which must be the stream's device.
 *   B             at most 65536 rows (LSG_ERR_ARG beyond).
 * Calls that overlap in time on one GPU share that array and race: serialise
 * them (one stream, or events).  Nothing is allocated or freed.
 */
int lsg_exit_gate_noalloc(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                          const void* w, const void* bias, const float* F_prev, float* F_next,
                          const int32_t* slots, const int32_t* loop_step, int32_t loop_step_scalar,
                          float tau, int32_t min_loop_steps, int32_t lookahead, int32_t max_depth,
                          uint8_t* mask, int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit,
                          float* z_out, void* stream);

/*
 * One core step of the Ouro gate with the scheduler's exit routing.  Replaces,
 * besides what lsg_exit_gate replaces, the routing rules of CDBScheduler.
 * _consume_gate and _run_core (managers/cdb_scheduler.py:207-222,254-266).
 * Arguments as lsg_exit_gate, with mask = this step's gate signal (ouro.py:154,
 * no depth cap) and the compaction taken over `route`:
 *   disable_lookahead_exit  1: a row's request routes it in this step.
 *                 0 (the scheduler's default): the request recorded for the row's
 *                 state slot by the previous call on this workspace routes it (the
 *                 token ran in consecutive core steps, so it advanced since its
 *                 gate); this call's request is recorded for the next call.
 *   pending       i64[n_slots] pending-gate pool, indexed like F (slots[row] or
 *                 row), read and rewritten in place; opaque; zero-filled before
 *                 first use.  A routed row's entry is cleared; a caller that
 *                 moves a new token into a slot by other means (cancellation,
 *                 retraction) writes 0 there.  May be NULL when
 *                 disable_lookahead_exit = 1.
 *   replay_depth  i32[B] or NULL: a value rd > 0 replaces the row's request by
 *                 depth >= rd - (disable_lookahead_exit ? 0 : 1), depth =
 *                 loop_step + 1 (cdb_scheduler.py:207-213).
 *   route         u8[B] or NULL: 1 for rows routed to the coda in this step
 *                 (request as above, or depth >= max_depth when max_depth > 0).
 *   workspace     required (it carries the call serial number the pending pool
 *                 is tagged with); one workspace per sequence of core steps.
 */
int lsg_exit_gate_route(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                        const void* w, const void* bias, const float* F_prev, float* F_next,
                        const int32_t* slots, const int32_t* loop_step, int32_t loop_step_scalar,
                        float tau, int32_t min_loop_steps, int32_t lookahead, int32_t max_depth,
                        int32_t disable_lookahead_exit, int64_t* pending,
                        const int32_t* replay_depth, uint8_t* mask, uint8_t* route,
                        int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit, float* z_out,
                        void* workspace, size_t workspace_bytes, void* stream);

/*
 * cumulative_exit_probability alone (models/looped/exit_gates.py:6-15):
 * F_next = F_prev + (1 - F_prev) * sigmoid(float(z)), elementwise over B.
 * z has dtype fp32/bf16/fp16; F_next may alias F_prev.
 */
int lsg_cumulative_exit_probability(const void* z, int dtype, const float* F_prev, float* F_next,
                                    int64_t B, void* stream);

/*
 * Huginn gate (models/looped/huginn.py:184-194, exit_gates.py:18-24):
 * ratio = ||h - h_prev||_2 / max(||h||_2, eps) in float32, mask = ratio < tau,
 * plus the same optional compaction outputs as lsg_exit_gate.
 * workspace: >= lsg_workspace_bytes(LSG_OP_REL_CHANGE, B) bytes (zero-filled
 * before first use, then owned by the library) when exit_idx, keep_idx or n_exit
 * is requested.
 */
int lsg_relative_state_change(const void* h, const void* h_prev, int dtype, int64_t B, int64_t H,
                              int64_t ldh, int64_t ldp, float tau, float eps, float* ratio,
                              uint8_t* mask, int32_t* exit_idx, int32_t* keep_idx,
                              int32_t* n_exit, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Workspace bytes needed by an op (LSG_OP_*) for B rows. */
size_t lsg_workspace_bytes(int op, int64_t B);

/*
 * The coda's vocabulary projection (ParallelLMHead.forward,
 * python/loopsgl/layers/embedding.py:88-111, tp_size 1; called from
 * BaseLoopedForCausalLM.forward_coda, models/looped/base.py:166-168):
 *   logits[b, v] = bf16(sum_k hidden[b, k] * weight[v, k])
 * on MFMA with fp32 accumulation (the reference's F.linear in bf16).
 *   hidden  bf16 [B, H], row stride ld_hidden;  weight  bf16 [V, H], row stride
 *           ld_weight; H a multiple of 64, strides multiples of 8 (>= H), both
 *           16-byte aligned.
 *   logits  bf16 [B, V] out, row stride ld_logits >= V.
 */
int lsg_lm_head(const void* hidden, int64_t B, int64_t H, int64_t ld_hidden, const void* weight, int64_t V,
                int64_t ld_weight, void* logits, int64_t ld_logits, void* stream);

/*
 * The fused coda tail: the projection above followed by the token step, with
 * no fp32 [B, V] logits buffer.  Replaces lm_head -> the copy into
 * GraphCaptureBuffer.logits (model_executor/graph.py:34,
 * model_executor/cdb_graph.py:80-82) -> Sampler.sample (sample.py:107-112).
 * The bf16 logits and, per row and 96-column tile, their maximum and first
 * index go to the workspace; temperatures == NULL (all greedy) finishes from
 * the tile maxima alone (torch.argmax rules), otherwise lsg_sample runs on the
 * bf16 logits with the same per-row arguments as lsg_sample.
 *   workspace  >= lsg_lm_head_workspace_bytes(B, V) bytes, 16-byte aligned
 *              (contents need no initialisation).
 */
int lsg_lm_head_sample(const void* hidden, int64_t B, int64_t H, int64_t ld_hidden, const void* weight, int64_t V,
                       int64_t ld_weight, const float* temperatures, const int32_t* top_k, const float* top_p,
                       const float* uniforms, void* workspace, size_t workspace_bytes, int32_t* out_ids,
                       void* stream);
size_t lsg_lm_head_workspace_bytes(int64_t B, int64_t V);

/* Message of the last failed call on this host thread ("" if none). */
const char* lsg_last_error(void);

/* Library ABI version (this header: 1). */
int lsg_version(void);

#ifdef __cplusplus
}
#endif

#endif /* LOOPSGL_TOK_H */
