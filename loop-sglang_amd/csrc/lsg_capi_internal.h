// Error reporting shared by the C-ABI entry points (see include/loopsgl_tok.h).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/loopsgl_tok.h"

namespace lsg {

// Record a printf-style message in the calling thread's error slot; returns code.
int set_error(int code, const char* fmt, ...);
void clear_error();
// Turn a pending HIP launch error into LSG_ERR_HIP (message names `what`).
int check_launch(const char* what);

// The coda's vocabulary projection (lm_head.hip).
int lm_head_tiles(int64_t V);
int lm_head_launch(const void* h, int64_t B, int64_t H, int64_t ldh, const void* w, int64_t V, int64_t ldw,
                   void* logits, int64_t ldl, float* tmax, int32_t* targ, hipStream_t st);
int lm_head_argmax_launch(const float* tmax, const int32_t* targ, int ntiles, int64_t B, const int32_t* n_rows_dev,
                          int32_t* out, hipStream_t st);

}  // namespace lsg
