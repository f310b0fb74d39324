// Launch parameters of lsg_sample shared by the sampler kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lsg {

struct SampleParams {
  const void* logits;
  int64_t B_src, V, ld, B_out;
  const float* temps;
  const int32_t* top_k;
  const float* top_p;
  const float* uniforms;
  const int32_t* row_idx;
  const int32_t* n_rows_dev;
  int32_t* out;
};

// Launches the streamed row sampler (sample_quad.hip) when the batch has more
// rows than the device has compute units and the row shape is one it serves
// (16-byte aligned rows of exactly 256 * CAP chunks); returns false, launching
// nothing, otherwise.
bool quad_sample_launch(const SampleParams& P, int dtype, bool greedy, bool vec, hipStream_t st);

}  // namespace lsg
