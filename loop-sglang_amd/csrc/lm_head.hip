// The coda's vocabulary projection with a sampling epilogue (the fused coda
// tail of the decode step).
//
// Replaces, for the decode token path of Loop-SGLang:
//   ParallelLMHead.forward   python/loopsgl/layers/embedding.py:88-111
//     logits = F.linear(x, weight) in the model dtype (bf16), tp_size == 1
//   the copy into the fp32 graph buffer  model_executor/graph.py:34,
//     model_executor/cdb_graph.py:80-82 (GraphCaptureBuffer.logits)
//   BaseLoopedForCausalLM.forward_coda -> lm_head   models/looped/base.py:166-168
// The reference writes bf16 logits, copies them into an fp32 [B, V] buffer and
// the sampler re-reads that (12 bytes of logits traffic per vocabulary entry);
// here the projection writes the bf16 logits once (the values the reference's
// F.linear returns, up to the accumulation order of fp32 sums) with, per row
// and 96-column tile, the maximum and its first index, so greedy rows finish
// from those alone and sampled rows read the bf16 logits once.
//
// lm_head_kernel: C[b, v] = bf16(sum_k h[b, k] * W[v, k]) on MFMA
// (v_mfma_f32_32x32x16_bf16, fp32 accumulation).  One 256-thread workgroup per
// (256-row batch tile, 192-column vocabulary tile); W is streamed from HBM once
// per batch tile, h is re-read from L2.  K advances in steps of 64 through two
// LDS stages filled by direct-to-LDS loads (no register staging), one stage
// ahead of the MFMAs.  The length of each W row's read per stage sets the
// speed (HBM serves 128-byte row segments far better than 64-byte ones: K
// steps of 16 / 32 / 64 measured 106 / 76 / 64 us for the Ouro-shaped
// projection), and two 57 KB stages fill the LDS.  A stage row is 128 bytes
// (eight 16-byte chunks), chunk c of row r stored at position c ^ ((r >> 1) & 7),
// so the fragment reads of 16 consecutive rows hit distinct banks.  Eight waves
// (two per SIMD):
// wave w owns batch rows 64 (w % 4) .. +63 of the tile and columns
// 96 (w / 4) .. +95: 2 x 3 blocks of 32 x 32, 96 fp32 accumulators per lane.
// Operand layouts (checked on the device): A lane l holds row l % 32,
// k = 8 (l / 32) + q; B lane l holds column l % 32, same k; C lane l, register
// r holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
// Epilogue: the accumulators are rounded to bf16 (RNE) into LDS, then stored
// as 16-byte row segments; lane l of wave w then scans its 96 columns of row
// 64 (w % 4) + l for their maximum and first index (torch.argmax rules: NaN
// wins, first wins): row statistics per 96-column half tile.
//
// lm_head_argmax_kernel: per row, the first maximum over the tiles' maxima.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lsg_capi_internal.h"
#include "lsg_common.h"

namespace lsg {
namespace lmh {

constexpr int kMT = 256;   // batch rows per tile
constexpr int kNT = 192;   // vocabulary columns per tile
constexpr int kKT = 64;      // K per stage
constexpr int kRow = kKT;    // LDS row stride in bf16 (swizzled 16-byte chunks)
constexpr int kStages = 2;   // LDS stages (all but one in flight ahead of the MFMAs)
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kHalf = kNT / 2;  // columns per wave, and per row-statistics tile
constexpr int kStageA = kMT * kRow;  // bf16 elements of h per stage
constexpr int kStageB = kNT * kRow;  // bf16 elements of W per stage
constexpr int kLdsElems = kStages * (kStageA + kStageB);
// direct-to-LDS loads per wave per stage, 1 KB (kRPG rows of kCPR 16-byte
// chunks) each: h's and W's row groups spread over the waves (a wave past the
// last group loads its own group again, the same bytes to the same place)
constexpr int kCPR = kKT / 8, kRPG = 64 / kCPR;
constexpr int kGroupsA = kMT / kRPG, kGroupsB = kNT / kRPG;
constexpr int kLoadsA = (kGroupsA + kWaves - 1) / kWaves, kLoadsB = (kGroupsB + kWaves - 1) / kWaves;
constexpr int kLoads = kLoadsA + kLoadsB;
static_assert(kKT % 16 == 0 && kMT % kRPG == 0 && kNT % kRPG == 0, "stage shape");
// every wave's first load has a row group of its own (a wave past the last
// group reloads its own group, which must exist): fewer groups than waves
// would put rows past the stage
static_assert(kGroupsA >= kWaves && kGroupsB >= kWaves, "at least one row group per wave");
// epilogue: 64 rows x 96 columns of bf16 per wave, rows padded by 8
constexpr int kOutRow = kHalf + 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

struct Params {
  const uint16_t* h;   // [B, H] bf16, row stride ldh
  const uint16_t* w;   // [V, H] bf16, row stride ldw
  uint16_t* logits;    // [B, V] bf16, row stride ldl
  float* tmax;         // [B, ntiles] maxima per 96-column half tile (may be null)
  int32_t* targ;       // [B, ntiles] their first indices
  int64_t B, H, V, ldh, ldw, ldl;
  int ntiles;
};

__device__ __forceinline__ uint16_t f2bf(float f) {  // round to nearest even; NaN stays NaN
  const uint32_t b = __float_as_uint(f);
  if ((b & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((b >> 16) | 0x40u);
  return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf2f(uint32_t u16) { return __uint_as_float(u16 << 16); }

// Stage s of K into LDS buffer s % kStages by direct-to-LDS loads: a load of
// row group g writes rows 16 g .. 16 g + 15 of the stage (1 KB, lane i at byte
// 16 i: row i / 4, position i % 4), reading the chunk that belongs at that
// position.  Rows outside the matrices read the last row (their results are
// never stored).
// A 16-byte LDS read serves 16 lanes at a time: the fragment reads of 16
// consecutive rows (one chunk each) must fill 16 distinct 16-byte slots of a
// 256-byte bank line.  A 128-byte row puts rows of one parity in one half of
// the line, so chunk c of row r goes to position c ^ ((r >> 1) & 7).
__device__ __forceinline__ int swz(int row, int c) {
  static_assert(kCPR == 8, "swizzle for 128-byte stage rows");
  return c ^ ((row >> 1) & 7);
}

__device__ __forceinline__ void issue_stage(const Params& P, uint16_t* lds, int64_t m0, int64_t n0, int s, int kb) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  uint16_t* A = lds + (s % kStages) * (kStageA + kStageB);
  uint16_t* Bm = A + kStageA;
  const int64_t k0 = (int64_t)kb * kKT;
  const int rl = lane / kCPR, pos = lane % kCPR;
#pragma unroll
  for (int q = 0; q < kLoadsA; ++q) {
    const int g = q * kWaves + wid < kGroupsA ? q * kWaves + wid : wid;
    const int row = kRPG * g + rl;
    int64_t gr = m0 + row;
    gr = gr < P.B ? gr : P.B - 1;
    const uint16_t* src = P.h + gr * P.ldh + k0 + swz(row, pos) * 8;
    __builtin_amdgcn_global_load_lds(src, A + kRPG * g * kRow, 16, 0, 0);
  }
#pragma unroll
  for (int q = 0; q < kLoadsB; ++q) {
    const int g = q * kWaves + wid < kGroupsB ? q * kWaves + wid : wid;
    const int row = kRPG * g + rl;
    int64_t gr = n0 + row;
    gr = gr < P.V ? gr : P.V - 1;
    const uint16_t* src = P.w + gr * P.ldw + k0 + swz(row, pos) * 8;
    __builtin_amdgcn_global_load_lds(src, Bm + kRPG * g * kRow, 16, 0, 0);
  }
}

// Wait until at most n of this wave's loads are outstanding (n < 64).
template <int N>
__device__ __forceinline__ void wait_vm() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until stage s has landed: at most min(ahead, M) later stages' loads
// stay outstanding (loads retire in order).
template <int M>
__device__ __forceinline__ void wait_stages(int ahead) {
  if constexpr (M > 0) {
    if (ahead >= M) {
      wait_vm<M * kLoads>();
      return;
    }
    wait_stages<M - 1>(ahead);
  } else {
    wait_vm<0>();
  }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1))) void lm_head_kernel(Params P) {
  extern __shared__ __align__(16) uint16_t lds[];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t n0 = (int64_t)blockIdx.x * kNT, m0 = (int64_t)blockIdx.y * kMT;
  const int nst = (int)(P.H / kKT);
  const int wr = (wid & 3) * 64, wc = (wid >> 2) * kHalf;  // this wave's rows and columns of the tile
  f32x16 acc[2][3];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j) acc[i][j] = f32x16{};
  const int fr = lane & 31, fk = lane >> 5;  // fragment row/column and k chunk of this lane
  // Each workgroup starts at its own K block (and wraps around), so that at any
  // moment the workgroups read different 64-byte columns of their W rows: rows
  // 2^k bytes apart read at one offset would all land on the same HBM channel.
  const int kshift = (int)(blockIdx.x % (unsigned)nst);
  auto kblock = [&](int s) { const int b = s + kshift; return b >= nst ? b - nst : b; };
#pragma unroll
  for (int q = 0; q < kStages - 1; ++q)
    if (q < nst) issue_stage(P, lds, m0, n0, q, kblock(q));
  for (int s = 0; s < nst; ++s) {
    // stage s complete for this wave (loads retire in order), then for all
    wait_stages<kStages - 2>(nst - 1 - s);
    __syncthreads();  // also: every wave is done with stage s - 1's buffer
    if (s + kStages - 1 < nst) issue_stage(P, lds, m0, n0, s + kStages - 1, kblock(s + kStages - 1));
    const uint16_t* A = lds + (s % kStages) * (kStageA + kStageB);
    const uint16_t* Bm = A + kStageA;
#pragma unroll
    for (int kk = 0; kk < kKT / 16; ++kk) {
      const int c = 2 * kk + fk;  // 16-byte chunk of k
      bf16x8 af[2], bfr[3];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wr + i * 32 + fr;
        af[i] = *reinterpret_cast<const bf16x8*>(A + row * kRow + swz(row, c) * 8);
      }
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const int row = wc + j * 32 + fr;
        bfr[j] = *reinterpret_cast<const bf16x8*>(Bm + row * kRow + swz(row, c) * 8);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  }
  __syncthreads();  // every wave is done with the stages before the epilogue reuses LDS
  // epilogue: bf16 tile of this wave (64 rows x 96 columns) through LDS
  uint16_t* O = lds + wid * 64 * kOutRow;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int row = i * 32 + (q >> 2) * 8 + (lane >> 5) * 4 + (q & 3);
        O[row * kOutRow + j * 32 + fr] = f2bf(acc[i][j][q]);
      }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  // 16-byte stores: row segments of 12 chunks, lane l takes chunks l, l + 64, ...
  const int64_t c0 = n0 + wc;  // first column of this wave
  const int64_t nv = P.V - c0 < 0 ? 0 : (P.V - c0 < kHalf ? P.V - c0 : kHalf);
  const bool vec = (P.ldl % 8) == 0 && nv == kHalf && (reinterpret_cast<uintptr_t>(P.logits) & 15u) == 0;
  for (int c = lane; c < 64 * (kHalf / 8); c += 64) {
    const int row = c / (kHalf / 8), cc = c % (kHalf / 8);
    const int64_t gr = m0 + wr + row;
    if (gr >= P.B || cc * 8 >= nv) continue;
    uint16_t* dst = P.logits + gr * P.ldl + c0 + cc * 8;
    const v4u v = *reinterpret_cast<const v4u*>(O + row * kOutRow + cc * 8);
    if (vec) {
      *reinterpret_cast<v4u*>(dst) = v;
    } else {
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (cc * 8 + e < nv) dst[e] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
    }
  }
  // maximum and first index of this wave's 96 columns of row wr + lane
  if (P.tmax) {
    const int64_t gr = m0 + wr + lane;
    if (gr < P.B) {
      float mx = -INFINITY;
      int arg = -1;
      bool nan = false;
      for (int cc = 0; cc < kHalf / 8; ++cc) {
        const v4u v = *reinterpret_cast<const v4u*>(O + lane * kOutRow + cc * 8);
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = cc * 8 + e;
          const float x = bf2f((w4[e >> 1] >> (16 * (e & 1))) & 0xffffu);
          if (nan || c >= nv) continue;
          if (x != x) {
            nan = true;
            mx = x;
            arg = c;
          } else if (arg < 0 || x > mx) {
            mx = x;
            arg = c;
          }
        }
      }
      const int64_t t = (int64_t)blockIdx.x * 2 + (wid >> 2);
      P.tmax[gr * P.ntiles + t] = mx;
      P.targ[gr * P.ntiles + t] = arg < 0 ? 0x7fffffff : (int32_t)(c0 + arg);  // an empty half: no entry
    }
  }
}

// Per row: the first maximum over the tiles (tiles in vocabulary order; NaN
// wins, the first NaN tile's index; -0 == +0).  One wave per row.
__global__ __launch_bounds__(64) void lm_head_argmax_kernel(const float* tmax, const int32_t* targ, int ntiles,
                                                           int64_t B, const int32_t* n_rows_dev, int32_t* out) {
  const int64_t b = blockIdx.x;
  if (b >= B) return;
  if (n_rows_dev && b >= (int64_t)*n_rows_dev) return;
  const int lane = threadIdx.x;
  float mx = -INFINITY;
  int arg = 0x7fffffff;
  bool nan = false;
  for (int t = lane; t < ntiles; t += 64) {
    const float x = tmax[b * ntiles + t];
    const int a = targ[b * ntiles + t];
    if (nan || a == 0x7fffffff) continue;  // an empty half tile
    if (x != x) {
      nan = true;
      arg = a;
    } else if (arg == 0x7fffffff || x > mx) {
      mx = x;
      arg = a;
    }
  }
  // combine lanes: NaN lanes first (smallest index), else largest value, smallest index
  const int nanarg = wave_min_i(nan ? arg : 0x7fffffff);
  if (nanarg != 0x7fffffff) {
    if (lane == 0) out[b] = nanarg;
    return;
  }
  const float m = wave_max(arg == 0x7fffffff ? -INFINITY : mx);
  const int first = wave_min_i(arg != 0x7fffffff && mx == m ? arg : 0x7fffffff);
  if (lane == 0) out[b] = first == 0x7fffffff ? 0 : first;
}

}  // namespace lmh

size_t lm_head_lds_bytes() {
  const size_t stages = (size_t)lmh::kLdsElems * 2;
  const size_t out = (size_t)lmh::kWaves * 64 * lmh::kOutRow * 2;
  return stages > out ? stages : out;
}

// Row-statistics tiles: two per 192-column projection tile.
int lm_head_tiles(int64_t V) { return (int)(2 * ((V + lmh::kNT - 1) / lmh::kNT)); }

int lm_head_launch(const void* h, int64_t B, int64_t H, int64_t ldh, const void* w, int64_t V, int64_t ldw,
                   void* logits, int64_t ldl, float* tmax, int32_t* targ, hipStream_t st) {
  lmh::Params P;
  P.h = static_cast<const uint16_t*>(h);
  P.w = static_cast<const uint16_t*>(w);
  P.logits = static_cast<uint16_t*>(logits);
  P.tmax = tmax;
  P.targ = targ;
  P.B = B;
  P.H = H;
  P.V = V;
  P.ldh = ldh;
  P.ldw = ldw;
  P.ldl = ldl;
  P.ntiles = lm_head_tiles(V);
  const dim3 grid((unsigned)((V + lmh::kNT - 1) / lmh::kNT), (unsigned)((B + lmh::kMT - 1) / lmh::kMT));
  static bool attr_set[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return set_error(LSG_ERR_HIP, "lm_head: no device");
  if (!attr_set[dev]) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&lmh::lm_head_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lm_head_lds_bytes()) != hipSuccess)
      return set_error(LSG_ERR_HIP, "lm_head: cannot raise the kernel's LDS limit to %zu bytes", lm_head_lds_bytes());
    attr_set[dev] = true;
  }
  hipLaunchKernelGGL(lmh::lm_head_kernel, grid, dim3(lmh::kThreads), lm_head_lds_bytes(), st, P);
  return check_launch("lsg_lm_head");
}

int lm_head_argmax_launch(const float* tmax, const int32_t* targ, int ntiles, int64_t B, const int32_t* n_rows_dev,
                          int32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(lmh::lm_head_argmax_kernel, dim3((unsigned)B), dim3(64), 0, st, tmax, targ, ntiles, B,
                     n_rows_dev, out);
  return check_launch("lsg_lm_head_sample (argmax)");
}

}  // namespace lsg

namespace {
size_t align256(size_t n) { return (n + 255) / 256 * 256; }
int64_t padded_ld(int64_t V) { return (V + 7) / 8 * 8; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_lm_head_args(const void* hidden, int64_t B, int64_t H, int64_t ld_hidden, const void* weight, int64_t V,
                       int64_t ld_weight) {
  if (!hidden || !weight) return lsg::set_error(LSG_ERR_ARG, "lm_head: hidden and weight are required");
  if (B < 1 || V < 1) return lsg::set_error(LSG_ERR_ARG, "lm_head: B (%lld) and V (%lld) must be >= 1", (long long)B,
                                            (long long)V);
  if (H < 64 || H % 64 != 0)
    return lsg::set_error(LSG_ERR_ARG, "lm_head: H (%lld) must be a positive multiple of 64", (long long)H);
  if (ld_hidden < H || ld_weight < H || ld_hidden % 8 != 0 || ld_weight % 8 != 0)
    return lsg::set_error(LSG_ERR_ARG, "lm_head: row strides (%lld, %lld) must be >= H and multiples of 8",
                          (long long)ld_hidden, (long long)ld_weight);
  if (!aligned16(hidden) || !aligned16(weight))
    return lsg::set_error(LSG_ERR_ARG, "lm_head: hidden and weight must be 16-byte aligned");
  if ((B + 255) / 256 > 65535 || lsg::lm_head_tiles(V) > (1 << 30))
    return lsg::set_error(LSG_ERR_ARG, "lm_head: B (%lld) or V (%lld) too large", (long long)B, (long long)V);
  return LSG_OK;
}
}  // namespace

extern "C" size_t lsg_lm_head_workspace_bytes(int64_t B, int64_t V) {
  if (B < 1 || V < 1) return 0;
  const size_t tiles = (size_t)lsg::lm_head_tiles(V);
  return align256((size_t)B * (size_t)padded_ld(V) * 2) + 2 * align256((size_t)B * tiles * 4);
}

extern "C" int lsg_lm_head(const void* hidden, int64_t B, int64_t H, int64_t ld_hidden, const void* weight, int64_t V,
                           int64_t ld_weight, void* logits, int64_t ld_logits, void* stream) {
  lsg::clear_error();
  const int rc = check_lm_head_args(hidden, B, H, ld_hidden, weight, V, ld_weight);
  if (rc) return rc;
  if (!logits || ld_logits < V) return lsg::set_error(LSG_ERR_ARG, "lm_head: logits missing or ld_logits < V");
  return lsg::lm_head_launch(hidden, B, H, ld_hidden, weight, V, ld_weight, logits, ld_logits, nullptr, nullptr,
                             static_cast<hipStream_t>(stream));
}

extern "C" int lsg_lm_head_sample(const void* hidden, int64_t B, int64_t H, int64_t ld_hidden, const void* weight,
                                  int64_t V, int64_t ld_weight, const float* temperatures, const int32_t* top_k,
                                  const float* top_p, const float* uniforms, void* workspace, size_t workspace_bytes,
                                  int32_t* out_ids, void* stream) {
  lsg::clear_error();
  int rc = check_lm_head_args(hidden, B, H, ld_hidden, weight, V, ld_weight);
  if (rc) return rc;
  if (!out_ids) return lsg::set_error(LSG_ERR_ARG, "lm_head_sample: out_ids is required");
  if (temperatures && !uniforms) return lsg::set_error(LSG_ERR_ARG, "lm_head_sample: sampling needs uniforms");
  const size_t need = lsg_lm_head_workspace_bytes(B, V);
  if (!workspace || workspace_bytes < need || !aligned16(workspace))
    return lsg::set_error(LSG_ERR_WORKSPACE, "lm_head_sample: workspace needs %zu bytes, 16-byte aligned (got %zu)",
                          need, workspace_bytes);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t ldl = padded_ld(V);
  const int ntiles = lsg::lm_head_tiles(V);
  char* ws = static_cast<char*>(workspace);
  void* logits = ws;
  float* tmax = reinterpret_cast<float*>(ws + align256((size_t)B * (size_t)ldl * 2));
  int32_t* targ = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(tmax) + align256((size_t)B * ntiles * 4));
  rc = lsg::lm_head_launch(hidden, B, H, ld_hidden, weight, V, ld_weight, logits, ldl, tmax, targ, st);
  if (rc) return rc;
  if (!temperatures) return lsg::lm_head_argmax_launch(tmax, targ, ntiles, B, nullptr, out_ids, st);
  return lsg_sample(logits, LSG_DTYPE_BF16, B, V, ldl, temperatures, top_k, top_p, uniforms, nullptr, B, nullptr,
                    out_ids, stream);
}
