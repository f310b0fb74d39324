// Shared device helpers for the decode-token-path kernels (gfx950, wave64).
//
// Layout conventions used by every kernel in this library:
//   * A "row" is V (or H) elements of one dtype, with row stride ld elements.
//   * Rows are read in 16-byte "chunks" (8 bf16/fp16 or 4 fp32 elements).  Chunk c
//     of a row covers elements [c*EPV, c*EPV + EPV).  Workgroup thread t owns the
//     chunks c = j*NT + t (j = 0, 1, ...), so one wave instruction reads 64
//     consecutive chunks = 1 KiB of contiguous HBM (fully coalesced 128-bit loads).
//   * Elements past the row end are padding and read as -inf.
//   * All floating-point reductions use a fixed association order (xor-butterfly
//     inside a wave, then waves in index order), so results are deterministic and
//     bitwise identical in every lane.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lsg {

enum DType : int { kF32 = 0, kBF16 = 1, kF16 = 2 };

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Element types.  Each trait converts lane i of a 16-byte chunk to float, gives
// the padding pattern (-inf) and loads one element for unaligned rows.
// ---------------------------------------------------------------------------
struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int EPV = 4;
  static constexpr int kSize = 4;
  __device__ static __forceinline__ float get(const uint4& v, int i) {
    const uint32_t w = i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
    return __uint_as_float(w);
  }
  // (no unpacking: a second pass shares nothing with the first)
  __device__ static __forceinline__ float get_alt(const uint4& v, int i) { return get(v, i); }
  static constexpr bool kHasAlt = true;
  __device__ static __forceinline__ uint4 pad() {
    return make_uint4(0xff800000u, 0xff800000u, 0xff800000u, 0xff800000u);
  }
  __device__ static __forceinline__ uint32_t load_bits(const float* p) {
    return __float_as_uint(*p);
  }
  __device__ static __forceinline__ void set(uint4& v, int i, uint32_t b) {
    if (i == 0) v.x = b; else if (i == 1) v.y = b; else if (i == 2) v.z = b; else v.w = b;
  }
};

template <>
struct Elem<bf16_t> {
  static constexpr int EPV = 8;
  static constexpr int kSize = 2;
  __device__ static __forceinline__ float get(const uint4& v, int i) {
    const int k = i >> 1;
    const uint32_t w = k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
  // Same value through a byte permute: a second pass over the same registers
  // unpacks with different instructions, so the compiler cannot keep the first
  // pass's unpacked values alive for it (that would double the registers).
  __device__ static __forceinline__ float get_alt(const uint4& v, int i) {
    const int k = i >> 1;
    const uint32_t w = k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
    return __uint_as_float(__builtin_amdgcn_perm(0u, w, (i & 1) ? 0x03020c0cu : 0x01000c0cu));
  }
  static constexpr bool kHasAlt = true;
  __device__ static __forceinline__ uint4 pad() {
    return make_uint4(0xff80ff80u, 0xff80ff80u, 0xff80ff80u, 0xff80ff80u);
  }
  __device__ static __forceinline__ uint32_t load_bits(const bf16_t* p) { return p->bits; }
  __device__ static __forceinline__ void set(uint4& v, int i, uint32_t b) {
    const int k = i >> 1;
    uint32_t* w = k == 0 ? &v.x : (k == 1 ? &v.y : (k == 2 ? &v.z : &v.w));
    *w = (i & 1) ? ((*w & 0x0000ffffu) | (b << 16)) : ((*w & 0xffff0000u) | b);
  }
};

template <>
struct Elem<f16_t> {
  static constexpr int EPV = 8;
  static constexpr int kSize = 2;
  __device__ static __forceinline__ float get(const uint4& v, int i) {
    const int k = i >> 1;
    const uint32_t w = k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
    const uint16_t h = (i & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return (float)__builtin_bit_cast(_Float16, h);
  }
  // (same conversions: a second pass launders the registers instead)
  __device__ static __forceinline__ float get_alt(const uint4& v, int i) { return get(v, i); }
  static constexpr bool kHasAlt = false;
  __device__ static __forceinline__ uint4 pad() {
    return make_uint4(0xfc00fc00u, 0xfc00fc00u, 0xfc00fc00u, 0xfc00fc00u);
  }
  __device__ static __forceinline__ uint32_t load_bits(const f16_t* p) { return p->bits; }
  __device__ static __forceinline__ void set(uint4& v, int i, uint32_t b) {
    Elem<bf16_t>::set(v, i, b);
  }
};

// Load chunk c of a row of V elements.  VEC: the row start is 16-byte aligned, so
// every full chunk is one global_load_dwordx4; the partial tail chunk and all
// chunks of unaligned rows are assembled from element loads.
template <typename T, bool VEC>
__device__ __forceinline__ uint4 load_chunk(const T* __restrict__ row, int64_t c, int64_t V) {
  constexpr int EPV = Elem<T>::EPV;
  const int64_t e0 = c * EPV;
  if (e0 >= V) return Elem<T>::pad();
  if (VEC && e0 + EPV <= V) return *reinterpret_cast<const uint4*>(row + e0);
  uint4 v = Elem<T>::pad();
#pragma unroll
  for (int i = 0; i < EPV; ++i)
    if (e0 + i < V) Elem<T>::set(v, i, Elem<T>::load_bits(row + e0 + i));
  return v;
}

// Same with 32-bit indexing from a uniform row base pointer (keeps per-lane
// address math in one VGPR and lets loads use the scalar-base form).
template <typename T, bool VEC>
__device__ __forceinline__ uint4 load_chunk32(const char* __restrict__ base, uint32_t c,
                                              uint32_t V) {
  constexpr int EPV = Elem<T>::EPV;
  const uint32_t e0 = c * EPV;
  if (e0 >= V) return Elem<T>::pad();
  if (VEC && e0 + EPV <= V) return *reinterpret_cast<const uint4*>(base + (uint32_t)(c * 16u));
  uint4 v = Elem<T>::pad();
  const T* row = reinterpret_cast<const T*>(base);
#pragma unroll
  for (int i = 0; i < EPV; ++i)
    if (e0 + i < V) Elem<T>::set(v, i, Elem<T>::load_bits(row + (e0 + i)));
  return v;
}

template <typename T>
__device__ __forceinline__ float chunk_max(const uint4& v) {
  float m = Elem<T>::get(v, 0);
#pragma unroll
  for (int i = 1; i < Elem<T>::EPV; ++i) m = fmaxf(m, Elem<T>::get(v, i));
  return m;
}

template <typename T>
__device__ __forceinline__ float chunk_maximum(const uint4& v) {
  float m = Elem<T>::get(v, 0);
#pragma unroll
  for (int i = 1; i < Elem<T>::EPV; ++i) m = __builtin_elementwise_maximum(m, Elem<T>::get(v, i));
  return m;
}

// ---------------------------------------------------------------------------
// Move a wave-uniform value into scalar registers (frees a VGPR; the value must
// be identical in every active lane).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ uint32_t uni(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ float uni(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ double uni(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readfirstlane((int)(b & 0xffffffffll));
  const int hi = __builtin_amdgcn_readfirstlane((int)(b >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// ---------------------------------------------------------------------------
// DPP cross-lane helpers (GFX9 wave64).  dpp<CTRL, ROWMASK>(old, v): lanes in
// enabled rows read lane CTRL(i) of v; lanes whose source is invalid or whose
// row is disabled keep `old`.
//   row_shr:n = 0x110+n, row_ror:n = 0x120+n, row_bcast15 = 0x142,
//   row_bcast31 = 0x143.
// ---------------------------------------------------------------------------
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ int dpp_i(int old, int v) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWMASK, 0xf, false);
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __int_as_float(dpp_i<CTRL, ROWMASK>(__float_as_int(old), __float_as_int(v)));
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ double dpp_d(double old, double v) {
  const long long o = __double_as_longlong(old), x = __double_as_longlong(v);
  const int lo = dpp_i<CTRL, ROWMASK>((int)(o & 0xffffffffll), (int)(x & 0xffffffffll));
  const int hi = dpp_i<CTRL, ROWMASK>((int)(o >> 32), (int)(x >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffffll), lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Wave reductions.  Rows of 16 lanes are reduced with row_ror butterflies,
// then the four row results (lanes 0, 16, 32, 48) are combined in a fixed
// order in scalar registers: the result is deterministic and wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0x128>(v, v));
  v = fmaxf(v, dpp_f<0x124>(v, v));
  v = fmaxf(v, dpp_f<0x122>(v, v));
  v = fmaxf(v, dpp_f<0x121>(v, v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}
// NaN-propagating maximum (IEEE 754-2019 maximum; v_maximum3_f32 on gfx950).
__device__ __forceinline__ float fmaximum(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float wave_maximum(float v) {
  v = fmaximum(v, dpp_f<0x128>(v, v));
  v = fmaximum(v, dpp_f<0x124>(v, v));
  v = fmaximum(v, dpp_f<0x122>(v, v));
  v = fmaximum(v, dpp_f<0x121>(v, v));
  return fmaximum(fmaximum(readlane_f(v, 0), readlane_f(v, 16)),
                  fmaximum(readlane_f(v, 32), readlane_f(v, 48)));
}
__device__ __forceinline__ double wave_sum(double v) {
  v += dpp_d<0x128>(0.0, v);
  v += dpp_d<0x124>(0.0, v);
  v += dpp_d<0x122>(0.0, v);
  v += dpp_d<0x121>(0.0, v);
  return ((readlane_d(v, 0) + readlane_d(v, 16)) + readlane_d(v, 32)) + readlane_d(v, 48);
}
__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp_i<0x128>(0, v);
  v += dpp_i<0x124>(0, v);
  v += dpp_i<0x122>(0, v);
  v += dpp_i<0x121>(0, v);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) +
         __builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48);
}
__device__ __forceinline__ int wave_min_i(int v) {
  v = min(v, dpp_i<0x128>(v, v));
  v = min(v, dpp_i<0x124>(v, v));
  v = min(v, dpp_i<0x122>(v, v));
  v = min(v, dpp_i<0x121>(v, v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_max_i(int v) {
  v = max(v, dpp_i<0x128>(v, v));
  v = max(v, dpp_i<0x124>(v, v));
  v = max(v, dpp_i<0x122>(v, v));
  v = max(v, dpp_i<0x121>(v, v));
  return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Inclusive prefix sum across the wave in lane order: row_shr 1/2/4/8 inside
// each row of 16, then row_bcast15 / row_bcast31 carry row totals forward.
__device__ __forceinline__ double wave_incl_scan(double v, int /*lane*/) {
  v += dpp_d<0x111>(0.0, v);
  v += dpp_d<0x112>(0.0, v);
  v += dpp_d<0x114>(0.0, v);
  v += dpp_d<0x118>(0.0, v);
  v += dpp_d<0x142, 0xa>(0.0, v);
  v += dpp_d<0x143, 0xc>(0.0, v);
  return v;
}
__device__ __forceinline__ int wave_incl_scan_i(int v, int /*lane*/) {
  v += dpp_i<0x111>(0, v);
  v += dpp_i<0x112>(0, v);
  v += dpp_i<0x114>(0, v);
  v += dpp_i<0x118>(0, v);
  v += dpp_i<0x142, 0xa>(0, v);
  v += dpp_i<0x143, 0xc>(0, v);
  return v;
}
// Value of lane i-1 (0 in lane 0): wave_shr:1.
__device__ __forceinline__ double wave_shr1(double v) { return dpp_d<0x138>(0.0, v); }

// ---------------------------------------------------------------------------
// Workgroup reductions.  `red` is a __shared__ scratch area of at least NW
// elements of 8 bytes.  Wave results (already wave-uniform) are combined in
// wave order, so every thread returns the identical value.  Each call ends with
// a barrier, so the scratch can be reused immediately.
// ---------------------------------------------------------------------------
template <int NW>
__device__ __forceinline__ float wg_max(float v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_max(v);
  if (lane == 0) reinterpret_cast<float*>(red)[w] = v;
  __syncthreads();
  float r = reinterpret_cast<float*>(red)[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaxf(r, reinterpret_cast<float*>(red)[i]);
  __syncthreads();
  return uni(r);
}
template <int NW>
__device__ __forceinline__ float wg_maximum(float v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_maximum(v);
  if (lane == 0) reinterpret_cast<float*>(red)[w] = v;
  __syncthreads();
  float r = reinterpret_cast<float*>(red)[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = fmaximum(r, reinterpret_cast<float*>(red)[i]);
  __syncthreads();
  return uni(r);
}
template <int NW>
__device__ __forceinline__ double wg_sum(double v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) red[w] = v;
  __syncthreads();
  double r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r += red[i];
  __syncthreads();
  return uni(r);
}
template <int NW>
__device__ __forceinline__ int wg_sum_i(int v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum_i(v);
  if (lane == 0) reinterpret_cast<int*>(red)[w] = v;
  __syncthreads();
  int r = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) r += reinterpret_cast<int*>(red)[i];
  __syncthreads();
  return uni(r);
}
template <int NW>
__device__ __forceinline__ int wg_min_i(int v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_min_i(v);
  if (lane == 0) reinterpret_cast<int*>(red)[w] = v;
  __syncthreads();
  int r = reinterpret_cast<int*>(red)[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = min(r, reinterpret_cast<int*>(red)[i]);
  __syncthreads();
  return uni(r);
}
template <int NW>
__device__ __forceinline__ int wg_max_i(int v, double* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_max_i(v);
  if (lane == 0) reinterpret_cast<int*>(red)[w] = v;
  __syncthreads();
  int r = reinterpret_cast<int*>(red)[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = max(r, reinterpret_cast<int*>(red)[i]);
  __syncthreads();
  return uni(r);
}

// Workgroup exclusive/inclusive scan of a double (fixed order).  `red` needs NW
// doubles.  Returns the exclusive prefix; *incl gets the inclusive one and
// *total the workgroup total (identical in every thread).
template <int NW>
__device__ __forceinline__ double wg_scan(double v, double* red, double* incl, double* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const double wi = wave_incl_scan(v, lane);
  const double we = wave_shr1(wi);
  if (lane == 63) red[w] = wi;
  __syncthreads();
  // base(w) is the running sum of the preceding wave totals in index order, so
  // incl(last lane of wave w) == base(w + 1) == excl(first lane of wave w + 1).
  double base = 0.0, tot = 0.0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    if (i == w) base = tot;
    tot += red[i];
  }
  __syncthreads();
  *incl = base + wi;
  *total = uni(tot);
  return base + we;
}

// Order-preserving 32-bit key of a float: larger value -> larger key, -0 maps
// to +0.  Callers never pass NaN.
__device__ __forceinline__ uint32_t okey(float f) {
  uint32_t b = __float_as_uint(f + 0.0f);  // -0 -> +0
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

}  // namespace lsg
