// Token sampling over the vocabulary: greedy argmax, temperature softmax,
// top-k, top-p and one inverse-CDF draw per row with an explicit uniform.
//
// Replaces, for the decode token path of Loop-SGLang:
//   Sampler.sample            python/loopsgl/model_executor/sample.py:107-112
//   torch.argmax (greedy)     sample.py:110-111 (+ int32 cast, model_runner.py:279-280)
//   sample_impl -> flashinfer softmax / *_sampling_from_probs   sample.py:60-81
//
// One workgroup samples one row.  The row is read from HBM exactly once with
// coalesced 128-bit loads (wave w owns a contiguous span of the row and reads
// it 1 KiB per instruction) and stays in VGPRs (CAP chunks of 16 B per
// thread); the later passes (softmax normaliser, threshold search, CDF walk)
// run on registers and LDS.  Chunks past NT*CAP (very large V), and the rare
// exact slow path of the threshold search, re-read the row from global memory.
//
// Semantics (per row r, x = float32(logit), NaN treated as -inf):
//   T <= 0 or non-finite, or max x non-finite  -> id = argmax (torch rules)
//   m = max x,  e_i = 2^((x_i - m) * log2(e)/T)          (= exp((x_i - m)/T))
//   K = {x >= k-th largest x} if 1 <= k < V            (ties kept)
//   P = {x in K : x >= tau}, tau = largest x with mass(x >= tau) >= p * mass(K)
//   id = first index j in P (ascending) with cumsum_P(e)[j] > u * sum_P(e)
// Sums above the 16-byte chunk level are accumulated in float64 in a fixed
// order, so the result is deterministic and agrees with a float64 evaluation
// to ~1e-7 relative.
#include "lsg_capi_internal.h"
#include "lsg_common.h"

#include <type_traits>

namespace lsg {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBins = 64;   // thread-maximum histogram: bins of width 1 in log2 units
constexpr int kLMax = 64;   // max chunk loads per thread (V <= kLMax * NT * EPV)

struct SampleParams {
  const void* logits;
  int64_t B_src, V, ld;
  const float* temps;
  const int32_t* top_k;
  const float* top_p;
  const float* uniforms;
  const int32_t* row_idx;
  const int32_t* n_rows_dev;
  int32_t* out;
};

// exp of the scaled, max-shifted logit.  The clamp folds into v_exp_f32 and
// maps NaN (from a NaN logit) to 0.
__device__ __forceinline__ float ex2c(float y) {
  return __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(y), 0.0f, 1.0f);
}

template <typename T>
__device__ __forceinline__ float esum_chunk(const uint4& v, float gm, float c) {
  constexpr int EPV = Elem<T>::EPV;
  float e[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) e[i] = ex2c((Elem<T>::get(v, i) - gm) * c);
#pragma unroll
  for (int w = 1; w < EPV; w <<= 1)
#pragma unroll
    for (int i = 0; i < EPV; i += 2 * w) e[i] += e[i + w];
  return e[0];
}

// Same, counting only elements with x >= thr.
template <typename T>
__device__ __forceinline__ float esum_chunk_ge(const uint4& v, float gm, float c, float thr) {
  constexpr int EPV = Elem<T>::EPV;
  float e[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const float x = Elem<T>::get(v, i);
    e[i] = x >= thr ? ex2c((x - gm) * c) : 0.0f;
  }
#pragma unroll
  for (int w = 1; w < EPV; w <<= 1)
#pragma unroll
    for (int i = 0; i < EPV; i += 2 * w) e[i] += e[i + w];
  return e[0];
}

template <typename T>
__device__ __forceinline__ int count_chunk_ge(const uint4& v, float thr) {
  int n = 0;
#pragma unroll
  for (int i = 0; i < Elem<T>::EPV; ++i) n += Elem<T>::get(v, i) >= thr ? 1 : 0;
  return n;
}

// ---------------------------------------------------------------------------
// Row access.  Wave-blocked layout: wave w owns chunks [w*L*64, (w+1)*L*64);
// its j-th load reads the 64 consecutive chunks (w*L + j)*64 + lane (1 KiB).
// Index order is therefore (wave, j, lane, element).
// ---------------------------------------------------------------------------
template <typename T, int NT, bool VEC>
struct RowBase {
  static constexpr int EPV = Elem<T>::EPV;
  const char* base;
  uint32_t V;
  int L;
  uint32_t c0;  // chunk index of this thread's j = 0 load
  __device__ __forceinline__ void init(const void* logits, int64_t r, int64_t ld, int64_t Vv) {
    base = reinterpret_cast<const char*>(logits) + r * ld * (int64_t)Elem<T>::kSize;
    V = (uint32_t)Vv;
    const uint32_t NV = (V + EPV - 1) / EPV;
    L = (int)((NV + NT - 1) / NT);
    c0 = (uint32_t)(threadIdx.x >> 6) * (uint32_t)L * kWave + (threadIdx.x & 63);
  }
  __device__ __forceinline__ uint32_t chunk_index(int j) const { return c0 + (uint32_t)j * kWave; }
  __device__ __forceinline__ uint4 load(int j) const {
    return load_chunk32<T, VEC>(base, chunk_index(j), V);
  }
  __device__ __forceinline__ uint32_t elem_index(int j, int i) const {
    return chunk_index(j) * EPV + (uint32_t)i;
  }
};

// Chunk maxima in registers.  For 16-bit inputs the maximum is an exact input
// value, so two are packed per VGPR (raw 16-bit patterns).
template <typename T, int CAP>
struct ChunkMax {
  static constexpr int N = (CAP + 1) / 2;
  uint32_t w[N];
  __device__ __forceinline__ float get(int j) const {
    uint4 v;
    v.x = w[j >> 1] >> ((j & 1) * 16);
    return Elem<T>::get(v, 0);
  }
  __device__ __forceinline__ void set(int j, float m) {
    uint32_t bits;
    if constexpr (sizeof(T) == 2 && Elem<T>::EPV == 8 && std::is_same<T, bf16_t>::value)
      bits = __float_as_uint(m) >> 16;
    else
      bits = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)m);
    if (j & 1) w[j >> 1] = (w[j >> 1] & 0x0000ffffu) | (bits << 16);
    else w[j >> 1] = (w[j >> 1] & 0xffff0000u) | bits;
  }
  __device__ __forceinline__ void launder() {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(w[i]));
  }
};
template <int CAP>
struct ChunkMax<float, CAP> {
  float m[CAP];
  __device__ __forceinline__ float get(int j) const { return m[j]; }
  __device__ __forceinline__ void set(int j, float v) { m[j] = v; }
  __device__ __forceinline__ void launder() {
#pragma unroll
    for (int i = 0; i < CAP; ++i) asm volatile("" : "+v"(m[i]));
  }
};

// Row copy in registers for j < CAP (+ chunk maxima); j >= CAP streams.
template <typename T, int NT, int CAP, bool VEC>
struct RegRow : RowBase<T, NT, VEC> {
  using B = RowBase<T, NT, VEC>;
  uint4 d[CAP];
  ChunkMax<T, CAP> cm;
  __device__ __forceinline__ void fetch() {
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      if (j < B::L) d[j] = B::load(j);
  }
  // Tell the compiler the register copy may have changed, so values derived
  // from it (unpacked floats) are recomputed per pass instead of being hoisted
  // and kept live across passes (which would double the register footprint).
  __device__ __forceinline__ void launder() {
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      asm volatile("" : "+v"(d[j].x), "+v"(d[j].y), "+v"(d[j].z), "+v"(d[j].w));
    cm.launder();
  }
  // Apply f(j, chunk, chunk_max) to every chunk this thread owns, in index order.
  template <class F>
  __device__ __forceinline__ void each(F&& f) {
    launder();
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      if (j < B::L) f(j, d[j], cm.get(j));
    for (int j = CAP; j < B::L; ++j) {
      const uint4 v = B::load(j);
      f(j, v, chunk_max<T>(v));
    }
  }
  // Chunk with a runtime (workgroup-uniform) index, built with masked ORs: a
  // select chain would be folded back into a dynamic index, which moves d[] to
  // scratch memory.
  __device__ __forceinline__ uint4 chunk(int j) const {
    if (j >= CAP) return B::load(j);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int jj = 0; jj < CAP; ++jj) {
      const uint32_t m = 0u - (uint32_t)(jj == j);
      v.x |= d[jj].x & m;
      v.y |= d[jj].y & m;
      v.z |= d[jj].z & m;
      v.w |= d[jj].w & m;
    }
    return v;
  }
};

// Row re-read from global memory on every pass (exact slow path).
template <typename T, int NT, bool VEC>
struct MemRow : RowBase<T, NT, VEC> {
  using B = RowBase<T, NT, VEC>;
  template <class F>
  __device__ __forceinline__ void each(F&& f) {
    for (int j = 0; j < B::L; ++j) {
      const uint4 v = B::load(j);
      f(j, v, chunk_max<T>(v));
    }
  }
  __device__ __forceinline__ uint4 chunk(int j) const { return B::load(j); }
};

// argmax with torch semantics.  gm is the NaN-ignoring maximum, tm this
// thread's.  Returns the id (identical in every thread).
template <int NW, typename T, class Row>
__device__ __forceinline__ int32_t row_argmax(Row& R, float tm, float gm, double* red) {
  constexpr int EPV = Elem<T>::EPV;
  int nan = 0;
  R.each([&](int, const uint4& v, float) {
#pragma unroll
    for (int i = 0; i < EPV; ++i) nan |= __builtin_isnan(Elem<T>::get(v, i)) ? 1 : 0;
  });
  const int gnan = wg_max_i<NW>(nan, red);
  int first = 0x7fffffff;
  if (gnan ? nan : (tm == gm)) {
    R.each([&](int j, const uint4& v, float) {
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const float x = Elem<T>::get(v, i);
        const bool hit = gnan ? __builtin_isnan(x) : (x == gm);
        const uint32_t idx = R.elem_index(j, i);
        if (hit && first == 0x7fffffff && idx < R.V) first = (int)idx;
      }
    });
  }
  return wg_min_i<NW>(first, red);
}

// Resolve the output row b -> source row r; -1: skip the row, -2: invalid
// gather index (the output gets -1).
__device__ __forceinline__ int64_t resolve_row(const SampleParams& P, int b) {
  if (P.n_rows_dev && b >= *P.n_rows_dev) return -1;
  const int64_t r = P.row_idx ? (int64_t)P.row_idx[b] : (int64_t)b;
  if (r < 0 || r >= P.B_src) return -2;
  return r;
}

// ---------------------------------------------------------------------------
// Exact threshold search by bisection over order-preserving float keys.
// Returns thr: keep-mask x >= thr (top-k, then top-p within it).
// ---------------------------------------------------------------------------
template <int NW, typename T, class Row>
__device__ float select_exact(Row& R, float gm, float c, double Z, bool kon, int32_t k, bool pon,
                              float p, double* red) {
  float floor_thr = -INFINITY;
  if (kon) {
    uint32_t lo = okey(-INFINITY), hi = okey(gm) + 1u;
    while (hi - lo > 1u) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      const float th = okey_inv(mid);
      int n = 0;
      R.each([&](int, const uint4& v, float cmj) {
        if (cmj >= th) n += count_chunk_ge<T>(v, th);
      });
      if (wg_sum_i<NW>(n, red) >= k) lo = mid;
      else hi = mid;
    }
    floor_thr = okey_inv(lo);
  }
  if (!pon) return floor_thr;
  double zk = Z;
  if (kon) {
    double acc = 0.0;
    R.each([&](int, const uint4& v, float cmj) {
      if (cmj >= floor_thr) acc += (double)esum_chunk_ge<T>(v, gm, c, floor_thr);
    });
    zk = wg_sum<NW>(acc, red);
  }
  const double target = (double)p * zk;
  uint32_t lo = okey(floor_thr), hi = okey(gm) + 1u;
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    const float th = okey_inv(mid);
    double ms = 0.0;
    R.each([&](int, const uint4& v, float cmj) {
      if (cmj >= th) ms += (double)esum_chunk_ge<T>(v, gm, c, th);
    });
    if (wg_sum<NW>(ms, red) >= target) lo = mid;
    else hi = mid;
  }
  return okey_inv(lo);
}

// ---------------------------------------------------------------------------
// Inverse CDF in ascending index order over {x >= thr} (all when !masked).
// Index order is (wave, j, lane, element): find the wave whose prefix crosses
// U = u * total, then (inside that wave only) the column j, then the lane,
// then the element.  Every level reuses the same chunk masses summed in a
// fixed order, so the walk is deterministic.  s_cs[j*NT + t] holds the chunk
// masses for j < CAP (filled here unless cs_valid).
// ---------------------------------------------------------------------------
template <int NT, int CAP, typename T, class Row>
__device__ __forceinline__ void cdf_pick(Row& R, float gm, float c, bool masked, float thr,
                                         bool cs_valid, double tmass_valid, float u, float* s_cs,
                                         double* s_col, int32_t* out) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  double tmass = tmass_valid;
  if (!cs_valid) {
    tmass = 0.0;
    R.each([&](int j, const uint4& v, float cmj) {
      const float s = masked ? (cmj >= thr ? esum_chunk_ge<T>(v, gm, c, thr) : 0.0f)
                             : esum_chunk<T>(v, gm, c);
      if (j < CAP) s_cs[j * NT + t] = s;
      tmass += (double)s;
    });
  }
  {
    const double ws = wave_sum(tmass);
    if (lane == 0) s_col[wid] = ws;
  }
  __syncthreads();
  // Wave totals in index order: lane w of every wave holds wave w's total and
  // a wave scan gives the prefixes (identical in every wave).
  int wstar;
  double base, U;
  {
    const double sw = lane < NW ? s_col[lane] : 0.0;
    const double inc = wave_incl_scan(sw, lane);
    const double total = uni(__shfl(inc, NW - 1));
    U = (double)u * total;
    const double exc = inc - sw;  // only compared, never accumulated further
    const uint64_t cross = __ballot(lane < NW && inc > U);
    if (cross) {
      wstar = __ffsll((unsigned long long)cross) - 1;
    } else {  // u >= 1 or rounding: the last wave with mass
      const uint64_t pos = __ballot(lane < NW && sw > 0.0);
      wstar = pos ? 63 - __clzll((long long)pos) : 0;
    }
    (void)exc;
    double ex = __shfl_up(inc, 1);
    if (lane == 0) ex = 0.0;
    base = uni(__shfl(ex, wstar));
  }
  if (wid != wstar) return;
  auto colmass = [&](int j) -> float {
    if (j < CAP) return s_cs[j * NT + t];
    const uint4 v = R.chunk(j);
    return masked ? esum_chunk_ge<T>(v, gm, c, thr) : esum_chunk<T>(v, gm, c);
  };
  // column j inside the wave (sequential; one column mass at a time)
  int jstar = -1, jlast = 0;
  double jbase = base, cum = base;
  for (int j = 0; j < R.L; ++j) {
    const double col = wave_sum((double)colmass(j));
    if (col > 0.0) jlast = j;
    if (jstar < 0 && cum + col > U) {
      jstar = j;
      jbase = cum;
    }
    cum += col;
  }
  if (jstar < 0) {
    jstar = jlast;
    jbase = base;
    for (int j = 0; j < jlast; ++j) jbase += wave_sum((double)colmass(j));
  }
  // lane inside the column
  const float sme = colmass(jstar);
  const double incl = wave_incl_scan((double)sme, lane);
  double excl = __shfl_up(incl, 1);
  if (lane == 0) excl = 0.0;
  const bool cross = (sme > 0.0f) && (jbase + excl <= U) && (jbase + incl > U);
  const uint64_t bal = __ballot(cross);
  int owner;
  if (bal) {
    owner = __ffsll((unsigned long long)bal) - 1;
  } else {
    const uint64_t pos = __ballot(sme > 0.0f);
    owner = pos ? 63 - __clzll((long long)pos) : 0;
  }
  if (lane == owner) {
    const uint4 vj = R.chunk(jstar);
    double acc = jbase + excl;
    int pick = -1, lastpos = -1;
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      const float x = Elem<T>::get(vj, i);
      const float e = (!masked || x >= thr) ? ex2c((x - gm) * c) : 0.0f;
      if (e > 0.0f) {
        lastpos = i;
        acc += (double)e;
        if (pick < 0 && acc > U) pick = i;
      }
    }
    if (pick < 0) pick = lastpos < 0 ? 0 : lastpos;
    *out = (int32_t)R.elem_index(jstar, pick);
  }
}

// ---------------------------------------------------------------------------
// Greedy kernel: every row is argmax (Sampler.sample with temperatures None).
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC>
__global__ __launch_bounds__(NT) void greedy_kernel(SampleParams P) {
  constexpr int NW = NT / kWave;
  __shared__ double red[NW];
  const int b = blockIdx.x;
  const int64_t r = resolve_row(P, b);
  if (r == -1) return;
  if (r == -2) {
    if (threadIdx.x == 0) P.out[b] = -1;
    return;
  }
  RegRow<T, NT, CAP, VEC> R;
  R.init(P.logits, r, P.ld, P.V);
  R.fetch();
  float tm = -INFINITY;
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    if (j < R.L) {
      const float m = chunk_max<T>(R.d[j]);
      R.cm.set(j, m);
      tm = fmaxf(tm, m);
    }
  for (int j = CAP; j < R.L; ++j) tm = fmaxf(tm, chunk_max<T>(R.load(j)));
  const float gm = wg_max<NW>(tm, red);
  const int32_t id = row_argmax<NW, T>(R, tm, gm, red);
  if (threadIdx.x == 0) P.out[b] = id;
}

// ---------------------------------------------------------------------------
// Sampling kernel.
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 8)))
void sample_kernel(SampleParams P) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  constexpr int kWin = NT;  // candidate window: one entry per thread
  __shared__ double red[NW];
  __shared__ double s_col[NW];
  __shared__ float s_cs[CAP * NT];  // chunk masses, [j][t]
  __shared__ int s_hcnt[kBins];
  __shared__ float s_hmass[kBins];
  __shared__ uint64_t s_wkey[kWin];
  __shared__ uint64_t s_sorted[kWin];
  __shared__ int s_wn;
  __shared__ int s_pick;

  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int b = blockIdx.x;
  const int64_t r = resolve_row(P, b);
  if (r == -1) return;
  if (r == -2) {
    if (t == 0) P.out[b] = -1;
    return;
  }

  RegRow<T, NT, CAP, VEC> R;
  R.init(P.logits, r, P.ld, P.V);
  R.fetch();

  // ---- pass A: chunk maxima and the row maximum --------------------------
  float tm = -INFINITY;
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    if (j < R.L) {
      const float m = chunk_max<T>(R.d[j]);
      R.cm.set(j, m);
      tm = fmaxf(tm, m);
    }
  for (int j = CAP; j < R.L; ++j) tm = fmaxf(tm, chunk_max<T>(R.load(j)));
  const float gm = wg_max<NW>(tm, red);

  const float Tr = uni(P.temps[r]);
  if (!(Tr > 0.0f) || !(Tr < INFINITY) || !(gm > -INFINITY) || !(gm < INFINITY)) {
    // argmax rows inside a sampling batch are rare; re-read the row instead of
    // keeping this path's registers alongside the sampling path's.
    MemRow<T, NT, VEC> M;
    M.init(P.logits, r, P.ld, P.V);
    const int32_t id = row_argmax<NW, T>(M, tm, gm, red);
    if (t == 0) P.out[b] = id;
    return;
  }
  const float c = kLog2e / Tr;
  const float u = uni(P.uniforms[r]);

  // ---- pass B: softmax normaliser; chunk masses kept in LDS for the CDF ---
  R.launder();
  double zt = 0.0;
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    if (j < R.L) {
      const float s = esum_chunk<T>(R.d[j], gm, c);
      s_cs[j * NT + t] = s;
      zt += (double)s;
    }
  for (int j = CAP; j < R.L; ++j) zt += (double)esum_chunk<T>(R.load(j), gm, c);
  const double Z = wg_sum<NW>(zt, red);

  const int32_t k = uni(P.top_k ? P.top_k[r] : 0);
  const float p = uni(P.top_p ? P.top_p[r] : 1.0f);
  const bool kon = k >= 1 && (int64_t)k < (int64_t)R.V;
  const bool pon = p < 1.0f;

  if (!kon && !pon) {
    cdf_pick<NT, CAP, T>(R, gm, c, false, -INFINITY, true, zt, u, s_cs, s_col, &P.out[b]);
    return;
  }

  // ---- fast path: a candidate window bounded by the thread maxima ----------
  // Every thread maximum is a distinct element, so the window {y >= lo} holds
  // >= k elements once >= k thread maxima have y >= lo, and holds mass >= p*Z
  // once the thread maxima with y >= lo carry that much mass.
  if (t < kBins) {
    s_hcnt[t] = 0;
    s_hmass[t] = 0.0f;
  }
  if (t == 0) s_wn = 0;
  __syncthreads();
  {
    const float ytm = (tm - gm) * c;
    if (ytm >= -64.0f) {
      const int bin = min(kBins - 1, (int)(-ytm));
      atomicAdd(&s_hcnt[bin], 1);
      atomicAdd(&s_hmass[bin], ex2c(ytm));
    }
  }
  __syncthreads();
  if (wid == 0) {
    const int pc = wave_incl_scan_i(s_hcnt[lane], lane);
    const double pm = wave_incl_scan((double)s_hmass[lane], lane);
    const bool ok = kon ? (pc >= k) : (pm >= (double)p * Z);
    const uint64_t bal = __ballot(ok);
    if (lane == 0) s_pick = bal ? (__ffsll((unsigned long long)bal) - 1) : (kBins - 1);
  }
  __syncthreads();
  const float lo_y = -(float)(uni(s_pick) + 1);

  // collect the window (chunk maxima prune almost every chunk)
  R.each([&](int j, const uint4& v, float cmj) {
    if ((cmj - gm) * c >= lo_y) {
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const float x = Elem<T>::get(v, i);
        if ((x - gm) * c >= lo_y) {
          const int pos = atomicAdd(&s_wn, 1);
          if (pos < kWin) {
            const uint32_t idx = R.elem_index(j, i);
            s_wkey[pos] = ((uint64_t)okey(x) << 32) | (uint64_t)(0xffffffffu - idx);
          }
        }
      }
    }
  });
  __syncthreads();
  const int nw = uni(s_wn);
  bool ok = nw <= kWin;
  float thr = -INFINITY;
  if (ok) {
    // rank by counting (keys are unique), scatter into descending order
    if (t < nw) {
      const uint64_t mine = s_wkey[t];
      int rank = 0;
      for (int q = 0; q < nw; ++q) rank += s_wkey[q] > mine ? 1 : 0;
      s_sorted[rank] = mine;
    }
    __syncthreads();
    const uint64_t key = t < nw ? s_sorted[t] : 0ull;
    const uint32_t kx = (uint32_t)(key >> 32);
    const float x = okey_inv(kx);
    const float e = t < nw ? ex2c((x - gm) * c) : 0.0f;
    double pre, tot;
    wg_scan<NW>((double)e, red, &pre, &tot);  // pre = inclusive prefix in sorted order
    double ZK = Z;
    int limit = nw;
    if (kon) {
      // k-th largest value (nw >= k unless the window hit the y >= -64 cutoff,
      // in which case every element of the top-k set with non-negligible mass
      // is in the window)
      uint32_t kk;
      if (k <= nw) {
        if (t == k - 1) s_pick = (int)kx;
        __syncthreads();
        kk = uni((uint32_t)s_pick);
      } else {
        kk = uni((uint32_t)(s_sorted[nw - 1] >> 32));
      }
      const int inK = (t < nw && kx >= kk) ? 1 : 0;
      limit = wg_sum_i<NW>(inK, red);
      thr = uni(okey_inv(kk));
      ZK = wg_sum<NW>((t == limit - 1) ? pre : 0.0, red);  // inclusive prefix at limit-1
    }
    if (pon) {
      const double target = (double)p * ZK;
      const int first = (t < limit && pre >= target) ? t : 0x7fffffff;
      const int q = wg_min_i<NW>(first, red);
      if (q == 0x7fffffff) {
        ok = false;  // the window does not reach the top-p mass: exact path
      } else {
        if (t == q) s_pick = (int)kx;
        __syncthreads();
        thr = uni(okey_inv((uint32_t)s_pick));
      }
    }
    __syncthreads();
  }

  if (ok) {
    cdf_pick<NT, CAP, T>(R, gm, c, true, thr, false, 0.0, u, s_cs, s_col, &P.out[b]);
  } else {
    // Exact path on a global-memory view of the row (the register copy is
    // dead from here on, which keeps this path off the hot path's registers).
    MemRow<T, NT, VEC> M;
    M.init(P.logits, r, P.ld, P.V);
    thr = select_exact<NW, T>(M, gm, c, Z, kon, k, pon, p, red);
    cdf_pick<NT, CAP, T>(M, gm, c, true, thr, false, 0.0, u, s_cs, s_col, &P.out[b]);
  }
}

// ---------------------------------------------------------------------------
// Host launch.
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP>
static void launch_t(const SampleParams& P, int64_t B_out, bool greedy, bool vec,
                     hipStream_t st) {
  const dim3 grid((unsigned)B_out), block(NT);
  if (greedy) {
    if (vec) hipLaunchKernelGGL((greedy_kernel<T, NT, CAP, true>), grid, block, 0, st, P);
    else hipLaunchKernelGGL((greedy_kernel<T, NT, CAP, false>), grid, block, 0, st, P);
  } else {
    if (vec) hipLaunchKernelGGL((sample_kernel<T, NT, CAP, true>), grid, block, 0, st, P);
    else hipLaunchKernelGGL((sample_kernel<T, NT, CAP, false>), grid, block, 0, st, P);
  }
}

template <typename T>
static int launch_dtype(const SampleParams& P, int64_t B_out, bool greedy, bool vec,
                        hipStream_t st) {
  constexpr int EPV = Elem<T>::EPV;
  const int64_t NV = (P.V + EPV - 1) / EPV;
  // Workgroup size: the row fits in registers when NV <= NT * CAP.
  if (NV <= 256 * 8) launch_t<T, 256, 8>(P, B_out, greedy, vec, st);
  else if (NV <= 512 * 16) launch_t<T, 512, 16>(P, B_out, greedy, vec, st);
  else if (NV <= (int64_t)1024 * kLMax) launch_t<T, 1024, 16>(P, B_out, greedy, vec, st);
  else return set_error(LSG_ERR_ARG, "lsg_sample: V=%lld too large (max %lld elements)",
                        (long long)P.V, (long long)1024 * kLMax * EPV);
  return LSG_OK;
}

}  // namespace lsg

using namespace lsg;

extern "C" int lsg_sample(const void* logits, int dtype, int64_t B_src, int64_t V, int64_t ld,
                          const float* temperatures, const int32_t* top_k, const float* top_p,
                          const float* uniforms, const int32_t* row_idx, int64_t B_out,
                          const int32_t* n_rows_dev, int32_t* out_ids, void* stream) {
  clear_error();
  if (!logits || !out_ids) return set_error(LSG_ERR_ARG, "lsg_sample: null logits/out_ids");
  if (V < 1 || B_src < 0 || B_out < 0 || ld < V)
    return set_error(LSG_ERR_ARG, "lsg_sample: bad shape B_src=%lld V=%lld ld=%lld B_out=%lld",
                     (long long)B_src, (long long)V, (long long)ld, (long long)B_out);
  if (!row_idx && B_out > B_src)
    return set_error(LSG_ERR_ARG, "lsg_sample: B_out=%lld > B_src=%lld without row_idx",
                     (long long)B_out, (long long)B_src);
  if (B_out > 0x7fffffffLL) return set_error(LSG_ERR_ARG, "lsg_sample: B_out too large");
  if (temperatures && !uniforms)
    return set_error(LSG_ERR_ARG, "lsg_sample: non-greedy sampling needs uniforms");
  if (dtype != kF32 && dtype != kBF16 && dtype != kF16)
    return set_error(LSG_ERR_ARG, "lsg_sample: unknown dtype %d", dtype);
  if (B_out == 0) return LSG_OK;
  const size_t es = dtype == kF32 ? 4 : 2;
  const bool vec = ((uintptr_t)logits % 16 == 0) && ((ld * (int64_t)es) % 16 == 0);
  SampleParams P{logits, B_src, V, ld, temperatures, top_k, top_p, uniforms,
                 row_idx, n_rows_dev, out_ids};
  const bool greedy = temperatures == nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (dtype == kF32) rc = launch_dtype<float>(P, B_out, greedy, vec, st);
  else if (dtype == kBF16) rc = launch_dtype<bf16_t>(P, B_out, greedy, vec, st);
  else rc = launch_dtype<f16_t>(P, B_out, greedy, vec, st);
  if (rc != LSG_OK) return rc;
  return check_launch("lsg_sample");
}
