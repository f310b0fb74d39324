// Token sampling over the vocabulary: greedy argmax, temperature softmax,
// top-k, top-p and one inverse-CDF draw per row with an explicit uniform.
//
// Replaces, for the decode token path of Loop-SGLang:
//   Sampler.sample            python/loopsgl/model_executor/sample.py:107-112
//   torch.argmax (greedy)     sample.py:110-111 (+ int32 cast, model_runner.py:279-280)
//   sample_impl -> flashinfer softmax / *_sampling_from_probs   sample.py:60-81
//
// One workgroup samples one row at a time.  The row is read from HBM exactly
// once with coalesced 128-bit loads (wave w owns a contiguous span of the row
// and reads it 1 KiB per instruction) and stays in VGPRs (CAP chunks of 16 B
// per thread); the later passes (softmax normaliser, threshold search, CDF
// walk) run on registers and LDS.  For rows that fit twice in the register
// budget the kernel is persistent and double-buffered: while a workgroup works
// on one row, the loads of its next row are already in flight, so HBM streams
// continuously.  Chunks past NT*CAP (very large V), and the rare exact slow
// path of the threshold search, re-read the row from global memory.
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

#include <algorithm>
#include <type_traits>

namespace lsg {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kBins = 64;   // thread-maximum histogram: bins of width 1 in log2 units

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
    V = (uint32_t)uni((uint32_t)Vv);
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
  // Registers from a row staged in LDS (chunk c at s_row[c]); partial and
  // padding chunks, which the staging loads skipped, come from global memory.
  __device__ __forceinline__ void fetch_staged(const uint4* s_row) {
    constexpr int EPV = Elem<T>::EPV;
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      if (j < B::L) {
        const uint32_t c = B::chunk_index(j);
        d[j] = (c * EPV + EPV <= B::V) ? s_row[c] : B::load(j);
      }
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

// LDS shared by the per-row routines (one row at a time per workgroup).
template <int NT>
struct Smem {
  static constexpr int NW = NT / kWave;
  static constexpr int kWin = NT < 512 ? NT : 512;  // candidate window capacity
  double red[NW];
  double col[NW];
  int hcnt[kBins];
  float hmass[kBins];
  uint64_t wkey[kWin];    // candidate window (unsorted)
  uint64_t sorted[kWin];  // candidate window in descending key order
  int wn;
  int pick;
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
// then the element.  The wave that holds the crossing recomputes its chunk
// masses with the same arithmetic that produced the totals, so every level
// sees identical values and the walk is deterministic.  tmass is this
// thread's mass (all its chunks, masked like the walk).
// ---------------------------------------------------------------------------
template <int NT, typename T, class Row>
__device__ __forceinline__ void cdf_pick(Row& R, float gm, float c, bool masked, float thr,
                                         double tmass, float u, Smem<NT>& S, int32_t* out) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  {
    const double ws = wave_sum(tmass);
    if (lane == 0) S.col[wid] = ws;
  }
  __syncthreads();
  // Wave totals in index order: lane w of every wave holds wave w's total and a
  // wave scan gives the prefixes (identical in every wave).
  int wstar;
  double base, U;
  {
    const double sw = lane < NW ? S.col[lane] : 0.0;
    const double inc = wave_incl_scan(sw, lane);
    const double total = readlane_d(inc, NW - 1);
    U = (double)u * total;
    const uint64_t cross = __ballot(lane < NW && inc > U);
    if (cross) {
      wstar = __ffsll((unsigned long long)cross) - 1;
    } else {  // u >= 1 or rounding: the last wave with mass
      const uint64_t pos = __ballot(lane < NW && sw > 0.0);
      wstar = pos ? 63 - __clzll((long long)pos) : 0;
    }
    wstar = uni(wstar);
    base = readlane_d(wave_shr1(inc), wstar);
  }
  if (wid != wstar) return;
  // column j inside the wave: one pass over this wave's chunks in index order
  int jstar = -1, jlast = 0;
  double jbase = base, cum = base, cum_last = base;
  float sme = 0.0f, slast = 0.0f;
  R.each([&](int j, const uint4& v, float cmj) {
    const float sj = masked ? (cmj >= thr ? esum_chunk_ge<T>(v, gm, c, thr) : 0.0f)
                            : esum_chunk<T>(v, gm, c);
    const double col = wave_sum((double)sj);
    if (col > 0.0) {
      jlast = j;
      slast = sj;
      cum_last = cum;
    }
    if (jstar < 0 && cum + col > U) {
      jstar = j;
      jbase = cum;
      sme = sj;
    }
    cum += col;
  });
  if (jstar < 0) {  // u >= 1 or rounding: the last column with mass
    jstar = jlast;
    jbase = cum_last;
    sme = slast;
  }
  jstar = uni(jstar);
  // lane inside the column
  const double incl = wave_incl_scan((double)sme, lane);
  const double excl = wave_shr1(incl);
  const uint64_t bal = __ballot((sme > 0.0f) && (jbase + incl > U));
  int owner;
  if (bal) {
    owner = __ffsll((unsigned long long)bal) - 1;
  } else {
    const uint64_t pos = __ballot(sme > 0.0f);
    owner = pos ? 63 - __clzll((long long)pos) : 0;
  }
  const uint4 vj = R.chunk(jstar);
  if (lane == owner) {
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
// Candidate window bounded by a histogram of distinct elements (the thread
// maxima, or the chunk maxima): since they are distinct elements, the window
// {y >= lo} holds >= k elements once >= k of them have y >= lo, and holds mass
// >= p*Z once those with y >= lo carry that much mass.  Returns the bin b (the
// window is y >= -(b+1)) or -1 when no bin reaches the target.
// ---------------------------------------------------------------------------
template <int NT>
__device__ __forceinline__ int window_bin(Smem<NT>& S, bool kon, int32_t k, float p, double Z) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (wid == 0) {
    const int pc = wave_incl_scan_i(S.hcnt[lane], lane);
    const double pm = wave_incl_scan((double)S.hmass[lane], lane);
    const bool ok = kon ? (pc >= k) : (pm >= (double)p * Z);
    const uint64_t bal = __ballot(ok);
    if (lane == 0) S.pick = bal ? (__ffsll((unsigned long long)bal) - 1) : -1;
  }
  __syncthreads();
  const int bin = uni(S.pick);
  __syncthreads();
  return bin;
}

__device__ __forceinline__ int ybin(float y) { return min(kBins - 1, (int)(-y)); }

// ---------------------------------------------------------------------------
// One sampling row: row r of the logits -> out[b].  Every path is uniform
// across the workgroup (all threads reach the same barriers).
// ---------------------------------------------------------------------------
struct RowArgs {
  float T, p, u;
  int32_t k;
};

__device__ __forceinline__ RowArgs row_args(const SampleParams& P, int64_t r) {
  RowArgs a;
  a.T = P.temps ? uni(P.temps[r]) : 0.0f;
  a.u = P.uniforms ? uni(P.uniforms[r]) : 0.0f;
  a.k = uni(P.top_k ? P.top_k[r] : 0);
  a.p = uni(P.top_p ? P.top_p[r] : 1.0f);
  return a;
}

// ---------------------------------------------------------------------------
// Rare rows, outside the hot path's register allocation: they re-read the row
// from global memory.
//   mode 0: argmax (T <= 0, or a non-finite maximum, inside a sampling batch)
//   mode 1: exact top-k / top-p threshold, then the masked CDF walk
// ---------------------------------------------------------------------------
template <typename T, int NT, bool VEC>
__device__ __attribute__((noinline)) void rare_row(const void* logits, int64_t r, int64_t ld,
                                                   int64_t V, int mode, float tm, float gm, float c,
                                                   double Z, int32_t k, float p, float u,
                                                   Smem<NT>* Sp, int32_t* out) {
  constexpr int NW = NT / kWave;
  Smem<NT>& S = *Sp;
  MemRow<T, NT, VEC> M;
  M.init(logits, r, ld, V);
  if (mode == 0) {
    const int32_t id = row_argmax<NW, T>(M, tm, gm, S.red);
    if (threadIdx.x == 0) *out = id;
    return;
  }
  const bool kon = k >= 1 && (int64_t)k < V, pon = p < 1.0f;
  const float thr = select_exact<NW, T>(M, gm, c, Z, kon, k, pon, p, S.red);
  double tmass = 0.0;
  M.each([&](int, const uint4& v, float cmj) {
    if (cmj >= thr) tmass += (double)esum_chunk_ge<T>(v, gm, c, thr);
  });
  cdf_pick<NT, T>(M, gm, c, true, thr, tmass, u, S, out);
}

// ---------------------------------------------------------------------------
// Greedy row: torch.argmax.  NaN-propagating maxima make a NaN anywhere the
// row maximum, so one pass finds both the maximum and whether NaN is present;
// the chunk maxima then point at the single chunk holding the first hit.
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC>
__device__ __forceinline__ void greedy_row(RegRow<T, NT, CAP, VEC>& R, int32_t* out, Smem<NT>& S) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  __syncthreads();
  float tm = -INFINITY;
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    if (j < R.L) {
      const float m = chunk_maximum<T>(R.d[j]);
      R.cm.set(j, m);
      tm = fmaximum(tm, m);
    }
  for (int j = CAP; j < R.L; ++j) tm = fmaximum(tm, chunk_maximum<T>(R.load(j)));
  const float gm = wg_maximum<NW>(tm, S.red);
  const bool isn = gm != gm;
  int first = 0x7fffffff;
  if (isn ? (tm != tm) : (tm == gm)) {
    R.each([&](int j, const uint4& v, float cmj) {
      if (first == 0x7fffffff && (j >= CAP || (isn ? cmj != cmj : cmj == gm))) {
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          const float x = Elem<T>::get(v, i);
          const uint32_t idx = R.elem_index(j, i);
          if (first == 0x7fffffff && (isn ? x != x : x == gm) && idx < R.V) first = (int)idx;
        }
      }
    });
  }
  const int32_t id = wg_min_i<NW>(first, S.red);
  if (threadIdx.x == 0) *out = id;
}

// ---------------------------------------------------------------------------
// One sampling row: row r of the logits -> *out.  Every path is uniform across
// the workgroup (all threads reach the same barriers).
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC>
__device__ __forceinline__ void sample_row(RegRow<T, NT, CAP, VEC>& R, const SampleParams& P,
                                           int64_t r, const RowArgs& A, int32_t* out, Smem<NT>& S) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  constexpr int kWin = Smem<NT>::kWin;
  const int t = threadIdx.x, wid = t >> 6;
  __syncthreads();  // the previous row's readers of S are done

  // ---- pass A: chunk maxima and the row maximum (NaN ignored) ------------
  float tm = -INFINITY;
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    if (j < R.L) {
      const float m = chunk_max<T>(R.d[j]);
      R.cm.set(j, m);
      tm = fmaxf(tm, m);
    }
  for (int j = CAP; j < R.L; ++j) tm = fmaxf(tm, chunk_max<T>(R.load(j)));
  const float gm = wg_max<NW>(tm, S.red);

  if (!(A.T > 0.0f) || !(A.T < INFINITY) || !(gm > -INFINITY) || !(gm < INFINITY)) {
    rare_row<T, NT, VEC>(P.logits, r, P.ld, P.V, 0, tm, gm, 0.0f, 0.0, 0, 1.0f, 0.0f, &S, out);
    return;
  }
  const float c = kLog2e / A.T;

  // ---- pass B: softmax normaliser ------------------------------------------
  R.launder();
  double zt = 0.0;
#pragma unroll
  for (int j = 0; j < CAP; ++j)
    if (j < R.L) zt += (double)esum_chunk<T>(R.d[j], gm, c);
  for (int j = CAP; j < R.L; ++j) zt += (double)esum_chunk<T>(R.load(j), gm, c);
  const double Z = wg_sum<NW>(zt, S.red);

  const int32_t k = A.k;
  const float p = A.p;
  const bool kon = k >= 1 && (int64_t)k < (int64_t)R.V;
  const bool pon = p < 1.0f;
  if (!kon && !pon) {
    cdf_pick<NT, T>(R, gm, c, false, -INFINITY, zt, A.u, S, out);
    return;
  }

  // ---- candidate window from the thread maxima, else the chunk maxima (two
  // heavy tokens can share a thread, rarely a 16-byte chunk) ----------------
  if (t < kBins) {
    S.hcnt[t] = 0;
    S.hmass[t] = 0.0f;
  }
  if (t == 0) S.wn = 0;
  __syncthreads();
  {
    const float ytm = (tm - gm) * c;
    if (ytm >= -64.0f) {
      atomicAdd(&S.hcnt[ybin(ytm)], 1);
      atomicAdd(&S.hmass[ybin(ytm)], ex2c(ytm));
    }
  }
  int bin = window_bin(S, kon, k, p, Z);
  if (bin < 0) {
    if (t < kBins) {
      S.hcnt[t] = 0;
      S.hmass[t] = 0.0f;
    }
    __syncthreads();
    R.each([&](int, const uint4&, float cmj) {
      const float y = (cmj - gm) * c;
      if (y >= -64.0f) {
        atomicAdd(&S.hcnt[ybin(y)], 1);
        atomicAdd(&S.hmass[ybin(y)], ex2c(y));
      }
    });
    bin = window_bin(S, kon, k, p, Z);
  }
  const float lo_y = -(float)((bin < 0 ? kBins - 1 : bin) + 1);

  // collect the window (chunk maxima prune almost every chunk)
  R.each([&](int j, const uint4& v, float cmj) {
    if ((cmj - gm) * c >= lo_y) {
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const float x = Elem<T>::get(v, i);
        if ((x - gm) * c >= lo_y) {
          const int pos = atomicAdd(&S.wn, 1);
          if (pos < kWin) {
            const uint32_t idx = R.elem_index(j, i);
            S.wkey[pos] = ((uint64_t)okey(x) << 32) | (uint64_t)(0xffffffffu - idx);
          }
        }
      }
    }
  });
  __syncthreads();
  const int nw = uni(S.wn);
  bool ok = nw <= kWin;
  float thr = -INFINITY;
  if (nw <= kWave) {
    // Small window: wave 0 ranks, scans and thresholds it alone.
    if (wid == 0) {
      const int lane = t;
      const uint64_t mine = lane < nw ? S.wkey[lane] : 0ull;
      int rank = 0;
      for (int q = 0; q < nw; ++q) {
        const uint64_t other = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(mine >> 32), q) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)(mine & 0xffffffffu), q);
        rank += other > mine ? 1 : 0;
      }
      if (lane < nw) S.sorted[rank] = mine;
      __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes are done
      const uint64_t key = lane < nw ? S.sorted[lane] : 0ull;
      const uint32_t kx = (uint32_t)(key >> 32);
      const float e = lane < nw ? ex2c((okey_inv(kx) - gm) * c) : 0.0f;
      const double pre = wave_incl_scan((double)e, lane);  // inclusive prefix in sorted order
      double ZK = Z;
      int limit = nw;
      float th = -INFINITY;
      if (kon) {
        const uint32_t kk = (uint32_t)__builtin_amdgcn_readlane((int)kx, (k <= nw ? k : nw) - 1);
        limit = __popcll(__ballot(lane < nw && kx >= kk));
        th = okey_inv(kk);
        ZK = readlane_d(pre, limit - 1);
      }
      int good = 1;
      if (pon) {
        const uint64_t hit = __ballot(lane < limit && pre >= (double)p * ZK);
        if (hit)
          th = okey_inv((uint32_t)__builtin_amdgcn_readlane((int)kx, __ffsll((unsigned long long)hit) - 1));
        else
          good = 0;
      }
      if (lane == 0) {
        S.pick = (int)__float_as_uint(th);
        S.wn = good;
      }
    }
    __syncthreads();
    thr = uni(__uint_as_float((uint32_t)S.pick));
    ok = uni(S.wn) != 0;
  } else if (ok) {
    // rank by counting (keys are unique), scatter into descending order
    if (t < nw) {
      const uint64_t mine = S.wkey[t];
      int rank = 0;
      for (int q = 0; q < nw; ++q) rank += S.wkey[q] > mine ? 1 : 0;
      S.sorted[rank] = mine;
    }
    __syncthreads();
    const uint64_t key = t < nw ? S.sorted[t] : 0ull;
    const uint32_t kx = (uint32_t)(key >> 32);
    const float e = t < nw ? ex2c((okey_inv(kx) - gm) * c) : 0.0f;
    double pre, tot;
    wg_scan<NW>((double)e, S.red, &pre, &tot);  // pre = inclusive prefix in sorted order
    double ZK = Z;
    int limit = nw;
    if (kon) {
      // k-th largest value (nw >= k unless the window hit the y >= -64 cutoff,
      // in which case every top-k element with non-negligible mass is in it)
      uint32_t kk;
      if (k <= nw) {
        if (t == k - 1) S.pick = (int)kx;
        __syncthreads();
        kk = uni((uint32_t)S.pick);
      } else {
        kk = uni((uint32_t)(S.sorted[nw - 1] >> 32));
      }
      const int inK = (t < nw && kx >= kk) ? 1 : 0;
      limit = wg_sum_i<NW>(inK, S.red);
      thr = uni(okey_inv(kk));
      ZK = wg_sum<NW>((t == limit - 1) ? pre : 0.0, S.red);  // inclusive prefix at limit-1
    }
    if (pon) {
      const int first = (t < limit && pre >= (double)p * ZK) ? t : 0x7fffffff;
      const int q = wg_min_i<NW>(first, S.red);
      if (q == 0x7fffffff) {
        ok = false;  // the window does not reach the top-p mass: exact path
      } else {
        if (t == q) S.pick = (int)kx;
        __syncthreads();
        thr = uni(okey_inv((uint32_t)S.pick));
      }
    }
    __syncthreads();
  }

  if (ok) {
    double tmass = 0.0;
    R.each([&](int, const uint4& v, float cmj) {
      if (cmj >= thr) tmass += (double)esum_chunk_ge<T>(v, gm, c, thr);
    });
    cdf_pick<NT, T>(R, gm, c, true, thr, tmass, A.u, S, out);
  } else {
    rare_row<T, NT, VEC>(P.logits, r, P.ld, P.V, 1, tm, gm, c, Z, k, p, A.u, &S, out);
  }
}

// Output row b -> source row r: >= 0 valid, -1 past the end, -2 invalid gather index.
__device__ __forceinline__ int64_t source_row(const SampleParams& P, int64_t b, int64_t nrows) {
  if (b >= nrows) return -1;
  const int64_t r = P.row_idx ? (int64_t)P.row_idx[b] : b;
  return (r < 0 || r >= P.B_src) ? -2 : r;
}

template <bool GREEDY, typename T, int NT, int CAP, bool VEC>
__device__ __forceinline__ void handle_row(RegRow<T, NT, CAP, VEC>& R, const SampleParams& P,
                                           int64_t r, const RowArgs& A, int64_t b, Smem<NT>& S) {
  if (r == -2) {
    if (threadIdx.x == 0) P.out[b] = -1;
    return;
  }
  if (GREEDY) greedy_row(R, &P.out[b], S);
  else sample_row(R, P, r, A, &P.out[b], S);
}

// Issue the direct-to-LDS loads of a row: wave w's j-th load writes the 1 KiB
// of chunks (w*L + j)*64 + lane to s_row at the same chunk position.  Lanes
// whose chunk is partial or past the row end load a harmless in-row address;
// RegRow::fetch_staged replaces those chunks.
template <typename T, int NT, int CAP>
__device__ __forceinline__ void stage_row(const char* base, uint32_t V, int L, uint4* s_row) {
  constexpr int EPV = Elem<T>::EPV;
  const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    if (j < L) {
      const uint32_t c = (w * (uint32_t)L + (uint32_t)j) * kWave + lane;
      const bool full = c * EPV + EPV <= V;
      const char* src = base + (full ? (uint32_t)(c * 16u) : 0u);
      __builtin_amdgcn_global_load_lds(
          (const void*)src,
          (__attribute__((address_space(3))) void*)(s_row + (w * (uint32_t)L + (uint32_t)j) * kWave), 16, 0,
          0);
    }
  }
}

// Rows b = blockIdx.x, blockIdx.x + gridDim.x, ...
//   STAGED: persistent; the next row streams into LDS (direct-to-LDS loads)
//           while this row is processed from registers.
//   else:   one row per workgroup.
template <bool GREEDY, bool STAGED, typename T, int NT, int CAP, bool VEC>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4, 8)))
void sampler_kernel(SampleParams P) {
  __shared__ Smem<NT> S;
  int64_t nrows = P.B_out;
  if (P.n_rows_dev) nrows = min(nrows, (int64_t)uni(*P.n_rows_dev));
  int64_t b = blockIdx.x;
  if constexpr (!STAGED) {
    const int64_t r = source_row(P, b, nrows);
    if (r == -1) return;
    RegRow<T, NT, CAP, VEC> R;
    RowArgs A{};
    if (r >= 0) {
      A = row_args(P, r);
      R.init(P.logits, r, P.ld, P.V);
      R.fetch();
    }
    handle_row<GREEDY>(R, P, r, A, b, S);
  } else {
    __shared__ uint4 s_row[NT * CAP];
    const int64_t G = gridDim.x;
    int64_t r = source_row(P, b, nrows);
    RegRow<T, NT, CAP, VEC> R;
    if (r >= 0) {
      R.init(P.logits, r, P.ld, P.V);
      stage_row<T, NT, CAP>(R.base, R.V, R.L, s_row);
    }
    while (r != -1) {
      // per-row arguments first: their loads then never queue behind the
      // staging loads of the next row
      RowArgs A{};
      if (r >= 0) A = row_args(P, r);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();  // the staged row is complete and visible
      if (r >= 0) {
        R.init(P.logits, r, P.ld, P.V);
        R.fetch_staged(s_row);
      }
      __syncthreads();  // every wave has read s_row
      const int64_t bn = b + G;
      const int64_t rn = source_row(P, bn, nrows);
      if (rn >= 0) {
        RowBase<T, NT, VEC> N;
        N.init(P.logits, rn, P.ld, P.V);
        stage_row<T, NT, CAP>(N.base, N.V, N.L, s_row);
      }
      handle_row<GREEDY>(R, P, r, A, b, S);
      b = bn;
      r = rn;
    }
  }
}

// ---------------------------------------------------------------------------
// Host launch.
// ---------------------------------------------------------------------------
static int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

template <bool GREEDY, bool STAGED, typename T, int NT, int CAP, bool VEC>
static void launch_k(const SampleParams& P, hipStream_t st) {
  int64_t grid = P.B_out;
  if (STAGED) {
    // persistent: as many workgroups as fit at once (LDS and registers allow
    // one 1024-thread or four 256-thread workgroups per CU)
    const int per_cu = NT >= 1024 ? 1 : 4;
    grid = std::min<int64_t>(P.B_out, (int64_t)num_cus() * per_cu);
  }
  hipLaunchKernelGGL((sampler_kernel<GREEDY, STAGED, T, NT, CAP, VEC>), dim3((unsigned)grid), dim3(NT), 0,
                     st, P);
}

template <typename T>
static int launch_dtype(const SampleParams& P, bool greedy, bool vec, hipStream_t st) {
  constexpr int EPV = Elem<T>::EPV;
  const int64_t NV = (P.V + EPV - 1) / EPV;
  // The row lives in registers when NV <= NT * CAP.  Aligned rows of up to
  // 8192 chunks (128 KiB) use the persistent kernel with LDS staging; longer
  // rows stream the chunks past NT * CAP.  Chunk byte offsets are 32-bit.
  if (NV >= (int64_t)1 << 27)
    return set_error(LSG_ERR_ARG, "lsg_sample: V=%lld too large", (long long)P.V);
  auto go = [&](auto greedy_tag) {
    constexpr bool G = decltype(greedy_tag)::value;
    if (!vec) launch_k<G, false, T, 1024, 16, false>(P, st);
    else if (NV <= 256 * 8) launch_k<G, true, T, 256, 8, true>(P, st);
    else if (NV <= 1024 * 8) launch_k<G, true, T, 1024, 8, true>(P, st);
    else launch_k<G, false, T, 1024, 16, true>(P, st);
  };
  if (greedy) go(std::true_type{});
  else go(std::false_type{});
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
  SampleParams P{logits, B_src, V, ld, B_out, temperatures, top_k, top_p, uniforms,
                 row_idx, n_rows_dev, out_ids};
  const bool greedy = temperatures == nullptr;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  int rc;
  if (dtype == kF32) rc = launch_dtype<float>(P, greedy, vec, st);
  else if (dtype == kBF16) rc = launch_dtype<bf16_t>(P, greedy, vec, st);
  else rc = launch_dtype<f16_t>(P, greedy, vec, st);
  if (rc != LSG_OK) return rc;
  return check_launch("lsg_sample");
}
