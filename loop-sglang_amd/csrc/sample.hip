// Token sampling over the vocabulary: greedy argmax, temperature softmax,
// top-k, top-p and one inverse-CDF draw per row with an explicit uniform.
//
// Replaces, for the decode token path of Loop-SGLang:
//   Sampler.sample            python/loopsgl/model_executor/sample.py:107-112
//   torch.argmax (greedy)     sample.py:110-111 (+ int32 cast, model_runner.py:279-280)
//   sample_impl -> flashinfer softmax / *_sampling_from_probs   sample.py:60-81
//
// One workgroup samples one row.  The row is read from HBM once with coalesced
// 128-bit loads (each wave instruction reads 1 KiB of contiguous logits) and
// held in registers for the two full passes (row maximum, softmax normaliser).
// The later steps (top-k / top-p threshold, inverse-CDF walk) touch only the
// few chunks whose maximum can matter and re-read those.  Rows of up to 65536
// bf16/f16 (32768 fp32) elements use 1024-thread workgroups of at most 64
// VGPRs, two resident per CU: one streams its row from HBM while the other
// computes.
//
// Semantics (per row r, x = float32(logit), NaN treated as -inf):
//   T <= 0 or non-finite, or max x non-finite  -> id = argmax (torch rules)
//   m = max x,  e_i = 2^((x_i - m) * log2(e)/T)          (= exp((x_i - m)/T))
//   K = {x >= k-th largest x} if 1 <= k < V            (ties kept)
//   P = {x in K : x >= tau}, tau = largest x with mass(x >= tau) >= p * mass(K)
//   id = first index j in P (ascending) with cumsum_P(e)[j] > u * sum_P(e)
// Sums above the 16-byte chunk level are accumulated in float64 in a fixed
// order, so the result is deterministic and agrees with a float64 evaluation to
// ~1e-7 relative.
#include "lsg_capi_internal.h"
#include "lsg_common.h"
#include "lsg_sample.h"

#include <algorithm>
#include <type_traits>

namespace lsg {

constexpr float kLog2e = 1.4426950408889634f;
// Row shapes (the FULL template argument): rows of any length, streaming the
// chunks past the register capacity; rows of at most NT*CAP chunks; rows of
// exactly NT*CAP full chunks.
constexpr int kStream = 0, kBounded = 2, kFull = 1;
constexpr int kBins = 64;  // histogram of y = log2(e / e_max): bins of width 1/2
constexpr int kRefBins = 256;             // exact refinement: bins per level
constexpr double kFix = 1099511627776.0;  // exact refinement: mass fixed point, 2^40
constexpr float kYMin = -32.0f;  // y covered by the histogram: [kYMin, 0]
// Scale of the per-wave mass histogram's 32-bit words.  A bin b collects at most
// 128 chunk maxima of mass <= 2^(-b/2) (<= 1 relative to the wave maximum) and
// 64 chunk remainders (EPV - 1) 2^ye with ye <= -1 in bins >= 2 (<= 3.5 each):
// at most 288, below 2^32 / 2^23 = 512.
constexpr float kWaveMassFix = 0x1p23f;
// Margin on the top-p histogram test: the bin is chosen where the float sum of
// the binned maxima reaches p*Z*(1 + 2^-10), so the window (a superset of those
// maxima, summed in double) always reaches p*Z despite the rounding of the
// float sums (at most 2048 terms: < 2^-13 relative) and of the per-wave
// reference shifts (< 2^-17 relative per term).
constexpr double kBinMargin = 1.0 + 1.0 / 1024.0;

// Phase stamps, compiled in only by the profiling build (-DLSG_PHASE_STAMPS):
// thread 0 of workgroup b writes the 100 MHz real-time counter at fixed points
// of its row to g_row_stamps[b * kRowStampSlots + slot] (slots: 0 kernel entry, 1 both
// passes done (barrier 1), 2 candidate window staged, 3 dense path: histogram
// done, 4 dense path: crossing bracketed, 5 dense path: bracket gathered,
// 7 threshold known on any path, 8 id written, by the lane writing it, 9 dense
// path: kept masses, 10 inverse-CDF barrier passed); slot 6
// holds the hardware id (bits 0-31),
// the XCC id (32-39) and the row's path (40-47: 1 unfiltered walk, 2 window of
// at most 128, 3 ranked window, 4 dense top-p, 5 exact refinement, 6 argmax).
constexpr int kRowStampSlots = 16, kRowStampRows = 8192;
enum RowPath { kRowWalk = 1, kRowSmall = 2, kRowRanked = 3, kRowDense = 4, kRowRefine = 5, kRowArgmax = 6 };
#ifdef LSG_PHASE_STAMPS
__device__ unsigned long long g_row_stamps[kRowStampRows * kRowStampSlots];
__device__ __forceinline__ void row_stamp_val(int slot, unsigned long long v) {
  if (threadIdx.x == 0 && blockIdx.x < (unsigned)kRowStampRows) g_row_stamps[blockIdx.x * kRowStampSlots + slot] = v;
}
__device__ __forceinline__ void row_stamp(int slot) { row_stamp_val(slot, __builtin_amdgcn_s_memrealtime()); }
__device__ __forceinline__ void row_stamp_end() {
  if (blockIdx.x < (unsigned)kRowStampRows)
    g_row_stamps[blockIdx.x * kRowStampSlots + 8] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void row_stamp_path(int path) {
  // HW_ID (hwreg 4: wave, SIMD, CU, SH, SE) and XCC_ID (hwreg 20)
  const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
  const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xffu;
  row_stamp_val(6, ((unsigned long long)path << 40) | ((unsigned long long)xcc << 32) | hw);
}
#else
__device__ __forceinline__ void row_stamp(int) {}
__device__ __forceinline__ void row_stamp_end() {}
__device__ __forceinline__ void row_stamp_path(int) {}
#endif

// exp2 clamped to [0, 1]; the clamp folds into v_exp_f32 and maps NaN (from a
// NaN logit) to 0.
__device__ __forceinline__ float ex2c(float y) {
  return __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(y), 0.0f, 1.0f);
}

// Smallest float >= a*b.
__device__ __forceinline__ float mul_up(float a, float b) {
  const float p = __fmul_rn(a, b);
  const float r = __builtin_fmaf(a, b, -p);  // a*b - p exactly (finite p)
  if (!(r > 0.0f)) return p;
  const uint32_t u = __float_as_uint(p);
  if (p > 0.0f) return __uint_as_float(u + 1u);
  if (p < 0.0f) return __uint_as_float(u - 1u);
  return __uint_as_float(1u);
}

// floor(e * 2^40) for a mass e in [0, 1], from its bits: the 24-bit
// significand shifted by the exponent (no double-precision conversion; zero
// and denormal masses, below 2^-126, give 0).
__device__ __forceinline__ unsigned long long fix40(float e) {
  const uint32_t b = __float_as_uint(e);
  const int E = (int)(b >> 23) - 110;  // e = m * 2^(E - 40), m the significand
  const unsigned long long m = (unsigned long long)((b & 0x7fffffu) | 0x800000u);
  if (b < 0x00800000u || E <= -24) return 0ull;
  return E >= 0 ? (m << E) : (m >> -E);
}

// Exponent map of one row: e(x) = 2^y(x), y(x) = (x - m) * c with c = log2(e)/T.
// When |m*c| < 2^22, y is one fma against b = m*c rounded up: every exponent is
// then <= 0 and all of them carry the same offset m*c - b in [-1/2, 0], which
// cancels in every ratio.  Otherwise y = (x - m) * c.  Both forms are
// fma(x - sa, c, sb): sa = 0, sb = -b for the first (x - 0 is x), sa = m,
// sb = 0 for the second (the product rounded once; only a -0 product turns
// into +0, which every use of y treats alike).
struct Ex {
  float c, nb, gm, sa, sb;
  bool fma;
  __device__ __forceinline__ void init(float gm_, float c_) {
    gm = gm_;
    c = c_;
    const float b = mul_up(gm, c);
    fma = __builtin_fabsf(b) < 4194304.0f;
    nb = -b;
    sa = fma ? 0.0f : gm;
    sb = fma ? nb : 0.0f;
  }
  // Same for wave-uniform arguments; the fields are kept in scalar registers.
  __device__ __forceinline__ void init_u(float gm_, float c_) {
    gm = uni(gm_);
    c = uni(c_);
    const float b = uni(mul_up(gm, c));
    fma = __builtin_fabsf(b) < 4194304.0f;
    nb = -b;
    sa = uni(fma ? 0.0f : gm);
    sb = uni(fma ? nb : 0.0f);
  }
  // two instructions per element whatever the form (no select between forms)
  __device__ __forceinline__ float y(float x) const { return __builtin_fmaf(x - sa, c, sb); }
  // y(x) for a known form (FMA == fma): one instruction per element instead
  // of both forms and a select
  template <bool FMA>
  __device__ __forceinline__ float yf(float x) const {
    return FMA ? __builtin_fmaf(x, c, nb) : (x - gm) * c;
  }
  __device__ __forceinline__ float e(float x) const { return ex2c(y(x)); }
};

// 2^(shift(a) - shift(b)): converts masses relative to a's maximum into masses
// relative to b's (a.gm <= b.gm, same c).  The shift of the fma form is the
// float -nb, that of the other form gm * c.
__device__ __forceinline__ float shift_diff(const Ex& a, const Ex& b) {
  if (a.fma && b.fma) return b.nb - a.nb;
  if (a.fma) return __builtin_fmaf(-b.gm, b.c, -a.nb);
  if (b.fma) return __builtin_fmaf(a.gm, a.c, b.nb);
  return (a.gm - b.gm) * a.c;
}
__device__ __forceinline__ float shift_ratio(const Ex& a, const Ex& b) { return ex2c(shift_diff(a, b)); }

// Smallest float x with X.y(x) >= ly (X.y is monotone non-decreasing in x), so
// that "X.y(x) >= ly" becomes one compare.  Starts from the algebraic inverse
// and steps one float at a time (order keys) until the test flips.  ly and X
// are wave-uniform.
__device__ __forceinline__ float x_at_least(const Ex& X, float ly) {
  float x = X.fma ? (ly - X.nb) / X.c : ly / X.c + X.gm;
  x = uni(x);
  if (X.y(x) >= ly) {
    for (int i = 0; i < 64; ++i) {
      const float xd = okey_inv(okey(x) - 1u);
      if (!(X.y(xd) >= ly)) break;
      x = xd;
    }
  } else {
    for (int i = 0; i < 64 && !(X.y(x) >= ly); ++i) x = okey_inv(okey(x) + 1u);
  }
  return uni(x);
}

template <int EPV>
__device__ __forceinline__ float tree_sum(float (&e)[EPV]) {
#pragma unroll
  for (int w = 1; w < EPV; w <<= 1)
#pragma unroll
    for (int i = 0; i < EPV; i += 2 * w) e[i] += e[i + w];
  return e[0];
}

// Mass of one chunk (pairwise tree in fp32); FMA selects the exponent form.
template <typename T, bool FMA>
__device__ __forceinline__ float esum_chunk(const uint4& v, const Ex& X) {
  constexpr int EPV = Elem<T>::EPV;
  float e[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const float x = Elem<T>::get_alt(v, i);
    e[i] = ex2c(FMA ? __builtin_fmaf(x, X.c, X.nb) : (x - X.gm) * X.c);
  }
  return tree_sum<EPV>(e);
}
template <typename T>
__device__ __forceinline__ float esum_chunk(const uint4& v, const Ex& X) {
  return X.fma ? esum_chunk<T, true>(v, X) : esum_chunk<T, false>(v, X);
}

// Same, counting only elements with x >= thr.
template <typename T>
__device__ __forceinline__ float esum_chunk_ge(const uint4& v, const Ex& X, float thr) {
  constexpr int EPV = Elem<T>::EPV;
  float e[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const float x = Elem<T>::get(v, i);
    e[i] = x >= thr ? X.e(x) : 0.0f;
  }
  return tree_sum<EPV>(e);
}

template <typename T>
__device__ __forceinline__ int count_chunk_ge(const uint4& v, float thr) {
  int n = 0;
#pragma unroll
  for (int i = 0; i < Elem<T>::EPV; ++i) n += Elem<T>::get(v, i) >= thr ? 1 : 0;
  return n;
}

// Significant low bit of the order-preserving key of a T value (its float
// image has that many trailing zero bits, or ones for negative values).
template <typename T>
struct KeyShift {
  static constexpr int value = 0;
};
template <>
struct KeyShift<bf16_t> {
  static constexpr int value = 16;
};
template <>
struct KeyShift<f16_t> {
  static constexpr int value = 13;
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
    if constexpr (std::is_same<T, bf16_t>::value) {
      bits = __float_as_uint(m) >> 16;
    } else {
      // The compiler evaluates the f16 maximum with v_max3_f16 and assumes it
      // clears the upper half of the destination register; on gfx950 the VOP3
      // form keeps it.  Make the value opaque so the mask below is kept.
      bits = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)m);
      asm volatile("" : "+v"(bits));
      bits &= 0xffffu;
    }
    if (j & 1) w[j >> 1] = (w[j >> 1] & 0x0000ffffu) | (bits << 16);
    else w[j >> 1] = (w[j >> 1] & 0xffff0000u) | bits;
  }
  __device__ __forceinline__ void launder() {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(w[i]));
  }
  __device__ __forceinline__ void store(uint32_t* p) const {
#pragma unroll
    for (int i = 0; i < N; ++i) p[i] = w[i];
  }
  __device__ __forceinline__ void load(const uint32_t* p) {
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = p[i];
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
  __device__ __forceinline__ void store(uint32_t* p) const {
#pragma unroll
    for (int i = 0; i < CAP; ++i) p[i] = __float_as_uint(m[i]);
  }
  __device__ __forceinline__ void load(const uint32_t* p) {
#pragma unroll
    for (int i = 0; i < CAP; ++i) m[i] = __uint_as_float(p[i]);
  }
};

// Tell the compiler a register chunk may have changed, so values derived from it
// (unpacked floats) are recomputed per pass instead of being hoisted and kept
// live across passes (which would double the register footprint).
__device__ __forceinline__ void launder(uint4& v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// Chunk j of CAP register chunks with a runtime index, built with masked ORs:
// a select chain would be folded back into a dynamic index, which moves the
// array to scratch memory.
template <int CAP>
__device__ __forceinline__ uint4 select_chunk(const uint4 (&d)[CAP], int j) {
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

// LDS shared by the per-row routines.
template <int NT>
struct Smem {
  static constexpr int NW = NT / kWave;
  static constexpr int kWin = NT < 512 ? NT : 512;  // candidate window capacity
  double red[NW];
  double wtot[NW];  // per-wave masses
  float wmax[NW];   // per-wave maxima
  int hcnt[kBins];
  float hmass[kBins];
  uint32_t wh[NW][kBins];  // per-wave histograms (count, or mass in kWaveMassFix fixed point)
  uint32_t kmin;           // smallest order key in the candidate window
  unsigned long long rbins[4][kRefBins + 1];  // exact refinement: bin copies by lane, one bin apart in bank order
  int rk_cnt[2 * kWave];    // small window: entries at or above each entry
  unsigned long long rk_fix[2 * kWave];  // and their mass, 2^-40 fixed point
  static constexpr int kSeg = kWave;     // candidates staged per wave
  union {
    uint64_t stage[NW * kSeg];  // per-wave candidate segments, in index order
    struct {
      uint64_t wkey[kWin];    // candidate window (unsorted)
      uint64_t sorted[kWin];  // candidate window in descending key order
    };
  };
  int wcnt[NW];            // candidates per wave
  double rZ;               // row normaliser, histogram bin and candidate floor,
  int rbin;                // derived by wave 0 for the whole workgroup
  float rxlo;
  int wn;
  int pick;
};

// ---------------------------------------------------------------------------
// A row in registers.  Wave-blocked layout: wave w owns chunks
// [w*L*64, (w+1)*L*64) (L = chunks per thread); its j-th load reads the 64
// consecutive chunks (w*L + j)*64 + lane (1 KiB of contiguous HBM), so the
// index order is (wave, j, lane, element).  Chunks j < CAP stay in registers;
// their maxima go to LDS.  Chunks j >= CAP (very long rows) are re-read on
// every pass.  FULL (kFull = 1): the row is exactly NT*CAP full chunks (every thread holds
// CAP chunks, no partial or padding chunk), so loads need no bounds checks.
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC, int FULL>
struct Row {
  static constexpr int EPV = Elem<T>::EPV;
  using CM = ChunkMax<T, CAP>;
  static constexpr int kCmWords = sizeof(CM) / 4;
  const char* base;
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t V;
  int L;
  uint32_t c0;  // chunk index of this thread's j = 0 load
  uint4 d[CAP];
  uint32_t* cmx;  // this thread's chunk maxima in LDS (kCmWords words)

  __device__ __forceinline__ void init(const void* logits, int64_t r, int64_t ld, int64_t Vv, uint32_t* cm_lds) {
    cmx = cm_lds + threadIdx.x * kCmWords;
    base = reinterpret_cast<const char*>(logits) + r * ld * (int64_t)Elem<T>::kSize;
    // Buffer resource over the row: full chunks load with one 32-bit lane
    // offset plus a scalar offset per j (one address register for every load).
    rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)0xffffffff, 0x00020000);
    V = (uint32_t)uni((uint32_t)Vv);
    const uint32_t NV = (V + EPV - 1) / EPV;
    L = FULL == kFull ? CAP : (int)((NV + NT - 1) / NT);
    c0 = (uint32_t)(threadIdx.x >> 6) * (uint32_t)L * kWave + (threadIdx.x & 63);
  }
  __device__ __forceinline__ bool has(int j) const { return FULL == kFull ? j < CAP : j < L; }
  // chunks of this thread (kBounded: at most CAP, so no chunk is streamed)
  __device__ __forceinline__ int nstream() const {
    return FULL == kFull ? CAP : FULL == kBounded ? min(L, CAP) : L;
  }
  __device__ __forceinline__ uint32_t chunk_index(int j) const { return c0 + (uint32_t)j * kWave; }
  __device__ __forceinline__ uint4 load(int j) const {
    if (FULL == kFull || (VEC && (chunk_index(j) + 1u) * EPV <= V)) {
      typedef uint32_t v4u __attribute__((ext_vector_type(4)));
      const v4u v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(c0 * 16u), j * kWave * 16, 0);
      return make_uint4(v.x, v.y, v.z, v.w);
    }
    return load_chunk32<T, VEC>(base, chunk_index(j), V);
  }
  __device__ __forceinline__ uint32_t elem_index(int j, int i) const {
    return chunk_index(j) * EPV + (uint32_t)i;
  }
  __device__ __forceinline__ void fetch() {
#pragma unroll
    for (int j = 0; j < CAP; ++j) d[j] = has(j) ? load(j) : Elem<T>::pad();
  }
  // Pass A: chunk maxima (NANPROP: NaN-propagating, else NaN ignored) to LDS;
  // returns this thread's maximum.
  template <bool NANPROP>
  __device__ __forceinline__ float maxima() {
    float tm = -INFINITY;
    CM cm;
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      cm.set(j, -INFINITY);
      if (has(j)) {
        const float m = NANPROP ? chunk_maximum<T>(d[j]) : chunk_max<T>(d[j]);
        cm.set(j, m);
        tm = NANPROP ? fmaximum(tm, m) : fmaxf(tm, m);
      }
    }
    cm.store(cmx);
    for (int j = CAP; j < nstream(); ++j) {
      const uint4 v = load(j);
      tm = NANPROP ? fmaximum(tm, chunk_maximum<T>(v)) : fmaxf(tm, chunk_max<T>(v));
    }
    return tm;
  }
  // Maximum of register chunk j, from LDS.
  __device__ __forceinline__ float cm_at(int j) const {
    if constexpr (sizeof(T) == 2) {
      uint4 v;
      v.x = cmx[j >> 1] >> ((j & 1) * 16);
      return Elem<T>::get(v, 0);
    } else {
      return __uint_as_float(cmx[j]);
    }
  }
  // The passes below run once per row on few chunks: compact loops (small code
  // keeps them in the instruction cache), chunks picked with a runtime index.
  __device__ __forceinline__ uint4 chunk(int j) const { return j < CAP ? select_chunk<CAP>(d, j) : load(j); }
  // f(j, chunk_max) over every chunk (register chunks: the stored maxima).
  template <class F>
  __device__ __forceinline__ void each_cm(F&& f) {
#pragma unroll 1
    for (int j = 0; j < nstream(); ++j) f(j, j < CAP ? cm_at(j) : chunk_max<T>(load(j)));
  }
  // f(j, chunk, chunk_max) over the chunks whose maximum passes keep().
  template <class K, class F>
  __device__ __forceinline__ void each_kept(K&& keep, F&& f) {
#pragma unroll 1
    for (int j = 0; j < nstream(); ++j) {
      if (j < CAP) {
        const float m = cm_at(j);
        if (keep(m)) f(j, select_chunk<CAP>(d, j), m);
      } else {
        const uint4 v = load(j);
        const float m = chunk_max<T>(v);
        if (keep(m)) f(j, v, m);
      }
    }
  }
  // Same, re-reading the chunks from memory (rare paths: the registers are
  // then free for the path's own state).
  template <class K, class F>
  __device__ __forceinline__ void each_kept_mem(K&& keep, F&& f) {
#pragma unroll 1
    for (int j = 0; j < nstream(); ++j) {
      if (j < CAP) {
        const float m = cm_at(j);
        if (keep(m)) f(j, load(j), m);
      } else {
        const uint4 v = load(j);
        const float m = chunk_max<T>(v);
        if (keep(m)) f(j, v, m);
      }
    }
  }
};

// ---------------------------------------------------------------------------
// argmax with torch semantics over a row whose chunk maxima ignore NaN.  gm is
// the NaN-ignoring maximum, tm this thread's.  Returns the id (identical in
// every thread).
// ---------------------------------------------------------------------------
template <int NW, typename T, class R_>
__device__ __forceinline__ int32_t row_argmax(R_& R, float tm, float gm, double* red) {
  constexpr int EPV = Elem<T>::EPV;
  int nan = 0;
  R.each_kept_mem([](float) { return true; }, [&](int, const uint4& v, float) {
#pragma unroll
    for (int i = 0; i < EPV; ++i) nan |= __builtin_isnan(Elem<T>::get(v, i)) ? 1 : 0;
  });
  const int gnan = wg_max_i<NW>(nan, red);
  int first = 0x7fffffff;
  if (gnan ? nan : (tm == gm)) {
    R.each_kept_mem([](float) { return true; }, [&](int j, const uint4& v, float) {
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

// Exact threshold search by bisection over order-preserving keys (16 steps for
// bf16, 19 for f16, 32 for fp32).  Returns thr: keep-mask x >= thr (top-k,
// then top-p within it).  Chunks whose maximum is below the probe are skipped.
template <int NW, typename T, class R_>
__device__ __forceinline__ float select_exact(R_& R, const Ex& X, double Z, bool kon, int32_t k, bool pon,
                                              float p, double* red) {
  constexpr int SH = KeyShift<T>::value;
  const uint32_t kmin = okey(-INFINITY) >> SH;
  auto th_of = [&](uint32_t kk) { return kk <= kmin ? -INFINITY : okey_inv(kk << SH); };
  const uint32_t khi = (okey(X.gm) >> SH) + 1u;
  float floor_thr = -INFINITY;
  if (kon) {
    uint32_t lo = kmin, hi = khi;
    while (hi - lo > 1u) {
      const uint32_t mid = lo + ((hi - lo) >> 1);
      const float th = th_of(mid);
      int n = 0;
      R.each_kept_mem([&](float m) { return m >= th; },
                      [&](int, const uint4& v, float) { n += count_chunk_ge<T>(v, th); });
      if (wg_sum_i<NW>(n, red) >= k) lo = mid;
      else hi = mid;
    }
    floor_thr = th_of(lo);
  }
  if (!pon) return floor_thr;
  double zk = Z;
  if (kon) {
    double acc = 0.0;
    R.each_kept_mem([&](float m) { return m >= floor_thr; },
                    [&](int, const uint4& v, float) { acc += (double)esum_chunk_ge<T>(v, X, floor_thr); });
    zk = wg_sum<NW>(acc, red);
  }
  const double target = (double)p * zk;
  uint32_t lo = floor_thr == -INFINITY ? kmin : (okey(floor_thr) >> SH), hi = khi;
  while (hi - lo > 1u) {
    const uint32_t mid = lo + ((hi - lo) >> 1);
    const float th = th_of(mid);
    double ms = 0.0;
    R.each_kept_mem([&](float m) { return m >= th; },
                    [&](int, const uint4& v, float) { ms += (double)esum_chunk_ge<T>(v, X, th); });
    if (wg_sum<NW>(ms, red) >= target) lo = mid;
    else hi = mid;
  }
  return th_of(lo);
}

// Histogram scan: the first bin b (from the top) at which the cumulative count
// reaches k (top-k) or the cumulative mass reaches p*Z (top-p); -1 if none.
template <int NT>
__device__ __forceinline__ int window_bin(Smem<NT>& S, bool kon, int32_t k, float p, double Z) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  __syncthreads();
  if (wid == 0) {
    const int pc = wave_incl_scan_i(S.hcnt[lane], lane);
    const double pm = wave_incl_scan((double)S.hmass[lane], lane);
    const bool ok = kon ? (pc >= k) : (pm >= (double)p * Z * kBinMargin);
    const uint64_t bal = __ballot(ok);
    if (lane == 0) S.pick = bal ? (__ffsll((unsigned long long)bal) - 1) : -1;
  }
  __syncthreads();
  const int bin = uni(S.pick);
  __syncthreads();
  return bin;
}

__device__ __forceinline__ int ybin(float y) { return min(kBins - 1, (int)(-2.0f * y)); }
// Lower edge of bin b.
__device__ __forceinline__ float bin_floor(int b) { return -0.5f * (float)(b + 1); }

// Threshold from a collected window of nw <= kWin candidates (S.wkey: order key
// of the value in the high word, ~index in the low word).  Returns false when
// the window does not reach the top-p mass (the exact search then decides).
template <int NT>
__device__ __forceinline__ bool window_threshold(Smem<NT>& S, int nw, bool kon, int32_t k, bool pon, float p, double Z,
                                 const Ex& X, float* thr_out) {
  constexpr int NW = NT / kWave;
  const int t = threadIdx.x, wid = t >> 6;
  float thr = -INFINITY;
  bool ok = true;
  if (nw <= kWave) {
    // Small window: wave 0 ranks, scans and thresholds it alone.
    if (wid == 0) {
      const int lane = t;
      const uint64_t mine = lane < nw ? S.wkey[lane] : 0ull;
      int rank = 0;
      for (int q = 0; q < nw; ++q) {
        const uint64_t other =
            ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(mine >> 32), q) << 32) |
            (uint32_t)__builtin_amdgcn_readlane((int)(mine & 0xffffffffu), q);
        rank += other > mine ? 1 : 0;
      }
      if (lane < nw) S.sorted[rank] = mine;
      __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS writes are done
      const uint64_t key = lane < nw ? S.sorted[lane] : 0ull;
      const uint32_t kx = (uint32_t)(key >> 32);
      const float e = lane < nw ? X.e(okey_inv(kx)) : 0.0f;
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
          th = okey_inv(
              (uint32_t)__builtin_amdgcn_readlane((int)kx, __ffsll((unsigned long long)hit) - 1));
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
  } else {
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
    const float e = t < nw ? X.e(okey_inv(kx)) : 0.0f;
    double pre, tot;
    wg_scan<NW>((double)e, S.red, &pre, &tot);  // pre = inclusive prefix in sorted order
    double ZK = Z;
    int limit = nw;
    if (kon) {
      // k-th largest value (the window holds at least k elements)
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
        ok = false;
      } else {
        if (t == q) S.pick = (int)kx;
        __syncthreads();
        thr = uni(okey_inv((uint32_t)S.pick));
      }
    }
    __syncthreads();
  }
  *thr_out = thr;
  return ok;
}

// Top-k / top-p threshold from a candidate window.  The window {y >= lo} is
// bounded with a histogram of distinct elements (the thread maxima, else the
// chunk maxima): once >= k of them have y >= lo, the window holds >= k
// elements, and once those carry mass >= p*Z, it holds the top-p set.  Returns
// false when no small window exists (the exact search then decides).
template <int NT, typename T, class R_>
__device__ __forceinline__ bool find_threshold(R_& R, float tm, const Ex& X, double Z, bool kon, int32_t k,
                                               bool pon, float p, Smem<NT>& S, float* thr) {
  constexpr int EPV = Elem<T>::EPV, kWin = Smem<NT>::kWin;
  const int t = threadIdx.x;
  if (t < kBins) {
    S.hcnt[t] = 0;
    S.hmass[t] = 0.0f;
  }
  if (t == 0) S.wn = 0;
  __syncthreads();
  {
    const float y = X.y(tm);
    if (y >= kYMin) {
      atomicAdd(&S.hcnt[ybin(y)], 1);
      atomicAdd(&S.hmass[ybin(y)], ex2c(y));
    }
  }
  int bin = window_bin(S, kon, k, p, Z);
  if (bin < 0) {
    if (t < kBins) {
      S.hcnt[t] = 0;
      S.hmass[t] = 0.0f;
    }
    __syncthreads();
    R.each_cm([&](int, float cmj) {
      const float y = X.y(cmj);
      if (y >= kYMin) {
        atomicAdd(&S.hcnt[ybin(y)], 1);
        atomicAdd(&S.hmass[ybin(y)], ex2c(y));
      }
    });
    bin = window_bin(S, kon, k, p, Z);
    if (bin < 0) return false;
  }
  const float lo_y = bin_floor(bin);
  R.each_kept([&](float m) { return X.y(m) >= lo_y; },
              [&](int j, const uint4& v, float) {
#pragma unroll
                for (int i = 0; i < EPV; ++i) {
                  const float x = Elem<T>::get(v, i);
                  if (X.y(x) >= lo_y) {
                    const int pos = atomicAdd(&S.wn, 1);
                    if (pos < kWin)
                      S.wkey[pos] = ((uint64_t)okey(x) << 32) | (uint64_t)(0xffffffffu - R.elem_index(j, i));
                  }
                }
              });
  __syncthreads();
  const int nw = uni(S.wn);
  if (nw > kWin) return false;
  return window_threshold<NT>(S, nw, kon, k, pon, p, Z, X, thr);
}

// ---------------------------------------------------------------------------
// Per-row arguments (uniform loads through the scalar cache).
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

// The same arguments as plain loads, made wave-uniform by uniform() where the
// row is processed.  They are vector loads: converting right after them waits
// for them, so the kernel issues them, then the row's chunks, then converts
// (the in-order counter then waits for the arguments only).
__device__ __forceinline__ RowArgs row_args_load(const SampleParams& P, int64_t r) {
  RowArgs a;
  a.T = P.temps ? P.temps[r] : 0.0f;
  a.u = P.uniforms ? P.uniforms[r] : 0.0f;
  a.k = P.top_k ? P.top_k[r] : 0;
  a.p = P.top_p ? P.top_p[r] : 1.0f;
  return a;
}
__device__ __forceinline__ RowArgs uniform(const RowArgs& a) { return RowArgs{uni(a.T), uni(a.p), uni(a.u), uni(a.k)}; }

// Output row b -> source row r: >= 0 valid, -1 past the end, -2 invalid gather index.
__device__ __forceinline__ int64_t source_row(const SampleParams& P, int64_t b, int64_t nrows) {
  if (b >= nrows) return -1;
  const int64_t r = P.row_idx ? (int64_t)uni((int)P.row_idx[b]) : b;
  return (r < 0 || r >= P.B_src) ? -2 : r;
}

// ---------------------------------------------------------------------------
// Greedy row: torch.argmax.  NaN-propagating maxima make a NaN anywhere the
// row maximum, so one pass finds both the maximum and whether NaN is present;
// the chunk maxima then point at the chunk holding the first hit.
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC, int FULL>
__device__ __forceinline__ void row_greedy(Row<T, NT, CAP, VEC, FULL>& R, int32_t* out, Smem<NT>& S) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  const float tm = R.template maxima<true>();
  const float gm = wg_maximum<NW>(tm, S.red);
  const bool isn = gm != gm;
  int first = 0x7fffffff;
  if (isn ? (tm != tm) : (tm == gm)) {
    // first chunk whose (NaN-propagating) maximum is the hit, then its first element
#pragma unroll 1
    for (int j = 0; j < R.nstream() && first == 0x7fffffff; ++j) {
      const uint4 v = R.chunk(j);
      const float cmj = j < CAP ? R.cm_at(j) : chunk_maximum<T>(v);
      if (isn ? cmj != cmj : cmj == gm) {
#pragma unroll 1
        for (int i = 0; i < EPV; ++i) {
          const float x = Elem<T>::get(v, i);
          const uint32_t idx = R.elem_index(j, i);
          if (first == 0x7fffffff && (isn ? x != x : x == gm) && idx < R.V) first = (int)idx;
        }
      }
    }
  }
  const int32_t id = wg_min_i<NW>(first, S.red);
  if (threadIdx.x == 0) *out = id;
}

// ---------------------------------------------------------------------------
// Inverse CDF inside the crossing wave of a wave-blocked row: the column j,
// then the lane, then the element whose prefix crosses U.  base is the mass of
// the waves before this one (row reference), fw converts this wave's masses
// into the row's reference (wave-uniform).  cs[j * NT] is this thread's mass of
// register chunk j; chunk_mass(j) recomputes that of a chunk j >= CAP and
// elem_mass(x) that of one element, with the arithmetic that produced cs.  REG:
// the chosen chunk is taken from registers, else re-read.  The owner lane
// writes the id.
// ---------------------------------------------------------------------------
template <bool REG, typename T, int NT, int CAP, bool VEC, int FULL, class CMass, class EMass>
__device__ __forceinline__ void wave_walk(Row<T, NT, CAP, VEC, FULL>& R, const float* cs, double fw, double base,
                                          double U, CMass&& chunk_mass, EMass&& elem_mass, int32_t* out) {
  constexpr int EPV = Elem<T>::EPV;
  const int lane = threadIdx.x & 63;
  int jstar = -1, jlast = 0;
  double jbase = base, cum = base, cum_last = base;
  float sme = 0.0f, slast = 0.0f;
  auto column = [&](int j, double col, float sj) {
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
  };
  {
    // the register columns' masses first (independent reductions), then the scan
    float sv[CAP];
    double colv[CAP];
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      sv[j] = R.has(j) ? cs[j * NT] : 0.0f;
      colv[j] = uni(wave_sum((double)sv[j]) * fw);  // wave-uniform: scalar registers
    }
#pragma unroll
    for (int j = 0; j < CAP; ++j)
      if (R.has(j)) column(j, colv[j], sv[j]);
  }
  for (int j = CAP; j < R.nstream(); ++j) {
    const float sj = chunk_mass(j);
    column(j, wave_sum((double)sj) * fw, sj);
  }
  if (jstar < 0) {
    jstar = jlast;
    jbase = cum_last;
    sme = slast;
  }
  jstar = uni(jstar);
  const double incl = wave_incl_scan((double)sme, lane) * fw;
  const double excl = wave_shr1(incl);
  int owner;
  {
    const uint64_t bal = __ballot(sme > 0.0f && jbase + incl > U);
    if (bal) {
      owner = __ffsll((unsigned long long)bal) - 1;
    } else {
      const uint64_t pos = __ballot(sme > 0.0f);
      owner = pos ? 63 - __clzll((long long)pos) : 0;
    }
  }
  if (lane != owner) return;
  const uint4 v = REG ? R.chunk(jstar) : R.load(jstar);
  float ev[EPV];
#pragma unroll
  for (int i = 0; i < EPV; ++i) ev[i] = elem_mass(Elem<T>::get(v, i));
  double a = jbase + excl;
  int pick = -1, lastpos = -1;
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    const double e = (double)ev[i] * fw;
    if (e > 0.0) {
      lastpos = i;
      a += e;
      if (pick < 0 && a > U) pick = i;
    }
  }
  if (pick < 0) pick = lastpos < 0 ? 0 : lastpos;
  *out = (int32_t)R.elem_index(jstar, pick);
  row_stamp_end();
}

// The crossing wave of U = u * (sum of the wave masses sw, one per lane < NW):
// sets wstar and base (mass of the waves before it); returns U.
template <int NW>
__device__ __forceinline__ double cross_wave(double sw, float u, int* wstar, double* base) {
  const int lane = threadIdx.x & 63;
  const double inc = wave_incl_scan(sw, lane);
  const double total = readlane_d(inc, NW - 1);
  asm volatile("" : "+s"(u));  // convert here: a hoisted double copy would be spilled
  const double U = (double)u * total;
  int w;
  const uint64_t cross = __ballot(lane < NW && inc > U);
  if (cross) {
    w = __ffsll((unsigned long long)cross) - 1;
  } else {  // u >= 1 or rounding: the last wave with mass
    const uint64_t pos = __ballot(lane < NW && sw > 0.0);
    w = pos ? 63 - __clzll((long long)pos) : 0;
  }
  w = uni(w);
  *wstar = w;
  *base = readlane_d(wave_shr1(inc), w);
  return U;
}

// Full inverse-CDF walk with the masses in the row's reference: wave totals
// through LDS (one barrier), crossing wave, then wave_walk.
template <bool REG, typename T, int NT, int CAP, bool VEC, int FULL, class CMass, class EMass>
__device__ __forceinline__ void cdf_walk(Row<T, NT, CAP, VEC, FULL>& R, double tmass, const float* cs,
                                         CMass&& chunk_mass, EMass&& elem_mass, float u, Smem<NT>& S,
                                         int32_t* out) {
  constexpr int NW = NT / kWave;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const double ws = wave_sum(tmass);
  if (lane == 0) S.wtot[wid] = ws;
  __syncthreads();
  row_stamp(10);
  int wstar;
  double base;
  const double U = cross_wave<NW>(lane < NW ? S.wtot[lane] : 0.0, u, &wstar, &base);
  if (wid != wstar) return;
  wave_walk<REG>(R, cs, 1.0, base, U, chunk_mass, elem_mass, out);
}

// This thread's chunk masses (register chunks) -> cs[j * NT] in LDS and its
// total mass (chunks past CAP included).
template <bool FMA, typename T, int NT, int CAP, bool VEC, int FULL>
__device__ __forceinline__ double row_masses(Row<T, NT, CAP, VEC, FULL>& R, const Ex& X, float* cs,
                                             float* cmass_max = nullptr) {
  double tmass = 0.0;
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    uint4 v = R.d[j];
    if constexpr (!Elem<T>::kHasAlt) launder(v);  // no unpacked value is shared with the maxima pass
    const float sj = R.has(j) ? esum_chunk<T, FMA>(v, X) : 0.0f;
    cs[j * NT] = sj;
    tmass += (double)sj;
    mx = fmaxf(mx, sj);
  }
  if (cmass_max) *cmass_max = mx;  // largest register chunk mass
  for (int j = CAP; j < R.nstream(); ++j) tmass += (double)esum_chunk<T, FMA>(R.load(j), X);
  return tmass;
}

// Masked chunk masses (x >= thr, relative to X) -> cs and the total; chunks are
// re-read from memory.
template <typename T, int NT, int CAP, bool VEC, int FULL>
__device__ __forceinline__ double masked_masses(Row<T, NT, CAP, VEC, FULL>& R, const Ex& X, float thr, float* cs) {
  double tmass = 0.0;
#pragma unroll 1
  for (int j = 0; j < R.nstream(); ++j) {
    float sj = 0.0f;
    if (j < CAP) {
      if (R.has(j) && R.cm_at(j) >= thr) sj = esum_chunk_ge<T>(R.load(j), X, thr);
      cs[j * NT] = sj;
    } else {
      const uint4 v = R.load(j);
      if (chunk_max<T>(v) >= thr) sj = esum_chunk_ge<T>(v, X, thr);
    }
    tmass += (double)sj;
  }
  return tmass;
}

// ---------------------------------------------------------------------------
// Sampling row, general form (rows with chunks past CAP): workgroup maximum,
// masses relative to it, threshold, walk.
// ---------------------------------------------------------------------------
template <typename T, int NT, int CAP, bool VEC, int FULL>
__device__ __forceinline__ void row_sample(Row<T, NT, CAP, VEC, FULL>& R, const RowArgs& A, int32_t* out,
                                           Smem<NT>& S, float* csum) {
  constexpr int NW = NT / kWave;
  float* cs = csum + threadIdx.x;
  const float tm = R.template maxima<false>();
  const float gm = wg_max<NW>(tm, S.red);
  if (!(A.T > 0.0f) || !(A.T < INFINITY) || !(gm > -INFINITY) || !(gm < INFINITY)) {
    const int32_t id = row_argmax<NW, T>(R, tm, gm, S.red);
    if (threadIdx.x == 0) *out = id;
    return;
  }
  Ex X;
  X.init_u(gm, kLog2e / A.T);
  double tmass = X.fma ? row_masses<true>(R, X, cs) : row_masses<false>(R, X, cs);
  const bool kon = A.k >= 1 && (uint32_t)A.k < R.V, pon = A.p < 1.0f;
  if (!kon && !pon) {
    cdf_walk<true>(R, tmass, cs, [&](int j) { return esum_chunk<T>(R.load(j), X); },
                   [&](float x) { return X.e(x); }, A.u, S, out);
    return;
  }
  const double Z = wg_sum<NW>(tmass, S.red);
  float thr;
  if (!find_threshold<NT, T>(R, tm, X, Z, kon, A.k, pon, A.p, S, &thr))
    thr = select_exact<NW, T>(R, X, Z, kon, A.k, pon, A.p, S.red);
  tmass = masked_masses(R, X, thr, cs);
  cdf_walk<false>(R, tmass, cs,
                  [&](int j) {
                    const uint4 v = R.load(j);
                    return chunk_max<T>(v) >= thr ? esum_chunk_ge<T>(v, X, thr) : 0.0f;
                  },
                  [&](float x) { return x >= thr ? X.e(x) : 0.0f; }, A.u, S, out);
}

// ---------------------------------------------------------------------------
// Sampling row held entirely in registers (no chunk is streamed):
//   1. chunk maxima and the wave maximum; the chunk masses relative to the
//      wave maximum (no workgroup maximum needed yet) and the wave total;
//   2. one barrier; every wave derives the row maximum and converts the wave
//      totals into the row's reference.
// Without top-k / top-p the wave totals locate the crossing wave, which finds
// the column, lane and element from its chunk masses (scaled by one factor).
// With a filter, a candidate window bounded by a histogram of the thread
// maxima is collected; a window of at most 64 elements is thresholded by every
// wave (same result everywhere, so no broadcast barrier) and wave 0 walks the
// kept elements in index order.  Larger windows take the general path.
// ---------------------------------------------------------------------------
template <int NW>
__device__ __forceinline__ float lds_max(const float* v) {
  const int lane = threadIdx.x & 63;
  return wave_max(lane < NW ? v[lane] : -INFINITY);
}



// Threshold of a window of nw <= 128 candidates (order key of the value in the
// high word of each entry, ~index in the low word, so keys are unique), from
// each entry's rank: cnt = entries at or above it, pre = their mass.  Entry q
// sits in lane q & 63, slot q >> 6 of the calling wave.  Returns the top-k /
// top-p threshold as the order key of the value (keep key >= it), or false
// when the window does not reach the top-k count / top-p mass.
__device__ __forceinline__ bool window_pick(const bool (&in)[2], const uint32_t (&kx)[2], const float (&em)[2],
                                            const int (&cnt)[2], const double (&pre)[2], int nw, bool kon,
                                            int32_t k, bool pon, float p, double Z, uint32_t* tkey) {
  // key of the slot flagged in ballot b0 (slot 0) or else b1 (slot 1)
  auto pick = [&](uint64_t b0, uint64_t b1) -> uint32_t {
    return b0 ? (uint32_t)__builtin_amdgcn_readlane((int)kx[0], __ffsll((unsigned long long)b0) - 1)
              : (uint32_t)__builtin_amdgcn_readlane((int)kx[1], __ffsll((unsigned long long)b1) - 1);
  };
  uint32_t th = 0u;  // keep values with key >= th
  double ZK = Z;
  if (kon) {
    const int target = k <= nw ? k : nw;  // the k-th largest
    const uint64_t b0 = __ballot(in[0] && cnt[0] == target), b1 = __ballot(in[1] && cnt[1] == target);
    if (!b0 && !b1) return false;
    th = pick(b0, b1);
    ZK = wave_sum((in[0] && kx[0] >= th ? (double)em[0] : 0.0) + (in[1] && kx[1] >= th ? (double)em[1] : 0.0));
  }
  if (pon) {
    bool hit[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) hit[h] = in[h] && kx[h] >= th && pre[h] >= (double)p * ZK;
    const int r = wave_min_i(min(hit[0] ? cnt[0] : 0x7fffffff, hit[1] ? cnt[1] : 0x7fffffff));
    const uint64_t b0 = __ballot(hit[0] && cnt[0] == r), b1 = __ballot(hit[1] && cnt[1] == r);
    if (!b0 && !b1) return false;
    th = pick(b0, b1);
  }
  *tkey = th;
  return true;
}

// ---------------------------------------------------------------------------
// Exact top-k (count target k) or top-p (mass target p * ZK) threshold by radix
// refinement in order-key space (key = okey(x) >> SH).  Members are the non-NaN
// elements with key >= klo; the boundary lies among them.  Each level splits
// the bracket [lo, hi) of keys that holds the boundary into 256 bins of 2^sh
// keys and accumulates per bin the member count (top-k) or mass (top-p, fixed
// point with 40 fraction bits: exact, order-independent sums) with one LDS
// atomic per member, into four copies of the bins picked by lane (fewer lanes
// on one address).  A scan from the top with the totals above the bracket
// picks the bin holding the boundary; the next level splits that bin, down to
// a single key (the answer; ties are kept): two levels for bf16 keys, three
// for fp16, four for fp32.  Returns false when the members never reach the
// target.  All waves of the workgroup call it together.
// ---------------------------------------------------------------------------
template <int NT, typename T, class R_>
__device__ __forceinline__ bool refine_threshold(R_& R, const Ex& X, double ZK, bool kon, int32_t k, float p,
                                                 uint32_t klo, Smem<NT>& S, uint32_t* thr_key) {
  constexpr int SH = KeyShift<T>::value, EPV = Elem<T>::EPV;
  const int t = threadIdx.x, lane = t & 63;
  uint32_t lo = klo, hi = (okey(X.gm) >> SH) + 1u;  // keys in [lo, hi)
  double above = 0.0;  // count or fixed-point mass of the members above hi
  const double target = kon ? (double)k : (double)p * ZK * kFix;
  unsigned long long* bins = S.rbins[0];
  for (int level = 0; level < 8; ++level) {
    if (hi <= lo) return false;
    int sh = 0;
    while (((hi - lo - 1u) >> sh) >= (uint32_t)kRefBins) ++sh;
    for (int i = t; i < 4 * (kRefBins + 1); i += NT) bins[i] = 0ull;
    __syncthreads();
    const uint32_t lo_ = lo, hi_ = hi;
    const float xlo = okey_inv(lo << SH);  // smallest value with key lo (NaN for lo == 0)
    unsigned long long* mine = S.rbins[lane & 3];
    R.each_kept_mem([&](float m) { return lo_ == 0u || m >= xlo; },
                    [&](int, const uint4& v, float) {
#pragma unroll
                      for (int i = 0; i < EPV; ++i) {
                        const float x = Elem<T>::get(v, i);
                        const uint32_t key = okey(x) >> SH;
                        if (x == x && key >= lo_ && key < hi_) {
                          const int b = (int)((hi_ - 1u - key) >> sh);
                          const unsigned long long add =
                              kon ? 1ull : fix40(X.e(x));
                          atomicAdd(&mine[b], add);
                        }
                      }
                    });
    __syncthreads();
    // lane l holds bins 4l .. 4l+3 (summed over the four copies), every wave
    double bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int bi = 4 * lane + q;
      bv[q] = (double)(S.rbins[0][bi] + S.rbins[1][bi] + S.rbins[2][bi] + S.rbins[3][bi]);
    }
    const double ls = (bv[0] + bv[1]) + (bv[2] + bv[3]);
    const double incl = wave_incl_scan(ls, lane);
    const uint64_t bal = __ballot(above + incl >= target);
    if (!bal) return false;
    const int lb = __ffsll((unsigned long long)bal) - 1;
    double acc = above + readlane_d(incl - ls, lb);  // members above lane lb's bins
    int bs = 4 * lb + 3;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const double vq = readlane_d(bv[q], lb);
      if (acc + vq >= target) {
        bs = 4 * lb + q;
        break;
      }
      acc += vq;
    }
    above = acc;  // members above bin bs
    const uint32_t nhi = hi - ((uint32_t)bs << sh);
    const uint32_t nlo = nhi - lo > (1u << sh) ? nhi - (1u << sh) : lo;
    __syncthreads();  // every wave has read the bins
    lo = nlo;
    hi = nhi;
    if (hi - lo == 1u) {
      *thr_key = lo;
      return true;
    }
  }
  return false;
}

// Floor for the k-th largest element from the threads' maxima (k <= NT): the
// k largest thread maxima are distinct elements, so at least k elements are at
// or above the k-th largest.  One radix level over the thread maxima's order
// keys in [lo, hi) (256 bins, counts; one LDS atomic per thread) returns the
// floor key of the bin holding it, or lo when k > NT or fewer than k threads
// have a maximum in range.  Reads only the chunk maxima (LDS); all waves call
// it together.
template <int NT, typename T, class R_>
__device__ __forceinline__ uint32_t chunk_max_floor(R_& R, int32_t k, uint32_t lo, uint32_t hi, Smem<NT>& S) {
  constexpr int SH = KeyShift<T>::value;
  const int t = threadIdx.x, lane = t & 63;
  if (hi <= lo + 1u) return lo;
  int sh = 0;
  while (((hi - lo - 1u) >> sh) >= (uint32_t)kRefBins) ++sh;
  unsigned long long* bins = S.rbins[0];
  for (int i = t; i < 4 * (kRefBins + 1); i += NT) bins[i] = 0ull;
  __syncthreads();
  unsigned long long* mine = S.rbins[lane & 3];
  float tmax = -INFINITY;
  bool any = false;
  R.each_cm([&](int, float m) {
    if (m == m) {
      tmax = fmaxf(tmax, m);
      any = true;
    }
  });
  const uint32_t key = okey(tmax) >> SH;
  if (any && k <= NT && key >= lo && key < hi) atomicAdd(&mine[(hi - 1u - key) >> sh], 1ull);
  __syncthreads();
  unsigned long long bv[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int bi = 4 * lane + q;
    bv[q] = S.rbins[0][bi] + S.rbins[1][bi] + S.rbins[2][bi] + S.rbins[3][bi];
  }
  const double ls = (double)((bv[0] + bv[1]) + (bv[2] + bv[3]));
  const double incl = wave_incl_scan(ls, lane);  // counts: exact in double
  const uint64_t bal = __ballot(incl >= (double)k);
  uint32_t fl = lo;
  if (bal) {
    const int lb = __ffsll((unsigned long long)bal) - 1;
    double acc = readlane_d(incl - ls, lb);
    int bs = 4 * lb + 3;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      acc += (double)__builtin_amdgcn_readlane((int)bv[q], lb);
      if (acc >= (double)k) {
        bs = 4 * lb + q;
        break;
      }
    }
    const uint32_t top = hi - ((uint32_t)bs << sh);  // bin bs holds keys [top - 2^sh, top)
    fl = top - lo > (1u << sh) ? top - (1u << sh) : lo;
  }
  __syncthreads();  // every wave has read the bins
  return fl;
}

// ---------------------------------------------------------------------------
// Exact top-p of a row held in registers whose top-p set is too large for a
// candidate window (near-flat rows keep thousands of elements).  One compute
// unit holds the row, so every full pass costs a few microseconds; the path
// makes two:
//   1. a histogram of the members (elements with y > -32) over bins of 1/64
//      binary order of y: per bin the count (bits 20-31) and the sum of the
//      members' offsets inside the bin (8-bit fixed point, bits 0-19), one
//      32-bit LDS add per element, no exponential.  A bin's mass is estimated
//      as count * 2^(-(b + mean offset)/64): the first-order error cancels, the
//      rest (second order, ~1.5e-5, and the offsets' quantisation, ~2e-5) is
//      far below 2^-12 of the bin's mass whatever the values (bf16 rows at low
//      temperature put their members on a few distinct offsets per bin), so
//      the exact crossing of p * Z lies between the first bins where the
//      estimate reaches p * Z (1 -+ 2^-12) (a block scan, every thread holding
//      two bins).  A bin of more than 4095 members wraps its word: its
//      estimate is then wrong, the check in step 3 fails and the exact
//      refinement decides (such rows are nearly constant, and overflow the
//      member segments anyway);
//   2. one pass over the register chunks: each chunk's mass above the bracket
//      (the float sums the inverse CDF uses) to the chunk-mass array, and the
//      members inside the bracket to per-wave LDS segments (a wave-uniform
//      count, no atomics), their positions kept in a bit mask;
//   3. wave 0 checks that the mass above the bracket is below p * Z and that
//      the bracket's members reach it, then splits their key range into 256
//      bins per level (2^-40 fixed-point masses, exact; one wave, so no
//      barrier) down to one key, the threshold;
//   4. the kept masses per chunk are the masses above the bracket plus the
//      kept members (a few per thread), and the inverse CDF walks them.
// Returns false (the exact refinement then decides; nothing it relies on has
// changed) when the bracket misses the crossing or a segment overflows.
// Every wave calls it together.
// ---------------------------------------------------------------------------
constexpr int kDenseRes = 64, kDenseOrders = 32;
constexpr int kDenseBins = kDenseRes * kDenseOrders;  // 2048
constexpr int kDenseCountShift = 20;                  // bin word: count << 20 | sum of 8-bit offsets

template <typename T, int NT, int CAP, bool VEC, int FULL>
__device__ __forceinline__ bool dense_topp(Row<T, NT, CAP, VEC, FULL>& R, const Ex& X, double Z, float p, float u,
                                           Smem<NT>& S, float* csum, int32_t* out) {
  constexpr int EPV = Elem<T>::EPV, SH = KeyShift<T>::value, NW = NT / kWave;
  constexpr int kSegC = 2 * Smem<NT>::kSeg;     // candidate keys per wave (u32 view of S.stage)
  static_assert(kSegC % kWave == 0, "segments hold whole rounds of a wave");
  constexpr int BPT = kDenseBins / NT;           // bins per thread in the scan
  static_assert(BPT * NT == kDenseBins && BPT >= 1, "bins split evenly over the threads");
  static_assert(CAP * EPV <= 64, "member positions fit one 64-bit mask");
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  uint32_t* hist = reinterpret_cast<uint32_t*>(csum);
  const float ylo = -(float)kDenseOrders;
  for (int i = t; i < kDenseBins; i += NT) hist[i] = 0u;
  if (t == 0) {
    S.rbin = -1;                 // bracket top bin (none yet)
    S.pick = kDenseBins - 1;     // bracket bottom bin
  }
  __syncthreads();
  // members: ylo < y <= 0, so bin = trunc(-64 y) lies in [0, kDenseBins)
  auto hist_pass = [&](auto form) {
    constexpr bool FMA = decltype(form)::value;
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      if (R.has(j) && X.y(R.cm_at(j)) > ylo) {
        uint4 v = R.d[j];
        launder(v);
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          const float y = X.template yf<FMA>(Elem<T>::get(v, i));
          if (y > ylo) {
            // q = floor(-64 * 256 y) (a power-of-two scale, exact): bin q >> 8,
            // the 8-bit offset inside the bin q & 255
            const uint32_t q = (uint32_t)(-(float)(kDenseRes * 256) * y);
            atomicAdd(&hist[q >> 8], (1u << kDenseCountShift) | (q & 255u));
          }
        }
      }
    }
  };
  if (X.fma) hist_pass(std::true_type{});
  else hist_pass(std::false_type{});
  __syncthreads();
  row_stamp(3);
  // block scan of the estimates (thread t: bins BPT*t ..)
  const double target = (double)p * Z;
  const double tL = target * (1.0 - 1.0 / 4096.0), tU = target * (1.0 + 1.0 / 4096.0);
  float est[BPT];
#pragma unroll
  for (int q = 0; q < BPT; ++q) {
    const uint32_t hv = hist[BPT * t + q];
    const uint32_t cnt = hv >> kDenseCountShift;
    const float osum = (float)(hv & ((1u << kDenseCountShift) - 1u));
    // mean offset of the members, the truncation of each offset added back
    const float mo = cnt ? osum / (256.0f * (float)cnt) + 0.5f / 256.0f : 0.0f;
    est[q] = (float)cnt * ex2c(-((float)(BPT * t + q) + mo) / (float)kDenseRes);
  }
  float ts = 0.0f;
#pragma unroll
  for (int q = 0; q < BPT; ++q) ts += est[q];
  const double wi = wave_incl_scan((double)ts, lane);
  if (lane == kWave - 1) S.red[wid] = wi;
  __syncthreads();  // every wave has read the histogram: the chunk-mass array is free
  {
    double base = 0.0;
    for (int q = 0; q < wid; ++q) base += S.red[q];
    double c = base + wi - (double)ts;  // estimate above bin BPT*t
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
      const double cn = c + (double)est[q];
      if (c < tL && cn >= tL) S.rbin = BPT * t + q;
      if (c < tU && cn >= tU) S.pick = BPT * t + q;
      c = cn;
    }
  }
  __syncthreads();
  row_stamp(4);
  const int b0 = uni(S.rbin), b1 = uni(S.pick);
  if (b0 < 0) return false;
  // the bracket: bins [b0, b1], i.e. yb < y <= yt
  const float yt = -(float)b0 / (float)kDenseRes;
  const float yb = b1 == kDenseBins - 1 ? ylo : -(float)(b1 + 1) / (float)kDenseRes;
  // one pass: chunk masses above the bracket (to the chunk-mass array),
  // members inside it (to this wave's segment)
  uint32_t* seg = reinterpret_cast<uint32_t*>(S.stage) + wid * kSegC;
  // the candidate list: refinement bin copies 1-3 (wave 0 bins with copy 0)
  uint32_t* list = reinterpret_cast<uint32_t*>(S.rbins[1]);
  constexpr int kList = (int)(3 * (kRefBins + 1) * sizeof(unsigned long long) / sizeof(uint32_t));
  int run = 0;
  float* cs = csum + t;
  double above = 0.0;
  uint64_t inm = 0ull;  // bit j * EPV + i: element i of chunk j lies in the bracket
  // (the generic y here: a copy per form spills registers)
  auto gather_pass = [&]() {
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      uint4 v = R.d[j];
      launder(v);
      float e[EPV];
      uint32_t mj = 0u;
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const float x = Elem<T>::get(v, i);
        const float y = X.y(x);
        e[i] = R.has(j) && y > yt ? ex2c(y) : 0.0f;
        const bool in = R.has(j) && y > yb && y <= yt;
        const uint64_t bm = __ballot(in);
        mj |= (uint32_t)((bm >> lane) & 1ull) << i;  // from the ballot: no flag stays live
        if (bm) {
          const int slot = run + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32),
                                                              __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u));
          if (in && slot < kSegC) seg[slot] = okey(x);
          run += (int)__popcll(bm);
        }
      }
      inm |= (uint64_t)mj << (j * EPV);
      const float cj = tree_sum<EPV>(e);
      cs[j * NT] = cj;
      above += (double)cj;
    }
  };
  gather_pass();
  above = wave_sum(above);
  if (lane == 0) {
    S.wtot[wid] = above;
    S.wcnt[wid] = run;
  }
  __syncthreads();
  row_stamp(5);
  int n = 0;
  bool ovf = false;
  double A = 0.0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    const int cq = S.wcnt[q];
    n += cq;
    ovf = ovf || cq > kSegC;
    A += S.wtot[q];
  }
  if (ovf || n < 1 || n > kList || !(A < target)) return false;
  // the segments -> one list (in the refinement bins' spare copies)
  {
    int pre = 0;
    for (int q = 0; q < wid; ++q) pre += S.wcnt[q];
#pragma unroll
    for (int r = 0; r < kSegC / kWave; ++r) {
      const int sl = r * kWave + lane;
      if (sl < run) list[pre + sl] = seg[sl];
    }
  }
  __syncthreads();
  auto each_cand = [&](auto&& f) {
    for (int i = lane; i < n; i += kWave) f(list[i]);
  };
  if (wid == 0) {
    // the threshold key among the candidates: keys in [lo, hi), fixed-point
    // mass above hi
    const double tfix = target * kFix;
    double Af = A * kFix;
    uint32_t kmn = 0xffffffffu, kmx = 0u;
    double tot = 0.0;
    each_cand([&](uint32_t kx) {
      kmn = min(kmn, kx >> SH);
      kmx = max(kmx, kx >> SH);
      tot += (double)fix40(X.e(okey_inv(kx)));
    });
    uint32_t lo = (uint32_t)wave_min_i((int)(kmn ^ 0x80000000u)) ^ 0x80000000u;
    uint32_t hi = ((uint32_t)wave_max_i((int)(kmx ^ 0x80000000u)) ^ 0x80000000u) + 1u;
    const int found = Af + wave_sum(tot) >= tfix ? 1 : 0;  // the bracket's members reach p * Z
    uint32_t tk = lo;
    unsigned long long* bins = S.rbins[0];
#pragma unroll 1
    for (int level = 0; level < 8 && found && hi - lo > 1u; ++level) {
      int sh = 0;
      while (((hi - lo - 1u) >> sh) >= (uint32_t)kRefBins) ++sh;
#pragma unroll
      for (int q = 0; q < 4; ++q) bins[4 * lane + q] = 0ull;
      each_cand([&](uint32_t kx) {
        const uint32_t kk = kx >> SH;
        if (kk >= lo && kk < hi) atomicAdd(&bins[(hi - 1u - kk) >> sh], fix40(X.e(okey_inv(kx))));
      });
      __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's LDS atomics are done
      double bv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[q] = (double)bins[4 * lane + q];
      const double bl = (bv[0] + bv[1]) + (bv[2] + bv[3]);
      const double binc = wave_incl_scan(bl, lane);
      const uint64_t bb = __ballot(Af + binc >= tfix);
      if (!bb) {  // rounding of the bin sums: keep the whole bracket
        tk = lo;
        break;
      }
      const int lq = __ffsll((unsigned long long)bb) - 1;
      double acc = Af + readlane_d(binc - bl, lq);
      int b2 = 4 * lq + 3;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const double vq = readlane_d(bv[q], lq);
        if (acc + vq >= tfix) {
          b2 = 4 * lq + q;
          break;
        }
        acc += vq;
      }
      Af = acc;
      const uint32_t nhi = hi - ((uint32_t)b2 << sh);
      lo = nhi - lo > (1u << sh) ? nhi - (1u << sh) : lo;
      hi = nhi;
      tk = lo;
    }
    if (lane == 0) {
      S.pick = (int)tk;
      S.rbin = found;
    }
  }
  __syncthreads();
  if (!S.rbin) return false;
  row_stamp(7);
  row_stamp_path(kRowDense);
  const float thr = okey_inv((uint32_t)S.pick << SH);
  // kept masses per register chunk: above the bracket, plus the kept members
  double tmass = 0.0;
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    uint32_t mb = (uint32_t)(inm >> (j * EPV)) & ((1u << EPV) - 1u);
    float cj = cs[j * NT];
    if (mb) {
      const uint4 v = R.d[j];
      for (; mb; mb &= mb - 1u) {
        const float x = Elem<T>::get(v, __builtin_ctz(mb));
        if (x >= thr) cj += X.e(x);
      }
      cs[j * NT] = cj;
    }
    tmass += (double)cj;
  }
  row_stamp(9);
  cdf_walk<true>(R, tmass, cs, [&](int) { return 0.0f; }, [&](float x) { return x >= thr ? X.e(x) : 0.0f; }, u, S,
                 out);
  return true;
}

template <typename T, int NT, int CAP, bool VEC, int FULL>
__device__ __forceinline__ void row_sample_fused(Row<T, NT, CAP, VEC, FULL>& R, const RowArgs& A, int32_t* out,
                                                 Smem<NT>& S, float* csum) {
  constexpr int NW = NT / kWave, EPV = Elem<T>::EPV;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  float* cs = csum + t;
  const bool kon = A.k >= 1 && (uint32_t)A.k < R.V, pon = A.p < 1.0f;
  if (t == 0) {
    S.wn = 0;
    S.kmin = 0xffffffffu;
  }
  if (kon || pon) S.wh[wid][lane] = 0u;  // this wave's histogram (LDS ops of a wave stay in order)

  const bool tvalid = A.T > 0.0f && A.T < INFINITY;
  const float c = tvalid ? kLog2e / A.T : 1.0f;
  // NaN-propagating maxima (v_maximum3, no operand canonicalisation); a wave
  // holding a NaN (sampled as -inf) redoes its maxima ignoring NaN.
  float tm = R.template maxima<true>();
  float wm = wave_maximum(tm);
  if (wm != wm) {
#pragma unroll
    for (int j = 0; j < CAP; ++j) launder(R.d[j]);  // no unpacked value shared with the first pass
    tm = R.template maxima<false>();
    wm = wave_max(tm);
  }
  Ex Xw;  // this wave's shift
  Xw.init_u(wm, c);
  double tmass = 0.0;
  float cmx = 0.0f;  // largest chunk mass of this thread
  if (tvalid) tmass = Xw.fma ? row_masses<true>(R, Xw, cs, &cmx) : row_masses<false>(R, Xw, cs, &cmx);
  {
    const double ws = wave_sum(tmass);
    if (lane == 0) {
      S.wtot[wid] = ws;
      S.wmax[wid] = wm;
    }
  }
  if (kon || pon) {
    // Histogram, relative to this wave's maximum, of the two largest chunk
    // maxima of each thread (distinct elements): count (top-k) or mass
    // (top-p) per bin of y = log2(mass).  Merged into the row's histogram
    // after the barrier.  Masses are added as truncated fixed-point integers
    // (32-bit integer LDS adds: on near-flat rows every lane's maxima share a
    // few bins, and float LDS adds to them took ~1.7 us longer); truncation
    // only lowers a bin's mass, so the floor stays a lower bound.
    typename Row<T, NT, CAP, VEC, FULL>::CM cmv;
    cmv.load(R.cmx);
    float y1 = -INFINITY, y2 = -INFINITY;
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      const float y = R.has(j) ? Xw.y(cmv.get(j)) : -INFINITY;
      y2 = fmaxf(y2, fminf(y1, y));
      y1 = fmaxf(y1, y);
    }
    uint32_t* h = S.wh[wid];
    if (y1 >= kYMin) {
      if (kon) atomicAdd(&h[ybin(y1)], 1u);
      else atomicAdd(&h[ybin(y1)], (uint32_t)(ex2c(y1) * kWaveMassFix));
    }
    if (y2 >= kYMin) {
      if (kon) atomicAdd(&h[ybin(y2)], 1u);
      else atomicAdd(&h[ybin(y2)], (uint32_t)(ex2c(y2) * kWaveMassFix));
    }
    if (!kon && y1 >= kYMin) {
      // The chunk of largest mass M (n = EPV elements, thread maximum m): at
      // any level L at or below y_e = log2((M - m) / (2 (n - 1))) its elements
      // at or above L weigh at least M - (n - 1) 2^L >= (M + m) / 2, which
      // covers what the two maxima above counted from it plus (M - m) / 2.
      // Adds (M - m) / 2 at y_e, so rows whose heaviest elements share a chunk
      // still get a bound.
      const float rest = cmx - ex2c(y1);
      const float ye = rest > 0.0f ? __log2f(rest * (0.5f / (float)(EPV - 1))) : -INFINITY;
      if (ye >= kYMin) atomicAdd(&h[ybin(ye)], (uint32_t)(0.5f * rest * kWaveMassFix));
    }
  }
  __syncthreads();
  row_stamp(1);
  // The rest of the row is short, latency-bound work: let it go ahead of the
  // co-resident workgroup's streaming passes.
  __builtin_amdgcn_s_setprio(2);
  const float gm = lds_max<NW>(S.wmax);
  if (!tvalid || !(gm > -INFINITY) || !(gm < INFINITY)) {
    const int32_t id = row_argmax<NW, T>(R, tm, gm, S.red);
    row_stamp(7);
    row_stamp_path(kRowArgmax);
    if (t == 0) *out = id;
    return;
  }
  Ex X;
  X.init_u(gm, c);
  double sw = 0.0;  // wave masses in the row's reference
  float fq = 0.0f;  // lane q < NW: wave q's mass factor and shift in bins
  int sq = kBins;
  auto wave_refs = [&]() {
    if (lane < NW) {
      Ex Xq;
      Xq.init(S.wmax[lane], c);
      const float d = shift_diff(Xq, X);  // <= 0
      fq = ex2c(d);
      sw = S.wtot[lane] * (double)fq;
      sq = d > -32.0f ? (int)__builtin_ceilf(-2.0f * d + 0x1p-10f) : kBins;
    }
  };

  if (!kon && !pon) {
    row_stamp(7);
    row_stamp_path(kRowWalk);
    wave_refs();
    int wstar;
    double base;
    const double U = cross_wave<NW>(sw, A.u, &wstar, &base);
    if (wid != wstar) return;
    const double fw = (double)shift_ratio(Xw, X);  // this wave's masses -> the row's
    wave_walk<true>(R, cs, fw, base, U, [&](int) { return 0.0f; }, [&](float x) { return Xw.e(x); }, out);
    return;
  }

  // ---- top-k / top-p: candidate window from the chunk maxima -------------
  // Wave 0 derives the normaliser, the histogram bin and the candidate floor
  // for the workgroup (done once, not by every wave: the waves would queue for
  // the same SIMDs); the others wait at the barrier.
  // The count (top-k) or mass (top-p) of distinct elements at or above a bin
  // floor bounds that of all elements from below, so the first bin reaching k
  // or p*Z bounds the threshold from below.  Row bin r gathers bin r - s_q of
  // every wave q: a wave bin's contents sit at least s_q/2 lower in the row's
  // reference (s_q = ceil(2 * shift), with a margin for the rounding of y).
  if (wid == 0) {
    wave_refs();
    const double Zw = wave_sum(sw);
    int pc = 0;
    float pmf = 0.0f;
    int sqs[NW];
    float fqs[NW];
    uint32_t v[NW];
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      sqs[q] = __builtin_amdgcn_readlane(sq, q);
      fqs[q] = readlane_f(fq, q);
    }
#pragma unroll
    for (int q = 0; q < NW; ++q) {  // independent loads (clamped index), issued back to back
      const int idx = lane - sqs[q];
      v[q] = S.wh[q][idx < 0 ? 0 : idx];
    }
    if (kon) {
#pragma unroll
      for (int q = 0; q < NW; ++q) pc += lane >= sqs[q] ? (int)v[q] : 0;
    } else {
#pragma unroll
      for (int q = 0; q < NW; ++q)
        pmf = __builtin_fmaf((float)v[q] * (1.0f / kWaveMassFix), lane >= sqs[q] ? fqs[q] : 0.0f, pmf);
    }
    const int pcs = wave_incl_scan_i(pc, lane);
    const double pm = wave_incl_scan((double)pmf, lane);
    const uint64_t bal = __ballot(kon ? (pcs >= A.k) : (pm >= (double)A.p * Zw * kBinMargin));
    const int b = bal ? (__ffsll((unsigned long long)bal) - 1) : -1;
    const float xl = b >= 0 ? x_at_least(X, bin_floor(b)) : 0.0f;
    if (lane == 0) {
      S.rZ = Zw;
      S.rbin = b;
      S.rxlo = xl;
    }
  }
  __syncthreads();
  if (t < 2 * kWave) {  // small-window ranks (accumulated after the next barrier)
    S.rk_cnt[t] = 0;
    S.rk_fix[t] = 0ull;
  }
  const double Z = uni(S.rZ);
  constexpr int SH = KeyShift<T>::value;
  int bin = uni(S.rbin);
  float xlo = 0.0f;
  if (bin >= 0) {
    xlo = uni(S.rxlo);
  } else if (kon) {
    // top-k beyond the histogram's reach (the k-th largest is more than 32
    // binary orders of magnitude below the maximum): the floor from the
    // threads' maxima bounds it instead
    const uint32_t kneg = okey(-INFINITY) >> SH;
    const uint32_t fl = chunk_max_floor<NT, T>(R, A.k, kneg, (okey(X.gm) >> SH) + 1u, S);
    if (fl > kneg) {
      bin = 0;
      xlo = okey_inv(fl << SH);  // x >= xlo exactly when key >= fl
    }
  }
  if (bin >= 0) {
    // Candidates: elements at or above the floor (x >= xlo), from the chunks
    // whose maximum reaches it.
    uint32_t km = 0;
    {
      typename Row<T, NT, CAP, VEC, FULL>::CM cmv;
      cmv.load(R.cmx);
#pragma unroll
      for (int j = 0; j < CAP; ++j)
        if (R.has(j) && cmv.get(j) >= xlo) km |= 1u << j;
    }
    // Each wave writes its candidates into its own segment in index order
    // (column j, then lane, then element): no atomics, and the window comes
    // out sorted by vocabulary index.
    uint64_t* seg = S.stage + wid * Smem<NT>::kSeg;
    int run = 0;  // candidates of this wave so far (wave-uniform)
    uint32_t kmn = 0xffffffffu;
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      const bool kj = (km >> j) & 1u;
      if (__ballot(kj)) {
        uint4 v = R.d[j];
        launder(v);
        int c = 0;
#pragma unroll
        for (int i = 0; i < EPV; ++i) c += kj && Elem<T>::get(v, i) >= xlo ? 1 : 0;
        const int incl = wave_incl_scan_i(c, lane);
        int pos = run + incl - c;
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          const float x = Elem<T>::get(v, i);
          if (kj && x >= xlo) {
            const uint32_t kx = okey(x);
            if (pos < Smem<NT>::kSeg)
              seg[pos] = ((uint64_t)kx << 32) | (uint64_t)(0xffffffffu - R.elem_index(j, i));
            ++pos;
            kmn = min(kmn, kx);
          }
        }
        run += __builtin_amdgcn_readlane(incl, 63);
      }
    }
    if (lane == 0) S.wcnt[wid] = run;
    if (run > 0) {
      kmn = (uint32_t)wave_min_i((int)(kmn ^ 0x80000000u)) ^ 0x80000000u;
      if (lane == 0) atomicMin(&S.kmin, kmn);
    }
  } else if (lane == 0) {
    S.wcnt[wid] = 0;
  }
  __syncthreads();
  row_stamp(2);
  // window size, segment bases (lane q < NW) and overflow of a segment
  const int cq = lane < NW ? S.wcnt[lane] : 0;
  const int bq_incl = wave_incl_scan_i(cq, lane);
  const int nw = bin >= 0 ? __builtin_amdgcn_readlane(bq_incl, NW - 1) : 0x7fffffff;
  const bool ovf = __ballot(lane < NW && cq > Smem<NT>::kSeg) != 0;
  if (nw <= 2 * kWave && !ovf) {
    // The window reaches the top-k count / top-p mass (bin test above).  Every
    // wave holds the whole window (entries lane and lane + 64, in index order)
    // and ranks it against its own segment; counts and masses (2^-40 fixed
    // point: exact, independent of the order of the LDS atomics) add up in
    // LDS.  Wave 0 then thresholds and walks it alone.
    int w0 = 0, bw0 = 0, w1 = 0, bw1 = 0;
#pragma unroll
    for (int q = 1; q < NW; ++q) {
      const int bq = __builtin_amdgcn_readlane(bq_incl - cq, q);
      if (lane >= bq) {
        w0 = q;
        bw0 = bq;
      }
      if (lane + kWave >= bq) {
        w1 = q;
        bw1 = bq;
      }
    }
    bool in[2];
    uint64_t mine[2];
    uint32_t kx[2];
    float em[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = lane + h * kWave;
      in[h] = q < nw;
      mine[h] = in[h] ? S.stage[(h ? w1 : w0) * Smem<NT>::kSeg + (q - (h ? bw1 : bw0))] : 0ull;
      kx[h] = (uint32_t)(mine[h] >> 32);
      em[h] = in[h] ? X.e(okey_inv(kx[h])) : 0.0f;
    }
    {
      const int cw = __builtin_amdgcn_readlane(cq, wid);
      const uint64_t* seg = S.stage + wid * Smem<NT>::kSeg;
      int cnt[2] = {0, 0};
      unsigned long long fix[2] = {0ull, 0ull};
      for (int i = 0; i < cw; ++i) {
        const uint64_t other = seg[i];
        const unsigned long long eo =
            (unsigned long long)((double)X.e(okey_inv((uint32_t)(other >> 32))) * kFix);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const bool ge = other >= mine[h];
          cnt[h] += ge ? 1 : 0;
          fix[h] += ge ? eo : 0ull;
        }
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
        if (in[h] && cnt[h] > 0) {
          atomicAdd(&S.rk_cnt[lane + h * kWave], cnt[h]);
          atomicAdd(&S.rk_fix[lane + h * kWave], fix[h]);
        }
    }
    __syncthreads();
    if (wid != 0) return;
    int cnt[2];
    double pre[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      cnt[h] = in[h] ? S.rk_cnt[lane + h * kWave] : 0;
      pre[h] = in[h] ? (double)S.rk_fix[lane + h * kWave] * (1.0 / kFix) : 0.0;
    }
    uint32_t tkey;
    if (!window_pick(in, kx, em, cnt, pre, nw, kon, A.k, pon, A.p, Z, &tkey)) tkey = 0u;  // unreachable
    row_stamp(7);
    row_stamp_path(kRowSmall);
    // inverse CDF over the kept entries (key >= tkey), in index order: slot 0
    // of lanes 0..63, then slot 1
    float ek[2];
    int32_t idx[2];
    bool kept[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      kept[h] = in[h] && kx[h] >= tkey;
      idx[h] = (int32_t)(0xffffffffu - (uint32_t)(mine[h] & 0xffffffffu));
      ek[h] = kept[h] ? em[h] : 0.0f;
    }
    const double pre0 = wave_incl_scan((double)ek[0], lane);
    const double pre1 = wave_incl_scan((double)ek[1], lane) + readlane_d(pre0, 63);
    const double total = readlane_d(pre1, 63);
    float u = A.u;
    asm volatile("" : "+s"(u));
    const double U = (double)u * total;
    const uint64_t c0 = __ballot(ek[0] > 0.0f && pre0 > U), c1 = __ballot(ek[1] > 0.0f && pre1 > U);
    const uint64_t p0 = __ballot(ek[0] > 0.0f), p1 = __ballot(ek[1] > 0.0f);
    const uint64_t k0 = __ballot(kept[0]), k1 = __ballot(kept[1]);
    int src = 0, h = 0;
    if (c0) src = __ffsll((unsigned long long)c0) - 1;
    else if (c1) src = __ffsll((unsigned long long)c1) - 1, h = 1;
    else if (p1) src = 63 - __clzll((long long)p1), h = 1;  // u >= 1 or rounding: last with mass
    else if (p0) src = 63 - __clzll((long long)p0);
    else if (k1) src = 63 - __clzll((long long)k1), h = 1;
    else if (k0) src = 63 - __clzll((long long)k0);
    const int id = __builtin_amdgcn_readlane(h ? idx[1] : idx[0], src);
    if (lane == 0) {
      *out = id;
      row_stamp_end();
    }
    return;
  }
  if (bin >= 0 && nw <= Smem<NT>::kWin && !ovf) {
    // compact the segments into S.wkey[0, nw): read, barrier, write (the
    // window overlaps the segments)
    const int q = wid;
    const int cw = __builtin_amdgcn_readlane(cq, q);
    const int bw = __builtin_amdgcn_readlane(bq_incl - cq, q);
    const uint64_t ent = lane < cw ? S.stage[q * Smem<NT>::kSeg + lane] : 0ull;
    __syncthreads();
    if (lane < cw) S.wkey[bw + lane] = ent;
    __syncthreads();
  }
  // ---- larger windows: ranked by the workgroup (<= 512 candidates), else an
  // exact refinement over the window (or over the row when there is no bound)
  if (bin >= 0 && nw <= Smem<NT>::kWin && !ovf) {
    float thr;
    if (window_threshold<NT>(S, nw, kon, A.k, pon, A.p, Z, X, &thr)) {
      row_stamp(7);
      row_stamp_path(kRowRanked);
      if constexpr (FULL != kStream && CAP <= 6) {
        // rows whose register chunks stay live for the dense top-p path: the
        // kept masses and the walk read the registers, not memory
        tmass = 0.0;
#pragma unroll
        for (int j = 0; j < CAP; ++j) {
          float sj = 0.0f;
          if (R.has(j) && R.cm_at(j) >= thr) {
            uint4 v = R.d[j];
            launder(v);
            sj = esum_chunk_ge<T>(v, X, thr);
          }
          cs[j * NT] = sj;
          tmass += (double)sj;
        }
        cdf_walk<true>(R, tmass, cs, [&](int) { return 0.0f; },
                       [&](float x) { return x >= thr ? X.e(x) : 0.0f; }, A.u, S, out);
      } else {
        tmass = masked_masses(R, X, thr, cs);
        cdf_walk<false>(R, tmass, cs, [&](int) { return 0.0f; },
                        [&](float x) { return x >= thr ? X.e(x) : 0.0f; }, A.u, S, out);
      }
      return;
    }
  }
  // Members: the candidate window, or (no bound) for top-k every non-NaN
  // element (the k-th largest can sit any distance below the maximum), for
  // top-p every element with mass at least 2^-40 of the maximum: below that,
  // the whole rest of the row weighs less than 2^-24 of Z, so a boundary there
  // is within the parity tolerance whichever way it falls.
  // (rows of up to six register chunks per thread: with more, the chunks and
  // the path's state exceed the 64 registers of a two-workgroup CU)
  if constexpr (FULL != kStream && CAP <= 6 && NT * CAP * sizeof(float) >= kDenseBins * sizeof(uint32_t)) {
    if (!kon && dense_topp(R, X, Z, A.p, A.u, S, csum, out)) return;
  }
  const uint32_t klo = bin >= 0 ? (uni(S.kmin) >> SH)
                                : (kon ? (okey(-INFINITY) >> SH) : (okey(x_at_least(X, -40.0f)) >> SH));
  uint32_t tk = 0;
  bool ok;
  if (kon) {
    ok = refine_threshold<NT, T>(R, X, Z, true, A.k, 1.0f, klo, S, &tk);
    if (ok && pon) {
      const float thr_k = okey_inv(tk << SH);
      double acc = 0.0;
      R.each_kept_mem([&](float m) { return m >= thr_k; },
                      [&](int, const uint4& v, float) { acc += (double)esum_chunk_ge<T>(v, X, thr_k); });
      const double ZK = wg_sum<NW>(acc, S.red);
      ok = refine_threshold<NT, T>(R, X, ZK, false, 0, A.p, tk, S, &tk);
    }
  } else {
    ok = refine_threshold<NT, T>(R, X, Z, false, 0, A.p, klo, S, &tk);
  }
  const float thr = ok ? okey_inv(tk << SH) : select_exact<NW, T>(R, X, Z, kon, A.k, pon, A.p, S.red);
  row_stamp(7);
  row_stamp_path(kRowRefine);
  tmass = masked_masses(R, X, thr, cs);
  cdf_walk<false>(R, tmass, cs, [&](int) { return 0.0f; }, [&](float x) { return x >= thr ? X.e(x) : 0.0f; },
                  A.u, S, out);
}

// One workgroup per output row b (grid = B_out).  WPE waves per SIMD: 8 lets two
// 1024-thread workgroups share a CU, so one streams its row while the other
// computes.
template <bool GREEDY, typename T, int NT, int CAP, bool VEC, int FULL, int WPE>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(WPE, 8)))
void sampler_kernel(SampleParams P) {
  __shared__ Smem<NT> S;
  __shared__ __align__(16) float csum[GREEDY ? 1 : NT * CAP];  // chunk masses, [j][thread]
  __shared__ uint32_t cmax[NT * Row<T, NT, CAP, VEC, FULL>::kCmWords];  // chunk maxima, [thread][j]
  int64_t nrows = P.B_out;
  if (P.n_rows_dev) nrows = min(nrows, (int64_t)uni(*P.n_rows_dev));
  const int64_t b = blockIdx.x;
  const int64_t r = source_row(P, b, nrows);
  if (r == -1) return;
  if (r == -2) {
    if (threadIdx.x == 0) P.out[b] = -1;
    return;
  }
  // The arguments' loads go out before the row's and are made wave-uniform
  // after it: converting right away would wait a full memory round trip
  // before the row is requested.
  row_stamp(0);
  RowArgs A{};
  if (!GREEDY) A = row_args_load(P, r);
  Row<T, NT, CAP, VEC, FULL> R;
  R.init(P.logits, r, P.ld, P.V, cmax);
  R.fetch();
  if (GREEDY) row_greedy(R, &P.out[b], S);
  else if (R.nstream() <= CAP) row_sample_fused(R, uniform(A), &P.out[b], S, csum);
  else row_sample(R, uniform(A), &P.out[b], S, csum);
}

// ---------------------------------------------------------------------------
// Host launch.  One workgroup per output row; rows past the device row count
// (n_rows_dev) exit at once.
//   chunks per row NV <= 256*8    256 threads, 8 chunks each in registers
//   NV == 1024*6 (e.g. 49152 bf16) 1024 threads, exactly 6 full chunks each
//   NV <= 1024*8                  1024 threads, 8 chunks each (two per CU)
//   NV == 1024*12 (49152 fp32)    1024 threads, exactly 12 full chunks each
//                                 (16 chunks spill registers)
//   NV <= 1024*16                 1024 threads, 16 chunks each (one per CU)
//   longer rows                   1024 threads, 16 chunks each, the rest streamed
// Unaligned rows (row start or stride not 16-byte aligned) use element loads.
// ---------------------------------------------------------------------------
template <class K>
static void launch(K kernel, int NT, const SampleParams& P, hipStream_t st) {
  hipLaunchKernelGGL(kernel, dim3((unsigned)P.B_out), dim3(NT), 0, st, P);
}

template <typename T, bool G>
static void launch_rows(const SampleParams& P, bool vec, hipStream_t st) {
  constexpr int EPV = Elem<T>::EPV;
  const int64_t NV = (P.V + EPV - 1) / EPV;
  if (!vec) launch(sampler_kernel<G, T, 1024, 16, false, kStream, 4>, 1024, P, st);
  else if (NV <= 256 * 8) launch(sampler_kernel<G, T, 256, 8, true, kBounded, 8>, 256, P, st);
  else if (NV == 1024 * 8 && P.V % EPV == 0) launch(sampler_kernel<G, T, 1024, 8, true, kFull, 8>, 1024, P, st);
  else if (NV == 1024 * 6 && P.V % EPV == 0) launch(sampler_kernel<G, T, 1024, 6, true, kFull, 8>, 1024, P, st);
  else if (NV <= 1024 * 8) launch(sampler_kernel<G, T, 1024, 8, true, kBounded, 8>, 1024, P, st);
  else if (NV == 1024 * 12 && P.V % EPV == 0) launch(sampler_kernel<G, T, 1024, 12, true, kFull, 4>, 1024, P, st);
  else if (NV == 1024 * 16 && P.V % EPV == 0) launch(sampler_kernel<G, T, 1024, 16, true, kFull, 4>, 1024, P, st);
  else if (NV <= 1024 * 16) launch(sampler_kernel<G, T, 1024, 16, true, kBounded, 4>, 1024, P, st);
  else launch(sampler_kernel<G, T, 1024, 16, true, kStream, 4>, 1024, P, st);
}

template <typename T>
static int launch_dtype(const SampleParams& P, bool greedy, bool vec, hipStream_t st) {
  constexpr int EPV = Elem<T>::EPV;
  const int64_t NV = (P.V + EPV - 1) / EPV;
  // Chunk byte offsets are 32-bit.
  if (NV >= (int64_t)1 << 27)
    return set_error(LSG_ERR_ARG, "lsg_sample: V=%lld too large", (long long)P.V);
  if (greedy) launch_rows<T, true>(P, vec, st);
  else launch_rows<T, false>(P, vec, st);
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
  if (quad_sample_launch(P, dtype, greedy, vec, st)) return check_launch("lsg_sample");
  int rc;
  if (dtype == kF32) rc = launch_dtype<float>(P, greedy, vec, st);
  else if (dtype == kBF16) rc = launch_dtype<bf16_t>(P, greedy, vec, st);
  else rc = launch_dtype<f16_t>(P, greedy, vec, st);
  if (rc != LSG_OK) return rc;
  return check_launch("lsg_sample");
}

#ifdef LSG_PHASE_STAMPS
// Copies the phase stamps of the one-row-per-workgroup sampler's last launch.
extern "C" int lsg_row_stamps_read(void* dst, size_t bytes) {
  const size_t n = sizeof(lsg::g_row_stamps);
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(lsg::g_row_stamps), bytes < n ? bytes : n, 0, hipMemcpyDeviceToHost);
}
#endif
