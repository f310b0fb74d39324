// Token sampling with one workgroup per row, the row streamed through registers.
//
// Replaces, for the decode token path of Loop-SGLang:
//   Sampler.sample            python/loopsgl/model_executor/sample.py:107-112
//   torch.argmax (greedy)     sample.py:110-111 (+ int32 cast, model_runner.py:279-280)
//   sample_impl -> flashinfer softmax / *_sampling_from_probs   sample.py:60-81
// for batches of more rows than compute units whose rows are exactly 256 * CAP
// 16-byte chunks (V = 65536 or 49152 for bf16/fp16, 32768 or 24576 for fp32;
// fp32 rows of 65536 take eight waves); sample.hip serves every other case with
// the same semantics:
//   T <= 0 or non-finite, or max x non-finite  -> id = argmax (torch rules)
//   m = max x (NaN ignored), e_i = 2^((x_i - m) * log2(e)/T)
//   K = {x >= k-th largest x} if 1 <= k < V            (ties kept)
//   P = {x in K : x >= tau}, tau = largest x with mass(x >= tau) >= p * mass(K)
//   id = first index j in P (ascending) with cumsum_P(e)[j] > u * sum_P(e)
//
// Structure (four four-wave rows resident per compute unit, so a batch of 1024
// rows runs in one generation):
//   * each lane streams its CAP nontemporal 128-bit loads through a rolling
//     window of 16; wave w owns chunks [w*CAP*64, (w+1)*CAP*64), its j-th load
//     reads the 64 chunks (w*CAP + j)*64 + lane (1 KiB contiguous), so index
//     order is (wave, j, lane, element);
//   * one pass over chunk pairs as they arrive: a running maximum per lane with
//     the masses rescaled whenever it rises (e = 2^((x - max) c) is exact near
//     the maximum, whatever the data), the lane's two largest pair maxima and a
//     16-bit upper bound of every chunk maximum (to LDS);
//   * barrier 1: the row maximum and normaliser from the wave summaries;
//     unfiltered rows walk the inverse CDF right away (crossing wave, chunk,
//     lane, element; chunks re-read from memory);
//   * top-k / top-p rows: a histogram of the lanes' two largest pair maxima
//     (distinct elements) bounds the threshold from below; every wave lists its
//     chunks whose bounds reach it and gathers them from memory, staging the
//     elements above the bound in index order; barrier 2; one wave finishes
//     the window: at most 64 entries from an LDS table (counts and masses at or
//     above each entry, a scan for the draw), up to 512 with a 1/8-binary-order
//     histogram and an exact resolution inside the crossing bin.  Larger
//     windows take the two-pass exact top-p or the exact radix refinement.
// Sums above the chunk level are float64; window masses are 2^-40 fixed point,
// so the threshold sums are exact and independent of atomic order.
#include <type_traits>

#include "lsg_capi_internal.h"
#include "lsg_common.h"
#include "lsg_sample.h"

namespace lsg {
namespace quad {

// A row is held by NW waves (NW * 64 threads, CAP 16-byte chunks per lane);
// the per-wave capacities of the window and of the exact top-p candidates
// shrink as NW grows, so their row totals stay fixed.
constexpr int seg_cap(int nw) { return 1024 / nw; }   // window entries staged per wave
constexpr int stg_cap(int nw) { return 512 / nw; }    // candidate chunks staged per wave
// exact top-p candidates per wave (four-wave rows: 1024, so that four rows fit
// one compute unit's LDS)
constexpr int cand_cap(int nw) { return nw == 4 ? 256 : 1536 / nw; }
// Loads in flight per lane during the pass: the row streams through a rolling
// window of 16 chunks per lane (the chunks are not kept: later phases re-read
// the few they need), so that four four-wave rows, or two eight-wave rows, are
// resident per compute unit (128 registers, four waves per SIMD).
constexpr int kLoadWindow = 16;
constexpr int kWavesPerEU = 4;
constexpr int kHB = 128;          // coarse histogram: bins of 1/4 binary order over y in [-32, 0]
constexpr int kFB = 256;          // fine histogram: bins of 1/8 binary order over y in [-32, 0]
constexpr int kFarBin0 = 0x42000000 >> 18;  // float bits of 32.0 >> 18: far-floor bin 1 starts at d = 32
constexpr int kWin = 512;         // window finished by one wave
constexpr int kHPL = kWin / kWave;  // window entries per lane in the finish
constexpr int kRB = 256;          // refinement bins per level
constexpr int kVB = 512;          // value bins bracketing an exact top-p threshold
constexpr double kFix = 1099511627776.0;  // 2^40
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kNonTemporal = 2;   // buffer-load cache policy: stream through the caches
// Top-p bin test margin: the bin is chosen where the float sums of the binned
// chunk maxima reach p*Z*(1 + 2^-10), so the window always reaches p*Z despite
// the rounding of those sums.
constexpr double kBinMargin = 1.0 + 1.0 / 1024.0;

// Phase stamps, compiled in only by the profiling build (-DLSG_PHASE_STAMPS):
// thread 0 of workgroup b writes the 100 MHz real-time counter at fixed points
// of its row to g_phase_stamps[b * 8 + slot] (slots: 0 kernel entry, 1 wave 0's
// pass done, 2 barrier 1 passed, 3 floor known, 4 candidates staged, 5 end,
// 7 the row's first loads issued); slot 6 holds the hardware id (bits 0-31),
// the XCC id (32-39) and the row's path (40-47: 1 window, 2 two-pass top-p,
// 3 exact refinement, 4 unfiltered walk, 5 argmax, 6 small window).
constexpr int kStampSlots = 8, kStampRows = 8192;
enum StampPath { kPathWindow = 1, kPathTopp = 2, kPathExact = 3, kPathWalk = 4, kPathArgmax = 5, kPathSmall = 6 };
#ifdef LSG_PHASE_STAMPS
__device__ unsigned long long g_phase_stamps[kStampRows * kStampSlots];
__device__ __forceinline__ void stamp_val(int slot, unsigned long long v) {
  if (threadIdx.x == 0 && blockIdx.x < (unsigned)kStampRows) g_phase_stamps[blockIdx.x * kStampSlots + slot] = v;
}
__device__ __forceinline__ void stamp(int slot) { stamp_val(slot, __builtin_amdgcn_s_memrealtime()); }
__device__ __forceinline__ void stamp_path(int path) {
  // HW_ID (hwreg 4: wave, SIMD, CU, SH, SE) and XCC_ID (hwreg 20)
  const uint32_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
  const uint32_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xffu;
  stamp_val(6, ((unsigned long long)path << 40) | ((unsigned long long)xcc << 32) | hw);
}
#else
__device__ __forceinline__ void stamp_val(int, unsigned long long) {}
__device__ __forceinline__ void stamp(int) {}
__device__ __forceinline__ void stamp_path(int) {}
#endif

// 2^y clamped to [0, 1]: folds into v_exp_f32's clamp, NaN -> 0.
__device__ __forceinline__ float ex2c(float y) {
  return __builtin_amdgcn_fmed3f(__builtin_amdgcn_exp2f(y), 0.0f, 1.0f);
}
// IEEE maximum (NaN-propagating, no operand canonicalisation): v_maximum3_f32.
__device__ __forceinline__ float fmx(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// floor(e * 2^40) for a mass e in [0, 1], from its bits (exact).
__device__ __forceinline__ unsigned long long fix40(float e) {
  const uint32_t b = __float_as_uint(e);
  const int E = (int)(b >> 23) - 110;
  const unsigned long long m = (unsigned long long)((b & 0x7fffffu) | 0x800000u);
  if (b < 0x00800000u || E <= -24) return 0ull;
  return E >= 0 ? (m << E) : (m >> -E);
}

// Upper bound of a float as a bf16 bit pattern (exact for bf16 values).
__device__ __forceinline__ uint32_t bf16_up(float m) {
  const uint32_t b = __float_as_uint(m);
  return (b & 0x80000000u) ? (b >> 16) : ((b + 0xffffu) >> 16);
}

// A 16-byte chunk as one 128-bit register tuple.
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Elements of a 16-byte chunk as floats.
template <typename T>
struct QE;
template <>
struct QE<bf16_t> {
  static constexpr int EPV = 8, SH = 16;
  __device__ static __forceinline__ void unpack(const v4u& v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = __uint_as_float(w[k] << 16);
      x[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
    }
  }
};
template <>
struct QE<f16_t> {
  static constexpr int EPV = 8, SH = 13;
  __device__ static __forceinline__ void unpack(const v4u& v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xffffu));
      x[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16));
    }
  }
};
template <>
struct QE<float> {
  static constexpr int EPV = 4, SH = 0;
  __device__ static __forceinline__ void unpack(const v4u& v, float (&x)[4]) {
    x[0] = __uint_as_float(v.x);
    x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z);
    x[3] = __uint_as_float(v.w);
  }
};

template <int N>
__device__ __forceinline__ float tree_sum(float (&e)[N]) {
#pragma unroll
  for (int w = 1; w < N; w <<= 1)
#pragma unroll
    for (int i = 0; i < N; i += 2 * w) e[i] += e[i + w];
  return e[0];
}

template <int CAP, int NW>
struct Smem {
  uint32_t cm[(NW * kWave)][CAP / 2 + 1];  // chunk-maximum upper bounds, two 16-bit patterns per word (odd stride: no bank conflicts)
  uint32_t wh[NW][kHB];      // per-wave coarse histograms (count, or mass as float bits)
  union {
    struct {                                      // top-k / top-p window
      uint64_t seg[NW][seg_cap(NW)];                    // window entries per wave, index order
      unsigned long long fmass[kFB];              // fine histogram: masses (2^-40 fixed point)
      uint32_t fcnt[kFB];                         // fine histogram: counts
      uint32_t smeta[NW][stg_cap(NW)];                  // candidate chunks per wave: column * 64 + lane
    };
    struct {                                      // exact refinement and its inverse CDF
      unsigned long long rb[4][kRB + 1];          // refinement bins, four copies by lane
      double colsum[NW][CAP];                    // kept mass per wave and chunk column
    };
    struct {                                      // exact top-p, pass 1
      uint32_t vh[NW][kVB + 1];                  // value histograms per wave (bin kVB: sink), 2^-16 of the bin top
    };
    struct {                                      // exact top-p, pass 2 and the threshold
      uint32_t ckey[NW][cand_cap(NW)];                    // bracket candidates per wave: order key >> SH,
      float cmass[NW][cand_cap(NW)];                      //   mass,
      uint32_t cpos[NW][cand_cap(NW)];                    //   (column * 64 + lane) * 8 + element
      double kbin[kRB];                           // key bins (masses)
      double ksum[NW][CAP];                      // kept mass per wave and chunk column
    };
  };
  float wmax[NW];
  double wz[NW];
  double red[NW];
  double rz;
  v4u lt[(NW * kWave)];  // per lane: largest, second-largest chunk maximum, chunk of the largest
  int cnt[NW];
  int imin;
};

// LDS of the all-greedy kernel.
template <int NW>
struct GSmem {
  float wmax[NW];
  int imin;
};

// A row in registers: CAP chunks per lane, wave-blocked.
template <typename T, int CAP>
struct Row {
  static constexpr int EPV = QE<T>::EPV;
  v4u d[CAP];
  __amdgpu_buffer_rsrc_t rs;
  uint32_t c0;  // chunk index of this lane's load j = 0
  __device__ __forceinline__ void init(const void* logits, int64_t r, int64_t ld, uint32_t V) {
    const char* base = reinterpret_cast<const char*>(logits) + r * ld * (int64_t)sizeof(T);
    rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)(V * (uint32_t)sizeof(T)),
                                           0x00020000);
    c0 = (uint32_t)(threadIdx.x >> 6) * (uint32_t)(CAP * kWave) + (threadIdx.x & 63);
  }
  // Load j of this lane (streamed past the caches).
  __device__ __forceinline__ void issue(int j) {
    d[j] = __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(c0 * 16u), j * kWave * 16, kNonTemporal);
  }
  // The first kLoadWindow loads; the pass issues the rest as it goes.
  __device__ __forceinline__ void fetch() {
    static_assert(CAP > kLoadWindow, "rows stream through the load window");
#pragma unroll
    for (int j = 0; j < kLoadWindow; ++j) issue(j);
  }
  // After chunk j is unpacked: the load that takes its place in the window.
  __device__ __forceinline__ void roll(int j) {
    if (j + kLoadWindow < CAP) issue(j + kLoadWindow);
  }
  // Chunk `chunk` of the row re-read from memory (cold paths: the register
  // copy is then no longer needed, so those paths add no register pressure).
  __device__ __forceinline__ v4u load_at(uint32_t chunk) const {
    return __builtin_amdgcn_raw_buffer_load_b128(rs, (int)(chunk * 16u), 0, 0);
  }
  __device__ __forceinline__ v4u load(int j) const { return load_at(c0 + (uint32_t)j * kWave); }
  __device__ __forceinline__ uint32_t elem(int j, int i) const { return (c0 + (uint32_t)j * kWave) * EPV + i; }
  // Mark the chunks as possibly changed, so that values unpacked from them in an
  // earlier phase are recomputed instead of kept live (which would double the
  // registers the row needs).
  __device__ __forceinline__ void launder() const {
#pragma unroll
    for (int j = 0; j < CAP; ++j) asm volatile("" : "+v"(const_cast<v4u&>(d[j])));
  }
};

// Chunk-maximum upper bound j of this thread, from LDS.
template <int CAP, int NW>
__device__ __forceinline__ float cm_at(const Smem<CAP, NW>& S, int j) {
  const uint32_t w = S.cm[threadIdx.x][j >> 1];
  return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
}

// f(j, chunk, keep) over this lane's chunks re-read from memory, eight loads
// in flight at a time; chunks whose maximum bound fails keep() in every lane of
// the wave are skipped (and not loaded by the lanes that fail it).
template <typename T, int CAP, class K, class F, int NW>
__device__ __forceinline__ void each_chunk_mem(const Row<T, CAP>& R, const Smem<CAP, NW>& S, K&& keep, F&& f) {
  static_assert(CAP % 8 == 0, "chunks are re-read in groups of eight");
#pragma unroll 1
  for (int jb = 0; jb < CAP; jb += 8) {
    v4u v[8];
    bool kp[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      kp[q] = keep(cm_at(S, jb + q));
      v[q] = kp[q] ? R.load(jb + q) : v4u{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (__ballot(kp[q])) f(jb + q, v[q], kp[q]);
  }
}

struct LaneStats {
  float ml, t1, t2;  // running maximum, two largest chunk-pair maxima
  int j1;            // chunk pair holding t1 (chunks 2 j1 and 2 j1 + 1)
  double S;          // mass relative to ml
};

// The pass over the lane's chunks, two at a time (loads already issued):
// running maximum, masses rescaled to it, the two largest chunk-pair maxima
// (distinct elements), chunk-maximum bounds to LDS.  The running maximum, its
// rescaling and the pair bookkeeping happen once per 16-byte chunk pair.
// NANIGN: NaN elements are ignored (a second pass for rows holding NaN);
// otherwise NaN propagates into the maximum and marks the row for that pass.
template <bool NANIGN, typename T, int CAP, int NW>
__device__ __forceinline__ LaneStats lane_pass(Row<T, CAP>& R, float c, Smem<CAP, NW>& S) {
  constexpr int EPV = QE<T>::EPV;
  static_assert(CAP % 2 == 0, "chunks are taken in pairs");
  LaneStats s{-INFINITY, -INFINITY, -INFINITY, 0, 0.0};
#pragma unroll
  for (int j = 0; j < CAP; j += 2) {
    float x[2 * EPV];
    // NANIGN (rare rows holding NaN): chunks re-read from memory, so this pass
    // adds no register pressure to the register-resident row
    QE<T>::unpack(NANIGN ? R.load(j) : R.d[j], *reinterpret_cast<float(*)[EPV]>(&x[0]));
    if constexpr (!NANIGN) R.roll(j);
    QE<T>::unpack(NANIGN ? R.load(j + 1) : R.d[j + 1], *reinterpret_cast<float(*)[EPV]>(&x[EPV]));
    if constexpr (!NANIGN) R.roll(j + 1);
    float cm0 = x[0], cm1 = x[EPV];
#pragma unroll
    for (int i = 1; i < EPV; ++i) {
      cm0 = NANIGN ? fmaxf(cm0, x[i]) : fmx(cm0, x[i]);
      cm1 = NANIGN ? fmaxf(cm1, x[EPV + i]) : fmx(cm1, x[EPV + i]);
    }
    const float cp = NANIGN ? fmaxf(cm0, cm1) : fmx(cm0, cm1);
    const float mn = NANIGN ? fmaxf(s.ml, cp) : fmx(s.ml, cp);
    const float f = ex2c((s.ml - mn) * c);
    // masses in quarters of the pair (fewer values live at once)
    float cs;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float e[EPV / 2];
#pragma unroll
      for (int i = 0; i < EPV / 2; ++i) e[i] = ex2c((x[h * (EPV / 2) + i] - mn) * c);
      cs = h ? cs + tree_sum(e) : tree_sum(e);
      asm volatile("" : "+v"(cs));
    }
    s.S = __builtin_fma(s.S, (double)f, (double)cs);
    s.ml = mn;
    const float ct = NANIGN ? (cp == cp ? cp : -INFINITY) : cp;
    s.t2 = __builtin_amdgcn_fmed3f(s.t1, s.t2, ct);
    s.j1 = ct > s.t1 ? (j >> 1) : s.j1;
    s.t1 = fmx(s.t1, ct);
    // (a bf16 chunk maximum is its own bound)
    if constexpr (std::is_same<T, bf16_t>::value)
      S.cm[threadIdx.x][j >> 1] = (__float_as_uint(cm0) >> 16) | (__float_as_uint(cm1) & 0xffff0000u);
    else
      S.cm[threadIdx.x][j >> 1] = bf16_up(cm0) | (bf16_up(cm1) << 16);
    // materialise the running state here (not sunk to its first use, which
    // would keep every chunk's operands live), one pair at a time
    asm volatile("" : "+v"(s.ml), "+v"(s.t1), "+v"(s.t2), "+v"(s.j1), "+v"(s.S));
    __builtin_amdgcn_sched_barrier(0);
  }
  return s;
}

// Maximum pass only (argmax): NaN-propagating lane maximum and the first chunk
// at which it was reached (for NaN: the first chunk holding a NaN).  Streaming
// (!MEM), the lane keeps a copy of that chunk in *best as it goes.
template <bool MEM, typename T, int CAP>
__device__ __forceinline__ float lane_max(Row<T, CAP>& R, int* fj, v4u* best) {
  constexpr int EPV = QE<T>::EPV;
  constexpr bool ST = !MEM;
  float ml = -INFINITY;
  int f = 0;
  v4u bv = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < CAP; ++j) {
    float x[EPV];
    QE<T>::unpack(MEM ? R.load(j) : R.d[j], x);
    float cm = x[0];
#pragma unroll
    for (int i = 1; i < EPV; ++i) cm = fmx(cm, x[i]);
    // chunk 0 seeds the copy (a lane of -inf reaches its maximum there)
    const bool hit = j == 0 || cm > ml || (cm != cm && ml == ml);
    f = hit ? j : f;
    if constexpr (ST) {
      bv.x = hit ? R.d[j].x : bv.x;
      bv.y = hit ? R.d[j].y : bv.y;
      bv.z = hit ? R.d[j].z : bv.z;
      bv.w = hit ? R.d[j].w : bv.w;
      R.roll(j);
    }
    ml = fmx(ml, cm);
    if constexpr (ST) asm volatile("" : "+v"(ml), "+v"(f), "+v"(bv));
    else asm volatile("" : "+v"(ml), "+v"(f));
    __builtin_amdgcn_sched_barrier(0);
  }
  *fj = f;
  *best = bv;
  return ml;
}

// Sum of one double per wave over the workgroup, in wave order (all waves call).
template <int CAP, int NW>
__device__ __forceinline__ double wg_sum(Smem<CAP, NW>& S, double wv) {
  if ((threadIdx.x & 63) == 0) S.red[threadIdx.x >> 6] = wv;
  __syncthreads();
  double r = S.red[0];
#pragma unroll
  for (int q = 1; q < NW; ++q) r += S.red[q];
  __syncthreads();
  return r;
}

// torch.argmax over the row (first maximum; the first NaN if any): every wave calls.
// MEM: the chunks are re-read from memory (a rare path of the sampling kernel).
template <bool MEM, int NW, typename T, int CAP, class SM>
__device__ __forceinline__ void row_argmax(Row<T, CAP>& R, SM& S, int32_t* out) {
  constexpr int EPV = QE<T>::EPV;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int fj;
  v4u best;
  const float ml = lane_max<MEM>(R, &fj, &best);
  const float wm = wave_maximum(ml);
  __syncthreads();  // earlier readers of S are done
  if (threadIdx.x == 0) S.imin = 0x7fffffff;
  if (lane == 0) S.wmax[wid] = wm;
  __syncthreads();
  float mw = S.wmax[0];
#pragma unroll
  for (int q = 1; q < NW; ++q) mw = fmx(mw, S.wmax[q]);
  const float m = uni(mw);
  const bool isn = m != m;
  const bool cand = isn ? (ml != ml) : (ml == m);
  // the chunk where this lane first reached the maximum
  const v4u v = MEM ? R.load(fj) : best;
  float x[EPV];
  QE<T>::unpack(v, x);
  int first = 0x7fffffff;
#pragma unroll
  for (int i = EPV - 1; i >= 0; --i) {
    const bool hit = (int)isn ? (x[i] != x[i]) : (x[i] == m);
    first = hit ? (int)R.elem(fj, i) : first;
  }
  first = cand ? first : 0x7fffffff;
  const int wf = wave_min_i(first);
  if (lane == 0 && wf != 0x7fffffff) atomicMin(&S.imin, wf);
  __syncthreads();
  if (threadIdx.x == 0) *out = S.imin;
}

// Wave q's mass in the row frame (maximum m), recomputed from the published
// wave summaries wherever needed (identical in every wave; keeping the waves'
// masses live across the tail would cost registers the row needs).
template <int CAP, int NW>
__device__ __forceinline__ double wave_mass(const Smem<CAP, NW>& S, int q, float m, float c) {
  return S.wz[q] * (double)ex2c((S.wmax[q] - m) * c);
}

// Inverse CDF in index order (wave, chunk column j, lane, element) over
// kept masses.  The crossing wave of U = u * Z comes from the waves' masses Zq
// (identical in every wave); the others return.  Sets *Uw (mass to go from
// the start of the crossing wave).
// Sum over the waves, in wave order, of zq(q) (a wave's mass read from LDS).
template <int NW, class ZQ>
__device__ __forceinline__ double wave_total(ZQ&& zq) {
  double z = zq(0);
#pragma unroll
  for (int q = 1; q < NW; ++q) z += zq(q);
  return z;
}

template <int NW, class ZQ>
__device__ __forceinline__ int cross_wave(ZQ&& zq, float u, double* Uw) {
  const double Z = wave_total<NW>(zq);
  const double U = (double)uni(u) * Z;
  int ws = -1, wl = 0;
  double acc = 0.0, bw = 0.0, bl = 0.0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    const double z = zq(q);
    if (z > 0.0) {
      wl = q;
      bl = acc;
    }
    if (ws < 0 && acc + z > U) {
      ws = q;
      bw = acc;
    }
    acc += z;
  }
  if (ws < 0) {  // u >= 1 or rounding: the last wave with mass
    ws = wl;
    bw = bl;
  }
  *Uw = U - bw;
  return ws;
}

// In the crossing wave ws, with the crossing column js (colex: the wave's mass
// in the columns before it): v is this lane's chunk of column js; finds the
// lane, then the element, and writes the id.
template <typename T, int CAP, class EM>
__device__ __forceinline__ void finish_column(const v4u& v, int ws, int js, double colex, double Uw, EM&& emass,
                                              int32_t* out) {
  constexpr int EPV = QE<T>::EPV;
  const int lane = threadIdx.x & 63;
  float x[EPV], em[EPV];
  QE<T>::unpack(v, x);
  double lm = 0.0;
#pragma unroll
  for (int i = 0; i < EPV; ++i) {
    em[i] = emass(x[i]);
    lm += (double)em[i];
  }
  const double inc = colex + wave_incl_scan(lm, lane);
  const double exc = inc - lm;
  int ls;
  {
    const uint64_t hit = __ballot(lm > 0.0 && inc > Uw);
    const uint64_t pos = __ballot(lm > 0.0);
    ls = hit ? __ffsll((unsigned long long)hit) - 1 : (pos ? 63 - __clzll((long long)pos) : 0);
  }
  if (lane == ls) {
    double a = exc;
    int pick = -1, last = -1;
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      if (em[i] > 0.0f) {
        last = i;
        a += (double)em[i];
        if (pick < 0 && a > Uw) pick = i;
      }
    }
    if (pick < 0) pick = last < 0 ? 0 : last;
    *out = (int32_t)(((uint32_t)(ws * CAP + js) * kWave + (uint32_t)ls) * EPV + pick);
  }
}

// Unfiltered rows: the crossing wave re-reads its chunks from memory, eight
// columns in flight at a time, sums the columns in order until U is crossed,
// then finishes that column.  (The register copy of the row is left to the
// top-k / top-p path, which needs it on every row.)
template <typename T, int CAP, class EM, int NW>
__device__ __forceinline__ void walk_cols(const Row<T, CAP>& R, const Smem<CAP, NW>& S, float m, float c, float u,
                                          EM&& emass, int32_t* out) {
  constexpr int EPV = QE<T>::EPV;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  double Uw;
  const int ws = cross_wave<NW>([&](int q) { return wave_mass(S, q, m, c); }, u, &Uw);
  if (wid != ws) return;
  double acc = 0.0, accl = 0.0;
  int js = -1, jl = 0;
#pragma unroll 1
  for (int jb = 0; jb < CAP && js < 0; jb += 8) {
    v4u v[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = R.load(jb + q);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (js < 0) {
        float x[EPV], e[EPV];
        QE<T>::unpack(v[q], x);
#pragma unroll
        for (int i = 0; i < EPV; ++i) e[i] = emass(x[i]);
        const double C = wave_sum((double)tree_sum(e));
        if (C > 0.0) {
          jl = jb + q;
          accl = acc;
        }
        if (acc + C > Uw) js = jb + q;
        else acc += C;
      }
    }
  }
  if (js < 0) {  // rounding: the last column with mass
    js = jl;
    acc = accl;
  }
  finish_column<T, CAP>(R.load(js), ws, js, acc, Uw, emass, out);
}

// Bitwise OR over the wave (identical in every lane).
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
  v |= (uint32_t)dpp_i<0x128>(0, (int)v);
  v |= (uint32_t)dpp_i<0x124>(0, (int)v);
  v |= (uint32_t)dpp_i<0x122>(0, (int)v);
  v |= (uint32_t)dpp_i<0x121>(0, (int)v);
  return (uint32_t)(__builtin_amdgcn_readlane((int)v, 0) | __builtin_amdgcn_readlane((int)v, 16) |
                    __builtin_amdgcn_readlane((int)v, 32) | __builtin_amdgcn_readlane((int)v, 48));
}

// Smallest value with order key >= kk (keys below -inf's are NaN patterns).
__device__ __forceinline__ float key_value(uint32_t kk) {
  return kk <= okey(-INFINITY) ? -INFINITY : okey_inv(kk);
}

// Exact top-k (count target) or top-p (mass target, 2^-40 fixed point) threshold
// by radix refinement over order keys (okey(x) >> SH) of the members: non-NaN
// elements with y(x) >= Lm and x >= xmin.  Each level splits the bracket
// [lo, hi) holding the boundary into 256 bins (one LDS atomic per member, four
// bin copies picked by lane); the scan from the top with the totals above the
// bracket picks the bin; down to one key (ties kept).  Every wave calls.
template <typename T, int CAP, int NW>
__device__ __forceinline__ bool refine(const Row<T, CAP>& R, Smem<CAP, NW>& S, float m, float c, float Lm, float xmin, bool kon,
                       double target, uint32_t* thr_key) {
  constexpr int EPV = QE<T>::EPV, SH = QE<T>::SH;
  const int t = threadIdx.x, lane = t & 63;
  uint32_t lo = okey(xmin) >> SH, hi = (okey(m) >> SH) + 1u;
  double above = 0.0;
  for (int level = 0; level < 8; ++level) {
    if (hi <= lo) return false;
    int sh = 0;
    while (((hi - lo - 1u) >> sh) >= (uint32_t)kRB) ++sh;
    for (int i = t; i < 4 * (kRB + 1); i += (NW * kWave)) (&S.rb[0][0])[i] = 0ull;
    __syncthreads();
    const uint32_t lo_ = lo, hi_ = hi;
    const float xlo = key_value(lo << SH);
    unsigned long long* mine = S.rb[lane & 3];
    each_chunk_mem(R, S, [&](float cb) { return cb >= xlo && (cb - m) * c >= Lm; },
                   [&](int, const v4u& v, bool may) {
                     float x[EPV];
                     QE<T>::unpack(v, x);
#pragma unroll
                     for (int i = 0; i < EPV; ++i) {
                       const uint32_t key = okey(x[i]) >> SH;
                       const float y = (x[i] - m) * c;
                       if (may && x[i] == x[i] && x[i] >= xmin && y >= Lm && key >= lo_ && key < hi_)
                         atomicAdd(&mine[(hi_ - 1u - key) >> sh], kon ? 1ull : fix40(ex2c(y)));
                     }
                   });
    __syncthreads();
    double bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int bi = 4 * lane + q;
      bv[q] = (double)(S.rb[0][bi] + S.rb[1][bi] + S.rb[2][bi] + S.rb[3][bi]);
    }
    const double ls = (bv[0] + bv[1]) + (bv[2] + bv[3]);
    const double incl = wave_incl_scan(ls, lane);
    const uint64_t bal = __ballot(above + incl >= target);
    __syncthreads();  // every wave has read the bins
    if (!bal) return false;
    const int lb = __ffsll((unsigned long long)bal) - 1;
    double a = above + readlane_d(incl - ls, lb);
    int bs = 4 * lb + 3;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const double vq = readlane_d(bv[q], lb);
      if (a + vq >= target) {
        bs = 4 * lb + q;
        break;
      }
      a += vq;
    }
    above = a;
    const uint32_t nhi = hi - ((uint32_t)bs << sh);
    const uint32_t nlo = nhi - lo > (1u << sh) ? nhi - (1u << sh) : lo;
    lo = nlo;
    hi = nhi;
    if (hi - lo == 1u) {
      *thr_key = lo << SH;
      return true;
    }
  }
  return false;
}

template <typename T, int CAP, int NW>
__device__ __forceinline__ void kept_draw(const Row<T, CAP>& R, Smem<CAP, NW>& S, const double (*colsum)[CAP], float m,
                                          float c, float thr, float u, int32_t* out);

// Fallback for top-k / top-p rows without a usable window: exact refinement,
// then the inverse CDF over {x >= thr} with fresh masses.  Every wave calls.
template <typename T, int CAP, int NW>
__device__ __forceinline__ void row_exact(const Row<T, CAP>& R, Smem<CAP, NW>& S, float m, float c, double Z, bool kon, int32_t k,
                          bool pon, float p, float Lm, float u, int32_t* out) {
  constexpr int EPV = QE<T>::EPV;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float thr = -INFINITY;
  uint32_t tk;
  if (kon) {
    if (refine(R, S, m, c, Lm, -INFINITY, true, (double)k, &tk)) thr = key_value(tk);
  }
  if (pon) {
    double ZK = Z;
    if (kon) {
      double acc = 0.0;
      each_chunk_mem(R, S, [&](float cb) { return cb >= thr; }, [&](int, const v4u& v, bool keep) {
        float x[EPV];
        QE<T>::unpack(v, x);
#pragma unroll
        for (int i = 0; i < EPV; ++i) acc += (keep && x[i] >= thr) ? (double)ex2c((x[i] - m) * c) : 0.0;
      });
      ZK = wg_sum(S, wave_sum(acc));
    }
    // members below 2^-40 of the maximum weigh < 2^-24 of Z altogether
    const float Lp = fmaxf(Lm, -40.0f);
    if (refine(R, S, m, c, Lp, thr, false, (double)p * ZK * kFix, &tk)) thr = fmaxf(thr, key_value(tk));
  }
  auto emass = [&](float x) { return x >= thr ? ex2c((x - m) * c) : 0.0f; };
  // kept mass per chunk column of this wave (columns no lane keeps stay 0)
  if (lane < CAP) S.colsum[wid][lane] = 0.0;
  each_chunk_mem(R, S, [&](float cb) { return cb >= thr; }, [&](int j, const v4u& v, bool keep) {
    float x[EPV];
    QE<T>::unpack(v, x);
    float e[EPV];
#pragma unroll
    for (int i = 0; i < EPV; ++i) e[i] = keep ? emass(x[i]) : 0.0f;
    const double C = wave_sum((double)tree_sum(e));
    if (lane == 0) S.colsum[wid][j] = C;
  });
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
  kept_draw(R, S, S.colsum, m, c, thr, u, out);
}

// Inverse CDF over the kept elements {x >= thr} given their mass per wave and
// chunk column (this wave's row of colsum complete and visible to it).
template <typename T, int CAP, int NW>
__device__ __forceinline__ void kept_draw(const Row<T, CAP>& R, Smem<CAP, NW>& S, const double (*colsum)[CAP], float m,
                                          float c, float thr, float u, int32_t* out) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  auto emass = [&](float x) { return x >= thr ? ex2c((x - m) * c) : 0.0f; };
  const double cs = lane < CAP ? colsum[wid][lane] : 0.0;
  const double cinc = wave_incl_scan(cs, lane);
  if (lane == 63) S.wz[wid] = cinc;
  __syncthreads();
  double Uw;
  const int ws = cross_wave<NW>([&](int q) { return S.wz[q]; }, u, &Uw);
  if (wid != ws) return;
  int js;
  {
    const uint64_t hit = __ballot(cs > 0.0 && cinc > Uw);
    const uint64_t pos = __ballot(cs > 0.0);
    js = hit ? __ffsll((unsigned long long)hit) - 1 : (pos ? 63 - __clzll((long long)pos) : 0);
  }
  const double colex = readlane_d(cinc - cs, js);
  finish_column<T, CAP>(R.load(js), ws, js, colex, Uw, emass, out);
}

// Exact top-p (no top-k) for rows without a usable window, in two passes over
// the row.  The threshold's value y* = (x* - m) c lies above
// ylo = log2((1 - p) Z / V): the elements below ylo weigh less than (1 - p) Z
// together.  Pass 1 builds kVB equal-width value bins over [ylo, 0], each
// holding its members' masses relative to the bin top in 2^-16 fixed point
// (integer sums, at most 2^-15 low relative to the exact bin mass); the
// cumulative from the top then brackets y* between bins b1 (cumulative
// >= p Z (1 - 2^-14)) and b2 (>= p Z (1 + 2^-20)): bins above b1 are kept,
// bins below b2 dropped, whatever the rounding.  Pass 2 sums the kept mass per
// chunk column and lists the bracket's elements (key, mass, position) in LDS,
// where key bins settle the exact threshold key; the kept candidates' masses
// then join their columns and the inverse CDF runs as in row_exact.  Returns
// false (uniformly, having written nothing) when the bracket cannot be formed
// or its candidates overflow cand_cap(NW) per wave.  Every wave calls.
template <typename T, int CAP, int NW>
__device__ __forceinline__ bool row_topp_fast(const Row<T, CAP>& R, Smem<CAP, NW>& S, float m, float c, double Z, float p,
                                              float Lm, float u, int64_t V, int32_t* out) {
  constexpr int EPV = QE<T>::EPV, SH = QE<T>::SH;
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const double target = (double)p * Z;
  float ylo = log2f((float)((1.0 - (double)p) * Z / (double)V)) - 0.01f;
  ylo = fmaxf(ylo, fmaxf(Lm, -40.0f));
  if (!(ylo < -0x1p-10f)) return false;
  const float s = (float)kVB / -ylo, w = -ylo / (float)kVB;
  auto vbin = [&](float y) { return min(kVB - 1, (int)(-y * s)); };
  // pass 1: value histograms
  for (int i = t; i < NW * (kVB + 1); i += (NW * kWave)) (&S.vh[0][0])[i] = 0u;
  __syncthreads();
  {
    uint32_t* vh = S.vh[wid];
    each_chunk_mem(R, S, [&](float cb) { return (cb - m) * c >= ylo; }, [&](int, const v4u& v, bool may) {
      float x[EPV];
      QE<T>::unpack(v, x);
#pragma unroll
      for (int i = 0; i < EPV; ++i) {
        const float y = (x[i] - m) * c;
        const int b = vbin(y);
        const bool ok = may && y >= ylo;
        const float er = ex2c(y + (float)b * w);
        atomicAdd(&vh[ok ? b : kVB], (uint32_t)(er * 65536.0f));
      }
    });
  }
  __syncthreads();
  // bracket (every wave alike): lane l holds bins 8l .. 8l+7
  int b1 = -1, b2 = -1;
  {
    double bm[8], ls = 0.0;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int b = 8 * lane + q;
      uint64_t hsum = 0;
#pragma unroll
      for (int q = 0; q < NW; ++q) hsum += S.vh[q][b];
      bm[q] = (double)hsum * (double)__builtin_amdgcn_exp2f(-((float)b * w)) * 0x1p-16;
      ls += bm[q];
    }
    const double incl = wave_incl_scan(ls, lane);
    const double t1 = target * (1.0 - 0x1p-14), t2 = target * (1.0 + 0x1p-20);
    const uint64_t bal1 = __ballot(incl >= t1), bal2 = __ballot(incl >= t2);
    if (bal1 && bal2) {
      const int l1 = __ffsll((unsigned long long)bal1) - 1, l2 = __ffsll((unsigned long long)bal2) - 1;
      double a1 = readlane_d(incl - ls, l1), a2 = readlane_d(incl - ls, l2);
      b1 = 8 * l1 + 7;
      b2 = 8 * l2 + 7;
#pragma unroll
      for (int q = 7; q >= 0; --q) {  // first bin of the lane reaching each target
        const double v1 = readlane_d(bm[q], l1), v2 = readlane_d(bm[q], l2);
        double c1 = a1, c2 = a2;
#pragma unroll
        for (int r = 0; r < q; ++r) {
          c1 += readlane_d(bm[r], l1);
          c2 += readlane_d(bm[r], l2);
        }
        if (c1 + v1 >= t1) b1 = 8 * l1 + q;
        if (c2 + v2 >= t2) b2 = 8 * l2 + q;
      }
    }
  }
  __syncthreads();  // every wave has read the histograms
  if (b1 < 0 || b2 < 0) return false;
  // pass 2: kept mass per column (bins above b1), candidates (bins b1 .. b2)
  int nc = 0;
  if (lane < CAP) S.ksum[wid][lane] = 0.0;
  each_chunk_mem(R, S, [&](float cb) { return (cb - m) * c >= ylo; }, [&](int j, const v4u& v, bool may) {
    float x[EPV], e[EPV];
    QE<T>::unpack(v, x);
#pragma unroll
    for (int i = 0; i < EPV; ++i) {
      const float y = (x[i] - m) * c;
      const int b = vbin(y);
      const bool ok = may && y >= ylo;
      const float ei = ex2c(y);
      e[i] = ok && b < b1 ? ei : 0.0f;
      const bool cd = ok && b >= b1 && b <= b2;
      const uint64_t bal = __ballot(cd);
      if (bal) {
        const int pos = nc + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (cd && pos < cand_cap(NW)) {
          S.ckey[wid][pos] = okey(x[i]) >> SH;
          S.cmass[wid][pos] = ei;
          S.cpos[wid][pos] = ((uint32_t)(j * kWave + lane) << 3) | (uint32_t)i;
        }
        nc += (int)__popcll(bal);
      }
    }
    const double C = wave_sum((double)tree_sum(e));
    if (lane == 0) S.ksum[wid][j] = C;
  });
  if (lane == 0) S.cnt[wid] = nc;
  __syncthreads();
  int cq[NW];
  bool ovf = false;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    cq[q] = uni(S.cnt[q]);
    ovf = ovf || cq[q] > cand_cap(NW);
  }
  if (ovf) return false;
  // mass above the bracket: every kept column sum so far
  double above = 0.0;
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    const double cs = lane < CAP ? S.ksum[q][lane] : 0.0;
    above += wave_sum(cs);
  }
  // key bracket of bins b1 .. b2: their y range widened by half a bin, mapped
  // back to x, then a few more keys for the rounding of that mapping
  constexpr uint32_t kSlack = SH ? 2u : 64u;
  uint32_t hi = (okey(fminf(m, m + (-(float)b1 * w + 0.5f * w) / c)) >> SH) + 1u + kSlack;
  hi = min(hi, (okey(m) >> SH) + 1u);
  const uint32_t kb = okey(m + (-(float)(b2 + 1) * w - 0.5f * w) / c) >> SH;
  uint32_t lo = kb > kSlack ? kb - kSlack : 0u;
  uint32_t thr_key = 0u;
  bool found = false;
  for (int level = 0; level < 6 && !found; ++level) {
    if (hi <= lo) return false;
    int sh = 0;
    while (((hi - lo - 1u) >> sh) >= (uint32_t)kRB) ++sh;
    if (t < kRB) S.kbin[t] = 0.0;
    __syncthreads();
    for (int q = t; q < NW * cand_cap(NW); q += (NW * kWave)) {
      const int cw = q / cand_cap(NW), ci = q - cw * cand_cap(NW);
      if (ci < S.cnt[cw]) {
        const uint32_t key = S.ckey[cw][ci];
        if (key >= lo && key < hi) atomicAdd(&S.kbin[(hi - 1u - key) >> sh], (double)S.cmass[cw][ci]);
      }
    }
    __syncthreads();
    double bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = S.kbin[4 * lane + q];
    const double ls = (bv[0] + bv[1]) + (bv[2] + bv[3]);
    const double incl = wave_incl_scan(ls, lane);
    const uint64_t bal = __ballot(above + incl >= target);
    __syncthreads();  // every wave has read the bins
    if (!bal) return false;
    const int lb = __ffsll((unsigned long long)bal) - 1;
    double a = above + readlane_d(incl - ls, lb);
    int bs = 4 * lb + 3;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const double vq = readlane_d(bv[q], lb);
      if (a + vq >= target) {
        bs = 4 * lb + q;
        break;
      }
      a += vq;
    }
    above = a;
    const uint32_t nhi = hi - ((uint32_t)bs << sh);
    const uint32_t nlo = nhi - lo > (1u << sh) ? nhi - (1u << sh) : lo;
    lo = nlo;
    hi = nhi;
    if (hi - lo == 1u) {
      thr_key = lo;
      found = true;
    }
  }
  if (!found) return false;
  // the kept candidates join their columns
  for (int q = t; q < NW * cand_cap(NW); q += (NW * kWave)) {
    const int cw = q / cand_cap(NW), ci = q - cw * cand_cap(NW);
    if (ci < S.cnt[cw] && S.ckey[cw][ci] >= thr_key)
      atomicAdd(&S.ksum[cw][(S.cpos[cw][ci] >> 3) / kWave], (double)S.cmass[cw][ci]);
  }
  __syncthreads();
  kept_draw(R, S, S.ksum, m, c, key_value(thr_key << SH), u, out);
  return true;
}

// Entry ranked r-th largest (1-based) among the window entries of one fine bin
// (flag `inb` per slot); keys are unique.  Wave 0 only.
__device__ __forceinline__ uint64_t bin_rank(const uint64_t (&key)[kHPL], const bool (&inb)[kHPL], int r) {
  uint64_t best = 0ull;
  bool done = false;
#pragma unroll 1
  for (int h = 0; h < kHPL && !done; ++h) {
    uint64_t b = __ballot(inb[h]);
    while (b && !done) {
      const int l = __ffsll((unsigned long long)b) - 1;
      b &= b - 1;
      const uint64_t kq = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(key[h] >> 32), l) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane((int)(key[h] & 0xffffffffu), l);
      int gt = 0;
#pragma unroll
      for (int g = 0; g < kHPL; ++g) gt += (inb[g] && key[g] > kq) ? 1 : 0;
      if (wave_sum_i(gt) == r - 1) {
        best = kq;
        done = true;
      }
    }
  }
  return best;
}

// Window finish by wave 0: lane l holds window positions kHPL*l .. kHPL*l + kHPL-1
// (nw <= kWin, index order).  Threshold from the fine histograms, exact inside
// the crossing bin; then the inverse CDF over the kept entries.
template <int CAP, int NW>
__device__ __forceinline__ void window_finish(Smem<CAP, NW>& S, int nw, const int (&cq)[NW], float m, float c, double Z, bool kon,
                              int32_t k, bool pon, float p, float u, int32_t* out) {
  const int lane = threadIdx.x & 63;
  int base[NW];
  base[0] = 0;
#pragma unroll
  for (int q = 1; q < NW; ++q) base[q] = base[q - 1] + cq[q - 1];
  bool in[kHPL];
  uint64_t key[kHPL];
  uint32_t kx[kHPL];
  float e[kHPL];
  int fb[kHPL];
#pragma unroll
  for (int h = 0; h < kHPL; ++h) {
    const int q = kHPL * lane + h;  // lane-major
    in[h] = q < nw;
    int w = 0, off = q;
#pragma unroll
    for (int g = 1; g < NW; ++g) {
      const bool ge = q >= base[g];
      w = ge ? g : w;
      off = ge ? q - base[g] : off;
    }
    key[h] = in[h] ? S.seg[w][off] : 0ull;
    kx[h] = (uint32_t)(key[h] >> 32);
    const float x = okey_inv(kx[h]);
    const float y = (x - m) * c;
    e[h] = in[h] ? ex2c(y) : 0.0f;
    fb[h] = in[h] ? min(kFB - 1, (int)(-8.0f * y)) : 0;
  }
  uint32_t thr = 0u;  // keep entries with value key >= thr
  double ZK = Z;
  // Cumulative fine-bin totals from the top: lane l owns bins 4l .. 4l+3.
  auto crossing = [&](const double (&bv)[4], double target, int* bin, double* above) -> bool {
    const double ls = (bv[0] + bv[1]) + (bv[2] + bv[3]);
    const double incl = wave_incl_scan(ls, lane);
    const uint64_t bal = __ballot(incl >= target);
    if (!bal) return false;
    const int lb = __ffsll((unsigned long long)bal) - 1;
    double a = readlane_d(incl - ls, lb);
    int bs = 4 * lb + 3;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const double vq = readlane_d(bv[q], lb);
      if (a + vq >= target) {
        bs = 4 * lb + q;
        break;
      }
      a += vq;
    }
    *bin = bs;
    *above = a;
    return true;
  };
  bool inK[kHPL];
#pragma unroll
  for (int h = 0; h < kHPL; ++h) inK[h] = in[h];
  if (kon) {
#pragma unroll
    for (int q = 0; q < 4; ++q) S.fcnt[4 * lane + q] = 0u;
    __builtin_amdgcn_s_waitcnt(0xc07f);
#pragma unroll
    for (int h = 0; h < kHPL; ++h)
      if (in[h]) atomicAdd(&S.fcnt[fb[h]], 1u);
    __builtin_amdgcn_s_waitcnt(0xc07f);
    double bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = (double)S.fcnt[4 * lane + q];
    int bk;
    double above;
    const int kk = k < nw ? k : nw;
    if (crossing(bv, (double)kk, &bk, &above)) {
      bool inb[kHPL];
#pragma unroll
      for (int h = 0; h < kHPL; ++h) inb[h] = in[h] && fb[h] == bk;
      const uint64_t kth = bin_rank(key, inb, kk - (int)above);
      thr = (uint32_t)(kth >> 32);
    }
    double zk = 0.0;
#pragma unroll
    for (int h = 0; h < kHPL; ++h) {
      inK[h] = in[h] && kx[h] >= thr;
      zk += inK[h] ? (double)e[h] : 0.0;
    }
    ZK = wave_sum(zk);
  }
  if (pon) {
    const double target = (double)p * ZK * kFix;
#pragma unroll
    for (int q = 0; q < 4; ++q) S.fmass[4 * lane + q] = 0ull;
    __builtin_amdgcn_s_waitcnt(0xc07f);
#pragma unroll
    for (int h = 0; h < kHPL; ++h)
      if (inK[h]) atomicAdd(&S.fmass[fb[h]], fix40(e[h]));
    __builtin_amdgcn_s_waitcnt(0xc07f);
    double bv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) bv[q] = (double)S.fmass[4 * lane + q];
    int bp;
    double above;
    if (crossing(bv, target, &bp, &above)) {
      // distinct value keys of the crossing bin, from the top, until the target is met
      bool rem[kHPL];
#pragma unroll
      for (int h = 0; h < kHPL; ++h) rem[h] = inK[h] && fb[h] == bp;
      double a = above;
      uint32_t t2 = thr;
#pragma unroll 1
      for (int it = 0; it < kWin; ++it) {
        uint32_t mk = 0u;
#pragma unroll
        for (int h = 0; h < kHPL; ++h) mk = max(mk, rem[h] ? kx[h] : 0u);
        const uint32_t vmax = (uint32_t)wave_max_i((int)(mk ^ 0x80000000u)) ^ 0x80000000u;
        if (vmax == 0u) break;
        double s = 0.0;
#pragma unroll
        for (int h = 0; h < kHPL; ++h) {
          const bool eq = rem[h] && kx[h] == vmax;
          s += eq ? (double)fix40(e[h]) : 0.0;
          rem[h] = rem[h] && !eq;
        }
        a += wave_sum(s);
        t2 = vmax;
        if (a >= target) break;
      }
      thr = max(thr, t2);
    }
  }
  // inverse CDF over the kept entries in index order (lane-major positions)
  float ek[kHPL];
  bool kept[kHPL];
  bool anyk = false;
  double ls = 0.0;
#pragma unroll
  for (int h = 0; h < kHPL; ++h) {
    kept[h] = inK[h] && kx[h] >= thr;
    ek[h] = kept[h] ? e[h] : 0.0f;
    ls += (double)ek[h];
    anyk = anyk || kept[h];
  }
  const double inc = wave_incl_scan(ls, lane);
  const double U = (double)uni(u) * readlane_d(inc, 63);
  int src;
  {
    const uint64_t hit = __ballot(ls > 0.0 && inc > U);
    const uint64_t pos = __ballot(ls > 0.0);
    const uint64_t any = __ballot(anyk);
    src = hit ? __ffsll((unsigned long long)hit) - 1
              : (pos ? 63 - __clzll((long long)pos) : (any ? 63 - __clzll((long long)any) : 0));
  }
  if (lane == src) {
    double a = inc - ls;
    int pick = -1, lastm = -1, lastk = 0;
#pragma unroll
    for (int h = 0; h < kHPL; ++h) {
      if (kept[h]) lastk = h;
      if (ek[h] > 0.0f) {
        lastm = h;
        a += (double)ek[h];
        if (pick < 0 && a > U) pick = h;
      }
    }
    if (pick < 0) pick = lastm >= 0 ? lastm : lastk;
    uint32_t lo = 0;
#pragma unroll
    for (int h = 0; h < kHPL; ++h)
      if (h == pick) lo = (uint32_t)(key[h] & 0xffffffffu);
    *out = (int32_t)(0xffffffffu - lo);
  }
}


__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) {
  return (uint32_t)wave_max_i((int)(v ^ 0x80000000u)) ^ 0x80000000u;
}

// Finish of a window of at most 64 entries by wave 0, one entry per lane in
// index order.  Each lane writes its (value key, 2^-40 fixed-point mass) to an
// LDS table, then reads the whole table (broadcast reads): the k-th largest
// value key is the largest key with at least k entries at or above it, the
// top-p threshold the largest kept key whose mass at or above it reaches p * Z
// (ties kept); the inverse CDF is one wave scan over the kept masses.
template <int CAP, int NW>
__device__ __forceinline__ void small_finish(Smem<CAP, NW>& S, int n, const int (&cq)[NW], float m, float c, double Z,
                                             bool kon, int32_t k, bool pon, float p, float u, int32_t* out) {
  const int lane = threadIdx.x & 63;
  int w = 0, off = lane, base = 0;
#pragma unroll
  for (int g = 1; g < NW; ++g) {
    base += cq[g - 1];
    const bool ge = lane >= base;
    w = ge ? g : w;
    off = ge ? lane - base : off;
  }
  const bool in = lane < n;
  const uint64_t key = in ? S.seg[w][off] : 0ull;
  const uint32_t kx = (uint32_t)(key >> 32);
  const uint32_t idx = 0xffffffffu - (uint32_t)(key & 0xffffffffu);
  const float e = in ? ex2c((okey_inv(kx) - m) * c) : 0.0f;
  const double f = (double)fix40(e);  // exact (< 2^40), and so are sums of 64 of them
  // the table: entry j = (value key, mass) at fmass[2 j], fmass[2 j + 1]
  unsigned long long* tab = S.fmass;
  if (in) {
    tab[2 * lane] = (unsigned long long)kx;
    tab[2 * lane + 1] = (unsigned long long)__double_as_longlong(f);
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's table writes are done
  __builtin_amdgcn_wave_barrier();
  uint32_t thr = 0u;  // keep entries with value key >= thr
  double ZK = Z;
  if (kon) {
    int cnt = 0;
#pragma unroll 8
    for (int j = 0; j < n; ++j) cnt += (uint32_t)tab[2 * j] >= kx ? 1 : 0;
    const int kk = k < n ? k : n;
    thr = wave_max_u(in && cnt >= kk ? kx : 0u);
    ZK = wave_sum(in && kx >= thr ? (double)e : 0.0);
  }
  if (pon) {
    const double target = (double)p * ZK * kFix;
    double A = 0.0;
#pragma unroll 8
    for (int j = 0; j < n; ++j) {
      const uint32_t kj = (uint32_t)tab[2 * j];
      const double fj = __longlong_as_double((long long)tab[2 * j + 1]);
      A += (kj >= kx && kj >= thr) ? fj : 0.0;
    }
    thr = max(thr, wave_max_u(in && kx >= thr && A >= target ? kx : 0u));
  }
  // inverse CDF in vocabulary (lane) order over the kept entries
  const bool kept = in && kx >= thr;
  const double ek = kept ? (double)e : 0.0;
  const double inc = wave_incl_scan(ek, lane);
  const double U = (double)uni(u) * readlane_d(inc, 63);
  const uint64_t hit = __ballot(ek > 0.0 && inc > U);
  int src;
  if (hit) {
    src = __ffsll((unsigned long long)hit) - 1;
  } else {  // rounding (u ~ 1): the last kept entry with mass, else the last kept
    const uint64_t pos = __ballot(ek > 0.0), any = __ballot(kept);
    src = pos ? 63 - __clzll((long long)pos) : (any ? 63 - __clzll((long long)any) : 0);
  }
  if (lane == src) *out = (int32_t)idx;
}

// Row statistics after the pass, published per wave before barrier 1.
template <typename T, int CAP, int NW>
__device__ __forceinline__ void publish(const LaneStats& s, float c, bool kon, bool pon, Smem<CAP, NW>& S) {
  constexpr int N = CAP * QE<T>::EPV;  // elements per lane
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const float wm = wave_maximum(s.ml);
  const double sl = s.S * (double)ex2c((s.ml - wm) * c);  // this lane's mass, wave frame
  const double wz = wave_sum(sl);
  if (kon || pon) {
    // two largest chunk maxima of each lane (distinct elements), wave frame
    uint32_t* h = S.wh[wid];
    const float y1 = (s.t1 - wm) * c, y2 = (s.t2 - wm) * c;
    if (y1 >= -32.0f) {
      const int b = min(kHB - 1, (int)(-4.0f * y1));
      if (kon) atomicAdd(&h[b], 1u);
      else atomicAdd(reinterpret_cast<float*>(&h[b]), ex2c(y1));
    }
    if (y2 >= -32.0f) {
      const int b = min(kHB - 1, (int)(-4.0f * y2));
      if (kon) atomicAdd(&h[b], 1u);
      else atomicAdd(reinterpret_cast<float*>(&h[b]), ex2c(y2));
    }
    if (!kon) {
      // The lane's other N - 2 elements weigh R: at any level L at or below
      // y_e = log2(R / (2 (N - 2))) those at or above L weigh at least
      // R - (N - 2) 2^L >= R / 2, so R / 2 counts at y_e.
      const float rest = (float)(sl - (double)ex2c(y1) - (double)ex2c(y2));
      const float ye = rest > 0.0f ? __log2f(rest * (0.5f / (float)(N - 2))) : -INFINITY;
      if (ye >= -32.0f) atomicAdd(reinterpret_cast<float*>(&h[min(kHB - 1, (int)(-4.0f * ye))]), 0.5f * rest);
    }
  }
  if (lane == 0) {
    S.wmax[wid] = wm;
    S.wz[wid] = wz;
  }
  if (kon || pon) S.lt[threadIdx.x] = v4u{__float_as_uint(s.t1), __float_as_uint(s.t2), (uint32_t)s.j1, 0u};
}

template <typename T, int CAP, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(kWavesPerEU)))
void quad_sample_kernel(SampleParams P) {
  constexpr int EPV = QE<T>::EPV;
  __shared__ Smem<CAP, NW> S;
  stamp(0);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int64_t nrows = P.B_out;
  if (P.n_rows_dev) nrows = min(nrows, (int64_t)uni(*P.n_rows_dev));
  const int64_t b = blockIdx.x;
  if (b >= nrows) return;
  const int64_t r = P.row_idx ? (int64_t)uni((int)P.row_idx[b]) : b;
  if (r < 0 || r >= P.B_src) {
    if (threadIdx.x == 0) P.out[b] = -1;
    return;
  }
  int32_t* out = &P.out[b];
  // Per-row arguments: issued before the row (the in-order load counter then
  // waits for them alone), through buffer resources that read 0 for an absent
  // array.
  const uint32_t ab = (uint32_t)min<int64_t>(P.B_src * 4, 0x7fffffff);
  auto arg = [&](const void* a) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(a), (short)0, a ? (int)ab : 0, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(r * 4), 0, 0);
  };
  const uint32_t aT = arg(P.temps), aU = arg(P.uniforms), aK = arg(P.top_k), aP = arg(P.top_p);
  Row<T, CAP> R;
  R.init(P.logits, r, P.ld, (uint32_t)P.V);
  R.fetch();
  stamp(7);
  const float Tr = __uint_as_float(uni(aT));
  const float u = __uint_as_float(uni(aU));
  const int32_t k = (int32_t)uni(aK);
  const float p = __uint_as_float(uni(aP) | (P.top_p ? 0u : 0x3f800000u));  // absent: 0 | bits of 1.0
  const bool tvalid = Tr > 0.0f && Tr < INFINITY;
  const float c = tvalid ? kLog2e / Tr : 1.0f;
  const bool kon = k >= 1 && (int64_t)k < P.V, pon = p < 1.0f;
  float m = -INFINITY;
  if (tvalid) {
    if (kon || pon) S.wh[wid][lane] = S.wh[wid][lane + kWave] = 0u;  // this wave's histogram (a wave's LDS ops stay in order)
    if (kon && threadIdx.x < kFB) S.fcnt[threadIdx.x] = 0u;   // the far-floor histogram (ordered by barrier 1)
    publish<T, CAP>(lane_pass<false>(R, c, S), c, kon, pon, S);
    stamp(1);
    __syncthreads();
    stamp(2);
    m = S.wmax[0];
#pragma unroll
    for (int q = 1; q < NW; ++q) m = fmx(m, S.wmax[q]);
    if (m != m) {
      // NaN present: NaN carries no mass; pass again ignoring it
      __syncthreads();
      if (kon || pon) S.wh[wid][lane] = S.wh[wid][lane + kWave] = 0u;
      publish<T, CAP>(lane_pass<true>(R, c, S), c, kon, pon, S);
      __syncthreads();
      m = S.wmax[0];
#pragma unroll
      for (int q = 1; q < NW; ++q) m = fmaxf(m, S.wmax[q]);
    }
  }
  if (!tvalid || !(m > -INFINITY) || !(m < INFINITY)) {
    row_argmax<true, NW>(R, S, out);
    stamp(5);
    stamp_path(kPathArgmax);
    return;
  }
  __builtin_amdgcn_s_setprio(2);
  m = uni(m);
  if (!kon && !pon) {
    walk_cols(R, S, m, c, u, [&](float x) { return ex2c((x - m) * c); }, out);
    stamp(5);
    stamp_path(kPathWalk);
    return;
  }
  // ---- top-k / top-p: floor from the merged histograms (row bin b gathers
  // wave q's bin b - s_q, s_q = ceil(4 * (its shift below the row maximum));
  // lane l holds row bins 2l and 2l + 1)
  int bstar;
  {
    int pc[2] = {0, 0};
    float pmf[2] = {0.0f, 0.0f};
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      const float wmq = uni(S.wmax[q]);
      const float D = (m - wmq) * c;
      const int sq = D < 32.0f ? (int)__builtin_ceilf(4.0f * D + 0x1p-8f) : kHB;
      const float fq = ex2c((wmq - m) * c);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int idx = 2 * lane + h - sq;
        const uint32_t v = S.wh[q][idx < 0 ? 0 : idx];
        if (idx >= 0) {
          if (kon) pc[h] += (int)v;
          else pmf[h] = __builtin_fmaf(__uint_as_float(v), fq, pmf[h]);
        }
      }
    }
    int lb = -1, hb = 1;
    if (kon) {
      const int inc = wave_incl_scan_i(pc[0] + pc[1], lane);
      const uint64_t bal = __ballot(inc >= k);
      if (bal) {
        lb = __ffsll((unsigned long long)bal) - 1;
        const int before = __builtin_amdgcn_readlane(inc - pc[0] - pc[1], lb);
        hb = before + __builtin_amdgcn_readlane(pc[0], lb) >= k ? 0 : 1;
      }
    } else {
      const double Zr = wave_total<NW>([&](int q) { return wave_mass(S, q, m, c); });
      if (threadIdx.x == 0) S.rz = Zr;  // the row normaliser, for the window finish
      const double tgt = (double)p * Zr * kBinMargin;
      const double inc = wave_incl_scan((double)pmf[0] + (double)pmf[1], lane);
      const uint64_t bal = __ballot(inc >= tgt);
      if (bal) {
        lb = __ffsll((unsigned long long)bal) - 1;
        const double before = readlane_d(inc - ((double)pmf[0] + (double)pmf[1]), lb);
        hb = before + (double)readlane_f(pmf[0], lb) >= tgt ? 0 : 1;
      }
    }
    bstar = lb < 0 ? -1 : 2 * lb + hb;
  }
  float Lm = -INFINITY;
  bool flr = bstar >= 0;
  if (flr) {
    Lm = -0.25f * (float)(bstar + 1) - 0x1p-8f;
  } else if (kon && k <= 2 * NW * kWave) {
    // The k-th largest element lies more than 32 binary orders below the
    // maximum (heavy tails, low temperature): bin the lanes' two largest pair
    // maxima (distinct elements) by their distance d = -y below it, bin 0 for
    // d <= 32, then 1/32 binary order per bin (the float bits of d from 32
    // on; bin kFB - 1 collects the rest).  The top bins holding k of them
    // bound the k-th largest element from below.
    const v4u lt = S.lt[threadIdx.x];
    auto far_bin = [&](uint32_t xb) {
      const float y = (__uint_as_float(xb) - m) * c;
      return y >= -32.0f ? 0 : min(kFB - 1, (int)(__float_as_uint(-y) >> 18) - kFarBin0 + 1);
    };
    atomicAdd(&S.fcnt[far_bin(lt.x)], 1u);
    atomicAdd(&S.fcnt[far_bin(lt.y)], 1u);
    __syncthreads();
    int pc[4], s4 = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pc[q] = (int)S.fcnt[4 * lane + q];
      s4 += pc[q];
    }
    const int inc = wave_incl_scan_i(s4, lane);
    const uint64_t bal = __ballot(inc >= k);
    if (bal) {
      const int lb = __ffsll((unsigned long long)bal) - 1;
      int a = __builtin_amdgcn_readlane(inc - s4, lb), bs = 4 * lb + 3;
#pragma unroll
      for (int q = 0; q < 3; ++q) {
        const int vq = __builtin_amdgcn_readlane(pc[q], lb);
        if (a + vq >= k) {
          bs = 4 * lb + q;
          break;
        }
        a += vq;
      }
      if (bs < kFB - 1) {  // bin bs holds d < the bottom of bin bs + 1
        flr = true;
        Lm = bs == 0 ? -32.0f : -__uint_as_float((uint32_t)(bs + kFarBin0) << 18);
      }
    }
  }
  stamp(3);
  if (flr) {
    // stage this wave's elements with y >= Lm, in index order (j, lane, element)
    uint64_t* seg = S.seg[wid];
    int run = 0;
    // this lane's chunks whose maximum bound reaches the floor (all bound
    // words read at once), and the columns where any lane has one
    // (a lane whose second-largest chunk-pair maximum is below the floor has
    // at most the two chunks of its largest pair there; only lanes with more
    // read their chunk bounds)
    const v4u lt = S.lt[threadIdx.x];
    const bool t2in = (__uint_as_float(lt.y) - m) * c >= Lm;
    uint32_t hm = 0u;
    if ((__uint_as_float(lt.x) - m) * c >= Lm) {  // the chunks of the largest pair whose bounds reach the floor
      const uint32_t w = S.cm[threadIdx.x][lt.z];
      hm = (((__uint_as_float(w << 16) - m) * c >= Lm ? 1u : 0u) |
            ((__uint_as_float(w & 0xffff0000u) - m) * c >= Lm ? 2u : 0u)) << (2 * lt.z);
    }
    if (__ballot(t2in) && t2in) {
      hm = 0u;
#pragma unroll
      for (int q = 0; q < CAP / 2; ++q) {
        const uint32_t w = S.cm[threadIdx.x][q];
        hm |= ((__uint_as_float(w << 16) - m) * c >= Lm ? 1u : 0u) << (2 * q);
        hm |= ((__uint_as_float(w & 0xffff0000u) - m) * c >= Lm ? 1u : 0u) << (2 * q + 1);
      }
    }
    const uint32_t cols = uni(wave_or(hm));
    // A: the lanes holding a candidate chunk list it in this wave's staging
    // area, over the occupied columns in order (a scalar loop over their bits;
    // slots in (column, lane) = index order)
    uint32_t* meta = S.smeta[wid];
    int ns = 0;
    for (uint32_t cb = cols; cb; cb &= cb - 1u) {
      const int j = __builtin_ctz(cb);
      const bool hj = (hm >> j) & 1u;
      const uint64_t bj = __ballot(hj);
      const int slot = ns + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bj >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)bj, 0u));
      if (hj && slot < stg_cap(NW)) meta[slot] = (uint32_t)(j * kWave + lane);
      ns += (int)__popcll(bj);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // this wave's staging writes are done
    __builtin_amdgcn_wave_barrier();
    // B: lane i gathers staged chunks i and i + 64 from memory (all rounds'
    // loads at once) and writes their elements above the floor (slot order is
    // index order)
    if (ns <= stg_cap(NW)) {
      constexpr int NR = (stg_cap(NW) + kWave - 1) / kWave;
      v4u gv[NR];
#pragma unroll
      for (int rr = 0; rr < NR; ++rr) {
        const int sl = rr * kWave + lane;
        const uint32_t mt = meta[sl < ns ? sl : 0];
        const uint32_t ci = ((uint32_t)wid * CAP + (mt >> 6)) * kWave + (mt & 63u);
        gv[rr] = sl < ns ? R.load_at(ci) : v4u{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int rr = 0; rr < NR; ++rr) {
        const int r0 = rr * kWave;
        if (r0 >= ns) break;
        const bool act = r0 + lane < ns;
        const v4u v = gv[rr];
        const uint32_t mt = meta[act ? r0 + lane : 0];
        const uint32_t ci = ((uint32_t)wid * CAP + (mt >> 6)) * kWave + (mt & 63u);  // chunk index in the row
        float x[EPV];
        QE<T>::unpack(v, x);
        int cnt = 0;
#pragma unroll
        for (int i = 0; i < EPV; ++i) cnt += (act && (x[i] - m) * c >= Lm) ? 1 : 0;
        const int incl = wave_incl_scan_i(cnt, lane);
        int pos = run + incl - cnt;
#pragma unroll
        for (int i = 0; i < EPV; ++i) {
          if (act && (x[i] - m) * c >= Lm) {
            if (pos < seg_cap(NW)) seg[pos] = ((uint64_t)okey(x[i]) << 32) | (uint64_t)(0xffffffffu - (ci * EPV + i));
            ++pos;
          }
        }
        run += __builtin_amdgcn_readlane(incl, 63);
      }
    } else {
      run = seg_cap(NW) + 1;  // too many candidate chunks: the exact path decides
    }
    if (lane == 0) S.cnt[wid] = run;
  }
  __syncthreads();
  stamp(4);
  if (flr) {
    int cq[NW], nw = 0;
    bool ovf = false;
#pragma unroll
    for (int q = 0; q < NW; ++q) {
      cq[q] = uni(S.cnt[q]);
      nw += cq[q];
      ovf = ovf || cq[q] > seg_cap(NW);
    }
    if (!ovf && nw >= 1 && nw <= kWave) {
      if (wid == 0) small_finish(S, nw, cq, m, c, (!kon && pon) ? S.rz : 0.0, kon, k, pon, p, u, out);
      stamp(5);
      stamp_path(kPathSmall);
      return;
    }
    if (!ovf && nw <= kWin) {
      if (wid == 0) window_finish(S, nw, cq, m, c, (!kon && pon) ? S.rz : 0.0, kon, k, pon, p, u, out);
      stamp(5);
      stamp_path(kPathWindow);
      return;
    }
  }
  const double Zr = wave_total<NW>([&](int q) { return wave_mass(S, q, m, c); });
  if (!kon && row_topp_fast(R, S, m, c, Zr, p, Lm, u, P.V, out)) {
    stamp(5);
    stamp_path(kPathTopp);
    return;
  }
  row_exact(R, S, m, c, Zr, kon, k, pon, p, Lm, u, out);
  stamp(5);
  stamp_path(kPathExact);
}

// All-greedy batch: torch.argmax per row.
template <typename T, int CAP, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(kWavesPerEU)))
void quad_greedy_kernel(SampleParams P) {
  __shared__ GSmem<NW> S;
  int64_t nrows = P.B_out;
  if (P.n_rows_dev) nrows = min(nrows, (int64_t)uni(*P.n_rows_dev));
  const int64_t b = blockIdx.x;
  if (b >= nrows) return;
  const int64_t r = P.row_idx ? (int64_t)uni((int)P.row_idx[b]) : b;
  if (r < 0 || r >= P.B_src) {
    if (threadIdx.x == 0) P.out[b] = -1;
    return;
  }
  Row<T, CAP> R;
  R.init(P.logits, r, P.ld, (uint32_t)P.V);
  R.fetch();
  row_argmax<false, NW>(R, S, &P.out[b]);
}

template <typename T, int CAP, int NW>
static void launch(const SampleParams& P, bool greedy, hipStream_t st) {
  if (greedy)
    hipLaunchKernelGGL((quad_greedy_kernel<T, CAP, NW>), dim3((unsigned)P.B_out), dim3(NW * kWave), 0, st, P);
  else
    hipLaunchKernelGGL((quad_sample_kernel<T, CAP, NW>), dim3((unsigned)P.B_out), dim3(NW * kWave), 0, st, P);
}

// Row shapes this file serves: 4 waves x 32 or 24 chunks per lane (four rows
// per compute unit), and fp32 rows of 65536 as 8 waves x 32 chunks (two rows
// per compute unit).  Batches with no more rows than compute units are left to
// sample.hip's sixteen-wave rows (one row per compute unit, all of its SIMDs
// busy), which finish such batches sooner.
template <typename T>
static bool launch_dtype(const SampleParams& P, bool greedy, hipStream_t st) {
  constexpr int EPV = QE<T>::EPV;
  if (P.V % EPV != 0) return false;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (P.B_out <= (int64_t)cus) return false;
  const int64_t NV = P.V / EPV;
  if (NV == 4 * kWave * 32) launch<T, 32, 4>(P, greedy, st);
  else if (NV == 4 * kWave * 24) launch<T, 24, 4>(P, greedy, st);
  else if constexpr (sizeof(T) == 4) {
    if (NV == 8 * kWave * 32) launch<T, 32, 8>(P, greedy, st);
    else return false;
  } else {
    return false;
  }
  return true;
}

}  // namespace quad

#ifdef LSG_PHASE_STAMPS
// Copy of the phase stamps (profiling build only): kStampRows x kStampSlots
// 64-bit words.
extern "C" int lsg_phase_stamps_read(void* dst, size_t bytes) {
  const size_t n = sizeof(quad::g_phase_stamps);
  return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(quad::g_phase_stamps), bytes < n ? bytes : n, 0,
                                  hipMemcpyDeviceToHost);
}
#endif

bool quad_sample_launch(const SampleParams& P, int dtype, bool greedy, bool vec, hipStream_t st) {
  if (!vec) return false;
  if (dtype == kF32) return quad::launch_dtype<float>(P, greedy, st);
  if (dtype == kBF16) return quad::launch_dtype<bf16_t>(P, greedy, st);
  if (dtype == kF16) return quad::launch_dtype<f16_t>(P, greedy, st);
  return false;
}

}  // namespace lsg
