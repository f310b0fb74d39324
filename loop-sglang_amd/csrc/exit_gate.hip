// Continuous Depth Batching exit gates with on-device stable exit compaction.
//
// Replaces, for the decode token path of Loop-SGLang:
//   OuroModel.exit_signal        python/loopsgl/models/looped/ouro.py:142-155
//     gate linear                layers/linear.py:32-33 (F.linear, output in model dtype)
//     cumulative_exit_probability models/looped/exit_gates.py:6-15
//   HuginnModel.exit_signal      models/looped/huginn.py:184-194, exit_gates.py:18-24
//   the host stable filter       managers/cdb_scheduler.py:215-228 (exit_idx / keep_idx)
//   exit-state pool traffic      model_executor/cdb_model_runner.py:94-109 (slots)
//
// One launch: TPR threads reduce one row's gate dot product (fp32 accumulate),
// the row leader applies the gate arithmetic, and the last workgroup to finish
// (arrival counter in the workspace) performs the stable compaction from a
// per-row bitmask.  The workspace is left zero-filled for the next call.
//
// Compiled with -ffp-contract=off: F' = F + (1 - F) * lambda is three separately
// rounded fp32 operations, as torch evaluates it eagerly (one kernel per op).
#include "lsg_capi_internal.h"
#include "lsg_common.h"

namespace lsg {

constexpr int kGateThreads = 256;

struct GateParams {
  const void* h;
  const void* hp;  // Huginn: previous state
  int64_t B, H, ldh, ldp;
  const void* w;
  const void* bias;
  const float* F_prev;
  float* F_next;
  const int32_t* slots;
  const int32_t* loop_step;
  int32_t loop_step_scalar;
  float tau, eps;
  int32_t min_loop_steps, lookahead, max_depth;
  uint8_t* mask;
  float* aux_out;  // z (Ouro) or ratio (Huginn)
  int32_t* exit_idx;
  int32_t* keep_idx;
  int32_t* n_exit;
  uint32_t* counter;  // workspace: arrival counter
  uint32_t* bits;     // workspace: one bit per row
};

template <typename T>
__device__ __forceinline__ float round_to(float v);
template <>
__device__ __forceinline__ float round_to<float>(float v) {
  return v;
}
template <>
__device__ __forceinline__ float round_to<bf16_t>(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7fffffffu) > 0x7f800000u) return __uint_as_float((b | 0x00400000u) & 0xffff0000u);
  b += 0x7fffu + ((b >> 16) & 1u);  // round to nearest even
  return __uint_as_float(b & 0xffff0000u);
}
template <>
__device__ __forceinline__ float round_to<f16_t>(float v) {
  return (float)(_Float16)v;  // round to nearest even
}

template <typename T>
__device__ __forceinline__ float load_one(const void* p) {
  uint4 v = Elem<T>::pad();
  Elem<T>::set(v, 0, Elem<T>::load_bits(reinterpret_cast<const T*>(p)));
  return Elem<T>::get(v, 0);
}

// lambda = float32(sigmoid(z)) from a float64 evaluation (rounded once), then
// F' = F + (1 - F) * lambda in three rounded float32 steps (exit_gates.py:13-15).
__device__ __forceinline__ float gate_update(float F, float z) {
  const float lam = (float)(1.0 / (1.0 + exp(-(double)z)));
  const float t1 = 1.0f - F;
  const float t2 = t1 * lam;
  return F + t2;
}

// Sum of one value per thread over the TPR threads of a row (fixed order).
template <int TPR>
__device__ __forceinline__ float row_sum(float v, float* s_part) {
  // wave butterfly (identical in every lane), then waves of the row in order
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  if constexpr (TPR > kWave) {
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) s_part[w] = v;
    __syncthreads();
    const int w0 = (threadIdx.x / TPR) * (TPR / kWave);
    float s = s_part[w0];
#pragma unroll
    for (int i = 1; i < TPR / kWave; ++i) s += s_part[w0 + i];
    __syncthreads();
    return s;
  } else {
    return v;
  }
}

// Stable compaction of the row bitmask by the last workgroup (256 threads).
__device__ void compact_rows(const GateParams& P) {
  __shared__ int s_wave[kGateThreads / kWave];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int64_t nwords = (P.B + 31) / 32;
  int64_t base = 0;
  for (int64_t w0 = 0; w0 < nwords; w0 += kGateThreads) {
    const int64_t wi = w0 + t;
    uint32_t m = 0;
    int nvalid = 0;
    if (wi < nwords) {
      m = atomicExch(&P.bits[wi], 0u);  // read and clear
      nvalid = (int)min<int64_t>(32, P.B - wi * 32);
      if (nvalid < 32) m &= (1u << nvalid) - 1u;
    }
    const int ce = __popc(m);
    const int incl = wave_incl_scan_i(ce, lane);
    if (lane == 63) s_wave[w] = incl;
    __syncthreads();
    int wbase = 0, tile = 0;
#pragma unroll
    for (int i = 0; i < kGateThreads / kWave; ++i) {
      if (i < w) wbase += s_wave[i];
      tile += s_wave[i];
    }
    __syncthreads();
    int64_t pe = base + wbase + (incl - ce);
    int64_t pk = wi * 32 - pe;
    for (int bit = 0; bit < nvalid; ++bit) {
      const int32_t row = (int32_t)(wi * 32 + bit);
      if ((m >> bit) & 1u) {
        if (P.exit_idx) P.exit_idx[pe] = row;
        ++pe;
      } else {
        if (P.keep_idx) P.keep_idx[pk] = row;
        ++pk;
      }
    }
    base += tile;
  }
  if (t == 0) {
    if (P.n_exit) *P.n_exit = (int32_t)base;
    atomicExch(P.counter, 0u);
  }
}

// Publication and arrival counting, once per workgroup: the row leaders set
// their exit bits in LDS (bits [0, RPB) of s_bits, rows row0 .. row0+RPB-1 in
// one 32-bit word since RPB divides 32); thread 0 ORs them into the workspace
// bitmask, fences (orders the bits before its arrival) and counts the arrival.
// The last workgroup to arrive compacts.  No other cross-workgroup data: the
// per-row outputs are read by later kernels only.
template <int RPB>
__device__ __forceinline__ void finish_block(const GateParams& P, const uint32_t* s_bits) {
  if (!P.counter) return;
  static_assert(32 % RPB == 0, "a workgroup's rows share one bitmask word");
  __shared__ int s_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t row0 = (int64_t)blockIdx.x * RPB;
    const uint32_t b = *s_bits;
    if (b) atomicOr(&P.bits[row0 >> 5], b << (row0 & 31));
    __threadfence();
    const uint32_t prev = atomicAdd(P.counter, 1u);
    s_last = prev == gridDim.x - 1;
  }
  __syncthreads();
  if (s_last) {
    __threadfence();
    compact_rows(P);
  }
}

// f(a_i, b_i) over this thread's elements of two rows: chunks c = tr,
// tr + TPR, ... in order, elements in order (the sequence of a plain loop).
// Full 16-byte chunks load four pairs at a time, so their loads are in flight
// together; the partial last chunk is bounds-checked.
template <typename T, int TPR, bool VEC, class F>
__device__ __forceinline__ void row_pairs(const T* a, const T* b, int64_t H, int tr, F&& f) {
  constexpr int EPV = Elem<T>::EPV, U = 4;
  const int64_t nfull = VEC ? H / EPV : 0;
  int64_t c = tr;
  for (; c + (U - 1) * TPR < nfull; c += U * TPR) {
    uint4 av[U], bv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      av[u] = *reinterpret_cast<const uint4*>(a + (c + u * TPR) * EPV);
      bv[u] = *reinterpret_cast<const uint4*>(b + (c + u * TPR) * EPV);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < EPV; ++i) f(Elem<T>::get(av[u], i), Elem<T>::get(bv[u], i));
  }
  const int64_t nch = (H + EPV - 1) / EPV;
  for (; c < nch; c += TPR) {
    const uint4 av = load_chunk<T, VEC>(a, c, H), bv = load_chunk<T, VEC>(b, c, H);
#pragma unroll
    for (int i = 0; i < EPV; ++i)
      if (c * EPV + i < H) f(Elem<T>::get(av, i), Elem<T>::get(bv, i));
  }
}

template <typename T, int TPR, bool VEC>
__global__ __launch_bounds__(kGateThreads) void ouro_gate_kernel(GateParams P) {
  constexpr int EPV = Elem<T>::EPV, RPB = kGateThreads / TPR;
  __shared__ float s_part[kGateThreads / kWave];
  __shared__ uint32_t s_bits;
  if (threadIdx.x == 0) s_bits = 0u;
  __syncthreads();  // cleared before any row leader sets its bit
  const int tr = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int64_t nch = (P.H + EPV - 1) / EPV;
  float acc = 0.0f;
  if (row < P.B) {
    const T* hrow = reinterpret_cast<const T*>(P.h) + row * P.ldh;
    const T* wrow = reinterpret_cast<const T*>(P.w);
    row_pairs<T, TPR, VEC>(hrow, wrow, P.H, tr, [&](float x, float y) { acc = fmaf(x, y, acc); });
  }
  acc = row_sum<TPR>(acc, s_part);
  if (row < P.B && tr == 0) {
    const float bv = P.bias ? load_one<T>(P.bias) : 0.0f;
    const float z = round_to<T>(acc + bv);
    const int64_t s = P.slots ? (int64_t)P.slots[row] : row;
    const float F = P.F_prev ? P.F_prev[s] : 0.0f;
    const float Fn = gate_update(F, z);
    const int32_t ls = P.loop_step ? P.loop_step[row] : P.loop_step_scalar;
    int m = (Fn >= P.tau) && (ls + 1 + P.lookahead >= P.min_loop_steps);
    if (P.max_depth > 0 && ls + 1 >= P.max_depth) m = 1;
    P.F_next[s] = Fn;
    P.mask[row] = (uint8_t)m;
    if (P.aux_out) P.aux_out[row] = z;
    if (m) atomicOr(&s_bits, 1u << (threadIdx.x / TPR));
  }
  finish_block<RPB>(P, &s_bits);
}

template <typename T, int TPR, bool VEC>
__global__ __launch_bounds__(kGateThreads) void rel_change_kernel(GateParams P) {
  constexpr int EPV = Elem<T>::EPV, RPB = kGateThreads / TPR;
  __shared__ float s_part[kGateThreads / kWave];
  __shared__ uint32_t s_bits;
  if (threadIdx.x == 0) s_bits = 0u;
  __syncthreads();  // cleared before any row leader sets its bit
  const int tr = threadIdx.x % TPR;
  const int64_t row = (int64_t)blockIdx.x * RPB + threadIdx.x / TPR;
  const int64_t nch = (P.H + EPV - 1) / EPV;
  float d2 = 0.0f, n2 = 0.0f;
  if (row < P.B) {
    const T* a = reinterpret_cast<const T*>(P.h) + row * P.ldh;
    const T* bp = reinterpret_cast<const T*>(P.hp) + row * P.ldp;
    row_pairs<T, TPR, VEC>(a, bp, P.H, tr, [&](float x, float y) {
      const float dd = x - y;
      d2 = fmaf(dd, dd, d2);
      n2 = fmaf(x, x, n2);
    });
  }
  d2 = row_sum<TPR>(d2, s_part);
  n2 = row_sum<TPR>(n2, s_part);
  if (row < P.B && tr == 0) {
    const float ratio = sqrtf(d2) / fmaxf(sqrtf(n2), P.eps);
    const int m = ratio < P.tau;
    P.mask[row] = (uint8_t)m;
    if (P.aux_out) P.aux_out[row] = ratio;
    if (m) atomicOr(&s_bits, 1u << (threadIdx.x / TPR));
  }
  finish_block<RPB>(P, &s_bits);
}

template <typename T>
__global__ void cum_exit_kernel(const void* z, const float* F_prev, float* F_next, int64_t B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) F_next[i] = gate_update(F_prev[i], load_one<T>(reinterpret_cast<const T*>(z) + i));
}

enum class GateKind { kOuro, kRelChange };

template <typename T, int TPR, bool VEC>
static void launch_kind(GateKind kind, const GateParams& P, hipStream_t st) {
  constexpr int RPB = kGateThreads / TPR;
  const dim3 grid((unsigned)(P.B > 0 ? (P.B + RPB - 1) / RPB : 1)), block(kGateThreads);
  if (kind == GateKind::kOuro) hipLaunchKernelGGL((ouro_gate_kernel<T, TPR, VEC>), grid, block, 0, st, P);
  else hipLaunchKernelGGL((rel_change_kernel<T, TPR, VEC>), grid, block, 0, st, P);
}

template <typename T>
static void launch_rows(GateKind kind, const GateParams& P, bool vec, hipStream_t st) {
  constexpr int EPV = Elem<T>::EPV;
  const int64_t nch = (P.H + EPV - 1) / EPV;
  // one wave per row, four rows per workgroup: a row's loads are issued
  // back to back (nch / 64 chunks per thread), and publication costs one
  // fence and one counter atomic per four rows
  (void)nch;
  vec ? launch_kind<T, kWave, true>(kind, P, st) : launch_kind<T, kWave, false>(kind, P, st);
}

static int dispatch_rows(GateKind kind, int dtype, const GateParams& P, bool vec, hipStream_t st) {
  if (dtype == kF32) launch_rows<float>(kind, P, vec, st);
  else if (dtype == kBF16) launch_rows<bf16_t>(kind, P, vec, st);
  else if (dtype == kF16) launch_rows<f16_t>(kind, P, vec, st);
  else return set_error(LSG_ERR_ARG, "unknown dtype %d", dtype);
  return LSG_OK;
}

static int setup_workspace(GateParams& P, int op, void* ws, size_t ws_bytes, const char* fn) {
  const bool want = P.exit_idx || P.keep_idx || P.n_exit;
  if (!want) {
    P.counter = nullptr;
    P.bits = nullptr;
    return LSG_OK;
  }
  const size_t need = lsg_workspace_bytes(op, P.B);
  if (!ws || ws_bytes < need || ((uintptr_t)ws % 16) != 0)
    return set_error(LSG_ERR_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) needed, got %zu",
                     fn, need, ws ? ws_bytes : (size_t)0);
  P.counter = reinterpret_cast<uint32_t*>(ws);
  P.bits = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(ws) + 256);
  return LSG_OK;
}

static bool rows_vec(const void* base, int64_t ld, int dtype) {
  const int64_t es = dtype == kF32 ? 4 : 2;
  return ((uintptr_t)base % 16 == 0) && ((ld * es) % 16 == 0);
}

}  // namespace lsg

using namespace lsg;

extern "C" int lsg_exit_gate(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                             const void* w, const void* bias, const float* F_prev, float* F_next,
                             const int32_t* slots, const int32_t* loop_step,
                             int32_t loop_step_scalar, float tau, int32_t min_loop_steps,
                             int32_t lookahead, int32_t max_depth, uint8_t* mask,
                             int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit, float* z_out,
                             void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if ((B > 0 && (!h || !w || !F_next || !mask)) || B < 0 || H < 1 || (B > 0 && ldh < H))
    return set_error(LSG_ERR_ARG, "lsg_exit_gate: bad arguments (B=%lld H=%lld ldh=%lld)",
                     (long long)B, (long long)H, (long long)ldh);
  if (B > 0x7fffffffLL) return set_error(LSG_ERR_ARG, "lsg_exit_gate: B exceeds int32 rows");
  GateParams P{};
  P.h = h;
  P.B = B;
  P.H = H;
  P.ldh = ldh;
  P.w = w;
  P.bias = bias;
  P.F_prev = F_prev;
  P.F_next = F_next;
  P.slots = slots;
  P.loop_step = loop_step;
  P.loop_step_scalar = loop_step_scalar;
  P.tau = tau;
  P.min_loop_steps = min_loop_steps;
  P.lookahead = lookahead ? 1 : 0;
  P.max_depth = max_depth;
  P.mask = mask;
  P.aux_out = z_out;
  P.exit_idx = exit_idx;
  P.keep_idx = keep_idx;
  P.n_exit = n_exit;
  int rc = setup_workspace(P, LSG_OP_EXIT_GATE, workspace, workspace_bytes, "lsg_exit_gate");
  if (rc != LSG_OK) return rc;
  if (B == 0 && !P.counter) return LSG_OK;
  const bool vec = rows_vec(h, ldh, dtype) && rows_vec(w, H, dtype);
  rc = dispatch_rows(GateKind::kOuro, dtype, P, vec, reinterpret_cast<hipStream_t>(stream));
  if (rc != LSG_OK) return rc;
  return check_launch("lsg_exit_gate");
}

extern "C" int lsg_relative_state_change(const void* h, const void* h_prev, int dtype, int64_t B,
                                         int64_t H, int64_t ldh, int64_t ldp, float tau,
                                         float eps, float* ratio, uint8_t* mask,
                                         int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if ((B > 0 && (!h || !h_prev || !mask)) || B < 0 || H < 1 || (B > 0 && (ldh < H || ldp < H)))
    return set_error(LSG_ERR_ARG, "lsg_relative_state_change: bad arguments");
  if (B > 0x7fffffffLL) return set_error(LSG_ERR_ARG, "lsg_relative_state_change: B too large");
  GateParams P{};
  P.h = h;
  P.hp = h_prev;
  P.B = B;
  P.H = H;
  P.ldh = ldh;
  P.ldp = ldp;
  P.tau = tau;
  P.eps = eps;
  P.mask = mask;
  P.aux_out = ratio;
  P.exit_idx = exit_idx;
  P.keep_idx = keep_idx;
  P.n_exit = n_exit;
  int rc = setup_workspace(P, LSG_OP_REL_CHANGE, workspace, workspace_bytes,
                           "lsg_relative_state_change");
  if (rc != LSG_OK) return rc;
  if (B == 0 && !P.counter) return LSG_OK;
  const bool vec = rows_vec(h, ldh, dtype) && rows_vec(h_prev, ldp, dtype);
  rc = dispatch_rows(GateKind::kRelChange, dtype, P, vec, reinterpret_cast<hipStream_t>(stream));
  if (rc != LSG_OK) return rc;
  return check_launch("lsg_relative_state_change");
}

extern "C" int lsg_cumulative_exit_probability(const void* z, int dtype, const float* F_prev,
                                               float* F_next, int64_t B, void* stream) {
  clear_error();
  if (B < 0 || (B > 0 && (!z || !F_prev || !F_next)))
    return set_error(LSG_ERR_ARG, "lsg_cumulative_exit_probability: bad arguments");
  if (B == 0) return LSG_OK;
  const dim3 grid((unsigned)((B + 255) / 256)), block(256);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dtype == kF32) hipLaunchKernelGGL(cum_exit_kernel<float>, grid, block, 0, st, z, F_prev, F_next, B);
  else if (dtype == kBF16) hipLaunchKernelGGL(cum_exit_kernel<bf16_t>, grid, block, 0, st, z, F_prev, F_next, B);
  else if (dtype == kF16) hipLaunchKernelGGL(cum_exit_kernel<f16_t>, grid, block, 0, st, z, F_prev, F_next, B);
  else return set_error(LSG_ERR_ARG, "lsg_cumulative_exit_probability: unknown dtype %d", dtype);
  return check_launch("lsg_cumulative_exit_probability");
}
