// Continuous Depth Batching exit gates with on-device exit routing and stable
// exit compaction.
//
// Replaces, for the decode token path of Loop-SGLang:
//   OuroModel.exit_signal        python/loopsgl/models/looped/ouro.py:142-155
//     gate linear                layers/linear.py:32-33 (F.linear, output in model dtype)
//     cumulative_exit_probability models/looped/exit_gates.py:6-15
//   HuginnModel.exit_signal      models/looped/huginn.py:184-194, exit_gates.py:18-24
//   CDBScheduler._consume_gate   managers/cdb_scheduler.py:189-229 (routing: lookahead
//                                delay, replay depths, depth cap; the stable exit/keep filter)
//   exit-state pool traffic      model_executor/cdb_model_runner.py:94-109 (slots)
//
// One launch: one wave reduces one row's gate dot product (fp32 accumulate),
// the row leader applies the gate arithmetic and the routing rule, and the
// workgroups' routed-row counts are prefix-summed by a decoupled look-back:
// each workgroup publishes its count (tagged with the call's serial number),
// sums its predecessors' counts from their published words and writes its own
// rows' exit/keep positions.  No workgroup waits for a later one, nothing is
// fenced, and the workspace never has to be cleared: the serial number kept in
// it tells this call's words from older ones.
//
// Compiled with -ffp-contract=off: lambda = 1 / (1 + exp(-z)) and
// F' = F + (1 - F) * lambda are separately rounded fp32 operations, as torch
// evaluates them (one rounding per op).
#include <mutex>

#include "lsg_capi_internal.h"
#include "lsg_common.h"

namespace lsg {

constexpr int kGateThreads = 512;
constexpr int kGateRows = kGateThreads / kWave;  // one wave per row
// Published word of a workgroup: serial << 32 | state << 30 | count.
constexpr unsigned long long kStateAgg = 1ull << 30;  // count of its own rows
constexpr unsigned long long kStateInc = 2ull << 30;  // count of all rows up to its own
constexpr uint32_t kCountMask = (1u << 30) - 1u;
constexpr uint32_t kSpinLimit = 1u << 22;  // polls before a look-back gives up (never reached)

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
  int32_t direct;       // route on this step's own request (no pending pool)
  int32_t cap_in_mask;  // the depth cap is part of mask (lsg_exit_gate)
  long long* pending;   // per state slot: (serial + 1) << 32 | request, or 0
  const int32_t* replay;
  uint8_t* mask;
  uint8_t* route;
  float* aux_out;  // z (Ouro) or ratio (Huginn)
  int32_t* exit_idx;
  int32_t* keep_idx;
  int32_t* n_exit;
  uint32_t* serial;             // workspace: call serial number, error flag
  unsigned long long* tiles;    // workspace: one published word per workgroup
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

// lambda = 1 / (1 + exp(-z)) in float32, each operation rounded once, with
// exp(-z) correctly rounded to float32 (a float64 exp rounded once; for every
// bf16 and fp16 z the float64 value is far enough from a float32 rounding
// boundary for that rounding to be the correct one); then
// F' = F + (1 - F) * lambda in three rounded float32 steps.  torch evaluates
// sigmoid(float(z)) as 1 / (1 + exp(-z)) in float32 (exit_gates.py:13-15).
__device__ __forceinline__ float sigmoid_f32(float z) {
  const float e = (float)exp(-(double)z);
  const float d = 1.0f + e;
  return 1.0f / d;
}

__device__ __forceinline__ float gate_update(float F, float z) {
  const float lam = sigmoid_f32(z);
  const float t1 = 1.0f - F;
  const float t2 = t1 * lam;
  return F + t2;
}

__device__ __forceinline__ float wave_total(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);  // identical in every lane
  return v;
}

__device__ __forceinline__ unsigned long long load_word(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_word(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Number of routed rows in workgroups [0, b) from their published words (one
// wave, result uniform).  Lane i polls workgroup hi - i; a window is usable
// once every lane up to the nearest inclusive word has a word of this call;
// workgroups before 0 count as an inclusive zero.  The published words are
// whole 64-bit values, so a poll sees either an old word or this call's.
__device__ int64_t look_back(const GateParams& P, int64_t b, uint32_t serial, bool* ok) {
  const int lane = threadIdx.x & 63;
  int64_t excl = 0;
  int64_t hi = b - 1;
  uint32_t polls = 0;
  while (hi >= 0) {
    const int64_t idx = hi - lane;
    const unsigned long long v =
        idx >= 0 ? load_word(P.tiles + idx) : (((unsigned long long)serial << 32) | kStateInc);
    const bool cur = (uint32_t)(v >> 32) == serial && (v & (kStateAgg | kStateInc)) != 0;
    const bool inc = cur && (v & kStateInc) != 0;
    const unsigned long long incm = __ballot(inc), curm = __ballot(cur);
    const int stop = incm ? __builtin_ctzll(incm) : 63;
    const unsigned long long need = (2ull << stop) - 1ull;
    if ((curm & need) != need) {
      if (++polls > kSpinLimit) {
        *ok = false;
        return 0;
      }
      __builtin_amdgcn_s_sleep(1);
      continue;
    }
    const int c = lane <= stop ? (int)(v & kCountMask) : 0;
    excl += wave_sum_i(c);
    if (incm) break;
    hi -= 64;
  }
  return excl;
}

// Routing and compaction, once per workgroup.  s_route[i] is 1 when row
// row0 + i is routed (rows past B are 0).  Workgroup b publishes its count,
// looks back for the count before it, publishes the inclusive count and then
// every row leader writes its row into exit_idx or keep_idx at its stable
// position.  The last workgroup writes n_exit and advances the serial number
// once every workgroup has published (so every workgroup has read it).
__device__ __forceinline__ void compact_block(const GateParams& P, const uint8_t* s_route,
                                              uint32_t serial, bool leader, int64_t row) {
  __shared__ int64_t s_excl;
  const int64_t b = blockIdx.x;
  const int wid = threadIdx.x >> 6;
  __syncthreads();  // s_route complete
  if (wid == 0) {
    int agg = 0;
#pragma unroll
    for (int i = 0; i < kGateRows; ++i) agg += s_route[i];
    const unsigned long long tag = (unsigned long long)serial << 32;
    if (b > 0 && threadIdx.x == 0) store_word(P.tiles + b, tag | kStateAgg | (unsigned)agg);
    bool ok = true;
    const int64_t excl = b > 0 ? look_back(P, b, serial, &ok) : 0;
    if (threadIdx.x == 0) {
      store_word(P.tiles + b, tag | kStateInc | (unsigned)((excl + agg) & kCountMask));
      if (!ok) __hip_atomic_fetch_or(P.serial + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (b == (int64_t)gridDim.x - 1) {
        if (P.n_exit) *P.n_exit = (int32_t)(excl + agg);
        __hip_atomic_store(P.serial, serial + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      s_excl = excl;
    }
  }
  __syncthreads();
  if (leader && row < P.B) {
    int before = 0;
    for (int i = 0; i < wid; ++i) before += s_route[i];
    const int64_t pe = s_excl + before;
    if (s_route[wid]) {
      if (P.exit_idx) P.exit_idx[pe] = (int32_t)row;
    } else if (P.keep_idx) {
      P.keep_idx[row - pe] = (int32_t)row;
    }
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

// Routing of one Ouro row (cdb_scheduler.py:207-222,254-266).  The request is
// the gate's signal, or with a replay depth rd > 0, depth >= rd - delay.  With
// direct routing the request routes the row now; otherwise the request recorded
// for the row's state slot by the previous call routes it (a token present in
// consecutive core steps has advanced since its gate), and this call's request
// is recorded unless the row leaves now.  The depth cap always routes.
__device__ __forceinline__ int route_row(const GateParams& P, int m, int32_t depth, int64_t s,
                                         int64_t row, long long pend, uint32_t serial) {
  const int cap = P.max_depth > 0 && depth >= P.max_depth;
  int req = m;
  if (P.replay) {
    const int32_t rd = P.replay[row];
    if (rd > 0) req = depth >= rd - (P.direct ? 0 : 1);
  }
  if (P.direct) return cap | req;
  const int prev = (uint32_t)((unsigned long long)pend >> 32) == serial && (pend & 1);
  const int r = cap | prev;
  P.pending[s] = r ? 0 : (long long)(((unsigned long long)(serial + 1u) << 32) | (unsigned)req);
  return r;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kGateThreads) void ouro_gate_kernel(GateParams P) {
  __shared__ uint8_t s_route[kGateRows];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kGateRows + wid;
  const bool leader = lane == 0;
  const bool live = row < P.B;
  // per-row scalars first, so their latency hides under the row loads (the
  // state of a row indexed through a state-pool slot waits for the slot)
  uint32_t serial = 0;
  if (P.serial) serial = __hip_atomic_load(P.serial, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int64_t s = row;
  int32_t ls = P.loop_step_scalar;
  float bv = 0.0f, F = 0.0f;
  long long pend = 0;
  if (live && leader) {
    if (P.bias) bv = load_one<T>(P.bias);
    if (P.loop_step) ls = P.loop_step[row];
    if (P.slots) {
      s = P.slots[row];
    } else {
      if (P.F_prev) F = P.F_prev[row];
      if (!P.direct) pend = P.pending[row];
    }
  }
  float acc = 0.0f;
  if (live) {
    const T* hrow = reinterpret_cast<const T*>(P.h) + row * P.ldh;
    row_pairs<T, kWave, VEC>(hrow, reinterpret_cast<const T*>(P.w), P.H, lane,
                             [&](float x, float y) { acc = fmaf(x, y, acc); });
  }
  if (live && leader && P.slots) {
    if (P.F_prev) F = P.F_prev[s];
    if (!P.direct) pend = P.pending[s];
  }
  acc = wave_total(acc);
  int r = 0;
  if (live && leader) {
    const float z = round_to<T>(acc + bv);
    const float Fn = gate_update(F, z);
    const int32_t depth = ls + 1;
    const int m = (Fn >= P.tau) && (depth + P.lookahead >= P.min_loop_steps);
    r = route_row(P, m, depth, s, row, pend, serial);
    P.F_next[s] = Fn;
    P.mask[row] = (uint8_t)(P.cap_in_mask ? r : m);
    if (P.route) P.route[row] = (uint8_t)r;
    if (P.aux_out) P.aux_out[row] = z;
  }
  if (!P.tiles) return;
  if (leader) s_route[wid] = (uint8_t)r;
  compact_block(P, s_route, serial, leader, row);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kGateThreads) void rel_change_kernel(GateParams P) {
  __shared__ uint8_t s_route[kGateRows];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kGateRows + wid;
  const bool leader = lane == 0;
  const bool live = row < P.B;
  uint32_t serial = 0;
  if (P.serial) serial = __hip_atomic_load(P.serial, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float d2 = 0.0f, n2 = 0.0f;
  if (live) {
    const T* a = reinterpret_cast<const T*>(P.h) + row * P.ldh;
    const T* bp = reinterpret_cast<const T*>(P.hp) + row * P.ldp;
    row_pairs<T, kWave, VEC>(a, bp, P.H, lane, [&](float x, float y) {
      const float dd = x - y;
      d2 = fmaf(dd, dd, d2);
      n2 = fmaf(x, x, n2);
    });
  }
  d2 = wave_total(d2);
  n2 = wave_total(n2);
  int m = 0;
  if (live && leader) {
    const float ratio = sqrtf(d2) / fmaxf(sqrtf(n2), P.eps);
    m = ratio < P.tau;
    P.mask[row] = (uint8_t)m;
    if (P.aux_out) P.aux_out[row] = ratio;
  }
  if (!P.tiles) return;
  if (leader) s_route[wid] = (uint8_t)m;
  compact_block(P, s_route, serial, leader, row);
}

template <typename T>
__global__ void cum_exit_kernel(const void* z, const float* F_prev, float* F_next, int64_t B) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < B) F_next[i] = gate_update(F_prev[i], load_one<T>(reinterpret_cast<const T*>(z) + i));
}

enum class GateKind { kOuro, kRelChange };

template <typename T, bool VEC>
static void launch_kind(GateKind kind, const GateParams& P, hipStream_t st) {
  const dim3 grid((unsigned)(P.B > 0 ? (P.B + kGateRows - 1) / kGateRows : 1)), block(kGateThreads);
  if (kind == GateKind::kOuro) hipLaunchKernelGGL((ouro_gate_kernel<T, VEC>), grid, block, 0, st, P);
  else hipLaunchKernelGGL((rel_change_kernel<T, VEC>), grid, block, 0, st, P);
}

static int dispatch_rows(GateKind kind, int dtype, const GateParams& P, bool vec, hipStream_t st) {
  if (dtype == kF32) vec ? launch_kind<float, true>(kind, P, st) : launch_kind<float, false>(kind, P, st);
  else if (dtype == kBF16) vec ? launch_kind<bf16_t, true>(kind, P, st) : launch_kind<bf16_t, false>(kind, P, st);
  else if (dtype == kF16) vec ? launch_kind<f16_t, true>(kind, P, st) : launch_kind<f16_t, false>(kind, P, st);
  else return set_error(LSG_ERR_ARG, "unknown dtype %d", dtype);
  return LSG_OK;
}

// Workspace layout: serial number and error flag (256 B), then one 64-bit
// published word per workgroup of kGateRows rows.
static int setup_workspace(GateParams& P, int op, bool want, void* ws, size_t ws_bytes,
                           const char* fn) {
  if (!want) {
    P.serial = nullptr;
    P.tiles = nullptr;
    return LSG_OK;
  }
  if (P.B >= (int64_t)kCountMask)
    return set_error(LSG_ERR_ARG, "%s: exit compaction supports B < %u rows", fn, kCountMask);
  const size_t need = lsg_workspace_bytes(op, P.B);
  if (!ws || ws_bytes < need || ((uintptr_t)ws % 16) != 0)
    return set_error(LSG_ERR_WORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) needed, got %zu",
                     fn, need, ws ? ws_bytes : (size_t)0);
  P.serial = reinterpret_cast<uint32_t*>(ws);
  P.tiles = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws) + 256);
  return LSG_OK;
}

static bool rows_vec(const void* base, int64_t ld, int dtype) {
  const int64_t es = dtype == kF32 ? 4 : 2;
  return ((uintptr_t)base % 16 == 0) && ((ld * es) % 16 == 0);
}

static int gate_common(const char* fn, const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                       const void* w, const void* bias, const float* F_prev, float* F_next,
                       const int32_t* slots, const int32_t* loop_step, int32_t loop_step_scalar,
                       float tau, int32_t min_loop_steps, int32_t lookahead, int32_t max_depth,
                       int32_t direct, int32_t cap_in_mask, int64_t* pending,
                       const int32_t* replay_depth, uint8_t* mask, uint8_t* route,
                       int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit, float* z_out,
                       void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if ((B > 0 && (!h || !w || !F_next || !mask)) || B < 0 || H < 1 || (B > 0 && ldh < H))
    return set_error(LSG_ERR_ARG, "%s: bad arguments (B=%lld H=%lld ldh=%lld)", fn, (long long)B,
                     (long long)H, (long long)ldh);
  if (B > 0x7fffffffLL) return set_error(LSG_ERR_ARG, "%s: B exceeds int32 rows", fn);
  if (!direct && !pending)
    return set_error(LSG_ERR_ARG, "%s: lookahead routing needs the pending-gate pool", fn);
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
  P.direct = direct ? 1 : 0;
  P.cap_in_mask = cap_in_mask;
  P.pending = reinterpret_cast<long long*>(pending);
  P.replay = replay_depth;
  P.mask = mask;
  P.route = route;
  P.aux_out = z_out;
  P.exit_idx = exit_idx;
  P.keep_idx = keep_idx;
  P.n_exit = n_exit;
  const bool want = exit_idx || keep_idx || n_exit || !direct;
  int rc = setup_workspace(P, LSG_OP_EXIT_GATE, want, workspace, workspace_bytes, fn);
  if (rc != LSG_OK) return rc;
  if (B == 0 && !P.tiles) return LSG_OK;
  const bool vec = rows_vec(h, ldh, dtype) && rows_vec(w, H, dtype);
  rc = dispatch_rows(GateKind::kOuro, dtype, P, vec, reinterpret_cast<hipStream_t>(stream));
  if (rc != LSG_OK) return rc;
  return check_launch(fn);
}

// Workspace of lsg_exit_gate_noalloc: a file-scope device array, one copy per
// GPU, zero at load and never cleared afterwards (the call serial number kept in
// it tells each call's published words from older ones).  Its host-side name is
// not a device address: kernels get the address hipGetSymbolAddress returns for
// the current device, looked up once per device.
constexpr int64_t kNoAllocMaxRows = 65536;
constexpr size_t kScratchBytes = 256 + (size_t)(kNoAllocMaxRows / kGateRows) * 8;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

static int scratch_for_current_device(void** out, const char* fn) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(LSG_ERR_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return set_error(LSG_ERR_ARG, "%s: device %d out of range", fn, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(LSG_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", fn, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LSG_OK;
}

}  // namespace lsg

using namespace lsg;

extern "C" int lsg_exit_gate_noalloc(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                                     const void* w, const void* bias, const float* F_prev,
                                     float* F_next, const int32_t* slots,
                                     const int32_t* loop_step, int32_t loop_step_scalar, float tau,
                                     int32_t min_loop_steps, int32_t lookahead, int32_t max_depth,
                                     uint8_t* mask, int32_t* exit_idx, int32_t* keep_idx,
                                     int32_t* n_exit, float* z_out, void* stream) {
  clear_error();
  if (B > kNoAllocMaxRows)
    return set_error(LSG_ERR_ARG, "lsg_exit_gate_noalloc: B=%lld exceeds the static workspace's %lld rows",
                     (long long)B, (long long)kNoAllocMaxRows);
  void* ws = nullptr;
  if (exit_idx || keep_idx || n_exit) {
    const int rc = scratch_for_current_device(&ws, "lsg_exit_gate_noalloc");
    if (rc != LSG_OK) return rc;
  }
  return gate_common("lsg_exit_gate_noalloc", h, dtype, B, H, ldh, w, bias, F_prev, F_next, slots,
                     loop_step, loop_step_scalar, tau, min_loop_steps, lookahead, max_depth, 1, 1,
                     nullptr, nullptr, mask, nullptr, exit_idx, keep_idx, n_exit, z_out, ws,
                     ws ? kScratchBytes : 0, stream);
}

extern "C" int lsg_exit_gate(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                             const void* w, const void* bias, const float* F_prev, float* F_next,
                             const int32_t* slots, const int32_t* loop_step,
                             int32_t loop_step_scalar, float tau, int32_t min_loop_steps,
                             int32_t lookahead, int32_t max_depth, uint8_t* mask,
                             int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit, float* z_out,
                             void* workspace, size_t workspace_bytes, void* stream) {
  return gate_common("lsg_exit_gate", h, dtype, B, H, ldh, w, bias, F_prev, F_next, slots,
                     loop_step, loop_step_scalar, tau, min_loop_steps, lookahead, max_depth, 1, 1,
                     nullptr, nullptr, mask, nullptr, exit_idx, keep_idx, n_exit, z_out, workspace,
                     workspace_bytes, stream);
}

extern "C" int lsg_exit_gate_route(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh,
                                   const void* w, const void* bias, const float* F_prev,
                                   float* F_next, const int32_t* slots, const int32_t* loop_step,
                                   int32_t loop_step_scalar, float tau, int32_t min_loop_steps,
                                   int32_t lookahead, int32_t max_depth,
                                   int32_t disable_lookahead_exit, int64_t* pending,
                                   const int32_t* replay_depth, uint8_t* mask, uint8_t* route,
                                   int32_t* exit_idx, int32_t* keep_idx, int32_t* n_exit,
                                   float* z_out, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  return gate_common("lsg_exit_gate_route", h, dtype, B, H, ldh, w, bias, F_prev, F_next, slots,
                     loop_step, loop_step_scalar, tau, min_loop_steps, lookahead, max_depth,
                     disable_lookahead_exit ? 1 : 0, 0, pending, replay_depth, mask, route,
                     exit_idx, keep_idx, n_exit, z_out, workspace, workspace_bytes, stream);
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
  P.direct = 1;
  P.mask = mask;
  P.aux_out = ratio;
  P.exit_idx = exit_idx;
  P.keep_idx = keep_idx;
  P.n_exit = n_exit;
  int rc = setup_workspace(P, LSG_OP_REL_CHANGE, exit_idx || keep_idx || n_exit, workspace,
                           workspace_bytes, "lsg_relative_state_change");
  if (rc != LSG_OK) return rc;
  if (B == 0 && !P.tiles) return LSG_OK;
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
