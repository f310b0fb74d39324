/*
 * CPU oracle for the per-step decode token path of Loop-SGLang.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or the timed CPU baseline).  The product path never calls it.
 *
 * It restates, in plain C with float64 arithmetic, the semantics of:
 *   - greedy sampling:  python/loopsgl/model_executor/sample.py:110-111
 *                       (torch.argmax over the row; first maximum; NaN wins)
 *                       and the int32 cast at model_executor/model_runner.py:279-280
 *   - non-greedy sampling: sample.py:60-81,112 (softmax with temperature, then
 *                       top-k / top-p / top-k-then-top-p filtering and one draw).
 *                       The draw itself lives in flashinfer-python==0.6.6, which
 *                       is not vendored; the inverse-CDF rule below is this
 *                       build's own definition (one explicit uniform per row).
 *   - the Ouro exit gate: models/looped/ouro.py:142-155 (gate logit, threshold,
 *                       depth gate), models/looped/exit_gates.py:6-15 (sigmoid and
 *                       cumulative exit probability), layers/linear.py:32-33
 *                       (F.linear with bias, output rounded to the model dtype).
 *   - exit compaction:  managers/cdb_scheduler.py:215-228 (stable filter of
 *                       exited rows, in gate-row order).
 *   - the Huginn gate:  models/looped/huginn.py:184-194 and exit_gates.py:18-24.
 *
 * Every function reports, per row, whether the result sits so close to a
 * decision boundary that an fp32 device computation may legitimately differ
 * (the "ambiguous" flag).  Rows that are not flagged must match bit-exactly.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   orc_argmax        -> torch.argmax on CPU (the reference's own call), incl.
 *                        NaN, +-0, +-inf and ties.
 *   orc_sample        -> softmax vs torch.softmax; top-k / top-p kept sets vs the
 *                        HF transformers TopK/TopP warpers on tie-free rows;
 *                        inverse CDF vs numpy.searchsorted; closed forms
 *                        (uniform rows, one-hot rows); brute force on tiny V.
 *   orc_exit_gate     -> the reference's KATs (tests/core/test_exit_gates.py),
 *                        the product form 1 - prod(1 - lambda), scipy expit,
 *                        numpy.nonzero for the compaction.
 *   orc_rel_change    -> the reference's Huginn KAT and numpy.linalg.norm.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

enum { ORC_F32 = 0, ORC_BF16 = 1, ORC_F16 = 2 };

static float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
  if (e == 0) {
    if (m == 0) {
      u = s;
    } else { /* subnormal: renormalise */
      int sh = 0;
      while (!(m & 0x400)) { m <<= 1; ++sh; }
      m &= 0x3ff;
      u = s | ((uint32_t)(127 - 15 - sh + 1) << 23) | (m << 13);
    }
  } else if (e == 31) {
    u = s | 0x7f800000u | (m << 13);
  } else {
    u = s | ((e - 15 + 127) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float load_elem(const void* base, int dtype, int64_t i) {
  if (dtype == ORC_F32) return ((const float*)base)[i];
  if (dtype == ORC_BF16) return bf16_to_f32(((const uint16_t*)base)[i]);
  return f16_to_f32(((const uint16_t*)base)[i]);
}

static size_t elem_size(int dtype) { return dtype == ORC_F32 ? 4 : 2; }

/* Round a float64 to bf16 (round to nearest even), returned as the float value. */
static double round_bf16(double v) {
  if (isnan(v)) return v;
  int ex;
  if (v == 0.0 || isinf(v)) return v;
  frexp(v, &ex); /* v = m * 2^ex, 0.5 <= |m| < 1 */
  /* bf16 has 8 significant bits (1 implicit + 7). */
  int e = ex;
  if (e < -125) e = -125; /* subnormal range of bf16 (same exponent range as f32) */
  double q = ldexp(1.0, e - 8); /* spacing of representable values */
  double n = v / q;
  double fl = floor(n), diff = n - fl, r;
  if (diff > 0.5) r = fl + 1;
  else if (diff < 0.5) r = fl;
  else r = (fmod(fl, 2.0) == 0.0) ? fl : fl + 1;
  double out = r * q;
  if (fabs(out) > 3.3895313892515355e38) out = copysign(INFINITY, v); /* bf16 max */
  return out;
}

/* Round a float64 to IEEE fp16 (round to nearest even). */
static double round_f16(double v) {
  if (isnan(v) || isinf(v) || v == 0.0) return v;
  int ex;
  frexp(v, &ex);
  int e = ex;
  if (e < -13) e = -13; /* fp16 subnormal spacing 2^-24 */
  double q = ldexp(1.0, e - 11);
  double n = v / q, fl = floor(n), diff = n - fl, r;
  if (diff > 0.5) r = fl + 1;
  else if (diff < 0.5) r = fl;
  else r = (fmod(fl, 2.0) == 0.0) ? fl : fl + 1;
  double out = r * q;
  if (fabs(out) >= 65520.0) out = copysign(INFINITY, v);
  return out;
}

static double round_to_dtype(double v, int dtype) {
  if (dtype == ORC_F32) return (double)(float)v;
  if (dtype == ORC_BF16) return round_bf16(v);
  return round_f16(v);
}

/* --------------------------------------------------------------------------
 * Greedy: torch.argmax semantics.  NaN compares greater than everything and the
 * first NaN wins; otherwise the first strict maximum wins (+0 == -0).
 * sample.py:110-111, model_runner.py:279-280.
 * ------------------------------------------------------------------------ */
static int32_t argmax_row(const void* row, int dtype, int64_t V) {
  int32_t bi = 0;
  float bv = load_elem(row, dtype, 0);
  for (int64_t i = 1; i < V; ++i) {
    if (isnan(bv)) break;
    float x = load_elem(row, dtype, i);
    if (isnan(x) || x > bv) {
      bv = x;
      bi = (int32_t)i;
    }
  }
  return bi;
}

void orc_argmax(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld,
                int32_t* out, int nthreads) {
  const char* base = (const char*)logits;
  size_t es = elem_size(dtype);
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < B; ++r) out[r] = argmax_row(base + (size_t)r * ld * es, dtype, V);
  (void)nthreads;
}

/* Order-preserving 64-bit sort key: descending by value (NaN as -inf, -0 as +0),
 * ties broken by ascending index. */
static uint32_t okey(float f) {
  uint32_t b;
  if (isnan(f)) f = -INFINITY;
  if (f == 0.0f) f = 0.0f; /* -0 -> +0 */
  memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static int cmp_desc_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

static int cmp_asc_i64(const void* a, const void* b) {
  int64_t x = *(const int64_t*)a, y = *(const int64_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

/* --------------------------------------------------------------------------
 * Non-greedy sampling of one row (build definition of sample.py:60-81,112):
 *   x_i  = float32(logit_i);  NaN is treated as -inf.
 *   m    = max_i x_i.  If m is not finite, or T is not a finite positive
 *          number, the row is decided by argmax (torch semantics).
 *   e_i  = exp((x_i - m) / T)                      (S2)
 *   K    = {i : x_i >= x_(k)} if 1 <= k < V, else all rows  (S3, ties kept)
 *   Z_K  = sum_K e_i
 *   P    = {i in K : x_i >= tau}, tau = max{theta : sum_{K, x>=theta} e >= p Z_K}
 *          if p < 1, else K                        (S4, ties kept)
 *   id   = min{j in P : sum_{i in P, i<=j} e_i > u * sum_P e}   (S5)
 * amb bit 0: the CDF at the chosen boundary lies within tol of u.
 * amb bit 1: the top-p mass at tau lies within tol of p.  The row then also
 *            has an alternative id: the draw from the other kept set a float
 *            evaluation of the same comparison can produce (the next tie group
 *            included when the crossing group's mass reaches p*Z_K by less than
 *            tol, the crossing group left out when the mass above it falls short
 *            of p*Z_K by less than tol).
 * amb bit 2: that alternative draw's CDF lies within tol of u.
 * ------------------------------------------------------------------------ */
typedef struct {
  uint64_t* keys;
  int64_t* idx;
  double* e;
  int64_t cap;
} scratch_t;

/* Inverse CDF over the first nP entries of the descending key order, in
 * ascending index order (S5); sets `flag` in *amb when the CDF at the chosen
 * boundary lies within tol of u. */
static int32_t walk_prefix(scratch_t* s, int64_t nP, float u, double tol, uint8_t* amb, uint8_t flag) {
  for (int64_t q = 0; q < nP; ++q) s->idx[q] = (int64_t)(0xffffffffu - (uint32_t)s->keys[q]);
  qsort(s->idx, (size_t)nP, sizeof(int64_t), cmp_asc_i64);
  double sigma = 0.0;
  for (int64_t q = 0; q < nP; ++q) sigma += s->e[s->idx[q]];
  double U = (double)u * sigma, cum = 0.0;
  int64_t last_pos = -1;
  for (int64_t q = 0; q < nP; ++q) {
    double ei = s->e[s->idx[q]];
    if (ei <= 0.0) continue;
    double prev = cum;
    cum += ei;
    last_pos = q;
    if (cum > U) {
      if ((cum - U) < tol * sigma || (U - prev) < tol * sigma) *amb |= flag;
      return (int32_t)s->idx[q];
    }
  }
  *amb |= flag; /* u >= 1 or rounding: fall back to the last element with mass */
  return last_pos >= 0 ? (int32_t)s->idx[last_pos] : (int32_t)s->idx[0];
}

static int32_t sample_row(const void* row, int dtype, int64_t V, float T, int32_t k, float p,
                          float u, double tol, uint8_t* amb, int32_t* alt, scratch_t* s) {
  *amb = 0;
  double m = -INFINITY;
  int any = 0;
  for (int64_t i = 0; i < V; ++i) {
    float x = load_elem(row, dtype, i);
    if (isnan(x)) continue;
    if (!any || x > m) m = x;
    any = 1;
  }
  if (!any || !isfinite(m) || !(T > 0.0f) || !isfinite(T)) return argmax_row(row, dtype, V);

  if (s->cap < V) {
    s->keys = (uint64_t*)realloc(s->keys, (size_t)V * sizeof(uint64_t));
    s->idx = (int64_t*)realloc(s->idx, (size_t)V * sizeof(int64_t));
    s->e = (double*)realloc(s->e, (size_t)V * sizeof(double));
    s->cap = V;
  }
  double Td = (double)T;
  for (int64_t i = 0; i < V; ++i) {
    float x = load_elem(row, dtype, i);
    s->e[i] = isnan(x) ? 0.0 : exp(((double)x - m) / Td);
    s->keys[i] = ((uint64_t)okey(x) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  }
  qsort(s->keys, (size_t)V, sizeof(uint64_t), cmp_desc_u64);

  int kon = (k >= 1 && (int64_t)k < V);
  int pon = (p < 1.0f);
  /* nK = |K| (prefix length of the sorted order, ties at the boundary included) */
  int64_t nK = V;
  if (kon) {
    uint32_t kb = (uint32_t)(s->keys[k - 1] >> 32);
    nK = k;
    while (nK < V && (uint32_t)(s->keys[nK] >> 32) == kb) ++nK;
  }
  double ZK = 0.0;
  for (int64_t q = 0; q < nK; ++q) ZK += s->e[0xffffffffu - (uint32_t)s->keys[q]];

  int64_t nP = nK, nP_alt = nK;
  if (pon) {
    double target = (double)p * ZK, cum = 0.0;
    int64_t q = 0;
    for (; q < nK; ++q) {
      /* process one tie group at a time */
      uint32_t kb = (uint32_t)(s->keys[q] >> 32);
      double above = cum;
      int64_t g = q;
      while (g < nK && (uint32_t)(s->keys[g] >> 32) == kb) {
        cum += s->e[0xffffffffu - (uint32_t)s->keys[g]];
        ++g;
      }
      if (cum >= target) {
        nP = nP_alt = g;
        if ((cum - target) < tol * ZK) {  /* alternative: the next tie group kept too */
          *amb |= 2;
          if (g < nK) {
            uint32_t nb = (uint32_t)(s->keys[g] >> 32);
            nP_alt = g;
            while (nP_alt < nK && (uint32_t)(s->keys[nP_alt] >> 32) == nb) ++nP_alt;
          }
        } else if ((target - above) < tol * ZK) {  /* alternative: this group left out */
          *amb |= 2;
          if (q > 0) nP_alt = q;
        }
        break;
      }
      q = g - 1;
    }
    if (q >= nK) nP = nK; /* unreachable in exact arithmetic (p < 1) */
  }

  int32_t id = walk_prefix(s, nP, u, tol, amb, 1);
  if (alt) *alt = id;
  if (alt && (*amb & 2) && nP_alt != nP) *alt = walk_prefix(s, nP_alt, u, tol, amb, 4);
  return id;
}

void orc_sample(const void* logits, int dtype, int64_t B, int64_t V, int64_t ld,
                const float* temps, const int32_t* top_k, const float* top_p,
                const float* uniforms, int32_t* out_ids, uint8_t* out_amb, double tol,
                int nthreads, int32_t* out_alt) {
  const char* base = (const char*)logits;
  size_t es = elem_size(dtype);
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    scratch_t s = {0, 0, 0, 0};
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
    for (int64_t r = 0; r < B; ++r) {
      const void* row = base + (size_t)r * ld * es;
      uint8_t a = 0;
      int32_t alt = 0;
      if (!temps) {
        out_ids[r] = alt = argmax_row(row, dtype, V);
      } else {
        out_ids[r] = sample_row(row, dtype, V, temps[r], top_k ? top_k[r] : 0,
                                top_p ? top_p[r] : 1.0f, uniforms ? uniforms[r] : 0.0f, tol,
                                &a, &alt, &s);
      }
      if (out_amb) out_amb[r] = a;
      if (out_alt) out_alt[r] = alt;
    }
    free(s.keys);
    free(s.idx);
    free(s.e);
  }
  (void)nthreads;
}

/* --------------------------------------------------------------------------
 * Ouro exit gate (G1-G5).
 *   z      = round_dtype( sum_h h[r,h] * w[h] + b )       (layers/linear.py:32-33)
 *   lambda = 1 / (1 + exp(-z)) in float32, one rounding per op, exp(-z)
 *            correctly rounded to float32  (torch's sigmoid(float(z)), exit_gates.py:13)
 *   F'     = F + (1 - F) * lambda  as three float32 ops     (exit_gates.py:13-15)
 *   depth  = loop_step + 1 + lookahead                      (ouro.py:152)
 *   mask   = (F' >= tau) & (depth >= min_loop_steps)        (ouro.py:153-154)
 *            | (max_depth > 0 & loop_step + 1 >= max_depth) (cdb_scheduler.py:221,262-266)
 *   exit_idx / keep_idx: ascending rows with mask 1 / 0    (cdb_scheduler.py:215-228)
 * amb bit 0: the exit decision may differ from the reference's (bit 2 or bit 3
 *            changes it).
 * amb bit 2: z itself may round differently under fp32 accumulation.
 * amb bit 3: |F' - tau| < 1e-6 in the float64 shadow F + (1 - F) * sigmoid(z):
 *            an exp or sigmoid that differs by an ulp can flip the compare.
 * ------------------------------------------------------------------------ */
/* lambda = 1 / (1 + exp(-z)) in float32 with exp(-z) rounded once from float64
 * (x86-64 SSE arithmetic: no excess precision), then
 * F' = F + (1 - F) * lambda as three separately rounded float32 ops. */
static float sigmoid_f32(double z) {
  volatile float e = (float)exp(-z);
  volatile float d = 1.0f + e;
  volatile float lam = 1.0f / d;
  return lam;
}

static float gate_update(float F, double z) {
  float lam = sigmoid_f32(z);
  volatile float t1 = 1.0f - F;
  volatile float t2 = t1 * lam;
  volatile float Fn = F + t2;
  return Fn;
}

static int gate_mask(float Fn, int32_t ls, float tau, int32_t min_loop_steps, int32_t lookahead,
                     int32_t max_depth) {
  int exit_depth = ls + 1 + (lookahead ? 1 : 0);
  int m = (Fn >= tau) && (exit_depth >= min_loop_steps);
  if (max_depth > 0 && ls + 1 >= max_depth) m = 1;
  return m;
}

/* 1 when the float64 shadow of F' lies within 1e-6 of tau and the compare
 * decides the mask (depth test passed, no depth cap). */
static int tau_band(float F, double z, int32_t ls, float tau, int32_t min_loop_steps,
                    int32_t lookahead, int32_t max_depth) {
  if (ls + 1 + (lookahead ? 1 : 0) < min_loop_steps) return 0;
  if (max_depth > 0 && ls + 1 >= max_depth) return 0;
  double lam = 1.0 / (1.0 + exp(-z));
  double F64 = (double)F + (1.0 - (double)F) * lam;
  return fabs(F64 - (double)tau) < 1e-6;
}

void orc_exit_gate(const void* h, int dtype, int64_t B, int64_t H, int64_t ldh, const void* w,
                   const void* bias, const float* F_prev, const int32_t* loop_step,
                   int32_t loop_step_scalar, float tau, int32_t min_loop_steps, int32_t lookahead,
                   int32_t max_depth, float* F_next, uint8_t* mask, int32_t* exit_idx,
                   int32_t* keep_idx, int32_t* n_exit, float* z_out, uint8_t* amb) {
  const char* hb = (const char*)h;
  size_t es = elem_size(dtype);
  double bv = bias ? (double)load_elem(bias, dtype, 0) : 0.0;
  for (int64_t r = 0; r < B; ++r) {
    const void* row = hb + (size_t)r * ldh * es;
    double acc = 0.0, mag = 0.0;
    for (int64_t i = 0; i < H; ++i) {
      double t = (double)load_elem(row, dtype, i) * (double)load_elem(w, dtype, i);
      acc += t;
      mag += fabs(t);
    }
    double v = acc + bv;
    /* fp32 accumulation error bound of a device reduction (per-lane sequential
     * over about H/64 terms, a 6-level tree, then the bias add), doubled. */
    double gam = 2.0 * ((double)H / 64.0 + 8.0) * ldexp(1.0, -24) * (mag + fabs(bv));
    double z = round_to_dtype(v, dtype);
    int32_t ls = loop_step ? loop_step[r] : loop_step_scalar;
    float F = F_prev ? F_prev[r] : 0.0f;
    float Fn = gate_update(F, z);
    int m = gate_mask(Fn, ls, tau, min_loop_steps, lookahead, max_depth);
    uint8_t a = 0;
    if (isfinite(v)) {
      double zlo = round_to_dtype(v - gam, dtype), zhi = round_to_dtype(v + gam, dtype);
      if (zlo != zhi) {
        a |= 4; /* z itself may round differently on the device */
        int mlo = gate_mask(gate_update(F, zlo), ls, tau, min_loop_steps, lookahead, max_depth);
        int mhi = gate_mask(gate_update(F, zhi), ls, tau, min_loop_steps, lookahead, max_depth);
        if (mlo != mhi) a |= 1; /* the exit decision itself may differ */
      }
    }
    if (tau_band(F, z, ls, tau, min_loop_steps, lookahead, max_depth)) a |= 8 | 1;
    if (z_out) z_out[r] = (float)z;
    F_next[r] = Fn;
    mask[r] = (uint8_t)m;
    if (amb) amb[r] = a;
  }
  int32_t ne = 0, nk = 0;
  for (int64_t r = 0; r < B; ++r) {
    if (mask[r]) {
      if (exit_idx) exit_idx[ne] = (int32_t)r;
      ++ne;
    } else {
      if (keep_idx) keep_idx[nk] = (int32_t)r;
      ++nk;
    }
  }
  if (n_exit) *n_exit = ne;
}

/* cumulative_exit_probability alone (exit_gates.py:6-15) on given gate logits. */
void orc_cumulative_exit_probability(const float* z, const float* F_prev, int64_t B, float* F_next) {
  for (int64_t r = 0; r < B; ++r) {
    F_next[r] = gate_update(F_prev[r], (double)z[r]);
  }
}

/* --------------------------------------------------------------------------
 * Huginn gate (G6): ratio = ||h - h_prev||_2 / max(||h||_2, 1e-9), mask = ratio < tau.
 * huginn.py:184-194, exit_gates.py:18-24.  amb bit 0: |ratio - tau| <= tol*max(tau,1e-30).
 * ------------------------------------------------------------------------ */
void orc_rel_change(const void* h, const void* hp, int dtype, int64_t B, int64_t H, int64_t ldh,
                    int64_t ldp, float tau, double tol, float* ratio_out, uint8_t* mask,
                    uint8_t* amb) {
  size_t es = elem_size(dtype);
  for (int64_t r = 0; r < B; ++r) {
    const char* a = (const char*)h + (size_t)r * ldh * es;
    const char* b = (const char*)hp + (size_t)r * ldp * es;
    double d2 = 0.0, n2 = 0.0;
    for (int64_t i = 0; i < H; ++i) {
      double x = load_elem(a, dtype, i), y = load_elem(b, dtype, i);
      d2 += (x - y) * (x - y);
      n2 += x * x;
    }
    double den = sqrt(n2);
    if (den < 1e-9) den = 1e-9;
    double ratio = sqrt(d2) / den;
    if (ratio_out) ratio_out[r] = (float)ratio;
    mask[r] = (uint8_t)(ratio < (double)tau);
    if (amb) amb[r] = (uint8_t)(fabs(ratio - (double)tau) <= tol * fmax(fabs((double)tau), 1e-30));
  }
}
