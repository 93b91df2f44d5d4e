/*
 * maxsim_oracle.c - CPU restatement of flash_maxsim's scoring path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg. It is never part
 * of the product path: flash_maxsim_amd runs only its HIP kernels.
 *
 * Functions and the reference code they restate (roipony/flash-maxsim 0.1.0):
 *   oracle_maxsim        maxsim_naive            flash_maxsim/flash_maxsim.py:294-301
 *                        (NaN rule of torch.max: a NaN similarity is the max,
 *                        the first NaN its index)
 *                        + varlen mask            flash_maxsim.py:297-300, :121,:129
 *                        + argmax (first max)     flash_maxsim.py:132-135
 *                        + batched / per-query    flash_maxsim.py:94-100, :233-250
 *                        + sparse row gather      flash_maxsim/flash_maxsim_sparse.py:62-71, :153-157
 *   oracle_maxsim_int8   maxsim_naive(dequantize_int8(...))  flash_maxsim_quant.py:31-33
 *   oracle_quantize_int8 quantize_int8            flash_maxsim/flash_maxsim_quant.py:23-28
 *   oracle_bwd           backward kernels         flash_maxsim/flash_maxsim.py:153-188
 *   oracle_f32_to_f16    IEEE binary32 -> binary16, round to nearest even
 *                        (the .half() casts of flash_maxsim_quant.py:28)
 *
 * Similarities are accumulated in double: the oracle is the exact-arithmetic
 * target the fp32 GPU results are held to. Quantisation follows torch's
 * float32 elementwise arithmetic exactly (build with -ffp-contract=off).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Dot product of two float rows in double, four interleaved partial sums
 * combined as (s0 + s1) + (s2 + s3): a fixed order independent of the
 * compiler. */
static double dot_f64(const float* a, const float* b, int64_t d) {
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
  int64_t k = 0;
  for (; k + 4 <= d; k += 4) {
    s0 += (double)a[k] * (double)b[k];
    s1 += (double)a[k + 1] * (double)b[k + 1];
    s2 += (double)a[k + 2] * (double)b[k + 2];
    s3 += (double)a[k + 3] * (double)b[k + 3];
  }
  for (; k < d; ++k) s0 += (double)a[k] * (double)b[k];
  return (s0 + s1) + (s2 + s3);
}

typedef struct {
  const float* Q;        /* [Nq, Lq_rows, d] */
  const float* D;        /* [B', Ld, d] */
  const int32_t* lengths;/* [B'] or NULL */
  const int32_t* qidx;   /* [B, Lq] or NULL (sparse) */
  const float* scales;   /* int8 variant: [B, Ld] or NULL */
  const float* mins;
  const uint8_t* codes;  /* int8 variant: [B, Ld, d] */
  int64_t Nq, B, Lq, Lq_rows, Ld, d;
  int shared;
  double* scores;        /* [Nq, B] */
  int32_t* argmax;       /* [Nq*B, Lq] or NULL */
  double* best;          /* [Nq*B, Lq] or NULL: the max similarity */
  int64_t begin, end;    /* item range of this worker */
} job_t;

static void score_item(const job_t* J, int64_t item, float* rowbuf) {
  const int64_t qi = item / J->B, b = item % J->B;
  const int64_t drow = J->shared ? b : item;
  int64_t len = J->lengths ? J->lengths[drow] : J->Ld;
  if (len < 0) len = 0;
  if (len > J->Ld) len = J->Ld;
  const int64_t d = J->d;
  double total = 0.0;
  for (int64_t q = 0; q < J->Lq; ++q) {
    int64_t row = q;
    if (J->qidx) row = J->qidx[b * J->Lq + q];
    const float* qv = NULL;
    if (row >= 0 && row < J->Lq_rows) qv = J->Q + (qi * J->Lq_rows + row) * d;
    double m = -INFINITY;
    int32_t mi = 0;
    for (int64_t j = 0; j < len; ++j) {
      const float* dv;
      if (J->codes) {
        /* dequantize_int8: code * scale + min in float32 (flash_maxsim_quant.py:33) */
        const uint8_t* c = J->codes + (drow * J->Ld + j) * d;
        const float s = J->scales[drow * J->Ld + j], mn = J->mins[drow * J->Ld + j];
        for (int64_t k = 0; k < d; ++k) rowbuf[k] = (float)c[k] * s + mn;
        dv = rowbuf;
      } else {
        dv = J->D + (drow * J->Ld + j) * d;
      }
      const double s = qv ? dot_f64(qv, dv, d) : 0.0;
      /* torch.max over the masked row (flash_maxsim.py:301): the first index
       * reaching the max wins (strict); a NaN similarity is the max and the
       * first NaN keeps it (torch.max propagates NaN and returns its index). */
      if (m == m && !(s <= m)) {
        m = s;
        mi = (int32_t)j;
      }
    }
    total += m;
    if (J->argmax) J->argmax[item * J->Lq + q] = mi;
    if (J->best) J->best[item * J->Lq + q] = m;
  }
  J->scores[item] = total;
}

static void* worker(void* arg) {
  const job_t* J = (const job_t*)arg;
  float* rowbuf = J->codes ? (float*)malloc(sizeof(float) * (size_t)(J->d > 0 ? J->d : 1)) : NULL;
  for (int64_t it = J->begin; it < J->end; ++it) score_item(J, it, rowbuf);
  free(rowbuf);
  return NULL;
}

static void run_jobs(job_t base, int nthreads) {
  const int64_t items = base.Nq * base.B;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  if (items < nthreads) nthreads = items > 0 ? (int)items : 1;
  pthread_t th[256];
  job_t jobs[256];
  for (int t = 0; t < nthreads; ++t) {
    jobs[t] = base;
    jobs[t].begin = items * t / nthreads;
    jobs[t].end = items * (t + 1) / nthreads;
  }
  for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, worker, &jobs[t]);
  worker(&jobs[0]);
  for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
}

/* scores[qi*B + b] = sum_q max_{j < len} <Q[qi, row_q], D[drow, j]>, see above.
 * Q is [Nq, Lq_rows, d]; row_q = q, or qidx[b*Lq + q] when qidx != NULL (an
 * index outside [0, Lq_rows) is a zero query token). drow = b if shared else
 * qi*B + b. len = clamp(lengths[drow], 0, Ld). len == 0 gives -inf, argmax 0. */
void oracle_maxsim(const float* Q, const float* D, const int32_t* lengths, const int32_t* qidx,
                   int64_t Nq, int64_t B, int64_t Lq, int64_t Lq_rows, int64_t Ld, int64_t d,
                   int shared, double* scores, int32_t* argmax, double* best, int nthreads) {
  job_t J;
  memset(&J, 0, sizeof(J));
  J.Q = Q;
  J.D = D;
  J.lengths = lengths;
  J.qidx = qidx;
  J.Nq = Nq;
  J.B = B;
  J.Lq = Lq;
  J.Lq_rows = Lq_rows;
  J.Ld = Ld;
  J.d = d;
  J.shared = shared;
  J.scores = scores;
  J.argmax = argmax;
  J.best = best;
  run_jobs(J, nthreads);
}

/* Single-query MaxSim against dequantize_int8(codes, scales, mins). */
void oracle_maxsim_int8(const float* Q, const uint8_t* codes, const float* scales, const float* mins,
                        const int32_t* lengths, int64_t B, int64_t Lq, int64_t Ld, int64_t d,
                        double* scores, int nthreads) {
  job_t J;
  memset(&J, 0, sizeof(J));
  J.Q = Q;
  J.codes = codes;
  J.scales = scales;
  J.mins = mins;
  J.lengths = lengths;
  J.Nq = 1;
  J.B = B;
  J.Lq = Lq;
  J.Lq_rows = Lq;
  J.Ld = Ld;
  J.d = d;
  J.shared = 1;
  J.scores = scores;
  run_jobs(J, nthreads);
}

/* IEEE binary32 -> binary16 bits, round to nearest, ties to even. */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof(x));
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
  const int e = (int)exp - 127 + 15; /* biased binary16 exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - e; /* 13 dropped bits plus the denormal shift */
    uint32_t h = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* carry may reach inf: correct */
  return (uint16_t)h;
}

/* quantize_int8 (flash_maxsim_quant.py:23-28) per token row of d floats:
 *   min, max over the row; scale = max((max - min) / 255, 1e-8) in float32;
 *   code = clamp(round_half_even((x - min) / scale), 0, 255);
 *   stored scale and min are the binary16 roundings of the float32 values. */
void oracle_quantize_int8(const float* D, int64_t rows, int64_t d, uint8_t* codes, uint16_t* scale_h,
                          uint16_t* min_h, float* scale_f) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = D + r * d;
    float mn = x[0], mx = x[0];
    for (int64_t k = 1; k < d; ++k) {
      if (x[k] < mn) mn = x[k];
      if (x[k] > mx) mx = x[k];
    }
    float s = (mx - mn) / 255.0f;
    if (s < 1e-8f) s = 1e-8f;
    for (int64_t k = 0; k < d; ++k) {
      float v = nearbyintf((x[k] - mn) / s);
      if (v < 0.0f) v = 0.0f;
      if (v > 255.0f) v = 255.0f;
      codes[r * d + k] = (uint8_t)v;
    }
    scale_h[r] = oracle_f32_to_f16(s);
    min_h[r] = oracle_f32_to_f16(mn);
    if (scale_f) scale_f[r] = s;
  }
}

/* Backward through the argmax (flash_maxsim.py:153-188), in double:
 *   dQ[q, k]    = sum_b g[b] * D[b, argmax[b, q], k]
 *   dD[b, j, k] = g[b] * sum_{q : argmax[b, q] = j} Q[q, k]   (zero elsewhere) */
void oracle_bwd(const float* Q, const float* D, const int32_t* argmax, const double* g, int64_t B,
                int64_t Lq, int64_t Ld, int64_t d, double* dQ, double* dD) {
  if (dQ) memset(dQ, 0, sizeof(double) * (size_t)(Lq * d));
  if (dD) memset(dD, 0, sizeof(double) * (size_t)(B * Ld * d));
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t q = 0; q < Lq; ++q) {
      const int64_t j = argmax[b * Lq + q];
      if (j < 0 || j >= Ld) continue;
      const float* dv = D + (b * Ld + j) * d;
      const float* qv = Q + q * d;
      if (dQ)
        for (int64_t k = 0; k < d; ++k) dQ[q * d + k] += g[b] * (double)dv[k];
      if (dD)
        for (int64_t k = 0; k < d; ++k) dD[(b * Ld + j) * d + k] += g[b] * (double)qv[k];
    }
  }
}
