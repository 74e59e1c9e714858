/*
 * CPU oracle for the WKV7 hot path.  TEST INFRASTRUCTURE ONLY: this file is
 * the checker that tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline use; no product code path links or calls it.
 *
 * It restates the reference's per-token recurrence in plain C:
 *   - retention: recurrent_retention,
 *       csrc/sm120/tmix/wkv7/recurrent_decay.cuh:10-22, i.e.
 *       w = exp(-exp(-1/2) * sigmoid(logit + bias))
 *   - recurrence, slot gather/scatter, bias before the sigmoid, pre-update S
 *     for sa and post-update S for y, scale on y only:
 *       tests/tmix/wkv7/test.py:29-85 (rwkv7_decay_logits_reference)
 *   - post-chunk boundary snapshots and state_dot_a (per-token sa):
 *       csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cu:32-97
 *
 * wkv7_oracle_f64 evaluates in double precision (the parity reference);
 * wkv7_cpu_f32 is the same recurrence in float, parallel over
 * (sequence, head) with OpenMP (the timed CPU baseline).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

double wkv7_oracle_retention(double x) {
  return exp(-exp(-0.5) / (1.0 + exp(-x)));
}

/*
 * Packed varlen recurrence.
 *   cu[n+1]            token offsets of the n sequences
 *   slots[n] or NULL   state slot of each sequence (NULL: identity)
 *   state              [slots, H, D, D] (k rows, v columns), in place;
 *                      NULL means zero initial state and no write-back
 *   tokens             [total, H, D] as float (bf16/fp16 values widened)
 *   bias               [H, D] or NULL
 *   y                  [total, H, D] output
 *   sa                 [total, H, D] per-token pre-update sa, or NULL
 *   boundary           [n, H, per_seq, D, D] post-chunk snapshots every
 *                      `blen` tokens of each sequence, or NULL
 */
#define WKV7_BODY(REAL, RET)                                                  \
  {                                                                           \
    const int64_t t0 = cu[s], t1 = cu[s + 1];                                 \
    const int64_t slot = slots ? slots[s] : s;                                \
    REAL* S = (REAL*)malloc(sizeof(REAL) * D * D);                            \
    REAL* w = (REAL*)malloc(sizeof(REAL) * D);                                \
    REAL* sav = (REAL*)malloc(sizeof(REAL) * D);                              \
    REAL* st = state ? state + (slot * H + h) * (int64_t)D * D : NULL;       \
    for (int64_t i = 0; i < (int64_t)D * D; ++i) S[i] = st ? st[i] : 0;      \
    for (int64_t t = t0; t < t1; ++t) {                                       \
      const int64_t o = (t * H + h) * (int64_t)D;                             \
      for (int kk = 0; kk < D; ++kk) {                                        \
        REAL x = (REAL)logits[o + kk];                                        \
        if (bias) x += (REAL)bias[h * D + kk];                                \
        w[kk] = RET(x);                                                       \
      }                                                                       \
      for (int vv = 0; vv < D; ++vv) sav[vv] = 0;                             \
      for (int kk = 0; kk < D; ++kk) {                                        \
        const REAL ak = (REAL)a[o + kk];                                      \
        const REAL* row = S + (int64_t)kk * D;                                \
        for (int vv = 0; vv < D; ++vv) sav[vv] += ak * row[vv];               \
      }                                                                       \
      if (sa)                                                                 \
        for (int vv = 0; vv < D; ++vv) sa[o + vv] = sav[vv];                  \
      for (int kk = 0; kk < D; ++kk) {                                        \
        const REAL wk = w[kk], bk = (REAL)b[o + kk], kv = (REAL)k[o + kk];    \
        REAL* row = S + (int64_t)kk * D;                                      \
        for (int vv = 0; vv < D; ++vv)                                        \
          row[vv] = wk * row[vv] + bk * sav[vv] + kv * (REAL)v[o + vv];       \
      }                                                                       \
      for (int vv = 0; vv < D; ++vv) sav[vv] = 0;                             \
      for (int kk = 0; kk < D; ++kk) {                                        \
        const REAL rk = (REAL)r[o + kk];                                      \
        const REAL* row = S + (int64_t)kk * D;                                \
        for (int vv = 0; vv < D; ++vv) sav[vv] += rk * row[vv];               \
      }                                                                       \
      for (int vv = 0; vv < D; ++vv) y[o + vv] = (REAL)scale * sav[vv];       \
      if (boundary && ((t - t0 + 1) % blen) == 0) {                           \
        const int64_t c = (t - t0 + 1) / blen - 1;                            \
        REAL* bd = boundary + (((int64_t)s * H + h) * per_seq + c) * D * D;  \
        memcpy(bd, S, sizeof(REAL) * D * D);                                  \
      }                                                                       \
    }                                                                         \
    if (st) memcpy(st, S, sizeof(REAL) * D * D);                              \
    free(S);                                                                  \
    free(w);                                                                  \
    free(sav);                                                                \
  }

static double ret_f64(double x) { return wkv7_oracle_retention(x); }
static float ret_f32(float x) { return expf(-0.60653065971263342f / (1.0f + expf(-x))); }

void wkv7_oracle_f64(int n, int H, int D, const int32_t* cu, const int32_t* slots,
                     double* state, const float* r, const float* logits,
                     const float* bias, const float* k, const float* v,
                     const float* a, const float* b, double scale, double* y,
                     double* sa, double* boundary, int blen, int per_seq) {
  for (int s = 0; s < n; ++s)
    for (int h = 0; h < H; ++h) WKV7_BODY(double, ret_f64)
}

void wkv7_cpu_f32(int n, int H, int D, const int32_t* cu, const int32_t* slots,
                  float* state, const float* r, const float* logits,
                  const float* bias, const float* k, const float* v, const float* a,
                  const float* b, double scale, float* y, int threads) {
  float* sa = NULL;
  float* boundary = NULL;
  const int blen = 1, per_seq = 0;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
#endif
  for (int s = 0; s < n; ++s)
    for (int h = 0; h < H; ++h) WKV7_BODY(float, ret_f32)
  (void)threads;
}

int wkv7_cpu_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
