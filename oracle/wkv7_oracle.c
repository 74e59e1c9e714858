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
  /* (sequence, head) pairs are independent (distinct state blocks and output
   * rows), and each is evaluated in the same order whatever the thread
   * count, so the result does not depend on the threading */
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
#endif
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

/*
 * Reverse-mode gradient of the [B,T,H,D] training-layout recurrence with zero
 * initial state (the pretrain path): given dy, returns the gradients of
 * L = sum(y * dy) with respect to r, the decay logits w, k, v, a and b.
 *
 * Restates the backward that csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cu:163-286
 * computes (autograd of tests/tmix/wkv7/pretrain/test.py:44-65 in the
 * reference's own test), derived here from the forward
 *   S_t = diag(w_t) S_{t-1} + b_t sa_t^T + k_t v_t^T,  sa_t = S_{t-1}^T a_t,
 *   y_t = S_t^T r_t,  w_t = exp(-exp(-1/2) sigmoid(logit_t)):
 * with P_t = dL/dS_t (all paths),
 *   P_t  = r_t dy_t^T + (diag(w_{t+1}) + a_{t+1} b_{t+1}^T) P_{t+1}
 *   dr_t = S_t dy_t           dk_t = P_t v_t        dv_t = P_t^T k_t
 *   dsa  = P_t^T b_t          db_t = P_t sa_t       da_t = S_{t-1} dsa
 *   dw_t = rowsum(P_t o S_{t-1}),  dlogit = dw * w * (-exp(-1/2)) s (1 - s).
 * Every state S_t of a (batch, head) is kept (T+1 matrices), so the pass
 * recomputes nothing and divides by nothing.  Double precision throughout.
 */
void wkv7_oracle_pretrain_bwd_f64(int B, int T, int H, int D, const float* r,
                                  const float* logits, const float* k, const float* v,
                                  const float* a, const float* b, const float* dy,
                                  double* dr, double* dlogit, double* dk, double* dv,
                                  double* da, double* db) {
  const int64_t DD = (int64_t)D * D;
  double* S = (double*)malloc(sizeof(double) * DD * (T + 1));
  double* P = (double*)malloc(sizeof(double) * DD);
  double* w = (double*)malloc(sizeof(double) * T * D);
  double* sa = (double*)malloc(sizeof(double) * T * D);
  double* dsa = (double*)malloc(sizeof(double) * D);
  for (int bb = 0; bb < B; ++bb)
    for (int h = 0; h < H; ++h) {
#define OFF(t) ((((int64_t)bb * T + (t)) * H + h) * D)
      memset(S, 0, sizeof(double) * DD);
      for (int t = 0; t < T; ++t) {
        const int64_t o = OFF(t);
        const double* Sp = S + DD * t;
        double* Sn = S + DD * (t + 1);
        for (int i = 0; i < D; ++i) w[t * D + i] = wkv7_oracle_retention(logits[o + i]);
        for (int j = 0; j < D; ++j) {
          double acc = 0;
          for (int i = 0; i < D; ++i) acc += Sp[(int64_t)i * D + j] * a[o + i];
          sa[t * D + j] = acc;
        }
        for (int i = 0; i < D; ++i)
          for (int j = 0; j < D; ++j)
            Sn[(int64_t)i * D + j] = w[t * D + i] * Sp[(int64_t)i * D + j] +
                                     b[o + i] * sa[t * D + j] + (double)k[o + i] * v[o + j];
      }
      memset(P, 0, sizeof(double) * DD);
      for (int t = T - 1; t >= 0; --t) {
        const int64_t o = OFF(t);
        const double* Sp = S + DD * t;
        const double* Sn = S + DD * (t + 1);
        for (int i = 0; i < D; ++i)
          for (int j = 0; j < D; ++j) P[(int64_t)i * D + j] += (double)r[o + i] * dy[o + j];
        for (int i = 0; i < D; ++i) {
          double gr = 0, gk = 0, gb = 0, gw = 0;
          for (int j = 0; j < D; ++j) {
            const double p = P[(int64_t)i * D + j];
            gr += Sn[(int64_t)i * D + j] * dy[o + j];
            gk += p * v[o + j];
            gb += p * sa[t * D + j];
            gw += p * Sp[(int64_t)i * D + j];
          }
          const double sg = 1.0 / (1.0 + exp(-(double)logits[o + i]));
          dr[o + i] = gr;
          dk[o + i] = gk;
          db[o + i] = gb;
          dlogit[o + i] = gw * w[t * D + i] * (-exp(-0.5)) * sg * (1.0 - sg);
        }
        for (int j = 0; j < D; ++j) {
          double gv = 0, gs = 0;
          for (int i = 0; i < D; ++i) {
            gv += P[(int64_t)i * D + j] * k[o + i];
            gs += P[(int64_t)i * D + j] * b[o + i];
          }
          dv[o + j] = gv;
          dsa[j] = gs;
        }
        for (int i = 0; i < D; ++i) {
          double g = 0;
          for (int j = 0; j < D; ++j) g += Sp[(int64_t)i * D + j] * dsa[j];
          da[o + i] = g;
        }
        for (int i = 0; i < D; ++i)
          for (int j = 0; j < D; ++j)
            P[(int64_t)i * D + j] = w[t * D + i] * P[(int64_t)i * D + j] + a[o + i] * dsa[j];
      }
#undef OFF
    }
  free(S);
  free(P);
  free(w);
  free(sa);
  free(dsa);
}

/*
 * StateTune: the recurrence with a trainable initial state, walked over a
 * chunk list (csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_forward.cu:32-131,
 * the reference test's _reference loop tests/tmix/wkv7/statetune/test.py:43-91).
 * Sequence s runs its chunks offsets[s] .. offsets[s+1]-1 in order, chunk c
 * covering tokens [starts[c], ends[c]) of the packed [T,H,D] tensors, from
 * state0[s] ([B,H,D,D], k rows, v columns).  Forward outputs:
 *   y         [T,H,D]   scale * S_t^T r_t           (rows of chunk tokens only)
 *   sa        [T,H,D]   S_{t-1}^T a_t
 *   boundary  [C,H,D,D] the state at the start of chunk c
 *   state_out [B,H,D,D] the state after the sequence's last chunk
 * Backward (dy and/or dfinal may be NULL = zero cotangent): the gradients of
 * L = sum(y * dy) + sum(S_final * dfinal) with respect to r, the decay
 * logits, k, v, a, b (rows of chunk tokens only) and state0 (dstate0), with
 * the adjoint of the pretrain backward above plus
 *   P_final = dfinal,  dr_t = scale * S_t dy_t,  P_t += scale * r_t dy_t^T,
 *   dstate0 = (diag(w_first) + a_first b_first^T) P_first
 * (P carried to before the sequence's first token).  Every state of a
 * sequence is kept; no division.  Double precision throughout.
 */
void wkv7_oracle_statetune_f64(int B, int T, int H, int D, const int32_t* offsets,
                               const int32_t* starts, const int32_t* ends,
                               const float* state0, const float* r, const float* logits,
                               const float* k, const float* v, const float* a,
                               const float* b, double scale, const float* dy,
                               const float* dfinal, double* y, double* sa_out,
                               double* boundary, double* state_out, double* dr,
                               double* dlogit, double* dk, double* dv, double* da,
                               double* db, double* dstate0) {
  const int64_t DD = (int64_t)D * D;
  int32_t* toks = (int32_t*)malloc(sizeof(int32_t) * (T > 0 ? T : 1));
  double* S = (double*)malloc(sizeof(double) * DD * (T + 1));
  double* P = (double*)malloc(sizeof(double) * DD);
  double* w = (double*)malloc(sizeof(double) * D);
  double* sa = (double*)malloc(sizeof(double) * (int64_t)(T > 0 ? T : 1) * D);
  double* dsa = (double*)malloc(sizeof(double) * D);
  for (int s = 0; s < B; ++s)
    for (int h = 0; h < H; ++h) {
      /* the sequence's tokens in execution order */
      int n = 0;
      for (int c = offsets[s]; c < offsets[s + 1]; ++c)
        for (int t = starts[c]; t < ends[c]; ++t) toks[n++] = t;
      const float* s0 = state0 + ((int64_t)s * H + h) * DD;
      for (int64_t e = 0; e < DD; ++e) S[e] = s0[e];
      int m = 0;
      for (int c = offsets[s]; c < offsets[s + 1]; ++c) {
        memcpy(boundary + ((int64_t)c * H + h) * DD, S + DD * m, sizeof(double) * DD);
        for (int t = starts[c]; t < ends[c]; ++t, ++m) {
          const int64_t o = ((int64_t)t * H + h) * D;
          const double* Sp = S + DD * m;
          double* Sn = S + DD * (m + 1);
          for (int i = 0; i < D; ++i) w[i] = wkv7_oracle_retention(logits[o + i]);
          for (int j = 0; j < D; ++j) {
            double acc = 0;
            for (int i = 0; i < D; ++i) acc += Sp[(int64_t)i * D + j] * a[o + i];
            sa[(int64_t)m * D + j] = acc;
            sa_out[o + j] = acc;
          }
          for (int i = 0; i < D; ++i)
            for (int j = 0; j < D; ++j)
              Sn[(int64_t)i * D + j] = w[i] * Sp[(int64_t)i * D + j] +
                                       b[o + i] * sa[(int64_t)m * D + j] +
                                       (double)k[o + i] * v[o + j];
          for (int j = 0; j < D; ++j) {
            double acc = 0;
            for (int i = 0; i < D; ++i) acc += (double)r[o + i] * Sn[(int64_t)i * D + j];
            y[o + j] = scale * acc;
          }
        }
      }
      memcpy(state_out + ((int64_t)s * H + h) * DD, S + DD * n, sizeof(double) * DD);
      /* backward */
      for (int64_t e = 0; e < DD; ++e)
        P[e] = dfinal ? dfinal[((int64_t)s * H + h) * DD + e] : 0.0;
      for (m = n - 1; m >= 0; --m) {
        const int t = toks[m];
        const int64_t o = ((int64_t)t * H + h) * D;
        const double* Sp = S + DD * m;
        const double* Sn = S + DD * (m + 1);
        for (int i = 0; i < D; ++i) w[i] = wkv7_oracle_retention(logits[o + i]);
        if (dy)
          for (int i = 0; i < D; ++i)
            for (int j = 0; j < D; ++j)
              P[(int64_t)i * D + j] += scale * (double)r[o + i] * dy[o + j];
        for (int i = 0; i < D; ++i) {
          double gr = 0, gk = 0, gb = 0, gw = 0;
          for (int j = 0; j < D; ++j) {
            const double p = P[(int64_t)i * D + j];
            if (dy) gr += Sn[(int64_t)i * D + j] * dy[o + j];
            gk += p * v[o + j];
            gb += p * sa[(int64_t)m * D + j];
            gw += p * Sp[(int64_t)i * D + j];
          }
          const double sg = 1.0 / (1.0 + exp(-(double)logits[o + i]));
          dr[o + i] = scale * gr;
          dk[o + i] = gk;
          db[o + i] = gb;
          dlogit[o + i] = gw * w[i] * (-exp(-0.5)) * sg * (1.0 - sg);
        }
        for (int j = 0; j < D; ++j) {
          double gv = 0, gs = 0;
          for (int i = 0; i < D; ++i) {
            gv += P[(int64_t)i * D + j] * k[o + i];
            gs += P[(int64_t)i * D + j] * b[o + i];
          }
          dv[o + j] = gv;
          dsa[j] = gs;
        }
        for (int i = 0; i < D; ++i) {
          double g = 0;
          for (int j = 0; j < D; ++j) g += Sp[(int64_t)i * D + j] * dsa[j];
          da[o + i] = g;
        }
        for (int i = 0; i < D; ++i)
          for (int j = 0; j < D; ++j)
            P[(int64_t)i * D + j] = w[i] * P[(int64_t)i * D + j] + a[o + i] * dsa[j];
      }
      memcpy(dstate0 + ((int64_t)s * H + h) * DD, P, sizeof(double) * DD);
    }
  free(toks);
  free(S);
  free(P);
  free(w);
  free(sa);
  free(dsa);
}
