// StateTune: the WKV7 recurrence from a trainable initial state, walked over
// a chunk list, and its training backward (initial-state gradient included).
// Replaces statetune_tmix_wkv7_recurrent_fp32io16_forward_kernel and
// statetune_tmix_wkv7_recurrent_fp32io16_backward{,_large}_kernel
// (csrc/sm120/tmix/wkv7/statetune_recurrent_fp32io16_forward.cu:32-131,
//  statetune_recurrent_fp32io16_backward.cu:49-255 and 317-502).
//
// Sequence s runs chunks offsets[s] .. offsets[s+1]-1 in order; chunk c
// covers the token rows [starts[c], ends[c]) of the packed [T,H,D] tensors.
// The forward writes y = scale * S_t^T r_t, sa_t = S_{t-1}^T a_t, the state
// at the start of every chunk (boundary [C,H,D,D]) and the final state in
// place.
//
// Work layout.  Every pass splits a (sequence, head) over G = D^2/4096
// workgroups of 256 lanes; each workgroup owns 4096/D "lines" (state columns
// for the column passes, rows for the row pass) with L = D/16 lanes per line,
// each lane holding E = 16 consecutive elements of its line; reductions
// along a line are DPP sums over its L lanes.  The token operands of a tile
// of TT tokens are staged through LDS as fp32 (TT = 16, 8 at D = 256); the
// LDS reads are broadcasts, the L lanes of a line reading disjoint slices.
//
// Backward, with P_t = dL/dS_t:
//   P_t   = scale r_t dy_t^T + (diag(w_{t+1}) + a_{t+1} b_{t+1}^T) P_{t+1},
//   P_end = dL/dS_final,  dL/dS_init = (diag(w_first) + a b^T) P_first.
// The column recurrence of P is local to a column once dsa = P^T b is known,
// and the row recurrences of S and P are local to a row once dsa is known,
// so the backward is three launches:
//   1. replay: every chunk reruns the forward from its boundary state (chunks
//      in parallel) and keeps the state at each TT-aligned token inside the
//      chunk, so the row pass never walks S back more than TT/2 - 1 tokens;
//   2. value pass (columns): P columns backwards in time -> dv, dsa;
//   3. key pass (rows): per tile, rebuild S forward from the tile's start
//      state (chunk boundary or replay snapshot), keeping the middle state;
//      then walk backwards with P rows -> dr, dw, dk, db, da, and finally
//      dL/dS_init.
#include "recurrent.h"

namespace fr2 {
namespace {

constexpr float kWScale = -0.6065306597126334f;  // -exp(-1/2)
constexpr int kThreads = 256;

template <int D>
struct St {
  // lanes per line (16 elements each); 16 lanes per line at every D (D/16
  // elements each) measured ~6 % slower at D = 64: the per-token chain is
  // reduction and LDS latency, not element work
  static constexpr int L = D / 16;
  static constexpr int E = D / L;                 // elements per lane
  static constexpr int LINES = kThreads / L;      // lines per workgroup
  static constexpr int G = D / LINES;             // workgroups per (seq, head)
  static constexpr int TT = D == 256 ? 8 : 16;    // tokens per tile
};

// sum over the L lanes of a line (aligned groups of L inside a 16-lane row)
template <int L>
__device__ __forceinline__ float line_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
  if constexpr (L >= 8)   // row_half_mirror: lane i <- lane 7-i within 8
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xf, 0xf, false));
  if constexpr (L >= 16)  // row_mirror: lane i <- lane 15-i
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xf, 0xf, false));
  return x;
}

template <int E>
__device__ __forceinline__ void lds16(const float* src, float* dst) {
#pragma unroll
  for (int x = 0; x < E; x += 4) {
    const f4 v = *reinterpret_cast<const f4*>(src + x);
    dst[x] = v[0]; dst[x + 1] = v[1]; dst[x + 2] = v[2]; dst[x + 3] = v[3];
  }
}

template <int E>
__device__ __forceinline__ void store16(float* dst, const float* src) {
#pragma unroll
  for (int x = 0; x < E; x += 4) {
    f4 v;
    v[0] = src[x]; v[1] = src[x + 1]; v[2] = src[x + 2]; v[3] = src[x + 3];
    *reinterpret_cast<f4*>(dst + x) = v;
  }
}

// 8 consecutive token elements (16-byte aligned) widened to fp32
template <class Io>
__device__ __forceinline__ void ld8(const void* base, int64_t off, float* f) {
  const Raw8 x =
      *reinterpret_cast<const Raw8*>(static_cast<const typename Io::raw*>(base) + off);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = raw8_get<Io>(x, i);
}

__device__ __forceinline__ void st8(float* dst, const float* f) {
  f4 lo, hi;
  lo[0] = f[0]; lo[1] = f[1]; lo[2] = f[2]; lo[3] = f[3];
  hi[0] = f[4]; hi[1] = f[5]; hi[2] = f[6]; hi[3] = f[7];
  *reinterpret_cast<f4*>(dst) = lo;
  *reinterpret_cast<f4*>(dst + 4) = hi;
}

__device__ __forceinline__ int clampi(int x, int lo, int hi) { return min(max(x, lo), hi); }

// Chunk c's token range and sequence s's chunk range, clamped so that any
// metadata stays inside the tensors.
__device__ __forceinline__ void chunk_range(const StateTuneArgs& p, int c, int& s, int& e) {
  const int T = static_cast<int>(p.tokens);
  s = clampi(p.starts[c], 0, T);
  e = clampi(p.ends[c], s, T);
}
__device__ __forceinline__ void seq_chunks(const StateTuneArgs& p, int seq, int& c0, int& c1) {
  c0 = clampi(p.offsets[seq], 0, p.num_chunks);
  c1 = clampi(p.offsets[seq + 1], c0, p.num_chunks);
}

// ---------------------------------------------------------------------------
// forward (kReplay = false: one workgroup per (sequence, head, column group))
// and replay (kReplay = true: one per (chunk, head, column group), from the
// chunk's boundary state, writing only the TT-aligned snapshots)
// ---------------------------------------------------------------------------
template <int D, class Io, bool kReplay>
__global__ __launch_bounds__(kThreads) void st_forward_kernel(StateTuneArgs p) {
  using C = St<D>;
  constexpr int L = C::L, E = C::E, LINES = C::LINES, G = C::G, TT = C::TT;
  constexpr int UF = D / 8, UP = LINES / 8, UT = 5 * UF + UP;
  __shared__ __align__(16) float tok[TT][5][D];   // r, w (retention), k, a, b
  __shared__ __align__(16) float vv[TT][LINES];   // v on this group's columns

  const int g = blockIdx.x % G;
  const int h = (blockIdx.x / G) % p.heads;
  const int unit = blockIdx.x / (G * p.heads);
  const int tid = threadIdx.x, line = tid / L, q = tid % L;
  const int j = g * LINES + line;
  const int64_t DD = static_cast<int64_t>(D) * D;
  const int64_t stride = static_cast<int64_t>(p.heads) * D;
  const void* const srcs[5] = {p.r, p.w, p.k, p.a, p.b};
  using raw = typename Io::raw;

  int c0, c1;
  const float* sin;
  if constexpr (kReplay) {
    c0 = unit;
    c1 = unit + 1;
    sin = p.boundary + (static_cast<int64_t>(unit) * p.heads + h) * DD;
  } else {
    seq_chunks(p, unit, c0, c1);
    sin = p.state + (static_cast<int64_t>(unit) * p.heads + h) * DD;
  }
  const int64_t col = static_cast<int64_t>(q) * E * D + j;   // element (qE, j)
  float S[E];
#pragma unroll
  for (int e = 0; e < E; ++e) S[e] = sin[col + e * D];

  for (int c = c0; c < c1; ++c) {
    int s, e;
    chunk_range(p, c, s, e);
    if constexpr (!kReplay) {
      float* bd = p.boundary + (static_cast<int64_t>(c) * p.heads + h) * DD + col;
#pragma unroll
      for (int x = 0; x < E; ++x) bd[x * D] = S[x];
    }
    for (int t0 = s; t0 < e;) {
      const int tn = min(e, (t0 / TT + 1) * TT);
      const int n = tn - t0;
      if constexpr (kReplay) {
        if (t0 > s) {
          float* sp = p.snap + (static_cast<int64_t>(t0 / TT) * p.heads + h) * DD + col;
#pragma unroll
          for (int x = 0; x < E; ++x) sp[x * D] = S[x];
        }
      }
      __syncthreads();   // the previous tile's LDS reads are done
      for (int u = tid; u < n * UT; u += kThreads) {
        const int tt = u / UT, rem = u % UT;
        const int64_t row = (t0 + tt) * stride + static_cast<int64_t>(h) * D;
        float f[8];
        if (rem < 5 * UF) {
          const int m = rem / UF, gg = rem % UF;
          ld8<Io>(srcs[m], row + 8 * gg, f);
          if (m == 1) {
#pragma unroll
            for (int x = 0; x < 8; ++x) f[x] = retention_from_logit(f[x]);
          }
          st8(&tok[tt][m][8 * gg], f);
        } else {
          const int gg = rem - 5 * UF;
          ld8<Io>(p.v, row + g * LINES + 8 * gg, f);
          st8(&vv[tt][8 * gg], f);
        }
      }
      __syncthreads();
      for (int tt = 0; tt < n; ++tt) {
        float A[E], W[E], B[E], K[E];
        lds16<E>(&tok[tt][3][q * E], A);
        float sp = 0.0f;
#pragma unroll
        for (int x = 0; x < E; ++x) sp = fmaf(A[x], S[x], sp);
        const float sa = line_sum<L>(sp);
        lds16<E>(&tok[tt][1][q * E], W);
        lds16<E>(&tok[tt][4][q * E], B);
        lds16<E>(&tok[tt][2][q * E], K);
        const float vj = vv[tt][line];
#pragma unroll
        for (int x = 0; x < E; ++x) S[x] = fmaf(K[x], vj, fmaf(B[x], sa, W[x] * S[x]));
        if constexpr (!kReplay) {
          float R[E];
          lds16<E>(&tok[tt][0][q * E], R);
          float yp = 0.0f;
#pragma unroll
          for (int x = 0; x < E; ++x) yp = fmaf(R[x], S[x], yp);
          const float yv = line_sum<L>(yp);
          const int64_t o = (t0 + tt) * stride + static_cast<int64_t>(h) * D + j;
          if (q == 0) static_cast<raw*>(p.y)[o] = Io::from_f32(p.scale * yv);
          if (q == 1) p.sa[o] = sa;
        }
      }
      t0 = tn;
    }
  }
  if constexpr (!kReplay) {
    float* so = p.state + (static_cast<int64_t>(unit) * p.heads + h) * DD + col;
#pragma unroll
    for (int x = 0; x < E; ++x) so[x * D] = S[x];
  }
}

// ---------------------------------------------------------------------------
// value pass: P columns backwards over the sequence -> dv, dsa
// ---------------------------------------------------------------------------
template <int D, class Io>
__global__ __launch_bounds__(kThreads) void st_value_kernel(StateTuneArgs p) {
  using C = St<D>;
  constexpr int L = C::L, E = C::E, LINES = C::LINES, G = C::G, TT = C::TT;
  constexpr int UF = D / 8, UP = LINES / 8, UT = 5 * UF + UP;
  __shared__ __align__(16) float tok[TT][5][D];   // r, w (retention), k, a, b
  __shared__ __align__(16) float dyv[TT][LINES];  // dy on this group's columns

  const int g = blockIdx.x % G;
  const int h = (blockIdx.x / G) % p.heads;
  const int seq = blockIdx.x / (G * p.heads);
  const int tid = threadIdx.x, line = tid / L, q = tid % L;
  const int j = g * LINES + line;
  const int64_t DD = static_cast<int64_t>(D) * D;
  const int64_t stride = static_cast<int64_t>(p.heads) * D;
  const void* const srcs[5] = {p.r, p.w, p.k, p.a, p.b};
  using raw = typename Io::raw;

  const int64_t col = static_cast<int64_t>(q) * E * D + j;
  float P[E];
  const float* pf = p.dfinal ? p.dfinal + (static_cast<int64_t>(seq) * p.heads + h) * DD + col
                             : nullptr;
#pragma unroll
  for (int x = 0; x < E; ++x) P[x] = pf ? pf[x * D] : 0.0f;

  int c0, c1;
  seq_chunks(p, seq, c0, c1);
  for (int c = c1 - 1; c >= c0; --c) {
    int s, e;
    chunk_range(p, c, s, e);
    for (int te = e; te > s;) {
      const int t0 = max(s, ((te - 1) / TT) * TT);
      const int n = te - t0;
      __syncthreads();
      for (int u = tid; u < n * UT; u += kThreads) {
        const int tt = u / UT, rem = u % UT;
        const int64_t row = (t0 + tt) * stride + static_cast<int64_t>(h) * D;
        float f[8];
        if (rem < 5 * UF) {
          const int m = rem / UF, gg = rem % UF;
          ld8<Io>(srcs[m], row + 8 * gg, f);
          if (m == 1) {
#pragma unroll
            for (int x = 0; x < 8; ++x) f[x] = retention_from_logit(f[x]);
          }
          st8(&tok[tt][m][8 * gg], f);
        } else {
          const int gg = rem - 5 * UF;
          if (p.dy != nullptr) {
            ld8<Io>(p.dy, row + g * LINES + 8 * gg, f);
          } else {
#pragma unroll
            for (int x = 0; x < 8; ++x) f[x] = 0.0f;
          }
          st8(&dyv[tt][8 * gg], f);
        }
      }
      __syncthreads();
      for (int tt = n - 1; tt >= 0; --tt) {
        float R[E], K[E], B[E];
        lds16<E>(&tok[tt][0][q * E], R);
        const float sdy = p.scale * dyv[tt][line];
#pragma unroll
        for (int x = 0; x < E; ++x) P[x] = fmaf(R[x], sdy, P[x]);
        lds16<E>(&tok[tt][2][q * E], K);
        lds16<E>(&tok[tt][4][q * E], B);
        float vp = 0.0f, dp = 0.0f;
#pragma unroll
        for (int x = 0; x < E; ++x) {
          vp = fmaf(K[x], P[x], vp);
          dp = fmaf(B[x], P[x], dp);
        }
        const float dvj = line_sum<L>(vp);
        const float dsj = line_sum<L>(dp);
        const int64_t o = (t0 + tt) * stride + static_cast<int64_t>(h) * D + j;
        if (q == 0 && p.dv != nullptr) static_cast<raw*>(p.dv)[o] = Io::from_f32(dvj);
        if (q == 1) p.dsa[o] = dsj;
        float W[E], A[E];
        lds16<E>(&tok[tt][1][q * E], W);
        lds16<E>(&tok[tt][3][q * E], A);
#pragma unroll
        for (int x = 0; x < E; ++x) P[x] = fmaf(W[x], P[x], A[x] * dsj);
      }
      te = t0;
    }
  }
}

// ---------------------------------------------------------------------------
// key pass: S and P rows backwards over the sequence -> dr dw dk db da, dS0
// ---------------------------------------------------------------------------
template <int D, class Io>
__global__ __launch_bounds__(kThreads) void st_key_kernel(StateTuneArgs p) {
  using C = St<D>;
  constexpr int L = C::L, E = C::E, LINES = C::LINES, G = C::G, TT = C::TT;
  constexpr int UB = D / 8, UF = D / 4, UR = LINES / 8;
  constexpr int UT = 2 * UB + 2 * UF + 5 * UR;
  __shared__ __align__(16) float vec[TT][4][D];       // dy, v, sa, dsa
  __shared__ __align__(16) float rows[TT][6][LINES];  // r, w, k, a, b, dw/dlogit factor

  const int g = blockIdx.x % G;
  const int h = (blockIdx.x / G) % p.heads;
  const int seq = blockIdx.x / (G * p.heads);
  const int tid = threadIdx.x, line = tid / L, q = tid % L;
  const int i = g * LINES + line;                     // key row
  const int64_t DD = static_cast<int64_t>(D) * D;
  const int64_t stride = static_cast<int64_t>(p.heads) * D;
  const void* const rsrc[5] = {p.r, p.w, p.k, p.a, p.b};
  using raw = typename Io::raw;

  const int64_t rowoff = static_cast<int64_t>(i) * D + q * E;   // element (i, qE)
  float P[E];
  if (p.dfinal != nullptr) {
    lds16<E>(p.dfinal + (static_cast<int64_t>(seq) * p.heads + h) * DD + rowoff, P);
  } else {
#pragma unroll
    for (int x = 0; x < E; ++x) P[x] = 0.0f;
  }

  int c0, c1;
  seq_chunks(p, seq, c0, c1);
  for (int c = c1 - 1; c >= c0; --c) {
    int s, e;
    chunk_range(p, c, s, e);
    for (int te = e; te > s;) {
      const int t0 = max(s, ((te - 1) / TT) * TT);
      const int n = te - t0;
      __syncthreads();
      for (int u = tid; u < n * UT; u += kThreads) {
        const int tt = u / UT, rem = u % UT;
        const int64_t row = (t0 + tt) * stride + static_cast<int64_t>(h) * D;
        float f[8];
        if (rem < 2 * UB) {
          const int m = rem / UB, gg = rem % UB;
          const void* src = m == 0 ? p.dy : p.v;
          if (src != nullptr) {
            ld8<Io>(src, row + 8 * gg, f);
          } else {
#pragma unroll
            for (int x = 0; x < 8; ++x) f[x] = 0.0f;
          }
          st8(&vec[tt][m][8 * gg], f);
        } else if (rem < 2 * UB + 2 * UF) {
          const int r2 = rem - 2 * UB, m = r2 / UF, gg = r2 % UF;
          const float* src = (m == 0 ? p.sa : p.dsa) + row + 4 * gg;
          *reinterpret_cast<f4*>(&vec[tt][2 + m][4 * gg]) = *reinterpret_cast<const f4*>(src);
        } else {
          const int r3 = rem - 2 * UB - 2 * UF, m = r3 / UR, gg = r3 % UR;
          ld8<Io>(rsrc[m], row + g * LINES + 8 * gg, f);
          if (m == 1) {
            float fs[8];
#pragma unroll
            for (int x = 0; x < 8; ++x) {
              const float sg = 1.0f / (1.0f + __builtin_amdgcn_exp2f(kNegLog2e * f[x]));
              const float w = retention_from_logit(f[x]);
              fs[x] = kWScale * w * sg * (1.0f - sg);
              f[x] = w;
            }
            st8(&rows[tt][5][8 * gg], fs);
          }
          st8(&rows[tt][m][8 * gg], f);
        }
      }
      __syncthreads();

      // the tile's start state: the chunk's boundary or the replay snapshot
      const float* org = t0 == s
          ? p.boundary + (static_cast<int64_t>(c) * p.heads + h) * DD + rowoff
          : p.snap + (static_cast<int64_t>(t0 / TT) * p.heads + h) * DD + rowoff;
      float Org[E], Mid[E], S[E];
      lds16<E>(org, Org);
      // rebuild forwards (the forward's own arithmetic), keeping the state
      // after token m-1
      const int m = n / 2;
#pragma unroll
      for (int x = 0; x < E; ++x) {
        S[x] = Org[x];
        Mid[x] = Org[x];
      }
      for (int tt = 0; tt < n; ++tt) {
        const float wi = rows[tt][1][line], ki = rows[tt][2][line], bi = rows[tt][4][line];
        float V[E], SA[E];
        lds16<E>(&vec[tt][1][q * E], V);
        lds16<E>(&vec[tt][2][q * E], SA);
#pragma unroll
        for (int x = 0; x < E; ++x) S[x] = fmaf(ki, V[x], fmaf(bi, SA[x], wi * S[x]));
        if (tt == m - 1) {
#pragma unroll
          for (int x = 0; x < E; ++x) Mid[x] = S[x];
        }
      }
      // walk backwards: S is S_t (post-update), P is carried to P_t
      for (int tt = n - 1; tt >= 0; --tt) {
        const float ri = rows[tt][0][line], wi = rows[tt][1][line];
        const float ki = rows[tt][2][line], ai = rows[tt][3][line];
        const float bi = rows[tt][4][line], wsi = rows[tt][5][line];
        float DY[E], V[E], SA[E], DS[E];
        lds16<E>(&vec[tt][0][q * E], DY);
        lds16<E>(&vec[tt][1][q * E], V);
        lds16<E>(&vec[tt][2][q * E], SA);
        lds16<E>(&vec[tt][3][q * E], DS);
        const float sri = p.scale * ri;
        float pr = 0.0f, pk = 0.0f, pb = 0.0f;
#pragma unroll
        for (int x = 0; x < E; ++x) {
          P[x] = fmaf(sri, DY[x], P[x]);
          pr = fmaf(S[x], DY[x], pr);
          pk = fmaf(P[x], V[x], pk);
          pb = fmaf(P[x], SA[x], pb);
        }
        if (tt == 0) {
#pragma unroll
          for (int x = 0; x < E; ++x) S[x] = Org[x];
        } else if (tt == m) {
#pragma unroll
          for (int x = 0; x < E; ++x) S[x] = Mid[x];
        } else {
          const float rw = __builtin_amdgcn_rcpf(wi);
#pragma unroll
          for (int x = 0; x < E; ++x) S[x] = (S[x] - ki * V[x] - bi * SA[x]) * rw;
        }
        float pa = 0.0f, pw = 0.0f;
#pragma unroll
        for (int x = 0; x < E; ++x) {
          pa = fmaf(S[x], DS[x], pa);
          pw = fmaf(P[x], S[x], pw);
        }
        pr = line_sum<L>(pr);
        pk = line_sum<L>(pk);
        pb = line_sum<L>(pb);
        pa = line_sum<L>(pa);
        pw = line_sum<L>(pw);
        const int64_t o = (t0 + tt) * stride + static_cast<int64_t>(h) * D + i;
        if (q == 0) {
          if (p.dr != nullptr) static_cast<raw*>(p.dr)[o] = Io::from_f32(p.scale * pr);
          if (p.da != nullptr) static_cast<raw*>(p.da)[o] = Io::from_f32(pa);
        } else if (q == 1) {
          if (p.dw != nullptr) static_cast<raw*>(p.dw)[o] = Io::from_f32(pw * wsi);
        } else if (q == 2) {
          if (p.dk != nullptr) static_cast<raw*>(p.dk)[o] = Io::from_f32(pk);
        } else if (q == 3) {
          if (p.db != nullptr) static_cast<raw*>(p.db)[o] = Io::from_f32(pb);
        }
#pragma unroll
        for (int x = 0; x < E; ++x) P[x] = fmaf(wi, P[x], ai * DS[x]);
      }
      te = t0;
    }
  }
  if (p.dstate0 != nullptr)
    store16<E>(p.dstate0 + (static_cast<int64_t>(seq) * p.heads + h) * DD + rowoff, P);
}

template <int D, class Io>
int forward_d(const StateTuneArgs& p, hipStream_t s) {
  constexpr int G = St<D>::G;
  const int64_t blocks = static_cast<int64_t>(p.num_seq) * p.heads * G;
  if (blocks > 0x7fffffff) return FR2_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL((st_forward_kernel<D, Io, false>), dim3(blocks), dim3(kThreads), 0, s, p);
  return record_launch();
}

template <int D, class Io>
int backward_d(const StateTuneArgs& p, hipStream_t s) {
  constexpr int G = St<D>::G;
  const int64_t seq_blocks = static_cast<int64_t>(p.num_seq) * p.heads * G;
  const int64_t chunk_blocks = static_cast<int64_t>(p.num_chunks) * p.heads * G;
  if (seq_blocks > 0x7fffffff || chunk_blocks > 0x7fffffff) return FR2_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL((st_forward_kernel<D, Io, true>), dim3(chunk_blocks), dim3(kThreads), 0, s,
                     p);
  hipLaunchKernelGGL((st_value_kernel<D, Io>), dim3(seq_blocks), dim3(kThreads), 0, s, p);
  hipLaunchKernelGGL((st_key_kernel<D, Io>), dim3(seq_blocks), dim3(kThreads), 0, s, p);
  return record_launch();
}

// boundary[b * nck + j] (the state at the start of chunk j of sequence b,
// chunks of chunk_len tokens): j = 0 from state (before the forward runs),
// j > 0 from the post-16-token snapshot that ends at token j * chunk_len
__global__ __launch_bounds__(256) void st_gather_kernel(int H, int nck, int chunk_len,
                                                         bool first, const float* state,
                                                         const float* snap, int snaps_per_seq,
                                                         float* boundary) {
  constexpr int DD = 64 * 64;
  const int c = blockIdx.x / H, h = blockIdx.x % H;
  const int b = c / nck, j = c % nck;
  if ((j == 0) != first) return;
  const float* src =
      j == 0 ? state + (static_cast<int64_t>(b) * H + h) * DD
             : snap + ((static_cast<int64_t>(b) * H + h) * snaps_per_seq + j * chunk_len / 16 - 1) *
                          DD;
  float* dst = boundary + static_cast<int64_t>(blockIdx.x) * DD;
  for (int x = threadIdx.x; x < DD / 4; x += 256)
    reinterpret_cast<f4*>(dst)[x] = reinterpret_cast<const f4*>(src)[x];
}

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// ---- ragged chunk lists on the chunked kernels (the padded layout) ----
// Each sequence's chunks are laid out back to back in a [B, Tp] token grid,
// every chunk starting on a 16-token boundary; the rows in between (and at
// the end of a sequence) hold identity tokens (r = k = v = a = b = 0 and a
// decay logit of -80, whose retention is exactly 1 in fp32), which leave the
// state, and the backward's adjoint, exactly unchanged.  row_source[pr] is
// the packed token row of padded row pr, or -1 for an identity row.

// dst[n][pr] = src[n][row_source[pr]] (16-byte pieces of a row of row_bytes),
// or the fill pattern for identity rows; n < ntens.
struct PadRowsArgs {
  const void* src[8];
  void* dst[8];
  uint32_t fill[8];   // 32-bit fill pattern of identity rows
  int ntens = 0;
};
__global__ __launch_bounds__(256) void pad_rows_kernel(PadRowsArgs a, const int32_t* row_source,
                                                       int64_t rows, int row_pieces) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= rows * row_pieces) return;
  const int64_t pr = idx / row_pieces;
  const int piece = static_cast<int>(idx - pr * row_pieces);
  const int32_t srow = row_source[pr];
  for (int n = 0; n < a.ntens; ++n) {
    u4 val;
    if (srow >= 0) {
      val = reinterpret_cast<const u4*>(a.src[n])[static_cast<int64_t>(srow) * row_pieces + piece];
    } else {
      val = u4{a.fill[n], a.fill[n], a.fill[n], a.fill[n]};
    }
    reinterpret_cast<u4*>(a.dst[n])[pr * row_pieces + piece] = val;
  }
}
// dst[n][row_source[pr]] = src[n][pr] for the rows that have a source
__global__ __launch_bounds__(256) void unpad_rows_kernel(PadRowsArgs a, const int32_t* row_source,
                                                         int64_t rows, int row_pieces) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= rows * row_pieces) return;
  const int64_t pr = idx / row_pieces;
  const int piece = static_cast<int>(idx - pr * row_pieces);
  const int32_t srow = row_source[pr];
  if (srow < 0) return;
  for (int n = 0; n < a.ntens; ++n)
    reinterpret_cast<u4*>(a.dst[n])[static_cast<int64_t>(srow) * row_pieces + piece] =
        reinterpret_cast<const u4*>(a.src[n])[pr * row_pieces + piece];
}

// boundary[c] = the state at padded position chunk_pstart[c] of sequence
// chunk_seq[c]: the initial state when that is 0 (first pass, before the
// forward replaces it), else the post-16-token snapshot ending there
__global__ __launch_bounds__(256) void st_gather_padded_kernel(
    int H, const int32_t* chunk_seq, const int32_t* chunk_pstart, bool first, const float* state,
    const float* snap, int snaps_per_seq, float* boundary) {
  constexpr int DD = 64 * 64;
  const int c = blockIdx.x / H, h = blockIdx.x % H;
  const int b = chunk_seq[c], ps = chunk_pstart[c];
  if ((ps == 0) != first) return;
  const float* src =
      ps == 0 ? state + (static_cast<int64_t>(b) * H + h) * DD
              : snap + ((static_cast<int64_t>(b) * H + h) * snaps_per_seq + ps / 16 - 1) * DD;
  float* dst = boundary + static_cast<int64_t>(blockIdx.x) * DD;
  for (int x = threadIdx.x; x < DD / 4; x += 256)
    reinterpret_cast<f4*>(dst)[x] = reinterpret_cast<const f4*>(src)[x];
}

// init[b] = boundary[seq_first_chunk[b]] (its initial state), or zeros for a
// sequence without chunks (its rows are all identity tokens)
__global__ __launch_bounds__(256) void st_initial_states_kernel(int H,
                                                                const int32_t* seq_first_chunk,
                                                                const float* boundary,
                                                                float* init) {
  constexpr int DD = 64 * 64;
  const int b = blockIdx.x / H, h = blockIdx.x % H;
  const int c = seq_first_chunk[b];
  float* dst = init + static_cast<int64_t>(blockIdx.x) * DD;
  for (int x = threadIdx.x; x < DD / 4; x += 256)
    reinterpret_cast<f4*>(dst)[x] =
        c >= 0 ? reinterpret_cast<const f4*>(boundary + (static_cast<int64_t>(c) * H + h) * DD)[x]
               : f4{0.f, 0.f, 0.f, 0.f};
}

// bf16 fill patterns of the identity rows
constexpr uint32_t kZeroPair = 0u;
constexpr uint32_t kIdentityLogitPair = 0xC2A0C2A0u;   // bf16 -80.0 twice

int pad_rows(const PadRowsArgs& a, const int32_t* row_source, int64_t rows, int row_pieces,
             bool unpad, hipStream_t s) {
  const int64_t n = rows * row_pieces;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffff) return FR2_ERR_INVALID_ARGUMENT;
  if (unpad)
    hipLaunchKernelGGL(unpad_rows_kernel, dim3(blocks), dim3(256), 0, s, a, row_source, rows,
                       row_pieces);
  else
    hipLaunchKernelGGL(pad_rows_kernel, dim3(blocks), dim3(256), 0, s, a, row_source, rows,
                       row_pieces);
  return FR2_OK;
}

}  // namespace

int launch_statetune_uniform_forward(int B, int T, int H, int chunk_len, const StateTuneArgs& a,
                                     float* snap, hipStream_t s) {
  const int nck = T / chunk_len;
  const int64_t blocks = static_cast<int64_t>(B) * nck * H;
  if (blocks > 0x7fffffff) return FR2_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(st_gather_kernel, dim3(blocks), dim3(256), 0, s, H, nck, chunk_len, true,
                     a.state, snap, T / 16, a.boundary);
  SegArgs v;
  v.uniform_len = T;
  v.num_heads = H;
  v.out_elems = static_cast<int64_t>(B) * T * H * 64;
  v.state_in = a.state;
  v.state_out = a.state;
  v.r = a.r; v.logits = a.w; v.k = a.k; v.v = a.v; v.a = a.a; v.b = a.b;
  v.y = a.y;
  v.sa_out = a.sa;
  v.boundary = snap;
  v.boundary_len = 16;
  v.boundary_per_seg = T / 16;
  v.scale = a.scale;
  const int rc = launch_chunked(FR2_DTYPE_BFLOAT16, v, B, T, s);
  if (rc != FR2_OK) return rc;
  hipLaunchKernelGGL(st_gather_kernel, dim3(blocks), dim3(256), 0, s, H, nck, chunk_len, false,
                     a.state, snap, T / 16, a.boundary);
  return record_launch();
}

int launch_statetune_uniform_backward(int B, int T, int H, int chunk_len, const StateTuneArgs& a,
                                      const float* snap, float* workspace, hipStream_t s) {
  PretrainBwdArgs p;
  p.batch = B; p.tokens = T; p.heads = H;
  p.r = a.r; p.w = a.w; p.k = a.k; p.v = a.v; p.a = a.a; p.b = a.b; p.dy = a.dy;
  p.boundary = snap;
  p.state_dot_a = a.sa;
  p.workspace = workspace;
  p.dr = a.dr; p.dw = a.dw; p.dk = a.dk; p.dv = a.dv; p.da = a.da; p.db = a.db;
  p.scale = a.scale;
  p.state0 = a.boundary;   // chunk 0 of sequence b is boundary[b * nck]
  p.state0_stride = static_cast<int64_t>(T / chunk_len) * H * 64 * 64;
  p.dfinal = a.dfinal;
  p.dstate0 = a.dstate0;
  p.pfirst = workspace + pretrain_backward_workspace_floats(B, T, H, 64);
  return launch_pretrain_backward(64, p, s);
}

int64_t statetune_backward_workspace_floats(int64_t T, int H, int D) {
  const int TT = D == 256 ? 8 : 16;
  return T * H * D + ((T + TT - 1) / TT) * H * static_cast<int64_t>(D) * D;
}

int launch_statetune_forward(int D, int dtype, const StateTuneArgs& p, hipStream_t s) {
  const bool bf = dtype == FR2_DTYPE_BFLOAT16;
  switch (D) {
    case 64: return bf ? forward_d<64, IoBF16>(p, s) : forward_d<64, IoF16>(p, s);
    case 128: return bf ? forward_d<128, IoBF16>(p, s) : forward_d<128, IoF16>(p, s);
    case 256: return bf ? forward_d<256, IoBF16>(p, s) : forward_d<256, IoF16>(p, s);
    default: return FR2_ERR_UNSUPPORTED;
  }
}

int launch_statetune_backward(int D, int dtype, StateTuneArgs p, float* workspace,
                              hipStream_t s) {
  p.dsa = workspace;
  p.snap = workspace + p.tokens * p.heads * D;
  const bool bf = dtype == FR2_DTYPE_BFLOAT16;
  switch (D) {
    case 64: return bf ? backward_d<64, IoBF16>(p, s) : backward_d<64, IoF16>(p, s);
    case 128: return bf ? backward_d<128, IoBF16>(p, s) : backward_d<128, IoF16>(p, s);
    case 256: return bf ? backward_d<256, IoBF16>(p, s) : backward_d<256, IoF16>(p, s);
    default: return FR2_ERR_UNSUPPORTED;
  }
}

int64_t statetune_padded_workspace_bytes(int B, int Tp, int H, bool backward) {
  const int64_t rows = static_cast<int64_t>(B) * Tp, row = static_cast<int64_t>(H) * 64;
  if (!backward) return rows * row * (7 * 2 + 4);   // r w k v a b y (bf16), sa (fp32)
  // r w k v a b dy and the six gradients (bf16), sa (fp32), the initial
  // states, then the pretrain backward's own workspace
  return rows * row * (13 * 2 + 4) + static_cast<int64_t>(B) * H * 64 * 64 * 4 +
         (pretrain_backward_workspace_floats(B, Tp, H, 64) + static_cast<int64_t>(B) * H * 64 * 64) *
             4;
}

int launch_statetune_padded_forward(int B, int Tp, int H, int C, const int32_t* row_source,
                                    const int32_t* chunk_seq, const int32_t* chunk_pstart,
                                    const StateTuneArgs& a, float* snap, void* ws,
                                    hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(B) * Tp;
  const int64_t row = static_cast<int64_t>(H) * 64;
  const int pieces = static_cast<int>(row * 2 / 16);   // 16-byte pieces of a bf16 row
  char* w = static_cast<char*>(ws);
  void* pad[7];
  for (int n = 0; n < 7; ++n) pad[n] = w + n * rows * row * 2;
  float* sa_pad = reinterpret_cast<float*>(w + 7 * rows * row * 2);
  PadRowsArgs g;
  const void* src[6] = {a.r, a.w, a.k, a.v, a.a, a.b};
  for (int n = 0; n < 6; ++n) {
    g.src[n] = src[n];
    g.dst[n] = pad[n];
    g.fill[n] = n == 1 ? kIdentityLogitPair : kZeroPair;
  }
  g.ntens = 6;
  int rc = pad_rows(g, row_source, rows, pieces, false, s);
  if (rc != FR2_OK) return rc;
  const int64_t cblocks = static_cast<int64_t>(C) * H;
  if (cblocks > 0x7fffffff) return FR2_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(st_gather_padded_kernel, dim3(cblocks), dim3(256), 0, s, H, chunk_seq,
                     chunk_pstart, true, a.state, snap, Tp / 16, a.boundary);
  SegArgs v;
  v.uniform_len = Tp;
  v.num_heads = H;
  v.out_elems = rows * row;
  v.state_in = a.state;
  v.state_out = a.state;
  v.r = pad[0]; v.logits = pad[1]; v.k = pad[2]; v.v = pad[3]; v.a = pad[4]; v.b = pad[5];
  v.y = pad[6];
  v.sa_out = sa_pad;
  v.boundary = snap;
  v.boundary_len = 16;
  v.boundary_per_seg = Tp / 16;
  v.scale = a.scale;
  rc = launch_chunked(FR2_DTYPE_BFLOAT16, v, B, Tp, s);
  if (rc != FR2_OK) return rc;
  hipLaunchKernelGGL(st_gather_padded_kernel, dim3(cblocks), dim3(256), 0, s, H, chunk_seq,
                     chunk_pstart, false, a.state, snap, Tp / 16, a.boundary);
  // y and sa back to the packed rows
  PadRowsArgs u;
  u.src[0] = pad[6];
  u.dst[0] = a.y;
  u.ntens = 1;
  rc = pad_rows(u, row_source, rows, pieces, true, s);
  if (rc != FR2_OK) return rc;
  u.src[0] = sa_pad;
  u.dst[0] = a.sa;
  rc = pad_rows(u, row_source, rows, pieces * 2, true, s);
  if (rc != FR2_OK) return rc;
  return record_launch();
}

int launch_statetune_padded_backward(int B, int Tp, int H, const int32_t* row_source,
                                     const int32_t* seq_first_chunk, const StateTuneArgs& a,
                                     const float* snap, void* ws, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(B) * Tp;
  const int64_t row = static_cast<int64_t>(H) * 64;
  const int pieces = static_cast<int>(row * 2 / 16);
  char* w = static_cast<char*>(ws);
  void* pad[13];   // r w k v a b dy, then dr dw dk dv da db
  for (int n = 0; n < 13; ++n) pad[n] = w + n * rows * row * 2;
  float* sa_pad = reinterpret_cast<float*>(w + 13 * rows * row * 2);
  float* init = sa_pad + rows * row;
  float* bws = init + static_cast<int64_t>(B) * H * 64 * 64;
  PadRowsArgs g;
  const void* src[7] = {a.r, a.w, a.k, a.v, a.a, a.b, a.dy};
  for (int n = 0; n < 7; ++n) {
    g.src[n] = src[n];
    g.dst[n] = pad[n];
    g.fill[n] = n == 1 ? kIdentityLogitPair : kZeroPair;
  }
  g.ntens = 7;
  int rc = pad_rows(g, row_source, rows, pieces, false, s);
  if (rc != FR2_OK) return rc;
  PadRowsArgs gs;
  gs.src[0] = a.sa;
  gs.dst[0] = sa_pad;
  gs.fill[0] = 0u;
  gs.ntens = 1;
  rc = pad_rows(gs, row_source, rows, pieces * 2, false, s);
  if (rc != FR2_OK) return rc;
  hipLaunchKernelGGL(st_initial_states_kernel, dim3(B * H), dim3(256), 0, s, H, seq_first_chunk,
                     a.boundary, init);
  PretrainBwdArgs p;
  p.batch = B; p.tokens = Tp; p.heads = H;
  p.r = pad[0]; p.w = pad[1]; p.k = pad[2]; p.v = pad[3]; p.a = pad[4]; p.b = pad[5];
  p.dy = pad[6];
  p.boundary = snap;
  p.state_dot_a = sa_pad;
  p.workspace = bws;
  p.dr = pad[7]; p.dw = pad[8]; p.dk = pad[9]; p.dv = pad[10]; p.da = pad[11]; p.db = pad[12];
  p.scale = a.scale;
  p.state0 = init;
  p.state0_stride = static_cast<int64_t>(H) * 64 * 64;
  p.dfinal = a.dfinal;
  p.dstate0 = a.dstate0;
  p.pfirst = bws + pretrain_backward_workspace_floats(B, Tp, H, 64);
  rc = launch_pretrain_backward(64, p, s);
  if (rc != FR2_OK) return rc;
  PadRowsArgs u;
  void* dst[6] = {a.dr, a.dw, a.dk, a.dv, a.da, a.db};
  for (int n = 0; n < 6; ++n) {
    u.src[n] = pad[7 + n];
    u.dst[n] = dst[n];
  }
  u.ntens = 6;
  rc = pad_rows(u, row_source, rows, pieces, true, s);
  if (rc != FR2_OK) return rc;
  return record_launch();
}

}  // namespace fr2
