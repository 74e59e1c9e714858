// WKV7 recurrence kernels for gfx950: token-serial (state resident in VGPRs
// across the whole sequence) and decode (state streamed from HBM with 16-byte
// loads, T small).  Both are driven by one segment descriptor so that the
// packed varlen, [B,T,H,D] pretrain, bf16-state, RL/Infctx and chunk-replay
// contracts share the same code.
//
// Per token and head (fp32):
//   sa[v] = sum_k a[k] S[k,v]; S[k,v] = w[k] S[k,v] + b[k] sa[v] + k[k] v[v];
//   y[v]  = scale * sum_k r[k] S[k,v]
// (reference oracle: tests/tmix/wkv7/test.py:66-83; kernel semantics:
//  csrc/sm120/tmix/wkv7/infer_recurrent_fp32io16_forward_varlen.cu:90-192).
#include "recurrent.h"

#include <array>
#include <type_traits>

namespace fr2 {

// Returns false when this workgroup has nothing to do (fail-closed status or
// an inactive sequence).  On a bad status the whole grid writes NaN.
template <class Io>
__device__ __forceinline__ bool check_status(const SegArgs& p, int seg,
                                             int64_t block, int64_t blocks) {
  if (p.status == nullptr) return true;
  if (p.status[0] != 0) {
    fill_output_nan<Io>(static_cast<typename Io::raw*>(p.y), p.out_elems, block,
                        blocks);
    return false;
  }
  return seg < p.status[2];
}

// ---------------------------------------------------------------------------
// Token-serial kernel.  One workgroup of KS*D threads per (segment, head).
// Thread (q, v) = (tid / D, tid % D) owns state column v for the key rows
// [q*R, q*R+R), R = D/KS, in registers for the whole segment.  KS = 4, or 8
// when the launch has at most one workgroup per CU (half the serial work per
// wave per token, two waves per SIMD; D = 64 and 128).  Inputs are
// staged TT = 1024/D tokens at a time through LDS as fp32 (the retention is
// computed once while staging).  The sa reduction over the 4 key quarters goes
// through a double-buffered LDS array (one barrier per token); the y partials
// of a tile are reduced after the tile and stored coalesced.
// ---------------------------------------------------------------------------
// St = StF16 selects the FP16-state (Albatross) update: the staged retention
// becomes delta = fp16(w - 1 + dither(phase)), the update is
// S + S*delta + b*sa + k*v evaluated in fp32 and rounded to fp16 after every
// token (the state registers always hold fp16 values), and y is read from
// the rounded state (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:243-336).
template <int D, class Io, class St, int KS = 4>
__global__ __launch_bounds__(KS * D) void serial_kernel(SegArgs p) {
  constexpr bool kAlbatross = __is_same(St, StF16);
  using raw = typename Io::raw;
  constexpr int NT = KS * D;
  constexpr int R = D / KS;
  constexpr int TT = 1024 / D;
  constexpr int V8 = D / 8;

  __shared__ __attribute__((aligned(16))) float s_in[6][TT][D];
  __shared__ float s_red[2][KS][D];
  __shared__ float s_y[TT][KS][D];

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int v = tid % D;
  const int q = tid / D;
  const int H = p.num_heads;
  if (!check_status<Io>(p, seg, static_cast<int64_t>(seg) * gridDim.x + h,
                        static_cast<int64_t>(gridDim.x) * gridDim.y))
    return;
  int t0, t1, slot;
  resolve_segment(p, seg, t0, t1, slot);

  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  const int elapsed_base = (kAlbatross && p.elapsed != nullptr) ? p.elapsed[slot] : 0;
  float S[R];
  if (p.state_in != nullptr) {
    const typename St::raw* sin = static_cast<const typename St::raw*>(p.state_in);
#pragma unroll
    for (int j = 0; j < R; ++j) S[j] = St::to_f32(sin[sbase + (q * R + j) * D + v]);
  } else {
#pragma unroll
    for (int j = 0; j < R; ++j) S[j] = 0.0f;
  }

  const raw* src[6] = {
      static_cast<const raw*>(p.r), static_cast<const raw*>(p.logits),
      static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
      static_cast<const raw*>(p.a), static_cast<const raw*>(p.b)};
  const raw* bias = static_cast<const raw*>(p.bias);
  raw* y = static_cast<raw*>(p.y);

  for (int tile = t0; tile < t1; tile += TT) {
    const int n = min(TT, t1 - tile);
    __syncthreads();  // previous tile fully consumed
    for (int idx = tid; idx < 6 * TT * V8; idx += NT) {
      const int which = idx / (TT * V8);
      const int rem = idx - which * (TT * V8);
      const int tt = rem / V8;
      const int c8 = rem - tt * V8;
      if (tt < n) {
        const int64_t off = (static_cast<int64_t>(tile + tt) * H + h) * D + c8 * 8;
        const Raw8 pk = *reinterpret_cast<const Raw8*>(src[which] + off);
        float f[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = raw8_get<Io>(pk, i);
        if (which == 1) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float x = f[i];
            if (bias != nullptr) x += Io::to_f32(bias[h * D + c8 * 8 + i]);
            if constexpr (kAlbatross)
              f[i] = albatross_delta(x, elapsed_base + h * D + c8 * 8 + i + (tile + tt - t0));
            else
              f[i] = retention_from_logit(x);
          }
        }
        float4* dst = reinterpret_cast<float4*>(&s_in[which][tt][c8 * 8]);
        dst[0] = make_float4(f[0], f[1], f[2], f[3]);
        dst[1] = make_float4(f[4], f[5], f[6], f[7]);
      }
    }
    __syncthreads();

    for (int tt = 0; tt < n; ++tt) {
      const float* Ar = &s_in[4][tt][q * R];
      float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
      for (int j = 0; j < R; j += 4) {
        p0 = fmaf(Ar[j + 0], S[j + 0], p0);
        p1 = fmaf(Ar[j + 1], S[j + 1], p1);
        p2 = fmaf(Ar[j + 2], S[j + 2], p2);
        p3 = fmaf(Ar[j + 3], S[j + 3], p3);
      }
      s_red[tt & 1][q][v] = (p0 + p1) + (p2 + p3);
      __syncthreads();
      float sa = 0.f;
#pragma unroll
      for (int qq = 0; qq < KS; ++qq) sa += s_red[tt & 1][qq][v];
      if (p.sa_out != nullptr && q == 0)
        p.sa_out[(static_cast<int64_t>(tile + tt) * H + h) * D + v] = sa;

      const float vv = s_in[3][tt][v];
      const float* Wr = &s_in[1][tt][q * R];
      const float* Kr = &s_in[2][tt][q * R];
      const float* Br = &s_in[5][tt][q * R];
      const float* Rr = &s_in[0][tt][q * R];
      float y0 = 0.f, y1 = 0.f, y2 = 0.f, y3 = 0.f;
      if constexpr (kAlbatross) {
        // Wr holds delta: fp16(S + S*delta + b*sa + k*v)
#pragma unroll
        for (int j = 0; j < R; ++j) {
          float u = fmaf(S[j], Wr[j], S[j]);
          u = fmaf(Br[j], sa, u);
          u = fmaf(Kr[j], vv, u);
          S[j] = St::to_f32(St::from_f32(u));
        }
      }
#pragma unroll
      for (int j = 0; j < R; j += 4) {
        if constexpr (!kAlbatross) {
          S[j + 0] = fmaf(Wr[j + 0], S[j + 0], fmaf(Br[j + 0], sa, Kr[j + 0] * vv));
          S[j + 1] = fmaf(Wr[j + 1], S[j + 1], fmaf(Br[j + 1], sa, Kr[j + 1] * vv));
          S[j + 2] = fmaf(Wr[j + 2], S[j + 2], fmaf(Br[j + 2], sa, Kr[j + 2] * vv));
          S[j + 3] = fmaf(Wr[j + 3], S[j + 3], fmaf(Br[j + 3], sa, Kr[j + 3] * vv));
        }
        y0 = fmaf(Rr[j + 0], S[j + 0], y0);
        y1 = fmaf(Rr[j + 1], S[j + 1], y1);
        y2 = fmaf(Rr[j + 2], S[j + 2], y2);
        y3 = fmaf(Rr[j + 3], S[j + 3], y3);
      }
      s_y[tt][q][v] = (y0 + y1) + (y2 + y3);

      if (p.boundary != nullptr) {
        const int pos = tile + tt - t0 + 1;
        if (pos % p.boundary_len == 0) {
          const int c = pos / p.boundary_len - 1;
          float* bd = p.boundary +
                      ((static_cast<int64_t>(seg) * H + h) * p.boundary_per_seg + c) *
                          D * D;
#pragma unroll
          for (int j = 0; j < R; ++j) bd[(q * R + j) * D + v] = S[j];
        }
      }
    }
    __syncthreads();
    for (int idx = tid; idx < n * D; idx += NT) {
      const int tt = idx / D;
      const int vv = idx - tt * D;
      float acc = 0.f;
#pragma unroll
      for (int qq = 0; qq < KS; ++qq) acc += s_y[tt][qq][vv];
      y[(static_cast<int64_t>(tile + tt) * H + h) * D + vv] = Io::from_f32(p.scale * acc);
    }
  }

  if (p.state_out != nullptr) {
    typename St::raw* sout = static_cast<typename St::raw*>(p.state_out);
#pragma unroll
    for (int j = 0; j < R; ++j) sout[sbase + (q * R + j) * D + v] = St::from_f32(S[j]);
  }
}

// ---------------------------------------------------------------------------
// Token-serial kernel without a per-token workgroup barrier (D = 64, fp32 or
// bf16 state).  Four waves per (segment, head); wave w owns the value columns
// [16w, 16w+16) for all 64 keys: lane l holds column 16w + l%16 of the key
// rows 16g .. 16g+15, g = l/16, in registers.  sa is reduced over the four
// key groups inside the wave: with both operands equal, the two results of
// v_permlane16_swap / v_permlane32_swap sum to the row-pair / half-wave sum,
// whichever way the rows move.  Tokens are staged through LDS per tile as in
// serial_kernel; the y partials of the four key groups are summed at the end
// of a tile.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float sum_key_groups(float x) {
  const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                    false, false);
  const float s1 = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(s1), __float_as_uint(s1),
                                                    false, false);
  return __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
}

template <class Io, class St>
__global__ __launch_bounds__(256) void serial64w_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr int D = 64;
  constexpr int NT = 256;
  constexpr int TT = 16;
  constexpr int V8 = D / 8;

  __shared__ __attribute__((aligned(16))) float s_in[6][TT][D];
  __shared__ float s_y[TT][4][D];

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int c = 16 * (tid >> 6) + (lane & 15);   // value column
  const int g = lane >> 4;                       // key group: keys 16g .. 16g+15
  const int H = p.num_heads;
  if (!check_status<Io>(p, seg, static_cast<int64_t>(seg) * gridDim.x + h,
                        static_cast<int64_t>(gridDim.x) * gridDim.y))
    return;
  int t0, t1, slot;
  resolve_segment(p, seg, t0, t1, slot);

  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  float S[16];
  if (p.state_in != nullptr) {
    const typename St::raw* sin = static_cast<const typename St::raw*>(p.state_in);
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j] = St::to_f32(sin[sbase + (16 * g + j) * D + c]);
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j] = 0.0f;
  }

  const raw* src[6] = {
      static_cast<const raw*>(p.r), static_cast<const raw*>(p.logits),
      static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
      static_cast<const raw*>(p.a), static_cast<const raw*>(p.b)};
  const raw* bias = static_cast<const raw*>(p.bias);
  raw* y = static_cast<raw*>(p.y);

  // the 6 x TT x 64 token values of a tile are 768 16-byte pieces, three per
  // thread; the next tile's pieces are loaded into registers while the
  // current tile computes
  constexpr int PER = 6 * TT * V8 / NT;
  static_assert(PER * NT == 6 * TT * V8, "tile pieces must divide evenly");
  Raw8 pre[PER];
  auto fetch = [&](int tile) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = tid + u * NT;
      const int which = idx / (TT * V8);
      const int rem = idx - which * (TT * V8);
      const int tt = rem / V8;
      const int c8 = rem - tt * V8;
      // rows past the segment repeat its last row (in bounds; never consumed)
      const int row = min(tile + tt, t1 - 1);
      pre[u] = *reinterpret_cast<const Raw8*>(src[which] +
                                              (static_cast<int64_t>(row) * H + h) * D + c8 * 8);
    }
  };
  if (t0 < t1) fetch(t0);
  for (int tile = t0; tile < t1; tile += TT) {
    const int n = min(TT, t1 - tile);
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = tid + u * NT;
      const int which = idx / (TT * V8);
      const int rem = idx - which * (TT * V8);
      const int tt = rem / V8;
      const int c8 = rem - tt * V8;
      float f[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = raw8_get<Io>(pre[u], i);
      if (which == 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float x = f[i];
          if (bias != nullptr) x += Io::to_f32(bias[h * D + c8 * 8 + i]);
          f[i] = retention_from_logit(x);
        }
      }
      float4* dst = reinterpret_cast<float4*>(&s_in[which][tt][c8 * 8]);
      dst[0] = make_float4(f[0], f[1], f[2], f[3]);
      dst[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
    __syncthreads();
    if (tile + TT < t1) fetch(tile + TT);

    for (int tt = 0; tt < n; ++tt) {
      // the token's rows for this lane's 16 keys (broadcast reads within a
      // key group)
      float av[16], wv[16], kv[16], bv[16], rv[16];
#pragma unroll
      for (int j = 0; j < 16; j += 4) {
        *reinterpret_cast<float4*>(&av[j]) = *reinterpret_cast<const float4*>(&s_in[4][tt][16 * g + j]);
        *reinterpret_cast<float4*>(&wv[j]) = *reinterpret_cast<const float4*>(&s_in[1][tt][16 * g + j]);
        *reinterpret_cast<float4*>(&kv[j]) = *reinterpret_cast<const float4*>(&s_in[2][tt][16 * g + j]);
        *reinterpret_cast<float4*>(&bv[j]) = *reinterpret_cast<const float4*>(&s_in[5][tt][16 * g + j]);
        *reinterpret_cast<float4*>(&rv[j]) = *reinterpret_cast<const float4*>(&s_in[0][tt][16 * g + j]);
      }
      const float vv = s_in[3][tt][c];
      float p0 = 0.f, p1 = 0.f, p2 = 0.f, p3 = 0.f;
#pragma unroll
      for (int j = 0; j < 16; j += 4) {
        p0 = fmaf(av[j + 0], S[j + 0], p0);
        p1 = fmaf(av[j + 1], S[j + 1], p1);
        p2 = fmaf(av[j + 2], S[j + 2], p2);
        p3 = fmaf(av[j + 3], S[j + 3], p3);
      }
      const float sa = sum_key_groups((p0 + p1) + (p2 + p3));
      if (p.sa_out != nullptr && g == 0)
        p.sa_out[(static_cast<int64_t>(tile + tt) * H + h) * D + c] = sa;
      float y0 = 0.f, y1 = 0.f, y2 = 0.f, y3 = 0.f;
#pragma unroll
      for (int j = 0; j < 16; j += 4) {
        S[j + 0] = fmaf(wv[j + 0], S[j + 0], fmaf(bv[j + 0], sa, kv[j + 0] * vv));
        S[j + 1] = fmaf(wv[j + 1], S[j + 1], fmaf(bv[j + 1], sa, kv[j + 1] * vv));
        S[j + 2] = fmaf(wv[j + 2], S[j + 2], fmaf(bv[j + 2], sa, kv[j + 2] * vv));
        S[j + 3] = fmaf(wv[j + 3], S[j + 3], fmaf(bv[j + 3], sa, kv[j + 3] * vv));
        y0 = fmaf(rv[j + 0], S[j + 0], y0);
        y1 = fmaf(rv[j + 1], S[j + 1], y1);
        y2 = fmaf(rv[j + 2], S[j + 2], y2);
        y3 = fmaf(rv[j + 3], S[j + 3], y3);
      }
      s_y[tt][g][c] = (y0 + y1) + (y2 + y3);

      if (p.boundary != nullptr) {
        const int pos = tile + tt - t0 + 1;
        if (pos % p.boundary_len == 0) {
          const int cb = pos / p.boundary_len - 1;
          float* bd = p.boundary +
                      ((static_cast<int64_t>(seg) * H + h) * p.boundary_per_seg + cb) * D * D;
#pragma unroll
          for (int j = 0; j < 16; ++j) bd[(16 * g + j) * D + c] = S[j];
        }
      }
    }
    __syncthreads();
    for (int idx = tid; idx < n * D; idx += NT) {
      const int tt = idx / D;
      const int vc = idx - tt * D;
      const float acc = (s_y[tt][0][vc] + s_y[tt][1][vc]) + (s_y[tt][2][vc] + s_y[tt][3][vc]);
      y[(static_cast<int64_t>(tile + tt) * H + h) * D + vc] = Io::from_f32(p.scale * acc);
    }
  }

  if (p.state_out != nullptr) {
    typename St::raw* sout = static_cast<typename St::raw*>(p.state_out);
#pragma unroll
    for (int j = 0; j < 16; ++j) sout[sbase + (16 * g + j) * D + c] = St::from_f32(S[j]);
  }
}

// ---------------------------------------------------------------------------
// FP16-state (Albatross) token-serial kernel at D = 64 without a per-token
// workgroup barrier.  Per token the state update is elementwise on the VALU
// and the two dot products over the 64 keys (sa = a^T S before the update,
// y = r^T S after it) run on the matrix cores: the state is fp16 by contract
// and the token values a, r are fp16, so every product is exact and the
// fp32 accumulation rounds only the sums.
//
// Four waves per (segment, head); wave w owns value columns [16w, 16w+16).
// Lane (j, q) = (lane % 16, lane / 16) holds column 16w + j for keys
// 32m + 8q + e (m = 0, 1; e = 0..7) twice: as fp32 (the update's operand)
// and as packed fp16 pairs, which are as they stand the B operand of
// v_mfma_f32_16x16x32_f16 for the two K steps m.  The A operand is the
// token's a (or r) row replicated over the 16 rows, so every lane of a
// column receives the dot product of its column.
// The update S = fp16(S + S delta + b sa + k v) needs per key delta, b, k:
// lane j of row q loads those of key 32(j / 8) + 8q + j % 8, which are
// exactly the row's 16 state keys, and the DPP row broadcast
// (row_newbcast) hands key j's values to the whole row inside the FMAs
// (v_fmac_f32_dpp).  The fp32 result is rounded to fp16 two keys at a time
// (v_cvt_pk_f16_f32), which forms the packed B operand, and widened back
// for the next token's update: fp32 arithmetic, then the fp16 rounding, as
// the reference's test contract states it (tests/tmix/wkv7/test.py:88-149).
// Token values are staged per 16-token tile through LDS.
// ---------------------------------------------------------------------------
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// S32[8m + e] = fma(k_j, v, fma(b_j, sa, fma(d_j, S, S))) in fp32 for the
// eight keys j = 8m + e of block m, stage by stage (no instruction waits on
// the one before it), each key's d, b, k broadcast from lane j of the row.
// The leading s_nop covers the wait states before the DPP reads (the
// compiler does not see inside an asm block; sa arrives through a DPP move
// the compiler emits, so its matrix-core wait is the compiler's).
#define FR2_H_BLOCK0 \
  "v_fmac_f32_dpp %0, %8, %0 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %1, %8, %1 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %2, %8, %2 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %3, %8, %3 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %4, %8, %4 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %5, %8, %5 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %6, %8, %6 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %7, %8, %7 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %0, %9, %11 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %1, %9, %11 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %2, %9, %11 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %3, %9, %11 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %4, %9, %11 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %5, %9, %11 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %6, %9, %11 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %7, %9, %11 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %0, %10, %12 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %1, %10, %12 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %2, %10, %12 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %3, %10, %12 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %4, %10, %12 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %5, %10, %12 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %6, %10, %12 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %7, %10, %12 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
#define FR2_H_BLOCK8 \
  "v_fmac_f32_dpp %0, %8, %0 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %1, %8, %1 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %2, %8, %2 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %3, %8, %3 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %4, %8, %4 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %5, %8, %5 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %6, %8, %6 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %7, %8, %7 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %0, %9, %11 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %1, %9, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %2, %9, %11 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %3, %9, %11 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %4, %9, %11 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %5, %9, %11 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %6, %9, %11 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %7, %9, %11 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %0, %10, %12 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %1, %10, %12 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %2, %10, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %3, %10, %12 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %4, %10, %12 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %5, %10, %12 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %6, %10, %12 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"  \
  "v_fmac_f32_dpp %7, %10, %12 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
__device__ __forceinline__ void albatross_update_block(float (&S32)[16], float d, float b,
                                                       float k, float sa, float v, int m) {
  float* s = &S32[8 * m];
  if (m == 0) {
    asm volatile("s_nop 1\n\t" FR2_H_BLOCK0
                 : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3]), "+v"(s[4]), "+v"(s[5]),
                   "+v"(s[6]), "+v"(s[7])
                 : "v"(d), "v"(b), "v"(k), "v"(sa), "v"(v));
  } else {
    asm volatile("s_nop 1\n\t" FR2_H_BLOCK8
                 : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3]), "+v"(s[4]), "+v"(s[5]),
                   "+v"(s[6]), "+v"(s[7])
                 : "v"(d), "v"(b), "v"(k), "v"(sa), "v"(v));
  }
}
#undef FR2_H_BLOCK0
#undef FR2_H_BLOCK8

// x^T S for the lane's column: x's 64 fp16 values as the A operand (every
// row the same), the packed state as the B operand of the two K steps
__device__ __forceinline__ float state_dot_f16(h8 x0, h8 x1, const uint32_t (&S16)[8]) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const h8 b0 = __builtin_bit_cast(h8, u32x4{S16[0], S16[1], S16[2], S16[3]});
  const h8 b1 = __builtin_bit_cast(h8, u32x4{S16[4], S16[5], S16[6], S16[7]});
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, b0, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, b1, acc, 0, 0, 0);
  return acc[0];
}

template <class Io>
__global__ __launch_bounds__(256) void serial64h_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr int D = 64;
  constexpr int NT = 256;
  constexpr int TT = 32;
  constexpr int TP = TT + 4;   // token pitch of the transposed rows (16-byte reads)
  constexpr int V8 = D / 8;

  // per-key values, transposed ([tensor][key][token], fp32): delta, k, b;
  // v by value column
  __shared__ __attribute__((aligned(16))) float s_t[4][D][TP];
  // the a and r rows as they arrive (fp16), the matrix cores' A operands
  __shared__ __attribute__((aligned(16))) _Float16 s_ar[2][TT][D];
  __shared__ float s_y[TT][D];

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int j = lane & 15;
  const int q = lane >> 4;
  const int col = 16 * (tid >> 6) + j;                 // value column
  const int kown = 32 * (j >> 3) + 8 * q + (j & 7);    // key whose values this lane loads
  const int H = p.num_heads;
  if (!check_status<Io>(p, seg, static_cast<int64_t>(seg) * gridDim.x + h,
                        static_cast<int64_t>(gridDim.x) * gridDim.y))
    return;
  int t0, t1, slot;
  resolve_segment(p, seg, t0, t1, slot);

  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  const int elapsed_base = p.elapsed != nullptr ? p.elapsed[slot] : 0;
  float S32[16];
  uint32_t S16[8];
  {
    const uint16_t* sin = static_cast<const uint16_t*>(p.state_in);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const uint16_t lo = sin[sbase + (32 * m + 8 * q + e) * D + col];
        const uint16_t hi = sin[sbase + (32 * m + 8 * q + e + 1) * D + col];
        S16[4 * m + e / 2] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
        S32[8 * m + e] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
        S32[8 * m + e + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
      }
    }
  }

  const raw* src[6] = {
      static_cast<const raw*>(p.r), static_cast<const raw*>(p.logits),
      static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
      static_cast<const raw*>(p.a), static_cast<const raw*>(p.b)};
  const raw* bias = static_cast<const raw*>(p.bias);
  raw* y = static_cast<raw*>(p.y);

  constexpr int PER = 6 * TT * V8 / NT;
  static_assert(PER * NT == 6 * TT * V8, "tile pieces must divide evenly");
  Raw8 pre[PER];
  auto fetch = [&](int tile) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = tid + u * NT;
      const int which = idx / (TT * V8);
      const int rem = idx - which * (TT * V8);
      const int tt = rem / V8;
      const int c8 = rem - tt * V8;
      // rows past the segment repeat its last row (in bounds; never consumed)
      const int row = min(tile + tt, t1 - 1);
      pre[u] = *reinterpret_cast<const Raw8*>(src[which] +
                                              (static_cast<int64_t>(row) * H + h) * D + c8 * 8);
    }
  };
  auto a_row = [&](int which, int tt, int m) {
    return *reinterpret_cast<const h8*>(&s_ar[which][tt][32 * m + 8 * q]);
  };
  if (t0 < t1) fetch(t0);
  for (int tile = t0; tile < t1; tile += TT) {
    const int n = min(TT, t1 - tile);
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int idx = tid + u * NT;
      const int which = idx / (TT * V8);
      const int rem = idx - which * (TT * V8);
      const int tt = rem / V8;
      const int c8 = rem - tt * V8;
      if (which == 0 || which == 4) {
        // r, a: fp16 rows as loaded
        *reinterpret_cast<Raw8*>(&s_ar[which == 4 ? 0 : 1][tt][c8 * 8]) = pre[u];
        continue;
      }
      float f[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) f[i] = raw8_get<Io>(pre[u], i);
      if (which == 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float x = f[i];
          if (bias != nullptr) x += Io::to_f32(bias[h * D + c8 * 8 + i]);
          f[i] = albatross_delta(x, elapsed_base + h * D + c8 * 8 + i + (tile + tt - t0));
        }
      }
      // delta, k, v, b -> rows 0, 1, 2, 3 of s_t
      const int slot_t = which == 1 ? 0 : which == 2 ? 1 : which == 3 ? 2 : 3;
#pragma unroll
      for (int i = 0; i < 8; ++i) s_t[slot_t][c8 * 8 + i][tt] = f[i];
    }
    __syncthreads();
    if (tile + TT < t1) fetch(tile + TT);

    // sa of the tile's first token; every later one comes with the y pass
    float sa = state_dot_f16(a_row(0, 0, 0), a_row(0, 0, 1), S16);
    // one token: the update, the state rounded to fp16 (packed pairs: the
    // matrix cores' B operand), the next token's sa (the critical path) and
    // y, and the state widened back for the next update
    float y_prev = 0.f;   // the previous token's y, stored one token late
    auto step = [&](int tt, bool has_next, float d, float b, float k, float v) {
      // (storing y right after its matrix-core pass would stall the wave
      // until that pass completes, in front of the next token's work)
      if (tt > 0) s_y[tt - 1][col] = y_prev;
      // A operands of this token's y and the next token's sa, requested
      // before the update so that their LDS latency hides behind it
      const int tn = has_next ? tt + 1 : tt;
      const h8 an0 = a_row(0, tn, 0), an1 = a_row(0, tn, 1);
      const h8 r0 = a_row(1, tt, 0), r1 = a_row(1, tt, 1);
      // sa passes through a DPP move the compiler emits, so the compiler
      // places the matrix-core result wait before it
      const float sa_v =
          __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sa), 0xe4, 0xf, 0xf, false));
      albatross_update_block(S32, d, b, k, sa_v, v, 0);
      albatross_update_block(S32, d, b, k, sa_v, v, 1);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        S16[e] = __builtin_bit_cast(
            uint32_t, __builtin_convertvector(f32x2{S32[2 * e], S32[2 * e + 1]}, f16x2));
      }
      if (has_next) sa = state_dot_f16(an0, an1, S16);
      y_prev = state_dot_f16(r0, r1, S16);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = S16[e];
        S32[2 * e] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
        S32[2 * e + 1] =
            static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
      }
    };
    auto group = [&](int t4) {
      return std::array<f4, 4>{*reinterpret_cast<const f4*>(&s_t[0][kown][t4]),
                               *reinterpret_cast<const f4*>(&s_t[3][kown][t4]),
                               *reinterpret_cast<const f4*>(&s_t[1][kown][t4]),
                               *reinterpret_cast<const f4*>(&s_t[2][col][t4])};
    };
    if (n == TT) {
      // full tile: straight-line code within each group of four tokens
#pragma unroll 2
      for (int t4 = 0; t4 < TT; t4 += 4) {
        const auto gv = group(t4);
#pragma unroll
        for (int u = 0; u < 4; ++u)
          step(t4 + u, t4 + u + 1 < TT, gv[0][u], gv[1][u], gv[2][u], gv[3][u]);
      }
    } else {
      for (int t4 = 0; t4 < n; t4 += 4) {
        const auto gv = group(t4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (t4 + u >= n) break;
          step(t4 + u, t4 + u + 1 < n, gv[0][u], gv[1][u], gv[2][u], gv[3][u]);
        }
      }
    }
    s_y[n - 1][col] = y_prev;
    __syncthreads();
    for (int idx = tid; idx < n * D; idx += NT) {
      const int tt = idx / D;
      const int vc = idx - tt * D;
      y[(static_cast<int64_t>(tile + tt) * H + h) * D + vc] = Io::from_f32(p.scale * s_y[tt][vc]);
    }
  }

  uint16_t* sout = static_cast<uint16_t*>(p.state_out);
#pragma unroll
  for (int m = 0; m < 2; ++m) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      sout[sbase + (32 * m + 8 * q + e) * D + col] = static_cast<uint16_t>(S16[4 * m + e / 2]);
      sout[sbase + (32 * m + 8 * q + e + 1) * D + col] =
          static_cast<uint16_t>(S16[4 * m + e / 2] >> 16);
    }
  }
}

// ---------------------------------------------------------------------------
// Decode kernel (D = 64, fp32 state).  One wavefront per (segment, head).
// Lane l owns columns 4*(l%16)..+3 of key rows {l/16 + 4j : j < 16}: the 16 KiB
// state moves as 16 dwordx4 loads per lane, each wave instruction covering 4
// full 256-byte rows.  sa and y are reduced over the 4 row groups with two
// cross-lane xor exchanges.  Token vectors go through a 1.5 KiB LDS buffer in
// which key k sits at (k%4)*16 + k/4, so every lane reads its 16 keys as four
// 16-byte LDS reads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f4 shfl_xor4(f4 x, int m) {
  return f4{__shfl_xor(x.x, m), __shfl_xor(x.y, m), __shfl_xor(x.z, m),
            __shfl_xor(x.w, m)};
}

// St = StF16: FP16 state pool with the Albatross delta update (see
// serial_kernel); the staged retention becomes delta and each updated value
// is rounded to fp16 before it feeds y and the store.
// kSa: also write every token's pre-update sa (the rl_infctx replay).
template <class Io, class St, bool kSa = false>
__device__ __forceinline__ void decode64_body(const SegArgs& p) {
  constexpr bool kAlbatross = __is_same(St, StF16);
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  using raw = typename Io::raw;
  constexpr int D = 64;
  __shared__ __attribute__((aligned(16))) float s_in[6][D];

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int lane = threadIdx.x;
  const int H = p.num_heads;
  if (!check_status<Io>(p, seg, static_cast<int64_t>(seg) * gridDim.x + h,
                        static_cast<int64_t>(gridDim.x) * gridDim.y))
    return;
  int t0, t1, slot;
  resolve_segment(p, seg, t0, t1, slot);

  const int c4 = lane & 15;
  const int rq = lane >> 4;
  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  // The FP16 state stays packed in registers (two per 4-vector instead of
  // four): every value is an fp16 number anyway, and the halved register
  // count lets more waves stay resident.
  using Reg = std::conditional_t<kAlbatross, h4, f4>;
  Reg S[16];
  auto get = [&](int j) -> f4 {
    if constexpr (kAlbatross) return __builtin_convertvector(S[j], f4);
    else return S[j];
  };
  const int elapsed_base = (kAlbatross && p.elapsed != nullptr) ? p.elapsed[slot] : 0;
  if (p.state_in != nullptr) {
    const typename St::raw* sin =
        static_cast<const typename St::raw*>(p.state_in) + sbase + rq * D + 4 * c4;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      S[j] = __builtin_nontemporal_load(reinterpret_cast<const Reg*>(sin + 4 * j * D));
    }
  } else {
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j] = Reg{0, 0, 0, 0};
  }

  const raw* rp = static_cast<const raw*>(p.r);
  const raw* lp = static_cast<const raw*>(p.logits);
  const raw* kp = static_cast<const raw*>(p.k);
  const raw* vp = static_cast<const raw*>(p.v);
  const raw* ap = static_cast<const raw*>(p.a);
  const raw* bp = static_cast<const raw*>(p.b);
  const raw* bias = static_cast<const raw*>(p.bias);
  raw* y = static_cast<raw*>(p.y);
  const int pk = (lane & 3) * 16 + (lane >> 2);

  for (int t = t0; t < t1; ++t) {
    const int64_t base = (static_cast<int64_t>(t) * H + h) * D;
    float x = Io::to_f32(lp[base + lane]);
    if (bias != nullptr) x += Io::to_f32(bias[h * D + lane]);
    s_in[0][pk] = Io::to_f32(rp[base + lane]);
    if constexpr (kAlbatross)
      s_in[1][pk] = albatross_delta(x, elapsed_base + h * D + lane + (t - t0));
    else
      s_in[1][pk] = retention_from_logit(x);
    s_in[2][pk] = Io::to_f32(kp[base + lane]);
    s_in[3][lane] = Io::to_f32(vp[base + lane]);
    s_in[4][pk] = Io::to_f32(ap[base + lane]);
    s_in[5][pk] = Io::to_f32(bp[base + lane]);
    __syncthreads();

    const float* Ar = &s_in[4][rq * 16];
    f4 sa = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float aj = Ar[j];
      const f4 sj = get(j);
      sa.x = fmaf(aj, sj.x, sa.x);
      sa.y = fmaf(aj, sj.y, sa.y);
      sa.z = fmaf(aj, sj.z, sa.z);
      sa.w = fmaf(aj, sj.w, sa.w);
    }
    f4 o = shfl_xor4(sa, 16);
    sa.x += o.x; sa.y += o.y; sa.z += o.z; sa.w += o.w;
    o = shfl_xor4(sa, 32);
    sa.x += o.x; sa.y += o.y; sa.z += o.z; sa.w += o.w;
    // the replay contract's per-token pre-update sa (fp32, [T, H, D])
    if constexpr (kSa) {
      if (rq == 0) *reinterpret_cast<f4*>(p.sa_out + base + 4 * c4) = sa;
    }

    const f4 vv = *reinterpret_cast<const f4*>(&s_in[3][4 * c4]);
    const float* Rr = &s_in[0][rq * 16];
    const float* Wr = &s_in[1][rq * 16];
    const float* Kr = &s_in[2][rq * 16];
    const float* Br = &s_in[5][rq * 16];
    f4 yy = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float wj = Wr[j], bj = Br[j], kj = Kr[j], rj = Rr[j];
      f4 sj = get(j);
      if constexpr (kAlbatross) {
        // wj holds delta: fp16(S + S*delta + b*sa + k*v)
        f4 u;
        u.x = fmaf(kj, vv.x, fmaf(bj, sa.x, fmaf(sj.x, wj, sj.x)));
        u.y = fmaf(kj, vv.y, fmaf(bj, sa.y, fmaf(sj.y, wj, sj.y)));
        u.z = fmaf(kj, vv.z, fmaf(bj, sa.z, fmaf(sj.z, wj, sj.z)));
        u.w = fmaf(kj, vv.w, fmaf(bj, sa.w, fmaf(sj.w, wj, sj.w)));
        S[j] = __builtin_convertvector(u, h4);
        sj = __builtin_convertvector(S[j], f4);
      } else {
        sj.x = fmaf(wj, sj.x, fmaf(bj, sa.x, kj * vv.x));
        sj.y = fmaf(wj, sj.y, fmaf(bj, sa.y, kj * vv.y));
        sj.z = fmaf(wj, sj.z, fmaf(bj, sa.z, kj * vv.z));
        sj.w = fmaf(wj, sj.w, fmaf(bj, sa.w, kj * vv.w));
        S[j] = sj;
      }
      yy.x = fmaf(rj, sj.x, yy.x);
      yy.y = fmaf(rj, sj.y, yy.y);
      yy.z = fmaf(rj, sj.z, yy.z);
      yy.w = fmaf(rj, sj.w, yy.w);
    }
    o = shfl_xor4(yy, 16);
    yy.x += o.x; yy.y += o.y; yy.z += o.z; yy.w += o.w;
    o = shfl_xor4(yy, 32);
    yy.x += o.x; yy.y += o.y; yy.z += o.z; yy.w += o.w;
    if (rq == 0) {
      raw* dst = y + base + 4 * c4;
      dst[0] = Io::from_f32(p.scale * yy.x);
      dst[1] = Io::from_f32(p.scale * yy.y);
      dst[2] = Io::from_f32(p.scale * yy.z);
      dst[3] = Io::from_f32(p.scale * yy.w);
    }
    __syncthreads();
  }

  if (p.state_out != nullptr) {
    typename St::raw* sout =
        static_cast<typename St::raw*>(p.state_out) + sbase + rq * D + 4 * c4;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      __builtin_nontemporal_store(S[j], reinterpret_cast<Reg*>(sout + 4 * j * D));
  }
}

template <class Io, class St, bool kSa = false>
__global__ __launch_bounds__(64) void decode64_kernel(SegArgs p) {
  decode64_body<Io, St, kSa>(p);
}
// The FP16-state form holds its state packed (32 registers).  Capped at 96
// registers (five waves per SIMD) it spills 26 values and runs no faster
// than at 128 (config-2 shape: 0.0238 ms both; 80 registers, six waves:
// 0.0359 ms), so it keeps 128 (2 spilled values).
template <class Io>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(4))) void decode64_f16s_kernel(
    SegArgs p) {
  decode64_body<Io, StF16>(p);
}

// ---------------------------------------------------------------------------
// Host-side launch helpers.
// ---------------------------------------------------------------------------
constexpr int64_t kSerialWideUnits = 256;

template <class Io, class St>
static int launch_serial_io(int D, const SegArgs& p, int nseg, hipStream_t s) {
  const dim3 grid(p.num_heads, nseg);
  // at most one workgroup per CU: split the key rows 8 ways (config-1 batch
  // at D = 64: 2.17 vs 2.61 ms); with more workgroups the 4-way split packs
  // better (2 048 units of 100 tokens: 0.239 vs 0.292 ms)
  const bool wide = static_cast<int64_t>(p.num_heads) * nseg <= kSerialWideUnits;
  switch (D) {
    case 64:
      // fp32 / bf16 state: the kernel without a per-token barrier (many
      // 100-token sequences: 0.204 vs 0.243 ms; the config-1 batch: 2.11 vs
      // 2.18 ms); the FP16-state update keeps the KS-way kernel
      if constexpr (!__is_same(St, StF16)) {
        hipLaunchKernelGGL((serial64w_kernel<Io, St>), grid, dim3(256), 0, s, p);
        break;
      }
      if (wide)
        hipLaunchKernelGGL((serial_kernel<64, Io, St, 8>), grid, dim3(512), 0, s, p);
      else
        hipLaunchKernelGGL((serial_kernel<64, Io, St>), grid, dim3(256), 0, s, p);
      break;
    case 128:
      if (wide)
        hipLaunchKernelGGL((serial_kernel<128, Io, St, 8>), grid, dim3(1024), 0, s, p);
      else
        hipLaunchKernelGGL((serial_kernel<128, Io, St>), grid, dim3(512), 0, s, p);
      break;
    case 256:
      hipLaunchKernelGGL((serial_kernel<256, Io, St>), grid, dim3(1024), 0, s, p);
      break;
    default:
      return FR2_ERR_UNSUPPORTED;
  }
  return record_launch();
}

// Adds each active sequence's token count to its slot's elapsed count
// (csrc/sm120/tmix/wkv7/infer_recurrent_fp16_forward_varlen.cu:60-75); an
// invalid ticket leaves every count untouched.  Runs after the recurrence on
// the same stream, so no recurrence workgroup reads a count this writes.
__global__ __launch_bounds__(256) void advance_elapsed_kernel(SegArgs p, int nseg,
                                                              int32_t* elapsed) {
  const int seg = static_cast<int>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (seg >= nseg) return;
  if (p.status != nullptr && (p.status[0] != 0 || seg >= p.status[2])) return;
  int t0, t1, slot;
  resolve_segment(p, seg, t0, t1, slot);
  elapsed[slot] += t1 - t0;
}

// requests with at most this many tokens per sequence stream the state once
constexpr int kFp16DecodeMaxSeqlen = 4;

int launch_fp16_state(int D, const SegArgs& p, int nseg, int max_seqlen, int32_t* elapsed,
                      hipStream_t s, bool advance, int family) {
  if (elapsed == nullptr || p.sa_out != nullptr || p.boundary != nullptr)
    return FR2_ERR_INVALID_ARGUMENT;
  SegArgs q = p;
  q.elapsed = elapsed;
  if (family < 0) {
    // D = 64: short requests stream the state once; longer ones run the
    // barrier-free token-serial kernel
    family = D != 64 ? kFp16Serial
             : (max_seqlen > 0 && max_seqlen <= kFp16DecodeMaxSeqlen) ? kFp16Decode
                                                                       : kFp16SerialWave;
  }
  if ((family == kFp16Decode || family == kFp16SerialWave) && D != 64) return FR2_ERR_UNSUPPORTED;
  if (family == kFp16Decode) {
    hipLaunchKernelGGL((decode64_f16s_kernel<IoF16>), dim3(p.num_heads, nseg), dim3(64), 0, s,
                       q);
  } else if (family == kFp16SerialWave) {
    hipLaunchKernelGGL((serial64h_kernel<IoF16>), dim3(p.num_heads, nseg), dim3(256), 0, s, q);
  } else if (family == kFp16Serial) {
    const int rc = launch_serial_io<IoF16, StF16>(D, q, nseg, s);
    if (rc != FR2_OK) return rc;
  } else {
    return FR2_ERR_INVALID_ARGUMENT;
  }
  const int rc = record_launch();
  if (rc != FR2_OK) return rc;
  return advance ? launch_advance_elapsed(p, nseg, elapsed, s) : FR2_OK;
}

int launch_advance_elapsed(const SegArgs& p, int nseg, int32_t* elapsed, hipStream_t s) {
  if (elapsed == nullptr) return FR2_ERR_INVALID_ARGUMENT;
  SegArgs q = p;
  q.elapsed = elapsed;
  hipLaunchKernelGGL(advance_elapsed_kernel, dim3((nseg + 255) / 256), dim3(256), 0, s, q, nseg,
                     elapsed);
  return record_launch();
}

int launch_serial(int D, int dtype, bool bf16_state, const SegArgs& p, int nseg,
                  hipStream_t s) {
  if (bf16_state) {
    if (dtype != FR2_DTYPE_BFLOAT16) return FR2_ERR_UNSUPPORTED;
    return launch_serial_io<IoBF16, StBF16>(D, p, nseg, s);
  }
  if (dtype == FR2_DTYPE_BFLOAT16) return launch_serial_io<IoBF16, StF32>(D, p, nseg, s);
  if (dtype == FR2_DTYPE_FLOAT16) return launch_serial_io<IoF16, StF32>(D, p, nseg, s);
  return FR2_ERR_UNSUPPORTED;
}

int launch_decode(int D, int dtype, const SegArgs& p, int nseg, hipStream_t s) {
  if (D != 64 || p.boundary != nullptr) return FR2_ERR_UNSUPPORTED;
  const dim3 grid(p.num_heads, nseg);
  const bool sa = p.sa_out != nullptr;
  if (dtype == FR2_DTYPE_BFLOAT16) {
    if (sa)
      hipLaunchKernelGGL((decode64_kernel<IoBF16, StF32, true>), grid, dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL((decode64_kernel<IoBF16, StF32>), grid, dim3(64), 0, s, p);
  } else if (dtype == FR2_DTYPE_FLOAT16) {
    if (sa)
      hipLaunchKernelGGL((decode64_kernel<IoF16, StF32, true>), grid, dim3(64), 0, s, p);
    else
      hipLaunchKernelGGL((decode64_kernel<IoF16, StF32>), grid, dim3(64), 0, s, p);
  } else {
    return FR2_ERR_UNSUPPORTED;
  }
  return record_launch();
}

}  // namespace fr2
