// Chunked WKV7 prefill with one wavefront per (sequence, head) unit (D = 64,
// fp32 state carry), for launches with many units.
//
// Same chunk algebra as chunk.hip (L = 16 tokens, S0 = start-of-chunk state,
// gamma_t = cumulative retention inside the chunk):
//   A~ = a*gamma_{t-1}, R~ = r*gamma_t, B^ = b/gamma_t, K^ = k/gamma_t
//   T = (I - strict_tril(A~ B^T))^-1
//   U = T (A~ S0 + Mak V),  Y = R~ S0 + Mrb U + Mrk V,
//   S_L = diag(gamma_L) (S0 + B^^T U + K^^T V)
// with every product on v_mfma_f32_16x16x32_bf16 over bf16 hi/lo split
// operands (fp32-level accuracy).
//
// chunk64_kernel spreads one unit over a 512-thread workgroup whose waves
// hand operators to each other through LDS; that is the fastest form when
// there is at most one unit per CU.  With many units the per-unit pipeline's
// hand-offs and shared operand reads cost more than they save: here one
// wave does all of a unit's work, keeping the whole 64x64 state in 64
// accumulator registers, and the SIMDs hide one wave's latency with another
// unit's wave.  Nothing is exchanged between waves; LDS holds only each
// wave's own transposes (B^, K^ and V rows read back as K = token operands)
// and output staging.
//
// Register layout of lane (i, q) = (lane % 16, lane / 16):
//   token operands (the A-operand layout): token i of the chunk, keys
//     32m + 8q .. 32m + 8q + 7 for the two K steps m = 0, 1;
//   state tile S[kb][vb] (accumulator layout): value column 16vb + i, keys
//     32(kb/2) + 8q + 4(kb%2) + e, e = 0..3.  With this key order the tiles
//     2m and 2m+1 of a column block are the B operand of K step m as they
//     stand, and the transposed reads of B^ / K^ address the same keys.
#include "mfma.h"
#include "recurrent.h"

namespace fr2 {
namespace {

constexpr int D = 64;
constexpr int L = 16;
// waves (units) per workgroup: occupancy is set by the per-SIMD wave bound
// either way; two-wave workgroups free their LDS at a finer grain
// (2 048 x 100 tokens: 1.94 vs 1.98 ms for four, 2.06 for eight; config 3
// equal; same process, outputs bit-identical)
constexpr int WPB = 2;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegExpHalf = -0.6065306597126334f;   // -exp(-1/2)

constexpr int kOrderMaxSeqs = 256;   // longest-first order up to this many sequences
constexpr int kOrderMinSeqlen = 256; // ... whose longest has at least this many tokens

constexpr int YPW = D + 8;            // padded row of the staged outputs

// One wave's LDS: its chunk's B^, K^ (hi and lo) and V rows, read back
// transposed, gamma_L and the chunk's staged y rows; with the fused readout
// (kRO) also each token's r k' r_k sum and the GroupNorm weight and bias.
template <bool kVExact, bool kRO>
struct alignas(16) WaveLds {
  static constexpr int TP = kVExact ? D + 16 : D + 8;   // token row pitch
  float gl[D];
  __bf16 b_h[L][TP], b_l[L][TP], k_h[L][TP], k_l[L][TP], v_h[L][TP];
  __bf16 v_l[kVExact ? 1 : L][TP];                       // fp16 tokens only
  uint16_t yb[L][YPW];                                   // the chunk's y rows
  float rkv[kRO ? L : 4];
  float lnw[kRO ? D : 4], lnb[kRO ? D : 4];   // the readout's GroupNorm weight and bias
};
using WaveLdsB = WaveLds<true, false>;
using WaveLdsH = WaveLds<false, false>;
using WaveLdsBR = WaveLds<true, true>;
using WaveLdsHR = WaveLds<false, true>;
static_assert(sizeof(WaveLdsB::b_h) >= kOrderMaxSeqs * sizeof(int),
              "the sequence lengths of the longest-first order fit in b_h");
static_assert(sizeof(WaveLdsB) % 16 == 0 && sizeof(WaveLdsH) % 16 == 0 &&
                  sizeof(WaveLdsBR) % 16 == 0 && sizeof(WaveLdsHR) % 16 == 0,
              "wave blocks must keep 16-byte alignment");
static_assert(offsetof(WaveLdsB, b_h) % 16 == 0 && offsetof(WaveLdsH, v_l) % 16 == 0 &&
                  offsetof(WaveLdsBR, yb) % 16 == 0 && offsetof(WaveLdsHR, yb) % 16 == 0,
              "row arrays must be 16-byte aligned");

// Longest-first order of the sequences of a packed batch: with one wave per
// unit, a long sequence is one long serial chain, so it has to start first
// (the units of shorter sequences fill the SIMDs around it).  Returns the
// index of the sequence of rank `rank` among sequences [0, n) by decreasing
// length (ties by index), or -1 when rank >= n.  `len` is wave-private LDS
// for n ints (rounded up to 4); the ranking costs each wave O(n^2 / 64)
// comparisons, so it is used for small n only (kOrderMaxSeqs).
__device__ __attribute__((noinline)) int seq_of_rank(const int32_t* bounds, int n, int rank, int* len,
                                                     int lane) {
  // lengths padded to a multiple of 4 with -1 (shorter than any sequence),
  // compared four at a time from one 16-byte LDS read
  const int n4 = (n + 3) & ~3;
  for (int k = lane; k < n4; k += 64) len[k] = k < n ? bounds[k + 1] - bounds[k] : -1;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);   // one wave: its LDS accesses complete in order
  for (int j0 = 0; j0 < n; j0 += 64) {
    const int j = j0 + lane;
    const int lj = j < n ? len[j] : -1;
    int r = 0;
    for (int k = 0; k < n4; k += 4) {
      const int4 l4 = *reinterpret_cast<const int4*>(&len[k]);
      r += (l4.x > lj || (l4.x == lj && k < j)) ? 1 : 0;
      r += (l4.y > lj || (l4.y == lj && k + 1 < j)) ? 1 : 0;
      r += (l4.z > lj || (l4.z == lj && k + 2 < j)) ? 1 : 0;
      r += (l4.w > lj || (l4.w == lj && k + 3 < j)) ? 1 : 0;
    }
    const uint64_t hit = __ballot(j < n && r == rank);
    if (hit != 0) return j0 + __builtin_ctzll(hit);
  }
  return -1;
}

// key held by item e of state tile kb in lane group q
__device__ __forceinline__ int tile_key(int kb, int q, int e) {
  return 32 * (kb >> 1) + 8 * q + 4 * (kb & 1) + e;
}

// kOrder: the units run in longest-first order of their sequences (packed
// batches of at most kOrderMaxSeqs sequences).  kSa: also write every
// token's pre-update sa = S_{t-1}^T a_t (the rows of U) to p.sa_out (the
// rl_infctx replay).  kKK: the kk / a-gate stage of wkv_prepare in the load
// stage (k is the projected key, slot a the a-gate logits a12; the gated
// key goes to p.new_k), and kRO with it the readout's elementwise stage in
// the output write-back (p.ro_out; y itself only when p.y is set).
template <class Io, bool kOrder, bool kSa = false, bool kKK = false, bool kRO = false>
__global__ __launch_bounds__(64 * WPB, 2) void chunk64w_kernel(SegArgs p, int nunits) {
  using raw = typename Io::raw;
  constexpr bool kVExact = !__is_same(Io, IoF16);
  __shared__ WaveLds<kVExact, kRO> lds[WPB];
  // per-channel parameters of each wave's head, staged once: -log2(e) times
  // the decay bias, and (fused stages) k_k, the a-gate bias a0, k_a, r_k
  // (kept apart from the wave blocks, whose layout they would shift)
  __shared__ __attribute__((aligned(16))) float chp_all[WPB][(kKK || kRO) ? 5 : 1][D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15;
  const int q = lane >> 4;
  const int H = p.num_heads;
  raw* yout = static_cast<raw*>(p.y);
  if (p.status != nullptr && p.status[0] != 0) {
    if (!kRO || yout != nullptr) fill_output_nan<Io>(yout, p.out_elems, blockIdx.x, gridDim.x);
    if constexpr (kRO)
      fill_output_nan<Io>(static_cast<raw*>(p.ro_out), p.out_elems, blockIdx.x, gridDim.x);
    return;
  }
  // the heads of a sequence are adjacent units (adjacent 128-byte pieces of
  // every token row)
  const int unit = blockIdx.x * WPB + wv;
  if (unit >= nunits) return;
  WaveLds<kVExact, kRO>& sm = lds[wv];
  int seg = unit / H;
  const int h = unit - seg * H;
  const int nseq = nunits / H;
  const int nactive = p.status != nullptr ? min(p.status[2], nseq) : nseq;
  if (seg >= nactive) return;
  if (kOrder && nactive > 1) {
    // wave-uniform: keep the unit's indices in scalar registers
    seg = __builtin_amdgcn_readfirstlane(
        seq_of_rank(p.bounds, nactive, seg, reinterpret_cast<int*>(&sm.b_h[0][0]), lane));
    if (seg < 0) return;
  }
  int t0, t1, slot;
  resolve_segment(p, seg, t0, t1, slot);

  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(H) * D;
  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;

  f32x4 S[4][4];   // [kb][vb]
  // fp32 state, or (bf16-state contract) bf16 widened once; the state stays
  // fp32 for the whole call and is rounded back once at the end (one branch
  // around each loop: a per-element select compiles to a branch per load)
  if (p.state_in != nullptr && p.state_bf16) {
    const uint16_t* sinb = static_cast<const uint16_t*>(p.state_in) + sbase + i;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          S[kb][vb][e] = IoBF16::to_f32(sinb[tile_key(kb, q, e) * D + 16 * vb]);
  } else if (p.state_in != nullptr) {
    const float* sin = static_cast<const float*>(p.state_in) + sbase + i;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][vb][e] = sin[tile_key(kb, q, e) * D + 16 * vb];
  } else {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int vb = 0; vb < 4; ++vb) S[kb][vb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // token rows of lane (i, q): row t of tensor j, keys 32m + 8q ..
  const raw* src[6] = {static_cast<const raw*>(p.r), static_cast<const raw*>(p.logits),
                       static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
                       static_cast<const raw*>(p.a), static_cast<const raw*>(p.b)};
  const raw* bias = static_cast<const raw*>(p.bias);
  // Addresses: a wave-uniform 64-bit base per chunk (kept in scalar
  // registers) plus a 32-bit per-lane byte offset within the chunk's 16 rows,
  // so that no 64-bit per-lane pointer has to stay live (or spill) across
  // the loop.  Rows past the segment end are read from its last row (always
  // in bounds) and zeroed when used.
  const int64_t rs_bytes = row_stride * static_cast<int64_t>(sizeof(raw));
  // the fp32 row stride in bytes, 32 bits (a row is H * 64 elements)
  const uint32_t rs4 = static_cast<uint32_t>(row_stride * static_cast<int64_t>(sizeof(float)));
  auto chunk_base = [&](const void* ptr, int c) {
    return static_cast<const char*>(ptr) + static_cast<int64_t>(t0 + c * L) * rs_bytes +
           head_off * static_cast<int64_t>(sizeof(raw));
  };
  // plain (cached) loads: a lane's two 16-byte pieces of a row are half
  // cache lines whose other halves the neighbouring lanes load in the same
  // instruction pair, and measured 2-5 % faster than non-temporal loads
  auto load_rows = [&](u32x4 (&dst)[6][2], int c) {
    const uint32_t lane_b = static_cast<uint32_t>(
        static_cast<int64_t>(min(t0 + c * L + i, t1 - 1) - (t0 + c * L)) * rs_bytes +
        16 * q);
#pragma unroll
    for (int j = 0; j < 6; ++j) {
      const char* base = chunk_base(src[j], c);
#pragma unroll
      for (int m = 0; m < 2; ++m)
        dst[j][m] = (kKK && j == 5)   // b is formed from the key with the gate stage
                        ? u32x4{0u, 0u, 0u, 0u}
                        : *reinterpret_cast<const u32x4*>(base + lane_b + 64 * m);
    }
  };
  // per-channel parameters of the lane's 8 keys of K step m (read where used:
  // they would otherwise hold 16-64 registers across the whole loop)
  // (called with the chunk's opaque lane index, so that the per-lane
  // addresses are formed per chunk instead of being hoisted and spilled)
  // They come from the wave's LDS copy (staged below): a global load here
  // would be issued after the next chunk's row requests, and the vector-
  // memory counter is in order, so waiting for it waited for those rows.
  auto channel8 = [&](int which, int m, float* out, int lq) {
    const float* a = &chp_all[wv][which][32 * m + 8 * lq];
    *reinterpret_cast<f32x4*>(out) = *reinterpret_cast<const f32x4*>(a);
    *reinterpret_cast<f32x4*>(out + 4) = *reinterpret_cast<const f32x4*>(a + 4);
  };
  {
    auto stage = [&](int which, const void* base, float scale) {
      chp_all[wv][which][lane] =
          base != nullptr ? scale * Io::to_f32(static_cast<const raw*>(base)[head_off + lane]) : 0.0f;
    };
    if (bias != nullptr) stage(0, bias, -kLog2e);
    if constexpr (kKK) {
      stage(1, p.kk_scale, 1.0f);
      stage(2, p.a_bias, 1.0f);
      stage(3, p.k_a, 1.0f);
    }
    if constexpr (kRO) stage(4, p.ro_rk, 1.0f);
  }

  constexpr float kC = kNegExpHalf * kLog2e;
  constexpr float kInvC = 1.0f / kC;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const int nchunks = (t1 - t0 + L - 1) / L;
  if constexpr (kRO) {
    sm.lnw[lane] = Io::to_f32(static_cast<const raw*>(p.ro_lnw)[head_off + lane]);
    sm.lnb[lane] = Io::to_f32(static_cast<const raw*>(p.ro_lnb)[head_off + lane]);
  }
  u32x4 rows[6][2];
  if (nchunks > 0) load_rows(rows, 0);
  for (int c = 0; c < nchunks; ++c) {
    // the lane's (i, q), opaque once per chunk: the token masks and the
    // identity derived from them are then formed where used instead of being
    // hoisted out of the loop into registers (where they would spill)
    int li = i, lq = q;
    asm volatile("" : "+v"(li), "+v"(lq));
    const bool valid = t0 + c * L + i < t1;
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    // ---- operands of the chunk (keys of K step m in registers)
    Sp8 As[2], Rs[2], Bs[2], Ks[2];
    // fused kk stage: 1 / |k k_k| over the token's 64 keys (the four lanes of
    // token i hold 16 each)
    float kinv = 0.0f;
    if constexpr (kKK) {
      float ss = 0.0f;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        float xk[8], kks[8];
        unpack8<Io>(rows[2][m], xk);
        channel8(1, m, kks, lq);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float u = xk[e] * kks[e];
          ss = __builtin_fmaf(u, u, ss);
        }
      }
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      kinv = __builtin_amdgcn_rcpf(fmaxf(__builtin_sqrtf(ss), 1.0e-12f));
    }
    float rkv_part = 0.0f;   // fused readout: sum over the lane's keys of r k' r_k
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      __builtin_amdgcn_sched_barrier(0);
      float xr[8], xl[8], xk[8], xa[8], xb[8];
      unpack8<Io>(valid ? rows[0][m] : zero4, xr);
      unpack8<Io>(rows[1][m], xl);
      if constexpr (kKK) {
        // u = k k_k, kk = u / |u|, g = sigmoid(a0 + a12), k' = k (1 + (g - 1) k_a),
        // a = -kk, b = kk g (csrc/prepare.hip kk_a_gate_kernel, in fp32)
        float kks[8], a0[8], ka[8], x12[8];
        unpack8<Io>(rows[2][m], xk);
        unpack8<Io>(rows[4][m], x12);
        channel8(1, m, kks, lq);
        channel8(2, m, a0, lq);
        channel8(3, m, ka, lq);
        u32x4 packed;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float kk = xk[e] * kks[e] * kinv;
          const float g = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2e * (a0[e] + x12[e])));
          const float nk = xk[e] * __builtin_fmaf(g - 1.0f, ka[e], 1.0f);
          xa[e] = -kk;
          xb[e] = valid ? kk * g : 0.0f;
          xk[e] = valid ? nk : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          packed[j] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Io::from_f32(xk[2 * j]))) |
                      (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Io::from_f32(xk[2 * j + 1])))
                       << 16);
        if (valid)
          *reinterpret_cast<u32x4*>(const_cast<char*>(chunk_base(p.new_k, c)) +
                                    static_cast<uint32_t>(li * rs_bytes + 16 * lq + 64 * m)) = packed;
        if constexpr (kRO) {
          // the readout's residual weight uses the key as stored
          float kq[8], rk[8];
          unpack8<Io>(packed, kq);
          channel8(4, m, rk, lq);
#pragma unroll
          for (int e = 0; e < 8; ++e) rkv_part = __builtin_fmaf(xr[e] * kq[e], rk[e], rkv_part);
        }
      } else {
        unpack8<Io>(valid ? rows[2][m] : zero4, xk);
        unpack8<Io>(valid ? rows[4][m] : zero4, xa);
        unpack8<Io>(valid ? rows[5][m] : zero4, xb);
      }
      float nb[8];   // -log2(e) decay_bias
      if (bias != nullptr) {
        channel8(0, m, nb, lq);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) nb[e] = 0.f;
      }
      // log2 of the retention, log2(w) = c sigmoid(x) with c = -exp(-1/2)
      // log2(e), as 1 / ((1 + 2^(-log2(e) x)) / c); then its prefix sum over
      // the chunk's tokens (the 16 lanes of a DPP row)
      float g2[8], gm[8], gp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) g2[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(xl[e], -kLog2e, nb[e]));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float lw2 = __builtin_amdgcn_rcpf(__builtin_fmaf(g2[e], kInvC, kInvC));
        g2[e] = valid ? lw2 : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) g2[e] += row_shr<1>(g2[e]);
#pragma unroll
      for (int e = 0; e < 8; ++e) g2[e] += row_shr<2>(g2[e]);
#pragma unroll
      for (int e = 0; e < 8; ++e) g2[e] += row_shr<4>(g2[e]);
#pragma unroll
      for (int e = 0; e < 8; ++e) g2[e] += row_shr<8>(g2[e]);
#pragma unroll
      for (int e = 0; e < 8; ++e) gm[e] = __builtin_amdgcn_exp2f(g2[e]);      // gamma_t
#pragma unroll
      for (int e = 0; e < 8; ++e) gp[e] = row_prev(gm[e], 1.0f);              // gamma_{t-1}
      float at[8], rt[8], bh[8], kh[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ig = __builtin_amdgcn_exp2f(-g2[e]);                     // 1 / gamma_t
        at[e] = xa[e] * gp[e];
        rt[e] = xr[e] * gm[e];
        bh[e] = xb[e] * ig;
        kh[e] = xk[e] * ig;
      }
      if (i == L - 1) {
        *reinterpret_cast<f32x4*>(&sm.gl[32 * m + 8 * q]) = f32x4{gm[0], gm[1], gm[2], gm[3]};
        *reinterpret_cast<f32x4*>(&sm.gl[32 * m + 8 * q + 4]) = f32x4{gm[4], gm[5], gm[6], gm[7]};
      }
      As[m] = split8(at);
      Rs[m] = split8(rt);
      Bs[m] = split8(bh);
      Ks[m] = split8(kh);
      const int col = 32 * m + 8 * q;
      *reinterpret_cast<bf16x8*>(&sm.b_h[i][col]) = Bs[m].hi;
      *reinterpret_cast<bf16x8*>(&sm.b_l[i][col]) = Bs[m].lo;
      *reinterpret_cast<bf16x8*>(&sm.k_h[i][col]) = Ks[m].hi;
      *reinterpret_cast<bf16x8*>(&sm.k_l[i][col]) = Ks[m].lo;
      const u32x4 vraw = valid ? rows[3][m] : zero4;
      if constexpr (kVExact) {
        *reinterpret_cast<u32x4*>(&sm.v_h[i][col]) = vraw;      // bf16 values are exact
      } else {
        float xv[8];
        unpack8<Io>(vraw, xv);
        const Sp8 vs = split8(xv);
        *reinterpret_cast<bf16x8*>(&sm.v_h[i][col]) = vs.hi;
        *reinterpret_cast<bf16x8*>(&sm.v_l[i][col]) = vs.lo;
      }
    }

    if constexpr (kRO) {
      rkv_part += __shfl_xor(rkv_part, 16);
      rkv_part += __shfl_xor(rkv_part, 32);
      if (q == 0) sm.rkv[i] = rkv_part;
    }

    // ---- token-token blocks over the 64 keys.  mma32(X, Y) gives lane
    // (i, q) item e = X_{4q+e} . Y_i, so each block is formed directly in
    // the orientation its consumer needs.
    __builtin_amdgcn_sched_barrier(0);
    f32x4 mab = zero, mabt = zero, makt = zero, mrbt = zero, mrkt = zero;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      mab = mma32x3(As[m], Bs[m], mab);     // Mab[4q+e][i]
      mabt = mma32x3(Bs[m], As[m], mabt);   // Mab[i][4q+e]
      makt = mma32x3(Ks[m], As[m], makt);   // Mak[i][4q+e]  (A-operand form)
      mrbt = mma32x3(Bs[m], Rs[m], mrbt);   // Mrb[i][4q+e]
      mrkt = mma32x3(Ks[m], Rs[m], mrkt);   // Mrk[i][4q+e]
    }
    f32x4 M, Mt, mak, mrb, mrk;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = 4 * lq + e;
      M[e] = (s > li) ? mab[e] : 0.f;
      Mt[e] = (li > s) ? mabt[e] : 0.f;
      mak[e] = (li > s) ? makt[e] : 0.f;
      mrb[e] = (li >= s) ? mrbt[e] : 0.f;
      mrk[e] = (li >= s) ? mrkt[e] : 0.f;
    }
    __builtin_amdgcn_sched_barrier(0);
    const AOp Ta = t_inverse(M, Mt, li, lq);
    const AOp Mak = as_a(split4(mak));
    const AOp Mrb = as_a(split4(mrb));
    const AOp Mrk = as_a(split4(mrk));

    // ---- state chain.  B^^T and K^^T as A operands (row = key of tile kb,
    // K = token); gamma_L of the tile rows is read where it is applied.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int trow = 4 * q + (i >> 2);
#pragma unroll
    for (int vb = 0; vb < 4; ++vb) {
      // the column blocks in two regions of two: a scheduler free to hoist
      // every block's LDS reads to the top needs ~100 more registers
      if (vb == 2) __builtin_amdgcn_sched_barrier(0);
      Sp8 Sb[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const Split4 x = split4(S[2 * m][vb]), y = split4(S[2 * m + 1][vb]);
        Sb[m].hi = __builtin_bit_cast(bf16x8, u32x4{x.h0, x.h1, y.h0, y.h1});
        Sb[m].lo = __builtin_bit_cast(bf16x8, u32x4{x.l0, x.l1, y.l0, y.l1});
      }
      // V[4q+e][16vb+i] as the K = token operand
      const bf16x4 vh = tr_rows(&sm.v_h[trow][16 * vb + 4 * (i & 3)]);
      auto times_v = [&](AOp a, f32x4 acc) {
        if constexpr (kVExact) {
          return mm_ax(a, as_bx(vh), acc);
        } else {
          const bf16x4 vl = tr_rows(&sm.v_l[trow][16 * vb + 4 * (i & 3)]);
          return mm_ab(a, as_b(vh, vl), acc);
        }
      };
      f32x4 X = times_v(Mak, zero);
      f32x4 Y = times_v(Mrk, zero);
      X = mma32x3(As[0], Sb[0], X);
      X = mma32x3(As[1], Sb[1], X);
      Y = mma32x3(Rs[0], Sb[0], Y);
      Y = mma32x3(Rs[1], Sb[1], Y);
      const f32x4 Uf = mm_ab(Ta, as_b(split4(X)), zero);
      if constexpr (kSa) {
        // sa rows 4q + e, column 16vb + i
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t0 + c * L + 4 * q + e < t1)
            *reinterpret_cast<float*>(
                reinterpret_cast<char*>(p.sa_out + (static_cast<int64_t>(t0 + c * L) * row_stride +
                                                    head_off)) +
                (static_cast<uint32_t>(4 * q + e) * rs4 + (16 * vb + i) * 4u)) = Uf[e];
      }
      const BOp Us = as_b(split4(Uf));
      Y = mm_ab(Mrb, Us, Y);
      // y rows 4q + e, column 16vb + i, staged in LDS: the chunk's rows then
      // leave as whole 32-byte pieces (2-byte stores straight from the
      // accumulators cost a quarter of the kernel's time)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        sm.yb[4 * q + e][16 * vb + i] = __builtin_bit_cast(uint16_t, Io::from_f32(p.scale * Y[e]));
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        // B^^T and K^^T of tile kb as A operands (row = key, K = token)
        const int col = 32 * (kb >> 1) + 8 * (i & 3) + 4 * (kb & 1);
        const AOp Bt = __builtin_shufflevector(tr_rows(&sm.b_h[trow][col]),
                                               tr_rows(&sm.b_l[trow][col]), 0, 1, 2, 3, 4, 5, 6, 7);
        const AOp Kt = __builtin_shufflevector(tr_rows(&sm.k_h[trow][col]),
                                               tr_rows(&sm.k_l[trow][col]), 0, 1, 2, 3, 4, 5, 6, 7);
        f32x4 acc = mm_ab(Bt, Us, S[kb][vb]);
        acc = times_v(Kt, acc);
        S[kb][vb] = acc * *reinterpret_cast<const f32x4*>(&sm.gl[tile_key(kb, q, 0)]);
      }
    }
    // the next chunk's rows are requested before this chunk's output stores
    // (the other units' waves on the SIMD cover their latency)
    __builtin_amdgcn_sched_barrier(0);
    // fused readout: this lane's 16 gate values of the chunk's write-back
    // (token lane / 4, channels 16 (lane % 4) ..), requested where they are
    // used: requested a chunk ahead, their 8 registers stayed live through
    // the whole chunk and pushed other values into scratch (3.48 vs 3.01 ms
    // on a 2 048 x 100-token serving batch)
    u32x4 gpre[2];
    if constexpr (kRO) {
      const char* gb = chunk_base(p.ro_g, c) +
                       static_cast<uint32_t>((min(t0 + c * L + (lane >> 2), t1 - 1) - (t0 + c * L)) *
                                                 rs_bytes +
                                             32 * (lane & 3));
      gpre[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gb));
      gpre[1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(gb + 16));
    }
    if constexpr (kRO) {
      // fused readout of the chunk's rows: lane l takes 16 channels of token
      // l / 4; GroupNorm over the head's 64 channels (4 lanes per token),
      // the r k' r_k residual and the gate:
      //   out = (GroupNorm(y) ln_w + ln_b + (sum r k' r_k) v) g
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const int orow = lane >> 2, oc = 16 * (lane & 3);
      const int tok = t0 + c * L + orow;
      // byte offset of this lane's 16 channels within the chunk's rows
      const uint32_t rb = static_cast<uint32_t>((min(tok, t1 - 1) - (t0 + c * L)) * rs_bytes +
                                                oc * sizeof(raw));
      const u32x4 yp[2] = {*reinterpret_cast<const u32x4*>(&sm.yb[orow][oc]),
                           *reinterpret_cast<const u32x4*>(&sm.yb[orow][oc + 8])};
      float yv[16];
      unpack8<Io>(yp[0], yv);
      unpack8<Io>(yp[1], yv + 8);
      float s1 = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) s1 += yv[e];
      s1 += __shfl_xor(s1, 1);
      s1 += __shfl_xor(s1, 2);
      const float mean = s1 * (1.0f / D);
      float s2 = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) s2 = __builtin_fmaf(yv[e] - mean, yv[e] - mean, s2);
      s2 += __shfl_xor(s2, 1);
      s2 += __shfl_xor(s2, 2);
      const float inv = 1.0f / __builtin_sqrtf(s2 * (1.0f / D) + 64.0e-5f);
      const float rkv = sm.rkv[orow];
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        // ln weight / bias from LDS, v from this chunk's V rows in LDS (for
        // fp16 tokens hi + lo, which is exact), the gate from the prefetch
        float w8[8], b8[8], v8[8], g8[8];
        const int ch = oc + 8 * hp;
        *reinterpret_cast<f32x4*>(w8) = *reinterpret_cast<const f32x4*>(&sm.lnw[ch]);
        *reinterpret_cast<f32x4*>(w8 + 4) = *reinterpret_cast<const f32x4*>(&sm.lnw[ch + 4]);
        *reinterpret_cast<f32x4*>(b8) = *reinterpret_cast<const f32x4*>(&sm.lnb[ch]);
        *reinterpret_cast<f32x4*>(b8 + 4) = *reinterpret_cast<const f32x4*>(&sm.lnb[ch + 4]);
        if constexpr (kVExact) {
          unpack8<IoBF16>(*reinterpret_cast<const u32x4*>(&sm.v_h[orow][ch]), v8);
        } else {
          float vl8[8];
          unpack8<IoBF16>(*reinterpret_cast<const u32x4*>(&sm.v_h[orow][ch]), v8);
          unpack8<IoBF16>(*reinterpret_cast<const u32x4*>(&sm.v_l[orow][ch]), vl8);
#pragma unroll
          for (int e = 0; e < 8; ++e) v8[e] += vl8[e];
        }
        unpack8<Io>(gpre[hp], g8);
        // y re-read from LDS rather than kept live since the statistics
        float y8[8];
        unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.yb[orow][ch]), y8);
        u32x4 packed;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float o2[2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int e = 2 * j + h2;
            o2[h2] = (__builtin_fmaf((y8[e] - mean) * inv, w8[e], b8[e]) + rkv * v8[e]) *
                     g8[e];
          }
          packed[j] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Io::from_f32(o2[0]))) |
                      (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Io::from_f32(o2[1])))
                       << 16);
        }
        if (tok < t1) {
          *reinterpret_cast<u32x4*>(const_cast<char*>(chunk_base(p.ro_out, c)) + rb + 16 * hp) =
              packed;
          if (yout != nullptr)
            *reinterpret_cast<u32x4*>(const_cast<char*>(chunk_base(yout, c)) + rb + 16 * hp) =
                yp[hp];
        }
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    if (c + 1 < nchunks) load_rows(rows, c + 1);
    if constexpr (!kRO) {
      // the staged y rows: lane l writes 16 channels of token l / 4 (issued
      // after the next chunk's row loads, which then do not wait for them)
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      const int orow = lane >> 2, oc = 16 * (lane & 3);
      if (t0 + c * L + orow < t1) {
        char* dst = const_cast<char*>(chunk_base(yout, c)) +
                    static_cast<uint32_t>(orow * rs_bytes + oc * sizeof(raw));
        *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(&sm.yb[orow][oc]);
        *reinterpret_cast<u32x4*>(dst + 16) = *reinterpret_cast<const u32x4*>(&sm.yb[orow][oc + 8]);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  }

  if (p.state_out != nullptr && p.state_bf16) {
    uint16_t* soutb = static_cast<uint16_t*>(p.state_out) + sbase + i;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          soutb[tile_key(kb, q, e) * D + 16 * vb] = IoBF16::from_f32(S[kb][vb][e]);
  } else if (p.state_out != nullptr) {
    float* sout = static_cast<float*>(p.state_out) + sbase + i;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sout[tile_key(kb, q, e) * D + 16 * vb] = S[kb][vb][e];
  }
}

}  // namespace

namespace {

template <class Io>
void launch_wave_io(const SegArgs& p, int n, bool order, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((n + WPB - 1) / WPB)), block(64 * WPB);
  const bool kk = p.kk_scale != nullptr, ro = p.ro_out != nullptr;
  if (p.sa_out != nullptr)
    hipLaunchKernelGGL((chunk64w_kernel<Io, false, true>), grid, block, 0, s, p, n);
  else if (kk && ro && order)
    hipLaunchKernelGGL((chunk64w_kernel<Io, true, false, true, true>), grid, block, 0, s, p, n);
  else if (kk && ro)
    hipLaunchKernelGGL((chunk64w_kernel<Io, false, false, true, true>), grid, block, 0, s, p, n);
  else if (kk && order)
    hipLaunchKernelGGL((chunk64w_kernel<Io, true, false, true>), grid, block, 0, s, p, n);
  else if (kk)
    hipLaunchKernelGGL((chunk64w_kernel<Io, false, false, true>), grid, block, 0, s, p, n);
  else if (order)
    hipLaunchKernelGGL((chunk64w_kernel<Io, true>), grid, block, 0, s, p, n);
  else
    hipLaunchKernelGGL((chunk64w_kernel<Io, false>), grid, block, 0, s, p, n);
}

}  // namespace

bool wave_longest_first(int nseg, int max_seqlen, int64_t total_tokens) {
  return nseg > 1 && nseg <= kOrderMaxSeqs && max_seqlen >= kOrderMinSeqlen &&
         4 * static_cast<int64_t>(max_seqlen) * nseg > 5 * total_tokens;
}

int launch_chunked_wave(int dtype, const SegArgs& p, int nseg, int max_seqlen, hipStream_t s) {
  if (p.boundary != nullptr || p.reverse || p.split_pieces > 0) return FR2_ERR_UNSUPPORTED;
  const bool kk = p.kk_scale != nullptr, ro = p.ro_out != nullptr;
  // the fused stages: the gate needs all its inputs, the readout needs the
  // gate, and neither combines with the replay's sa output or a bf16 state
  if ((kk || ro) && (p.sa_out != nullptr || p.state_bf16 || p.a_bias == nullptr ||
                     p.k_a == nullptr || p.new_k == nullptr || !kk))
    return FR2_ERR_INVALID_ARGUMENT;
  if (ro && (p.ro_g == nullptr || p.ro_rk == nullptr || p.ro_lnw == nullptr ||
             p.ro_lnb == nullptr))
    return FR2_ERR_INVALID_ARGUMENT;
  const int64_t units = static_cast<int64_t>(nseg) * p.num_heads;
  if (units <= 0 || units > (int64_t{1} << 30)) return FR2_ERR_INVALID_ARGUMENT;
  // the longest-first order pays when a long sequence would otherwise start
  // late: packed batches of at most kOrderMaxSeqs sequences whose longest is
  // at least kOrderMinSeqlen tokens and a quarter above the mean (the ranking
  // costs each wave O(n^2 / 256) LDS steps)
  const int64_t total = p.out_elems / (static_cast<int64_t>(p.num_heads) * D);
  const bool order = p.uniform_len <= 0 && p.chunk_offsets == nullptr && p.ends == nullptr &&
                     wave_longest_first(nseg, max_seqlen, total);
  const int n = static_cast<int>(units);
  if (dtype == FR2_DTYPE_BFLOAT16)
    launch_wave_io<IoBF16>(p, n, order, s);
  else if (dtype == FR2_DTYPE_FLOAT16)
    launch_wave_io<IoF16>(p, n, order, s);
  else
    return FR2_ERR_UNSUPPORTED;
  return record_launch();
}

}  // namespace fr2
