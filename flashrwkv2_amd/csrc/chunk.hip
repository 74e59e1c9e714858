// Chunked WKV7 prefill on gfx950 matrix cores (D = 64, fp32 state carry).
//
// Chunk algebra (L = 16 tokens, rows = tokens, S0 = start-of-chunk state,
// g_t = sum_{s<=t} log w_s inside the chunk, gamma_t = exp(g_t)):
//   A~ = a*gamma_{t-1}, R~ = r*gamma_t, B^ = b/gamma_t, K^ = k/gamma_t
//   Mab = strict_tril(A~ B^T), Mak = strict_tril(A~ K^T)
//   Mrb = tril(R~ B^T),        Mrk = tril(R~ K^T)
//   T = (I - Mab)^-1
//   U (the per-token sa rows) = T (A~ S0 + Mak V)
//   Y = R~ S0 + Mrb U + Mrk V                     (y = scale * Y)
//   S_L = diag(gamma_L) (S0 + B^^T U + K^^T V)
// which is the per-token recurrence
//   sa_t = S_{t-1}^T a_t, S_t = diag(w_t) S_{t-1} + b_t sa_t^T + k_t v_t^T,
//   y_t = scale * S_t^T r_t
// unrolled over the chunk.  Every product runs on
// v_mfma_f32_16x16x32_bf16 with both operands split into bf16 hi + lo
// (hi*hi + hi*lo + lo*hi, fp32 accumulation): fp32-level accuracy.  Raw bf16
// token values (V) are exact and carry no lo part.
//
// Work layout: one 512-thread workgroup per (sequence, head), walking the
// sequence in groups of G = 2 chunks, with two wave roles that run
// concurrently on the 4 SIMDs:
//   key waves (4-7), one (chunk, key half) each, prepare the operators of the
//     NEXT group: token rows loaded straight from HBM (prefetched one group
//     ahead), decays by a 16-lane DPP scan over tokens, operands built in
//     registers, the token-token blocks computed from those registers (each
//     lane's 8 keys are its own MFMA K positions); after the mid-iteration
//     barrier they store the operands for the state waves, and one of the two
//     waves of a chunk forms T by repeated squaring (I+M)(I+M^2)(I+M^4)(I+M^8)
//     (both orientations of every factor in registers);
//   state waves (0-3), state columns [16w, 16w+16) each, run the sequential
//     state path of the CURRENT group, one chunk per half-iteration.  The
//     state never leaves fp32 accumulator registers: accumulator rows are fed
//     to the matrix cores as B-operand K positions directly (the K order of a
//     dot product is free), and the accumulator layout of U is already the
//     B-operand layout of B^^T U.
// Operators are double-buffered in LDS by group parity; outputs are staged in
// LDS and written back as full 128-byte rows by the key waves.
#include "mfma.h"
#include "recurrent.h"

#include <atomic>
#include <cstddef>
#include <type_traits>

namespace fr2 {
namespace {

constexpr int D = 64;
constexpr int L = 16;          // tokens per chunk
constexpr int G = 2;           // chunks per group
constexpr int GT = L * G;      // tokens per group
constexpr int NT = 512;        // 8 wavefronts: 4 state + 4 key
constexpr int MPP = L + 4;     // padded row of the partial token-token blocks
constexpr int YP = D + 8;      // padded row of the staged outputs
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegExpHalf = -0.6065306597126334f;   // -exp(-1/2)

// Operators of one chunk consumed by the state path.  For bf16 tokens V is
// exact in bf16 (no lo part); fp16 tokens need V's lo part.
//
// Every row array is addressed through the piece swizzles a_col, b_col and
// aop_piece (unswizzled, the same accesses cost ~430 bank-conflict cycles
// per chunk).
template <bool kVExact>
struct alignas(16) ChunkOps {
  static constexpr int RP = D;                      // key row length
  static constexpr int TP = D + 16;                 // token row of B^, K^, V
  float gl[D];                        // gamma_L (read as 16-byte vectors)
  __bf16 at_h[L][RP], at_l[L][RP];    // A~ rows, keys at key_pos()
  __bf16 r_h[L][RP], r_l[L][RP];      // R~ rows, keys at key_pos()
  __bf16 b_h[L][TP], b_l[L][TP];      // B^ rows (natural key order)
  __bf16 k_h[L][TP], k_l[L][TP];      // K^ rows
  __bf16 v_h[L][TP];                  // V rows
  __bf16 v_l[kVExact ? 1 : L][TP];    // V lo part (fp16 tokens only)
  // 16x16 token-token operators in A-operand form: row i, positions
  // 8q..8q+7 = (hi of columns 4q..4q+3, lo of columns 4q..4q+3)
  __bf16 t[L][2 * L];                 // T
  __bf16 mak[L][2 * L], mrb[L][2 * L], mrk[L][2 * L];   // masked Mak, Mrb, Mrk
};
// every 16-byte vector access above needs its array 16-byte aligned
static_assert(offsetof(ChunkOps<true>, at_h) % 16 == 0 && offsetof(ChunkOps<true>, t) % 16 == 0 &&
                  offsetof(ChunkOps<false>, t) % 16 == 0,
              "row arrays must be 16-byte aligned");
static_assert(sizeof(ChunkOps<true>) % 16 == 0 && sizeof(ChunkOps<false>) % 16 == 0,
              "operator blocks must keep 16-byte alignment");

template <bool kVExact>
struct alignas(16) Smem {
  ChunkOps<kVExact> ops[2][G];        // [group parity][chunk]
  // partial token-token blocks, transposed (mpart[..][s][t] = P[t][s]) with
  // rows padded to MPP floats so that both the 16-byte row accesses and the
  // strided column reads spread over the banks
  float mpart[2][G][2][4][L][MPP];    // [group parity][chunk][key half][block][s][t]
  uint16_t yb[2][GT][YP];             // outputs of a group, by parity (padded rows)
  // fused readout: sum over a key half of r k' r_k per token of a group, by
  // group index mod 4 (written by the key waves building group g after the
  // state waves finished g - 2, read by the write-back of group g, which the
  // state waves run after finishing g + 1)
  float rkv[4][2][GT];
  // progress counters, each written by one wave only: groups whose operators
  // key wave w has stored, groups whose part-1 partials it has stored, and
  // groups state wave w has finished / whose output rows it has written back
  // (consumed has a slot for each of the summary pass's eight state waves)
  int ready[4], part1[4], drained[4], consumed[8];
  int fault;                          // a bounded wait gave up
};

// Column position of key k in the A~ / R~ rows: for each half m = k/32 the 32
// keys are ordered so that lane group q of the state product reads its 8 keys
// (the rows its state accumulators hold) as one contiguous 16-byte run.
__device__ __forceinline__ int key_pos(int k) {
  const int m = k >> 5, kk = k & 31;
  return 32 * m + 8 * ((kk & 15) >> 2) + 4 * (kk >> 4) + (kk & 3);
}

// A operand against the state: row t = lane%16 of X; positions 8q+idx map to
// key (2m + idx/4)*16 + 4q + idx%4, i.e. the rows the lane's state
// accumulators hold.
template <int RP>
__device__ __forceinline__ Sp8 rows_vs_state(const __bf16 (*xh)[RP], const __bf16 (*xl)[RP],
                                             int m, int i, int q) {
  Sp8 s;
  s.hi = *reinterpret_cast<const bf16x8*>(&xh[i][a_col(i, 32 * m + 8 * q)]);
  s.lo = *reinterpret_cast<const bf16x8*>(&xl[i][a_col(i, 32 * m + 8 * q)]);
  return s;
}

__device__ __forceinline__ AOp load_aop(const __bf16 (*x)[2 * L], int i, int q) {
  return *reinterpret_cast<const AOp*>(&x[i][8 * aop_piece(i, q)]);
}
__device__ __forceinline__ void store_aop(__bf16 (*x)[2 * L], int i, int q, const AOp& v) {
  *reinterpret_cast<AOp*>(&x[i][8 * aop_piece(i, q)]) = v;
}

// ---------------------------------------------------------------------------
// key side, part 1: operands of chunk cc (keys 32hh + 8q + e of token i) and
// the partial token-token blocks over this lane's keys.  The operand values
// stay in registers until part 2 stores them for the state waves.
// ---------------------------------------------------------------------------
struct KeyRegs {
  Sp8 As, Rs, Bs, Ks, Vs;
};

// kFull: every token of the chunk is inside the sequence (no masking).
// nbias8 holds -log2(e) * decay_bias for the lane's keys.
// kUnitW: reverse mode, where unit_w marks a lane whose shifted retention
// row lies past the segment (unit retention).
// kSum: summary pass (no R~ operands, no R-side blocks).
// Per-lane channel parameters of the fused kk / a-gate stage: k_k for the
// lane's keys of both key halves (own first), a0 and k_a for its own keys.
struct KkParams {
  float kk_own[8], kk_other[8], a0[8], ka[8];
};

template <class Io, bool kVExact, bool kFull, bool kUnitW = false, bool kSum = false,
          bool kKK = false, bool kRO = false>
__device__ __forceinline__ void key_part1(Smem<kVExact>& sm, ChunkOps<kVExact>& op,
                                          const u32x4 (&raw)[6], const float (&nbias8)[8],
                                          bool valid, int mp, int cc, int hh, int i, int q,
                                          KeyRegs& kr, bool unit_w = false,
                                          float kscale = 1.0f, const KkParams* kp = nullptr,
                                          typename Io::raw* new_k_row = nullptr,
                                          const float* rk8 = nullptr, float* rkv_row = nullptr) {
  const int kbase = 32 * hh + 8 * q;
  // tokens past the sequence end (their rows repeat the last token) carry
  // zero operands and a unit retention
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  auto tok = [&](int j) { return (kFull || valid) ? raw[j] : zero4; };
  float xr[8], xl[8], xk[8], xa[8], xb[8];
  if constexpr (!kSum) unpack8<Io>(tok(0), xr);
  unpack8<Io>(raw[1], xl);
  unpack8<Io>(tok(2), xk);
  if constexpr (kKK) {
    // Fused producer stage (the kk / a gate of wkv_prepare): raw[4] holds
    // the a-gate logits a12 and raw[5] the same 8 key positions of the other
    // key half, for the kk norm over all 64 keys:
    //   u = k k_k, kk = u / max(|u|, 1e-12), g = sigmoid(a0 + a12),
    //   k' = k (1 + (g - 1) k_a), a = -kk, b = kk g.
    float xo[8], x12[8];
    unpack8<Io>(tok(5), xo);
    unpack8<Io>(tok(4), x12);
    float u[8], ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      u[e] = xk[e] * kp->kk_own[e];
      const float w = xo[e] * kp->kk_other[e];
      ss = __builtin_fmaf(u[e], u[e], __builtin_fmaf(w, w, ss));
    }
    // the four lanes of token i (groups q = 0..3) hold all 64 keys
    ss += __shfl_xor(ss, 16);
    ss += __shfl_xor(ss, 32);
    const float inv = __builtin_amdgcn_rcpf(fmaxf(__builtin_sqrtf(ss), 1.0e-12f));
    float nk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float g = __builtin_amdgcn_rcpf(
          1.0f + __builtin_amdgcn_exp2f(-kLog2e * (kp->a0[e] + x12[e])));
      const float kk = u[e] * inv;
      nk[e] = xk[e] * __builtin_fmaf(g - 1.0f, kp->ka[e], 1.0f);
      xa[e] = -kk;
      xb[e] = kk * g;
    }
    if (new_k_row != nullptr && (kFull || valid)) {
      u32x4 packed;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = __builtin_bit_cast(uint16_t, Io::from_f32(nk[2 * j]));
        const uint32_t hi = __builtin_bit_cast(uint16_t, Io::from_f32(nk[2 * j + 1]));
        packed[j] = lo | (hi << 16);
      }
      *reinterpret_cast<u32x4*>(new_k_row) = packed;
    }
    // the recurrence uses the gated key (masked rows stay zero)
#pragma unroll
    for (int e = 0; e < 8; ++e) xk[e] = (kFull || valid) ? nk[e] : 0.0f;
  } else {
    unpack8<Io>(tok(4), xa);
    unpack8<Io>(tok(5), xb);
  }
  if constexpr (kRO) {
    // the readout's per-token residual weight over this lane's keys, summed
    // over the four lanes of the token: sum r k' r_k with k' as stored
    float part = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float kq = kKK ? Io::to_f32(Io::from_f32(xk[e])) : xk[e];
      part = __builtin_fmaf(xr[e] * kq, rk8[e], part);
    }
    part += __shfl_xor(part, 16);
    part += __shfl_xor(part, 32);
    if (q == 0) rkv_row[i] = part;
  }
  // base-2 log of the retention, log2(w) = c sigmoid(x) with
  // c = -exp(-1/2) log2(e), evaluated as 1 / ((1 + 2^(-log2(e) x)) / c)
  constexpr float kC = kNegExpHalf * kLog2e;
  constexpr float kInvC = 1.0f / kC;
  float at[8], rt[8], bh[8], kh[8];
  if constexpr (kSum) {
    // key by key: the summary pass runs 12 waves (168 registers each), where
    // the staged form below would spill
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ex = __builtin_amdgcn_exp2f(__builtin_fmaf(xl[e], -kLog2e, nbias8[e]));
      float lw2 = __builtin_amdgcn_rcpf(__builtin_fmaf(ex, kInvC, kInvC));
      if constexpr (!kFull) lw2 = valid ? lw2 : 0.0f;
      const float g2 = row_scan(lw2);
      const float gm = __builtin_amdgcn_exp2f(g2);
      const float ig = __builtin_amdgcn_exp2f(-g2);
      at[e] = xa[e] * row_prev(gm, 1.0f);
      bh[e] = xb[e] * ig;
      kh[e] = xk[e] * ig;
      if (i == L - 1) op.gl[kbase + e] = gm;
    }
  } else {
  // Stage by stage over the lane's eight keys: the eight chains are
  // independent, so each stage's instructions (DPP steps included) issue
  // back to back instead of waiting on one key's dependent chain.
  float g2[8], gm[8], gp[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    g2[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(xl[e], -kLog2e, nbias8[e]));
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float lw2 = __builtin_amdgcn_rcpf(__builtin_fmaf(g2[e], kInvC, kInvC));
    if constexpr (!kFull) lw2 = valid ? lw2 : 0.0f;
    if constexpr (kUnitW) lw2 = unit_w ? 0.0f : lw2;
    g2[e] = lw2;
  }
  // inclusive prefix sum over the 16 tokens (the lanes of a DPP row)
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
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float ig = __builtin_amdgcn_exp2f(-g2[e]);                     // 1 / gamma_t
    at[e] = xa[e] * gp[e];
    if constexpr (!kSum) rt[e] = xr[e] * gm[e];
    bh[e] = xb[e] * ig;
    kh[e] = xk[e] * ig;
    if constexpr (kUnitW) kh[e] *= kscale;   // reverse mode: k is r_t, times scale
  }
  if (i == L - 1) {
    *reinterpret_cast<f32x4*>(&op.gl[kbase]) = f32x4{gm[0], gm[1], gm[2], gm[3]};
    *reinterpret_cast<f32x4*>(&op.gl[kbase + 4]) = f32x4{gm[4], gm[5], gm[6], gm[7]};
  }
  }
  kr.As = split8(at);
  if constexpr (!kSum) kr.Rs = split8(rt);
  kr.Bs = split8(bh);
  kr.Ks = split8(kh);
  const u32x4 vraw = tok(3);
  if constexpr (kVExact) {
    kr.Vs.hi = __builtin_bit_cast(bf16x8, vraw);       // bf16 values are exact
  } else {
    float xv[8];
    unpack8<Io>(vraw, xv);
    kr.Vs = split8(xv);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const f32x4 pab = mma32x3(kr.As, kr.Bs, zero);
  const f32x4 pak = mma32x3(kr.As, kr.Ks, zero);
  // lane (i, q) holds P[4q+e][i]: one 16-byte store per block
  *reinterpret_cast<f32x4*>(&sm.mpart[mp][cc][hh][0][i][4 * q]) = pab;
  *reinterpret_cast<f32x4*>(&sm.mpart[mp][cc][hh][1][i][4 * q]) = pak;
  if constexpr (!kSum) {
    const f32x4 prb = mma32x3(kr.Rs, kr.Bs, zero);
    const f32x4 prk = mma32x3(kr.Rs, kr.Ks, zero);
    *reinterpret_cast<f32x4*>(&sm.mpart[mp][cc][hh][2][i][4 * q]) = prb;
    *reinterpret_cast<f32x4*>(&sm.mpart[mp][cc][hh][3][i][4 * q]) = prk;
  }
}

// ---------------------------------------------------------------------------
// key side, part 2: store the operands; the wave whose key half hh equals
// the group parity mp forms T, the other one the masked Mak, Mrb, Mrk (the
// T chain is the heavier role: alternating it spreads it over all four SIMDs)
// ---------------------------------------------------------------------------
template <bool kVExact, bool kSum = false>
__device__ __forceinline__ void key_part2(Smem<kVExact>& sm, ChunkOps<kVExact>& op, int mp,
                                          int cc, int hh, int i, int q, const KeyRegs& kr) {
  const int kbase = 32 * hh + 8 * q;
  {
    // keys kbase..kbase+7 land in two 4-key runs of the permuted rows
    const int p0 = key_pos(kbase), p1 = key_pos(kbase + 4);
    if constexpr (!kSum) {
      *reinterpret_cast<bf16x4*>(&op.r_h[i][a_col(i, p0)]) = kr.Rs.hi.lo;
      *reinterpret_cast<bf16x4*>(&op.r_h[i][a_col(i, p1)]) = kr.Rs.hi.hi;
      *reinterpret_cast<bf16x4*>(&op.r_l[i][a_col(i, p0)]) = kr.Rs.lo.lo;
      *reinterpret_cast<bf16x4*>(&op.r_l[i][a_col(i, p1)]) = kr.Rs.lo.hi;
    }
    *reinterpret_cast<bf16x4*>(&op.at_h[i][a_col(i, p0)]) = kr.As.hi.lo;
    *reinterpret_cast<bf16x4*>(&op.at_h[i][a_col(i, p1)]) = kr.As.hi.hi;
    *reinterpret_cast<bf16x4*>(&op.at_l[i][a_col(i, p0)]) = kr.As.lo.lo;
    *reinterpret_cast<bf16x4*>(&op.at_l[i][a_col(i, p1)]) = kr.As.lo.hi;
  }
  *reinterpret_cast<bf16x8*>(&op.b_h[i][b_col(i, kbase)]) = kr.Bs.hi;
  *reinterpret_cast<bf16x8*>(&op.b_l[i][b_col(i, kbase)]) = kr.Bs.lo;
  *reinterpret_cast<bf16x8*>(&op.k_h[i][b_col(i, kbase)]) = kr.Ks.hi;
  *reinterpret_cast<bf16x8*>(&op.k_l[i][b_col(i, kbase)]) = kr.Ks.lo;
  *reinterpret_cast<bf16x8*>(&op.v_h[i][b_col(i, kbase)]) = kr.Vs.hi;
  if constexpr (!kVExact) *reinterpret_cast<bf16x8*>(&op.v_l[i][b_col(i, kbase)]) = kr.Vs.lo;
  // P[t][s] of block b, summed over the two key halves, is
  // mp0[0][b][s][t] + mp0[1][b][s][t]
  const float (*mp0)[4][L][MPP] = sm.mpart[mp][cc];
  if (hh == mp) {
    // M[e] = Mab[4q+e][i] (accumulator layout), Mt[e] = Mab[i][4q+e]
    const f32x4 m4 = *reinterpret_cast<const f32x4*>(&mp0[0][0][i][4 * q]) +
                     *reinterpret_cast<const f32x4*>(&mp0[1][0][i][4 * q]);
    f32x4 M, Mt;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * q + e;
      const float mt = mp0[0][0][r][i] + mp0[1][0][r][i];
      M[e] = (r > i) ? m4[e] : 0.f;
      Mt[e] = (i > r) ? mt : 0.f;
    }
    store_aop(op.t, i, q, t_inverse(M, Mt, i, q));
  } else {
    f32x4 mak, mrb, mrk;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = 4 * q + e;       // A-operand layout: row i, K = s
      const float v1 = mp0[0][1][s][i] + mp0[1][1][s][i];
      mak[e] = (i > s) ? v1 : 0.f;
      if constexpr (!kSum) {
        const float v2 = mp0[0][2][s][i] + mp0[1][2][s][i];
        const float v3 = mp0[0][3][s][i] + mp0[1][3][s][i];
        mrb[e] = (i >= s) ? v2 : 0.f;
        mrk[e] = (i >= s) ? v3 : 0.f;
      }
    }
    store_aop(op.mak, i, q, as_a(split4(mak)));
    if constexpr (!kSum) {
      store_aop(op.mrb, i, q, as_a(split4(mrb)));
      store_aop(op.mrk, i, q, as_a(split4(mrk)));
    }
  }
}

// ---------------------------------------------------------------------------
// state side: one chunk for the columns [16w, 16w+16) held in S.  The
// operand reads of a chunk are separate from its arithmetic so that the
// reads of the next chunk can be issued before this chunk's dependent chain.
// ---------------------------------------------------------------------------
template <bool kVExact>
struct StateOps {
  AOp Ta, Mak, Mrb, Mrk;
  bf16x4 vh, vl;
  Sp8 Aa0, Aa1, Ra0, Ra1;
  AOp Bt[4], Kt[4];
  f32x4 gl[4];
};

// operands the chain needs first: Mak, Mrk, V and the A~ / R~ rows
template <bool kVExact, bool kSum = false>
__device__ __forceinline__ void state_load_early(StateOps<kVExact>& o, const ChunkOps<kVExact>& op,
                                                 int vcol, int i, int q) {
  o.Mak = load_aop(op.mak, i, q);
  if constexpr (!kSum) o.Mrk = load_aop(op.mrk, i, q);
  // transposed operands straight from the token rows (see tr_rows)
  const int trow = 4 * q + (i >> 2), tcol = 4 * (i & 3);
  const int vc0 = 16 * (vcol >> 4) + tcol;
  o.vh = tr_rows(&op.v_h[trow][b_col(trow, vc0)]);                                   // V[4q+e][vcol]
  if constexpr (!kVExact) o.vl = tr_rows(&op.v_l[trow][b_col(trow, vc0)]);
  o.Aa0 = rows_vs_state(op.at_h, op.at_l, 0, i, q);
  o.Aa1 = rows_vs_state(op.at_h, op.at_l, 1, i, q);
  if constexpr (!kSum) {
    o.Ra0 = rows_vs_state(op.r_h, op.r_l, 0, i, q);
    o.Ra1 = rows_vs_state(op.r_h, op.r_l, 1, i, q);
  }
}
// the rest: T, Mrb, B^^T, K^^T and gamma_L
template <bool kVExact, bool kSum = false>
__device__ __forceinline__ void state_load_late(StateOps<kVExact>& o, const ChunkOps<kVExact>& op,
                                                int vcol, int i, int q) {
  (void)vcol;
  o.Ta = load_aop(op.t, i, q);
  if constexpr (!kSum) o.Mrb = load_aop(op.mrb, i, q);
  const int trow = 4 * q + (i >> 2), tcol = 4 * (i & 3);
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    // B^^T, K^^T as A operands: row 16kb+i, K = token
    o.Bt[kb] = __builtin_shufflevector(tr_rows(&op.b_h[trow][b_col(trow, kb * 16 + tcol)]),
                                       tr_rows(&op.b_l[trow][b_col(trow, kb * 16 + tcol)]), 0, 1, 2, 3, 4,
                                       5, 6, 7);
    o.Kt[kb] = __builtin_shufflevector(tr_rows(&op.k_h[trow][b_col(trow, kb * 16 + tcol)]),
                                       tr_rows(&op.k_l[trow][b_col(trow, kb * 16 + tcol)]), 0, 1, 2, 3, 4,
                                       5, 6, 7);
    o.gl[kb] = *reinterpret_cast<const f32x4*>(&op.gl[kb * 16 + 4 * q]);
  }
}
template <bool kVExact, bool kSum = false>
__device__ __forceinline__ StateOps<kVExact> state_load(const ChunkOps<kVExact>& op, int vcol,
                                                        int i, int q) {
  StateOps<kVExact> o;
  state_load_early<kVExact, kSum>(o, op, vcol, i, q);
  state_load_late<kVExact, kSum>(o, op, vcol, i, q);
  return o;
}

// Where the sa rows 4q+e (e = 0..3) of a chunk go: row row0 + dir*e of the
// column pointer col (rows of row_stride floats), except that e = 0 goes to
// row `wrap` when wrap >= 0 (the reverse mode's position 0).  Kept as a few
// integers and formed at the store, so that no per-row pointers stay live
// across the chain.
struct SaRows {
  float* col = nullptr;
  int64_t row_stride = 0;
  int row0 = 0, dir = 1, wrap = -1;
  __device__ __forceinline__ float* at(int e) const {
    const int row = (e == 0 && wrap >= 0) ? wrap : row0 + dir * e;
    return col + static_cast<int64_t>(row) * row_stride;
  }
};

// The value of the lane whose index within its quad differs in bit 0
// (quad_xor1) or bit 1 (quad_xor2): DPP quad permutations.
__device__ __forceinline__ float quad_xor1(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xb1, 0xf, 0xf, false));
}
__device__ __forceinline__ float quad_xor2(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4e, 0xf, 0xf, false));
}

// Store of state tile kb held in accumulator layout (lane (i, q), item e:
// key row 16 kb + 4 q + e of column `col` = col0 + i) into a row-major
// [key][value] D x D block at `blk`, as 16-byte row pieces: a 4 x 4
// transpose inside each quad of lanes (DPP) gives lane (4j + m, q) key row
// 16 kb + 4 q + m, columns col0 + 4 j..+3.
__device__ __forceinline__ void store_state_tile(float* blk, int col0, const f32x4& v, int kb,
                                                 int i, int q) {
  const int m4 = i & 3;
  f32x4 t, u;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x = quad_xor1(v[e ^ 1]);
    t[e] = ((m4 ^ e) & 1) ? x : v[e];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x = quad_xor2(t[e ^ 2]);
    u[e] = ((m4 ^ e) & 2) ? x : t[e];
  }
  *reinterpret_cast<f32x4*>(blk + (16 * kb + 4 * q + m4) * D + col0 + 4 * (i >> 2)) = u;
}

// With kTrain the chunk also writes its per-token sa rows (U, fp32) of tokens
// 4q..4q+3 to sa_rows.at(0..3) — or, with sa_lds set, stages them in that
// [token][column] LDS tile for the caller to write back — and, when bnd_col
// is set, its post-chunk state column to bnd_col[key * D].
// kSum (summary pass): the state update only, no outputs; with no_v the
// value rows count as zero (the transition of the chunk).
constexpr int UP = D + 4;   // padded row of a staged sa tile (fp32)
template <class Io, bool kVExact, bool kTrain = false, bool kSum = false>
__device__ __forceinline__ void state_compute(const StateOps<kVExact>& o, f32x4 (&S)[4],
                                              uint16_t (*yrows)[YP], int vcol, int i, int q,
                                              float scale, const SaRows& sa_rows = SaRows{},
                                              float* bnd_col = nullptr, bool no_v = false,
                                              float (*sa_lds)[UP] = nullptr) {
  using raw = typename Io::raw;
  // S split as B operand against the permuted A~ / R~ rows: K positions
  // 8q..8q+7 = rows 32m + 4q + (0..3) then 32m + 16 + 4q + (0..3)
  Sp8 Sb[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const Split4 a = split4(S[2 * m]), b = split4(S[2 * m + 1]);
    Sb[m].hi = __builtin_bit_cast(bf16x8, u32x4{a.h0, a.h1, b.h0, b.h1});
    Sb[m].lo = __builtin_bit_cast(bf16x8, u32x4{a.l0, a.l1, b.l0, b.l1});
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  // X = A~ S0 + Mak V,  U = T X,  Y = R~ S0 + Mrb U + Mrk V
  f32x4 X, Y;
  if constexpr (kSum) {
    // X = A~ S0 + Mak V, U = T X, S_L = diag(gamma_L) (S0 + B^^T U + K^^T V)
    (void)yrows; (void)scale; (void)Y;
    // A x V for the token-indexed A operand (exact bf16 V: one instruction)
    auto times_v = [&](AOp a, f32x4 c) {
      if (no_v) return c;
      if constexpr (kVExact) return mm_ax(a, as_bx(o.vh), c);
      else return mm_ab(a, as_b(o.vh, o.vl), c);
    };
    X = times_v(o.Mak, zero);
    X = mma32x3(o.Aa0, Sb[0], X);
    X = mma32x3(o.Aa1, Sb[1], X);
    const BOp Us = as_b(split4(mm_ab(o.Ta, as_b(split4(X)), zero)));
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 acc = mm_ab(o.Bt[kb], Us, S[kb]);
      acc = times_v(o.Kt[kb], acc);
      S[kb] = acc * o.gl[kb];
    }
  } else if constexpr (kVExact) {
    const BX Vx = as_bx(o.vh);
    X = mm_ax(o.Mak, Vx, zero);
    Y = mm_ax(o.Mrk, Vx, zero);
    X = mma32x3(o.Aa0, Sb[0], X);
    X = mma32x3(o.Aa1, Sb[1], X);
    Y = mma32x3(o.Ra0, Sb[0], Y);
    Y = mma32x3(o.Ra1, Sb[1], Y);
    const f32x4 Uf = mm_ab(o.Ta, as_b(split4(X)), zero);
    const BOp Us = as_b(split4(Uf));
    Y = mm_ab(o.Mrb, Us, Y);
    if constexpr (kTrain) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (sa_lds != nullptr)
          sa_lds[4 * q + e][vcol] = Uf[e];
        else
          *sa_rows.at(e) = Uf[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const raw yv = Io::from_f32(scale * Y[e]);
      yrows[4 * q + e][vcol] = __builtin_bit_cast(uint16_t, yv);
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 acc = mm_ab(o.Bt[kb], Us, S[kb]);
      acc = mm_ax(o.Kt[kb], Vx, acc);
      S[kb] = acc * o.gl[kb];
      if constexpr (kTrain) {
        // (column stores: the quad transpose of store_state_tile, on these
        // state waves' chain, measured 0.683 vs 0.662 ms for the forward)
        if (bnd_col != nullptr) {
#pragma unroll
          for (int e = 0; e < 4; ++e) bnd_col[(16 * kb + 4 * q + e) * D] = S[kb][e];
        }
      }
    }
  } else {
    const BOp Vs = as_b(o.vh, o.vl);
    X = mm_ab(o.Mak, Vs, zero);
    Y = mm_ab(o.Mrk, Vs, zero);
    X = mma32x3(o.Aa0, Sb[0], X);
    X = mma32x3(o.Aa1, Sb[1], X);
    Y = mma32x3(o.Ra0, Sb[0], Y);
    Y = mma32x3(o.Ra1, Sb[1], Y);
    const f32x4 Uf = mm_ab(o.Ta, as_b(split4(X)), zero);
    const BOp Us = as_b(split4(Uf));
    Y = mm_ab(o.Mrb, Us, Y);
    if constexpr (kTrain) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (sa_lds != nullptr)
          sa_lds[4 * q + e][vcol] = Uf[e];
        else
          *sa_rows.at(e) = Uf[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const raw yv = Io::from_f32(scale * Y[e]);
      yrows[4 * q + e][vcol] = __builtin_bit_cast(uint16_t, yv);
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4 acc = mm_ab(o.Bt[kb], Us, S[kb]);
      acc = mm_ab(o.Kt[kb], Vs, acc);
      S[kb] = acc * o.gl[kb];
      if constexpr (kTrain) {
        // (column stores: the quad transpose of store_state_tile, on these
        // state waves' chain, measured 0.683 vs 0.662 ms for the forward)
        if (bnd_col != nullptr) {
#pragma unroll
          for (int e = 0; e < 4; ++e) bnd_col[(16 * kb + 4 * q + e) * D] = S[kb][e];
        }
      }
    }
  }
}

// Progress counters in LDS.  Producers and consumers exchange LDS data only,
// so ordering needs only the LDS counter: a wave publishes a counter after
// waiting for its own LDS operations to complete (lgkmcnt(0)); a waiting wave
// polls the counter, and its later LDS reads issue after the poll returned.
// Compiler fences keep the memory operations on their side of each step.
// (Acquire/release atomics would also wait for outstanding global loads,
// stalling the row prefetch.)  Every wait is bounded by the launch's spin
// limit so that every wave finishes; a wait that gives up raises the block's
// fault flag, and the block then fails closed at its end (NaN outputs, state
// untouched, the library's fault counter incremented).
__device__ __forceinline__ void signal(int* c, int v) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): own LDS stores have landed
  __hip_atomic_store(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
__device__ __forceinline__ int peek(int* c) {
  return __hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void raise_fault(int* fault) {
  __hip_atomic_store(fault, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Once the block's fault flag is up its results are NaN whatever happens, so
// every later wait returns at once instead of polling to its limit (a real
// stall then costs one wait's limit, not one per hand-off of the sequence).
__device__ __forceinline__ void wait_ge(int* c, int v, int limit, int* fault) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  int it = 0;
  for (; it < limit && peek(c) < v && peek(fault) == 0; ++it) __builtin_amdgcn_s_sleep(1);
  if (it == limit && peek(c) < v) raise_fault(fault);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// wait until all four counters c[0..3] (kEight: c[0..7]) reach v
template <bool kEight = false>
__device__ __forceinline__ void wait_min_ge(int* c, int v, int limit, int* fault) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  auto low = [&]() {
    int m = min(min(peek(c), peek(c + 1)), min(peek(c + 2), peek(c + 3)));
    if constexpr (kEight) m = min(m, min(min(peek(c + 4), peek(c + 5)), min(peek(c + 6), peek(c + 7))));
    return m;
  };
  int it = 0;
  for (; it < limit && low() < v && peek(fault) == 0; ++it) __builtin_amdgcn_s_sleep(1);
  if (it == limit && low() < v) raise_fault(fault);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Fused readout write-back of group gi (the state waves run it one group
// late, in place of the plain y write-back): thread (o_tok, o_c8) takes 8
// channels of token o_tok of the group's staged y rows.  GroupNorm over the
// head's 64 channels (the 8 consecutive lanes of a token hold 8 channels
// each), the r k' r_k residual whose two key-half sums the key waves left in
// sm.rkv, and the gate:
//   out = (GroupNorm(y) * ln_w + ln_b + (sum r k' r_k) v) * g.
template <class Io, bool kVExact>
__device__ __forceinline__ void readout_write_back(const Smem<kVExact>& sm, const SegArgs& p,
                                                   int gi, int o_tok, int o_c8, int t0,
                                                   int seg_len, int64_t row_stride,
                                                   int64_t head_off) {
  using raw = typename Io::raw;
  // this thread's 8 channels of ln_w / ln_b (read here rather than held in
  // registers across the key waves' loop)
  float ro_w[8], ro_b[8];
  unpack8<Io>(*reinterpret_cast<const u32x4*>(static_cast<const raw*>(p.ro_lnw) + head_off +
                                              o_c8 * 8), ro_w);
  unpack8<Io>(*reinterpret_cast<const u32x4*>(static_cast<const raw*>(p.ro_lnb) + head_off +
                                              o_c8 * 8), ro_b);
  const int pos = gi * GT + o_tok;   // position in the segment
  const bool in_seg = pos < seg_len;
  const int64_t roff =
      static_cast<int64_t>(t0 + min(pos, seg_len - 1)) * row_stride + head_off + o_c8 * 8;
  const u32x4 ypiece = *reinterpret_cast<const u32x4*>(&sm.yb[gi & 1][o_tok][o_c8 * 8]);
  const u32x4 vraw = *reinterpret_cast<const u32x4*>(static_cast<const raw*>(p.v) + roff);
  const u32x4 graw = *reinterpret_cast<const u32x4*>(static_cast<const raw*>(p.ro_g) + roff);
  float yv[8], vv[8], gv[8];
  unpack8<Io>(ypiece, yv);
  unpack8<Io>(vraw, vv);
  unpack8<Io>(graw, gv);
  float s1 = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s1 += yv[e];
  s1 += __shfl_xor(s1, 1);
  s1 += __shfl_xor(s1, 2);
  s1 += __shfl_xor(s1, 4);
  const float mean = s1 * (1.0f / D);
  float s2 = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s2 = __builtin_fmaf(yv[e] - mean, yv[e] - mean, s2);
  s2 += __shfl_xor(s2, 1);
  s2 += __shfl_xor(s2, 2);
  s2 += __shfl_xor(s2, 4);
  const float inv = 1.0f / __builtin_sqrtf(s2 * (1.0f / D) + 64.0e-5f);
  const float rkv = sm.rkv[gi & 3][0][o_tok] + sm.rkv[gi & 3][1][o_tok];
  u32x4 packed;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float o2[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int e = 2 * j + h2;
      o2[h2] = (__builtin_fmaf((yv[e] - mean) * inv, ro_w[e], ro_b[e]) + rkv * vv[e]) * gv[e];
    }
    packed[j] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Io::from_f32(o2[0]))) |
                (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, Io::from_f32(o2[1]))) << 16);
  }
  if (in_seg) {
    *reinterpret_cast<u32x4*>(static_cast<raw*>(p.ro_out) + roff) = packed;
    if (p.y != nullptr) *reinterpret_cast<u32x4*>(static_cast<raw*>(p.y) + roff) = ypiece;
  }
}

// kTrain: the training-forward contract (pretrain path) also writes every
// token's sa (p.sa_out) and the post-chunk state of every 16-token chunk
// (p.boundary, [segment, H, boundary_per_seg, D, D]).
// kSum: the summary pass of a sequence split: block y = n * (pieces - 1) + j
// summarises piece j < last of sequence n with 12 waves.  The four key waves
// prepare the operators once; state waves 0-3 carry the piece's final state
// from a zero start (F) and state waves 4-7 its transition, the state from
// an identity start with V = 0 (Phi), to split_summary[(n * (pieces - 1) +
// j) * 2 + {0: F, 1: Phi}, H, D, D].  Nothing else is written.
constexpr int NT_SUM = 768;
template <class Io, bool kTrain, bool kRev = false, bool kSum = false, bool kKK = false,
          bool kRO = false>
__global__ __launch_bounds__(kSum ? NT_SUM : NT) void chunk64_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr bool kVExact = !__is_same(Io, IoF16);
  __shared__ Smem<kVExact> sm;

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a scalar: the role branches below are uniform per wave, so
  // each wave runs only its own role's code (no exec-masked pass through the
  // other role, whose matrix instructions would run regardless of exec)
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15;
  const int q = lane >> 4;
  const int H = p.num_heads;

  // sequence split: which sequence, piece and (summary) kind this block is
  const int npc = p.split_pieces;
  int seq = seg, piece = 0;
  if (kSum || npc > 0) {
    const int cnt = p.split_count > 0 ? p.split_count : (kSum ? npc - 1 : npc);
    seq = seg / cnt;
    piece = p.split_first + seg % cnt;
  }
  if (p.status != nullptr) {
    if (p.status[0] != 0) {
      if constexpr (!kSum) {
        const int64_t blk = static_cast<int64_t>(seg) * gridDim.x + h;
        const int64_t nblk = static_cast<int64_t>(gridDim.x) * gridDim.y;
        if (!kRO || p.y != nullptr)
          fill_output_nan<Io>(static_cast<raw*>(p.y), p.out_elems, blk, nblk);
        if constexpr (kRO)
          fill_output_nan<Io>(static_cast<raw*>(p.ro_out), p.out_elems, blk, nblk);
      }
      return;
    }
    if (seq >= p.status[2]) return;
  }
  int t0, t1;
  bool last_piece = true;
  if (kSum || npc > 0) {
    const int q0 = p.bounds[seq], q1 = p.bounds[seq + 1];
    int start, plen, last;
    split_piece(p, q1 - q0, piece, start, plen, last);
    // pieces past the sequence's last have nothing to do; the summary pass
    // covers the pieces before the last only
    if (piece > last || (kSum && piece >= last)) return;
    last_piece = piece == last;
    t0 = q0 + start;
    t1 = min(t0 + plen, q1);
  } else if (p.uniform_len > 0) {
    t0 = seg * p.uniform_len;
    t1 = t0 + p.uniform_len;
  } else if (p.chunk_offsets != nullptr) {
    t0 = p.bounds[p.chunk_offsets[seg]];
    t1 = p.ends[p.chunk_offsets[seg + 1] - 1];
  } else if (p.ends != nullptr) {
    t0 = p.bounds[seg];
    t1 = p.ends[seg];
  } else {
    t0 = p.bounds[seg];
    t1 = p.bounds[seg + 1];
  }
  const int slot = p.slots ? p.slots[seq] : seq;
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(H) * D;
  const int ngroups = (t1 - t0 + GT - 1) / GT;
  raw* yout = static_cast<raw*>(p.y);

  if (tid < 21) (&sm.ready[0])[tid] = 0;
  __syncthreads();   // the only workgroup barrier: counters are zero

  constexpr int kStateWaves = kSum ? 8 : 4;
  // state waves: columns [16wv, 16wv+16); in the summary pass waves 4-7
  // repeat the columns for the transition (kind 1)
  const int vcol = 16 * (wv & 3) + i;
  const int kind = kSum ? (wv >> 2) : 0;
  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  const int64_t pbase = (static_cast<int64_t>(seq) * (npc > 0 ? npc : 1) + piece) * H + h;
  constexpr int kStateThreads = 64 * kStateWaves;
  if (wv < kStateWaves) {
    f32x4 S[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    // state of a piece after the first (real split pass): the combined
    // start state; the summary pass starts from zero (F) or identity (Phi)
    if constexpr (kSum) {
      if (kind == 1) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) S[kb][e] = (kb * 16 + 4 * q + e == vcol) ? 1.0f : 0.0f;
      }
    } else if (npc > 0 && !(piece == 0 && p.split_lead_pass)) {
      const float* sin = p.split_state + pbase * D * D;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = sin[(kb * 16 + 4 * q + e) * D + vcol];
    } else if (p.state_in != nullptr && p.state_bf16) {
      // (bf16-state contract) bf16 widened once; the state stays fp32 for
      // the whole call and is rounded back once at the end.  One branch
      // around each loop: a per-element select compiles to a branch and a
      // wait per load.
      const uint16_t* sinb = static_cast<const uint16_t*>(p.state_in) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = IoBF16::to_f32(sinb[(kb * 16 + 4 * q + e) * D]);
    } else if (p.state_in != nullptr) {
      const float* sin = static_cast<const float*>(p.state_in) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = sin[(kb * 16 + 4 * q + e) * D];
    }
    // outputs of a finished group: 16-byte pieces of the staged rows, token
    // tid/8, elements 8*(tid%8).. (the four state waves cover the 32 rows)
    const int o_tok = tid >> 3, o_c8 = tid & 7;
    const int seg_len = t1 - t0;
    auto write_out = [&](int gi) {
      if (gi < 0) return;
      wait_min_ge(sm.consumed, gi + 1, p.spin_limit, &sm.fault);   // every state wave staged its columns
      const int pos = gi * GT + o_tok;        // position in processing order
      if constexpr (kRO) {
        readout_write_back<Io, kVExact>(sm, p, gi, o_tok, o_c8, t0, seg_len, row_stride,
                                        head_off);
      } else if (pos < seg_len) {
        const int row = kRev ? t1 - 1 - pos : t0 + pos;
        *reinterpret_cast<u32x4*>(yout + static_cast<int64_t>(row) * row_stride + head_off +
                                  o_c8 * 8) =
            *reinterpret_cast<const u32x4*>(&sm.yb[gi & 1][o_tok][o_c8 * 8]);
      }
      signal(&sm.drained[wv], gi + 1);
    };
    // training outputs: sa column of this lane and the boundary column
    float* const sa_base = kTrain ? p.sa_out + head_off + vcol : nullptr;
    const int nsnap = (p.boundary_per_seg + p.boundary_every - 1) / p.boundary_every;
    float* const bnd_base =
        (kTrain && p.boundary != nullptr)
            ? p.boundary + (static_cast<int64_t>(seg) * H + h) * nsnap * D * D + vcol
            : nullptr;
    auto chunk = [&](const StateOps<kVExact>& o, int gi, int c) {
      const int ci = gi * G + c;   // chunk index within the segment
      SaRows sa_rows;
      if constexpr (kTrain) {
        // forward: rows t0 + pos; reverse: t0 + (n - pos) mod n, which is
        // t1 - pos except at pos = 0
        const int pos0 = ci * L + 4 * q;
        sa_rows.col = sa_base;
        sa_rows.row_stride = row_stride;
        sa_rows.row0 = kRev ? t1 - pos0 : t0 + pos0;
        sa_rows.dir = kRev ? -1 : 1;
        sa_rows.wrap = (kRev && pos0 == 0) ? t0 : -1;
      }
      const int bi = kRev ? p.boundary_per_seg - 1 - ci : ci;
      const bool keep = bnd_base != nullptr && bi % p.boundary_every == 0;
      state_compute<Io, kVExact, kTrain>(
          o, S, &sm.yb[gi & 1][c * L], vcol, i, q, p.scale, sa_rows,
          keep ? bnd_base + static_cast<int64_t>(bi / p.boundary_every) * D * D : nullptr);
    };
    auto chunk_sum = [&](const StateOps<kVExact>& o) {
      state_compute<Io, kVExact, false, true>(o, S, nullptr, vcol, i, q, 1.0f, SaRows{},
                                              nullptr, kind == 1);
    };
    auto group = [&](auto par_c, int gi) {
      constexpr int par = decltype(par_c)::value;
      wait_min_ge(sm.ready, gi + 1, p.spin_limit, &sm.fault);   // operators of group gi stored
      if constexpr (kSum) {
        // state update only: no outputs to stage or drain
        chunk_sum(state_load<kVExact, true>(sm.ops[par][0], vcol, i, q));
        if (t0 + gi * GT + L < t1) chunk_sum(state_load<kVExact, true>(sm.ops[par][1], vcol, i, q));
        signal(&sm.consumed[wv], gi + 1);
        return;
      }
      wait_min_ge(sm.drained, gi - 1, p.spin_limit, &sm.fault);   // outputs of group gi-2 written back
      if (!kTrain && t0 + gi * GT + GT <= t1) {
        // both chunks: the second chunk's first-needed operand reads (the
        // S-side rows and V-side blocks) go out before the first chunk's chain
        // (not in training mode, whose extra outputs would then spill)
        const StateOps<kVExact> o0 = state_load(sm.ops[par][0], vcol, i, q);
        StateOps<kVExact> o1;
        state_load_early(o1, sm.ops[par][1], vcol, i, q);
        chunk(o0, gi, 0);
        state_load_late(o1, sm.ops[par][1], vcol, i, q);
        chunk(o1, gi, 1);
      } else {
        chunk(state_load(sm.ops[par][0], vcol, i, q), gi, 0);
        if (t0 + gi * GT + L < t1) chunk(state_load(sm.ops[par][1], vcol, i, q), gi, 1);
      }
      signal(&sm.consumed[wv], gi + 1);
      write_out(gi - 1);
    };
    for (int gi = 0; gi < ngroups; gi += 2) {
      group(std::integral_constant<int, 0>{}, gi);
      if (gi + 1 < ngroups) group(std::integral_constant<int, 1>{}, gi + 1);
    }
    if constexpr (!kSum) write_out(ngroups - 1);
    // Every wave has left its loop (the key waves meet this barrier at the
    // end of their branch); a raised fault flag means a hand-off wait gave
    // up, so the values computed are not trustworthy: fail closed.
    __syncthreads();
    if (peek(&sm.fault) != 0) {
      if (tid == 0 && p.handoff_fault != nullptr) atomicAdd(p.handoff_fault, 1);
      const float qnan = quiet_nan();
      if constexpr (kSum) {
        // the pieces that start from this summary come out NaN as well
        float* sout = p.split_summary + (static_cast<int64_t>(seg) * 2 * H + h) * D * D;
        for (int e = tid; e < D * D; e += kStateThreads) {
          sout[e] = qnan;
          sout[static_cast<int64_t>(H) * D * D + e] = qnan;
        }
      } else {
        const raw nanv = Io::from_f32(qnan);
        if (yout != nullptr)
          for (int64_t e = tid; e < static_cast<int64_t>(t1 - t0) * D; e += kStateThreads)
            yout[(t0 + e / D) * row_stride + head_off + e % D] = nanv;
        if constexpr (kRO)
          for (int64_t e = tid; e < static_cast<int64_t>(t1 - t0) * D; e += kStateThreads)
            static_cast<raw*>(p.ro_out)[(t0 + e / D) * row_stride + head_off + e % D] = nanv;
        if constexpr (kTrain) {
          for (int64_t e = tid; e < static_cast<int64_t>(t1 - t0) * D; e += kStateThreads)
            p.sa_out[(t0 + e / D) * row_stride + head_off + e % D] = qnan;
        }
        if (npc > 0 && p.split_lead_pass && piece == 0 && !last_piece) {
          // the lead piece's successor starts from NaN
          float* sout = p.split_state + (pbase + H) * D * D;
          for (int e = tid; e < D * D; e += kStateThreads) sout[e] = qnan;
        }
      }
      return;
    }
    if constexpr (kSum) {
      float* sout = p.split_summary + ((static_cast<int64_t>(seg) * 2 + kind) * H + h) * D * D;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sout[(kb * 16 + 4 * q + e) * D + vcol] = S[kb][e];
    } else if (!last_piece) {
      // a piece before the last hands on nothing (its successor starts from
      // the combined state), except the lead pass's piece 0, whose end state
      // is piece 1's start
      if (p.split_lead_pass && piece == 0) {
        float* sout = p.split_state + (pbase + H) * D * D;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) sout[(kb * 16 + 4 * q + e) * D + vcol] = S[kb][e];
      }
    } else if (p.state_out != nullptr && p.state_bf16) {
      uint16_t* soutb = static_cast<uint16_t*>(p.state_out) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          soutb[(kb * 16 + 4 * q + e) * D] = IoBF16::from_f32(S[kb][e]);
    } else if (p.state_out != nullptr) {
      float* sout = static_cast<float*>(p.state_out) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sout[(kb * 16 + 4 * q + e) * D] = S[kb][e];
    }
  } else {
    // ---------------- key waves: chunk cc of each group, key half hh
    // The key waves are the pipeline's critical path and share each SIMD
    // with a state wave that has slack: let them win instruction issue.
    __builtin_amdgcn_s_setprio(2);
    const int kw = wv & 3;
    const int cc = kw >> 1;
    const int hh = kw & 1;
    const int partner = kw ^ 1;
    const int kbase = 32 * hh + 8 * q;
    float nbias8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      nbias8[e] = p.bias ? -kLog2e * Io::to_f32(static_cast<const raw*>(p.bias)[head_off + kbase + e])
                         : 0.f;
    const int kbase_other = 32 * (hh ^ 1) + 8 * q;
    float rk8[8];
    if constexpr (kRO) {
      const raw* rk = static_cast<const raw*>(p.ro_rk) + head_off + kbase;
#pragma unroll
      for (int e = 0; e < 8; ++e) rk8[e] = Io::to_f32(rk[e]);
    }
    KkParams kp;
    if constexpr (kKK) {
      const raw* kks = static_cast<const raw*>(p.kk_scale) + head_off;
      const raw* a0 = static_cast<const raw*>(p.a_bias) + head_off;
      const raw* ka = static_cast<const raw*>(p.k_a) + head_off;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kp.kk_own[e] = Io::to_f32(kks[kbase + e]);
        kp.kk_other[e] = Io::to_f32(kks[kbase_other + e]);
        kp.a0[e] = Io::to_f32(a0[kbase + e]);
        kp.ka[e] = Io::to_f32(ka[kbase + e]);
      }
    }
    // token rows of this lane (token i of chunk cc, keys kbase..+7), as
    // running pointers; the group stride is GT rows
    const int tok0 = t0 + cc * L + i;
    const raw* src[6];
    {
      const int64_t off = static_cast<int64_t>(kRev ? 0 : tok0) * row_stride + head_off + kbase;
      src[0] = static_cast<const raw*>(p.r) + off;
      src[1] = static_cast<const raw*>(p.logits) + off;
      src[2] = static_cast<const raw*>(p.k) + off;
      src[3] = static_cast<const raw*>(p.v) + off;
      src[4] = static_cast<const raw*>(p.a) + off;
      // fused kk / a gate: slot 5 reads the key's other half instead of b
      src[5] = kKK ? static_cast<const raw*>(p.k) + off + (kbase_other - kbase)
                   : static_cast<const raw*>(p.b) + off;
    }
    const int64_t gstride = static_cast<int64_t>(GT) * row_stride;
    // Rows past the sequence end are loaded from the last valid row (always
    // in bounds); key_part1 zeroes them when it consumes them.  A conditional
    // load would compile to a branch whose zeroing path waits for every
    // outstanding memory operation, the previous group's output stores
    // included, and a select right here would wait for the loads themselves.
    auto load_rows = [&](u32x4 (&dst)[6], int gi) {
      if constexpr (kRev) {
        const int pos = cc * L + i + gi * GT;   // position in processing order
#pragma unroll
        for (int j = 0; j < 6; ++j) {
          const int row = min(max(t1 - 1 - pos + ((p.shift_mask >> j) & 1), t0), t1 - 1);
          dst[j] = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4*>(src[j] + static_cast<int64_t>(row) * row_stride));
        }
      } else {
        const int tok = tok0 + gi * GT;
        const int64_t off = static_cast<int64_t>(min(tok, t1 - 1) - tok0) * row_stride;
#pragma unroll
        for (int j = 0; j < 6; ++j) {
          // the summary pass reads no r
          if (kSum && j == 0) {
            dst[j] = u32x4{0u, 0u, 0u, 0u};
            continue;
          }
          dst[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src[j] + off));
        }
      }
    };
    u32x4 rawA[6], rawB[6];
    KeyRegs kr;
    load_rows(rawA, 0);
    // group gn: prefetch the rows of gn + 1, wait until the state waves are
    // done with group gn - 2 (whose operator buffers gn reuses), then build
    // the operators of gn
    auto iter = [&](auto par_c, u32x4 (&cur)[6], u32x4 (&nxt)[6], int gn) {
      constexpr int par = decltype(par_c)::value;   // parity of gn
      if (gn + 1 < ngroups) load_rows(nxt, gn + 1);
      wait_min_ge<kSum>(sm.consumed, gn - 1, p.spin_limit, &sm.fault);   // group gn-2 no longer read
      const bool active = t0 + gn * GT + cc * L < t1;
      if constexpr (kRev) {
        // position 0 of the segment: the shifted rows lie past its end
        const bool void_row = gn == 0 && cc == 0 && i == 0;
        u32x4 rows[6];
#pragma unroll
        for (int j = 0; j < 6; ++j) {
          const bool z = void_row && ((p.shift_mask >> j) & 1) && j != 1;
          rows[j] = z ? u32x4{0u, 0u, 0u, 0u} : cur[j];
        }
        const bool unit_w = void_row && ((p.shift_mask >> 1) & 1);
        if (t0 + gn * GT + cc * L + L <= t1)
          key_part1<Io, kVExact, true, true>(sm, sm.ops[par][cc], rows, nbias8, true, par, cc,
                                             hh, i, q, kr, unit_w, p.kv_scale);
        else if (active)
          key_part1<Io, kVExact, false, true>(sm, sm.ops[par][cc], rows, nbias8,
                                              t0 + gn * GT + cc * L + i < t1, par, cc, hh, i, q,
                                              kr, unit_w, p.kv_scale);
      } else {
        raw* nk_row = nullptr;
        if constexpr (kKK)
          nk_row = static_cast<raw*>(p.new_k) +
                   static_cast<int64_t>(tok0 + gn * GT) * row_stride + head_off + kbase;
        if (t0 + gn * GT + cc * L + L <= t1)
          key_part1<Io, kVExact, true, false, kSum, kKK, kRO>(
              sm, sm.ops[par][cc], cur, nbias8, true, par, cc, hh, i, q, kr, false, 1.0f, &kp,
              nk_row, rk8, &sm.rkv[gn & 3][hh][cc * L]);
        else if (active)
          key_part1<Io, kVExact, false, false, kSum, kKK, kRO>(
              sm, sm.ops[par][cc], cur, nbias8, tok0 + gn * GT < t1, par, cc, hh, i, q, kr, false,
              1.0f, &kp, nk_row, rk8, &sm.rkv[gn & 3][hh][cc * L]);
      }
      signal(&sm.part1[kw], gn + 1);
      wait_ge(&sm.part1[partner], gn + 1, p.spin_limit, &sm.fault);
      if (active) key_part2<kVExact, kSum>(sm, sm.ops[par][cc], par, cc, hh, i, q, kr);
      if (!p.handoff_stall) signal(&sm.ready[kw], gn + 1);
    };
    for (int gn = 0; gn < ngroups; gn += 2) {
      iter(std::integral_constant<int, 0>{}, rawA, rawB, gn);
      if (gn + 1 < ngroups) iter(std::integral_constant<int, 1>{}, rawB, rawA, gn + 1);
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();   // pairs with the state waves' final barrier
  }

}


// ===========================================================================
// Ring variant of the workgroup-per-unit kernel (plain inference contract).
// Each key wave builds WHOLE chunks: key wave w (4..7) takes chunks
// w - 4, w, w + 4, ... of the unit, both key halves one after the other,
// accumulating the token-token blocks over all 64 keys in its own matrix
// accumulators, then forms T and the masked blocks itself.  So no partial
// blocks go through LDS and no key wave waits on a partner.  Operator blocks
// are a ring of R chunks in LDS (chunk c in slot c % R; R = 6 for bf16
// tokens, 5 for fp16), and a key wave may build chunk c as soon as the state
// waves have finished chunk c - R.  A key wave takes about three chunk
// periods to build a chunk, so with R = 4 the state waves waited on the
// ring; with R = 6 the four key waves' throughput sets the period.  The
// state waves run chunk after chunk as in chunk64_kernel and each writes its
// own 16 output columns, so they never wait on one another.
// ===========================================================================
// operator slots of the ring kernel (fp16 tokens carry V's lo part and
// fit one slot fewer in the 160 KB of LDS)
template <bool kVExact> constexpr int kRingOf = kVExact ? 6 : 5;
constexpr int kKeyW = 4;   // key waves of the ring kernel
constexpr int NTR = 64 * (4 + kKeyW);
template <bool kVExact>
struct alignas(16) SmemR {
  ChunkOps<kVExact> ops[kRingOf<kVExact>];   // ring by chunk index mod kRing
  uint16_t yb[L][YP];                 // staged output rows of the current chunk
  float ub[L][UP];                    // staged sa rows (the value pass)
  // progress counters, each written by one wave only: chunks key wave w has
  // built (its chunks are w, w + kKeyW, ...) and chunks state wave w has
  // finished
  int ready[kKeyW], consumed[4];
  int fault;
};

// Token-token products of the whole chunk, accumulated over both key halves:
// ab = Mab in accumulator layout (item e: Mab[4q+e][i]); abt, ak, rb, rk in
// A-operand layout (item e: X[i][4q+e]).
struct KeyAccR {
  f32x4 ab, abt, ak, rb, rk;
};

// One key half hh of chunk operators: as key_part1 (plain contract) plus the
// operand-row stores of key_part2, with the token-token products accumulated.
// kSum (summary pass): no R~ operand, no R-side products.
// Per-lane channel parameters of the fused kk / a-gate stage for the lane's
// eight keys of one key half: the kk scale, the a-gate bias a0 and k_a.
struct KkHalf {
  float kks[8], a0[8], ka[8];
};

// kKK (fused kk / a-gate stage): slot 4 of raw holds the a-gate logits a12,
// slot 5 is unused; kinv = 1 / max(|k k_k|, 1e-12) over the token's 64 keys;
// the gated key k' is stored to nk_row (when the token is in the segment):
//   kk = k k_k kinv, g = sigmoid(a0 + a12), k' = k (1 + (g - 1) k_a),
//   a = -kk, b = kk g.
// kRev (the training backward's value pass): unit_w marks a lane whose
// shifted retention row lies past the segment (unit retention), and K^ is
// scaled by kscale (k is r_t there, times the output scale).
template <class Io, bool kVExact, bool kFull, bool kSum = false, bool kKK = false,
          bool kRev = false>
__device__ __forceinline__ void key_half_ring(ChunkOps<kVExact>& op, const u32x4 (&raw)[6],
                                              const float (&nbias8)[8], bool valid, int hh,
                                              int i, int q, KeyAccR& acc,
                                              const KkHalf* kp = nullptr, float kinv = 0.0f,
                                              typename Io::raw* nk_row = nullptr,
                                              bool unit_w = false, float kscale = 1.0f) {
  const int kbase = 32 * hh + 8 * q;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
  auto tok = [&](int j) { return (kFull || valid) ? raw[j] : zero4; };
  float xr[8], xl[8], xk[8], xa[8], xb[8];
  if constexpr (!kSum) unpack8<Io>(tok(0), xr);
  unpack8<Io>(raw[1], xl);
  unpack8<Io>(tok(2), xk);
  if constexpr (kKK) {
    float x12[8], nk[8];
    unpack8<Io>(tok(4), x12);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float kk = xk[e] * kp->kks[e] * kinv;
      const float g = __builtin_amdgcn_rcpf(
          1.0f + __builtin_amdgcn_exp2f(-kLog2e * (kp->a0[e] + x12[e])));
      nk[e] = xk[e] * __builtin_fmaf(g - 1.0f, kp->ka[e], 1.0f);
      xa[e] = -kk;
      xb[e] = kk * g;
    }
    if (nk_row != nullptr && (kFull || valid)) {
      u32x4 packed;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = __builtin_bit_cast(uint16_t, Io::from_f32(nk[2 * j]));
        const uint32_t hi = __builtin_bit_cast(uint16_t, Io::from_f32(nk[2 * j + 1]));
        packed[j] = lo | (hi << 16);
      }
      *reinterpret_cast<u32x4*>(nk_row + kbase) = packed;
    }
    // the recurrence uses the gated key (masked rows stay zero)
#pragma unroll
    for (int e = 0; e < 8; ++e) xk[e] = (kFull || valid) ? nk[e] : 0.0f;
  } else {
    unpack8<Io>(tok(4), xa);
    unpack8<Io>(tok(5), xb);
  }
  constexpr float kC = kNegExpHalf * kLog2e;
  constexpr float kInvC = 1.0f / kC;
  float g2[8], gm[8], gp[8], at[8], rt[8], bh[8], kh[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    g2[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(xl[e], -kLog2e, nbias8[e]));
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float lw2 = __builtin_amdgcn_rcpf(__builtin_fmaf(g2[e], kInvC, kInvC));
    if constexpr (!kFull) lw2 = valid ? lw2 : 0.0f;
    if constexpr (kRev) lw2 = unit_w ? 0.0f : lw2;
    g2[e] = lw2;
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
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float ig = __builtin_amdgcn_exp2f(-g2[e]);                     // 1 / gamma_t
    at[e] = xa[e] * gp[e];
    if constexpr (!kSum) rt[e] = xr[e] * gm[e];
    bh[e] = xb[e] * ig;
    kh[e] = xk[e] * ig;
    if constexpr (kRev) kh[e] *= kscale;
  }
  if (i == L - 1) {
    *reinterpret_cast<f32x4*>(&op.gl[kbase]) = f32x4{gm[0], gm[1], gm[2], gm[3]};
    *reinterpret_cast<f32x4*>(&op.gl[kbase + 4]) = f32x4{gm[4], gm[5], gm[6], gm[7]};
  }
  Sp8 Rs;
  if constexpr (!kSum) Rs = split8(rt);
  const Sp8 As = split8(at), Bs = split8(bh), Ks = split8(kh);
  Sp8 Vs;
  const u32x4 vraw = tok(3);
  if constexpr (kVExact) {
    Vs.hi = __builtin_bit_cast(bf16x8, vraw);
  } else {
    float xv[8];
    unpack8<Io>(vraw, xv);
    Vs = split8(xv);
  }
  // operand rows for the state waves (keys kbase..kbase+7 land in two 4-key
  // runs of the permuted A~ / R~ rows)
  const int p0 = key_pos(kbase), p1 = key_pos(kbase + 4);
  if constexpr (!kSum) {
    *reinterpret_cast<bf16x4*>(&op.r_h[i][a_col(i, p0)]) = Rs.hi.lo;
    *reinterpret_cast<bf16x4*>(&op.r_h[i][a_col(i, p1)]) = Rs.hi.hi;
    *reinterpret_cast<bf16x4*>(&op.r_l[i][a_col(i, p0)]) = Rs.lo.lo;
    *reinterpret_cast<bf16x4*>(&op.r_l[i][a_col(i, p1)]) = Rs.lo.hi;
  }
  *reinterpret_cast<bf16x4*>(&op.at_h[i][a_col(i, p0)]) = As.hi.lo;
  *reinterpret_cast<bf16x4*>(&op.at_h[i][a_col(i, p1)]) = As.hi.hi;
  *reinterpret_cast<bf16x4*>(&op.at_l[i][a_col(i, p0)]) = As.lo.lo;
  *reinterpret_cast<bf16x4*>(&op.at_l[i][a_col(i, p1)]) = As.lo.hi;
  *reinterpret_cast<bf16x8*>(&op.b_h[i][b_col(i, kbase)]) = Bs.hi;
  *reinterpret_cast<bf16x8*>(&op.b_l[i][b_col(i, kbase)]) = Bs.lo;
  *reinterpret_cast<bf16x8*>(&op.k_h[i][b_col(i, kbase)]) = Ks.hi;
  *reinterpret_cast<bf16x8*>(&op.k_l[i][b_col(i, kbase)]) = Ks.lo;
  *reinterpret_cast<bf16x8*>(&op.v_h[i][b_col(i, kbase)]) = Vs.hi;
  if constexpr (!kVExact) *reinterpret_cast<bf16x8*>(&op.v_l[i][b_col(i, kbase)]) = Vs.lo;
  // mma32x3(X, Y), X, Y in the load layout: item e = X_{4q+e} . Y_i over
  // this lane's keys
  acc.ab = mma32x3(As, Bs, acc.ab);
  acc.abt = mma32x3(Bs, As, acc.abt);
  acc.ak = mma32x3(Ks, As, acc.ak);
  if constexpr (!kSum) {
    acc.rb = mma32x3(Bs, Rs, acc.rb);
    acc.rk = mma32x3(Ks, Rs, acc.rk);
  }
}

// T and the masked Mak, Mrb, Mrk of a chunk from its accumulated products
__device__ __forceinline__ void key_blocks_ring(ChunkOps<true>* op_t, ChunkOps<false>* op_f,
                                                const KeyAccR& acc, int i, int q) {
  f32x4 M, Mt, mak, mrb, mrk;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = 4 * q + e;
    M[e] = (r > i) ? acc.ab[e] : 0.f;
    Mt[e] = (i > r) ? acc.abt[e] : 0.f;
    mak[e] = (i > r) ? acc.ak[e] : 0.f;
    mrb[e] = (i >= r) ? acc.rb[e] : 0.f;
    mrk[e] = (i >= r) ? acc.rk[e] : 0.f;
  }
  const AOp t = t_inverse(M, Mt, i, q);
  if (op_t != nullptr) {
    store_aop(op_t->t, i, q, t);
    store_aop(op_t->mak, i, q, as_a(split4(mak)));
    store_aop(op_t->mrb, i, q, as_a(split4(mrb)));
    store_aop(op_t->mrk, i, q, as_a(split4(mrk)));
  } else {
    store_aop(op_f->t, i, q, t);
    store_aop(op_f->mak, i, q, as_a(split4(mak)));
    store_aop(op_f->mrb, i, q, as_a(split4(mrb)));
    store_aop(op_f->mrk, i, q, as_a(split4(mrk)));
  }
}

// T and the masked Mak of a summary chunk (no R-side blocks)
template <bool kVExact>
__device__ __forceinline__ void key_blocks_ring_sum(ChunkOps<kVExact>& op, const KeyAccR& acc,
                                                    int i, int q) {
  f32x4 M, Mt, mak;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int r = 4 * q + e;
    M[e] = (r > i) ? acc.ab[e] : 0.f;
    Mt[e] = (i > r) ? acc.abt[e] : 0.f;
    mak[e] = (i > r) ? acc.ak[e] : 0.f;
  }
  store_aop(op.t, i, q, t_inverse(M, Mt, i, q));
  store_aop(op.mak, i, q, as_a(split4(mak)));
}

// kKK: wkv_prepare's kk / a-gate stage fused into the key waves' load stage
// (p.k is the projected key, p.a the a-gate logits a12; the gated key goes
// to p.new_k), as in chunk64_kernel.
// kRev: the training backward's value pass (uniform segments, a multiple of
// 16 tokens): the recurrence runs from the segment's last token to its
// first, tensor j read one row later when bit j of p.shift_mask is set (a
// shifted row past the end reads as zero, with unit retention); y, the
// per-token sa (p.sa_out, fp32) and the state snapshots (p.boundary, at
// index boundary_per_seg - 1 - c for every boundary_every-th chunk) are
// written at the mirrored positions, as chunk64_kernel's reverse mode does.
// (The training forward, whose snapshot of every chunk the state waves
// would store, stays on chunk64_kernel: on this layout it ran 0.73 ms
// against 0.66.)
template <class Io, bool kKK = false, bool kRev = false>
__global__ __launch_bounds__(NTR) void chunk64r_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr bool kVExact = !__is_same(Io, IoF16);
  __shared__ SmemR<kVExact> sm;
  constexpr int kRing = kRingOf<kVExact>;

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15;
  const int q = lane >> 4;
  const int H = p.num_heads;

  // sequence split (real pieces): which sequence and piece this block is
  const int npc = p.split_pieces;
  int seq = seg, piece = 0;
  if (npc > 0) {
    const int cnt = p.split_count > 0 ? p.split_count : npc;
    seq = seg / cnt;
    piece = p.split_first + seg % cnt;
  }
  if (p.status != nullptr) {
    if (p.status[0] != 0) {
      const int64_t blk = static_cast<int64_t>(seg) * gridDim.x + h;
      const int64_t nblk = static_cast<int64_t>(gridDim.x) * gridDim.y;
      fill_output_nan<Io>(static_cast<raw*>(p.y), p.out_elems, blk, nblk);
      return;
    }
    if (seq >= p.status[2]) return;
  }
  int t0, t1;
  bool last_piece = true;
  if (npc > 0) {
    const int q0 = p.bounds[seq], q1 = p.bounds[seq + 1];
    int start, plen, last;
    split_piece(p, q1 - q0, piece, start, plen, last);
    if (piece > last) return;
    last_piece = piece == last;
    t0 = q0 + start;
    t1 = min(t0 + plen, q1);
  } else if (p.uniform_len > 0) {
    t0 = seg * p.uniform_len;
    t1 = t0 + p.uniform_len;
  } else if (p.chunk_offsets != nullptr) {
    // a sequence's list of contiguous chunks (the rl_infctx forward)
    t0 = p.bounds[p.chunk_offsets[seg]];
    t1 = p.ends[p.chunk_offsets[seg + 1] - 1];
  } else if (p.ends != nullptr) {
    t0 = p.bounds[seg];
    t1 = p.ends[seg];
  } else {
    t0 = p.bounds[seg];
    t1 = p.bounds[seg + 1];
  }
  const int slot = p.slots ? p.slots[seq] : seq;
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(H) * D;
  const int nchunks = (t1 - t0 + L - 1) / L;
  raw* yout = static_cast<raw*>(p.y);

  if (tid < kKeyW + 5) (&sm.ready[0])[tid] = 0;
  __syncthreads();   // the only workgroup barrier before the end: counters are zero

  const int vcol = 16 * (wv & 3) + i;
  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  const int64_t pbase = (static_cast<int64_t>(seq) * (npc > 0 ? npc : 1) + piece) * H + h;
  if (wv < 4) {
    // ---------------- state waves: columns [16wv, 16wv+16)
    f32x4 S[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (npc > 0 && !(piece == 0 && p.split_lead_pass)) {
      const float* sin = p.split_state + pbase * D * D;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = sin[(kb * 16 + 4 * q + e) * D + vcol];
    } else if (p.state_in != nullptr && p.state_bf16) {
      // (bf16-state contract) widened once; the state stays fp32 for the
      // whole call and is rounded back once at the end
      const uint16_t* sinb = static_cast<const uint16_t*>(p.state_in) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = IoBF16::to_f32(sinb[(kb * 16 + 4 * q + e) * D]);
    } else if (p.state_in != nullptr) {
      const float* sin = static_cast<const float*>(p.state_in) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = sin[(kb * 16 + 4 * q + e) * D];
    }
    // Each state wave writes its own 16 output columns: the chunk's rows are
    // staged in the wave's column band of yb (2-byte stores from the
    // accumulators) and read back as 16-byte pieces, lane l < 32 taking
    // row l / 2, columns 16 (wv % 4) + 8 (l % 2) .. + 7.  The band belongs
    // to this wave alone and its LDS accesses complete in order, so no wave
    // waits for another over the output.
    const int y_row = lane >> 1, y_c0 = 16 * (wv & 3) + 8 * (lane & 1);
    // value pass: sa column of this lane and its snapshot column
    float* const sa_base = kRev ? p.sa_out + head_off + vcol : nullptr;
    const int nsnap = kRev ? (p.boundary_per_seg + p.boundary_every - 1) / p.boundary_every : 0;
    float* const bnd_base =
        (kRev && p.boundary != nullptr)
            ? p.boundary + (static_cast<int64_t>(seg) * H + h) * nsnap * D * D + vcol
            : nullptr;
    for (int c = 0; c < nchunks; ++c) {
      wait_ge(&sm.ready[c % kKeyW], c / kKeyW + 1, p.spin_limit, &sm.fault);   // operators of c
      const StateOps<kVExact> o = state_load(sm.ops[c % kRing], vcol, i, q);
      if constexpr (kRev) {
        // sa goes to the staged tile (written back below), the snapshot is
        // stored here: state_compute gets neither row pointers nor a column
        const int bi = p.boundary_per_seg - 1 - c;
        const bool keep = bnd_base != nullptr && bi % p.boundary_every == 0;
        state_compute<Io, kVExact, true>(o, S, &sm.yb[0], vcol, i, q, p.scale, SaRows{}, nullptr,
                                         false, &sm.ub[0]);
        if (keep) {
          // the post-chunk state as 16-byte row pieces (store_state_tile)
          float* const snap = bnd_base - vcol + static_cast<int64_t>(bi / p.boundary_every) * D * D;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) store_state_tile(snap, 16 * (wv & 3), S[kb], kb, i, q);
        }
        // the staged sa rows of this wave's 16 columns as 16-byte pieces:
        // lane l takes token l / 4, columns 16 (wv % 4) + 4 (l % 4)..+3 (the
        // band is this wave's alone and its LDS accesses complete in order),
        // to row t0 + (n - pos) mod n of the segment, which is t1 - pos
        // except at pos = 0
        const int u_tok = lane >> 2, u_c = 16 * (wv & 3) + 4 * (lane & 3);
        const int upos = c * L + u_tok;
        const int urow = upos == 0 ? t0 : t1 - upos;
        *reinterpret_cast<f32x4*>(sa_base - vcol + static_cast<int64_t>(urow) * row_stride + u_c) =
            *reinterpret_cast<const f32x4*>(&sm.ub[u_tok][u_c]);
      } else {
        state_compute<Io, kVExact>(o, S, &sm.yb[0], vcol, i, q, p.scale);
      }
      const int pos = c * L + y_row;   // position in processing order
      const int row = kRev ? t1 - 1 - pos : t0 + pos;
      if (lane < 32 && pos < t1 - t0) {
        const u32x4 piece = *reinterpret_cast<const u32x4*>(&sm.yb[y_row][y_c0]);
        *reinterpret_cast<u32x4*>(yout + static_cast<int64_t>(row) * row_stride + head_off +
                                  y_c0) = piece;
      }
      signal(&sm.consumed[wv], c + 1);
    }
    __syncthreads();
    if (peek(&sm.fault) != 0) {
      if (tid == 0 && p.handoff_fault != nullptr) atomicAdd(p.handoff_fault, 1);
      const float qnan = quiet_nan();
      const raw nanv = Io::from_f32(qnan);
      if (yout != nullptr)
        for (int64_t e = tid; e < static_cast<int64_t>(t1 - t0) * D; e += 256)
          yout[(t0 + e / D) * row_stride + head_off + e % D] = nanv;
      if constexpr (kRev) {
        for (int64_t e = tid; e < static_cast<int64_t>(t1 - t0) * D; e += 256)
          p.sa_out[(t0 + e / D) * row_stride + head_off + e % D] = qnan;
      }
      if (npc > 0 && p.split_lead_pass && piece == 0 && !last_piece) {
        float* sout = p.split_state + (pbase + H) * D * D;
        for (int e = tid; e < D * D; e += 256) sout[e] = qnan;
      }
      return;
    }
    if (!last_piece) {
      if (p.split_lead_pass && piece == 0) {
        float* sout = p.split_state + (pbase + H) * D * D;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) sout[(kb * 16 + 4 * q + e) * D + vcol] = S[kb][e];
      }
    } else if (p.state_out != nullptr && p.state_bf16) {
      uint16_t* soutb = static_cast<uint16_t*>(p.state_out) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          soutb[(kb * 16 + 4 * q + e) * D] = IoBF16::from_f32(S[kb][e]);
    } else if (p.state_out != nullptr) {
      float* sout = static_cast<float*>(p.state_out) + sbase + vcol;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sout[(kb * 16 + 4 * q + e) * D] = S[kb][e];
    }
  } else {
    // ---------------- key waves: whole chunks kw, kw + 4, ...
    const int kw = wv - 4;
    float nbias[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        nbias[hh][e] = p.bias ? -kLog2e * Io::to_f32(static_cast<const raw*>(p.bias)[
                                             head_off + 32 * hh + 8 * q + e])
                              : 0.f;
    const raw* src[6] = {
        static_cast<const raw*>(p.r), static_cast<const raw*>(p.logits),
        static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
        static_cast<const raw*>(p.a), kKK ? nullptr : static_cast<const raw*>(p.b)};
    u32x4 rawc[2][6];
    KkHalf kph[2];
    if constexpr (kKK) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int64_t ch = head_off + 32 * hh + 8 * q + e;
          kph[hh].kks[e] = Io::to_f32(static_cast<const raw*>(p.kk_scale)[ch]);
          kph[hh].a0[e] = Io::to_f32(static_cast<const raw*>(p.a_bias)[ch]);
          kph[hh].ka[e] = Io::to_f32(static_cast<const raw*>(p.k_a)[ch]);
        }
    }
    // rows past the sequence end are loaded from its last row (in bounds);
    // key_half_ring zeroes them
    auto load_chunk = [&](int c) {
      // reverse: position c L + i reads row t1 - 1 - pos, one row later for
      // the shifted tensors (clamped into the segment; the row past its end
      // is zeroed where it is consumed)
      const int row = kRev ? t1 - 1 - (c * L + i) : min(t0 + c * L + i, t1 - 1);
      const int64_t off = static_cast<int64_t>(row) * row_stride + head_off + 8 * q;
      const int64_t off_sh = static_cast<int64_t>(min(row + 1, t1 - 1)) * row_stride + head_off + 8 * q;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int j = 0; j < 6; ++j) {
          const int64_t o = (kRev && ((p.shift_mask >> j) & 1)) ? off_sh : off;
          rawc[hh][j] = (kKK && j == 5)   // b is formed from the key
                            ? u32x4{0u, 0u, 0u, 0u}
                            : __builtin_nontemporal_load(
                                  reinterpret_cast<const u32x4*>(src[j] + o + 32 * hh));
        }
    };
    if (kw < nchunks) load_chunk(kw);
    for (int c = kw; c < nchunks; c += kKeyW) {
      // chunk c - kRing no longer read
      wait_min_ge(sm.consumed, c - kRing + 1, p.spin_limit, &sm.fault);
      ChunkOps<kVExact>& op = sm.ops[c % kRing];
      const bool full = t0 + c * L + L <= t1;
      const bool valid = t0 + c * L + i < t1;
      KeyAccR acc;
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      acc.ab = z; acc.abt = z; acc.ak = z; acc.rb = z; acc.rk = z;
      float kinv = 0.0f;
      raw* nk_row = nullptr;
      if constexpr (kKK) {
        // 1 / |k k_k| over the token's 64 keys (the four lanes of token i
        // hold 16 each)
        float ss = 0.0f;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float xk[8];
          unpack8<Io>(rawc[hh][2], xk);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float u = xk[e] * kph[hh].kks[e];
            ss = __builtin_fmaf(u, u, ss);
          }
        }
        ss += __shfl_xor(ss, 16);
        ss += __shfl_xor(ss, 32);
        kinv = __builtin_amdgcn_rcpf(fmaxf(__builtin_sqrtf(ss), 1.0e-12f));
        nk_row = static_cast<raw*>(p.new_k) +
                 static_cast<int64_t>(t0 + c * L + i) * row_stride + head_off;
      }
      if constexpr (kRev) {
        // position 0 of the segment: its shifted rows lie past the end
        const bool void_row = c == 0 && i == 0;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int j = 0; j < 6; ++j)
            if (j != 1 && void_row && ((p.shift_mask >> j) & 1)) rawc[hh][j] = u32x4{0u, 0u, 0u, 0u};
        const bool unit_w = void_row && ((p.shift_mask >> 1) & 1);
        key_half_ring<Io, kVExact, true, false, false, true>(op, rawc[0], nbias[0], true, 0, i, q,
                                                            acc, nullptr, 0.0f, nullptr, unit_w,
                                                            p.kv_scale);
        key_half_ring<Io, kVExact, true, false, false, true>(op, rawc[1], nbias[1], true, 1, i, q,
                                                            acc, nullptr, 0.0f, nullptr, unit_w,
                                                            p.kv_scale);
      } else if (full) {
        key_half_ring<Io, kVExact, true, false, kKK>(op, rawc[0], nbias[0], true, 0, i, q, acc,
                                                     &kph[0], kinv, nk_row);
        key_half_ring<Io, kVExact, true, false, kKK>(op, rawc[1], nbias[1], true, 1, i, q, acc,
                                                     &kph[1], kinv, nk_row);
      } else {
        key_half_ring<Io, kVExact, false, false, kKK>(op, rawc[0], nbias[0], valid, 0, i, q,
                                                      acc, &kph[0], kinv, nk_row);
        key_half_ring<Io, kVExact, false, false, kKK>(op, rawc[1], nbias[1], valid, 1, i, q,
                                                      acc, &kph[1], kinv, nk_row);
      }
      if (c + kKeyW < nchunks) load_chunk(c + kKeyW);
      if constexpr (kVExact)
        key_blocks_ring(&op, nullptr, acc, i, q);
      else
        key_blocks_ring(nullptr, &op, acc, i, q);
      if (!p.handoff_stall) signal(&sm.ready[kw], (c - kw) / kKeyW + 1);
    }
    __syncthreads();   // pairs with the state waves' final barrier
  }
}

// Summary pass of a sequence split on the ring layout: block y = n * count +
// j summarises piece split_first + j of sequence n (only pieces before the
// sequence's last).  Four key waves build whole chunks into the operator
// ring as in chunk64r_kernel, without R~ and the R-side blocks.  Each of the
// four state waves carries, for its 16 columns, both the piece's zero-start
// final state F and its transition Phi (identity start, V = 0): two
// independent chains over the same operands, read from LDS once.  Writes
// split_summary[(y * 2 + {0: F, 1: Phi}) * H + h]; nothing else.
template <class Io>
__global__ __launch_bounds__(NTR) void chunk64rs_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr bool kVExact = !__is_same(Io, IoF16);
  __shared__ SmemR<kVExact> sm;
  constexpr int kRing = kRingOf<kVExact>;

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int i = lane & 15;
  const int q = lane >> 4;
  const int H = p.num_heads;
  const int cnt = p.split_count > 0 ? p.split_count : p.split_pieces - 1;
  const int seq = seg / cnt, piece = p.split_first + seg % cnt;
  if (p.status != nullptr && (p.status[0] != 0 || seq >= p.status[2])) return;
  const int q0 = p.bounds[seq], q1 = p.bounds[seq + 1];
  int start, plen, last;
  split_piece(p, q1 - q0, piece, start, plen, last);
  if (piece >= last) return;
  const int t0 = q0 + start;
  const int t1 = min(t0 + plen, q1);
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(H) * D;
  const int nchunks = (t1 - t0 + L - 1) / L;

  if (tid < kKeyW + 5) (&sm.ready[0])[tid] = 0;
  __syncthreads();   // the only workgroup barrier before the end: counters are zero

  const int vcol = 16 * (wv & 3) + i;
  if (wv < 4) {
    f32x4 F[4], Phi[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        F[kb][e] = 0.0f;
        Phi[kb][e] = (kb * 16 + 4 * q + e == vcol) ? 1.0f : 0.0f;
      }
    for (int c = 0; c < nchunks; ++c) {
      wait_ge(&sm.ready[c % kKeyW], c / kKeyW + 1, p.spin_limit, &sm.fault);   // operators of c
      // every operand is in registers before the slot is released
      const StateOps<kVExact> o = state_load<kVExact, true>(sm.ops[c % kRing], vcol, i, q);
      signal(&sm.consumed[wv], c + 1);
      state_compute<Io, kVExact, false, true>(o, F, nullptr, vcol, i, q, 1.0f, SaRows{},
                                              nullptr, false);
      state_compute<Io, kVExact, false, true>(o, Phi, nullptr, vcol, i, q, 1.0f, SaRows{},
                                              nullptr, true);
    }
    __syncthreads();
    float* sout = p.split_summary + (static_cast<int64_t>(seg) * 2 * H + h) * D * D;
    float* pout = sout + static_cast<int64_t>(H) * D * D;
    if (peek(&sm.fault) != 0) {
      // the pieces that start from this summary come out NaN as well
      if (tid == 0 && p.handoff_fault != nullptr) atomicAdd(p.handoff_fault, 1);
      const float qnan = quiet_nan();
      for (int e = tid; e < D * D; e += 256) {
        sout[e] = qnan;
        pout[e] = qnan;
      }
      return;
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sout[(kb * 16 + 4 * q + e) * D + vcol] = F[kb][e];
        pout[(kb * 16 + 4 * q + e) * D + vcol] = Phi[kb][e];
      }
  } else {
    // ---------------- key waves: whole chunks kw, kw + 4, ...
    const int kw = wv - 4;
    float nbias[2][8];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        nbias[hh][e] = p.bias ? -kLog2e * Io::to_f32(static_cast<const raw*>(p.bias)[
                                             head_off + 32 * hh + 8 * q + e])
                              : 0.f;
    const raw* src[6] = {
        nullptr, static_cast<const raw*>(p.logits),
        static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
        static_cast<const raw*>(p.a), static_cast<const raw*>(p.b)};
    u32x4 rawc[2][6];
    auto load_chunk = [&](int c) {
      const int row = min(t0 + c * L + i, t1 - 1);
      const int64_t off = static_cast<int64_t>(row) * row_stride + head_off + 8 * q;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        rawc[hh][0] = u32x4{0u, 0u, 0u, 0u};   // r: not read by the summary
#pragma unroll
        for (int j = 1; j < 6; ++j)
          rawc[hh][j] = __builtin_nontemporal_load(
              reinterpret_cast<const u32x4*>(src[j] + off + 32 * hh));
      }
    };
    if (kw < nchunks) load_chunk(kw);
    for (int c = kw; c < nchunks; c += kKeyW) {
      // chunk c - kRing no longer read
      wait_min_ge(sm.consumed, c - kRing + 1, p.spin_limit, &sm.fault);
      ChunkOps<kVExact>& op = sm.ops[c % kRing];
      const bool full = t0 + c * L + L <= t1;
      const bool valid = t0 + c * L + i < t1;
      KeyAccR acc;
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      acc.ab = z; acc.abt = z; acc.ak = z; acc.rb = z; acc.rk = z;
      if (full) {
        key_half_ring<Io, kVExact, true, true>(op, rawc[0], nbias[0], true, 0, i, q, acc);
        key_half_ring<Io, kVExact, true, true>(op, rawc[1], nbias[1], true, 1, i, q, acc);
      } else {
        key_half_ring<Io, kVExact, false, true>(op, rawc[0], nbias[0], valid, 0, i, q, acc);
        key_half_ring<Io, kVExact, false, true>(op, rawc[1], nbias[1], valid, 1, i, q, acc);
      }
      if (c + kKeyW < nchunks) load_chunk(c + kKeyW);
      key_blocks_ring_sum(op, acc, i, q);
      if (!p.handoff_stall) signal(&sm.ready[kw], (c - kw) / kKeyW + 1);
    }
    __syncthreads();   // pairs with the state waves' final barrier
  }
}

}  // namespace

namespace {
// Blocks of the chunked kernels whose wave hand-off gave up, per device (each
// device holds its own copy; read through fr2_handoff_fault_count).
__device__ int g_handoff_faults;
std::atomic<int> g_spin_limit{1 << 20};
std::atomic<bool> g_handoff_stall{false};
std::atomic<int> g_chunk_ring{1};
std::atomic<int*> g_fault_ptr[64];
}  // namespace

int* handoff_fault_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  int* ptr = g_fault_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    if (hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(g_handoff_faults)) !=
        hipSuccess)
      return nullptr;
    g_fault_ptr[dev].store(ptr, std::memory_order_release);
  }
  return ptr;
}
int handoff_spin_limit() { return g_spin_limit.load(std::memory_order_relaxed); }
bool handoff_stall() { return g_handoff_stall.load(std::memory_order_relaxed); }
bool chunk_ring_enabled() { return g_chunk_ring.load(std::memory_order_relaxed) != 0; }
void set_chunk_ring(int on) { g_chunk_ring.store(on, std::memory_order_relaxed); }
void set_handoff_stall(bool on) { g_handoff_stall.store(on, std::memory_order_relaxed); }
void set_handoff_spin_limit(int polls) {
  g_spin_limit.store(polls < 0 ? (1 << 20) : polls, std::memory_order_relaxed);
}

// the ring variant covers the inference contracts (fp32 or bf16 state,
// packed, uniform or chunk-list segments); the training outputs (boundary
// snapshots, sa) and the fused read-out stay on chunk64_kernel
bool ring_contract(const SegArgs& p) {
  return chunk_ring_enabled() && p.boundary == nullptr && p.sa_out == nullptr &&
         p.ro_out == nullptr;
}

int launch_chunked(int dtype, const SegArgs& args, int nseg, int max_seqlen, hipStream_t s) {
  (void)max_seqlen;
  SegArgs p = args;
  p.spin_limit = handoff_spin_limit();
  p.handoff_stall = handoff_stall();
  p.handoff_fault = handoff_fault_word();
  const bool train = p.sa_out != nullptr || p.boundary != nullptr || p.reverse;
  const dim3 grid(p.num_heads, nseg);
  if (train) {
    // the training contract: uniform segments whose length is a multiple of
    // the 16-token chunk, both outputs present, bf16 tokens (an initial
    // state, or in reverse mode an initial dL/dS, may be given)
    if (p.sa_out == nullptr || (p.boundary == nullptr && !p.reverse) || p.boundary_len != L ||
        p.uniform_len <= 0 || p.uniform_len % L != 0 || dtype != FR2_DTYPE_BFLOAT16)
      return FR2_ERR_UNSUPPORTED;
    if (p.reverse && chunk_ring_enabled())
      hipLaunchKernelGGL((chunk64r_kernel<IoBF16, false, true>), grid, dim3(NTR), 0, s, p);
    else if (p.reverse)
      hipLaunchKernelGGL((chunk64_kernel<IoBF16, true, true>), grid, dim3(NT), 0, s, p);
    else
      hipLaunchKernelGGL((chunk64_kernel<IoBF16, true>), grid, dim3(NT), 0, s, p);
  } else if (!ring_contract(p)) {
    if (dtype == FR2_DTYPE_BFLOAT16)
      hipLaunchKernelGGL((chunk64_kernel<IoBF16, false>), grid, dim3(NT), 0, s, p);
    else if (dtype == FR2_DTYPE_FLOAT16)
      hipLaunchKernelGGL((chunk64_kernel<IoF16, false>), grid, dim3(NT), 0, s, p);
    else
      return FR2_ERR_UNSUPPORTED;
  } else if (dtype == FR2_DTYPE_BFLOAT16) {
    hipLaunchKernelGGL((chunk64r_kernel<IoBF16>), grid, dim3(NTR), 0, s, p);
  } else if (dtype == FR2_DTYPE_FLOAT16) {
    hipLaunchKernelGGL((chunk64r_kernel<IoF16>), grid, dim3(NTR), 0, s, p);
  } else {
    return FR2_ERR_UNSUPPORTED;
  }
  return record_launch();
}

int launch_chunked_kk(int dtype, const SegArgs& args, int nseg, hipStream_t s) {
  if (args.sa_out != nullptr || args.boundary != nullptr || args.reverse ||
      args.split_pieces > 0 || args.state_bf16 || args.kk_scale == nullptr ||
      args.a_bias == nullptr || args.k_a == nullptr || args.new_k == nullptr)
    return FR2_ERR_INVALID_ARGUMENT;
  SegArgs p = args;
  p.spin_limit = handoff_spin_limit();
  p.handoff_stall = handoff_stall();
  p.handoff_fault = handoff_fault_word();
  const dim3 grid(p.num_heads, nseg);
  const bool ro = p.ro_out != nullptr;
  if (ro && (p.ro_g == nullptr || p.ro_rk == nullptr || p.ro_lnw == nullptr ||
             p.ro_lnb == nullptr))
    return FR2_ERR_INVALID_ARGUMENT;
  // the fused read-out needs a token's whole output row at the write-back:
  // chunk64_kernel; the kk / a-gate stage alone runs on the ring variant
  const bool ring = !ro && ring_contract(p);
  if (dtype == FR2_DTYPE_BFLOAT16) {
    if (ro)
      hipLaunchKernelGGL((chunk64_kernel<IoBF16, false, false, false, true, true>), grid,
                         dim3(NT), 0, s, p);
    else if (ring)
      hipLaunchKernelGGL((chunk64r_kernel<IoBF16, true>), grid, dim3(NTR), 0, s, p);
    else
      hipLaunchKernelGGL((chunk64_kernel<IoBF16, false, false, false, true>), grid, dim3(NT), 0,
                         s, p);
  } else if (dtype == FR2_DTYPE_FLOAT16) {
    if (ro)
      hipLaunchKernelGGL((chunk64_kernel<IoF16, false, false, false, true, true>), grid, dim3(NT),
                         0, s, p);
    else if (ring)
      hipLaunchKernelGGL((chunk64r_kernel<IoF16, true>), grid, dim3(NTR), 0, s, p);
    else
      hipLaunchKernelGGL((chunk64_kernel<IoF16, false, false, false, true>), grid, dim3(NT), 0,
                         s, p);
  } else {
    return FR2_ERR_UNSUPPORTED;
  }
  return record_launch();
}

namespace {

// Start states of the pieces of a split sequence: S(j+1) = Phi_j S(j) + F_j,
// written to split_state[n * pieces + j + 1].  Classic split (split_first
// 0): S(0) = the slot state, also copied to split_state[n * pieces] (the real
// pass's last piece overwrites the slot while its first piece may not have
// read it yet, so every piece starts from this copy).  Lead split
// (split_first 1): S(1) is piece 0's end state, already in
// split_state[n * pieces + 1] from the lead pass.  The summaries of pieces
// split_first.. are at index n * split_count + (j - split_first).
// One 256-thread block per (head, sequence); thread t owns column t % 64 of
// rows 16 (t / 64) .. +15.
__global__ __launch_bounds__(256) void split_combine_kernel(SegArgs p) {
  __shared__ float phi[D][D + 1];
  __shared__ float st[D][D + 1];
  const int h = blockIdx.x, n = blockIdx.y, tid = threadIdx.x, H = p.num_heads;
  if (p.status != nullptr && (p.status[0] != 0 || n >= p.status[2])) return;
  int start, plen, last;
  split_piece(p, p.bounds[n + 1] - p.bounds[n], 0, start, plen, last);
  const int c = tid & 63, r0 = (tid >> 6) * 16;
  const int j0 = p.split_first;
  if (j0 == 0) {
    const int slot = p.slots ? p.slots[n] : n;
    // the slot state: fp32, or (bf16-state contract) bf16 widened once
    const int64_t s0 = (static_cast<int64_t>(slot) * H + h) * D * D;
    const float* s0f = static_cast<const float*>(p.state_in) + s0;
    const uint16_t* s0b = static_cast<const uint16_t*>(p.state_in) + s0;
    float* out0 = p.split_state + (static_cast<int64_t>(n) * p.split_pieces * H + h) * D * D;
    for (int r = r0; r < r0 + 16; ++r) {
      st[r][c] = p.state_bf16 ? IoBF16::to_f32(s0b[r * D + c]) : s0f[r * D + c];
      out0[r * D + c] = st[r][c];
    }
  } else {
    // pieces 0 and 1 need no combined start: the lead pass handed piece 1 its
    // start directly
    if (last <= 1) return;
    const float* s1 =
        p.split_state + ((static_cast<int64_t>(n) * p.split_pieces + 1) * H + h) * D * D;
    for (int r = r0; r < r0 + 16; ++r) st[r][c] = s1[r * D + c];
  }
  const int cnt = p.split_count > 0 ? p.split_count : p.split_pieces - 1;
  for (int j = j0; j < last; ++j) {
    const int64_t pair = static_cast<int64_t>(n) * cnt + (j - j0);
    const float* f = p.split_summary + ((pair * 2) * H + h) * D * D;
    const float* ph = p.split_summary + ((pair * 2 + 1) * H + h) * D * D;
    for (int r = r0; r < r0 + 16; ++r) phi[r][c] = ph[r * D + c];
    __syncthreads();
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = f[(r0 + e) * D + c];
    for (int k = 0; k < D; ++k) {
      const float sk = st[k][c];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = __builtin_fmaf(phi[r0 + e][k], sk, acc[e]);
    }
    __syncthreads();   // every thread is done reading st and phi
    float* out = p.split_state +
                 ((static_cast<int64_t>(n) * p.split_pieces + j + 1) * H + h) * D * D;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      st[r0 + e][c] = acc[e];
      out[(r0 + e) * D + c] = acc[e];
    }
  }
}

}  // namespace

int64_t split_workspace_floats(int nseg, int H, int pieces) {
  return static_cast<int64_t>(nseg) * (3 * pieces - 2) * H * D * D;
}

namespace {

// Fork/join events of the pipelined split, created once per thread and
// device (an event recorded by one thread is never re-recorded by another
// while its wait is pending).
struct SplitEvents {
  hipEvent_t fork = nullptr, join = nullptr;
};
thread_local SplitEvents t_split_events[64];

bool split_events(SplitEvents*& ev) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
  ev = &t_split_events[dev];
  if (ev->fork == nullptr &&
      hipEventCreateWithFlags(&ev->fork, hipEventDisableTiming) != hipSuccess) {
    ev->fork = nullptr;
    return false;
  }
  if (ev->join == nullptr &&
      hipEventCreateWithFlags(&ev->join, hipEventDisableTiming) != hipSuccess) {
    ev->join = nullptr;
    return false;
  }
  return true;
}

// a real (non-summary) pass: the ring variant when it is selected
template <class Io>
void launch_real_pass(dim3 grid, hipStream_t s, const SegArgs& p) {
  if (ring_contract(p))
    hipLaunchKernelGGL((chunk64r_kernel<Io>), grid, dim3(NTR), 0, s, p);
  else
    hipLaunchKernelGGL((chunk64_kernel<Io, false>), grid, dim3(NT), 0, s, p);
}

// the summary pass: the ring variant when it is selected
template <class Io>
void launch_summary_pass(dim3 grid, hipStream_t s, const SegArgs& p) {
  if (chunk_ring_enabled())
    hipLaunchKernelGGL((chunk64rs_kernel<Io>), grid, dim3(NTR), 0, s, p);
  else
    hipLaunchKernelGGL((chunk64_kernel<Io, false, false, true>), grid, dim3(NT_SUM), 0, s, p);
}

template <class Io>
int launch_split_kernels(const SegArgs& p, int nseg, int pieces, hipStream_t s,
                         hipStream_t aux) {
  const int H = p.num_heads;
  if (p.split_lead <= 0) {
    // classic: summaries of pieces 0..P-2, combine from the slot, every piece
    const dim3 gsum(H, nseg * (pieces - 1)), gcomb(H, nseg), greal(H, nseg * pieces);
    launch_summary_pass<Io>(gsum, s, p);
    hipLaunchKernelGGL(split_combine_kernel, gcomb, dim3(256), 0, s, p);
    launch_real_pass<Io>(greal, s, p);
    return FR2_OK;
  }
  // lead: piece 0 (from the slot) on the aux stream, concurrently with the
  // summaries of pieces 1..P-2; then the combine from piece 0's end state and
  // pieces 1..P-1.  Without a usable second stream (or its events) the same
  // passes run on one stream, with the same results.
  SplitEvents* ev = nullptr;
  if (aux != nullptr) {
    if (!split_events(ev) || hipEventRecord(ev->fork, s) != hipSuccess ||
        hipStreamWaitEvent(aux, ev->fork, 0) != hipSuccess) {
      (void)hipGetLastError();
      aux = nullptr;   // nothing is enqueued yet: one stream is still legal
    }
  }
  const hipStream_t s_lead = aux != nullptr ? aux : s;
  SegArgs pl = p;
  pl.split_first = 0;
  pl.split_count = 1;
  pl.split_lead_pass = true;
  launch_real_pass<Io>(dim3(H, nseg), s_lead, pl);
  SegArgs ps = p;
  ps.split_first = 1;
  ps.split_count = pieces - 2;
  if (pieces > 2)
    launch_summary_pass<Io>(dim3(H, nseg * (pieces - 2)), s, ps);
  if (aux != nullptr) {
    // the join cannot be replaced by a host wait: that is illegal while the
    // streams are being captured into a graph
    if (hipEventRecord(ev->join, aux) != hipSuccess ||
        hipStreamWaitEvent(s, ev->join, 0) != hipSuccess)
      return FR2_ERR_LAUNCH;
  }
  if (pieces > 2) hipLaunchKernelGGL(split_combine_kernel, dim3(H, nseg), dim3(256), 0, s, ps);
  SegArgs pr = p;
  pr.split_first = 1;
  pr.split_count = pieces - 1;
  launch_real_pass<Io>(dim3(H, nseg * (pieces - 1)), s, pr);
  return FR2_OK;
}

}  // namespace

int launch_chunked_split(int dtype, SegArgs p, int nseg, int pieces, int piece_len,
                         int lead_len, float* workspace, hipStream_t s, hipStream_t aux) {
  if (p.sa_out != nullptr || p.boundary != nullptr || p.reverse ||
      p.uniform_len > 0 || p.ends != nullptr || p.chunk_offsets != nullptr)
    return FR2_ERR_UNSUPPORTED;
  if (pieces < 2 || piece_len <= 0 || piece_len % GT != 0 || lead_len < 0 ||
      lead_len % GT != 0 || workspace == nullptr || p.state_in == nullptr ||
      p.state_out != p.state_in || static_cast<int64_t>(nseg) * pieces > 65535)
    return FR2_ERR_INVALID_ARGUMENT;
  if (dtype != FR2_DTYPE_BFLOAT16 && dtype != FR2_DTYPE_FLOAT16) return FR2_ERR_UNSUPPORTED;
  p.spin_limit = handoff_spin_limit();
  p.handoff_stall = handoff_stall();
  p.handoff_fault = handoff_fault_word();
  p.split_pieces = pieces;
  p.split_len = piece_len;
  p.split_lead = lead_len;
  p.split_summary = workspace;
  p.split_state = workspace + static_cast<int64_t>(nseg) * (pieces - 1) * 2 * p.num_heads * D * D;
  const int rc = dtype == FR2_DTYPE_BFLOAT16 ? launch_split_kernels<IoBF16>(p, nseg, pieces, s, aux)
                                             : launch_split_kernels<IoF16>(p, nseg, pieces, s, aux);
  const int lrc = record_launch();
  return rc != FR2_OK ? rc : lrc;
}

}  // namespace fr2
