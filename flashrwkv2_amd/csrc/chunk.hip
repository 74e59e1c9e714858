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
#include "recurrent.h"

#include <cstddef>
#include <type_traits>

namespace fr2 {
namespace {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int D = 64;
constexpr int L = 16;          // tokens per chunk
constexpr int G = 2;           // chunks per group
constexpr int GT = L * G;      // tokens per group
constexpr int NT = 512;        // 8 wavefronts: 4 state + 4 key
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegExpHalf = -0.6065306597126334f;   // -exp(-1/2)

__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct Sp4 { bf16x4 hi, lo; };
struct Sp8 { bf16x8 hi, lo; };

__device__ __forceinline__ Sp4 split4(f32x4 x) {
  Sp4 s;
  s.hi = __builtin_convertvector(x, bf16x4);
  s.lo = __builtin_convertvector(x - __builtin_convertvector(s.hi, f32x4), bf16x4);
  return s;
}
typedef float f32x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ Sp8 split8(const float* x) {
  f32x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = x[e];
  Sp8 s;
  s.hi = __builtin_convertvector(v, bf16x8);
  s.lo = __builtin_convertvector(v - __builtin_convertvector(s.hi, f32x8), bf16x8);
  return s;
}

__device__ __forceinline__ f32x4 mma32x3(const Sp8& a, const Sp8& b, f32x4 c) {
  c = mma32(a.lo, b.hi, c);
  c = mma32(a.hi, b.lo, c);
  return mma32(a.hi, b.hi, c);
}

// K = 16 products packed into K = 32 instructions: lane group q supplies K
// positions 8q..8q+7 = (first operand's 4q..4q+3, second's 4q..4q+3), so
// [x | y] x [u ; v] = x u + y v.  Every product of the kernel runs on the one
// K = 32 opcode: with this toolchain an accumulator produced by
// v_mfma_f32_16x16x32_bf16 and consumed as src C by v_mfma_f32_16x16x16_bf16
// gave wrong sums on gfx950, while same-opcode chains are exact.
__device__ __forceinline__ bf16x8 cat4(bf16x4 x, bf16x4 y) {
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ f32x4 mma2(bf16x4 x, bf16x4 y, bf16x4 u, bf16x4 v, f32x4 c) {
  return mma32(cat4(x, y), cat4(u, v), c);
}
// c += a b (split operands): a.hi b.lo + a.lo b.hi, then a.hi b.hi
__device__ __forceinline__ f32x4 mma16x3p(Sp4 a, Sp4 b, f32x4 c) {
  const bf16x4 z = {};
  c = mma2(a.hi, a.lo, b.lo, b.hi, c);
  return mma2(a.hi, z, b.hi, z, c);
}
// c += a b with b exact in bf16: [a.hi | a.lo] x [b ; b]
__device__ __forceinline__ f32x4 mma16x2p(Sp4 a, bf16x4 b, f32x4 c) {
  return mma2(a.hi, a.lo, b, b, c);
}

// X Y for 16x16 matrices held in accumulator layout (lane l: column l%16,
// rows 4(l/16)+e): the accumulator layout of X^T is the A-operand layout of X
// and the accumulator layout of Y is the B-operand layout of Y.
__device__ __forceinline__ f32x4 mm(const Sp4& xt, const Sp4& y, f32x4 c) {
  return mma16x3p(xt, y, c);
}

// Inclusive prefix sum over the 16 lanes of a DPP row (the token axis).
template <int N>
__device__ __forceinline__ float row_shr(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x110 + N, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_scan(float x) {
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  return x;
}

// Eight 16-bit token values packed in a 16-byte vector, widened to fp32.
template <class Io>
__device__ __forceinline__ void unpack8(u32x4 v, float* out) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t w = v[e];
    if constexpr (__is_same(Io, IoBF16)) {
      out[2 * e] = __uint_as_float(w << 16);
      out[2 * e + 1] = __uint_as_float(w & 0xffff0000u);
    } else {
      out[2 * e] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
      out[2 * e + 1] =
          static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
    }
  }
}

__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * kLog2e);
}

// Operators of one chunk consumed by the state path.  For bf16 tokens V is
// exact in bf16 (no lo part) and the rows are padded for bank spread; fp16
// tokens need V's lo part and use unpadded rows to fit the LDS budget.
template <bool kVExact>
struct alignas(16) ChunkOps {
  static constexpr int RP = kVExact ? D + 8 : D;    // key row length
  static constexpr int LP = kVExact ? L + 4 : L;    // token row of transposed arrays
  float gl[D];                        // gamma_L (read as 16-byte vectors)
  __bf16 at_h[L][RP], at_l[L][RP];    // A~ rows, keys at key_pos()
  __bf16 r_h[L][RP], r_l[L][RP];      // R~ rows, keys at key_pos()
  __bf16 bT_h[D][LP], bT_l[D][LP];    // B^ transposed
  __bf16 kT_h[D][LP], kT_l[D][LP];    // K^ transposed
  __bf16 vT_h[D][LP];                 // V transposed
  __bf16 vT_l[kVExact ? 1 : D][LP];   // V lo part (fp16 tokens only)
  __bf16 t_h[L][L], t_l[L][L];        // T
  __bf16 mak_h[L][L], mak_l[L][L];    // Mak, Mrb, Mrk (masked)
  __bf16 mrb_h[L][L], mrb_l[L][L];
  __bf16 mrk_h[L][L], mrk_l[L][L];
};
// every 16-byte vector access above needs its array 16-byte aligned
static_assert(offsetof(ChunkOps<true>, at_h) % 16 == 0 && offsetof(ChunkOps<true>, r_h) % 16 == 0,
              "row arrays must be 16-byte aligned");
static_assert(sizeof(ChunkOps<true>) % 16 == 0 && sizeof(ChunkOps<false>) % 16 == 0,
              "operator blocks must keep 16-byte alignment");

template <bool kVExact>
struct alignas(16) Smem {
  ChunkOps<kVExact> ops[2][G];        // [group parity][chunk]
  float mpart[G][2][4][L][L];         // [chunk][key half][block][t][s]
  uint16_t yb[2][GT][D];              // outputs of a group, by parity
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
  s.hi = *reinterpret_cast<const bf16x8*>(&xh[i][32 * m + 8 * q]);
  s.lo = *reinterpret_cast<const bf16x8*>(&xl[i][32 * m + 8 * q]);
  return s;
}

template <int N>
__device__ __forceinline__ Sp4 load_a16(const __bf16 (*h)[N], const __bf16 (*l)[N], int row,
                                        int q) {
  Sp4 s;
  s.hi = *reinterpret_cast<const bf16x4*>(&h[row][4 * q]);
  s.lo = *reinterpret_cast<const bf16x4*>(&l[row][4 * q]);
  return s;
}

// ---------------------------------------------------------------------------
// key side, part 1: operands of chunk cc (keys 32hh + 8q + e of token i) and
// the partial token-token blocks over this lane's keys.  The operand values
// stay in registers until part 2 stores them for the state waves.
// ---------------------------------------------------------------------------
struct KeyRegs {
  Sp8 As, Rs, Bs, Ks, Vs;
};

template <class Io, bool kVExact>
__device__ __forceinline__ void key_part1(Smem<kVExact>& sm, ChunkOps<kVExact>& op,
                                          const u32x4 (&raw)[6], const float (&bias8)[8],
                                          bool valid, int cc, int hh, int i, int q,
                                          KeyRegs& kr) {
  const int kbase = 32 * hh + 8 * q;
  float xr[8], xl[8], xk[8], xv[8], xa[8], xb[8];
  unpack8<Io>(raw[0], xr);
  unpack8<Io>(raw[1], xl);
  unpack8<Io>(raw[2], xk);
  unpack8<Io>(raw[3], xv);
  unpack8<Io>(raw[4], xa);
  unpack8<Io>(raw[5], xb);
  float at[8], rt[8], bh[8], kh[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = xl[e] + bias8[e];
    const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2e * x));
    // base-2 log of the retention: log2(w) = -exp(-1/2) log2(e) sigmoid(x)
    const float lw2 = valid ? (kNegExpHalf * kLog2e) * sig : 0.0f;
    const float g2 = row_scan(lw2);
    const float gm = __builtin_amdgcn_exp2f(g2);
    const float gp = __builtin_amdgcn_exp2f(g2 - lw2);
    const float ig = __builtin_amdgcn_exp2f(-g2);
    at[e] = xa[e] * gp;
    rt[e] = xr[e] * gm;
    bh[e] = xb[e] * ig;
    kh[e] = xk[e] * ig;
    if (i == L - 1) op.gl[kbase + e] = gm;
  }
  kr.As = split8(at);
  kr.Rs = split8(rt);
  kr.Bs = split8(bh);
  kr.Ks = split8(kh);
  if constexpr (kVExact) {
    f32x8 v8;
#pragma unroll
    for (int e = 0; e < 8; ++e) v8[e] = xv[e];
    kr.Vs.hi = __builtin_convertvector(v8, bf16x8);
  } else {
    kr.Vs = split8(xv);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const f32x4 pab = mma32x3(kr.As, kr.Bs, zero);
  const f32x4 pak = mma32x3(kr.As, kr.Ks, zero);
  const f32x4 prb = mma32x3(kr.Rs, kr.Bs, zero);
  const f32x4 prk = mma32x3(kr.Rs, kr.Ks, zero);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    sm.mpart[cc][hh][0][4 * q + e][i] = pab[e];
    sm.mpart[cc][hh][1][4 * q + e][i] = pak[e];
    sm.mpart[cc][hh][2][4 * q + e][i] = prb[e];
    sm.mpart[cc][hh][3][4 * q + e][i] = prk[e];
  }
}

// ---------------------------------------------------------------------------
// key side, part 2: store the operands; hh = 0 forms T, hh = 1 the masked
// Mak, Mrb, Mrk
// ---------------------------------------------------------------------------
template <bool kVExact>
__device__ __forceinline__ void key_part2(Smem<kVExact>& sm, ChunkOps<kVExact>& op, int cc,
                                          int hh, int i, int q, const KeyRegs& kr) {
  const int kbase = 32 * hh + 8 * q;
  {
    // keys kbase..kbase+7 land in two 4-key runs of the permuted rows
    const int p0 = key_pos(kbase), p1 = key_pos(kbase + 4);
    *reinterpret_cast<bf16x4*>(&op.r_h[i][p0]) = kr.Rs.hi.lo;
    *reinterpret_cast<bf16x4*>(&op.r_h[i][p1]) = kr.Rs.hi.hi;
    *reinterpret_cast<bf16x4*>(&op.r_l[i][p0]) = kr.Rs.lo.lo;
    *reinterpret_cast<bf16x4*>(&op.r_l[i][p1]) = kr.Rs.lo.hi;
    *reinterpret_cast<bf16x4*>(&op.at_h[i][p0]) = kr.As.hi.lo;
    *reinterpret_cast<bf16x4*>(&op.at_h[i][p1]) = kr.As.hi.hi;
    *reinterpret_cast<bf16x4*>(&op.at_l[i][p0]) = kr.As.lo.lo;
    *reinterpret_cast<bf16x4*>(&op.at_l[i][p1]) = kr.As.lo.hi;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = kbase + e;
    op.bT_h[k][i] = kr.Bs.hi[e];
    op.bT_l[k][i] = kr.Bs.lo[e];
    op.kT_h[k][i] = kr.Ks.hi[e];
    op.kT_l[k][i] = kr.Ks.lo[e];
    op.vT_h[k][i] = kr.Vs.hi[e];
    if constexpr (!kVExact) op.vT_l[k][i] = kr.Vs.lo[e];
  }
  const float (*mp0)[4][L][L] = sm.mpart[cc];
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  if (hh == 0) {
    f32x4 M, Mt, I4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * q + e;
      M[e] = (r > i) ? mp0[0][0][r][i] + mp0[1][0][r][i] : 0.f;
      Mt[e] = (i > r) ? mp0[0][0][i][r] + mp0[1][0][i][r] : 0.f;
      I4[e] = (r == i) ? 1.0f : 0.0f;
    }
    // T = (I - Mab)^-1 = (I+M)(I+M^2)(I+M^4)(I+M^8) (M strictly lower,
    // 16x16), keeping both orientations of each factor in accumulator
    // registers; every factor is split into hi/lo once.
    const Sp4 sM = split4(M), sMt = split4(Mt);
    const f32x4 M2 = mm(sMt, sM, zero);
    const f32x4 M2t = mm(sM, sMt, zero);
    const Sp4 sM2 = split4(M2), sM2t = split4(M2t);
    const f32x4 T1t = I4 + Mt;
    const f32x4 T2t = mm(sM2, split4(T1t), T1t);
    const f32x4 M4 = mm(sM2t, sM2, zero);
    const f32x4 M4t = mm(sM2, sM2t, zero);
    const Sp4 sM4 = split4(M4);
    const f32x4 T4t = mm(sM4, split4(T2t), T2t);
    const f32x4 M8 = mm(split4(M4t), sM4, zero);
    const f32x4 Tt = mm(split4(M8), split4(T4t), T4t);   // accumulator of T^T
    const Sp4 Ta = split4(Tt);                            // = A operand of T
    *reinterpret_cast<bf16x4*>(&op.t_h[i][4 * q]) = Ta.hi;
    *reinterpret_cast<bf16x4*>(&op.t_l[i][4 * q]) = Ta.lo;
  } else {
    f32x4 mak, mrb, mrk;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int s = 4 * q + e;       // A-operand layout: row i, K = s
      mak[e] = (i > s) ? mp0[0][1][i][s] + mp0[1][1][i][s] : 0.f;
      mrb[e] = (i >= s) ? mp0[0][2][i][s] + mp0[1][2][i][s] : 0.f;
      mrk[e] = (i >= s) ? mp0[0][3][i][s] + mp0[1][3][i][s] : 0.f;
    }
    const Sp4 Mak = split4(mak), Mrb = split4(mrb), Mrk = split4(mrk);
    *reinterpret_cast<bf16x4*>(&op.mak_h[i][4 * q]) = Mak.hi;
    *reinterpret_cast<bf16x4*>(&op.mak_l[i][4 * q]) = Mak.lo;
    *reinterpret_cast<bf16x4*>(&op.mrb_h[i][4 * q]) = Mrb.hi;
    *reinterpret_cast<bf16x4*>(&op.mrb_l[i][4 * q]) = Mrb.lo;
    *reinterpret_cast<bf16x4*>(&op.mrk_h[i][4 * q]) = Mrk.hi;
    *reinterpret_cast<bf16x4*>(&op.mrk_l[i][4 * q]) = Mrk.lo;
  }
}

// ---------------------------------------------------------------------------
// state side: one chunk for the columns [16w, 16w+16) held in S
// ---------------------------------------------------------------------------
template <class Io, bool kVExact>
__device__ __forceinline__ void state_chunk(const ChunkOps<kVExact>& op, f32x4 (&S)[4],
                                            uint16_t (*yrows)[D], int vcol, int i, int q,
                                            float scale) {
  using raw = typename Io::raw;
  // all operand reads of the chunk first, so that their LDS latency overlaps
  const Sp4 Ta = load_a16(op.t_h, op.t_l, i, q);
  const Sp4 Mak = load_a16(op.mak_h, op.mak_l, i, q);
  const Sp4 Mrb = load_a16(op.mrb_h, op.mrb_l, i, q);
  const Sp4 Mrk = load_a16(op.mrk_h, op.mrk_l, i, q);
  Sp4 Vb;
  Vb.hi = *reinterpret_cast<const bf16x4*>(&op.vT_h[vcol][4 * q]);   // V[4q+e][vcol]
  if constexpr (!kVExact) Vb.lo = *reinterpret_cast<const bf16x4*>(&op.vT_l[vcol][4 * q]);
  const Sp8 Aa0 = rows_vs_state(op.at_h, op.at_l, 0, i, q);
  const Sp8 Aa1 = rows_vs_state(op.at_h, op.at_l, 1, i, q);
  const Sp8 Ra0 = rows_vs_state(op.r_h, op.r_l, 0, i, q);
  const Sp8 Ra1 = rows_vs_state(op.r_h, op.r_l, 1, i, q);
  Sp4 Bt[4], Kt[4];
  f32x4 gl[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    Bt[kb] = load_a16(op.bT_h, op.bT_l, kb * 16 + i, q);
    Kt[kb] = load_a16(op.kT_h, op.kT_l, kb * 16 + i, q);
    gl[kb] = *reinterpret_cast<const f32x4*>(&op.gl[kb * 16 + 4 * q]);
  }
  Sp8 Sb[2];
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const Sp4 lo = split4(S[2 * m]);
    const Sp4 hi = split4(S[2 * m + 1]);
    Sb[m].hi = cat4(lo.hi, hi.hi);
    Sb[m].lo = cat4(lo.lo, hi.lo);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  // X = A~ S0 + Mak V,  U = T X,  Y = R~ S0 + Mrb U + Mrk V
  f32x4 X = kVExact ? mma16x2p(Mak, Vb.hi, zero) : mma16x3p(Mak, Vb, zero);
  X = mma32x3(Aa0, Sb[0], X);
  X = mma32x3(Aa1, Sb[1], X);
  f32x4 Y = kVExact ? mma16x2p(Mrk, Vb.hi, zero) : mma16x3p(Mrk, Vb, zero);
  Y = mma32x3(Ra0, Sb[0], Y);
  Y = mma32x3(Ra1, Sb[1], Y);
  const f32x4 U = mma16x3p(Ta, split4(X), zero);
  const Sp4 Us = split4(U);
  Y = mma16x3p(Mrb, Us, Y);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const raw yv = Io::from_f32(scale * Y[e]);
    yrows[4 * q + e][vcol] = __builtin_bit_cast(uint16_t, yv);
  }
  // S += B^^T U + K^^T V: five (bf16 V) or six (fp16 V) K = 16 terms in
  // three K = 32 products
  const bf16x4 z = {};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    f32x4 acc = S[kb];
    acc = mma2(Bt[kb].hi, Bt[kb].lo, Us.lo, Us.hi, acc);
    acc = mma2(Bt[kb].hi, Kt[kb].hi, Us.hi, Vb.hi, acc);
    acc = kVExact ? mma2(Kt[kb].lo, z, Vb.hi, z, acc) : mma2(Kt[kb].lo, Kt[kb].hi, Vb.hi, Vb.lo, acc);
    S[kb] = acc * gl[kb];
  }
}

template <class Io>
__global__ __launch_bounds__(NT) void chunk64_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr bool kVExact = !__is_same(Io, IoF16);
  __shared__ Smem<kVExact> sm;

  const int h = blockIdx.x;
  const int seg = blockIdx.y;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int i = lane & 15;
  const int q = lane >> 4;
  const int H = p.num_heads;

  if (p.status != nullptr) {
    if (p.status[0] != 0) {
      fill_output_nan<Io>(static_cast<raw*>(p.y), p.out_elems,
                          static_cast<int64_t>(seg) * gridDim.x + h,
                          static_cast<int64_t>(gridDim.x) * gridDim.y);
      return;
    }
    if (seg >= p.status[2]) return;
  }
  int t0, t1;
  if (p.uniform_len > 0) {
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
  const int slot = p.slots ? p.slots[seg] : seg;
  const int64_t head_off = static_cast<int64_t>(h) * D;
  const int64_t row_stride = static_cast<int64_t>(H) * D;
  const int ngroups = (t1 - t0 + GT - 1) / GT;
  raw* yout = static_cast<raw*>(p.y);

  if (wv < 4) {
    // ---------------- state waves: columns [16wv, 16wv+16)
    const int vcol = 16 * wv + i;
    const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
    f32x4 S[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (p.state_in != nullptr) {
      const float* sin = static_cast<const float*>(p.state_in);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) S[kb][e] = sin[sbase + (kb * 16 + 4 * q + e) * D + vcol];
    }
    __syncthreads();  // prologue: operators of group 0 (part 1)
    __syncthreads();  // prologue: operators of group 0 (part 2)
    auto group = [&](auto par_c, int gi) {
      constexpr int par = decltype(par_c)::value;
      const int g0 = t0 + gi * GT;
      state_chunk<Io, kVExact>(sm.ops[par][0], S, &sm.yb[par][0], vcol, i, q, p.scale);
      __syncthreads();
      if (g0 + L < t1)
        state_chunk<Io, kVExact>(sm.ops[par][1], S, &sm.yb[par][L], vcol, i, q, p.scale);
      __syncthreads();
    };
    for (int gi = 0; gi < ngroups; gi += 2) {
      group(std::integral_constant<int, 0>{}, gi);
      if (gi + 1 < ngroups) group(std::integral_constant<int, 1>{}, gi + 1);
    }
    if (p.state_out != nullptr) {
      float* sout = static_cast<float*>(p.state_out);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) sout[sbase + (kb * 16 + 4 * q + e) * D + vcol] = S[kb][e];
    }
  } else {
    // ---------------- key waves: chunk cc of the group, key half hh
    const int kw = wv & 3;
    const int cc = kw >> 1;
    const int hh = kw & 1;
    const int kbase = 32 * hh + 8 * q;
    float bias8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      bias8[e] = p.bias ? Io::to_f32(static_cast<const raw*>(p.bias)[head_off + kbase + e]) : 0.f;
    // token rows of this lane (token i of chunk cc, keys kbase..+7), as
    // running pointers; the group stride is GT rows
    const int tok0 = t0 + cc * L + i;
    const raw* src[6];
    {
      const int64_t off = static_cast<int64_t>(tok0) * row_stride + head_off + kbase;
      src[0] = static_cast<const raw*>(p.r) + off;
      src[1] = static_cast<const raw*>(p.logits) + off;
      src[2] = static_cast<const raw*>(p.k) + off;
      src[3] = static_cast<const raw*>(p.v) + off;
      src[4] = static_cast<const raw*>(p.a) + off;
      src[5] = static_cast<const raw*>(p.b) + off;
    }
    const int64_t gstride = static_cast<int64_t>(GT) * row_stride;
    const u32x4 zero4 = {0u, 0u, 0u, 0u};
    auto load_rows = [&](u32x4 (&dst)[6], int gi) {
      const bool ok = tok0 + gi * GT < t1;
      const int64_t off = static_cast<int64_t>(gi) * gstride;
#pragma unroll
      for (int j = 0; j < 6; ++j)
        dst[j] = ok ? *reinterpret_cast<const u32x4*>(src[j] + off) : zero4;
    };
    // output rows of a finished group: 16-byte pieces, token kt/8, elements 8*(kt%8)..
    const int kt = tid - 256;
    const int o_tok = kt >> 3, o_c8 = kt & 7;
    raw* const ybase = yout + static_cast<int64_t>(t0 + o_tok) * row_stride + head_off + o_c8 * 8;
    auto write_out = [&](int gi, int par) {
      if (t0 + gi * GT + o_tok < t1)
        *reinterpret_cast<u32x4*>(ybase + static_cast<int64_t>(gi) * gstride) =
            *reinterpret_cast<const u32x4*>(&sm.yb[par][o_tok][o_c8 * 8]);
    };
    u32x4 rawA[6], rawB[6];
    KeyRegs kr;
    load_rows(rawA, 0);
    if (ngroups > 1) load_rows(rawB, 1);
    // prologue: group 0 from rawA
    {
      const bool active = cc * L < t1 - t0;
      if (active)
        key_part1<Io, kVExact>(sm, sm.ops[0][cc], rawA, bias8, tok0 < t1, cc, hh, i, q, kr);
      __syncthreads();
      if (active) key_part2(sm, sm.ops[0][cc], cc, hh, i, q, kr);
      __syncthreads();
    }
    // iteration gi prepares group gn = gi + 1 (parity of gn) from the rows
    // prefetched one group ahead, and writes out the outputs of group gi - 1
    auto iter = [&](auto par_c, u32x4 (&cur)[6], u32x4 (&nxt)[6], int gi) {
      constexpr int par = decltype(par_c)::value;   // parity of gn
      const int gn = gi + 1;
      const bool active = gn < ngroups && t0 + gn * GT + cc * L < t1;
      if (gn + 1 < ngroups) load_rows(cur, gn + 1);   // cur was consumed last time
      if (gi > 0) write_out(gi - 1, par);             // parity of gi - 1 == parity of gn
      if (active)
        key_part1<Io, kVExact>(sm, sm.ops[par][cc], nxt, bias8, tok0 + gn * GT < t1, cc, hh,
                               i, q, kr);
      __syncthreads();
      if (active) key_part2(sm, sm.ops[par][cc], cc, hh, i, q, kr);
      __syncthreads();
    };
    // rawA holds group 0 (consumed), rawB group 1; alternate the two buffers
    for (int gi = 0; gi < ngroups; gi += 2) {
      iter(std::integral_constant<int, 1>{}, rawA, rawB, gi);
      if (gi + 1 < ngroups) iter(std::integral_constant<int, 0>{}, rawB, rawA, gi + 1);
    }
    if (ngroups > 0) write_out(ngroups - 1, (ngroups - 1) & 1);
  }
}

}  // namespace

int launch_chunked(int dtype, const SegArgs& p, int nseg, int max_seqlen, hipStream_t s) {
  (void)max_seqlen;
  if (p.sa_out != nullptr || p.boundary != nullptr) return FR2_ERR_UNSUPPORTED;
  const dim3 grid(p.num_heads, nseg);
  if (dtype == FR2_DTYPE_BFLOAT16)
    hipLaunchKernelGGL((chunk64_kernel<IoBF16>), grid, dim3(NT), 0, s, p);
  else if (dtype == FR2_DTYPE_FLOAT16)
    hipLaunchKernelGGL((chunk64_kernel<IoF16>), grid, dim3(NT), 0, s, p);
  else
    return FR2_ERR_UNSUPPORTED;
  return record_launch();
}

}  // namespace fr2
