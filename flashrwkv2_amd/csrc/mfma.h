// gfx950 matrix-core helpers shared by the chunked WKV7 kernels: bf16 hi/lo
// split operands on v_mfma_f32_16x16x32_bf16, accumulator / operand layout
// conversions, DPP row scans over the 16-lane token axis and the LDS
// transpose read.
//
// v_mfma_f32_16x16x32_bf16 layouts (lane l, group q = l/16):
//   A[i][k]: lane i + 16 (k/8), 8 consecutive k per lane;
//   B[k][j]: lane j + 16 (k/8);
//   D[i][j]: lane j + 16 (i/4), item i%4.
#pragma once

#include "common.h"

namespace fr2 {
namespace {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef __bf16 bf16x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Two fp32 values rounded (nearest-even) to bf16 and packed: v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16(float x0, float x1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{x0, x1}, bf16x2));
}
// hi/lo split of two values: hi = bf16(x), lo = bf16(x - hi), packed pairs.
// The residuals x - hi come from v_dot2c_f32_bf16 against the packed pairs
// (-1, 0) and (0, -1): x + (-1) hi + 0 = x - hi, which is exact in fp32 (hi
// is x rounded to 8 significant bits), so no intermediate rounding occurs.
// Two VALU instructions per value (two conversions and two dot products per
// pair) instead of three with an explicit widening of hi.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  // the selector pairs are passed in scalar registers
  uint32_t m0 = 0x0000bf80u, m1 = 0xbf800000u;
  asm("" : "+s"(m0), "+s"(m1));
  const bf16x2 h = __builtin_bit_cast(bf16x2, pack_bf16(x0, x1));
  const float r0 = __builtin_amdgcn_fdot2_f32_bf16(h, __builtin_bit_cast(bf16x2, m0), x0, false);
  const float r1 = __builtin_amdgcn_fdot2_f32_bf16(h, __builtin_bit_cast(bf16x2, m1), x1, false);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = pack_bf16(r0, r1);
}

struct Sp8 { bf16x8 hi, lo; };

// split of eight values (a 16-byte hi vector and a 16-byte lo vector)
__device__ __forceinline__ Sp8 split8(const float* x) {
  u32x4 h, l;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t hj, lj;
    split2(x[2 * j], x[2 * j + 1], hj, lj);
    h[j] = hj;
    l[j] = lj;
  }
  return Sp8{__builtin_bit_cast(bf16x8, h), __builtin_bit_cast(bf16x8, l)};
}

__device__ __forceinline__ f32x4 mma32x3(const Sp8& a, const Sp8& b, f32x4 c) {
  c = mma32(a.lo, b.hi, c);
  c = mma32(a.hi, b.lo, c);
  return mma32(a.hi, b.hi, c);
}

// K = 16 products on the K = 32 instruction.  Lane group q supplies K
// positions 8q..8q+7 = (first half's 4q..4q+3, second half's 4q..4q+3), so
// [x | y] x [u ; v] = x u + y v.  Operand forms:
//   AOp  (A side, split):   [hi | lo]                      one bf16x8
//   BOp  (B side, split):   [lo | hi | 0 | 0], read through the windows
//                           [lo | hi] and [hi | 0]
//   BX   (B side, exact):   [v | v]
// so  AOp x BOp = hi.lo + lo.hi, then hi.hi + lo.0  (two instructions) and
//     AOp x BX  = hi.v + lo.v                        (one instruction).
// Every product of the kernel runs on the one K = 32 opcode: with this
// toolchain an accumulator produced by v_mfma_f32_16x16x32_bf16 and consumed
// as src C by v_mfma_f32_16x16x16_bf16 gave wrong sums on gfx950.
typedef bf16x8 AOp;
typedef bf16x16 BOp;
typedef bf16x8 BX;

__device__ __forceinline__ f32x4 mm_ab(AOp a, BOp b, f32x4 c) {
  c = mma32(a, __builtin_shufflevector(b, b, 0, 1, 2, 3, 4, 5, 6, 7), c);
  return mma32(a, __builtin_shufflevector(b, b, 4, 5, 6, 7, 8, 9, 10, 11), c);
}
__device__ __forceinline__ f32x4 mm_ax(AOp a, BX b, f32x4 c) { return mma32(a, b, c); }

// 16x16 matrices held in accumulator layout (lane l: column l%16, rows
// 4(l/16)+e): the accumulator layout of X^T is the A-operand layout of X and
// the accumulator layout of Y is the B-operand layout of Y.
struct Split4 { uint32_t h0, h1, l0, l1; };
__device__ __forceinline__ Split4 split4(f32x4 x) {
  Split4 s;
  split2(x[0], x[1], s.h0, s.l0);
  split2(x[2], x[3], s.h1, s.l1);
  return s;
}
__device__ __forceinline__ AOp as_a(const Split4& s) {
  return __builtin_bit_cast(AOp, u32x4{s.h0, s.h1, s.l0, s.l1});
}
__device__ __forceinline__ BOp as_b(const Split4& s) {
  typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
  return __builtin_bit_cast(BOp, u32x8{s.l0, s.l1, s.h0, s.h1, 0u, 0u, 0u, 0u});
}
__device__ __forceinline__ BX as_bx(bf16x4 v) { return __builtin_shufflevector(v, v, 0, 1, 2, 3, 0, 1, 2, 3); }
__device__ __forceinline__ BOp as_b(bf16x4 hi, bf16x4 lo) {
  const bf16x4 z = {};
  return __builtin_shufflevector(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7),
                                 __builtin_shufflevector(z, z, 0, 1, 2, 3, 4, 5, 6, 7), 0, 1, 2,
                                 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

// T = (I - M)^-1 for a strictly lower triangular 16x16 M, given in both
// accumulator orientations (lane (i, q): M[e] = M[4q+e][i], Mt[e] =
// M[i][4q+e]).  Returns the A operand of T.
//
// Blocked over the four 4x4 diagonal blocks: with MD the block-diagonal part
// of M and MO the rest (strictly block-lower),
//   D = (I - MD)^-1 = (I + MD)(I + MD^2)             (4x4 blocks: MD^4 = 0)
//   I - M = (I - MD)(I - N),  N = D MO               (strictly block-lower)
//   T = (I - N)^-1 D = (I + N)(I + N^2) D            (N^4 = 0)
// Every intermediate is a product of at most three factors of bounded size,
// so the sums stay of the order of T itself.  The doubling form
// (I+M)(I+M^2)(I+M^4)(I+M^8) over the whole block builds M^8, whose entries
// are sums over up to C(15, 8) paths: with strongly correlated keys and an
// in-context rate near 1 (Mab close to a constant below the diagonal) they
// reach 10^3 while T stays of order 1, and the cancellation lost the output
// gate even with split operands.
// Products X Y are mm_ab(A form of X = split of acc(X^T), B form of Y = split
// of acc(Y)); each needed orientation is formed as its own product.
__device__ __forceinline__ AOp t_inverse(f32x4 M, f32x4 Mt, int i, int q) {
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 I4;
#pragma unroll
  for (int e = 0; e < 4; ++e) I4[e] = (4 * q + e == i) ? 1.0f : 0.0f;
  // rows 4q..4q+3 and column i (or the transpose) lie in one diagonal block
  // exactly when q == i / 4, for all four items of the lane
  const bool diag = q == (i >> 2);
  const f32x4 MD = diag ? M : zero, MDt = diag ? Mt : zero, MO = diag ? zero : M;
  const f32x4 MD2 = mm_ab(as_a(split4(MDt)), as_b(split4(MD)), zero);   // MD^2
  const f32x4 E = I4 + MD, Et = I4 + MDt;                               // I + MD, (I + MD)^T
  const Split4 sMD2 = split4(MD2), sEt = split4(Et);
  const f32x4 Dm = mm_ab(as_a(sEt), as_b(sMD2), E);     // D = (I + MD) + (I + MD) MD^2
  const f32x4 Dt = mm_ab(as_a(sMD2), as_b(sEt), Et);    // D^T
  const Split4 sD = split4(Dm), sDt = split4(Dt), sMO = split4(MO);
  const f32x4 N = mm_ab(as_a(sDt), as_b(sMO), zero);    // N = D MO
  const f32x4 Nt = mm_ab(as_a(sMO), as_b(sDt), zero);   // N^T = MO^T D^T
  const f32x4 N2 = mm_ab(as_a(split4(Nt)), as_b(split4(N)), zero);     // N^2
  const f32x4 Ft = I4 + Nt;                                             // (I + N)^T
  // (I + N)(I + N^2) = (I + N) + (I + N) N^2, transposed
  const f32x4 Tpt = mm_ab(as_a(split4(N2)), as_b(split4(Ft)), Ft);
  const f32x4 Tt = mm_ab(as_a(sD), as_b(split4(Tpt)), zero);            // T^T = D^T Tp^T
  return as_a(split4(Tt));                                              // = A operand of T
}

// LDS row swizzles of the chunk operators: the 16-byte pieces of a row are
// permuted by an XOR with bits of the row index, so that the lanes of one
// LDS access spread over the banks.  Each was chosen from bank-conflict
// counter readings (SQ_LDS_BANK_CONFLICT) of its array's access patterns on
// gfx950.  Columns are in bf16 units; an access never crosses a piece.
//   a_col: the A~ / R~ rows (128 bytes), piece XOR row & 7: the 16-byte
//     reads against the state conflict-free, the 8-byte operand stores at
//     half the unswizzled excess;
//   b_col: the B^ / K^ / V token rows (160 bytes), piece XOR (row >> 2) & 3:
//     the 16-byte row stores and the transposed 8-byte reads conflict-free;
//   aop_piece: the 16 x 16 token-token blocks (64-byte rows), piece XOR
//     (row >> 1) & 3: their 16-byte stores and reads conflict-free.
__device__ __forceinline__ int a_col(int row, int col) {
  return (((col >> 3) ^ (row & 7)) << 3) | (col & 7);
}
__device__ __forceinline__ int b_col(int row, int col) {
  return (((col >> 3) ^ ((row >> 2) & 3)) << 3) | (col & 7);
}
__device__ __forceinline__ int aop_piece(int i, int q) { return q ^ ((i >> 1) & 3); }

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
// x of the previous token in the DPP row; `first` for token 0
__device__ __forceinline__ float row_prev(float x, float first) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(first), __float_as_int(x),
                                                    0x111, 0xf, 0xf, false));
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

// LDS transpose read (ds_read_b64_tr_b16): within each 16-lane group G, lane
// g receives item e = element g%4 of the 8-byte piece addressed by lane
// 4e + g/4 of its group.  With lane g of group q addressing
// &X[4q + g/4][c0 + 4(g%4)] of a row-major [token][column] array, lane g
// receives X[4q+e][c0+g]: the K = 16 A-operand layout of X^T (row c0+g,
// K = token), or equally the B-operand layout of X (K = token, column c0+g).
__device__ __forceinline__ bf16x4 tr_rows(const __bf16* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  lds_s16x4* lp = (lds_s16x4*)(p);
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(lp));
}


}  // namespace
}  // namespace fr2
