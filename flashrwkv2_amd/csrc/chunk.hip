// Chunked WKV7 prefill on gfx950 matrix cores (D = 64, fp32 state carry).
//
// Chunk algebra (L = 16 tokens, rows = tokens, S0 = start-of-chunk state,
// g_t = sum_{s<=t} log w_s inside the chunk, gamma_t = exp(g_t)):
//   A~ = a*gamma_{t-1}, R~ = r*gamma_t, B^ = b/gamma_t, K^ = k/gamma_t
//   Mab = strict_tril(A~ B^T), Mak = strict_tril(A~ K^T)
//   Mrb = tril(R~ B^T),        Mrk = tril(R~ K^T)
//   T = (I - Mab)^-1,  W = T A~,  Z = T (Mak V)
//   U (the per-token sa rows) = W S0 + Z
//   Y = R~ S0 + Mrb U + Mrk V                     (y = scale * Y)
//   S_L = diag(gamma_L) (S0 + B^^T U + K^^T V)
// which is the per-token recurrence
//   sa_t = S_{t-1}^T a_t, S_t = diag(w_t) S_{t-1} + b_t sa_t^T + k_t v_t^T,
//   y_t = scale * S_t^T r_t
// unrolled over the chunk.  Every product runs on
// v_mfma_f32_16x16x{16,32}_bf16 with both operands split into bf16 hi + lo
// (hi*hi + hi*lo + lo*hi, fp32 accumulation): fp32-level accuracy.  Raw bf16
// token values (V) are exact and carry no lo part.
//
// Work layout: one 512-thread workgroup (8 wavefronts) per (sequence, head),
// walking the sequence in groups of 4 chunks (64 tokens):
//   phase A (all 8 waves, one (chunk, key-half) each): decays by a 16-lane DPP
//     scan over tokens, operands built in registers, the four token-token
//     blocks computed from those registers (each lane's 8 keys are its own MFMA
//     K positions), then T by repeated squaring (I+M)(I+M^2)(I+M^4)(I+M^8)
//     with both orientations of every factor in registers, and W = T A~;
//   phase B (waves 0-3, state columns [16w, 16w+16) each): the state path for
//     the 4 chunks in order.  The state never leaves fp32 accumulator
//     registers: accumulator rows are fed to the matrix cores as B-operand K
//     positions directly (the K order of a dot product is free), and the
//     accumulator layout of U is already the B-operand layout of B^^T U.
// The next group's token rows are prefetched into registers during the
// iteration and staged in LDS at its end.
#include "recurrent.h"

namespace fr2 {
namespace {

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int D = 64;
constexpr int L = 16;          // tokens per chunk
constexpr int G = 4;           // chunks per group
constexpr int GT = L * G;      // tokens per group
constexpr int NT = 512;        // 8 wavefronts
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegExpHalf = -0.6065306597126334f;   // -exp(-1/2)

__device__ __forceinline__ f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct Sp4 { bf16x4 hi, lo; };
struct Sp8 { bf16x8 hi, lo; };

__device__ __forceinline__ Sp4 split4(f32x4 x) {
  Sp4 s;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const __bf16 h = static_cast<__bf16>(x[e]);
    s.hi[e] = h;
    s.lo[e] = static_cast<__bf16>(x[e] - static_cast<float>(h));
  }
  return s;
}
__device__ __forceinline__ Sp8 split8(const float* x) {
  Sp8 s;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = static_cast<__bf16>(x[e]);
    s.hi[e] = h;
    s.lo[e] = static_cast<__bf16>(x[e] - static_cast<float>(h));
  }
  return s;
}

__device__ __forceinline__ f32x4 mma16x3(Sp4 a, Sp4 b, f32x4 c) {
  c = mma16(a.lo, b.hi, c);
  c = mma16(a.hi, b.lo, c);
  return mma16(a.hi, b.hi, c);
}
__device__ __forceinline__ f32x4 mma16x2(Sp4 a, bf16x4 b, f32x4 c) {
  c = mma16(a.lo, b, c);
  return mma16(a.hi, b, c);
}
__device__ __forceinline__ f32x4 mma32x3(const Sp8& a, const Sp8& b, f32x4 c) {
  c = mma32(a.lo, b.hi, c);
  c = mma32(a.hi, b.lo, c);
  return mma32(a.hi, b.hi, c);
}

// X Y for 16x16 matrices held in accumulator layout (lane l: column l%16,
// rows 4(l/16)+e): the accumulator layout of X^T is the A-operand layout of X
// and the accumulator layout of Y is the B-operand layout of Y.
__device__ __forceinline__ f32x4 mm(f32x4 xt, f32x4 y, f32x4 c) {
  return mma16x3(split4(xt), split4(y), c);
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

// Operators of one chunk consumed by the state path.
constexpr int RP = D + 8;          // padded row (bank spread)

// Column position of key k in the W / R~ rows: for each half m = k/32 the 32
// keys are ordered so that lane group q of the state product reads its 8 keys
// (the rows its state accumulators hold) as one contiguous 16-byte run.
__device__ __forceinline__ int key_pos(int k) {
  const int m = k >> 5, kk = k & 31;
  return 32 * m + 8 * ((kk & 15) >> 2) + 4 * (kk >> 4) + (kk & 3);
}

struct alignas(16) ChunkOps {
  __bf16 w_h[L][RP], w_l[L][RP];    // W rows, keys at key_pos()
  __bf16 r_h[L][RP], r_l[L][RP];    // R~ rows, keys at key_pos()
  __bf16 bT_h[D][L], bT_l[D][L];    // B^ transposed
  __bf16 kT_h[D][L], kT_l[D][L];    // K^ transposed
  __bf16 vT_h[D][L], vT_l[D][L];    // V transposed (lo = 0 for bf16 tokens)
  __bf16 t_h[L][L], t_l[L][L];      // T
  __bf16 mak_h[L][L], mak_l[L][L];  // Mak, Mrb, Mrk (masked)
  __bf16 mrb_h[L][L], mrb_l[L][L];
  __bf16 mrk_h[L][L], mrk_l[L][L];
  float gl[D];                      // gamma_L
};

struct alignas(16) Scratch {
  float mpart[G][2][4][L][L];       // [chunk][key half][block][t][s]
  __bf16 atT_h[G][D][L], atT_l[G][D][L];
};

struct alignas(16) Smem {
  union {
    uint16_t raw[6][GT][D];         // staged token rows of the group
    Scratch s;
  } u;
  ChunkOps ops[G];
  uint16_t yb[GT][D];               // the group's outputs, written out as full rows
};
static_assert(sizeof(Scratch) <= sizeof(uint16_t) * 6 * GT * D, "scratch alias");

// A operand against the state: row t = lane%16 of X; positions 8q+idx map to
// key (2m + idx/4)*16 + 4q + idx%4, i.e. the rows the lane's state
// accumulators hold.
__device__ __forceinline__ Sp8 rows_vs_state(const __bf16 (*xh)[RP], const __bf16 (*xl)[RP],
                                             int m, int i, int q) {
  Sp8 s;
  s.hi = *reinterpret_cast<const bf16x8*>(&xh[i][32 * m + 8 * q]);
  s.lo = *reinterpret_cast<const bf16x8*>(&xl[i][32 * m + 8 * q]);
  return s;
}

__device__ __forceinline__ Sp4 load_a16(const __bf16 (*h)[L], const __bf16 (*l)[L], int row,
                                        int q) {
  Sp4 s;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    s.hi[e] = h[row][4 * q + e];
    s.lo[e] = l[row][4 * q + e];
  }
  return s;
}

template <class Io>
__global__ __launch_bounds__(NT) void chunk64_kernel(SegArgs p) {
  using raw = typename Io::raw;
  constexpr bool kVExact = !__is_same(Io, IoF16);
  __shared__ Smem sm;

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

  // phase-A role: chunk cc of the group, key half hh, keys 32hh + 8q + e
  const int cc = wv >> 1;
  const int hh = wv & 1;
  const int kbase = 32 * hh + 8 * q;
  float bias8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    bias8[e] = p.bias ? Io::to_f32(static_cast<const raw*>(p.bias)[head_off + kbase + e]) : 0.f;

  // phase-B role (waves 0-3): state columns [16wv, 16wv+16)
  const bool state_wave = wv < 4;
  const int vcol = 16 * wv + i;
  const int64_t sbase = (static_cast<int64_t>(slot) * H + h) * D * D;
  f32x4 S[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) S[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (state_wave && p.state_in != nullptr) {
    const float* sin = static_cast<const float*>(p.state_in);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) S[kb][e] = sin[sbase + (kb * 16 + 4 * q + e) * D + vcol];
  }

  const raw* const srcs[6] = {
      static_cast<const raw*>(p.r), static_cast<const raw*>(p.logits),
      static_cast<const raw*>(p.k), static_cast<const raw*>(p.v),
      static_cast<const raw*>(p.a), static_cast<const raw*>(p.b)};
  raw* yout = static_cast<raw*>(p.y);

  // staging: thread loads, for each of the 6 inputs, token tid/8 of the group,
  // elements 8*(tid%8)..+7
  const int st_tok = tid >> 3;
  const int st_c8 = tid & 7;
  u32x4 pf0, pf1, pf2, pf3, pf4, pf5;
  const u32x4 zero4 = {0u, 0u, 0u, 0u};
#define FR2_ISSUE_LOADS(G0)                                                              \
  {                                                                                       \
    const bool ok_ = (G0) + st_tok < t1;                                                  \
    const int64_t off_ =                                                                  \
        static_cast<int64_t>((G0) + st_tok) * row_stride + head_off + st_c8 * 8;          \
    pf0 = ok_ ? *reinterpret_cast<const u32x4*>(srcs[0] + off_) : zero4;                  \
    pf1 = ok_ ? *reinterpret_cast<const u32x4*>(srcs[1] + off_) : zero4;                  \
    pf2 = ok_ ? *reinterpret_cast<const u32x4*>(srcs[2] + off_) : zero4;                  \
    pf3 = ok_ ? *reinterpret_cast<const u32x4*>(srcs[3] + off_) : zero4;                  \
    pf4 = ok_ ? *reinterpret_cast<const u32x4*>(srcs[4] + off_) : zero4;                  \
    pf5 = ok_ ? *reinterpret_cast<const u32x4*>(srcs[5] + off_) : zero4;                  \
  }
#define FR2_STAGE_LOADS()                                                \
  {                                                                      \
    *reinterpret_cast<u32x4*>(&sm.u.raw[0][st_tok][st_c8 * 8]) = pf0;     \
    *reinterpret_cast<u32x4*>(&sm.u.raw[1][st_tok][st_c8 * 8]) = pf1;     \
    *reinterpret_cast<u32x4*>(&sm.u.raw[2][st_tok][st_c8 * 8]) = pf2;     \
    *reinterpret_cast<u32x4*>(&sm.u.raw[3][st_tok][st_c8 * 8]) = pf3;     \
    *reinterpret_cast<u32x4*>(&sm.u.raw[4][st_tok][st_c8 * 8]) = pf4;     \
    *reinterpret_cast<u32x4*>(&sm.u.raw[5][st_tok][st_c8 * 8]) = pf5;     \
  }

  FR2_ISSUE_LOADS(t0);
  FR2_STAGE_LOADS();
  __syncthreads();

  // outputs of a finished group: 16-byte row pieces, token tid/8, elements 8*(tid%8)..
#define FR2_WRITE_OUTPUTS(G0)                                                          \
  {                                                                                     \
    if ((G0) + st_tok < t1)                                                             \
      *reinterpret_cast<u32x4*>(yout + static_cast<int64_t>((G0) + st_tok) * row_stride + \
                                head_off + st_c8 * 8) =                                 \
          *reinterpret_cast<const u32x4*>(&sm.yb[st_tok][st_c8 * 8]);                   \
  }

  for (int g0 = t0; g0 < t1; g0 += GT) {
    const int ng = min(GT, t1 - g0);
    const int nchunks = (ng + L - 1) / L;
    if (g0 + GT < t1) FR2_ISSUE_LOADS(g0 + GT);
    if (g0 > t0) FR2_WRITE_OUTPUTS(g0 - GT);

    // ---------------- phase A1: token rows -> operands, token-token blocks
    const bool a_active = cc < nchunks;
    const int tok = cc * L + i;                 // token of this lane in the group
    const bool valid = tok < ng;
    float xr[8], xk[8], xv[8], xa[8], xb[8], lw[8];
    if (a_active) {
      float xl[8];
      unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.u.raw[0][tok][kbase]), xr);
      unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.u.raw[1][tok][kbase]), xl);
      unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.u.raw[2][tok][kbase]), xk);
      unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.u.raw[3][tok][kbase]), xv);
      unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.u.raw[4][tok][kbase]), xa);
      unpack8<Io>(*reinterpret_cast<const u32x4*>(&sm.u.raw[5][tok][kbase]), xb);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = xl[e] + bias8[e];
        const float sig = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLog2e * x));
        lw[e] = valid ? kNegExpHalf * sig : 0.0f;
      }
    }
    __syncthreads();   // token rows consumed; the staging area becomes scratch

    if (a_active) {
      float at[8], rt[8], bh[8], kh[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float g = row_scan(lw[e]);
        const float gm = fast_exp(g);
        const float gp = fast_exp(g - lw[e]);
        const float ig = fast_exp(-g);
        at[e] = xa[e] * gp;
        rt[e] = xr[e] * gm;
        bh[e] = xb[e] * ig;
        kh[e] = xk[e] * ig;
        if (i == L - 1) sm.ops[cc].gl[kbase + e] = gm;
      }
      const Sp8 As = split8(at), Rs = split8(rt), Bs = split8(bh), Ks = split8(kh);
      ChunkOps& op = sm.ops[cc];
      {
        // keys kbase..kbase+7 land in two 4-key runs of the permuted row
        const int p0 = key_pos(kbase), p1 = key_pos(kbase + 4);
        *reinterpret_cast<bf16x4*>(&op.r_h[i][p0]) = Rs.hi.lo;
        *reinterpret_cast<bf16x4*>(&op.r_h[i][p1]) = Rs.hi.hi;
        *reinterpret_cast<bf16x4*>(&op.r_l[i][p0]) = Rs.lo.lo;
        *reinterpret_cast<bf16x4*>(&op.r_l[i][p1]) = Rs.lo.hi;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = kbase + e;
        op.bT_h[k][i] = Bs.hi[e];
        op.bT_l[k][i] = Bs.lo[e];
        op.kT_h[k][i] = Ks.hi[e];
        op.kT_l[k][i] = Ks.lo[e];
        const __bf16 vh = static_cast<__bf16>(xv[e]);
        op.vT_h[k][i] = vh;
        op.vT_l[k][i] = static_cast<__bf16>(xv[e] - static_cast<float>(vh));
        sm.u.s.atT_h[cc][k][i] = As.hi[e];
        sm.u.s.atT_l[cc][k][i] = As.lo[e];
      }
      // partial token-token blocks over this lane's 8 keys per row group
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 pab = mma32x3(As, Bs, zero);
      const f32x4 pak = mma32x3(As, Ks, zero);
      const f32x4 prb = mma32x3(Rs, Bs, zero);
      const f32x4 prk = mma32x3(Rs, Ks, zero);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sm.u.s.mpart[cc][hh][0][4 * q + e][i] = pab[e];
        sm.u.s.mpart[cc][hh][1][4 * q + e][i] = pak[e];
        sm.u.s.mpart[cc][hh][2][4 * q + e][i] = prb[e];
        sm.u.s.mpart[cc][hh][3][4 * q + e][i] = prk[e];
      }
    }
    __syncthreads();

    // ---------------- phase A2: T, W (and the masked blocks for the state path)
    if (a_active) {
      const float (*mp0)[4][L][L] = sm.u.s.mpart[cc];
      f32x4 M, Mt, I4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * q + e;
        M[e] = (r > i) ? mp0[0][0][r][i] + mp0[1][0][r][i] : 0.f;
        Mt[e] = (i > r) ? mp0[0][0][i][r] + mp0[1][0][i][r] : 0.f;
        I4[e] = (r == i) ? 1.0f : 0.0f;
      }
      // T = (I - Mab)^-1 = (I+M)(I+M^2)(I+M^4)(I+M^8) (M strictly lower, 16x16),
      // keeping both orientations of each factor in accumulator registers.
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
      const f32x4 M2 = mm(Mt, M, zero);
      const f32x4 M2t = mm(M, Mt, zero);
      const f32x4 T2t = mm(M2, I4 + Mt, I4 + Mt);
      const f32x4 M4 = mm(M2t, M2, zero);
      const f32x4 M4t = mm(M2, M2t, zero);
      const f32x4 T4t = mm(M4, T2t, T2t);
      const f32x4 M8 = mm(M4t, M4, zero);
      const f32x4 Tt = mm(M8, T4t, T4t);     // accumulator of T^T = A operand of T
      const Sp4 Ta = split4(Tt);
      ChunkOps& op = sm.ops[cc];
      if (hh == 0) {
        f32x4 mak, mrb, mrk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int s = 4 * q + e;       // A-operand layout: row i, K = s
          mak[e] = (i > s) ? mp0[0][1][i][s] + mp0[1][1][i][s] : 0.f;
          mrb[e] = (i >= s) ? mp0[0][2][i][s] + mp0[1][2][i][s] : 0.f;
          mrk[e] = (i >= s) ? mp0[0][3][i][s] + mp0[1][3][i][s] : 0.f;
        }
        const Sp4 a1 = split4(mak), a2 = split4(mrb), a3 = split4(mrk);
        *reinterpret_cast<bf16x4*>(&op.t_h[i][4 * q]) = Ta.hi;
        *reinterpret_cast<bf16x4*>(&op.t_l[i][4 * q]) = Ta.lo;
        *reinterpret_cast<bf16x4*>(&op.mak_h[i][4 * q]) = a1.hi;
        *reinterpret_cast<bf16x4*>(&op.mak_l[i][4 * q]) = a1.lo;
        *reinterpret_cast<bf16x4*>(&op.mrb_h[i][4 * q]) = a2.hi;
        *reinterpret_cast<bf16x4*>(&op.mrb_l[i][4 * q]) = a2.lo;
        *reinterpret_cast<bf16x4*>(&op.mrk_h[i][4 * q]) = a3.hi;
        *reinterpret_cast<bf16x4*>(&op.mrk_l[i][4 * q]) = a3.lo;
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int kc = 32 * hh + 16 * j + i;
        const Sp4 Ab = load_a16(sm.u.s.atT_h[cc], sm.u.s.atT_l[cc], kc, q);
        const Sp4 Ws = split4(mma16x3(Ta, Ab, zero));   // W[4q+e][kc]
        const int pc = key_pos(kc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          op.w_h[4 * q + e][pc] = Ws.hi[e];
          op.w_l[4 * q + e][pc] = Ws.lo[e];
        }
      }
    }
    __syncthreads();

    // ---------------- phase B: state path, chunk by chunk
    if (state_wave) {
      for (int c = 0; c < nchunks; ++c) {
        const ChunkOps& op = sm.ops[c];
        // all operand reads of the chunk first, so that their LDS latency overlaps
        const Sp4 Ta = load_a16(op.t_h, op.t_l, i, q);
        const Sp4 Mak = load_a16(op.mak_h, op.mak_l, i, q);
        const Sp4 Mrb = load_a16(op.mrb_h, op.mrb_l, i, q);
        const Sp4 Mrk = load_a16(op.mrk_h, op.mrk_l, i, q);
        const Sp4 Vb = load_a16(op.vT_h, op.vT_l, vcol, q);   // V[4q+e][vcol]
        const Sp8 Wa0 = rows_vs_state(op.w_h, op.w_l, 0, i, q);
        const Sp8 Wa1 = rows_vs_state(op.w_h, op.w_l, 1, i, q);
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
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            Sb[m].hi[e] = lo.hi[e];
            Sb[m].hi[4 + e] = hi.hi[e];
            Sb[m].lo[e] = lo.lo[e];
            Sb[m].lo[4 + e] = hi.lo[e];
          }
        }
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        const f32x4 Zp = kVExact ? mma16x2(Mak, Vb.hi, zero) : mma16x3(Mak, Vb, zero);
        f32x4 Y = mma32x3(Ra0, Sb[0], zero);
        Y = mma32x3(Ra1, Sb[1], Y);
        f32x4 U = mma32x3(Wa0, Sb[0], zero);
        U = mma32x3(Wa1, Sb[1], U);
        U = mma16x3(Ta, split4(Zp), U);
        const Sp4 Us = split4(U);
        Y = mma16x3(Mrb, Us, Y);
        Y = kVExact ? mma16x2(Mrk, Vb.hi, Y) : mma16x3(Mrk, Vb, Y);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const raw yv = Io::from_f32(p.scale * Y[e]);
          sm.yb[c * L + 4 * q + e][vcol] = __builtin_bit_cast(uint16_t, yv);
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          S[kb] = mma16x3(Bt[kb], Us, S[kb]);
          S[kb] = kVExact ? mma16x2(Kt[kb], Vb.hi, S[kb]) : mma16x3(Kt[kb], Vb, S[kb]);
          S[kb] *= gl[kb];
        }
      }
    }
    if (g0 + GT < t1) FR2_STAGE_LOADS();   // staging/scratch is free after phase A2
    __syncthreads();
  }

  if (t1 > t0) FR2_WRITE_OUTPUTS(t0 + ((t1 - t0 - 1) / GT) * GT);
#undef FR2_ISSUE_LOADS
#undef FR2_STAGE_LOADS
#undef FR2_WRITE_OUTPUTS
  if (state_wave && p.state_out != nullptr) {
    float* sout = static_cast<float*>(p.state_out);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int e = 0; e < 4; ++e) sout[sbase + (kb * 16 + 4 * q + e) * D + vcol] = S[kb][e];
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
