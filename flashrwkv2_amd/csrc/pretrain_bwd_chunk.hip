// Key-row pass of the training backward in chunk form on the matrix cores
// (D = 64).  With the value pass done (dsa known, and P snapshots every
// kCps chunks), everything the key rows need inside a 16-token chunk is a
// product of the chunk's start state S0, the carried gradient Pc (dL/dS of
// the chunk's last token from the future) and 16x16 token blocks:
//
//   gamma_t = prod_{u<=t} w_u (per key row), gp_t = gamma_{t-1},
//   B^ = b/gamma, K^ = k/gamma, R^ = r gamma/gamma_15, A^ = a gp/gamma_15,
//   rho_t = gamma_15/gamma_t
//   dr = gamma o (S0 DY^T + B^^T [SA DY^T]_{s<=t} + K^^T [V DY^T]_{s<=t})
//   da = gp    o (S0 DSA^T + B^^T [SA DSA^T]_{s<t} + K^^T [V DSA^T]_{s<t})
//   dk = rho   o (Pc V^T + R^^T [DY V^T]_{s>=t} + A^^T [DSA V^T]_{s>t})
//   db = rho   o (Pc SA^T + R^^T [DY SA^T]_{s>=t} + A^^T [DSA SA^T]_{s>t})
//   carry to the previous chunk: Pc' = gamma_15 o (Pc + R^^T DY + A^_{s>0}^T DSA)
//                                      + a_0 dsa_0^T
//
// and dw needs no state product at all: with Z_t = rowsum(P_t o S_t),
//   w_t dw_t = Z_t - b_t db_t - k_t dk_t,
//   Z_{t-1}  = w_t dw_t + a_t da_t + r_{t-1} dr_{t-1},
//   Z_15     = r_15 dr_15 + gamma_15 (rowsum(Pc o S0) + sum_s B^_s (Pc SA^T)_s
//                                     + K^_s (Pc V^T)_s),
// a per-row scan over the chunk's tokens.  Nothing walks backwards through
// 1/w, so the pass does not depend on how the forward produced its
// snapshots.
//
// Work layout: one 256-thread workgroup per (batch, head, span of kCps
// chunks), walking its chunks backwards and carrying Pc in registers; it
// starts from the value pass's snapshot of P at the span's end.  Wave w owns
// key rows [16w, 16w+16).  Products over the 64 values use the K = 32
// instruction with both operands in one permuted value order (lane group q
// holds values 16vb+4q..16vb+4q+3 of every value block vb), the order in
// which the accumulator of Pc^T already lies, so the carry feeds the next
// chunk's products without a relayout.  Every fp32 operand is a bf16 hi/lo
// split (fp32-level accuracy); bf16 token values (dy, v) are exact.
#include "mfma.h"
#include "recurrent.h"

namespace fr2 {
namespace {

constexpr int kD = 64;
constexpr int kL = 16;
constexpr int kKNT = 256;
constexpr float kLg2e = 1.4426950408889634f;
constexpr float kNegEh = -0.6065306597126334f;   // -exp(-1/2)
constexpr float kCl = kNegEh * kLg2e;            // log2(w) = kCl * sigmoid(x)

struct KPassArgs {
  int T, H, nspan, cps;
  const uint16_t *r, *w, *k, *v, *a, *b, *dy;
  const float *sa, *dsa, *bnd, *pbnd;
  uint16_t *dr, *dw, *dk, *db, *da;
  // StateTune: y = scale * S^T r, the start state of chunk 0 (sequence b at
  // state0 + b * state0_stride, [H,D,D]; null: zero) and dL/dS_final
  // ([B,H,D,D]; null: zero)
  float scale;
  const float* state0;
  int64_t state0_stride;
  const float* dfinal;
};

// LDS row pitches chosen against bank conflicts (64 banks of 4 bytes): a
// [key][token] row of 20 floats puts keys 4 apart 16 banks apart, so the
// [4q+e][n] scalar reads, the [4kg+e][tp] stores and the [n][4q] 16-byte
// reads all spread over the 64 banks; a [token][value] row of 72 bf16
// (36 banks) does the same for the 8-byte tile stores [n][16vb+4q].
constexpr int kFP = 20;
constexpr int kTP = 72;

struct alignas(32) KSmem {
  // per (key row, token) factors of the chunk: [key][token]
  float bh[kD][kFP], kh[kD][kFP], rh[kD][kFP], ah[kD][kFP];
  float gm[kD][kFP], wsf[kD][kFP];
  // masked token-token blocks in B-operand form, one per lane: the [lo | hi]
  // half of the BOp (its upper half is zero)
  bf16x8 gram[8][64];
  // the chunk's DY and V, and SA and DSA as bf16 (hi, lo) splits,
  // [token][value]: staged once per workgroup, read by every wave as matrix
  // operands and (DY, DSA) transposed by the carry
  __bf16 dyh[kL][kTP], vh[kL][kTP], sah[kL][kTP], sal[kL][kTP], dsh[kL][kTP], dsl[kL][kTP];
  float dsa0[kD];   // dsa of the chunk's first token (fp32)
};

// the stored half of a BOp ([lo | hi]) and the full operand rebuilt from it
__device__ __forceinline__ bf16x8 half_b(BOp b) {
  return __builtin_shufflevector(b, b, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ BOp full_b(bf16x8 h) {
  const bf16x8 z = {};
  return __builtin_shufflevector(h, z, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}

__device__ __forceinline__ f32x4 mma32x2(const Sp8& a, bf16x8 b, f32x4 c) {
  c = mma32(a.lo, b, c);
  return mma32(a.hi, b, c);
}
__device__ __forceinline__ f32x4 mma32x2b(bf16x8 a, const Sp8& b, f32x4 c) {
  c = mma32(a, b.lo, c);
  return mma32(a, b.hi, c);
}

// full sum over the 16 lanes of a DPP row, in every lane of the row
__device__ __forceinline__ float row_allsum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xf, 0xf, false));
  return x;
}
// lane 15 of the lane's DPP row, in every lane of the row (row_newbcast)
__device__ __forceinline__ float row_last(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x15f, 0xf, 0xf, false));
}
// inclusive suffix sum over the 16 lanes of a DPP row (row_shl: lane l
// reads lane l+N, zero past the row end)
__device__ __forceinline__ float row_suffix(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x101, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x102, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x104, 0xf, 0xf, true));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x108, 0xf, 0xf, true));
  return x;
}

// Workgroup barrier over LDS only: the waves exchange data through LDS
// alone, so the barrier waits for the wave's own LDS operations (lgkmcnt)
// and not for its outstanding global loads, which __syncthreads' release
// fence would wait for (the next chunk's requests stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ f32x4 ld_f4(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}
__device__ __forceinline__ f32x4 ld_f4_lds(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}
__device__ __forceinline__ bf16x8 cat8(bf16x4 x, bf16x4 y) {
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ float bf(uint16_t x) { return __uint_as_float(static_cast<uint32_t>(x) << 16); }

__global__ __launch_bounds__(kKNT, 3) void key_chunk_kernel(KPassArgs p) {
  __shared__ KSmem sm;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int n = lane & 15, q = lane >> 4;
  // Workgroup order: every (batch, head)'s spans but its last first, then
  // the last spans (shorter when the span length does not divide the chunk
  // count), which fill the final round of workgroups.
  const int nfull = p.nspan - 1;
  const int nlead = static_cast<int>(gridDim.x / p.nspan) * nfull;
  const int gid = static_cast<int>(blockIdx.x);
  const int span = gid < nlead ? gid % nfull : nfull;
  const int bh = gid < nlead ? gid / nfull : gid - nlead;
  const int bidx = bh / p.H, h = bh % p.H;
  const int nchunk = p.T / kL;
  const int64_t stride = static_cast<int64_t>(p.H) * kD;
  const int64_t base0 = (static_cast<int64_t>(bidx) * p.T * p.H + h) * kD;
  auto tok = [&](int t) { return base0 + static_cast<int64_t>(t) * stride; };
  const int row = 16 * wv + n;              // key row of this lane (A / carry layout)
  const int m_hi = min(p.cps * (span + 1), nchunk) - 1;
  const int m_lo = p.cps * span;

  // ---- carry into the span's last chunk: G_u^T P_u of the span's end token
  f32x4 PcT[4];
#pragma unroll
  for (int vb = 0; vb < 4; ++vb) PcT[vb] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (m_hi + 1 < nchunk) {
    const int u = kL * (m_hi + 1);
    const float* Pn = p.pbnd + (static_cast<int64_t>(bh) * p.nspan + span + 1) * kD * kD +
                      static_cast<int64_t>(row) * kD;
    const float x = bf(p.w[tok(u) + row]);
    const float wu = __builtin_amdgcn_exp2f(kCl * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLg2e * x)));
    const float au = bf(p.a[tok(u) + row]);
#pragma unroll
    for (int vb = 0; vb < 4; ++vb) {
      const int j0 = 16 * vb + 4 * q;
      const f32x4 pn = ld_f4(Pn + j0);
      const f32x4 du = ld_f4(p.dsa + tok(u) + j0);
      PcT[vb] = wu * pn + au * du;
    }
  } else if (p.dfinal != nullptr) {
    const float* Pf = p.dfinal + (static_cast<int64_t>(bh) * kD + row) * kD;
#pragma unroll
    for (int vb = 0; vb < 4; ++vb) PcT[vb] = ld_f4(Pf + 16 * vb + 4 * q);
  }

  // Global inputs of one chunk, requested a chunk ahead.  The inputs every
  // wave needs (dy, v, sa, dsa of the chunk's 16 tokens) are read once per
  // workgroup: thread (token tid / 16, values 4 (tid % 16)..+3) holds its
  // piece until the chunk starts and then stages it in LDS; the prep role's
  // rows (w, r, k, a, b of token tid % 16, keys 4 (tid / 16)..+3) are its
  // own.  About 22 registers stay live across a chunk, where the inputs
  // themselves (48 per lane for each wave's full copy) could not.
  struct Pf {
    u32x2 dy, v;
    f32x4 sa, ds;
    u32x2 rw, rr, rk, ra, rb;
  };
  const int tp = tid & 15, kg = tid >> 4;   // prep role: token tp, keys 4kg..4kg+3
  const int st_tok = tid >> 4, st_v = 4 * (tid & 15);   // staging role
  // Addresses: a block-uniform 64-bit chunk base plus a 32-bit lane offset
  // formed at each request (opaque to loop-invariant hoisting), so that no
  // per-lane 64-bit address stays live across the loop: such values
  // spilled, and each reload waited for every request in flight (the
  // vector-memory counter is in order).
  const int ih = static_cast<int>(stride);
  // the lane index rebuilt from the lane mask (no live input register)
  auto lane_now = [] {
    int l = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    asm volatile("" : "+v"(l));
    return l;
  };
  auto load = [&](Pf& f, int m) {
    const int64_t cb = tok(kL * m);
    const int t = 64 * wv + lane_now();   // the thread index
    const int so = (t >> 4) * ih + 4 * (t & 15), po = (t & 15) * ih + 4 * (t >> 4);
    f.dy = *reinterpret_cast<const u32x2*>(p.dy + cb + static_cast<uint32_t>(so));
    f.v = *reinterpret_cast<const u32x2*>(p.v + cb + static_cast<uint32_t>(so));
    f.sa = ld_f4(p.sa + cb + static_cast<uint32_t>(so));
    f.ds = ld_f4(p.dsa + cb + static_cast<uint32_t>(so));
    f.rw = *reinterpret_cast<const u32x2*>(p.w + cb + static_cast<uint32_t>(po));
    f.rr = *reinterpret_cast<const u32x2*>(p.r + cb + static_cast<uint32_t>(po));
    f.rk = *reinterpret_cast<const u32x2*>(p.k + cb + static_cast<uint32_t>(po));
    f.ra = *reinterpret_cast<const u32x2*>(p.a + cb + static_cast<uint32_t>(po));
    f.rb = *reinterpret_cast<const u32x2*>(p.b + cb + static_cast<uint32_t>(po));
  };
  auto load_s0 = [&](f32x4 (&S04)[4], int m) {
    // chunk 0 starts from state0, or from the zero state (then row 0 of
    // the snapshot of chunk 0 is loaded and discarded: always in bounds)
    const float* s0 =
        (m == 0 && p.state0 != nullptr)
            ? p.state0 + static_cast<int64_t>(bidx) * p.state0_stride +
                  static_cast<int64_t>(h) * kD * kD
            : p.bnd + (static_cast<int64_t>(bh) * nchunk + max(m - 1, 0)) * kD * kD;
    const int l = lane_now();
    const int ro = (16 * wv + (l & 15)) * kD + 4 * (l >> 4);
#pragma unroll
    for (int vb = 0; vb < 4; ++vb) S04[vb] = ld_f4(s0 + static_cast<uint32_t>(ro + 16 * vb));
  };
  f32x4 S04[4];
  load_s0(S04, m_hi);
  Pf pf;
  load(pf, m_hi);
  auto body = [&](int m) {
    const int t0 = kL * m;
    // the previous chunk's readers are done with the shared tiles (the
    // barriers order LDS only: the requests for the next chunk stay in
    // flight across them)
    lds_barrier();
    // ---------------- stage the chunk's shared inputs
    {
      *reinterpret_cast<u32x2*>(&sm.dyh[st_tok][st_v]) = pf.dy;
      *reinterpret_cast<u32x2*>(&sm.vh[st_tok][st_v]) = pf.v;
      uint32_t h0, l0, h1, l1;
      split2(pf.sa[0], pf.sa[1], h0, l0);
      split2(pf.sa[2], pf.sa[3], h1, l1);
      *reinterpret_cast<u32x2*>(&sm.sah[st_tok][st_v]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(&sm.sal[st_tok][st_v]) = u32x2{l0, l1};
      split2(pf.ds[0], pf.ds[1], h0, l0);
      split2(pf.ds[2], pf.ds[3], h1, l1);
      *reinterpret_cast<u32x2*>(&sm.dsh[st_tok][st_v]) = u32x2{h0, h1};
      *reinterpret_cast<u32x2*>(&sm.dsl[st_tok][st_v]) = u32x2{l0, l1};
      if (st_tok == 0) *reinterpret_cast<f32x4*>(&sm.dsa0[st_v]) = pf.ds;
    }
    const u32x2 rw = pf.rw, rr = pf.rr, rk = pf.rk, ra = pf.ra, rb = pf.rb;
    // the next (earlier) chunk's shared inputs are requested as soon as this
    // chunk's are staged: issued here rather than after the state products
    // they measured 2.3 % faster over the whole backward (1.088 -> 1.062 ms
    // at the config-1 shape), bit-identical
    if (m > m_lo) load(pf, m - 1);

    // ---------------- prep: decays and scaled per-(key, token) factors
    {
      auto el = [](u32x2 v, int e) {
        const uint32_t wd = v[e >> 1];
        return __uint_as_float((e & 1) ? (wd & 0xffff0000u) : (wd << 16));
      };
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = 4 * kg + e;
        const float x = el(rw, e);
        const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-kLg2e * x));
        const float lw2 = kCl * sg;
        const float G = row_scan(lw2);
        const float G15 = row_last(G);
        const float Gp = G - lw2;
        const float ig = __builtin_amdgcn_exp2f(-G);
        sm.gm[key][tp] = __builtin_amdgcn_exp2f(G);
        sm.wsf[key][tp] = kNegEh * sg * (1.0f - sg);
        const float xr = el(rr, e), xk = el(rk, e), xa = el(ra, e), xb = el(rb, e);
        sm.bh[key][tp] = xb * ig;
        sm.kh[key][tp] = xk * ig;
        sm.rh[key][tp] = xr * __builtin_amdgcn_exp2f(G - G15);
        sm.ah[key][tp] = xa * __builtin_amdgcn_exp2f(Gp - G15);
      }
    }
    lds_barrier();   // the staged inputs and the factors are in place

    // ---------------- operand blocks (K = 32: value blocks {2mb, 2mb+1}),
    // lane (n, q): token n, values 16vb + 4q..+3 of the staged rows
    bf16x4 DYb[4], Vb[4], SAh[4], SAl[4], DSh[4], DSl[4];
#pragma unroll
    for (int vb = 0; vb < 4; ++vb) {
      const int j0 = 16 * vb + 4 * q;
      DYb[vb] = *reinterpret_cast<const bf16x4*>(&sm.dyh[n][j0]);
      Vb[vb] = *reinterpret_cast<const bf16x4*>(&sm.vh[n][j0]);
      SAh[vb] = *reinterpret_cast<const bf16x4*>(&sm.sah[n][j0]);
      SAl[vb] = *reinterpret_cast<const bf16x4*>(&sm.sal[n][j0]);
      DSh[vb] = *reinterpret_cast<const bf16x4*>(&sm.dsh[n][j0]);
      DSl[vb] = *reinterpret_cast<const bf16x4*>(&sm.dsl[n][j0]);
    }
    const bf16x8 DY0 = cat8(DYb[0], DYb[1]), DY1 = cat8(DYb[2], DYb[3]);
    const bf16x8 V0 = cat8(Vb[0], Vb[1]), V1 = cat8(Vb[2], Vb[3]);
    const Sp8 SA0{cat8(SAh[0], SAh[1]), cat8(SAl[0], SAl[1])};
    const Sp8 SA1{cat8(SAh[2], SAh[3]), cat8(SAl[2], SAl[3])};
    const Sp8 DS0{cat8(DSh[0], DSh[1]), cat8(DSl[0], DSl[1])};
    const Sp8 DS1{cat8(DSh[2], DSh[3]), cat8(DSl[2], DSl[3])};
    float S0f[16];
#pragma unroll
    for (int vb = 0; vb < 4; ++vb)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        S0f[4 * vb + e] = (m > 0 || p.state0 != nullptr) ? S04[vb][e] : 0.0f;
    // ---------------- token-token blocks, two per wave
    {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      f32x4 g0, g1;
      // accumulator: G[s][t] at lane t + 16 (s/4), item s%4; the masks keep
      // s <= t (dr), s < t (da), s >= t / s > t (dk, db)
      auto mask = [&](f32x4 g, int lo) {   // keep s - t <= -lo (lo = 0 / 1) or
        f32x4 r;                           // s - t >= lo - 2 (lo = 2 / 3)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = 4 * q + e - n;
          const bool keep = lo < 2 ? d <= -lo : d >= lo - 2;
          r[e] = keep ? g[e] : 0.f;
        }
        return r;
      };
      if (wv == 0) {        // SA DY^T, V DY^T  (dr)
        g0 = mask(mma32x2(SA1, DY1, mma32x2(SA0, DY0, z)), 0);
        g1 = mask(mma32(V1, DY1, mma32(V0, DY0, z)), 0);
      } else if (wv == 1) { // SA DSA^T, V DSA^T  (da)
        g0 = mask(mma32x3(SA1, DS1, mma32x3(SA0, DS0, z)), 1);
        g1 = mask(mma32x2b(V1, DS1, mma32x2b(V0, DS0, z)), 1);
      } else if (wv == 2) { // DY V^T, DSA V^T  (dk)
        g0 = mask(mma32(DY1, V1, mma32(DY0, V0, z)), 2);
        g1 = mask(mma32x2(DS1, V1, mma32x2(DS0, V0, z)), 3);
      } else {              // DY SA^T, DSA SA^T  (db)
        g0 = mask(mma32x2b(DY1, SA1, mma32x2b(DY0, SA0, z)), 2);
        g1 = mask(mma32x3(DS1, SA1, mma32x3(DS0, SA0, z)), 3);
      }
      sm.gram[2 * wv][lane] = half_b(as_b(split4(g0)));
      sm.gram[2 * wv + 1][lane] = half_b(as_b(split4(g1)));
    }
    // ---------------- state-side products (rows of this wave)
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 DR, DA, DK0, DB0;
    {
      const Sp8 S00 = split8(&S0f[0]), S01 = split8(&S0f[8]);
      DR = mma32x2(S01, DY1, mma32x2(S00, DY0, zero));
      DA = mma32x3(S01, DS1, mma32x3(S00, DS0, zero));
      float pc[16];
#pragma unroll
      for (int vb = 0; vb < 4; ++vb)
#pragma unroll
        for (int e = 0; e < 4; ++e) pc[4 * vb + e] = PcT[vb][e];
      const Sp8 P0 = split8(&pc[0]), P1 = split8(&pc[8]);
      DK0 = mma32x2(P1, V1, mma32x2(P0, V0, zero));
      DB0 = mma32x3(P1, SA1, mma32x3(P0, SA0, zero));
    }
    // rowsum(Pc o S0) for row `row`, gathered over the four lane groups
    float pcs0 = 0.f;
#pragma unroll
    for (int vb = 0; vb < 4; ++vb)
#pragma unroll
      for (int e = 0; e < 4; ++e) pcs0 = fmaf(PcT[vb][e], S0f[4 * vb + e], pcs0);
    pcs0 += __shfl_xor(pcs0, 16);
    pcs0 += __shfl_xor(pcs0, 32);
    // the next (earlier) chunk's start state is requested here, a chunk
    // ahead (after the products, whose operands would otherwise share the
    // registers with it)
    if (m > m_lo) load_s0(S04, m - 1);

    lds_barrier();

    // ---------------- token-side products
    const f32x4 bh4 = ld_f4_lds(&sm.bh[row][4 * q]), kh4 = ld_f4_lds(&sm.kh[row][4 * q]);
    const f32x4 rh4 = ld_f4_lds(&sm.rh[row][4 * q]);
    f32x4 ah4 = ld_f4_lds(&sm.ah[row][4 * q]);
    // R^ enters P (and so dk, db and the carry) times the output scale
    const Split4 sBh = split4(bh4), sKh = split4(kh4), sRh = split4(p.scale * rh4),
                 sAh = split4(ah4);
    auto gram = [&](int g) { return full_b(sm.gram[g][lane]); };
    DR = mm_ab(as_a(sKh), gram(1), mm_ab(as_a(sBh), gram(0), DR));
    DA = mm_ab(as_a(sKh), gram(3), mm_ab(as_a(sBh), gram(2), DA));
    f32x4 DK = mm_ab(as_a(sAh), gram(5), mm_ab(as_a(sRh), gram(4), DK0));
    f32x4 DB = mm_ab(as_a(sAh), gram(7), mm_ab(as_a(sRh), gram(6), DB0));

    // ---------------- outputs: accumulator lane (token n, rows 4q+e of the wave)
    float dr[4], da[4], dk[4], db[4], dw[4];
    {
      const int t = n;
      // raw per-(row, token) values are rebuilt from the stored scaled ones:
      // b = B^ gamma, k = K^ gamma, r = R^ gamma_15 / gamma, a = A^ gamma_15 / gamma_{t-1}
      // (branch-free: token 0's terms are masked arithmetically, so that the
      // four rows' LDS reads and scans form one block the scheduler can
      // interleave, instead of a divergent branch per row)
      const float tpos = t > 0 ? 1.0f : 0.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int rk = 16 * wv + 4 * q + e;
        const float g = sm.gm[rk][t], g15 = sm.gm[rk][15];
        const float gm1 = sm.gm[rk][max(t - 1, 0)];
        const float gp = t > 0 ? gm1 : 1.0f;   // gamma_{t-1} (1 at t = 0)
        const float rho = g15 * __builtin_amdgcn_rcpf(g);   // gamma_15 / gamma_t
        dr[e] = p.scale * g * DR[e];
        da[e] = gp * DA[e];
        dk[e] = rho * DK[e];
        db[e] = rho * DB[e];
        // Z_15: r_15 dr_15 + gamma_15 (rowsum(Pc o S0) + sum_s B^_s DB0_s + K^_s DK0_s)
        const float bhv = sm.bh[rk][t], khv = sm.kh[rk][t];
        const float part = row_allsum(bhv * DB0[e] + khv * DK0[e]);
        const float rs0 = __shfl(pcs0, 4 * q + e);   // lanes 4q+e hold row 16wv+4q+e
        const float dr15 = row_last(dr[e]);
        const float z15 = sm.rh[rk][15] * dr15 + g15 * (rs0 + part);
        const float bd = bhv * g * db[e] + khv * g * dk[e];
        // inc_t = -b_t db_t - k_t dk_t + a_t da_t + r_{t-1} dr_{t-1}   (t >= 1)
        const float drp = row_prev(dr[e], 0.0f);
        const float igp = __builtin_amdgcn_rcpf(gp);
        const float rp = sm.rh[rk][max(t - 1, 0)] * g15 * igp;
        const float av = sm.ah[rk][t] * g15 * igp;
        const float inc = tpos * (-bd + av * da[e] + rp * drp);
        const float z = z15 + row_suffix(inc) - inc;   // Z_t
        dw[e] = (z - bd) * sm.wsf[rk][t];
      }
      const int64_t o = tok(t0 + t) + 16 * wv + 4 * q;
      auto st4 = [&](uint16_t* dst, const float* x) {
        u32x2 pk = {pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3])};
        *reinterpret_cast<u32x2*>(dst + o) = pk;
      };
      st4(p.dr, dr);
      st4(p.da, da);
      st4(p.dk, dk);
      st4(p.db, db);
      st4(p.dw, dw);
    }

    // ---------------- carry to the previous chunk (A layout of Pc^T)
    if (m > m_lo) {
      // B operands over tokens s for this lane's row: R^ and A^ with s >= 1
      ah4[0] = q == 0 ? 0.f : ah4[0];
      const BOp bR = as_b(sRh), bA = as_b(split4(ah4));
      const float g15 = sm.gm[row][15], a0 = sm.ah[row][0] * g15;   // gamma_{-1} = 1
#pragma unroll
      for (int vb = 0; vb < 4; ++vb) {
        // A = X^T (value 16vb+n, K = token 4q+e) through the transpose read
        const __bf16* dyp = &sm.dyh[4 * q + (n >> 2)][16 * vb + 4 * (n & 3)];
        const __bf16* dhp = &sm.dsh[4 * q + (n >> 2)][16 * vb + 4 * (n & 3)];
        const __bf16* dlp = &sm.dsl[4 * q + (n >> 2)][16 * vb + 4 * (n & 3)];
        const bf16x4 zz = {};
        const AOp aDY = cat8(tr_rows(dyp), zz);
        const AOp aDS = cat8(tr_rows(dhp), tr_rows(dlp));
        // accumulator: D[value 16vb+4q+e][row n] at lane n + 16q, item e
        f32x4 acc = mm_ab(aDS, bA, mm_ab(aDY, bR, PcT[vb]));
        const f32x4 d0 = ld_f4_lds(&sm.dsa0[16 * vb + 4 * q]);
        PcT[vb] = g15 * acc + a0 * d0;
      }
    }
  };
  for (int m = m_hi; m >= m_lo; --m) body(m);
}

}  // namespace

// Span length.  Short problems (fewer than 2 048 workgroups at 16-chunk
// spans, about 2.7 per slot of the 768 below) keep 8-chunk spans for the
// parallelism.  Larger ones take the length from 8 to 17 chunks that gives
// the shortest modelled makespan: the workgroups run three per CU on
// MI355X's 256 CUs (768 slots), each costing its chunks plus one chunk of
// span start-up, dispatched in the kernel's order (full spans first, each
// (batch, head)'s shorter last span after them) onto the least loaded slot.
// A length that leaves the last round mostly empty loses up to a round: at
// the config-1 shape (256 (batch, head) units of 256 chunks) 16-chunk spans
// are 4 096 workgroups = 5.3 rounds, and 17-chunk spans (15 full + one of a
// single chunk) run the whole backward 1.141 -> 1.086 ms (11: 1.081,
// 15: 1.086, 18: 1.092).  The choice depends on the shape alone, so the
// workspace query and the launch agree.
namespace {

// makespan of n_full jobs of length d then n_short of length e (e <= d),
// each on the least loaded of `slots` equal slots, in closed form: the full
// jobs leave two levels d apart; the short ones fill the lower level up to
// the upper one, then go round all slots, the lower of the two levels first
double greedy_makespan(int64_t n_full, double d, int64_t n_short, double e, int64_t slots) {
  const int64_t k = n_full / slots, r = n_full % slots;
  double lo = static_cast<double>(k) * d, hi = lo + d;
  int64_t clo = slots - r;
  const int64_t chi = r;
  int64_t left = n_short;
  if (left == 0) return chi > 0 ? hi : lo;
  if (chi == 0) return lo + static_cast<double>(left / slots) * e + (left % slots ? e : 0.0);
  const int64_t rounds = static_cast<int64_t>(ceil((hi - lo) / e));
  if (left <= rounds * clo)
    return fmax(hi, lo + static_cast<double>(left / clo) * e + (left % clo ? e : 0.0));
  left -= rounds * clo;
  lo += static_cast<double>(rounds) * e;   // now within e above hi
  double a = hi, b = lo;
  int64_t ca = chi;
  if (b < a) {
    const double t = a;
    a = b;
    b = t;
    ca = clo;
  }
  const double full = static_cast<double>(left / slots) * e;
  const int64_t rem = left % slots;
  a += full;
  b += full;
  if (rem == 0) return fmax(a, b);
  return rem <= ca ? fmax(b, a + e) : b + e;
}

}  // namespace

int key_chunk_span(int batch, int tokens, int heads) {
  const int64_t units = static_cast<int64_t>(batch) * heads;
  const int nchunk = tokens / kL;
  if (units * ((nchunk + 15) / 16) < 2048) return 8;
  constexpr int64_t kSlots = 3 * 256;
  constexpr double kStart = 1.0;   // span start-up, in chunks
  int best = 16;
  double best_t = 0.0;
  for (int cps = 17; cps >= 8; --cps) {   // ties keep the longer span
    const int nspan = (nchunk + cps - 1) / cps;
    const int last = nchunk - (nspan - 1) * cps;
    const double t = greedy_makespan(units * (nspan - 1), cps + kStart, units, last + kStart, kSlots);
    if (cps == 17 || t < best_t) {
      best = cps;
      best_t = t;
    }
  }
  return best;
}

int launch_key_chunk(const PretrainBwdArgs& a, const float* pbnd, int nspan, int cps,
                     hipStream_t s) {
  KPassArgs k;
  k.T = a.tokens;
  k.H = a.heads;
  k.nspan = nspan;
  k.cps = cps;
  k.r = static_cast<const uint16_t*>(a.r);
  k.w = static_cast<const uint16_t*>(a.w);
  k.k = static_cast<const uint16_t*>(a.k);
  k.v = static_cast<const uint16_t*>(a.v);
  k.a = static_cast<const uint16_t*>(a.a);
  k.b = static_cast<const uint16_t*>(a.b);
  k.dy = static_cast<const uint16_t*>(a.dy);
  k.sa = a.state_dot_a;
  k.dsa = a.workspace;
  k.bnd = a.boundary;
  k.pbnd = pbnd;
  k.dr = static_cast<uint16_t*>(a.dr);
  k.dw = static_cast<uint16_t*>(a.dw);
  k.dk = static_cast<uint16_t*>(a.dk);
  k.db = static_cast<uint16_t*>(a.db);
  k.da = static_cast<uint16_t*>(a.da);
  k.scale = a.scale;
  k.state0 = a.state0;
  k.state0_stride = a.state0_stride;
  k.dfinal = a.dfinal;
  const int64_t blocks = static_cast<int64_t>(a.batch) * a.heads * nspan;
  hipLaunchKernelGGL(key_chunk_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kKNT), 0, s, k);
  return record_launch();
}

}  // namespace fr2
