// Training backward of the [B,T,H,D] zero-state WKV7 recurrence (the
// pretrain path).  Replaces backward_kernel_preload / backward_kernel_split64
// / backward_value_columns + backward_key_rows
// (csrc/sm120/tmix/wkv7/pretrain_recurrent_bf16_forward.cu:163-486) with a
// two-kernel design of its own.
//
// With P_t = dL/dS_t (S_t the post-update state, [key][value]) the backward
// is
//   P_t   = r_t dy_t^T + (diag(w_{t+1}) + a_{t+1} b_{t+1}^T) P_{t+1}
//   dsa_t = P_t^T b_t,   dv_t = P_t^T k_t                  (value columns)
//   dr_t  = S_t dy_t,    dk_t = P_t v_t,   db_t = P_t sa_t,
//   da_t  = S_{t-1} dsa_t,   dw_t = rowsum(P_t o S_{t-1}) * dw/dlogit (key rows)
// and S_{t-1} = (S_t - k_t v_t^T - b_t sa_t^T) / w_t rebuilds the pre-update
// state from the forward's post-chunk snapshot (boundary) and its saved sa.
//
// The only quantity that couples key rows is dsa, a column reduction of P
// that feeds back into P's next step.  So:
//   1. the value pass runs the column recurrence of P backwards over T and
//      writes dv and dsa.  It is the forward recurrence in reverse time with
//      (k, v, r, a, b, w) <- (r_t, dy_t, k_t, b_{t+1}, a_{t+1}, w_{t+1}), so
//      at D = 64 it runs on the chunked MFMA kernel's reverse mode; other
//      head sizes use value_kernel (one workgroup per (batch, head), 4 lanes
//      per value column, D/4 keys each, DPP quad reductions);
//   2. key_kernel: rows are then independent; each workgroup owns 64 key rows
//      of one (batch, head) (4 lanes per row, D/4 values each) and walks T
//      backwards carrying its rows of S and P, writing dr, dw, dk, db, da.
// Token operands are staged through LDS as fp32, one tile of TT tokens at a
// time, double-buffered with the next tile's global loads in flight.  Lane
// 4c+q of each 16-lane DPP row (q = quarter of the reduced index, c = one of
// the row's four columns/rows) reads only its own D/16 operand values per
// token and receives the other three lanes' values of its quarter through
// DPP row rotations, folded into the FMAs as DPP operands: LDS delivers each
// operand value once per 16-lane row instead of once per lane.  The
// key kernel keeps S and P row-scaled (S = g Sh, P = hs Ph, g and hs per-row
// scalars) so the 1/w and w factors cost two multiplies per row instead of
// one per element; both scales restart at every 16-token boundary snapshot.
#include "recurrent.h"

namespace fr2 {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 16;                       // boundary snapshot period
constexpr float kWScale = -0.6065306597126334f;  // -exp(-1/2)

// sum over the 4 lanes of a DPP quad (result in every lane of the quad)
__device__ __forceinline__ float quad_sum(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xf, 0xf, false));
  return x;
}

__device__ __forceinline__ void widen8(u32x4 u, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}

template <int D>
struct Cfg {
  static constexpr int E = D / 4;                 // elements per lane
  static constexpr int Q = E / 4;                 // own operand values per lane per token
  static constexpr int TT = D <= 128 ? 16 : 8;    // tokens per LDS tile
};

// Lane 4c+q of a 16-lane DPP row receives the value of lane 4((c-m)&3)+q.
// Element e = m*Q + s of a lane therefore refers to index
//   q*E + Q*((c - m) & 3) + s
// of the D-long reduced axis.
// The rotated operand is always src0 of a VOP2 instruction with a DPP
// row_ror modifier, so the rotation costs no instruction: the compiler folds
// it into v_mul_f32 (mul_rot); for v_fmac_f32, which it does not fold on this
// target, fmac_rot writes the DPP form directly.  The rotated sources are
// LDS-loaded operand values that no VALU instruction writes, so the
// VALU-write -> DPP-read wait states never apply to them.
template <int M>
__device__ __forceinline__ float mul_rot(float x, float y) {
  if constexpr (M == 0) {
    return x * y;
  } else {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + 4 * M,
                                                      0xf, 0xf, true)) * y;
  }
}
// acc += rot_M(x) * y
template <int M>
__device__ __forceinline__ void fmac_rot(float& acc, float x, float y) {
  if constexpr (M == 0) {
    acc = fmaf(x, y, acc);
  } else if constexpr (M == 1) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_ror:4 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(x), "v"(y));
  } else if constexpr (M == 2) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_ror:8 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(x), "v"(y));
  } else {
    asm("v_fmac_f32_dpp %0, %1, %2 row_ror:12 row_mask:0xf bank_mask:0xf" : "+v"(acc) : "v"(x), "v"(y));
  }
}

template <int M>
struct IC {
  static constexpr int value = M;
};

__device__ __forceinline__ void store8(float* dst, const float* f) {
  *reinterpret_cast<float4*>(dst) = make_float4(f[0], f[1], f[2], f[3]);
  *reinterpret_cast<float4*>(dst + 4) = make_float4(f[4], f[5], f[6], f[7]);
}

template <int Q>
__device__ __forceinline__ void lds_read(const float* src, float* dst) {
#pragma unroll
  for (int x = 0; x < Q; x += 4) {
    const float4 v = *reinterpret_cast<const float4*>(src + x);
    dst[x] = v.x; dst[x + 1] = v.y; dst[x + 2] = v.z; dst[x + 3] = v.w;
  }
}

// ---------------------------------------------------------------------------
// 1. value columns: P^T recurrence, dv and dsa
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(4 * D) void value_kernel(
    int T, int H, const uint16_t* __restrict__ r, const uint16_t* __restrict__ wl,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ a,
    const uint16_t* __restrict__ b, const uint16_t* __restrict__ dy,
    uint16_t* __restrict__ dv, float* __restrict__ dsa) {
  using C = Cfg<D>;
  constexpr int NT = 4 * D, E = C::E, Q = C::Q, TT = C::TT;
  constexpr int kVec = 6;                    // r, w, k, a, b, dy
  constexpr int UPV = TT * D / 8;            // 16-byte units per vector per tile
  constexpr int NU = kVec * UPV;
  constexpr int UPT = (NU + NT - 1) / NT;
  __shared__ __align__(16) float buf[2][kVec][TT][D];

  const int bidx = blockIdx.x / H, h = blockIdx.x % H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int q = lane & 3, c4 = (lane >> 2) & 3;
  const int col = 16 * (tid >> 6) + 4 * (lane >> 4) + c4;   // value column
  const int own = q * E + Q * c4;                           // this lane's operand slice
  const int64_t stride = static_cast<int64_t>(H) * D;
  const int64_t base = (static_cast<int64_t>(bidx) * T * H + h) * D;

  u32x4 pre[UPT];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int idx = tid + u * NT;
      if (NU % NT == 0 || idx < NU) {
        const int m = idx / UPV, rem = idx % UPV;
        const int tt = rem / (D / 8), g = rem % (D / 8);
        const uint16_t* src = m == 0 ? r : m == 1 ? wl : m == 2 ? k : m == 3 ? a : m == 4 ? b : dy;
        pre[u] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(src + base + (t0 + tt) * stride + 8 * g));
      }
    }
  };
  auto store_tile = [&](int slot) {
#pragma unroll
    for (int u = 0; u < UPT; ++u) {
      const int idx = tid + u * NT;
      if (NU % NT == 0 || idx < NU) {
        const int m = idx / UPV, rem = idx % UPV;
        const int tt = rem / (D / 8), g = rem % (D / 8);
        float f[8];
        widen8(pre[u], f);
        if (m == 1) {
#pragma unroll
          for (int i = 0; i < 8; ++i) f[i] = retention_from_logit(f[i]);
        }
        store8(&buf[slot][m][tt][8 * g], f);
      }
    }
  };

  float P[E];
#pragma unroll
  for (int e = 0; e < E; ++e) P[e] = 0.0f;

  const int ntile = T / TT;
  load_tile((ntile - 1) * TT);
  store_tile(0);
  __syncthreads();
  for (int it = ntile - 1; it >= 0; --it) {
    const int slot = (ntile - 1 - it) & 1;
    if (it > 0) load_tile((it - 1) * TT);
    for (int tt = TT - 1; tt >= 0; --tt) {
      float R[Q], W[Q], K[Q], A[Q], Bv[Q];
      lds_read<Q>(&buf[slot][0][tt][own], R);
      lds_read<Q>(&buf[slot][2][tt][own], K);
      lds_read<Q>(&buf[slot][4][tt][own], Bv);
      const float dyc = buf[slot][5][tt][col];
      float dv0 = 0.0f, dv1 = 0.0f, ds0 = 0.0f, ds1 = 0.0f;
      auto part1 = [&](auto mc) {
        constexpr int m = decltype(mc)::value;
#pragma unroll
        for (int x = 0; x < Q; ++x) {
          float& p = P[m * Q + x];
          fmac_rot<m>(p, R[x], dyc);
          fmac_rot<m>((x & 1) ? dv1 : dv0, K[x], p);
          fmac_rot<m>((x & 1) ? ds1 : ds0, Bv[x], p);
        }
      };
      part1(IC<0>{}); part1(IC<1>{}); part1(IC<2>{}); part1(IC<3>{});
      lds_read<Q>(&buf[slot][1][tt][own], W);
      lds_read<Q>(&buf[slot][3][tt][own], A);
      const float dvs = quad_sum(dv0 + dv1);
      const float dss = quad_sum(ds0 + ds1);
      const int64_t o = base + static_cast<int64_t>(it * TT + tt) * stride + col;
      if (q == 0) dv[o] = IoBF16::from_f32(dvs);
      if (q == 1) dsa[o] = dss;
      auto part2 = [&](auto mc) {
        constexpr int m = decltype(mc)::value;
#pragma unroll
        for (int x = 0; x < Q; ++x) {
          float& p = P[m * Q + x];
          p = mul_rot<m>(W[x], p);
          fmac_rot<m>(p, A[x], dss);
        }
      };
      part2(IC<0>{}); part2(IC<1>{}); part2(IC<2>{}); part2(IC<3>{});
    }
    if (it > 0) store_tile(slot ^ 1);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// 2. key rows: S and P rows, dr dw dk db da
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void key_kernel(
    int T, int H, const uint16_t* __restrict__ r, const uint16_t* __restrict__ wl,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
    const uint16_t* __restrict__ dy, const float* __restrict__ boundary,
    const float* __restrict__ sa, const float* __restrict__ dsa,
    uint16_t* __restrict__ dr, uint16_t* __restrict__ dw, uint16_t* __restrict__ dk,
    uint16_t* __restrict__ db, uint16_t* __restrict__ da) {
  using C = Cfg<D>;
  constexpr int NT = 256, E = C::E, Q = C::Q, TT = C::TT, RG = D / 64;
  constexpr int UB = TT * D / 8;    // units per bf16 vector (dy, v)
  constexpr int UF = TT * D / 4;    // units per f32 vector (sa, dsa)
  constexpr int UR = TT * 8;        // units per row-scalar vector (64 rows)
  constexpr int NB = 2 * UB / NT;            // bf16 vector units per thread
  constexpr int NF = 2 * UF / NT;            // f32 vector units per thread
  constexpr int NR = (5 * UR + NT - 1) / NT; // row-scalar units per thread
  static_assert(2 * UB % NT == 0 && 2 * UF % NT == 0, "tile units must split evenly");
  // vec: dy, v, sa, dsa; rows: r, w, k, a, b and the logit derivative
  // factor of w, for this group's 64 rows
  __shared__ __align__(16) float vec[2][4][TT][D];
  __shared__ __align__(16) float rows[2][6][TT][64];

  const int rg = blockIdx.x % RG;
  const int bh = blockIdx.x / RG;
  const int bidx = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63;
  const int q = lane & 3, c4 = (lane >> 2) & 3;
  const int row = 16 * (tid >> 6) + 4 * (lane >> 4) + c4;   // key row within the group
  const int i = rg * 64 + row;
  const int own = q * E + Q * c4;                           // this lane's operand slice
  const int64_t stride = static_cast<int64_t>(H) * D;
  const int64_t base = (static_cast<int64_t>(bidx) * T * H + h) * D;
  const int nchunk = T / kChunk;
  const float* bnd_base = boundary + (static_cast<int64_t>(bh) * nchunk) * D * D +
                          static_cast<int64_t>(i) * D + q * E;  // + Q*((c4-m)&3) per m

  u32x4 preB[NB], preF[NF], preR[NR];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int idx = tid + u * NT;
      const int m = idx / UB, rem = idx % UB;
      const int tt = rem / (D / 8), g = rem % (D / 8);
      preB[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          (m == 0 ? dy : v) + base + (t0 + tt) * stride + 8 * g));
    }
#pragma unroll
    for (int u = 0; u < NF; ++u) {
      const int idx = tid + u * NT;
      const int m = idx / UF, rem = idx % UF;
      const int tt = rem / (D / 4), g = rem % (D / 4);
      preF[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          (m == 0 ? sa : dsa) + base + (t0 + tt) * stride + 4 * g));
    }
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int idx = tid + u * NT;
      if (5 * UR % NT == 0 || idx < 5 * UR) {
        const int m = idx / UR, rem = idx % UR;
        const int tt = rem / 8, g = rem % 8;
        const uint16_t* s = m == 0 ? r : m == 1 ? wl : m == 2 ? k : m == 3 ? a : b;
        preR[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
            s + base + (t0 + tt) * stride + rg * 64 + 8 * g));
      }
    }
  };
  auto store_tile = [&](int slot) {
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int idx = tid + u * NT;
      const int m = idx / UB, rem = idx % UB;
      const int tt = rem / (D / 8), g = rem % (D / 8);
      float f[8];
      widen8(preB[u], f);
      store8(&vec[slot][m][tt][8 * g], f);
    }
#pragma unroll
    for (int u = 0; u < NF; ++u) {
      const int idx = tid + u * NT;
      const int m = idx / UF, rem = idx % UF;
      const int tt = rem / (D / 4), g = rem % (D / 4);
      *reinterpret_cast<u32x4*>(&vec[slot][2 + m][tt][4 * g]) = preF[u];
    }
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int idx = tid + u * NT;
      if (5 * UR % NT == 0 || idx < 5 * UR) {
        const int m = idx / UR, rem = idx % UR;
        const int tt = rem / 8, g = rem % 8;
        float f[8];
        widen8(preR[u], f);
        if (m == 1) {
          float fs[8];
#pragma unroll
          for (int x = 0; x < 8; ++x) {
            const float s = 1.0f / (1.0f + __builtin_amdgcn_exp2f(kNegLog2e * f[x]));
            const float w = __builtin_amdgcn_exp2f(kNegExpHalfLog2e * s);
            f[x] = w;
            fs[x] = kWScale * w * s * (1.0f - s);
          }
          store8(&rows[slot][5][tt][8 * g], fs);
        }
        store8(&rows[slot][m][tt][8 * g], f);
      }
    }
  };

  // With whole-chunk tiles the key pass rebuilds each chunk's states
  // forwards from the chunk's start state and walks backwards through 1/w
  // for at most 8 tokens (from the rebuilt S_15 and S_7).  The 1/w walk
  // amplifies any mismatch between the saved sa and the snapshots by up to
  // exp(exp(-1/2))^n; rebuilding keeps n <= 8 and makes the walk start from
  // states consistent with sa, whatever forward kernel produced them.
  // (N = 256 tiles hold half a chunk: that path walks back from the chunk's
  // own snapshot, which the token-serial forward writes consistently.)
  constexpr bool kRecompute = TT == kChunk;
  float Sh[E], Ph[E], nb[E], Mid[kRecompute ? E : 1];
#pragma unroll
  for (int e = 0; e < E; ++e) Ph[e] = 0.0f;
  float hs = 1.0f, ihs = 1.0f, g = 1.0f, ig = 1.0f;

  auto load_bnd = [&](int ci) {
    const float* src = bnd_base + static_cast<int64_t>(ci) * D * D;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const f4* part = reinterpret_cast<const f4*>(src + Q * ((c4 - m) & 3));
#pragma unroll
      for (int x = 0; x < Q; x += 4) {
        const f4 y = __builtin_nontemporal_load(part + x / 4);
        nb[m * Q + x] = y[0]; nb[m * Q + x + 1] = y[1];
        nb[m * Q + x + 2] = y[2]; nb[m * Q + x + 3] = y[3];
      }
    }
  };

  const int ntile = T / TT;
  if constexpr (kRecompute) {
    if (nchunk >= 2) load_bnd(nchunk - 2);
  } else {
    load_bnd(nchunk - 1);
  }
  load_tile((ntile - 1) * TT);
  store_tile(0);
  __syncthreads();
  for (int it = ntile - 1; it >= 0; --it) {
    const int slot = (ntile - 1 - it) & 1;
    const int tend = it * TT + TT;
    if (tend % kChunk == 0) {
      const int ci = tend / kChunk - 1;
      if constexpr (kRecompute) {
        // rebuild the chunk's states forwards from its start state (the
        // previous chunk's snapshot, zero for the first chunk), in the scaled
        // form S_t = G_t Sh_t with G_t the running product of w_i; keep S_7
        float G = 1.0f, iG = 1.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) Sh[e] = ci > 0 ? nb[e] : 0.0f;
        if (ci >= 2) load_bnd(ci - 2);
        for (int tt = 0; tt < TT; ++tt) {
          const float wi = rows[slot][1][tt][row], ki = rows[slot][2][tt][row];
          const float bi = rows[slot][4][tt][row];
          float V[Q], SA[Q];
          lds_read<Q>(&vec[slot][1][tt][own], V);
          lds_read<Q>(&vec[slot][2][tt][own], SA);
          G *= wi;
          iG *= __builtin_amdgcn_rcpf(wi);
          const float kf = ki * iG, bf = bi * iG;
          auto fwd = [&](auto mc) {
            constexpr int m = decltype(mc)::value;
#pragma unroll
            for (int x = 0; x < Q; ++x) {
              fmac_rot<m>(Sh[m * Q + x], V[x], kf);
              fmac_rot<m>(Sh[m * Q + x], SA[x], bf);
            }
          };
          fwd(IC<0>{}); fwd(IC<1>{}); fwd(IC<2>{}); fwd(IC<3>{});
          if (tt == kChunk / 2 - 1) {
#pragma unroll
            for (int e = 0; e < E; ++e) Mid[e] = Sh[e] * G;
          }
        }
        g = G;
        ig = iG;
      } else {
        // restart S from the chunk's snapshot
#pragma unroll
        for (int e = 0; e < E; ++e) Sh[e] = nb[e];
        g = ig = 1.0f;
        if (ci > 0) load_bnd(ci - 1);
      }
      // fold the P scale
#pragma unroll
      for (int e = 0; e < E; ++e) Ph[e] *= hs;
      hs = ihs = 1.0f;
    }
    if (it > 0) load_tile((it - 1) * TT);
    for (int tt = TT - 1; tt >= 0; --tt) {
      const float ri = rows[slot][0][tt][row], wi = rows[slot][1][tt][row];
      const float ki = rows[slot][2][tt][row], ai = rows[slot][3][tt][row];
      const float bi = rows[slot][4][tt][row], wsi = rows[slot][5][tt][row];
      float DY[Q], V[Q], SA[Q], DS[Q];
      lds_read<Q>(&vec[slot][0][tt][own], DY);
      lds_read<Q>(&vec[slot][1][tt][own], V);
      lds_read<Q>(&vec[slot][2][tt][own], SA);
      lds_read<Q>(&vec[slot][3][tt][own], DS);
      const float rw = __builtin_amdgcn_rcpf(wi);
      const float kg = -ki * ig, bg = -bi * ig;
      const float g_prev = g * rw, ihs_prev = ihs * rw;
      const float rh = ri * ihs, ah = ai * ihs_prev;
      float pr = 0.0f, pw = 0.0f, pk = 0.0f, pb = 0.0f, pa = 0.0f;
      auto step = [&](auto mc) {
        constexpr int m = decltype(mc)::value;
#pragma unroll
        for (int x = 0; x < Q; ++x) {
          float& sh = Sh[m * Q + x];
          float& ph = Ph[m * Q + x];
          fmac_rot<m>(pr, DY[x], sh);
          fmac_rot<m>(sh, V[x], kg);
          fmac_rot<m>(sh, SA[x], bg);
          fmac_rot<m>(ph, DY[x], rh);
          pw = fmaf(ph, sh, pw);
          fmac_rot<m>(pk, V[x], ph);
          fmac_rot<m>(pb, SA[x], ph);
          fmac_rot<m>(pa, DS[x], sh);
          fmac_rot<m>(ph, DS[x], ah);
        }
      };
      step(IC<0>{}); step(IC<1>{}); step(IC<2>{}); step(IC<3>{});
      pr = quad_sum(pr) * g;
      pw = quad_sum(pw) * (g_prev * hs) * wsi;
      pk = quad_sum(pk) * hs;
      pb = quad_sum(pb) * hs;
      pa = quad_sum(pa) * g_prev;
      const int64_t o = base + static_cast<int64_t>(it * TT + tt) * stride + i;
      if (q == 0) {
        dr[o] = IoBF16::from_f32(pr);
        da[o] = IoBF16::from_f32(pa);
      } else if (q == 1) {
        dw[o] = IoBF16::from_f32(pw);
      } else if (q == 2) {
        dk[o] = IoBF16::from_f32(pk);
      } else {
        db[o] = IoBF16::from_f32(pb);
      }
      g = g_prev;
      ig *= wi;
      hs *= wi;
      ihs = ihs_prev;
      if (kRecompute && tt == kChunk / 2) {
        // S_7 from the forward rebuild: the backward walk rebuilds at most 8
        // steps through 1/w
#pragma unroll
        for (int e = 0; e < E; ++e) Sh[e] = Mid[e];
        g = ig = 1.0f;
      }
    }
    if (it > 0) store_tile(slot ^ 1);
    __syncthreads();
  }
}

// StateTune: the value pass ends with P at each sequence's first token t0
// (pfirst) but does not form dsa_t0 = P^T b_t0 (it writes zero there: with a
// zero initial state nothing reads it).  With a trainable initial state
// da_t0 = S_init dsa_t0 does, and dL/dS_init = diag(w_t0) P + a_t0 dsa_t0^T.
// One workgroup per (sequence, head), lane j = value column.
__global__ __launch_bounds__(64) void first_token_kernel(int T, int H, const uint16_t* wl,
                                                         const uint16_t* a, const uint16_t* b,
                                                         const float* pfirst, float* dsa,
                                                         float* dstate0) {
  constexpr int D = 64;
  const int bh = blockIdx.x, bidx = bh / H, h = bh % H, j = threadIdx.x;
  const int64_t row = (static_cast<int64_t>(bidx) * T * H + h) * D;   // token t0
  const float* P = pfirst + static_cast<int64_t>(bh) * D * D;
  float ds = 0.0f;
  for (int i = 0; i < D; ++i) ds = fmaf(P[i * D + j], IoBF16::to_f32(b[row + i]), ds);
  dsa[row + j] = ds;
  float* out = dstate0 + static_cast<int64_t>(bh) * D * D;
  for (int i = 0; i < D; ++i) {
    const float w = retention_from_logit(IoBF16::to_f32(wl[row + i]));
    out[i * D + j] = fmaf(w, P[i * D + j], IoBF16::to_f32(a[row + i]) * ds);
  }
}

template <int D>
int launch_d(const PretrainBwdArgs& p, hipStream_t s) {
  const auto* r = static_cast<const uint16_t*>(p.r);
  const auto* w = static_cast<const uint16_t*>(p.w);
  const auto* k = static_cast<const uint16_t*>(p.k);
  const auto* v = static_cast<const uint16_t*>(p.v);
  const auto* a = static_cast<const uint16_t*>(p.a);
  const auto* b = static_cast<const uint16_t*>(p.b);
  const auto* dy = static_cast<const uint16_t*>(p.dy);
  const int bh = p.batch * p.heads;
  if constexpr (D == 64) {
    // The value pass is the forward recurrence run backwards in time with
    // the roles (k, v, r, a, b, w) <- (r_t, dy_t, k_t, b_{t+1}, a_{t+1},
    // w_{t+1}): its state is P, its output dv and its sa the next token's
    // dsa.  At D = 64 it runs on the chunked MFMA kernel's reverse mode and
    // keeps P at the start of every span of chunks for the chunk-form key
    // pass (csrc/pretrain_bwd_chunk.hip).
    const int cps = key_chunk_span(p.batch, p.tokens, p.heads);
    const int nchunk = p.tokens / kChunk;
    const int nspan = (nchunk + cps - 1) / cps;
    float* pbnd = p.workspace + static_cast<int64_t>(p.batch) * p.tokens * p.heads * D;
    SegArgs v;
    v.uniform_len = p.tokens;
    v.num_heads = p.heads;
    v.out_elems = static_cast<int64_t>(p.batch) * p.tokens * p.heads * D;
    v.r = p.k;
    v.logits = p.w;
    v.k = p.r;
    v.v = p.dy;
    v.a = p.b;
    v.b = p.a;
    v.y = p.dv;
    v.sa_out = p.workspace;
    v.boundary = pbnd;
    v.boundary_len = kChunk;
    v.boundary_per_seg = nchunk;
    v.boundary_every = cps;
    v.reverse = true;
    v.shift_mask = (1 << 1) | (1 << 4) | (1 << 5);
    v.state_in = p.dfinal;     // P after the last token (StateTune), or zero
    v.kv_scale = p.scale;
    v.state_out = p.pfirst;    // P at token 0 (StateTune), or not written
    const int rc = launch_chunked(FR2_DTYPE_BFLOAT16, v, p.batch, p.tokens, s);
    if (rc != FR2_OK) return rc;
    if (p.pfirst != nullptr && p.dstate0 != nullptr)
      hipLaunchKernelGGL(first_token_kernel, dim3(bh), dim3(64), 0, s, p.tokens, p.heads, w, a, b,
                         p.pfirst, p.workspace, p.dstate0);
    return launch_key_chunk(p, pbnd, nspan, cps, s);
  } else {
    hipLaunchKernelGGL(value_kernel<D>, dim3(bh), dim3(4 * D), 0, s, p.tokens, p.heads, r, w, k,
                       a, b, dy, static_cast<uint16_t*>(p.dv), p.workspace);
  }
  hipLaunchKernelGGL(key_kernel<D>, dim3(bh * (D / 64)), dim3(256), 0, s, p.tokens, p.heads, r,
                     w, k, v, a, b, dy, p.boundary, p.state_dot_a, p.workspace,
                     static_cast<uint16_t*>(p.dr), static_cast<uint16_t*>(p.dw),
                     static_cast<uint16_t*>(p.dk), static_cast<uint16_t*>(p.db),
                     static_cast<uint16_t*>(p.da));
  return record_launch();
}

}  // namespace

int64_t pretrain_backward_workspace_floats(int B, int T, int H, int D) {
  int64_t n = static_cast<int64_t>(B) * T * H * D;
  if (D == 64) {
    const int cps = key_chunk_span(B, T, H);
    const int nspan = (T / kChunk + cps - 1) / cps;
    n += static_cast<int64_t>(B) * H * nspan * D * D;
  }
  return n;
}

int launch_pretrain_backward(int D, const PretrainBwdArgs& p, hipStream_t s) {
  switch (D) {
    case 64: return launch_d<64>(p, s);
    case 128: return launch_d<128>(p, s);
    case 256: return launch_d<256>(p, s);
    default: return FR2_ERR_UNSUPPORTED;
  }
}

}  // namespace fr2
