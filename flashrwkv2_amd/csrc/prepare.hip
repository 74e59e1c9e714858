// The WKV7 path's producer and consumer elementwise stages (fp16 I/O, fp32
// arithmetic), around the library GEMMs of the layer:
//   - kk / a gate  (csrc/sm120/tmix/wkv_prepare/internal/kk_a_gate/
//     infer_fp16_forward_varlen.cu): per (token, head)
//       u = k * k_k,  kk = u / max(|u|, 1e-12),  a = sigmoid(a0 + a12),
//       new_k = k * (1 + (a - 1) * k_a),  neg_kk = -kk,  kka = kk * a
//     i.e. the key and the recurrence's a = -kk, b = kk * a operands;
//   - low-rank activations (…/internal/lowrank/infer_fp16_forward_varlen.cu:
//     46-71, 864-865): tanh of the decay branch, sigmoid of the gate branch;
//   - value residual (…/internal/lowrank/infer_vres_fp16_forward_varlen.cu):
//       value + (v_first - value) * sigmoid(v0 + v12);
//   - readout prelinear (csrc/sm120/tmix/readout/infer_fp16_forward_varlen.cu):
//     per (token, head) group norm of the WKV output (eps 64e-5), the
//     r.k.r_k residual times v, and the output gate:
//       (norm(x) * ln_w + ln_b + sum(r * k * r_k) * v) * g.
// All are HBM-bound: each thread moves 8 consecutive fp16 values (16-byte
// accesses); a (token, head) group of D values is D/8 consecutive lanes, so
// its reductions are butterflies over those lanes.
#include "recurrent.h"

#include <math.h>

namespace fr2 {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr float kKkEps = 1.0e-12f;
constexpr float kLnEps = 64.0e-5f;

struct H8 {
  float f[8];
};

__device__ __forceinline__ H8 load8(const _Float16* p) {
  const u32x4 u = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  H8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t w = u[i];
    r.f[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
    r.f[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
  return r;
}

__device__ __forceinline__ void store8(_Float16* p, const float* f) {
  u32x4 u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f[2 * i]));
    const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(f[2 * i + 1]));
    u[i] = lo | (hi << 16);
  }
  __builtin_nontemporal_store(u, reinterpret_cast<u32x4*>(p));
}

// sum over the G consecutive lanes of a group (G a power of two <= 64)
template <int G>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
  for (int m = 1; m < G; m <<= 1) x += __shfl_xor(x, m, G);
  return x;
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

template <int D>
__global__ __launch_bounds__(kThreads) void kk_a_gate_kernel(
    int64_t groups, int H, const _Float16* __restrict__ k, const _Float16* __restrict__ k_k,
    const _Float16* __restrict__ a0, const _Float16* __restrict__ a12,
    const _Float16* __restrict__ k_a, _Float16* __restrict__ new_k,
    _Float16* __restrict__ neg_kk, _Float16* __restrict__ kka) {
  constexpr int G = D / 8;   // lanes per (token, head)
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t grp = gid / G;
  const int part = static_cast<int>(gid % G);
  const bool valid = grp < groups;
  const int64_t idx = grp * D + part * 8;
  const int c = static_cast<int>(grp % H) * D + part * 8;
  H8 kv{}, sc{};
  float u[8], ss = 0.0f;
  if (valid) {
    kv = load8(k + idx);
    sc = load8(k_k + c);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    u[e] = kv.f[e] * sc.f[e];
    ss = fmaf(u[e], u[e], ss);
  }
  ss = group_sum<G>(ss);
  if (!valid) return;
  const float inv = 1.0f / fmaxf(sqrtf(ss), kKkEps);
  const H8 b0 = load8(a0 + c), d12 = load8(a12 + idx), ka = load8(k_a + c);
  float o_k[8], o_n[8], o_b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float kk = u[e] * inv;
    const float av = sigmoid(b0.f[e] + d12.f[e]);
    o_k[e] = kv.f[e] * fmaf(av, ka.f[e], 1.0f - ka.f[e]);
    o_n[e] = -kk;
    o_b[e] = kk * av;
  }
  store8(new_k + idx, o_k);
  store8(neg_kk + idx, o_n);
  store8(kka + idx, o_b);
}

// tanh over [0, n_t) of the first tensor, sigmoid over [0, n_s) of the
// second; units of 8 values, scalar tail.
__global__ __launch_bounds__(kThreads) void lowrank_act_kernel(
    int64_t n_t, const _Float16* __restrict__ xt, _Float16* __restrict__ yt, int64_t n_s,
    const _Float16* __restrict__ xs, _Float16* __restrict__ ys) {
  const int64_t ut = (n_t + 7) / 8, us = (n_s + 7) / 8;
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= ut + us) return;
  const bool is_t = u < ut;
  const int64_t base = (is_t ? u : u - ut) * 8;
  const int64_t n = is_t ? n_t : n_s;
  const _Float16* x = is_t ? xt : xs;
  _Float16* y = is_t ? yt : ys;
  if (base + 8 <= n) {
    const H8 v = load8(x + base);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = is_t ? tanhf(v.f[e]) : sigmoid(v.f[e]);
    store8(y + base, o);
  } else {
    for (int64_t i = base; i < n; ++i) {
      const float v = static_cast<float>(x[i]);
      y[i] = static_cast<_Float16>(is_t ? tanhf(v) : sigmoid(v));
    }
  }
}

// value + (v_first - value) * sigmoid(v0 + v12) over [tokens, C], C % 8 == 0
__global__ __launch_bounds__(kThreads) void vres_kernel(
    int64_t units, int C, const _Float16* __restrict__ value,
    const _Float16* __restrict__ v_first, const _Float16* __restrict__ v0,
    const _Float16* __restrict__ v12, _Float16* __restrict__ out) {
  const int64_t u = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (u >= units) return;
  const int64_t idx = u * 8;
  const int c = static_cast<int>(idx % C);
  const H8 cur = load8(value + idx), first = load8(v_first + idx), base = load8(v0 + c),
           d = load8(v12 + idx);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    o[e] = fmaf(first.f[e] - cur.f[e], sigmoid(base.f[e] + d.f[e]), cur.f[e]);
  store8(out + idx, o);
}

template <int D>
__global__ __launch_bounds__(kThreads) void readout_prelinear_kernel(
    int64_t groups, int H, const _Float16* __restrict__ x, const _Float16* __restrict__ r,
    const _Float16* __restrict__ k, const _Float16* __restrict__ v,
    const _Float16* __restrict__ r_k, const _Float16* __restrict__ ln_w,
    const _Float16* __restrict__ ln_b, const _Float16* __restrict__ g,
    _Float16* __restrict__ out) {
  constexpr int G = D / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const int64_t grp = gid / G;
  const int part = static_cast<int>(gid % G);
  const bool valid = grp < groups;
  const int64_t idx = grp * D + part * 8;
  const int c = static_cast<int>(grp % H) * D + part * 8;
  H8 xv{}, rv{}, kv{}, rk{};
  if (valid) {
    xv = load8(x + idx);
    rv = load8(r + idx);
    kv = load8(k + idx);
    rk = load8(r_k + c);
  }
  float sx = 0.0f, rkv = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sx += xv.f[e];
    rkv = fmaf(rv.f[e] * kv.f[e], rk.f[e], rkv);
  }
  const float mean = group_sum<G>(sx) * (1.0f / D);
  float sd = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float d = xv.f[e] - mean;
    sd = fmaf(d, d, sd);
  }
  const float rstd = rsqrtf(group_sum<G>(sd) * (1.0f / D) + kLnEps);
  rkv = group_sum<G>(rkv);
  if (!valid) return;
  const H8 vv = load8(v + idx), gv = load8(g + idx), w = load8(ln_w + c), b = load8(ln_b + c);
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e)
    o[e] = (fmaf((xv.f[e] - mean) * rstd, w.f[e], b.f[e]) + rkv * vv.f[e]) * gv.f[e];
  store8(out + idx, o);
}

inline unsigned blocks_for(int64_t threads) {
  return static_cast<unsigned>((threads + kThreads - 1) / kThreads);
}

}  // namespace

int launch_kk_a_gate(int64_t tokens, int H, int D, const void* k, const void* k_k, const void* a0,
                     const void* a12, const void* k_a, void* new_k, void* neg_kk, void* kka,
                     hipStream_t s) {
  const int64_t groups = tokens * H;
  const auto* K = static_cast<const _Float16*>(k);
  const auto* KK = static_cast<const _Float16*>(k_k);
  const auto* A0 = static_cast<const _Float16*>(a0);
  const auto* A12 = static_cast<const _Float16*>(a12);
  const auto* KA = static_cast<const _Float16*>(k_a);
  auto* NK = static_cast<_Float16*>(new_k);
  auto* NN = static_cast<_Float16*>(neg_kk);
  auto* KB = static_cast<_Float16*>(kka);
  const unsigned blocks = blocks_for(groups * (D / 8));
  switch (D) {
    case 64:
      hipLaunchKernelGGL(kk_a_gate_kernel<64>, dim3(blocks), dim3(kThreads), 0, s, groups, H, K, KK,
                         A0, A12, KA, NK, NN, KB);
      break;
    case 128:
      hipLaunchKernelGGL(kk_a_gate_kernel<128>, dim3(blocks), dim3(kThreads), 0, s, groups, H, K,
                         KK, A0, A12, KA, NK, NN, KB);
      break;
    case 256:
      hipLaunchKernelGGL(kk_a_gate_kernel<256>, dim3(blocks), dim3(kThreads), 0, s, groups, H, K,
                         KK, A0, A12, KA, NK, NN, KB);
      break;
    default:
      return FR2_ERR_UNSUPPORTED;
  }
  return record_launch();
}

int launch_lowrank_act(int64_t n_t, const void* xt, void* yt, int64_t n_s, const void* xs, void* ys,
                       hipStream_t s) {
  const int64_t units = (n_t + 7) / 8 + (n_s + 7) / 8;
  if (units == 0) return FR2_OK;
  hipLaunchKernelGGL(lowrank_act_kernel, dim3(blocks_for(units)), dim3(kThreads), 0, s, n_t,
                     static_cast<const _Float16*>(xt), static_cast<_Float16*>(yt), n_s,
                     static_cast<const _Float16*>(xs), static_cast<_Float16*>(ys));
  return record_launch();
}

int launch_vres(int64_t tokens, int C, const void* value, const void* v_first, const void* v0,
                const void* v12, void* out, hipStream_t s) {
  const int64_t units = tokens * C / 8;
  hipLaunchKernelGGL(vres_kernel, dim3(blocks_for(units)), dim3(kThreads), 0, s, units, C,
                     static_cast<const _Float16*>(value), static_cast<const _Float16*>(v_first),
                     static_cast<const _Float16*>(v0), static_cast<const _Float16*>(v12),
                     static_cast<_Float16*>(out));
  return record_launch();
}

int launch_readout_prelinear(int64_t tokens, int H, int D, const void* x, const void* r,
                             const void* k, const void* v, const void* r_k, const void* ln_w,
                             const void* ln_b, const void* g, void* out, hipStream_t s) {
  const int64_t groups = tokens * H;
  const unsigned blocks = blocks_for(groups * (D / 8));
#define FR2_READOUT(DD)                                                                        \
  hipLaunchKernelGGL(readout_prelinear_kernel<DD>, dim3(blocks), dim3(kThreads), 0, s, groups, H, \
                     static_cast<const _Float16*>(x), static_cast<const _Float16*>(r),           \
                     static_cast<const _Float16*>(k), static_cast<const _Float16*>(v),           \
                     static_cast<const _Float16*>(r_k), static_cast<const _Float16*>(ln_w),      \
                     static_cast<const _Float16*>(ln_b), static_cast<const _Float16*>(g),        \
                     static_cast<_Float16*>(out))
  switch (D) {
    case 64: FR2_READOUT(64); break;
    case 128: FR2_READOUT(128); break;
    case 256: FR2_READOUT(256); break;
    default: return FR2_ERR_UNSUPPORTED;
  }
#undef FR2_READOUT
  return record_launch();
}

}  // namespace fr2
