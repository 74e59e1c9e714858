// Shared device helpers for the gfx950 WKV7 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fr2 {

// retention(x) = exp(-exp(-1/2) * sigmoid(x)), written with base-2
// exponentials: exp2(-exp(-1/2)*log2(e) / (1 + exp2(-log2(e) * x))).
// Same closed form as recurrent_retention in the reference
// (csrc/sm120/tmix/wkv7/recurrent_decay.cuh:18-22); the constants follow from
// the formula: exp(-1/2)*log2(e) = 0.87503877..., log2(e) = 1.44269504...
constexpr float kNegExpHalfLog2e = -0.8750387749145276f;
constexpr float kNegLog2e = -1.4426950408889634f;

__device__ __forceinline__ float retention_from_logit(float x) {
  const float e = __builtin_amdgcn_exp2f(kNegLog2e * x);
  return __builtin_amdgcn_exp2f(kNegExpHalfLog2e / (1.0f + e));
}

// ---- token I/O element types -------------------------------------------
struct IoBF16 {
  using raw = uint16_t;
  static __device__ __forceinline__ float to_f32(raw x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  // round to nearest even (v_cvt_pk_bf16_f32, one instruction); NaN stays
  // a quiet NaN.
  static __device__ __forceinline__ raw from_f32(float f) {
    return __builtin_bit_cast(raw, static_cast<__bf16>(f));
  }
};

struct IoF16 {
  using raw = _Float16;
  static __device__ __forceinline__ float to_f32(raw x) {
    return static_cast<float>(x);
  }
  static __device__ __forceinline__ raw from_f32(float f) {
    return static_cast<raw>(f);
  }
};

// ---- state element types -----------------------------------------------
struct StF32 {
  using raw = float;
  static __device__ __forceinline__ float to_f32(raw x) { return x; }
  static __device__ __forceinline__ raw from_f32(float f) { return f; }
};
struct StBF16 {
  using raw = uint16_t;
  static __device__ __forceinline__ float to_f32(raw x) {
    return IoBF16::to_f32(x);
  }
  static __device__ __forceinline__ raw from_f32(float f) {
    return IoBF16::from_f32(f);
  }
};

struct StF16 {
  using raw = _Float16;
  static __device__ __forceinline__ float to_f32(raw x) { return static_cast<float>(x); }
  static __device__ __forceinline__ raw from_f32(float f) { return static_cast<raw>(f); }
};

// FP16-state ("Albatross") contract, csrc/sm120/tmix/wkv7/recurrent_decay.cuh:36-46:
// the state update is state + state * delta with
//   delta = fp16(retention - 1 + dither(phase)),
//   dither(phase) = int32(0x9E3779B9 * phase mod 2^32) * 2^-41
// (a golden-ratio multiplicative hash scaled into (-2^-10, 2^-10)), and
// phase = elapsed[slot] + head * D + key + token offset in the sequence.
__device__ __forceinline__ float albatross_dither(int phase) {
  const uint32_t bits = 0x9E3779B9u * static_cast<uint32_t>(phase);
  return 4.547473508864641e-13f * static_cast<float>(static_cast<int32_t>(bits));
}
__device__ __forceinline__ float albatross_delta(float x, int phase) {
  const float d = retention_from_logit(x) - 1.0f + albatross_dither(phase);
  return static_cast<float>(static_cast<_Float16>(d));
}

// Native 4-wide float vector (usable with the nontemporal builtins).
typedef float f4 __attribute__((ext_vector_type(4)));

// 8 consecutive 16-bit token elements (one 16-byte global load).
struct alignas(16) Raw8 {
  uint16_t h[8];
};

template <class Io>
__device__ __forceinline__ float raw8_get(const Raw8& p, int i) {
  typename Io::raw x;
  __builtin_memcpy(&x, &p.h[i], 2);
  return Io::to_f32(x);
}

__device__ __forceinline__ float quiet_nan() { return __uint_as_float(0x7fc00000u); }

// Fail-closed fill: every output element becomes NaN (grid-stride over the
// whole output, shared by every workgroup of the launch).
template <class Io>
__device__ void fill_output_nan(typename Io::raw* out, int64_t n,
                                int64_t block, int64_t blocks) {
  const typename Io::raw nanv = Io::from_f32(quiet_nan());
  for (int64_t i = block * blockDim.x + threadIdx.x; i < n;
       i += blocks * blockDim.x) {
    out[i] = nanv;
  }
}

// Records the result of the launches just enqueued (hipGetLastError) and
// maps it to an fr2_status_t; the HIP error text stays readable through
// fr2_last_error() in the calling thread.
int record_launch();

// Sets the text fr2_last_error() reports in the calling thread (static
// storage only).
void set_last_error(const char* text);

}  // namespace fr2
