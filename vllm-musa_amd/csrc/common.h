// Shared device helpers for the gfx950 MoE / block-fp8 kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, OCP
// e4m3fn fp8 conversions in hardware, and the f8f6f4 / bf16 MFMA builtins.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vllm_musa_amd.h"

namespace vmamd {

constexpr int kWave = 64;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------- errors ---
// Host-side error reporting for the C ABI: each entry point returns a status
// code and leaves a message retrievable with vmamd_last_error().
void set_error(const char* fmt, ...);
int check_launch(const char* what);

#define VMAMD_REQUIRE(cond, ...)                \
  do {                                          \
    if (!(cond)) {                              \
      ::vmamd::set_error(__VA_ARGS__);          \
      return VMAMD_ERR_INVALID;                 \
    }                                           \
  } while (0)

// ------------------------------------------------------- scalar convert ---
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even float -> bf16 bits; NaN maps to the canonical quiet
// NaN 0x7fc0 (the same rule torch uses on the CPU).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Activation element types understood by the kernels.
enum DType : int { kF32 = VMAMD_DTYPE_F32, kF16 = VMAMD_DTYPE_F16, kBF16 = VMAMD_DTYPE_BF16 };

template <int DT> struct Elem;
template <> struct Elem<kBF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ float to_f(T v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ T from_f(float f) { return f32_to_bf16(f); }
};
template <> struct Elem<kF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return f16_to_f32(p[i]); }
  static __device__ __forceinline__ float to_f(T v) { return f16_to_f32(v); }
  static __device__ __forceinline__ T from_f(float f) { return f32_to_f16(f); }
};
template <> struct Elem<kF32> {
  using T = float;
  static __device__ __forceinline__ float load(const T* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ float to_f(T v) { return v; }
  static __device__ __forceinline__ T from_f(float f) { return f; }
};

// ---------------------------------------------------------------- fp8 -----
// OCP e4m3fn conversion in hardware (v_cvt_pk_fp8_f32): round to nearest
// even.  Callers clamp to [-448, 448] first, so saturation never triggers.
__device__ __forceinline__ uint32_t f32x2_to_fp8x2(float a, float b) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false)) & 0xffffu;
}
__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}
__device__ __forceinline__ float fp8_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(byte), 0);
}

// ----------------------------------------------------------- wave utils ---
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
// Max over aligned groups of `W` lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = W / 2; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Argmax over the wave with ties broken towards the lower index.
__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    float ov = __shfl_xor(v, m, kWave);
    int oi = __shfl_xor(idx, m, kWave);
    if (ov > v || (ov == v && oi < idx)) {
      v = ov;
      idx = oi;
    }
  }
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace vmamd
