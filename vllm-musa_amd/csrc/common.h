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

// moe_align_block_size and the 1x128 fp8 quantiser of bf16 activations
// x [rows, cols] (into xq [rows, cols], xs [rows, cols / 128]) as one launch
// (align.hip).
int align_and_group_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                              int block_size, const int32_t* expert_map, int64_t expert_map_len,
                              int32_t* sorted, int64_t capacity, int32_t* expert_ids, int32_t* ntpp,
                              int32_t* offsets, int32_t* active, int32_t* num_active,
                              const void* x, int64_t rows, int64_t cols, uint8_t* xq, float* xs,
                              hipStream_t st);
// The same with the w4afp8 per-row quantiser (eps 1e-4): xs [rows]; xq in
// w4 order with the block corrections xcorr [rows, cols / 128] (cols a
// multiple of 128).
int align_and_row_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                            int block_size, const int32_t* expert_map, int64_t expert_map_len,
                            int32_t* sorted, int64_t capacity, int32_t* expert_ids, int32_t* ntpp,
                            int32_t* offsets, int32_t* active, int32_t* num_active, const void* x,
                            int64_t rows, int64_t cols, uint8_t* xq, float* xs, float* xcorr,
                            hipStream_t st);

// Top-k combine (moe_sum.hip): out[t] = round(sum_k x[t, k] (* wts[t, k])) over
// the live slots; num_experts > 0 also drops slots whose local id is >= it.
int moe_sum_impl(const char* who, const void* x, int dtype, int64_t tokens, int topk,
                 int64_t hidden, const int32_t* topk_ids, const int32_t* expert_map,
                 int64_t expert_map_len, int num_experts, const float* wts, void* out,
                 vmamd_stream_t stream);

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
// Cross-lane moves in DPP form (a VALU operand modifier: no LDS round trip).
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes
constexpr int kDppMirror = 0x140;      // lane i <-> 15 - i within each 16 lanes

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Value of lane `src` (wave-uniform) in every lane.  A readlane reads the
// lane's register whether or not that lane is still active, so the 32- and
// 64-lane forms below need every lane of the wave live.
__device__ __forceinline__ float lane_value(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ int lane_value(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

// Max over aligned groups of `W` lanes (W a power of two <= 64), every lane of
// a group ending with it.  Max is order-independent, so the first four steps
// pair lanes with DPP moves inside each 16-lane row (quad swaps, then the 8-
// and 16-lane mirrors) and wider groups merge the rows' results read with
// v_readlane -- no LDS round trip.
template <int W>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (W >= 2) v = fmaxf(v, dpp_f<kDppXor1>(v));
  if constexpr (W >= 4) v = fmaxf(v, dpp_f<kDppXor2>(v));
  if constexpr (W >= 8) v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  if constexpr (W >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
  if constexpr (W == 32) {
    const float lo = fmaxf(lane_value(v, 0), lane_value(v, 16));
    const float hi = fmaxf(lane_value(v, 32), lane_value(v, 48));
    v = __lane_id() < 32 ? lo : hi;
  }
  if constexpr (W == 64)
    v = fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
  return v;
}
__device__ __forceinline__ float wave_max(float v) { return group_max<kWave>(v); }
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}

// Merge (v, idx) with a partner's under the order (value desc, index asc).
__device__ __forceinline__ void argmax_merge(float& v, int& idx, float ov, int oi) {
  if (ov > v || (ov == v && oi < idx)) {
    v = ov;
    idx = oi;
  }
}

// Argmax over the wave with ties broken towards the lower index; every lane
// ends with the result (every lane of the wave must be active).  The merge is
// a maximum under a total order, so any pairing that joins disjoint lane sets
// works: quad swaps and the 8- and 16-lane mirrors run as DPP moves inside
// each 16-lane row, then the four rows' results are read with v_readlane and
// merged as wave-uniform values.
__device__ __forceinline__ void wave_argmax(float& v, int& idx) {
  argmax_merge(v, idx, dpp_f<kDppXor1>(v), dpp_i<kDppXor1>(idx));
  argmax_merge(v, idx, dpp_f<kDppXor2>(v), dpp_i<kDppXor2>(idx));
  argmax_merge(v, idx, dpp_f<kDppHalfMirror>(v), dpp_i<kDppHalfMirror>(idx));
  argmax_merge(v, idx, dpp_f<kDppMirror>(v), dpp_i<kDppMirror>(idx));
  float v0 = lane_value(v, 0), v1 = lane_value(v, 16), v2 = lane_value(v, 32), v3 = lane_value(v, 48);
  int i0 = lane_value(idx, 0), i1 = lane_value(idx, 16), i2 = lane_value(idx, 32), i3 = lane_value(idx, 48);
  argmax_merge(v0, i0, v1, i1);
  argmax_merge(v2, i2, v3, i3);
  argmax_merge(v0, i0, v2, i2);
  v = v0;
  idx = i0;
}

// Top-2 (t1 >= t2) of the union of two disjoint value sets.
__device__ __forceinline__ void top2_merge(float& t1, float& t2, float o1, float o2) {
  const float hi = fmaxf(t1, o1), lo = fminf(t1, o1);
  t2 = fmaxf(lo, fmaxf(t2, o2));
  t1 = hi;
}

// Top-2 over aligned groups of S lanes (S a power of two <= 64), every lane
// of a group ending with its group's (t1, t2); the top-2 of a set does not
// depend on the merge order, so rows of 16 merge by DPP and wider groups
// through v_readlane (every lane of the wave must be active).
template <int S>
__device__ __forceinline__ void group_top2(float& t1, float& t2) {
  if constexpr (S >= 2) top2_merge(t1, t2, dpp_f<kDppXor1>(t1), dpp_f<kDppXor1>(t2));
  if constexpr (S >= 4) top2_merge(t1, t2, dpp_f<kDppXor2>(t1), dpp_f<kDppXor2>(t2));
  if constexpr (S >= 8) top2_merge(t1, t2, dpp_f<kDppHalfMirror>(t1), dpp_f<kDppHalfMirror>(t2));
  if constexpr (S >= 16) top2_merge(t1, t2, dpp_f<kDppMirror>(t1), dpp_f<kDppMirror>(t2));
  if constexpr (S >= 32) {
    float r1[4], r2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      r1[r] = lane_value(t1, 16 * r);
      r2[r] = lane_value(t2, 16 * r);
    }
    top2_merge(r1[0], r2[0], r1[1], r2[1]);
    top2_merge(r1[2], r2[2], r1[3], r2[3]);
    if constexpr (S == 64) {
      top2_merge(r1[0], r2[0], r1[2], r2[2]);
      t1 = r1[0];
      t2 = r2[0];
    } else {
      const bool lo = __lane_id() < 32;
      t1 = lo ? r1[0] : r1[2];
      t2 = lo ? r2[0] : r2[2];
    }
  }
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }

__device__ __forceinline__ int lane_id() { return __lane_id(); }

}  // namespace vmamd
