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

typedef int v16i __attribute__((ext_vector_type(16)));
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
// Transposed copies of the w4afp8 weight scales for the grouped GEMMs:
// in[m] = bf16 [E, n[m], 2 kp[m]] read as 32-bit words [E, n[m], kp[m]]
// (kp[m] even), out[m] = [E, kp[m], n[m]] (m = 0: W13, 1: W2; null in[m]:
// none).
struct W4ScalesT {
  const uint32_t* in[2];
  uint32_t* out[2];
  int n[2], kp[2];
  int E;
};
// The same with the w4afp8 per-row quantiser (eps 1e-4): xs [rows]; xq in
// w4 order with the block corrections xcorr [rows, cols / 128] (cols a
// multiple of 128); sct: also the scale transpositions (null: none).
int align_and_row_quant_fp8(const int32_t* topk_ids, int64_t numel, int num_experts,
                            int block_size, const int32_t* expert_map, int64_t expert_map_len,
                            int32_t* sorted, int64_t capacity, int32_t* expert_ids, int32_t* ntpp,
                            int32_t* offsets, int32_t* active, int32_t* num_active, const void* x,
                            int64_t rows, int64_t cols, uint8_t* xq, float* xs, float* xcorr,
                            hipStream_t st, const W4ScalesT* sct = nullptr);
// moe_align_block_size alone; with counts (align_counts_bytes of scratch)
// in two launches, the chunk histograms then the placement, instead of every
// workgroup histogramming all routes.
int align_routes(const int32_t* topk_ids, int64_t numel, int num_experts, int block_size,
                 const int32_t* expert_map, int64_t expert_map_len, int32_t* sorted, int64_t capacity,
                 int32_t* expert_ids, int32_t* ntpp, int32_t* offsets, int32_t* active, int32_t* num_active,
                 int32_t* counts, hipStream_t st);
// Bytes of the chunk-histogram scratch for numel routes over E experts.
size_t align_counts_bytes(int64_t numel, int E);

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
// NaN 0x7fc0 (the same rule torch uses on the CPU).  v_cvt_pk_bf16_f32 after
// replacing a NaN by 0x7fc00000: equal to the integer form (add 0x7fff plus
// the lowest kept bit, keep the top half; NaN -> 0x7fc0) on all 2^32 inputs,
// checked exhaustively on an MI355X.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const float g = f != f ? __uint_as_float(0x7fc00000u) : f;
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(g));
}
// Two at once (a in the low half): one conversion instruction for both.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const float qn = __uint_as_float(0x7fc00000u);
  const f32x2_t v = {a != a ? qn : a, b != b ? qn : b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
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

// x / s rounded once, as the IEEE division, from r = 1 / s (an IEEE
// division) for a positive normal s: q = x r, then one correction with the
// exact remainder x - q s (an FMA).  With r the correctly rounded reciprocal
// and q within an ulp of x / s, q + (x - q s) r rounded once is the
// correctly rounded quotient (Markstein's theorem; checked exactly against
// x / s on 290,000 quotients, half of them next to e4m3 rounding midpoints,
// and by every quantiser test against the oracle).  Below the normal range
// the last place may differ, far below what an fp8 code resolves.  Zero
// keeps x's sign, as the division does; a NaN x gives NaN.  An infinite x
// makes its group's s infinite, which the callers divide as before.
__device__ __forceinline__ float div_rn(float x, float s, float r) {
  const float q = x * r;
  const float e = __builtin_fmaf(-q, s, x);
  return __builtin_copysignf(__builtin_fmaf(e, r, q), x);
}

// e4m3 codes of clamp(x / s, -448, 448) for four values sharing s, r = 1 / s
// (NaN: -448, the reference's fp8_min).
__device__ __forceinline__ uint32_t quant4_e4m3(const float (&x)[4], float s, float r) {
  float o[4];
  if (s < __builtin_inff()) {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = x[i] != x[i] ? -448.0f : fminf(fmaxf(div_rn(x[i], s, r), -448.0f), 448.0f);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = x[i] != x[i] ? -448.0f : fminf(fmaxf(x[i] / s, -448.0f), 448.0f);
  }
  return f32x4_to_fp8x4(o[0], o[1], o[2], o[3]);
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

// (value, index) as one unsigned key under the order (value desc, index
// asc): the high word is the float's bits made monotonic as an unsigned
// integer (-0 taken as +0, NaN below every number), the low word the inverted
// index (0 <= index < 2^31).  Key 0 lies below every entry.
__device__ __forceinline__ uint64_t argmax_key(float v, int idx) {
  const uint32_t b = __float_as_uint(v + 0.0f);
  uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  if (v != v) o = 1u;
  return (static_cast<uint64_t>(o) << 32) | static_cast<uint32_t>(~idx);
}
__device__ __forceinline__ float argmax_key_value(uint64_t k) {
  const uint32_t o = static_cast<uint32_t>(k >> 32);
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}
__device__ __forceinline__ int argmax_key_index(uint64_t k) { return static_cast<int>(~static_cast<uint32_t>(k)); }
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

constexpr int kDppBcast15 = 0x142;  // lane 15 of each row to the next row
constexpr int kDppBcast31 = 0x143;  // lane 31 to rows 2 and 3
// DPP move of a 64-bit value; rows outside ROWS keep their own value.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const int lo = static_cast<int>(static_cast<uint32_t>(v)), hi = static_cast<int>(v >> 32);
  const uint32_t l = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROWS, 0xF, false));
  const uint32_t h = static_cast<uint32_t>(__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROWS, 0xF, false));
  return (static_cast<uint64_t>(h) << 32) | l;
}

// Maximum key over the wave, in every lane (every lane must be active):
// quad swaps and the 8- and 16-lane mirrors leave each 16-lane row's maximum
// in all its lanes, the row broadcasts carry rows 0-2 into row 3, and lane
// 63 is read out.  Branch-free: one 64-bit compare and two selects a level.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
  k = max_u64(k, dpp_u64<kDppXor1>(k));
  k = max_u64(k, dpp_u64<kDppXor2>(k));
  k = max_u64(k, dpp_u64<kDppHalfMirror>(k));
  k = max_u64(k, dpp_u64<kDppMirror>(k));
  k = max_u64(k, dpp_u64<kDppBcast15, 0xA>(k));
  k = max_u64(k, dpp_u64<kDppBcast31, 0xC>(k));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(k)), 63));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(k >> 32), 63));
  return (static_cast<uint64_t>(hi) << 32) | lo;
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
