// 1x128 activation quantisers and the SiLU-and-mul activation.
//
// Layout: one 128-element quant group is owned by 16 consecutive lanes, each
// holding 8 elements in registers (one 16-byte load for 2-byte types), so a
// wave64 quantises 4 groups and a 256-thread block 16 groups.  The group
// absmax is a 4-step xor-shuffle inside the 16-lane segment; scales and fp8
// bytes are written straight from registers (8 bytes per lane).
#include "quant_dev.h"

namespace vmamd {

// ----------------------------------------------------- group quantiser ---
template <int DT>
__global__ __launch_bounds__(kQuantThreads) void group_quant_fp8_kernel(
    const typename Elem<DT>::T* __restrict__ x, int64_t x_row_stride, int64_t groups_per_row,
    int64_t num_groups, bool vec, float eps, float qmin, float qmax, uint8_t* __restrict__ q,
    int64_t q_row_stride, float* __restrict__ s, int64_t s_stride_row, int64_t s_stride_group) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kLanesPerGroup;
  const int sub = threadIdx.x % kLanesPerGroup;
  if (g >= num_groups) return;
  group_quant_group<DT>(x, x_row_stride, groups_per_row, g, sub, vec, eps, qmin, qmax, q,
                        q_row_stride, s, s_stride_row, s_stride_group);
}

// -------------------------------------------------- SiLU and multiply -----
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

template <int DT>
__global__ __launch_bounds__(256) void silu_and_mul_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                           int64_t rows, int64_t d,
                                                           typename Elem<DT>::T* __restrict__ out) {
  const int64_t total = rows * d;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / d, c = i - r * d;
    const float g = Elem<DT>::load(x, r * 2 * d + c);
    const float u = Elem<DT>::load(x, r * 2 * d + d + c);
    out[i] = Elem<DT>::from_f(silu_f32(g) * u);
  }
}

// ------------------------------------------- SiLU-and-mul + quantiser ----
// value = round_T(silu(gate) * up) (CLAMP: with the reference's rounding of
// sigmoid, silu and product to T and the NaN -> fp8_min rule), then the 1x128
// quantiser on the rounded values.
template <int DT, bool CLAMP>
__global__ __launch_bounds__(kQuantThreads) void silu_mul_quant_fp8_kernel(
    const typename Elem<DT>::T* __restrict__ x, int64_t d, int64_t num_groups, float eps,
    float qmin, float qmax, float limit, uint8_t* __restrict__ q, float* __restrict__ s) {
  using E = Elem<DT>;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kGroupsPerBlock + threadIdx.x / kLanesPerGroup;
  const int sub = threadIdx.x % kLanesPerGroup;
  if (g >= num_groups) return;
  const int64_t groups_per_row = d / kGroup;
  const int64_t row = g / groups_per_row;
  const int64_t col = (g - row * groups_per_row) * kGroup + sub * kElemsPerLane;
  const typename E::T* gate_p = x + row * 2 * d + col;
  const typename E::T* up_p = gate_p + d;

  float v[8];
  bool to_min[8];
  float amax = eps;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float gate = E::load(gate_p, i);
    float up = E::load(up_p, i);
    float val;
    if constexpr (CLAMP) {
      const uint32_t gb = __float_as_uint(gate), ub = __float_as_uint(up);
      to_min[i] = ((gb & 0x7fffffffu) > 0x7f800000u) || gb == 0xff800000u ||
                  ((ub & 0x7fffffffu) > 0x7f800000u);
      const float L = E::to_f(E::from_f(limit));
      gate = gate > L ? L : gate;
      up = up < -L ? -L : (up > L ? L : up);
      const float sig = E::to_f(E::from_f(1.0f / (1.0f + expf(-gate))));
      const float silu = E::to_f(E::from_f(gate * sig));
      val = E::to_f(E::from_f(silu * up));
    } else {
      to_min[i] = false;
      val = E::to_f(E::from_f(silu_f32(gate) * up));
    }
    v[i] = val;
    amax = fmaxf(amax, fabsf(val));
  }
  amax = group_max<kLanesPerGroup>(amax);
  const float scale = amax / qmax;
  if (sub == 0) s[g] = scale;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    if (to_min[i]) v[i] = qmin * scale;  // quantises to exactly qmin
  *reinterpret_cast<uint2*>(q + row * d + col) = quant8(v, scale, qmin, qmax);
}



__global__ __launch_bounds__(kRowThreads) void row_quant_fp8_kernel(
    const uint16_t* __restrict__ x, int64_t x_row_stride, int cols, float eps, float qmin,
    float qmax, uint8_t* __restrict__ q, float* __restrict__ s) {
  __shared__ float red[kRowThreads / kWave];
  row_quant_part(x, x_row_stride, cols, eps, qmin, qmax, q, s, blockIdx.x, true, threadIdx.x, red);
}

}  // namespace vmamd

using namespace vmamd;

extern "C" int vmamd_per_token_group_quant_fp8(const void* x, int x_dtype, int64_t rows,
                                               int64_t cols, int64_t x_row_stride,
                                               int group_size, float eps, float fp8_min,
                                               float fp8_max, void* q, float* s,
                                               int64_t s_stride_row, int64_t s_stride_group,
                                               vmamd_stream_t stream) {
  VMAMD_REQUIRE(group_size == kGroup, "per_token_group_quant_fp8: group_size must be 128 (got %d)",
                group_size);
  VMAMD_REQUIRE(rows >= 0 && cols >= 0 && cols % kGroup == 0,
                "per_token_group_quant_fp8: cols (%lld) must be a multiple of 128",
                (long long)cols);
  VMAMD_REQUIRE(x_row_stride >= cols, "per_token_group_quant_fp8: row stride %lld < cols %lld",
                (long long)x_row_stride, (long long)cols);
  VMAMD_REQUIRE(fp8_max > 0.f, "per_token_group_quant_fp8: fp8_max must be positive");
  const int64_t groups_per_row = cols / kGroup;
  const int64_t num_groups = rows * groups_per_row;
  if (num_groups == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && q && s, "per_token_group_quant_fp8: null pointer");
  VMAMD_REQUIRE((reinterpret_cast<uintptr_t>(q) & 7) == 0,
                "per_token_group_quant_fp8: q must be 8-byte aligned");
  const int esize = x_dtype == kF32 ? 4 : 2;
  const bool vec = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && ((x_row_stride * esize) % 16 == 0);
  const int64_t blocks = (num_groups + kGroupsPerBlock - 1) / kGroupsPerBlock;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* qb = static_cast<uint8_t*>(q);
  switch (x_dtype) {
    case kBF16:
      group_quant_fp8_kernel<kBF16><<<blocks, kQuantThreads, 0, st>>>(
          static_cast<const uint16_t*>(x), x_row_stride, groups_per_row, num_groups, vec, eps,
          fp8_min, fp8_max, qb, cols, s, s_stride_row, s_stride_group);
      break;
    case kF16:
      group_quant_fp8_kernel<kF16><<<blocks, kQuantThreads, 0, st>>>(
          static_cast<const uint16_t*>(x), x_row_stride, groups_per_row, num_groups, vec, eps,
          fp8_min, fp8_max, qb, cols, s, s_stride_row, s_stride_group);
      break;
    case kF32:
      group_quant_fp8_kernel<kF32><<<blocks, kQuantThreads, 0, st>>>(
          static_cast<const float*>(x), x_row_stride, groups_per_row, num_groups, vec, eps,
          fp8_min, fp8_max, qb, cols, s, s_stride_row, s_stride_group);
      break;
    default:
      VMAMD_REQUIRE(false, "per_token_group_quant_fp8: unsupported dtype %d", x_dtype);
  }
  return check_launch("per_token_group_quant_fp8");
}

extern "C" int vmamd_silu_and_mul(const void* x, int dtype, int64_t rows, int64_t d, void* out,
                                  vmamd_stream_t stream) {
  VMAMD_REQUIRE(rows >= 0 && d >= 0, "silu_and_mul: negative size");
  if (rows * d == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && out, "silu_and_mul: null pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t total = rows * d;
  const int blocks = static_cast<int>(total / 256 + 1 < 65536 ? total / 256 + 1 : 65536);
  switch (dtype) {
    case kBF16:
      silu_and_mul_kernel<kBF16><<<blocks, 256, 0, st>>>(static_cast<const uint16_t*>(x), rows, d,
                                                         static_cast<uint16_t*>(out));
      break;
    case kF16:
      silu_and_mul_kernel<kF16><<<blocks, 256, 0, st>>>(static_cast<const uint16_t*>(x), rows, d,
                                                        static_cast<uint16_t*>(out));
      break;
    case kF32:
      silu_and_mul_kernel<kF32><<<blocks, 256, 0, st>>>(static_cast<const float*>(x), rows, d,
                                                        static_cast<float*>(out));
      break;
    default:
      VMAMD_REQUIRE(false, "silu_and_mul: unsupported dtype %d", dtype);
  }
  return check_launch("silu_and_mul");
}

extern "C" int vmamd_silu_and_mul_quant_fp8(const void* x, int dtype, int64_t rows, int64_t d,
                                            int group_size, float eps, float fp8_min,
                                            float fp8_max, float swiglu_limit, void* q, float* s,
                                            vmamd_stream_t stream) {
  VMAMD_REQUIRE(group_size == kGroup, "silu_and_mul_quant_fp8: group_size must be 128");
  VMAMD_REQUIRE(rows >= 0 && d >= 0 && d % kGroup == 0,
                "silu_and_mul_quant_fp8: d (%lld) must be a multiple of 128", (long long)d);
  VMAMD_REQUIRE(dtype == kBF16 || dtype == kF16, "silu_and_mul_quant_fp8: bf16/f16 input only");
  const int64_t num_groups = rows * (d / kGroup);
  if (num_groups == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && q && s, "silu_and_mul_quant_fp8: null pointer");
  VMAMD_REQUIRE((reinterpret_cast<uintptr_t>(q) & 7) == 0,
                "silu_and_mul_quant_fp8: q must be 8-byte aligned");
  const int64_t blocks = (num_groups + kGroupsPerBlock - 1) / kGroupsPerBlock;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool clamp = swiglu_limit > 0.f;
  const uint16_t* xi = static_cast<const uint16_t*>(x);
  uint8_t* qb = static_cast<uint8_t*>(q);
#define VMAMD_SMQ(DT, CL)                                                                    \
  silu_mul_quant_fp8_kernel<DT, CL><<<blocks, kQuantThreads, 0, st>>>(xi, d, num_groups, eps, \
                                                                      fp8_min, fp8_max,      \
                                                                      swiglu_limit, qb, s)
  if (dtype == kBF16) {
    if (clamp) VMAMD_SMQ(kBF16, true); else VMAMD_SMQ(kBF16, false);
  } else {
    if (clamp) VMAMD_SMQ(kF16, true); else VMAMD_SMQ(kF16, false);
  }
#undef VMAMD_SMQ
  return check_launch("silu_and_mul_quant_fp8");
}

extern "C" int vmamd_per_token_quant_fp8(const void* x, int64_t rows, int64_t cols,
                                         int64_t x_row_stride, float eps, float fp8_min,
                                         float fp8_max, void* q, float* s, vmamd_stream_t stream) {
  VMAMD_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= kRowThreads * 8 * kRowChunks,
                "per_token_quant_fp8: cols (%lld) must be a positive multiple of 8 up to %d",
                (long long)cols, kRowThreads * 8 * kRowChunks);
  VMAMD_REQUIRE(x_row_stride >= cols && x_row_stride % 8 == 0,
                "per_token_quant_fp8: row stride must be >= cols and a multiple of 8");
  VMAMD_REQUIRE(fp8_max > 0.f, "per_token_quant_fp8: fp8_max must be positive");
  VMAMD_REQUIRE(rows < (1ll << 31), "per_token_quant_fp8: too many rows");
  if (rows == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && q && s, "per_token_quant_fp8: null pointer");
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 8 == 0,
                "per_token_quant_fp8: x must be 16-byte and q 8-byte aligned");
  row_quant_fp8_kernel<<<static_cast<unsigned>(rows), kRowThreads, 0,
                         reinterpret_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(x), x_row_stride, static_cast<int>(cols), eps, fp8_min, fp8_max,
      static_cast<uint8_t*>(q), s);
  return check_launch("per_token_quant_fp8");
}
