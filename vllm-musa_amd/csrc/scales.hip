// Checkpoint scale-tensor conversion (load time, HBM-bound byte work).
//
// Weight scales come off disk in one of three encodings and the GEMMs want
// another:
//   e8m0 -> f32   an unsigned byte b is the float whose exponent field is b
//                 and whose mantissa is zero: bits = b << 23 (b = 0 gives
//                 +0.0, b = 255 gives +inf).  Reference: _upcast_e8m0_to_fp32
//                 (vllm_musa/model_executor/layers/quantization/utils/fp8_utils.py:13-15),
//                 also deepseek_v4_jit/fp8_einsum.py:54-57.
//   f32  -> bf16  round to nearest even, NaN -> 0x7fc0 (torch's .to(bfloat16)),
//                 used for the W4AFP8 group-128 expert scales
//                 (model_executor/layers/quantization/w4afp8.py:126-135).
//   plus the identity and widening pairs among {e8m0, f32, bf16} -> {f32, bf16}.
// Optionally the kernel counts destination values that are not finite and
// positive, the check the W4AFP8 loader applies after its bf16 cast
// (w4afp8.py:128-130); only lanes that find such a value touch the counter.
//
// Each lane handles 8 consecutive elements with one wide load and one wide
// store when both buffers are 16-byte aligned (the e8m0 -> f32 case reads 8 B
// and writes 32 B per lane), otherwise one element per lane; the grid strides
// over the tensor.
#include <float.h>

#include "common.h"

namespace vmamd {
namespace {

constexpr int kE8M0 = VMAMD_DTYPE_E8M0;

template <int DT> struct ScaleIn;
template <> struct ScaleIn<kE8M0> {
  using T = uint8_t;
  static __device__ __forceinline__ float to_f(T b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 23);
  }
};
template <> struct ScaleIn<kF32> {
  using T = float;
  static __device__ __forceinline__ float to_f(T v) { return v; }
};
template <> struct ScaleIn<kBF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float to_f(T h) { return bf16_to_f32(h); }
};

template <int DT> struct ScaleOut;
template <> struct ScaleOut<kF32> {
  using T = float;
  static __device__ __forceinline__ T from_f(float v) { return v; }
  static __device__ __forceinline__ float value(T v) { return v; }
};
template <> struct ScaleOut<kBF16> {
  using T = uint16_t;
  static __device__ __forceinline__ T from_f(float v) { return f32_to_bf16(v); }
  static __device__ __forceinline__ float value(T h) { return bf16_to_f32(h); }
};

template <typename T, int N>
struct alignas(N * sizeof(T) >= 16 ? 16 : N * sizeof(T)) Pack {
  T v[N];
};

__device__ __forceinline__ int scale_invalid(float v) { return !(v > 0.f && v <= FLT_MAX); }

template <int SRC, int DST, int VEC>
__global__ __launch_bounds__(256) void convert_scales_kernel(
    const typename ScaleIn<SRC>::T* __restrict__ src, int64_t n,
    typename ScaleOut<DST>::T* __restrict__ dst, int32_t* __restrict__ invalid) {
  using In = ScaleIn<SRC>;
  using Out = ScaleOut<DST>;
  using PI = Pack<typename In::T, VEC>;
  using PO = Pack<typename Out::T, VEC>;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x * VEC;
  int bad = 0;
  int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * VEC;
  for (; i + VEC <= n; i += stride) {
    const PI p = *reinterpret_cast<const PI*>(src + i);
    PO o;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      o.v[j] = Out::from_f(In::to_f(p.v[j]));
      bad += scale_invalid(Out::value(o.v[j]));
    }
    *reinterpret_cast<PO*>(dst + i) = o;
  }
  if (VEC > 1 && i < n) {  // the one lane that owns the ragged tail
    for (int64_t j = i; j < n; ++j) {
      const typename Out::T o = Out::from_f(In::to_f(src[j]));
      dst[j] = o;
      bad += scale_invalid(Out::value(o));
    }
  }
  if (invalid && bad) atomicAdd(invalid, bad);
}

int elem_size(int dt) {
  switch (dt) {
    case kE8M0: return 1;
    case kBF16: return 2;
    case kF32: return 4;
    default: return 0;
  }
}

template <int SRC, int DST>
void launch_convert(const void* src, int64_t n, void* dst, int32_t* invalid, bool vec,
                    hipStream_t st) {
  using SI = typename ScaleIn<SRC>::T;
  using SO = typename ScaleOut<DST>::T;
  const int vw = vec ? 8 : 1;
  const int64_t lanes = (n + vw - 1) / vw;
  const int64_t want = (lanes + 255) / 256;
  const int blocks = static_cast<int>(want < 8192 ? want : 8192);
  const SI* s = static_cast<const SI*>(src);
  SO* d = static_cast<SO*>(dst);
  if (vec)
    convert_scales_kernel<SRC, DST, 8><<<blocks, 256, 0, st>>>(s, n, d, invalid);
  else
    convert_scales_kernel<SRC, DST, 1><<<blocks, 256, 0, st>>>(s, n, d, invalid);
}

}  // namespace
}  // namespace vmamd

using namespace vmamd;

extern "C" int vmamd_convert_scales(const void* src, int src_dtype, int64_t n, void* dst,
                                    int dst_dtype, int32_t* invalid_count,
                                    vmamd_stream_t stream) {
  const char* who = "convert_scales";
  VMAMD_REQUIRE(n >= 0, "%s: negative element count", who);
  const int ss = elem_size(src_dtype);
  VMAMD_REQUIRE(ss != 0, "%s: unsupported source dtype %d", who, src_dtype);
  VMAMD_REQUIRE(dst_dtype == kF32 || dst_dtype == kBF16,
                "%s: unsupported destination dtype %d", who, dst_dtype);
  if (n == 0) return VMAMD_OK;
  VMAMD_REQUIRE(src && dst, "%s: null pointer", who);
  const int ds = elem_size(dst_dtype);
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  const uintptr_t s1 = s0 + static_cast<uintptr_t>(n) * ss, d1 = d0 + static_cast<uintptr_t>(n) * ds;
  // In place is fine element for element; any other overlap would race.
  VMAMD_REQUIRE((s0 == d0 && ss == ds) || s1 <= d0 || d1 <= s0,
                "%s: source and destination overlap", who);
  const bool vec = s0 % 16 == 0 && d0 % 16 == 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define VMAMD_CONV(S, D) launch_convert<S, D>(src, n, dst, invalid_count, vec, st)
  switch (src_dtype * 16 + dst_dtype) {
    case kE8M0 * 16 + kF32: VMAMD_CONV(kE8M0, kF32); break;
    case kE8M0 * 16 + kBF16: VMAMD_CONV(kE8M0, kBF16); break;
    case kF32 * 16 + kF32: VMAMD_CONV(kF32, kF32); break;
    case kF32 * 16 + kBF16: VMAMD_CONV(kF32, kBF16); break;
    case kBF16 * 16 + kF32: VMAMD_CONV(kBF16, kF32); break;
    case kBF16 * 16 + kBF16: VMAMD_CONV(kBF16, kBF16); break;
    default: VMAMD_REQUIRE(false, "%s: unsupported dtype pair %d -> %d", who, src_dtype, dst_dtype);
  }
#undef VMAMD_CONV
  return check_launch(who);
}
