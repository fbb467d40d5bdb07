// fp32 router-gate GEMM: logits[M, E] = x[M, K] . W[E, K]^T in IEEE fp32.
//
// The router's top-k is decided on these logits, so the kernel fixes one
// summation order per logit, independent of M, of the tile shape and of the
// launch (batch invariant, run-to-run deterministic):
//   lane l (0..63) of a wave owns the K elements 2l + 128i + j (i = 0..K/128-1,
//   j = 0, 1) and runs ONE fused-multiply-add chain over them in that order,
//     p_l = fma(x[k_last], w[k_last], ... fma(x[k_0], w[k_0], +0));
//   the 64 partials are then summed by an xor butterfly,
//     p_l <- p_l + p_{l^s} for s = 32, 16, 8, 4, 2, 1,
//   after which every lane holds the logit.
// Reference: router_gate_fp32 / _router_gate_fp32_kernel
// (vllm_musa/model_executor/layers/fused_moe/router/musa_router_gemm.py:140-266),
// a Triton fp32 FMA GEMM for the [M, 2688] x [128, 2688]^T Nemotron-H gate.
//
// The op is latency bound at decode sizes (the [128, 2688] fp32 weight is
// 1.38 MB): one wave per (TM rows x TN experts) tile, K split over the 64
// lanes so every weight load instruction reads 512 contiguous bytes of a row,
// and TM x TN independent chains per lane to cover the FMA latency.  x rows
// beyond M are clamped for the load and never stored.
#include "common.h"

namespace vmamd {
namespace {

template <bool XBF16>
__device__ __forceinline__ float2 load_x2(const void* x, int64_t elem) {
  if constexpr (XBF16) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(x) + elem);
    return make_float2(__uint_as_float(v << 16), __uint_as_float(v & 0xffff0000u));
  } else {
    return *reinterpret_cast<const float2*>(static_cast<const float*>(x) + elem);
  }
}

template <int TM, int TN, bool XBF16>
__global__ __launch_bounds__(64) void router_gate_kernel(const void* __restrict__ x,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ y, int M, int K,
                                                         int E) {
  const int lane = threadIdx.x;
  const int m0 = blockIdx.x * TM, n0 = blockIdx.y * TN;
  const int kb = K / 128;
  int64_t xrow[TM];
#pragma unroll
  for (int a = 0; a < TM; ++a) xrow[a] = static_cast<int64_t>(min(m0 + a, M - 1)) * K + 2 * lane;
  const float* wrow[TN];
#pragma unroll
  for (int b = 0; b < TN; ++b) wrow[b] = w + static_cast<int64_t>(n0 + b) * K + 2 * lane;

  float acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = 0.f;

#pragma unroll 21
  for (int i = 0; i < kb; ++i) {
    float2 xv[TM], wv[TN];
#pragma unroll
    for (int a = 0; a < TM; ++a) xv[a] = load_x2<XBF16>(x, xrow[a] + 128 * i);
#pragma unroll
    for (int b = 0; b < TN; ++b) wv[b] = *reinterpret_cast<const float2*>(wrow[b] + 128 * i);
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b) {
        acc[a][b] = __builtin_fmaf(xv[a].x, wv[b].x, acc[a][b]);
        acc[a][b] = __builtin_fmaf(xv[a].y, wv[b].y, acc[a][b]);
      }
  }

#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      float v = acc[a][b];
#pragma unroll
      for (int s = 32; s >= 1; s >>= 1) v = v + __shfl_xor(v, s, 64);
      if (lane == a * TN + b && m0 + a < M) y[static_cast<int64_t>(m0 + a) * E + n0 + b] = v;
    }
}

template <int TM, int TN, bool XBF16>
void launch_tile(const void* x, const float* w, float* y, int M, int K, int E, hipStream_t st) {
  const dim3 grid((M + TM - 1) / TM, E / TN);
  router_gate_kernel<TM, TN, XBF16><<<grid, 64, 0, st>>>(x, w, y, M, K, E);
}

template <bool XBF16>
void launch_router_gate(const void* x, const float* w, float* y, int M, int K, int E,
                        hipStream_t st) {
  // Tile shapes only change which wave computes a logit, never how.  Chosen by
  // a sweep at K = 2688, E = 128 on MI355X: one logit per wave while waves are
  // scarce, then taller tiles as M grows (the VALU issue rate bounds M >= 256).
  const bool even = E % 2 == 0;
  if (M <= 16)
    launch_tile<1, 1, XBF16>(x, w, y, M, K, E, st);
  else if (M <= 48 || !even)
    launch_tile<4, 1, XBF16>(x, w, y, M, K, E, st);
  else if (M <= 160)
    launch_tile<4, 2, XBF16>(x, w, y, M, K, E, st);
  else
    launch_tile<8, 2, XBF16>(x, w, y, M, K, E, st);
}

}  // namespace
}  // namespace vmamd

using namespace vmamd;

extern "C" int vmamd_router_gate_fp32(const void* x, int x_dtype, int64_t M, int64_t K,
                                      const float* w, int64_t E, float* y,
                                      vmamd_stream_t stream) {
  const char* who = "router_gate_fp32";
  VMAMD_REQUIRE(M >= 0 && K > 0 && E > 0, "%s: bad sizes M=%lld K=%lld E=%lld", who,
                static_cast<long long>(M), static_cast<long long>(K), static_cast<long long>(E));
  VMAMD_REQUIRE(K % 128 == 0, "%s: K=%lld must be a multiple of 128", who,
                static_cast<long long>(K));
  VMAMD_REQUIRE(M <= (1 << 30) && K <= (1 << 24) && E <= 65535, "%s: sizes out of range",
                who);
  VMAMD_REQUIRE(x_dtype == kF32 || x_dtype == kBF16, "%s: x must be f32 or bf16", who);
  if (M == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && w && y, "%s: null pointer", who);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(x) % (x_dtype == kF32 ? 8 : 4) == 0 &&
                    reinterpret_cast<uintptr_t>(w) % 8 == 0,
                "%s: x and w must be aligned to an element pair", who);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == kBF16)
    launch_router_gate<true>(x, w, y, static_cast<int>(M), static_cast<int>(K),
                             static_cast<int>(E), st);
  else
    launch_router_gate<false>(x, w, y, static_cast<int>(M), static_cast<int>(K),
                              static_cast<int>(E), st);
  return check_launch(who);
}
