// Top-k combine: out[t, h] = round(sum_k x[t, k, h] (* w[t, k])), fp32
// accumulation in slot order k = 0, 1, ..., one rounding to the output dtype;
// the routed weights w are applied here only when given (otherwise the expert
// outputs already carry them).  With topk_ids
// given, slots whose expert id is negative, or maps to a negative local id
// through expert_map, are skipped (their rows hold no expert output); the
// fused layers also pass their expert count, so that a slot whose (local) id
// is past the last expert -- a route the alignment drops -- is skipped too.
//
// Each thread owns 8 consecutive hidden elements of one token (16-byte loads
// for 2-byte types), so a wave streams 1 KiB contiguous per slot.
#include "common.h"

namespace vmamd {

// num_experts <= 0: no upper bound on the (local) id.
__device__ __forceinline__ bool slot_live(const int32_t* __restrict__ ids, const int32_t* __restrict__ map,
                                          int64_t map_len, int num_experts, int64_t route) {
  if (!ids) return true;
  int e = ids[route];
  if (e < 0) return false;
  if (map) {
    if (e >= map_len) return false;
    e = map[e];
    if (e < 0) return false;
  }
  return num_experts <= 0 || e < num_experts;
}

// Slots a thread loads up front (DeepSeek-V3 and most MoE layers use top-8).
constexpr int kSumSlots = 8;

template <int DT, bool VEC>
__global__ __launch_bounds__(256) void moe_sum_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                      int64_t tokens, int topk, int64_t hidden,
                                                      typename Elem<DT>::T* __restrict__ out,
                                                      const int32_t* __restrict__ ids,
                                                      const int32_t* __restrict__ map, int64_t map_len,
                                                      int num_experts, const float* __restrict__ wts) {
  using E = Elem<DT>;
  using T = typename E::T;
  const int64_t chunks = hidden / 8;
  const int64_t total = tokens * chunks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / chunks;
    const int64_t h = (i - t * chunks) * 8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if constexpr (VEC && sizeof(T) == 2) {
      if (topk <= kSumSlots) {
        // All slot rows are requested before the first add (one memory round
        // trip instead of topk), unconditionally (slots past topk re-read the
        // last row: a branch around a load would make it wait on its own);
        // dead slots are read too (their rows exist) and dropped by a select,
        // and the adds stay in slot order.
        uint4 raw[kSumSlots];
#pragma unroll
        for (int k = 0; k < kSumSlots; ++k) {
          const int kk = k < topk ? k : topk - 1;
          raw[k] = *reinterpret_cast<const uint4*>(x + (t * topk + kk) * hidden + h);
        }
#pragma unroll
        for (int k = 0; k < kSumSlots; ++k) {
          if (k >= topk) continue;
          const bool live = slot_live(ids, map, map_len, num_experts, t * topk + k);
          const float wk = wts ? wts[t * topk + k] : 1.0f;
          const uint16_t* p = reinterpret_cast<const uint16_t*>(&raw[k]);
          // One fused multiply-add per weighted slot (one rounding, as the
          // weighted combine is defined); a dead slot leaves acc untouched.
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float v = E::to_f(p[j]);
            const float a = wts ? __builtin_fmaf(v, wk, acc[j]) : acc[j] + v;
            acc[j] = live ? a : acc[j];
          }
        }
        T* dst = out + t * hidden + h;
        uint4 o;
        uint16_t* q = reinterpret_cast<uint16_t*>(&o);
#pragma unroll
        for (int j = 0; j < 8; ++j) q[j] = E::from_f(acc[j]);
        *reinterpret_cast<uint4*>(dst) = o;
        continue;
      }
    }
    for (int k = 0; k < topk; ++k) {
      if (!slot_live(ids, map, map_len, num_experts, t * topk + k)) continue;
      const T* src = x + (t * topk + k) * hidden + h;
      if constexpr (VEC && sizeof(T) == 2) {
        const uint4 raw = *reinterpret_cast<const uint4*>(src);
        const uint16_t* p = reinterpret_cast<const uint16_t*>(&raw);
        if (wts) {
          const float wk = wts[t * topk + k];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] += E::to_f(p[j]) * wk;
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[j] += E::to_f(p[j]);
        }
      } else {
        const float wk = wts ? wts[t * topk + k] : 1.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] += wts ? E::to_f(src[j]) * wk : E::to_f(src[j]);
      }
    }
    T* dst = out + t * hidden + h;
    if constexpr (VEC && sizeof(T) == 2) {
      uint4 raw;
      uint16_t* p = reinterpret_cast<uint16_t*>(&raw);
#pragma unroll
      for (int j = 0; j < 8; ++j) p[j] = E::from_f(acc[j]);
      *reinterpret_cast<uint4*>(dst) = raw;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[j] = E::from_f(acc[j]);
    }
  }
}

// Generic path for hidden sizes that are not a multiple of 8.
template <int DT>
__global__ __launch_bounds__(256) void moe_sum_scalar_kernel(const typename Elem<DT>::T* __restrict__ x,
                                                             int64_t tokens, int topk, int64_t hidden,
                                                             typename Elem<DT>::T* __restrict__ out,
                                                             const int32_t* __restrict__ ids,
                                                             const int32_t* __restrict__ map,
                                                             int64_t map_len, int num_experts,
                                                             const float* __restrict__ wts) {
  using E = Elem<DT>;
  const int64_t total = tokens * hidden;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / hidden, h = i - t * hidden;
    float acc = 0.f;
    for (int k = 0; k < topk; ++k)
      if (slot_live(ids, map, map_len, num_experts, t * topk + k)) {
        const float v = E::to_f(x[(t * topk + k) * hidden + h]);
        acc += wts ? v * wts[t * topk + k] : v;
      }
    out[i] = E::from_f(acc);
  }
}

}  // namespace vmamd

using namespace vmamd;

namespace vmamd {

int moe_sum_impl(const char* who, const void* x, int dtype, int64_t tokens, int topk,
                 int64_t hidden, const int32_t* topk_ids, const int32_t* expert_map,
                 int64_t expert_map_len, int num_experts, const float* wts, void* out,
                 vmamd_stream_t stream) {
  VMAMD_REQUIRE(tokens >= 0 && topk > 0 && hidden >= 0, "%s: bad sizes", who);
  VMAMD_REQUIRE(!expert_map || topk_ids, "%s: expert_map needs topk_ids", who);
  if (tokens * hidden == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && out, "%s: null pointer", who);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int esize = dtype == kF32 ? 4 : 2;
  const bool vec = hidden % 8 == 0 && esize == 2 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0;
  const int64_t work = hidden % 8 == 0 ? tokens * (hidden / 8) : tokens * hidden;
  const int blocks = static_cast<int>(work / 256 + 1 < 65536 ? work / 256 + 1 : 65536);
#define VMAMD_SUM(DT, TY)                                                                       \
  do {                                                                                          \
    const TY* xi = static_cast<const TY*>(x);                                                   \
    TY* oi = static_cast<TY*>(out);                                                             \
    if (hidden % 8 != 0)                                                                        \
      moe_sum_scalar_kernel<DT><<<blocks, 256, 0, st>>>(xi, tokens, topk, hidden, oi, topk_ids, \
                                                        expert_map, expert_map_len, num_experts,    \
                                                        wts);                                   \
    else if (vec)                                                                               \
      moe_sum_kernel<DT, true><<<blocks, 256, 0, st>>>(xi, tokens, topk, hidden, oi, topk_ids,  \
                                                       expert_map, expert_map_len, num_experts,     \
                                                       wts);                                    \
    else                                                                                        \
      moe_sum_kernel<DT, false><<<blocks, 256, 0, st>>>(xi, tokens, topk, hidden, oi, topk_ids, \
                                                        expert_map, expert_map_len, num_experts,    \
                                                        wts);                                   \
  } while (0)
  switch (dtype) {
    case kBF16: VMAMD_SUM(kBF16, uint16_t); break;
    case kF16: VMAMD_SUM(kF16, uint16_t); break;
    case kF32: VMAMD_SUM(kF32, float); break;
    default: VMAMD_REQUIRE(false, "%s: unsupported dtype %d", who, dtype);
  }
#undef VMAMD_SUM
  return check_launch(who);
}

}  // namespace vmamd

extern "C" int vmamd_moe_sum(const void* x, int dtype, int64_t tokens, int topk, int64_t hidden,
                             const int32_t* topk_ids, const int32_t* expert_map,
                             int64_t expert_map_len, void* out, vmamd_stream_t stream) {
  return moe_sum_impl("moe_sum", x, dtype, tokens, topk, hidden, topk_ids, expert_map,
                      expert_map_len, 0, nullptr, out, stream);
}

extern "C" int vmamd_moe_weighted_sum(const void* x, int dtype, int64_t tokens, int topk,
                                      int64_t hidden, const float* topk_weights,
                                      const int32_t* topk_ids, const int32_t* expert_map,
                                      int64_t expert_map_len, void* out, vmamd_stream_t stream) {
  VMAMD_REQUIRE(topk_weights || tokens * hidden == 0, "moe_weighted_sum: null topk_weights");
  return moe_sum_impl("moe_weighted_sum", x, dtype, tokens, topk, hidden, topk_ids, expert_map,
                      expert_map_len, 0, topk_weights, out, stream);
}
