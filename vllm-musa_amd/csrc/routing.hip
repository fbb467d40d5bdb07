// Router top-k kernels: softmax top-k, sigmoid top-k and grouped top-k.
//
// One wave64 owns one token row.  Expert e lives in lane e % 64, register
// slot e / 64, so the row is read with fully coalesced loads and every
// selection round is a 6-step wave argmax (ties to the lower expert id) whose
// first four steps are DPP lane moves and the last two shuffles.  Selection never depends on the order of a floating-point reduction:
//   - softmax top-k selects on the (biased) logits, which softmax preserves;
//   - sigmoid/softmax scores that feed a selection together with a bias are
//     evaluated in double precision and rounded once to float, so they are
//     the correctly rounded float values (up to a ~2^-29 chance per value of
//     a double-rounding tie), independent of the device's float exp.
#include <float.h>

#include "common.h"

namespace vmamd {

constexpr int kRouteWaves = 4;  // token rows per 256-thread block

template <int DT>
__device__ __forceinline__ float load_gate(const void* g, int64_t i) {
  return Elem<DT>::load(static_cast<const typename Elem<DT>::T*>(g), i);
}

// Correctly rounded (to float) logistic function, evaluated in double.
__device__ __forceinline__ float sigmoid_cr(float x) {
  return static_cast<float>(1.0 / (1.0 + exp(-static_cast<double>(x))));
}

// One selection round over the live entries of a wave: returns the winning
// (value, expert id) to every lane and retires the winner in its owner lane
// (id 0x7fffffff and -inf when no entry is live).  Ties go to the lower id:
// each entry is one 64-bit key (argmax_key) and the round is a wave maximum.
template <int VPT>
__device__ __forceinline__ int select_round(const float (&v)[VPT], uint32_t& alive, float& best) {
  const int lane = lane_id();
  uint64_t k = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i)
    if ((alive >> i) & 1u) k = max_u64(k, argmax_key(v[i], lane + kWave * i));
  k = wave_max_key(k);
  if (k == 0) {
    best = -INFINITY;
    return 0x7fffffff;
  }
  const int bi = argmax_key_index(k);
  if ((bi % kWave) == lane) alive &= ~(1u << (bi / kWave));
  best = argmax_key_value(k);
  return bi;
}

// Fused shared expert: one more output column per token, weight = sigmoid of
// the token's shared gate logit computed in fp32 and rounded to the logit
// dtype, id = the shared expert's id (topk_gating.mu:369-456 writes it in the
// same kernel as the routed top-k).  logits == nullptr: no shared column.
// tei (when not null, no shared column): token_expert_indices [tokens, topk],
// tei[t, k] = k * tokens + t, upstream fused_topk's third output.
struct SharedCol {
  const void* logits;
  int dtype;
  int32_t id;
  int32_t* tei;
};

template <int DT>
__device__ __forceinline__ float shared_weight(const typename Elem<DT>::T* logits, int64_t t) {
  const float s = 1.0f / (1.0f + expf(-Elem<DT>::load(logits, t)));
  return Elem<DT>::to_f(Elem<DT>::from_f(s));
}

__device__ __forceinline__ float shared_weight_rt(const SharedCol& sh, int64_t t) {
  switch (sh.dtype) {
    case kF32: return shared_weight<kF32>(static_cast<const float*>(sh.logits), t);
    case kF16: return shared_weight<kF16>(static_cast<const uint16_t*>(sh.logits), t);
    default: return shared_weight<kBF16>(static_cast<const uint16_t*>(sh.logits), t);
  }
}

// Output row r holds the routed top-k in columns [0, topk) and, with a shared
// column, that expert in column topk (row stride topk + 1).
__device__ __forceinline__ void write_shared(const SharedCol& sh, int lane, int topk, int64_t row,
                                             int64_t tokens, float* w_out, int32_t* id_out) {
  if (sh.tei && lane < topk) sh.tei[row * topk + lane] = static_cast<int32_t>(lane * tokens + row);
  if (sh.logits && lane == topk) {
    w_out[row * (topk + 1) + topk] = shared_weight_rt(sh, row);
    id_out[row * (topk + 1) + topk] = sh.id;
  }
}

// ------------------------------------------------------- softmax top-k ----
template <int DT, int VPT>
__global__ __launch_bounds__(kRouteWaves * kWave) void topk_softmax_kernel(
    const void* __restrict__ gating, int64_t tokens, int experts, int topk, bool renorm,
    float softcap, const float* __restrict__ bias, float* __restrict__ w_out,
    int32_t* __restrict__ id_out, SharedCol sh) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRouteWaves + threadIdx.x / kWave;
  if (row >= tokens) return;
  const int lane = lane_id();
  float v[VPT];
  uint32_t alive = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = lane + kWave * i;
    v[i] = -INFINITY;
    if (e < experts) {
      float x = load_gate<DT>(gating, row * experts + e);
      if (bias) x += bias[e];
      if (softcap > 0.f) x = tanhf(x / softcap) * softcap;
      v[i] = x;
      alive |= 1u << i;
    }
  }
  // Row max is the first selected value; softmax denominators use it.
  float first = 0.f, chosen_sum = 0.f, my_w = 0.f;
  int my_id = 0;
  for (int k = 0; k < topk; ++k) {
    float bv;
    const int bi = select_round<VPT>(v, alive, bv);
    if (k == 0) first = bv;
    const float ek = expf(bv - first);
    chosen_sum += ek;  // fixed order k = 0, 1, ... in every lane
    if (lane == k) {
      my_w = ek;
      my_id = bi;
    }
  }
  float denom = chosen_sum;
  if (!renorm) {
    // Full softmax denominator over all experts.
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (lane + kWave * i < experts) part += expf(v[i] - first);
    // Retired entries still hold their logits in v[], so the sum is complete.
    denom = wave_sum(part);
  }
  const int64_t ostride = sh.logits ? topk + 1 : topk;
  if (lane < topk) {
    w_out[row * ostride + lane] = my_w / denom;
    id_out[row * ostride + lane] = my_id;
  }
  write_shared(sh, lane, topk, row, tokens, w_out, id_out);
}

// ------------------------------------------------------- sigmoid top-k ----
template <int DT, int VPT>
__global__ __launch_bounds__(kRouteWaves * kWave) void topk_sigmoid_kernel(
    const void* __restrict__ gating, int64_t tokens, int experts, int topk, bool renorm,
    const float* __restrict__ bias, float* __restrict__ w_out, int32_t* __restrict__ id_out,
    SharedCol sh) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRouteWaves + threadIdx.x / kWave;
  if (row >= tokens) return;
  const int lane = lane_id();
  float sel[VPT], sc[VPT];
  uint32_t alive = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = lane + kWave * i;
    sel[i] = -INFINITY;
    sc[i] = 0.f;
    if (e < experts) {
      const float s = sigmoid_cr(load_gate<DT>(gating, row * experts + e));
      sc[i] = s;
      sel[i] = bias ? s + bias[e] : s;
      alive |= 1u << i;
    }
  }
  float my_w = 0.f, sum = 0.f;
  int my_id = 0;
  for (int k = 0; k < topk; ++k) {
    float bv;
    const int bi = select_round<VPT>(sel, alive, bv);
    // Fetch the unbiased score of the winner from its owner lane.
    float s_local = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (lane + kWave * i == bi) s_local = sc[i];
    const float s = lane_value(s_local, bi % kWave);  // bi is wave-uniform
    sum += s;
    if (lane == k) {
      my_w = s;
      my_id = bi;
    }
  }
  const int64_t ostride = sh.logits ? topk + 1 : topk;
  if (lane < topk) {
    w_out[row * ostride + lane] = renorm ? my_w / sum : my_w;
    id_out[row * ostride + lane] = my_id;
  }
  write_shared(sh, lane, topk, row, tokens, w_out, id_out);
}

// ------------------------------------------------------- grouped top-k ----
// Group g is the S consecutive experts g*S..g*S+S-1.  With S a power of two
// <= 64 a group occupies S aligned lanes of one register slot (expert e sits
// in lane e % 64, slot e / 64), so its top-2 is a log2(S)-step reduction; the
// scores are then gathered so that lane g holds group g's.
template <int VPT, int S>
__device__ __forceinline__ float group_scores_pow2(const float (&sel)[VPT], bool sum2, int groups) {
  constexpr int kSegs = kWave / S;  // groups per register slot
  const int lane = lane_id();
  float gs[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    float t1 = sel[i], t2 = -INFINITY;
    group_top2<S>(t1, t2);
    gs[i] = sum2 ? t1 + t2 : t1;
  }
  // Group j of slot i (score in lanes j*S .. j*S+S-1) goes to lane i*kSegs + j.
  float gv = -INFINITY;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    if constexpr (kSegs <= 4) {
#pragma unroll
      for (int j = 0; j < kSegs; ++j) {
        const float v = lane_value(gs[i], j * S);
        if (lane == i * kSegs + j) gv = v;
      }
    } else {
      const float v = __shfl(gs[i], (lane % kSegs) * S, kWave);
      if (lane / kSegs == i) gv = v;
    }
  }
  return lane < groups ? gv : -INFINITY;
}

// Any group size: the members of each group are broadcast in turn.
template <int VPT>
__device__ __forceinline__ float group_scores_serial(const float (&sel)[VPT], bool sum2, int groups,
                                                     int gsize) {
  const int lane = lane_id();
  float gv = -INFINITY;
  for (int g = 0; g < groups; ++g) {
    float t1 = -INFINITY, t2 = -INFINITY;
    for (int j = 0; j < gsize; ++j) {
      const int e = g * gsize + j;
      float mine = -INFINITY;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        if (lane + kWave * i == e) mine = sel[i];
      top2_merge(t1, t2, __shfl(mine, e % kWave, kWave), -INFINITY);
    }
    if (lane == g) gv = sum2 ? t1 + t2 : t1;
  }
  return gv;
}

// Scores per expert (softmax or sigmoid, double-evaluated), sel = score (+
// bias); group g is the S = experts / groups consecutive experts g*S..g*S+S-1.
template <int DT, int VPT>
__global__ __launch_bounds__(kRouteWaves * kWave) void grouped_topk_kernel(
    const void* __restrict__ gating, int64_t tokens, int experts, int groups, int topk_group,
    int topk, bool renorm, int scoring, float scale, const float* __restrict__ bias,
    float* __restrict__ w_out, int32_t* __restrict__ id_out) {
  const int wave = threadIdx.x / kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRouteWaves + wave;
  if (row >= tokens) return;
  const int lane = lane_id();
  const int gsize = experts / groups;

  float logit[VPT], sc[VPT], sel[VPT];
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = lane + kWave * i;
    logit[i] = e < experts ? load_gate<DT>(gating, row * experts + e) : -INFINITY;
  }
  if (scoring == VMAMD_SCORING_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPT; ++i) m = fmaxf(m, logit[i]);
    m = wave_max(m);
    double part = 0.0;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (lane + kWave * i < experts) part += exp(static_cast<double>(logit[i]) - m);
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) part += __shfl_xor(part, s, kWave);
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      sc[i] = lane + kWave * i < experts
                  ? static_cast<float>(exp(static_cast<double>(logit[i]) - m) / part)
                  : 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) sc[i] = lane + kWave * i < experts ? sigmoid_cr(logit[i]) : 0.f;
  }
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = lane + kWave * i;
    sel[i] = e < experts ? (bias ? sc[i] + bias[e] : sc[i]) : -INFINITY;
  }

  // Group scores (sum of the top-2 sel with a bias, else the max), gathered
  // so that lane g holds the score of group g.
  float gv;
  switch (gsize) {
    case 1: gv = group_scores_pow2<VPT, 1>(sel, bias != nullptr, groups); break;
    case 2: gv = group_scores_pow2<VPT, 2>(sel, bias != nullptr, groups); break;
    case 4: gv = group_scores_pow2<VPT, 4>(sel, bias != nullptr, groups); break;
    case 8: gv = group_scores_pow2<VPT, 8>(sel, bias != nullptr, groups); break;
    case 16: gv = group_scores_pow2<VPT, 16>(sel, bias != nullptr, groups); break;
    case 32: gv = group_scores_pow2<VPT, 32>(sel, bias != nullptr, groups); break;
    case 64: gv = group_scores_pow2<VPT, 64>(sel, bias != nullptr, groups); break;
    default: gv = group_scores_serial<VPT>(sel, bias != nullptr, groups, gsize); break;
  }
  uint64_t keep = 0;  // bit g set when group g is kept
  {
    uint32_t alive_g = lane < groups ? 1u : 0u;
    float gsel[1] = {gv};
    for (int k = 0; k < topk_group; ++k) {
      float bv;
      const int bg = select_round<1>(gsel, alive_g, bv);
      keep |= 1ull << bg;
    }
  }
  uint32_t alive = 0;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const int e = lane + kWave * i;
    if (e < experts && ((keep >> (e / gsize)) & 1ull)) alive |= 1u << i;
  }
  float my_w = 0.f, sum = 0.f;
  int my_id = 0;
  for (int k = 0; k < topk; ++k) {
    float bv;
    const int bi = select_round<VPT>(sel, alive, bv);
    float s_local = 0.f;
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      if (lane + kWave * i == bi) s_local = sc[i];
    const float s = lane_value(s_local, bi % kWave);  // bi is wave-uniform
    sum += s;
    if (lane == k) {
      my_w = s;
      my_id = bi;
    }
  }
  if (lane < topk) {
    float w = renorm ? my_w / sum : my_w;
    if (scale != 1.0f) w *= scale;
    w_out[row * topk + lane] = w;
    id_out[row * topk + lane] = my_id;
  }
}

static int vpt_for(int experts) {
  if (experts <= 64) return 1;
  if (experts <= 128) return 2;
  if (experts <= 256) return 4;
  if (experts <= 512) return 8;
  return 16;
}

}  // namespace vmamd

using namespace vmamd;

#define VMAMD_ROUTE_DISPATCH(KERNEL, ...)                                                      \
  do {                                                                                        \
    const int vpt_ = vpt_for(experts);                                                        \
    const int64_t blocks_ = (tokens + kRouteWaves - 1) / kRouteWaves;                         \
    hipStream_t st_ = reinterpret_cast<hipStream_t>(stream);                                  \
    switch (dtype * 32 + vpt_) {                                                              \
      case kF32 * 32 + 1: KERNEL<kF32, 1><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF32 * 32 + 2: KERNEL<kF32, 2><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF32 * 32 + 4: KERNEL<kF32, 4><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF32 * 32 + 8: KERNEL<kF32, 8><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF32 * 32 + 16: KERNEL<kF32, 16><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;    \
      case kF16 * 32 + 1: KERNEL<kF16, 1><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF16 * 32 + 2: KERNEL<kF16, 2><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF16 * 32 + 4: KERNEL<kF16, 4><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF16 * 32 + 8: KERNEL<kF16, 8><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;      \
      case kF16 * 32 + 16: KERNEL<kF16, 16><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;    \
      case kBF16 * 32 + 1: KERNEL<kBF16, 1><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;    \
      case kBF16 * 32 + 2: KERNEL<kBF16, 2><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;    \
      case kBF16 * 32 + 4: KERNEL<kBF16, 4><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;    \
      case kBF16 * 32 + 8: KERNEL<kBF16, 8><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;    \
      case kBF16 * 32 + 16: KERNEL<kBF16, 16><<<blocks_, 256, 0, st_>>>(__VA_ARGS__); break;  \
      default: VMAMD_REQUIRE(false, #KERNEL ": unsupported dtype %d", dtype);                 \
    }                                                                                         \
  } while (0)

namespace vmamd {
// Folded shared expert: the [T, K] routing plus one always-selected column
// (weight = sigmoid(shared gate logit) in fp32, rounded to the logit dtype;
// id = the shared expert's id).  One thread per output element.
template <int DT>
__global__ __launch_bounds__(256) void extend_topk_shared_kernel(
    const float* __restrict__ w_in, const int32_t* __restrict__ ids_in, int64_t tokens, int topk,
    const typename Elem<DT>::T* __restrict__ logits, int32_t shared_id, float* __restrict__ w_out,
    int32_t* __restrict__ ids_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int k1 = topk + 1;
  if (i >= tokens * k1) return;
  const int64_t t = i / k1;
  const int k = static_cast<int>(i - t * k1);
  if (k < topk) {
    w_out[i] = w_in[t * topk + k];
    ids_out[i] = ids_in[t * topk + k];
  } else {
    w_out[i] = shared_weight<DT>(logits, t);
    ids_out[i] = shared_id;
  }
}
}  // namespace vmamd

extern "C" int vmamd_extend_topk_with_shared(const float* topk_weights, const int32_t* topk_ids,
                                             int64_t tokens, int topk, const void* shared_logits,
                                             int dtype, int32_t shared_expert_id, float* out_weights,
                                             int32_t* out_ids, vmamd_stream_t stream) {
  using namespace vmamd;
  VMAMD_REQUIRE(tokens >= 0 && topk >= 0, "extend_topk_with_shared: bad sizes");
  if (tokens == 0) return VMAMD_OK;
  VMAMD_REQUIRE((topk_weights && topk_ids) || topk == 0, "extend_topk_with_shared: null routing");
  VMAMD_REQUIRE(shared_logits && out_weights && out_ids, "extend_topk_with_shared: null pointer");
  const int64_t n = tokens * (topk + 1);
  const int blocks = static_cast<int>((n + 255) / 256);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dtype) {
    case kF32:
      extend_topk_shared_kernel<kF32><<<blocks, 256, 0, st>>>(
          topk_weights, topk_ids, tokens, topk, static_cast<const float*>(shared_logits),
          shared_expert_id, out_weights, out_ids);
      break;
    case kF16:
      extend_topk_shared_kernel<kF16><<<blocks, 256, 0, st>>>(
          topk_weights, topk_ids, tokens, topk, static_cast<const uint16_t*>(shared_logits),
          shared_expert_id, out_weights, out_ids);
      break;
    case kBF16:
      extend_topk_shared_kernel<kBF16><<<blocks, 256, 0, st>>>(
          topk_weights, topk_ids, tokens, topk, static_cast<const uint16_t*>(shared_logits),
          shared_expert_id, out_weights, out_ids);
      break;
    default:
      VMAMD_REQUIRE(false, "extend_topk_with_shared: unsupported logit dtype %d", dtype);
  }
  return check_launch("extend_topk_with_shared");
}

extern "C" int vmamd_topk_softmax(const void* gating, int dtype, int64_t tokens, int experts,
                                  int topk, int renormalize, float softcap, const float* bias,
                                  float* topk_weights, int32_t* topk_ids,
                                  int32_t* token_expert_indices, vmamd_stream_t stream) {
  VMAMD_REQUIRE(experts > 0 && experts <= 1024, "topk_softmax: experts must be in [1, 1024] (got %d)",
                experts);
  VMAMD_REQUIRE(topk > 0 && topk <= experts && topk <= 64,
                "topk_softmax: topk must be in [1, min(experts, 64)] (got %d)", topk);
  VMAMD_REQUIRE(tokens >= 0, "topk_softmax: negative token count");
  if (tokens == 0) return VMAMD_OK;
  VMAMD_REQUIRE(gating && topk_weights && topk_ids, "topk_softmax: null pointer");
  VMAMD_REQUIRE(tokens * topk < (1ll << 31), "topk_softmax: too many routes");
  VMAMD_ROUTE_DISPATCH(topk_softmax_kernel, gating, tokens, experts, topk, renormalize != 0, softcap,
                       bias, topk_weights, topk_ids, SharedCol{nullptr, 0, 0, token_expert_indices});
  return check_launch("topk_softmax");
}

extern "C" int vmamd_topk_softmax_shared(const void* gating, int dtype, int64_t tokens,
                                         int experts, int topk, int renormalize, float softcap,
                                         const float* bias, const void* shared_logits,
                                         int shared_dtype, int32_t shared_expert_id,
                                         float* topk_weights, int32_t* topk_ids,
                                         vmamd_stream_t stream) {
  VMAMD_REQUIRE(experts > 0 && experts <= 1024,
                "topk_softmax_shared: experts must be in [1, 1024] (got %d)", experts);
  VMAMD_REQUIRE(topk > 0 && topk <= experts && topk < 64,
                "topk_softmax_shared: topk must be in [1, min(experts, 63)] (got %d)", topk);
  VMAMD_REQUIRE(shared_dtype == kF32 || shared_dtype == kF16 || shared_dtype == kBF16,
                "topk_softmax_shared: unsupported shared logit dtype %d", shared_dtype);
  VMAMD_REQUIRE(tokens >= 0, "topk_softmax_shared: negative token count");
  if (tokens == 0) return VMAMD_OK;
  VMAMD_REQUIRE(gating && shared_logits && topk_weights && topk_ids,
                "topk_softmax_shared: null pointer");
  VMAMD_ROUTE_DISPATCH(topk_softmax_kernel, gating, tokens, experts, topk, renormalize != 0, softcap,
                       bias, topk_weights, topk_ids,
                       SharedCol{shared_logits, shared_dtype, shared_expert_id, nullptr});
  return check_launch("topk_softmax_shared");
}

extern "C" int vmamd_topk_sigmoid(const void* gating, int dtype, int64_t tokens, int experts,
                                  int topk, int renormalize, const float* bias, float* topk_weights,
                                  int32_t* topk_ids, int32_t* token_expert_indices,
                                  vmamd_stream_t stream) {
  VMAMD_REQUIRE(experts > 0 && experts <= 1024, "topk_sigmoid: experts must be in [1, 1024] (got %d)",
                experts);
  VMAMD_REQUIRE(topk > 0 && topk <= experts && topk <= 64,
                "topk_sigmoid: topk must be in [1, min(experts, 64)] (got %d)", topk);
  VMAMD_REQUIRE(tokens >= 0, "topk_sigmoid: negative token count");
  if (tokens == 0) return VMAMD_OK;
  VMAMD_REQUIRE(gating && topk_weights && topk_ids, "topk_sigmoid: null pointer");
  VMAMD_REQUIRE(tokens * topk < (1ll << 31), "topk_sigmoid: too many routes");
  VMAMD_ROUTE_DISPATCH(topk_sigmoid_kernel, gating, tokens, experts, topk, renormalize != 0, bias,
                       topk_weights, topk_ids, SharedCol{nullptr, 0, 0, token_expert_indices});
  return check_launch("topk_sigmoid");
}

extern "C" int vmamd_topk_sigmoid_shared(const void* gating, int dtype, int64_t tokens,
                                         int experts, int topk, int renormalize, const float* bias,
                                         const void* shared_logits, int shared_dtype,
                                         int32_t shared_expert_id, float* topk_weights,
                                         int32_t* topk_ids, vmamd_stream_t stream) {
  VMAMD_REQUIRE(experts > 0 && experts <= 1024,
                "topk_sigmoid_shared: experts must be in [1, 1024] (got %d)", experts);
  VMAMD_REQUIRE(topk > 0 && topk <= experts && topk < 64,
                "topk_sigmoid_shared: topk must be in [1, min(experts, 63)] (got %d)", topk);
  VMAMD_REQUIRE(shared_dtype == kF32 || shared_dtype == kF16 || shared_dtype == kBF16,
                "topk_sigmoid_shared: unsupported shared logit dtype %d", shared_dtype);
  VMAMD_REQUIRE(tokens >= 0, "topk_sigmoid_shared: negative token count");
  if (tokens == 0) return VMAMD_OK;
  VMAMD_REQUIRE(gating && shared_logits && topk_weights && topk_ids,
                "topk_sigmoid_shared: null pointer");
  VMAMD_ROUTE_DISPATCH(topk_sigmoid_kernel, gating, tokens, experts, topk, renormalize != 0, bias,
                       topk_weights, topk_ids,
                       SharedCol{shared_logits, shared_dtype, shared_expert_id, nullptr});
  return check_launch("topk_sigmoid_shared");
}

extern "C" int vmamd_grouped_topk(const void* gating, int dtype, int64_t tokens, int experts,
                                  int num_expert_group, int topk_group, int topk, int renormalize,
                                  int scoring, float routed_scaling_factor, const float* bias,
                                  float* topk_weights, int32_t* topk_ids, vmamd_stream_t stream) {
  VMAMD_REQUIRE(experts > 0 && experts <= 1024, "grouped_topk: experts must be in [1, 1024] (got %d)",
                experts);
  VMAMD_REQUIRE(num_expert_group > 0 && num_expert_group <= 64 && experts % num_expert_group == 0,
                "grouped_topk: experts (%d) must split into 1..64 equal groups (got %d)", experts,
                num_expert_group);
  VMAMD_REQUIRE(topk_group > 0 && topk_group <= num_expert_group,
                "grouped_topk: topk_group must be in [1, num_expert_group] (got %d)", topk_group);
  VMAMD_REQUIRE(topk > 0 && topk <= 64 && topk <= topk_group * (experts / num_expert_group),
                "grouped_topk: topk (%d) exceeds the experts of the kept groups", topk);
  VMAMD_REQUIRE(!bias || experts / num_expert_group >= 2,
                "grouped_topk: the biased group score needs at least 2 experts per group");
  VMAMD_REQUIRE(scoring == VMAMD_SCORING_SOFTMAX || scoring == VMAMD_SCORING_SIGMOID,
                "grouped_topk: unknown scoring function %d", scoring);
  VMAMD_REQUIRE(tokens >= 0, "grouped_topk: negative token count");
  if (tokens == 0) return VMAMD_OK;
  VMAMD_REQUIRE(gating && topk_weights && topk_ids, "grouped_topk: null pointer");
  VMAMD_ROUTE_DISPATCH(grouped_topk_kernel, gating, tokens, experts, num_expert_group, topk_group,
                       topk, renormalize != 0, scoring, routed_scaling_factor, bias, topk_weights,
                       topk_ids);
  return check_launch("grouped_topk");
}
