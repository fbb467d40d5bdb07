// Fused-MoE expert GEMMs (W13 gate/up, W2 down) for three weight formats:
//
//   kFp8  128x128 block-fp8 weights, 1x128 fp8 activation groups:
//         xq [T, H] e4m3 + xs [T, H/128] f32; w13 [E, 2I, H] e4m3 +
//         w13_s [E, 2I/128, H/128] f32; w2 [E, H, I] + w2_s [E, H/128, I/128]
//   kBf16 bf16 weights and activations: x [T, H]; w13 [E, 2I, H]; w2 [E, H, I]
//   kW4   w4afp8: signed int4 weights two per byte (element 2j in the low
//         nibble of byte j), bf16 scale per (output row, 128-K group):
//         w13 [E, 2I, H/2] + [E, 2I, H/128]; w2 [E, H, I/2] + [E, H, I/128];
//         activations fp8 with one scale per row: xq [T, H] + xs [T]
//   kW8A16 the kFp8 weights against bf16 activations that are not quantised
//         (decode GEMVs only): x [T, H] bf16, a2 [T*topk, I] bf16
//   w13 rows [0, I) gate, [I, 2I) up; routes r = t * topk + k; sorted /
//   offsets / active come from moe_align_block_size.
//
// Every kind moves K in "steps": 128 K-elements for kFp8 / kW4 (one 16x16x128
// fp8 MFMA; kW4 nibbles are converted to e4m3 codes on the way in, every
// integer in [-8, 7] being exact in e4m3) and kW8A16 (four 16x16x32 bf16
// MFMAs on the exactly converted weights), 64 for kBf16 (two 16x16x32 bf16
// MFMAs).  Per step kFp8 promotes acc += p * sa[m] * sb[n/128], kW8A16
// acc += p * sb[n/128], kW4 promotes acc += p * sw[n] with the row's own
// weight scale and applies the activation row scale once at the end, kBf16
// accumulates directly.
//
// Decode path (few routes per expert): moe_gemv_kernel.  A wave owns 16
// weight rows of one active expert and a K range; it streams the rows from
// HBM once (no LDS) and applies each 16-row fragment to every 16-route block
// of that expert.  W13 writes fp32 split-K partials per route; the act
// kernels sum them in a fixed order, round gate/up to bf16, apply
// SiLU-and-mul and quantise a2.  W2 writes bf16(acc * routed weight) per
// route (kW4: bf16(acc * a2 row scale), the routed weight is applied by the
// combine), or fp32 partials reduced by moe_w2_reduce_kernel.
//
// Prefill path (many routes per expert): grouped MFMA GEMMs over 128-route
// blocks.  Tiles are ordered expert-major -- all blocks of one (expert,
// n-tile) are consecutive -- and each XCD takes a contiguous tile range, so
// the blocks of an expert that share a weight tile run together on one XCD
// and the tile is fetched from HBM once.  W13 covers 128 gate + 128 up rows
// per tile (interleaved by 16 so each lane holds matching gate/up values) and
// fuses SiLU-and-mul (and the kFp8 1x128 a2 quantiser) into its epilogue.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <type_traits>

#include "quant_dev.h"
#include "mfma_fp8.h"
#include "tile_pipe.h"

namespace vmamd {

constexpr int kFp8 = 0, kBf16 = 1, kW4 = 2, kW8A16 = 3;

// Bytes of one K step: activation row, weight row.
template <int KIND> struct KindBytes {
  static constexpr int kAct = KIND == kW8A16 ? 256 : 128;
  static constexpr int kW = KIND == kW4 ? 64 : 128;
  static constexpr int kElems = KIND == kBf16 ? 64 : 128;  // K elements per step
};

// Operands of a kind: per-step activation values (kFp8 group scales, kW4
// block corrections), f32 weight block scales [E, N/128, K/128] (kFp8,
// kW8A16), and the activation fragment (kW8A16: 32 bf16 values).
template <int KIND> struct KindOps {
  static constexpr bool kActScale = KIND == kFp8 || KIND == kW4;
  static constexpr bool kBlockScale = KIND == kFp8 || KIND == kW8A16;
  using AFrag = std::conditional_t<KIND == kW8A16, v16i, v8i>;
};

// --------------------------------------------------------------- helpers --
// x rounded to bf16 (nearest even) and back: v_cvt_pk_bf16_f32, the rounding
// of f32_to_bf16 for every number in one instruction (a NaN stays a NaN,
// with the hardware's payload; outputs go through f32_to_bf16).
__device__ __forceinline__ float bf16r(float x) {
  const __bf16 h = static_cast<__bf16>(x);
  return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h)) << 16);
}

// SiLU-and-mul on bf16-materialised gate/up; limit > 0 applies the clamped
// variant (gate <= L, up in [-L, L], sigmoid / silu / product each rounded to
// bf16).  Returns the bf16-rounded activation, or NaN for the clamped
// variant's exceptional inputs (quantised to fp8_min by the fp8 callers).
__device__ __forceinline__ float swiglu_bf16(float hg, float hu, float limit) {
  if (limit > 0.f) {
    const uint32_t gb = __float_as_uint(hg), ub = __float_as_uint(hu);
    const bool bad = ((gb & 0x7fffffffu) > 0x7f800000u) || gb == 0xff800000u ||
                     ((ub & 0x7fffffffu) > 0x7f800000u);
    const float L = bf16r(limit);
    float g = hg > L ? L : hg;
    float u = hu < -L ? -L : (hu > L ? L : hu);
    const float sig = bf16r(1.0f / (1.0f + expf(-g)));
    const float v = bf16r(bf16r(g * sig) * u);
    return bad ? __builtin_nanf("") : v;
  }
  return bf16r(hg / (1.0f + expf(-hg)) * hu);
}

// w4afp8 activation: the limit clamps gate <= L and up to [-L, L], then one
// rounding of silu(gate) * up to bf16.
__device__ __forceinline__ float swiglu_w4(float g, float u, float limit) {
  if (limit > 0.f) {
    g = fminf(g, limit);
    u = fmaxf(fminf(u, limit), -limit);
  }
  return bf16r(g / (1.0f + expf(-g)) * u);
}

template <int KIND>
__device__ __forceinline__ v8i weight_frag(const uint8_t* p, int g) {
  if constexpr (KIND == kW4) return w4_frag(ld16(p + 16 * g));
  else return global_frag(p, g);
}

// ---------------------------------------------------------- decode GEMV ---
constexpr int kMoeGemvWaves = 4;
constexpr int kGemvBlock = 16;  // routes per block (one MFMA column tile)
// K steps each wave keeps in flight (8 KiB of weights per wave; 4 and 8
// measured alike, 4 needs fewer registers), and the number of waves the
// split-K factor aims to launch (12 per CU: the single-block fp8 GEMV runs
// three waves per SIMD; 3072 measured 1-3 % faster than 4096 on the
// DeepSeek-V3 layer at T = 1, 4, 16).
constexpr int kGemvU = 4;
constexpr int kGemvTargetWaves = 3072;

// Raw buffer loads (gfx9 descriptor: base, no stride, num_records bytes):
// a lane whose byte offset is past num_records reads zeros and fetches
// nothing, which masks lanes without a branch.
constexpr int kBufferFlags = 0x00020000;
constexpr uint32_t kBufferOff = 0x80000000u;  // offset of a masked lane (buffers are < 2 GiB)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kBufferFlags);
}
__device__ __forceinline__ v4i buffer_ld16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0));
}
// Activation fragment at byte offset off (row + K-block start) of a buffer
// (kW4: the 32 contiguous bytes of lane group g, matching w4_frag; kW8A16:
// the bf16 activations of the K positions of the fp8 weight fragment,
// elements [16g, 16g + 16) and [64 + 16g, 80 + 16g) of the step).
template <int KIND>
__device__ __forceinline__ typename KindOps<KIND>::AFrag buffer_frag(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                                                     int g) {
  if constexpr (KIND == kW8A16) {
    const v4i a = buffer_ld16(rs, off + 32u * g), b = buffer_ld16(rs, off + 32u * g + 16u);
    const v4i c = buffer_ld16(rs, off + 128u + 32u * g), d = buffer_ld16(rs, off + 144u + 32u * g);
    return v16i{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3], c[0], c[1], c[2], c[3], d[0], d[1], d[2], d[3]};
  } else {
    const uint32_t o0 = KIND == kW4 ? 32u * g : 16u * g;
    const uint32_t o1 = KIND == kW4 ? 32u * g + 16u : 64u + 16u * g;
    const v4i lo = buffer_ld16(rs, off + o0);
    const v4i hi = buffer_ld16(rs, off + o1);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
}

// act: [rows, K] activation bytes (rows = numel / act_div, kW4 in w4 order,
// kBf16 / kW8A16 bf16), act_bytes its size (< 2^31); act_s: kFp8 [rows, K/128]
// group scales, kW4 [rows, K/128] offset corrections, otherwise unused.  ws:
// kFp8 / kW8A16 f32 block scales; kW4 bf16 row scales.  kW4 results are scaled by kW4Unit before they are
// stored.
//
// Start-up order: the expert id is the only load the weight stream depends
// on, so the first K group of weights is requested before the route list is
// resolved (offsets -> the block's route ids -> activation rows); every wave
// starts at once, so a serial chain of lookups in front of the stream would
// leave HBM idle.  The route ids are read with uniform (scalar) loads, which
// are counted apart from the vector loads, so waiting for them does not wait
// for the weights.  Columns of padding routes fetch no activation bytes.
// The single-block forms run three waves per SIMD (the 4-block variant two).
//
// VS (K/128 a multiple of U and aligned scale rows): kFp8 reads the U block
// scales of a group, and each route's U activation scales, with one 16-byte
// load each instead of U scattered ones; kW4 reads each of the lane's four
// rows' U bf16 scales with one 8-byte load instead of U 2-byte ones, and each
// route's U corrections with one 16-byte load.  Splits
// start on group boundaries, so with VS every group lies entirely inside its
// split.
// The software-pipelined single-block form (stream1; kW4 only with vector
// scales) keeps a group's loads in flight while the previous group computes;
// it fits three waves per SIMD.
template <int MAXB, int KIND, bool VS>
constexpr bool gemv_stream1() { return MAXB == 1 && (KIND != kW4 || VS); }

// Route slots of the decode GEMVs.  kGemvGrouped: blockIdx.y walks the
// active experts of the alignment, each wave one 16-row tile of that expert
// for all its routes.  kGemvDirect (one token): blockIdx.y is the route, its
// expert read from topk_ids, no alignment.  kGemvCombine (W2, one token per
// blockIdx.y): the workgroup is one 16-row tile, wave k computes route k and
// the top-k sum is taken in LDS (slot order, as moe_sum), so the layer output
// is written directly.
// kGemvDirectQ (kFp8 / kW4 with vector-loaded scales): kGemvDirect with act
// the bf16 x itself, each workgroup quantising its token's row into LDS with
// the quantiser's own code (kFp8: 1x128 groups; kW4: the per-row quantiser in
// w4 order with its block corrections, the token's row scale also written to
// xs_out by the workgroup of the token's first route slot) instead of a
// separate quantiser launch.
// kGemvDense (a plain GEMV, one expert): every row of act is a route of
// expert 0 in route-blocks of 16 consecutive rows; no alignment, no ids.
// kGemvDirectAct (kBf16 / kW8A16 W13, one token): the workgroup is one
// 16-column tile j of the activation for one route slot; wave w computes
// split w % splits of the gate rows (w < splits) or the up rows, the
// partials meet in LDS and are summed in split order -- the order of the
// activation kernels -- so the bf16 activation row is written by the W13
// launch itself, no partials and no activation launch.
constexpr int kGemvGrouped = 0, kGemvDirect = 1, kGemvCombine = 2, kGemvDirectQ = 3, kGemvDense = 4,
              kGemvDirectAct = 5;
constexpr int kMaxCombineSlots = 16;
// kW8A16 holds twice the activation registers: its combine workgroups take
// at most 8 slots, so that 256 VGPRs stay available.
constexpr int combine_slots(int kind) { return kind == kW8A16 ? 8 : kMaxCombineSlots; }
// Workgroup size bound of a mode: the combine one wave per slot, the fused
// activation two per split (kBf16 up to 8 splits; kW8A16, with twice the
// activation registers, up to 4).
constexpr int gemv_waves(int mode, int kind) {
  return mode == kGemvCombine ? combine_slots(kind) : mode == kGemvDirectAct ? (kind == kW8A16 ? 8 : 16) : kMoeGemvWaves;
}
constexpr int gemv_min_blocks(int mode, int maxb, int kind) {
  return mode == kGemvDirectAct ? 1 : (maxb == 1 && kind != kW8A16 ? 3 : 2);
}

// Local expert of a route, -1 when it is dropped (negative id, not mapped,
// or past the local experts) -- the rule of the alignment and of moe_sum.
__device__ __forceinline__ int route_expert(const int32_t* __restrict__ ids, int64_t route,
                                            const int32_t* __restrict__ emap, int64_t emap_len, int E) {
  int e = ids[route];
  if (e >= 0 && emap) e = e < emap_len ? emap[e] : -1;
  return e >= 0 && e < E ? e : -1;
}

template <int MAXB, int KIND, bool VS = false, int MODE = kGemvGrouped>
__global__ __launch_bounds__(gemv_waves(MODE, KIND) * kWave, gemv_min_blocks(MODE, MAXB, KIND)) void
moe_gemv_kernel(
    const uint8_t* __restrict__ act, int act_bytes, const float* __restrict__ act_s, int act_div,
    int K, const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ active, const int32_t* __restrict__ num_active,
    const uint8_t* __restrict__ w, const void* __restrict__ ws, int N, int numel, int splits,
    float* __restrict__ partial, const float* __restrict__ route_w, uint16_t* __restrict__ y,
    const int32_t* __restrict__ ids, const int32_t* __restrict__ emap, int64_t emap_len, int E_,
    uint16_t* __restrict__ comb, const float* __restrict__ comb_w, float* __restrict__ xs_out,
    float act_limit, int act_native) {
  using KB_ = KindBytes<KIND>;
  using AF = typename KindOps<KIND>::AFrag;
  constexpr bool kActS = KindOps<KIND>::kActScale, kBlkS = KindOps<KIND>::kBlockScale;
  constexpr int U = kGemvU;
  constexpr bool kStream1 = gemv_stream1<MAXB, KIND, VS>();
  static_assert(MODE == kGemvGrouped || MODE == kGemvDense || MAXB == 1,
                "direct route slots take one route per block");
  constexpr bool kQx = MODE == kGemvDirectQ;
  static_assert(!kQx || ((KIND == kFp8 || KIND == kW4) && VS && kStream1),
                "in-workgroup x quantiser: fp8 / w4, vector scales");
  constexpr bool kComb = MODE == kGemvCombine, kAct = MODE == kGemvDirectAct;
  static_assert(!kAct || KIND == kBf16 || KIND == kW8A16, "fused decode activation: bf16 activations");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const int li = lane % 16, lg = lane / 16;
  // kGemvDirectAct: wave -> (gate / up half, split); N / 32 = I / 16 tiles per half.
  const int act_splits = kAct ? splits : 1;
  const int ntile = kComb ? static_cast<int>(blockIdx.x)
                    : kAct ? (wave / act_splits) * (N / 32) + static_cast<int>(blockIdx.x)
                           : blockIdx.x * kMoeGemvWaves + wave;
  // Wave-uniform (workgroup-uniform for the combine and kGemvDirectAct,
  // whose only barrier comes after it); kGemvDirectQ leaves after its barrier.
  if (!kQx && ntile * 16 >= N) return;
  const int slot = kComb ? static_cast<int>(blockIdx.y * (blockDim.x / kWave)) + wave
                         : static_cast<int>(blockIdx.y);
  int e;
  bool dead = false;  // kGemvCombine: a dropped route still takes part in the sum's barrier
  if constexpr (MODE == kGemvGrouped) {
    // The exit test reads both values, so both loads are in flight together;
    // active[] has one entry per expert and gridDim.y never exceeds the
    // expert count, so the read is in bounds.
    e = active[slot];
    const int na = num_active[0];
    if (slot >= na || e < 0) return;
  } else if constexpr (MODE == kGemvDense) {
    e = 0;
  } else if constexpr (MODE == kGemvDirect || MODE == kGemvDirectQ || kAct) {
    e = route_expert(ids, slot, emap, emap_len, E_);  // workgroup-uniform
    // kW4: the workgroup that writes the token's row scale runs the quantiser
    // even when its route is dropped.
    const bool writes_xs = KIND == kW4 && kQx && blockIdx.x == 0 && blockIdx.z == 0 && slot % act_div == 0;
    if (e < 0 && !writes_xs) {
      if constexpr (kAct) {  // a dropped route's activation columns are zeros
        if (wave == 0 && lane < 16) y[static_cast<int64_t>(slot) * (N / 2) + static_cast<int>(blockIdx.x) * 16 + lane] = 0;
      }
      return;
    }
  } else {
    e = route_expert(ids, slot, emap, emap_len, E_);
    dead = e < 0;
    e = dead ? 0 : e;
  }
  extern __shared__ __attribute__((aligned(16))) uint8_t qx_lds[];
  const int split = kAct ? wave % act_splits : static_cast<int>(blockIdx.z);
  const int KS = K / KB_::kElems;                    // K steps
  const int arowb = KS * KB_::kAct;
  const int64_t wrowb = static_cast<int64_t>(KS) * KB_::kW;
  const int NB = (N + 127) / 128;
  const int groups = (KS + kGemvU - 1) / kGemvU;  // splits start on group boundaries
  // The combine runs all of K in one chain (splits: the grouped W2 path's
  // count, at most groups, so no split is empty).
  const int kb0 = kComb ? 0 : split * groups / splits * kGemvU;
  const int kb1 = kComb ? KS : min((split + 1) * groups / splits * kGemvU, KS);
  const int n = ntile * 16 + 4 * lg;
  const uint8_t* wrow = w + (static_cast<int64_t>(e) * N + ntile * 16 + li) * wrowb;
  const float* wsr = nullptr;                        // kFp8 / kW8A16: block scales of the 16 rows
  const uint16_t* wsw[4] = {nullptr, nullptr, nullptr, nullptr};  // kW4: scales of rows n..n+3
  if constexpr (kBlkS)
    wsr = static_cast<const float*>(ws) + (static_cast<int64_t>(e) * NB + (ntile * 16) / 128) * KS;
  if constexpr (KIND == kW4) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      wsw[r] = static_cast<const uint16_t*>(ws) + (static_cast<int64_t>(e) * N + n + r) * KS;
  }
  // Block scales of the wave's rows through a descriptor: uniform values
  // read by vector loads, which queue behind the weight loads instead of
  // making the weight stream wait for scalar loads.
  const __amdgpu_buffer_rsrc_t wsrs = buffer_rsrc(wsr, kBlkS ? KS * 4 : 0);
  const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(act, act_bytes);
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(act_s, kActS ? act_bytes / 32 : 0);
  const v4f zero = {0.f, 0.f, 0.f, 0.f};

  // One K group of weights (U steps from kb, clamped to the split's range).
  // kW4 with one route block keeps the weights packed (half the registers:
  // more waves, more bytes in flight) and converts each fragment right before
  // its MFMA; with several blocks a fragment is converted once per group.
  constexpr bool kRawW4 = KIND == kW4 && MAXB == 1;
  v8i wf[kRawW4 ? 1 : U];
  v4i wraw[kRawW4 ? U : 1];
  uint2 swr[4];  // kW4 + VS: packed bf16 scales, U per row
  float sb[U];
  v4f sw[U];
  auto load_w = [&](int kb) {
    if constexpr (VS) {
      const v4f s4 = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(wsrs, kb * 4, 0, 0));
#pragma unroll
      for (int u = 0; u < U; ++u) sb[u] = s4[u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = min(kb + u, kb1 - 1);
      if constexpr (kRawW4)
        wraw[u] = ld16(wrow + static_cast<int64_t>(k) * KB_::kW + 16 * lg);
      else
        wf[u] = weight_frag<KIND>(wrow + static_cast<int64_t>(k) * KB_::kW, lg);
      if constexpr (!VS) sb[u] = 0.f;
      sw[u] = zero;
      if constexpr (kBlkS && !VS)
        sb[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsrs, k * 4, 0, 0));
      if constexpr (KIND == kW4 && !VS)
        sw[u] = v4f{bf16_to_f32(wsw[0][k]), bf16_to_f32(wsw[1][k]), bf16_to_f32(wsw[2][k]),
                    bf16_to_f32(wsw[3][k])};
    }
    if constexpr (KIND == kW4 && VS) {  // each row's U scales: one 8-byte load
#pragma unroll
      for (int r = 0; r < 4; ++r) swr[r] = *reinterpret_cast<const uint2*>(wsw[r] + kb);
    }
  };
  // Scales of step u of the group for the lane's four rows (kW4).
  auto w4_scales = [&](int u) -> v4f {
    if constexpr (KIND == kW4 && VS) {
      auto pick = [u](const uint2& v) {
        const uint32_t w = u < 2 ? v.x : v.y;
        return __uint_as_float((u & 1) ? (w & 0xFFFF0000u) : (w << 16));
      };
      return v4f{pick(swr[0]), pick(swr[1]), pick(swr[2]), pick(swr[3])};
    } else {
      return sw[u];
    }
  };
  uint32_t aoff[MAXB];  // byte offset of each block's activation row (kBufferOff: padding)
  v4f acc[MAXB];
  // kGemvCombine: at each split boundary of the grouped W2 GEMV the split's
  // accumulator (times kW4Unit for kW4, as its partials) joins the sum of the
  // finished splits, added in split order as moe_w2_reduce_kernel adds them,
  // and the next split starts from zero.  Boundaries fall on group starts.
  v4f tot = zero;
  int cut = kComb && splits > 1 ? groups / splits * kGemvU : KS, cuts = 1;
  auto fold = [&](int kb) {
    if constexpr (kComb) {
      if (kb == cut) {  // uniform
        const v4f a = KIND == kW4 ? acc[0] * kW4Unit : acc[0];
        tot = cuts == 1 ? a : tot + a;
        acc[0] = zero;
        ++cuts;
        cut = cuts < splits ? cuts * groups / splits * kGemvU : KS;
      }
    }
  };
  // Activation loads and MFMAs of the group at kb with the weights in wf.
  // Steps past the split's end take masked (zero) activations, so the group
  // has no branches: their products are exactly zero.
  auto group = [&](int kb, int nb) {
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      if (b < nb) {
        AF xf[U];
        float as[U];
        if constexpr (VS && kActS) {  // scale byte offset = activation byte offset / 32
          const uint32_t off = aoff[b] != kBufferOff ? aoff[b] / 32 + static_cast<uint32_t>(kb * 4) : kBufferOff;
          const v4f s4 = __builtin_bit_cast(
              v4f, __builtin_amdgcn_raw_buffer_load_b128(srs, static_cast<int>(off), 0, 0));
#pragma unroll
          for (int u = 0; u < U; ++u) as[u] = s4[u];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const bool live = aoff[b] != kBufferOff && kb + u < kb1;
          const uint32_t off = live ? aoff[b] + static_cast<uint32_t>((kb + u) * KB_::kAct) : kBufferOff;
          xf[u] = buffer_frag<KIND>(ars, off, lg);
          if constexpr (!VS || !kActS) as[u] = 0.f;
          if constexpr (kActS && !VS)  // scale byte offset = activation byte offset / 32
            as[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  srs, static_cast<int>(live ? off / 32 : kBufferOff), 0, 0));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if constexpr (KIND == kFp8) {
            fma4(acc[b], mfma_fp8(wf[u], xf[u], zero), as[u] * sb[u]);
          } else if constexpr (KIND == kW8A16) {
            fma4(acc[b], mfma_w8a16(wf[u], xf[u], zero), sb[u]);
          } else if constexpr (KIND == kW4) {
            if constexpr (kRawW4)
              fma4v(acc[b], mfma_fp8(w4_frag(wraw[u]), xf[u], splat4(as[u])), w4_scales(u));
            else
              fma4v(acc[b], mfma_fp8(wf[u], xf[u], splat4(as[u])), w4_scales(u));
          } else {
            acc[b] = mfma_bf16x2(wf[u], xf[u], acc[b]);
          }
        }
      }
    }
  };

  // One route block (int4 only with vector-loaded scales: the other int4
  // form needs more registers than its occupancy leaves): the K loop is
  // software-pipelined.  Slot u
  // holds step kb + u's weights, activations and scales; right after its MFMA
  // the slot is refilled with step kb + U + u, and a group's vector-loaded
  // scales are copied out and their successors requested before its first
  // MFMA, so U steps stay in flight instead of draining at every group.
  // The weights of group kb0 were requested by the caller.
  auto stream1 = [&](int kbs) {
    AF xf[U];
    float as[U];
    auto load_act = [&](int kb, int u) {
      const bool live = aoff[0] != kBufferOff && kb + u < kb1;
      if constexpr (kQx) {  // the route's column (li == 0) from LDS, zeros elsewhere
        const int k = (kb + u) * 128;  // layouts of buffer_frag
        const int o0 = KIND == kW4 ? 32 * lg : 16 * lg, o1 = KIND == kW4 ? 32 * lg + 16 : 64 + 16 * lg;
        xf[u] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        if (live) {
          const v4i lo = lds_load<v4i>(qx_lds, k + o0);
          const v4i hi = lds_load<v4i>(qx_lds, k + o1);
          xf[u] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        return;
      }
      const uint32_t off = live ? aoff[0] + static_cast<uint32_t>((kb + u) * KB_::kAct) : kBufferOff;
      xf[u] = buffer_frag<KIND>(ars, off, lg);
      if constexpr (kActS && !VS)
        as[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              srs, static_cast<int>(live ? off / 32 : kBufferOff), 0, 0));
    };
    auto load_as_vs = [&](int kb) {  // the group's U activation scales
      if constexpr (kQx) return lds_load<v4f>(qx_lds, K + 4 * kb);
      const uint32_t off = aoff[0] != kBufferOff ? aoff[0] / 32 + static_cast<uint32_t>(kb * 4) : kBufferOff;
      return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(srs, static_cast<int>(off), 0, 0));
    };
    auto load_w_slot = [&](int kb, int u) {
      const int k = min(kb + u, kb1 - 1);
      if constexpr (kRawW4)
        wraw[u] = ld16(wrow + static_cast<int64_t>(k) * KB_::kW + 16 * lg);
      else
        wf[u] = weight_frag<KIND>(wrow + static_cast<int64_t>(k) * KB_::kW, lg);
      if constexpr (kBlkS && !VS)
        sb[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsrs, k * 4, 0, 0));
      if constexpr (KIND == kW4 && !VS)
        sw[u] = v4f{bf16_to_f32(wsw[0][k]), bf16_to_f32(wsw[1][k]), bf16_to_f32(wsw[2][k]),
                    bf16_to_f32(wsw[3][k])};
    };
    v4f asn = zero;
    if constexpr (VS && kActS) asn = load_as_vs(kbs);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (!VS || !kActS) as[u] = 0.f;
      load_act(kbs, u);
    }
    for (int kb = kbs; kb < kb1; kb += U) {
      const bool more = kb + U < kb1;  // uniform
      fold(kb);
      // This group's vector-loaded scales, then the next group's requests.
      float sbc[U];
      uint2 swc[4];
#pragma unroll
      for (int u = 0; u < U; ++u) sbc[u] = sb[u];
#pragma unroll
      for (int r = 0; r < 4; ++r) swc[r] = swr[r];
      if constexpr (VS) {
        if constexpr (kActS) {
#pragma unroll
          for (int u = 0; u < U; ++u) as[u] = asn[u];
        }
        if (more) {
          if constexpr (kActS) asn = load_as_vs(kb + U);
          if constexpr (kBlkS) {
            const v4f s4 = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(wsrs, (kb + U) * 4, 0, 0));
#pragma unroll
            for (int u = 0; u < U; ++u) sb[u] = s4[u];
          }
          if constexpr (KIND == kW4) {
#pragma unroll
            for (int r = 0; r < 4; ++r) swr[r] = *reinterpret_cast<const uint2*>(wsw[r] + kb + U);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if constexpr (KIND == kFp8) {
          fma4(acc[0], mfma_fp8(wf[u], xf[u], zero), as[u] * (VS ? sbc[u] : sb[u]));
        } else if constexpr (KIND == kW8A16) {
          fma4(acc[0], mfma_w8a16(wf[u], xf[u], zero), VS ? sbc[u] : sb[u]);
        } else if constexpr (KIND == kW4) {
          v4f sc;
          if constexpr (VS) {
            const uint32_t lo = u < 2 ? 0 : 1;
            auto pick = [&](const uint2& v) {
              const uint32_t w = lo ? v.y : v.x;
              return __uint_as_float((u & 1) ? (w & 0xFFFF0000u) : (w << 16));
            };
            sc = v4f{pick(swc[0]), pick(swc[1]), pick(swc[2]), pick(swc[3])};
          } else {
            sc = sw[u];
          }
          fma4v(acc[0], mfma_fp8(w4_frag(wraw[u]), xf[u], splat4(as[u])), sc);
        } else {
          acc[0] = mfma_bf16x2(wf[u], xf[u], acc[0]);
        }
        if (more) {
          load_w_slot(kb + U, u);
          load_act(kb + U, u);
        }
      }
    }
  };

  // kQx with kFp8: the first K group of weights is requested before the
  // workgroup quantises its token's row (the weights do not depend on it), so
  // the weight stream starts with the x loads instead of after the quantiser
  // (DeepSeek-V3 W13 at one token 47.8 -> 45.6 us).  kW4's row quantiser,
  // whose row maximum waits behind those loads, measured 15.0 -> 15.7 us and
  // keeps the order.
  constexpr bool kEarlyW = kQx && KIND == kFp8;
  if constexpr (kEarlyW) {
    if (e >= 0 && ntile * 16 < N) load_w(kb0);
  }
  // kQx LDS: [K] fp8 (kW4: w4 order), [K/128] f32 (kFp8: group scales,
  // kW4: block corrections), kW4 then the row scale and 4 wave maxima.
  if constexpr (kQx) {
    const int gpr = K / 128;
    const uint16_t* xrow = reinterpret_cast<const uint16_t*>(act) + static_cast<int64_t>(slot / act_div) * K;
    float* qs = reinterpret_cast<float*>(qx_lds + K);
    if constexpr (KIND == kFp8) {
      for (int g0 = 0; g0 < gpr; g0 += static_cast<int>(blockDim.x) / kLanesPerGroup) {
        const int g = g0 + static_cast<int>(threadIdx.x) / kLanesPerGroup;  // uniform over a group's lanes
        if (g < gpr)
          group_quant_group<kBF16>(xrow, K, gpr, g, threadIdx.x % kLanesPerGroup, true, 1e-10f, -448.f, 448.f,
                                   qx_lds, K, qs, 0, 1);
      }
      __syncthreads();
    } else {  // one kRowThreads part: the whole workgroup (it synchronises the block)
      float* rs = qs + gpr;
      row_quant_part<true>(xrow, K, K, 1e-4f, -448.f, 448.f, qx_lds, rs, 0, true, threadIdx.x, rs + 1, qs);
      __syncthreads();
      if (blockIdx.x == 0 && blockIdx.z == 0 && slot % act_div == 0 && threadIdx.x == 0)
        xs_out[slot / act_div] = rs[0];
      if (e < 0) return;  // the row scale's writer of a dropped route
    }
    if (ntile * 16 >= N) return;
  }
  int seg0 = 0, nblk = 1;
  if constexpr (MODE == kGemvGrouped) {
    seg0 = offsets[e];
    nblk = (offsets[e + 1] - seg0) / kGemvBlock;  // >= 1 for an active expert
  } else if constexpr (MODE == kGemvDense) {
    nblk = (numel + kGemvBlock - 1) / kGemvBlock;
  }
  int b0 = 0;
  if (!dead) do {
    if (!kEarlyW) load_w(kb0);  // first group: in flight while the routes are resolved
    const int nb = min(MAXB, nblk - b0);
    int rr[MAXB];
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      int r = numel;
      if constexpr (MODE == kGemvDense) {
        r = b < nb ? (b0 + b) * kGemvBlock + li : numel;  // rows past numel are padding
      } else if constexpr (MODE != kGemvGrouped) {
        r = li == 0 ? slot : numel;  // column 0 of the block holds the route
      } else if (b < nb) {
        const int32_t* bids = sorted + seg0 + (b0 + b) * kGemvBlock;
        int sid[kGemvBlock];
#pragma unroll
        for (int j = 0; j < kGemvBlock; ++j) sid[j] = bids[j];
        r = sid[0];
#pragma unroll
        for (int j = 1; j < kGemvBlock; ++j) r = li == j ? sid[j] : r;
      }
      const bool valid = r >= 0 && r < numel;
      rr[b] = valid ? r : -1;
      aoff[b] = valid ? static_cast<uint32_t>((r / act_div) * arowb) : kBufferOff;
      acc[b] = zero;
    }
    if constexpr (kStream1) {
      stream1(kb0);
    } else {
      group(kb0, nb);
      for (int kb = kb0 + U; kb < kb1; kb += U) {
        load_w(kb);
        fold(kb);
        group(kb, nb);
      }
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      if (b >= nb || rr[b] < 0) continue;
      const int r = rr[b];
      const v4f a = KIND == kW4 ? acc[b] * kW4Unit : acc[b];
      if constexpr (kComb || kAct) {
        break;  // the sum / the activation below
      } else if (y) {
        const float rw = route_w ? route_w[r] : 1.0f;
        *reinterpret_cast<uint2*>(y + static_cast<int64_t>(r) * N + n) =
            pack_bf16x4(a[0] * rw, a[1] * rw, a[2] * rw, a[3] * rw);
      } else {
        *reinterpret_cast<float4*>(partial + (static_cast<int64_t>(split) * numel + r) * N + n) =
            float4{a[0], a[1], a[2], a[3]};
      }
    }
    b0 += MAXB;
  } while (b0 < nblk);
  if constexpr (kComb) {  // the last split
    const v4f a = KIND == kW4 ? acc[0] * kW4Unit : acc[0];
    tot = cuts == 1 ? a : tot + a;
  }
  if constexpr (kAct) {
    // Gate / up sums over the splits in split order, times route_w (null:
    // times 1, exact), then the activation of the decode activation kernels:
    // act_native the reference GEMV's (fp32 through the SwiGLU, one rounding),
    // otherwise swiglu_bf16 on the bf16-rounded gate and up.
    __shared__ float apart[gemv_waves(kGemvDirectAct, KIND) * 16];
    if (li == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) apart[wave * 16 + 4 * lg + q] = acc[0][q];
    }
    __syncthreads();
    if (wave == 0 && lane < 16) {
      float g = apart[lane], u = apart[act_splits * 16 + lane];
      for (int s = 1; s < act_splits; ++s) {
        g += apart[s * 16 + lane];
        u += apart[(act_splits + s) * 16 + lane];
      }
      const int I = N / 2;
      float v;
      if (act_native) {
        if (route_w) {
          g *= route_w[slot];
          u *= route_w[slot];
        }
        if (act_limit > 0.f) {
          g = fminf(g, act_limit);
          u = fminf(fmaxf(u, -act_limit), act_limit);
        }
        v = g * (1.0f / (1.0f + expf(-g))) * u;
      } else {
        const float sc = route_w ? route_w[slot] : 1.0f;
        v = swiglu_bf16(bf16r(g * sc), bf16r(u * sc), act_limit);
      }
      y[static_cast<int64_t>(slot) * I + static_cast<int>(blockIdx.x) * 16 + lane] = f32_to_bf16(v);
    }
  }
  if constexpr (kComb) {
    // y_k = bf16(acc * route_w[k]) for the 16 rows (lanes of column 0), as
    // the per-route epilogue above; then the layer output = bf16 of the fp32
    // sum over the live slots in slot order, y_k times comb_w[k] by one fma
    // when given -- the rule of moe_sum.
    __shared__ float part[kMaxCombineSlots * 16];
    __shared__ int live[kMaxCombineSlots];
    if (li == 0 && !dead) {
      const float rw = route_w ? route_w[slot] : 1.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) part[wave * 16 + 4 * lg + q] = bf16r(tot[q] * rw);
    }
    if (lane == 0) live[wave] = dead ? 0 : 1;
    __syncthreads();
    if (wave == 0 && lane < 16) {
      const int nslots = blockDim.x / kWave;
      const int64_t first = static_cast<int64_t>(blockIdx.y) * nslots;
      float s = 0.0f;
      for (int k = 0; k < nslots; ++k) {
        if (!live[k]) continue;
        const float v = part[k * 16 + lane];
        s = comb_w ? __builtin_fmaf(v, comb_w[first + k], s) : s + v;
      }
      comb[static_cast<int64_t>(blockIdx.y) * N + ntile * 16 + lane] = f32_to_bf16(s);
    }
  }
}

// Gate/up sums of 8 consecutive columns c0.. of route r: split partials in a
// fixed order, times `scale`.
__device__ __forceinline__ void gate_up8(const float* __restrict__ partial, int splits, int numel,
                                         int I, int r, int c0, float scale, float (&g)[8],
                                         float (&u)[8]) {
  const int64_t plane = static_cast<int64_t>(numel) * 2 * I;
  const float* src = partial + static_cast<int64_t>(r) * 2 * I + c0;
#pragma unroll
  for (int j = 0; j < 8; j += 4) {
    float4 gs = *reinterpret_cast<const float4*>(src + j);
    float4 us = *reinterpret_cast<const float4*>(src + I + j);
    for (int s = 1; s < splits; ++s) {
      const float4 ga = *reinterpret_cast<const float4*>(src + s * plane + j);
      const float4 ua = *reinterpret_cast<const float4*>(src + s * plane + I + j);
      gs.x += ga.x; gs.y += ga.y; gs.z += ga.z; gs.w += ga.w;
      us.x += ua.x; us.y += ua.y; us.z += ua.z; us.w += ua.w;
    }
    g[j + 0] = gs.x * scale; g[j + 1] = gs.y * scale; g[j + 2] = gs.z * scale; g[j + 3] = gs.w * scale;
    u[j + 0] = us.x * scale; u[j + 1] = us.y * scale; u[j + 2] = us.z * scale; u[j + 3] = us.w * scale;
  }
}

// gate_up8 with the split count fixed (SPL <= 4): all loads are issued before
// the first add, which keeps the same summation order.
template <int SPL>
__device__ __forceinline__ void gate_up8_fixed(const float* __restrict__ partial, int numel, int I,
                                               int r, int c0, float (&g)[8], float (&u)[8]) {
  const int64_t plane = static_cast<int64_t>(numel) * 2 * I;
  const float* src = partial + static_cast<int64_t>(r) * 2 * I + c0;
  float4 gs[2][SPL], us[2][SPL];
#pragma unroll
  for (int s = 0; s < SPL; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      gs[h][s] = *reinterpret_cast<const float4*>(src + s * plane + 4 * h);
      us[h][s] = *reinterpret_cast<const float4*>(src + s * plane + I + 4 * h);
    }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float4 a = gs[h][0], b = us[h][0];
#pragma unroll
    for (int s = 1; s < SPL; ++s) {
      a.x += gs[h][s].x; a.y += gs[h][s].y; a.z += gs[h][s].z; a.w += gs[h][s].w;
      b.x += us[h][s].x; b.y += us[h][s].y; b.z += us[h][s].z; b.w += us[h][s].w;
    }
    g[4 * h + 0] = a.x; g[4 * h + 1] = a.y; g[4 * h + 2] = a.z; g[4 * h + 3] = a.w;
    u[4 * h + 0] = b.x; u[4 * h + 1] = b.y; u[4 * h + 2] = b.z; u[4 * h + 3] = b.w;
  }
}

// kFp8: activation then a2 quantisation per 1x128 group (one 16-lane segment
// per group, 8 columns per lane).  NaN activations (clamped variant) quantise
// to fp8_min.  SPL > 0: the split count, fixed at compile time; 0: runtime.
// route_w (apply_router_weight_on_input): gate/up sums times the route's
// weight before their bf16 rounding (null: times 1, which is exact).
template <int SPL>
__global__ __launch_bounds__(256) void moe_act_quant_kernel(const float* __restrict__ partial,
                                                            int splits, int numel, int I,
                                                            float limit, const float* __restrict__ route_w,
                                                            uint8_t* __restrict__ a2q,
                                                            float* __restrict__ a2s) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 16 + threadIdx.x / 16;
  const int sub = threadIdx.x % 16;
  const int gpr = I / 128;
  if (g >= static_cast<int64_t>(numel) * gpr) return;
  const int r = static_cast<int>(g / gpr);
  const int c0 = static_cast<int>(g % gpr) * 128 + sub * 8;
  float gv[8], uv[8], v[8];
  const float rw = route_w ? route_w[r] : 1.0f;
  if constexpr (SPL > 0)
    gate_up8_fixed<SPL>(partial, numel, I, r, c0, gv, uv);
  else
    gate_up8(partial, splits, numel, I, r, c0, 1.0f, gv, uv);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = swiglu_bf16(bf16r(gv[j] * rw), bf16r(uv[j] * rw), limit);
  float amax = 1e-10f;
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = group_max<16>(amax);
  const float scale = amax / 448.0f;
  if (sub == 0) a2s[static_cast<int64_t>(r) * gpr + c0 / 128] = scale;
  const float rs = 1.0f / scale;
  const float lo[4] = {v[0], v[1], v[2], v[3]}, hi[4] = {v[4], v[5], v[6], v[7]};
  uint2 out;
  out.x = quant4_e4m3(lo, scale, rs);
  out.y = quant4_e4m3(hi, scale, rs);
  *reinterpret_cast<uint2*>(a2q + static_cast<int64_t>(r) * I + c0) = out;
}

// kBf16 / kW4: a[r, c] = the bf16 activation, 8 columns per thread (16-byte
// store).  kW4 first scales the sums by the token's activation scale
// xs[r / topk] and rounds gate/up to bf16, then applies swiglu_w4; its a2
// quantiser (one scale per row) runs as a separate row kernel.  kBf16 scales
// the sums by route_w[r] when given (apply_router_weight_on_input).
template <int KIND>
__global__ __launch_bounds__(256) void moe_act_bf16_kernel(const float* __restrict__ partial,
                                                           int splits, int numel, int I,
                                                           float limit, const float* __restrict__ xs,
                                                           int topk, const float* __restrict__ route_w,
                                                           uint16_t* __restrict__ a2) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int cpr = I / 8;
  if (idx >= static_cast<int64_t>(numel) * cpr) return;
  const int r = static_cast<int>(idx / cpr);
  const int c0 = static_cast<int>(idx % cpr) * 8;
  const float scale = KIND == kW4 ? xs[r / topk] : (route_w ? route_w[r] : 1.0f);
  float gv[8], uv[8], v[8];
  gate_up8(partial, splits, numel, I, r, c0, scale, gv, uv);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    v[j] = KIND == kW4 ? swiglu_w4(bf16r(gv[j]), bf16r(uv[j]), limit)
                       : swiglu_bf16(bf16r(gv[j]), bf16r(uv[j]), limit);
  uint4 o;
  o.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  o.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
  o.z = static_cast<uint32_t>(f32_to_bf16(v[4])) | (static_cast<uint32_t>(f32_to_bf16(v[5])) << 16);
  o.w = static_cast<uint32_t>(f32_to_bf16(v[6])) | (static_cast<uint32_t>(f32_to_bf16(v[7])) << 16);
  *reinterpret_cast<uint4*>(a2 + static_cast<int64_t>(r) * I + c0) = o;
}

// A route's slot is live when its expert id is >= 0 and its local id
// (through expert_map when given) lies in [0, E): the rule of the alignment,
// which places no other route, so no other partial row is ever written.
// Without ids (a plain GEMV) every route is live.
__device__ __forceinline__ bool route_live(const int32_t* __restrict__ emap, int64_t emap_len, int E,
                                           int e) {
  if (e < 0) return false;
  if (emap) {
    if (e >= emap_len) return false;
    e = emap[e];
  }
  return e >= 0 && e < E;
}
__device__ __forceinline__ bool route_live_at(const int32_t* __restrict__ ids, int64_t r,
                                              const int32_t* __restrict__ emap, int64_t emap_len, int E) {
  return ids == nullptr || route_live(emap, emap_len, E, ids[r]);
}

// The reference's GEMV-MoE activation (csrc/musa/gemv.mu:472-487): per
// route r the gate/up sums of the W13 partials (split order), times
// route_w[r] when given (before the activation), the gate clamped to <= L and
// up to [-L, L] when L > 0, then g * sigmoid(g) * u in fp32 and one rounding
// to bf16; nothing is rounded before.  Routes without a live expert write
// zeros (gemv.mu:297-311).  8 columns per thread.
template <int SPL>
__global__ __launch_bounds__(256) void moe_act_native_kernel(const float* __restrict__ partial, int splits,
                                                             int numel, int I, float limit,
                                                             const float* __restrict__ route_w,
                                                             const int32_t* __restrict__ ids,
                                                             const int32_t* __restrict__ emap, int64_t emap_len,
                                                             int E, uint16_t* __restrict__ a2) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int cpr = I / 8;
  if (idx >= static_cast<int64_t>(numel) * cpr) return;
  const int r = static_cast<int>(idx / cpr);
  const int c0 = static_cast<int>(idx % cpr) * 8;
  uint4 o = {0u, 0u, 0u, 0u};
  if (route_live_at(ids, r, emap, emap_len, E)) {
    float gv[8], uv[8], v[8];
    if constexpr (SPL > 0)
      gate_up8_fixed<SPL>(partial, numel, I, r, c0, gv, uv);
    else
      gate_up8(partial, splits, numel, I, r, c0, 1.0f, gv, uv);
    const float rw = route_w ? route_w[r] : 1.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float g = route_w ? gv[j] * rw : gv[j];
      float u = route_w ? uv[j] * rw : uv[j];
      if (limit > 0.f) {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
      }
      v[j] = g * (1.0f / (1.0f + expf(-g))) * u;
    }
    o.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
    o.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
    o.z = static_cast<uint32_t>(f32_to_bf16(v[4])) | (static_cast<uint32_t>(f32_to_bf16(v[5])) << 16);
    o.w = static_cast<uint32_t>(f32_to_bf16(v[6])) | (static_cast<uint32_t>(f32_to_bf16(v[7])) << 16);
  }
  *reinterpret_cast<uint4*>(a2 + static_cast<int64_t>(r) * I + c0) = o;
}

// kW4 decode: moe_act_bf16_kernel<kW4> and the per-row a2 quantiser in one
// pass, one kRowThreads block per route row: the bf16-rounded activations stay
// in registers for the row maximum and the quantiser (the values the separate
// quantiser would read back), so neither the bf16 activation nor a second
// launch is needed.  a2q is written in w4 order with its block corrections
// a2corr [numel, I/128].  I <= kRowThreads * 8 * kRowChunks.
__global__ __launch_bounds__(kRowThreads) void moe_act_rowquant_w4_kernel(
    const float* __restrict__ partial, int splits, int numel, int I, float limit,
    const float* __restrict__ xs, int topk, uint8_t* __restrict__ a2q, float* __restrict__ a2s,
    float* __restrict__ a2corr) {
  __shared__ float red[kRowThreads / kWave];
  const int r = blockIdx.x;
  const int nchunk = I / 8;
  const float scale = xs[r / topk];
  float v[kRowChunks][8];
  float amax = 1e-4f;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int ch = threadIdx.x + c * kRowThreads;
    if (ch < nchunk) {
      float gv[8], uv[8];
      gate_up8(partial, splits, numel, I, r, ch * 8, scale, gv, uv);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[c][j] = bf16r(swiglu_w4(bf16r(gv[j]), bf16r(uv[j]), limit));
        amax = fmaxf(amax, fabsf(v[c][j]));
      }
    }
  }
  amax = wave_max(amax);
  if (lane_id() == 0) red[threadIdx.x / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
  const float s = amax / 448.0f;
  if (threadIdx.x == 0) a2s[r] = s;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int ch = threadIdx.x + c * kRowThreads;
    if (ch < nchunk)
      w4_store_chunk(a2q + static_cast<int64_t>(r) * I, a2corr + static_cast<int64_t>(r) * (I / 128), ch,
                     v[c], s, -448.0f, 448.0f);
  }
}

// kW4 prefill: the per-row a2 quantiser of the bf16 activation for the
// padded route rows below ntpp[0], in w4 order with the block corrections
// a2corr [rows, I/128].  CPL > 0: one wave per row (I <= 512 * CPL, four rows
// per workgroup); CPL = 0: one kRowThreads workgroup per row.
template <int CPL>
__global__ __launch_bounds__(kRowThreads) void moe_rowquant_w4_kernel(
    const uint16_t* __restrict__ a, int I, const int32_t* __restrict__ ntpp, uint8_t* __restrict__ a2q,
    float* __restrict__ a2s, float* __restrict__ a2corr) {
  if constexpr (CPL > 0) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kRowThreads / kWave) + threadIdx.x / kWave;
    row_quant_wave<true, CPL>(a, I, I, 1e-4f, -448.f, 448.f, a2q, a2s, row, row < ntpp[0], a2corr);
  } else {
    if (static_cast<int>(blockIdx.x) >= ntpp[0]) return;  // uniform: past the last block
    __shared__ float red[kRowThreads / kWave];
    row_quant_part<true>(a, I, I, 1e-4f, -448.f, 448.f, a2q, a2s, blockIdx.x, true, threadIdx.x, red,
                         a2corr);
  }
}

// Launch of moe_rowquant_w4_kernel over `rows` padded route rows.
static void launch_rowquant_w4(const uint16_t* a, int I, int64_t rows, const int32_t* ntpp,
                               uint8_t* a2q, float* a2s, float* a2corr, hipStream_t st) {
  const int cpl = (I + 511) / 512;
  const unsigned waves_grid = static_cast<unsigned>((rows + kRowThreads / kWave - 1) / (kRowThreads / kWave));
#define VMAMD_RQ(C) \
  moe_rowquant_w4_kernel<C><<<waves_grid, kRowThreads, 0, st>>>(a, I, ntpp, a2q, a2s, a2corr)
  switch (cpl) {
    case 1: VMAMD_RQ(1); break;
    case 2: VMAMD_RQ(2); break;
    case 3: VMAMD_RQ(3); break;
    case 4: VMAMD_RQ(4); break;
    case 5: case 6: VMAMD_RQ(6); break;
    case 7: case 8: VMAMD_RQ(8); break;
    default:
      moe_rowquant_w4_kernel<0><<<static_cast<unsigned>(rows), kRowThreads, 0, st>>>(a, I, ntpp, a2q, a2s,
                                                                                    a2corr);
  }
#undef VMAMD_RQ
}

// y[r, n] = bf16(sum_s partial[s, r, n] * w_r) for the W2 split path (kW4:
// w_r is the a2 row scale).  Rows of dead routes are left alone, or written
// as zeros with ZERO_DEAD (the reference GEMV's rule, gemv.mu:297-311).
template <bool ZERO_DEAD = false>
__global__ __launch_bounds__(256) void moe_w2_reduce_kernel(const float* __restrict__ partial,
                                                            int splits, int numel, int N,
                                                            const int32_t* __restrict__ ids,
                                                            const int32_t* __restrict__ emap,
                                                            int64_t emap_len, int E,
                                                            const float* __restrict__ route_w,
                                                            uint16_t* __restrict__ y) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int64_t mn = static_cast<int64_t>(numel) * N;
  if (i4 >= mn) return;
  const int r = static_cast<int>(i4 / N);
  if (!route_live_at(ids, r, emap, emap_len, E)) {
    if constexpr (ZERO_DEAD) *reinterpret_cast<uint2*>(y + i4) = uint2{0u, 0u};
    return;
  }
  float4 acc = *reinterpret_cast<const float4*>(partial + i4);
  for (int s = 1; s < splits; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(partial + s * mn + i4);
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const float rw = route_w ? route_w[r] : 1.0f;
  *reinterpret_cast<uint2*>(y + i4) = pack_bf16x4(acc.x * rw, acc.y * rw, acc.z * rw, acc.w * rw);
}

// Decode W2 with split-K partials, reduce and top-k combine in one pass:
//   out[t, n] = bf16( sum_k y_k ),  y_k = bf16(sum_s partial[s, r, n] * yscale[r])
// (kW4: sum_k fma(y_k, topk_weights[r], .), yscale being the a2 row scale),
// r = t * topk + k in slot order -- the same operations, in the same order, as
// moe_w2_reduce_kernel followed by the top-k sum, without the y round trip.
// Slots of dropped routes (negative id, or not local through expert_map) are
// skipped; their partial rows were never written.
template <bool WEIGHTED>
__global__ __launch_bounds__(256) void moe_w2_combine_kernel(
    const float* __restrict__ partial, int splits, int T, int topk, int N,
    const int32_t* __restrict__ ids, const int32_t* __restrict__ emap, int64_t emap_len, int E,
    const float* __restrict__ yscale, const float* __restrict__ topk_w, uint16_t* __restrict__ out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int cpr = N / 8;
  if (i >= static_cast<int64_t>(T) * cpr) return;
  const int t = static_cast<int>(i / cpr);
  const int n = static_cast<int>(i % cpr) * 8;
  const int64_t mn = static_cast<int64_t>(T) * topk * N;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < topk; ++k) {
    const int r = t * topk + k;
    if (!route_live(emap, emap_len, E, ids[r])) continue;
    const float* src = partial + static_cast<int64_t>(r) * N + n;
    float4 a = *reinterpret_cast<const float4*>(src);
    float4 b = *reinterpret_cast<const float4*>(src + 4);
    for (int sp = 1; sp < splits; ++sp) {
      const float4 c = *reinterpret_cast<const float4*>(src + sp * mn);
      const float4 d = *reinterpret_cast<const float4*>(src + sp * mn + 4);
      a.x += c.x; a.y += c.y; a.z += c.z; a.w += c.w;
      b.x += d.x; b.y += d.y; b.z += d.z; b.w += d.w;
    }
    const float sc = yscale ? yscale[r] : 1.0f;
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if constexpr (WEIGHTED) {
      const float wk = topk_w[r];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = fmaf(bf16r(v[j] * sc), wk, acc[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += bf16r(v[j] * sc);
    }
  }
  uint4 o;
  o.x = static_cast<uint32_t>(f32_to_bf16(acc[0])) | (static_cast<uint32_t>(f32_to_bf16(acc[1])) << 16);
  o.y = static_cast<uint32_t>(f32_to_bf16(acc[2])) | (static_cast<uint32_t>(f32_to_bf16(acc[3])) << 16);
  o.z = static_cast<uint32_t>(f32_to_bf16(acc[4])) | (static_cast<uint32_t>(f32_to_bf16(acc[5])) << 16);
  o.w = static_cast<uint32_t>(f32_to_bf16(acc[6])) | (static_cast<uint32_t>(f32_to_bf16(acc[7])) << 16);
  *reinterpret_cast<uint4*>(out + static_cast<int64_t>(t) * N + n) = o;
}

// moe_w2_combine_kernel for topk <= 8 and SPL = splits <= 4, with every
// load of a thread issued before its first add: dead slots read their own
// (in-bounds) rows and are dropped by a select, so no branch orders the
// loads.  Four columns per thread.  Same arithmetic, in the same order, as
// moe_w2_combine_kernel.
template <bool WEIGHTED, int SPL>
__global__ __launch_bounds__(256) void moe_w2_combine_fast_kernel(
    const float* __restrict__ partial, int T, int topk, int N, const int32_t* __restrict__ ids,
    const int32_t* __restrict__ emap, int64_t emap_len, int E, const float* __restrict__ yscale,
    const float* __restrict__ topk_w, uint16_t* __restrict__ out) {
  constexpr int KM = 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int cpr = N / 4;
  if (i >= static_cast<int64_t>(T) * cpr) return;
  const int t = static_cast<int>(i / cpr);
  const int n = static_cast<int>(i % cpr) * 4;
  const int64_t mn = static_cast<int64_t>(T) * topk * N;
  bool live[KM];
  float sc[KM], wk[KM];
  float4 p[KM][SPL];
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    const int kk = k < topk ? k : topk - 1;
    const int r = t * topk + kk;
    live[k] = k < topk && route_live(emap, emap_len, E, ids[r]);
    sc[k] = yscale ? yscale[r] : 1.0f;
    wk[k] = WEIGHTED ? topk_w[r] : 1.0f;
    const float* src = partial + static_cast<int64_t>(r) * N + n;
#pragma unroll
    for (int sp = 0; sp < SPL; ++sp) p[k][sp] = *reinterpret_cast<const float4*>(src + sp * mn);
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int k = 0; k < KM; ++k) {
    float4 a = p[k][0];
#pragma unroll
    for (int sp = 1; sp < SPL; ++sp) {
      a.x += p[k][sp].x; a.y += p[k][sp].y; a.z += p[k][sp].z; a.w += p[k][sp].w;
    }
    const float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float q = bf16r(v[j] * sc[k]);
      const float nx = WEIGHTED ? __builtin_fmaf(q, wk[k], acc[j]) : acc[j] + q;
      acc[j] = live[k] ? nx : acc[j];
    }
  }
  uint2 o;
  o.x = static_cast<uint32_t>(f32_to_bf16(acc[0])) | (static_cast<uint32_t>(f32_to_bf16(acc[1])) << 16);
  o.y = static_cast<uint32_t>(f32_to_bf16(acc[2])) | (static_cast<uint32_t>(f32_to_bf16(acc[3])) << 16);
  *reinterpret_cast<uint2*>(out + static_cast<int64_t>(t) * N + n) = o;
}

template <bool WEIGHTED>
static void launch_w2_combine(const float* partial, int splits, int T, int topk, int N,
                              const int32_t* ids, const int32_t* emap, int64_t emap_len, int E,
                              const float* yscale, const float* topk_w, uint16_t* out,
                              hipStream_t st) {
  if (topk <= 8 && splits >= 1 && splits <= 4 && N % 4 == 0) {
    const int64_t threads = static_cast<int64_t>(T) * (N / 4);
    const int blocks = static_cast<int>((threads + 255) / 256);
#define VMAMD_COMBINE(S)                                                                        \
  moe_w2_combine_fast_kernel<WEIGHTED, S><<<blocks, 256, 0, st>>>(partial, T, topk, N, ids, emap, \
                                                                  emap_len, E, yscale, topk_w, out)
    switch (splits) {
      case 1: VMAMD_COMBINE(1); break;
      case 2: VMAMD_COMBINE(2); break;
      case 3: VMAMD_COMBINE(3); break;
      default: VMAMD_COMBINE(4); break;
    }
#undef VMAMD_COMBINE
    return;
  }
  const int64_t chunks = static_cast<int64_t>(T) * (N / 8);
  const int blocks = static_cast<int>((chunks + 255) / 256);
  moe_w2_combine_kernel<WEIGHTED><<<blocks, 256, 0, st>>>(partial, splits, T, topk, N, ids, emap,
                                                          emap_len, E, yscale, topk_w, out);
}

// ------------------------------------------------------ prefill GEMMs -----
constexpr int kMoeBM = 128;

// Expert-major decode of a logical tile index: all blocks of (expert, tn)
// are consecutive.  The grid covers the worst case (max_tiles, a multiple of
// kXcds after xcd_grid); the tiles actually used are split into kXcds
// contiguous ranges, one per XCD (workgroup wg runs on XCD wg % kXcds), so
// every XCD gets an equal share whatever the routing.  Returns false for
// workgroups past the used tiles.  BM: routes per block (the alignment's
// block size).
template <int BM = kMoeBM>
__device__ __forceinline__ void moe_tile_decode(int L, const int32_t* __restrict__ offsets, int E, int TN,
                                                int& e_out, int& mb_out, int& tn_out) {
  // largest e with offsets[e] / BM * TN <= L (empty experts collapse onto the next)
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] / BM * TN <= L) lo = mid; else hi = mid - 1;
  }
  const int b0 = offsets[lo] / BM;
  const int nb = offsets[lo + 1] / BM - b0;
  const int local = L - b0 * TN;
  e_out = lo;
  tn_out = local / nb;
  mb_out = b0 + local % nb;
}

template <int BM = kMoeBM>
__device__ __forceinline__ bool moe_tile(int wg, int max_tiles, const int32_t* __restrict__ offsets,
                                         const int32_t* __restrict__ ntpp, const int32_t* __restrict__ eids,
                                         int E, int TN, int& e_out, int& mb_out, int& tn_out) {
  const int used = min(ntpp[0] / BM * TN, max_tiles);
  const int per = (used + kXcds - 1) / kXcds;
  const int q = wg / kXcds;
  if (q >= per) return false;
  const int L = (wg % kXcds) * per + q;
  if (L >= used) return false;
  if (eids) {
    // Tile L lies in block L / TN, whose expert the alignment recorded (its
    // block size is BM): one load, then the expert's two offsets together,
    // instead of a dependent binary search over the offsets.
    const int e = eids[L / TN];
    const int b0 = offsets[e] / BM;
    const int nb = offsets[e + 1] / BM - b0;
    const int local = L - b0 * TN;
    e_out = e;
    tn_out = local / nb;
    mb_out = b0 + local % nb;
  } else {
    moe_tile_decode<BM>(L, offsets, E, TN, e_out, mb_out, tn_out);
  }
  return true;
}

// ------------------------------------- prefill GEMMs on the DMA ring -------
// kFp8 / kBf16.  Tile: 128 routes x 256 weight rows, 8 waves as 2 (m) x 4 (n)
// with 64 x 64 per wave, 3-stage LDS ring fed by direct global->LDS loads
// (tile_pipe.h); each wave reads the next K step's fragments from LDS while
// the current step's MFMAs run.  W13: the 256 weight rows are 128 gate + 128
// up rows interleaved by 16 (epilogue: SiLU-and-mul, and for kFp8 the 1x128
// a2 quantiser); W2: 256 hidden rows (epilogue: routed weight).  Padding
// closes each expert's segment, so a wave whose first route is padding holds
// no route and skips its MFMAs (a wave-uniform test).  Padding rows load
// token 0's activations; their outputs are never used.
using MoePipeFp8 = TilePipe<true, 128, 256, 2, 4, 3>;
using MoePipeBf16 = TilePipe<false, 128, 256, 2, 4, 3>;
template <int KIND>
using MoePipe = typename std::conditional<KIND == kFp8, MoePipeFp8, MoePipeBf16>::type;

// scale_order bits of the fp8 grouped GEMMs (moe_gemm_dma_kernel,
// moe_big_kernel).  kActScalesInRoutes: the A operand's 1x128 scales are laid
// out [block, K step, BM routes] (W13: route_scales_kernel's copy of the x
// scales; W2: the a2 scales as a W13 launch with kA2ScalesInRoutes wrote
// them), so a K step's BM scales are one contiguous load.
constexpr int kActScalesInRoutes = 1, kA2ScalesInRoutes = 2;

template <int KIND, bool W13>
__global__ __launch_bounds__(512, 1) void moe_gemm_dma_kernel(
    const uint8_t* __restrict__ act, int act_bytes, const float* __restrict__ act_s, int topk, int K,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, const int32_t* __restrict__ eids, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N, int I, float limit,
    const float* __restrict__ route_w, uint8_t* __restrict__ a2, float* __restrict__ a2s,
    uint16_t* __restrict__ y, int scale_order) {
  using P = MoePipe<KIND>;
  using KB_ = KindBytes<KIND>;
  constexpr int NS = 3, BM = 128, BN = 256, WN = 4, MT = P::MT, NT = P::NT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  const int TN = W13 ? I / 128 : (N + BN - 1) / BN;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, eids, E, TN, e, mb, tn)) return;
  const int n0 = W13 ? tn * 128 : tn * BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / WN, wn = wave % WN, li = lane % 16, lg = lane / 16;
  const int KS = K / KB_::kElems;
  const int64_t rowb = static_cast<int64_t>(KS) * 128;
  const int NB = (N + 127) / 128;

  auto wrow = [&](int j) -> int {  // weight row of local tile row j
    if constexpr (W13) {
      const int p = j / 32, q = j % 32;
      return q < 16 ? n0 + 16 * p + q : I + n0 + 16 * p + (q - 16);
    } else {
      return min(n0 + j, N - 1);
    }
  };
  auto arow = [&](int r) -> int64_t {  // activation row of tile row r (-1: padding)
    const int rr = mb * BM + r;
    const int s = sorted[rr];
    if (s >= numel) return -1;
    return W13 ? static_cast<int64_t>(s / topk) : rr;
  };

  // W2 reads its activation rows through a buffer descriptor, where a padding
  // row's lanes get an offset past the end and fetch nothing (only padding
  // outputs, never stored, read those LDS bytes): its padding rows are rows
  // of their own.  W13's padding rows all read token 0's row, already in L2
  // (the buffer form measured up to 3 % slower there).
  P p;
  const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(act, act_bytes);
  uint32_t offA[P::kDmaA];
#pragma unroll
  for (int j = 0; j < P::kDmaA; ++j) {
    const int64_t ar = arow(P::rowA(wave, lane, j));
    if constexpr (W13)
      p.srcA[j] = act + max(ar, int64_t{0}) * rowb + P::chunk(lane);
    else
      offA[j] = ar >= 0 ? static_cast<uint32_t>(ar * rowb + P::chunk(lane)) : kBufferOff;
    p.ldsA[j] = (wave + j * P::kWaves) * 8 * 128;
  }
#pragma unroll
  for (int j = 0; j < P::kDmaB; ++j) {
    p.srcB[j] = w + (static_cast<int64_t>(e) * N + wrow(P::rowB(wave, lane, j))) * rowb + P::chunk(lane);
    p.ldsB[j] = P::kOffB + (wave + j * P::kWaves) * 8 * 128;
  }
  if constexpr (KIND == kFp8) {
    if (wave < BM / 64) {  // activation group scales of tile rows 64*wave + lane
      p.srcS = scale_order & kActScalesInRoutes
                   ? reinterpret_cast<const uint8_t*>(act_s + static_cast<int64_t>(mb) * KS * BM + 64 * wave + lane)
                   : reinterpret_cast<const uint8_t*>(act_s + max(arow(64 * wave + lane), int64_t{0}) * KS);
      p.ldsS = P::kOffSA + 64 * wave * 4;
    } else {  // weight-block scales: W13 gate / up block, W2 the tile's two 128-row blocks
      const int slot = min(lane, 1);
      const int brow = W13 ? (slot ? (I + n0) / 128 : n0 / 128) : min(n0 / 128 + slot, NB - 1);
      p.srcS = reinterpret_cast<const uint8_t*>(ws + (static_cast<int64_t>(e) * NB + brow) * KS);
      p.ldsS = P::kOffSB;
    }
    p.stepS = wave < BM / 64 && (scale_order & kActScalesInRoutes) ? BM * 4 : 4;
  }
  // Padding routes close a block, so a wave whose first route is padding
  // holds none.
  const bool wave_live = sorted[mb * BM + wm * P::WTM] < numel;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  struct Frags {
    v8i x[MT], w[NT];
    float sa[MT], sb0, sb1;
  };
  auto read = [&](const uint8_t* st, Frags& f) {
    if constexpr (KIND == kFp8) {
      if constexpr (W13) {
        f.sb0 = lds_load<float>(st, P::kOffSB);
        f.sb1 = lds_load<float>(st, P::kOffSB + 4);
      } else {
        f.sb0 = f.sb1 = lds_load<float>(st, P::kOffSB + (wn / 2) * 4);
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (KIND == kFp8)
        f.sa[mt] = lds_load<float>(st, P::kOffSA + (wm * P::WTM + mt * 16 + li) * 4);
      f.x[mt] = lds_frag(st, wm * P::WTM + mt * 16 + li, lg);
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) f.w[nt] = lds_frag(st + P::kOffB, wn * P::WTN + nt * 16 + li, lg);
  };
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  // MFMAs of all the wave's fragments (a partly padded wave computes its
  // padding too: a second, per-fragment form of this sequence costs register
  // spills).  kFp8: the scale promotion of MFMA i-1 (acc += p * sa * sb, 4
  // FMAs) runs while MFMA i executes -- products rotate through two
  // registers and the schedule is pinned to MFMA, 4 FMAs, MFMA, ... -- so the
  // matrix core does not wait for the promotion of its own last result.
  auto mma = [&](const Frags& f) {
    if (!wave_live) return;
    if constexpr (KIND == kFp8) {
      constexpr int NI = MT * NT;
      float sc[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        sc[mt][0] = f.sa[mt] * f.sb0;
        sc[mt][1] = W13 ? f.sa[mt] * f.sb1 : sc[mt][0];
      }
      v4f t[2];
#pragma unroll
      for (int i = 0; i <= NI; ++i) {
        if (i < NI) {
          t[i & 1] = mfma_fp8(f.w[i % NT], f.x[i / NT], zero);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        if (i > 0) {
          const int j = i - 1, mt = j / NT, nt = j % NT;
          fma4(acc[mt][nt], t[j & 1], sc[mt][nt & 1]);
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma_bf16x2(f.w[nt], f.x[mt], acc[mt][nt]);
    }
  };
  // Step kb: buffer kb % NS (whose fragments every wave read during step
  // kb - 1, as the barrier proves) is refilled with step kb + NS first, so
  // the DMA has almost two steps to land; then `nxt` is read (two LDS reads
  // after each MFMA) while `cur` runs on MFMA.  Issuing the refill ahead of
  // the MFMAs rather than after them measured 5-7 % faster on the DeepSeek-V3
  // layer at T=4096 (W13 2083 -> 1936 us, W2 1160 -> 1101 us).
  auto issue = [&](uint8_t* stage, int step) {
    const uint32_t ks = static_cast<uint32_t>(step) * 128;
#pragma unroll
    for (int j = 0; j < P::kDmaA; ++j) {
      if constexpr (W13)
        dma16(p.srcA[j] + static_cast<int64_t>(step) * 128, stage + p.ldsA[j]);
      else
        buffer_dma16(ars, offA[j] + ks, stage + p.ldsA[j]);
    }
#pragma unroll
    for (int j = 0; j < P::kDmaB; ++j) dma16(p.srcB[j] + static_cast<int64_t>(step) * 128, stage + p.ldsB[j]);
    if constexpr (KIND == kFp8) dma4(p.srcS + static_cast<int64_t>(step) * p.stepS, stage + p.ldsS);
  };
  auto step = [&](int kb, const Frags& cur, Frags& nxt) {
    wait_lgkmcnt0();
    wait_vmcnt<(NS - 2) * P::kIPS>();
    barrier_lds();
    issue(smem_dyn + (kb % NS) * P::kStage, min(kb + NS, KS - 1));
    read(smem_dyn + ((kb + 1) % NS) * P::kStage, nxt);
    mma(cur);
  };
#pragma unroll
  for (int s = 0; s < NS; ++s) issue(smem_dyn + s * P::kStage, min(s, KS - 1));
  wait_vmcnt<(NS - 1) * P::kIPS>();
  barrier_lds();
  Frags f0, f1;
  read(smem_dyn, f0);
  for (int kb = 0; kb < KS; kb += 2) {
    step(kb, f0, f1);
    if (kb + 1 < KS) step(kb + 1, f1, f0);
  }
  wait_lgkmcnt0();
  wait_vmcnt<0>();  // the ring's trailing DMAs land before LDS is reused or released
  barrier_lds();

  if constexpr (W13) {
    // route_w (apply_router_weight_on_input): gate/up times the route's weight
    // before their bf16 rounding; without it the factor is 1 (exact).
    float rw[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      rw[mt] = 1.0f;
      if (route_w) {
        const int r = sorted[static_cast<int64_t>(mb) * BM + wm * P::WTM + mt * 16 + li];
        rw[mt] = r < numel ? route_w[r] : 0.0f;
      }
    }
    if constexpr (KIND == kFp8) {
      // Activation, row amax across the 4 n-waves through LDS, 1x128 quantiser.
      float* red = reinterpret_cast<float*>(smem_dyn);  // [WN][BM]
      float v[MT][2][4];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float amax = 0.f;
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = swiglu_bf16(bf16r(acc[mt][2 * q][r] * rw[mt]),
                                        bf16r(acc[mt][2 * q + 1][r] * rw[mt]), limit);
            v[mt][q][r] = x;
            amax = fmaxf(amax, fabsf(x));
          }
        amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
        amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
        if (lg == 0) red[wn * BM + wm * P::WTM + mt * 16 + li] = amax;
      }
      __syncthreads();
      const int gpr = I / 128;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int ml = wm * P::WTM + mt * 16 + li;
        float amax = 1e-10f;
#pragma unroll
        for (int w4 = 0; w4 < WN; ++w4) amax = fmaxf(amax, red[w4 * BM + ml]);
        const float scale = amax / 448.0f, rs = 1.0f / scale;
        const int64_t row = static_cast<int64_t>(mb) * BM + ml;
        if (wn == 0 && lg == 0) {
          if (scale_order & kA2ScalesInRoutes)  // [block, I / 128, BM routes], as the W2 tiles read them
            a2s[(static_cast<int64_t>(mb) * gpr + tn) * BM + ml] = scale;
          else
            a2s[row * gpr + tn] = scale;
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
          *reinterpret_cast<uint32_t*>(a2 + row * I + col) = quant4_e4m3(v[mt][q], scale, rs);
        }
      }
    } else {
      uint16_t* a2b = reinterpret_cast<uint16_t*>(a2);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int64_t row = static_cast<int64_t>(mb) * BM + wm * P::WTM + mt * 16 + li;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            o[r] = swiglu_bf16(bf16r(acc[mt][2 * q][r] * rw[mt]), bf16r(acc[mt][2 * q + 1][r] * rw[mt]),
                               limit);
          const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
          *reinterpret_cast<uint2*>(a2b + row * I + col) = pack_bf16x4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = sorted[static_cast<int64_t>(mb) * BM + wm * P::WTM + mt * 16 + li];
      if (r >= numel) continue;
      const float rw = route_w ? route_w[r] : 1.0f;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int n = n0 + wn * P::WTN + nt * 16 + 4 * lg;
        if (n >= N) continue;
        const v4f a = acc[mt][nt];
        *reinterpret_cast<uint2*>(y + static_cast<int64_t>(r) * N + n) =
            pack_bf16x4(a[0] * rw, a[1] * rw, a[2] * rw, a[3] * rw);
      }
    }
  }
}

// The fp8 layer's x scales in route order for the grouped W13 GEMMs: out
// [(b * KS + k) * bm + j] = scale k of the token of route sorted[b * bm + j]
// (padding rows: token 0), over the used blocks (ntpp).  The W13 tiles then
// read one K step's scales of their BM routes from BM * 4 bytes in a row instead
// of one gathered token row per lane (DeepSeek-V3 T=4096: 256 lines a step).
// One thread per route row: its token's KS scales in 16-byte loads (KS % 4
// == 0, the host's condition), each K step's store coalesced across the
// wave's consecutive rows.
__global__ __launch_bounds__(256) void route_scales_kernel(const float* __restrict__ xs,
                                                           const int32_t* __restrict__ sorted,
                                                           const int32_t* __restrict__ ntpp, int numel, int topk,
                                                           int KS, int bm, float* __restrict__ out) {
  const int rows = ntpp[0];
  for (int r = blockIdx.x * blockDim.x + threadIdx.x; r < rows; r += gridDim.x * blockDim.x) {
    const int b = r / bm, j = r - b * bm;
    const int sr = sorted[r];
    const int t = sr < numel ? sr / topk : 0;
    const float4* src = reinterpret_cast<const float4*>(xs + static_cast<int64_t>(t) * KS);
    float* dst = out + static_cast<int64_t>(b) * KS * bm + j;
    for (int k4 = 0; k4 < KS / 4; ++k4) {
      const float4 v = src[k4];
      dst[(4 * k4 + 0) * bm] = v.x;
      dst[(4 * k4 + 1) * bm] = v.y;
      dst[(4 * k4 + 2) * bm] = v.z;
      dst[(4 * k4 + 3) * bm] = v.w;
    }
  }
}

// ------------------------------- fp8 prefill GEMMs on 256-route tiles ----
// For long prefills (block size 256): a CU's loads stream at the rate its
// vector cache keeps requests in flight, so the bytes a workgroup moves per
// flop set the pace, and a 256-route x 256-row tile moves 64 KiB per K step
// for twice the flops of the 128-route tile's 48 KiB.  A wave of 64 padding
// routes skips its MFMAs, so the larger block costs little where an
// expert's last block is mostly padding: an 8-row group of padding
// routes loads nothing (its LDS rows keep stale bytes, which reach only the
// padding routes' outputs, never stored).  8 waves as 4 (m: 64
// routes) x 2 (n: 128 weight rows), two LDS stages, all loads through buffer
// descriptors (activations, scales; the weights per expert), MFMA order and
// promotion as gemm_fp8_big_kernel.  W13: the 256 weight rows are 128 gate +
// 128 up rows interleaved by 16 (n tile 2q gate, 2q + 1 up); epilogue
// SiLU-and-mul and the 1x128 a2 quantiser; W2: 256 hidden rows, epilogue the
// routed weight.
//
// bf16 also runs the tile with 320 routes (MTV = 5: 80 routes per m-wave),
// for the route counts that would leave a 256-route block nearly empty:
// around 256 or 512 routes per expert an expert's last 256-route block
// holds a few dozen routes yet streams the expert's whole weight tile.  fp8
// keeps 256 routes (the promotion's registers leave no room for a fifth
// m-tile: 256 VGPRs, and W13 at T=4096 measured 12 % slower).
//
// A block whose live routes fit in kRows3 = 160 rows (an expert's only
// block at up to 160 routes, or its last one) runs a three-stage ring
// instead (fp8): its activation slot holds 160 rows, so three stages fit in
// the LDS and two K steps are in flight while one is computed.  Such a tile
// is bound by the latency of its weight stream, not by its few MFMAs.
template <int MTV, int NS>
struct MoeBigRing {
  static constexpr int kNS = NS;
  static constexpr int kRowsA = NS == 2 ? 64 * MTV : 160;  // activation slot rows
  static constexpr int kOffB = kRowsA * 128;
  static constexpr int kOffSA = kOffB + 256 * 128;
  static constexpr int kOffSB = kOffSA + 64 * MTV * 4;  // waves 0 .. BM/64 - 1 write 64 A scales each
  static constexpr int kStage = kOffSB + 256;           // the B-scale DMA writes 64 lanes x 4 bytes
};
template <int MTV>
struct MoeBigTile {
  static constexpr int BM = 64 * MTV, BN = 256, WN = 2, MT = MTV, NT = 8, WTM = 16 * MTV, kThreads = 512;
  using R2 = MoeBigRing<MTV, 2>;
  using R3 = MoeBigRing<MTV, 3>;
  static constexpr bool kRing3 = MTV == 4;  // (fp8 only, chosen in the kernel)
  static constexpr int kRows3 = R3::kRowsA;
  // The ring's stages, or the W2 output tile staged for its stores if that is larger.
  static constexpr int kRingLds = kRing3 && 3 * R3::kStage > 2 * R2::kStage ? 3 * R3::kStage : 2 * R2::kStage;
  static constexpr int kLds = kRingLds > BM * 512 ? kRingLds : BM * 512;
  static_assert(kLds <= 160 * 1024, "LDS stages exceed the CU's LDS");
};
constexpr int kMoeBigBM = 256, kMoeBig320 = 320;

template <int KIND, bool W13, int MTV = 4>
__global__ __launch_bounds__(512, 1) void moe_big_kernel(
    const uint8_t* __restrict__ act, int act_bytes, const float* __restrict__ act_s, int act_s_bytes,
    int topk, int K, const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, const int32_t* __restrict__ eids, int E, int numel, int max_tiles, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int I, float limit, const float* __restrict__ route_w,
    uint8_t* __restrict__ a2, float* __restrict__ a2s, uint16_t* __restrict__ y, int scale_order = 0) {
  using P = MoeBigTile<MTV>;
  constexpr int BM = P::BM, NT = P::NT, MT = P::MT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  const int TN = W13 ? I / 128 : (N + P::BN - 1) / P::BN;
  int e, mb, tn;
  if (!moe_tile<BM>(blockIdx.x, max_tiles, offsets, ntpp, eids, E, TN, e, mb, tn)) return;
  const int n0 = W13 ? tn * 128 : tn * P::BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / P::WN, wn = wave % P::WN;
  const int li = lane % 16, lg = lane / 16;
  constexpr bool kScaled = KIND == kFp8;
  const int KS = K / KindBytes<KIND>::kElems, NB = (N + 127) / 128;
  const int rowb = KS * 128;  // bytes per activation / weight row
  const int64_t base = static_cast<int64_t>(mb) * BM;

  auto wrow = [&](int j) -> int {  // weight row of local tile row j
    if constexpr (W13) {
      const int p = j / 32, q = j % 32;
      return q < 16 ? n0 + 16 * p + q : I + n0 + 16 * p + (q - 16);
    } else {
      return n0 + j;  // rows past N: past the descriptor's range
    }
  };
  auto arow = [&](int r) -> int {  // activation row of tile row r
    if constexpr (W13) {
      const int s = sorted[base + r];
      return s < numel ? s / topk : 0;
    } else {
      return static_cast<int>(base) + r;
    }
  };

  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(act, act_bytes);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(w + static_cast<int64_t>(e) * N * rowb, N * rowb);
  const uint32_t chunk = static_cast<uint32_t>(((lane % 8) ^ (lane / 8)) * 16);
  uint32_t offA[MT], offB[4];
  uint64_t liveA[MT];  // activation row groups holding a route (padding groups load nothing)
#pragma unroll
  for (int j = 0; j < MT; ++j) {
    const int r = (wave + 8 * j) * 8 + lane / 8;
    offA[j] = static_cast<uint32_t>(arow(r)) * rowb + chunk;
    liveA[j] = __builtin_amdgcn_ballot_w64(sorted[base + r] < numel);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) offB[j] = static_cast<uint32_t>(wrow((wave + 8 * j) * 8 + lane / 8)) * rowb + chunk;
  uint32_t offS = 0, stepS = 4;
  const bool sa_wave = wave < BM / 64;
  __amdgpu_buffer_rsrc_t rs = buffer_rsrc(act_s, 0);
  if (!kScaled) {
  } else if (sa_wave) {  // activation scales of tile rows 64 * wave + lane
    rs = buffer_rsrc(act_s, act_s_bytes);
    if (scale_order & kActScalesInRoutes) {  // [block, K step, BM routes]: one step's scales side by side
      offS = static_cast<uint32_t>((static_cast<int64_t>(mb) * KS * BM + 64 * wave + lane) * 4);
      stepS = BM * 4;
    } else {
      offS = static_cast<uint32_t>(arow(64 * wave + lane)) * KS * 4;
    }
  } else {  // weight-block scales: W13 gate / up block, W2 the tile's two 128-row blocks
    const int slot = min(lane, 1);
    const int brow = W13 ? (slot ? (I + n0) / 128 : n0 / 128) : min(n0 / 128 + slot, NB - 1);
    rs = buffer_rsrc(ws, E * NB * KS * 4);
    offS = static_cast<uint32_t>((e * NB + brow) * KS) * 4;
  }
  // One stage of the ring R (the activation row groups that hold a route,
  // the weight rows, the scales).
  auto issue = [&](uint8_t* stage, int step, auto ring) {
    using R = decltype(ring);
    const uint32_t ks = static_cast<uint32_t>(step) * 128;
#pragma unroll
    for (int j = 0; j < MT; ++j)
      if (liveA[j]) buffer_dma16(ra, offA[j] + ks, stage + (wave + 8 * j) * 8 * 128);
#pragma unroll
    for (int j = 0; j < 4; ++j) buffer_dma16(rb, offB[j] + ks, stage + R::kOffB + (wave + 8 * j) * 8 * 128);
    if (kScaled && wave <= BM / 64)
      buffer_dma4(rs, offS + step * stepS, stage + (sa_wave ? R::kOffSA + 64 * wave * 4 : R::kOffSB));
  };
  // This wave's loads per stage, for the three-stage ring's vmcnt.
  int dmas = 4 + (kScaled && wave <= BM / 64 ? 1 : 0);
#pragma unroll
  for (int j = 0; j < MT; ++j) dmas += liveA[j] ? 1 : 0;
  dmas = __builtin_amdgcn_readfirstlane(dmas);
  // Padding routes close a block, so the wave's 16-route m-tiles that hold a
  // route are a prefix: mlive of them (0: the wave holds none and skips its
  // MFMAs).  The MFMAs of the m-tiles past it are skipped too (their
  // accumulators stay zero; they hold only padding routes, whose outputs
  // nothing reads).
  int mlive = 0;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) mlive += sorted[base + wm * P::WTM + mt * 16] < numel ? 1 : 0;
  mlive = __builtin_amdgcn_readfirstlane(mlive);

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  const int nw = wn * 16 * NT;  // the wave's first local weight row

  // One K step from LDS stage `st` (see gemm_fp8_big_kernel) over the first
  // ML m-tiles.  W13: n tile nt takes the gate (even) or up (odd) block
  // scale.  bf16: two chained MFMAs per fragment pair into the accumulators,
  // no scales.
  auto mma = [&](const uint8_t* st, auto ml_tag, auto ring) {
    constexpr int ML = decltype(ml_tag)::value;
    using R = decltype(ring);
    float sb0 = 0.f, sb1 = 0.f, sa[MT], sc[MT][2];
    if constexpr (kScaled) {
      sb0 = lds_load<float>(st, R::kOffSB + (W13 ? 0 : 4 * wn));
      sb1 = W13 ? lds_load<float>(st, R::kOffSB + 4) : sb0;
#pragma unroll
      for (int mt = 0; mt < ML; ++mt) sa[mt] = lds_load<float>(st, R::kOffSA + (wm * P::WTM + mt * 16 + li) * 4);
    }
    v8i wf[2], x[MT];
    wf[0] = lds_frag(st + R::kOffB, nw + li, lg);
#pragma unroll
    for (int mt = 0; mt < ML; ++mt) x[mt] = lds_frag(st, wm * P::WTM + mt * 16 + li, lg);
    __builtin_amdgcn_sched_barrier(0);
    v4f t[2];
    constexpr int NI = ML * NT;
#pragma unroll
    for (int i = 0; i <= NI; ++i) {
      const int nt = i / ML, mt = i % ML;
      if (i < NI) {
        if constexpr (kScaled)
          t[i & 1] = mfma_fp8(wf[nt & 1], x[mt], zero);
        else
          acc[mt][nt] = mfma_bf16x2(wf[nt & 1], x[mt], acc[mt][nt]);
        __builtin_amdgcn_sched_barrier(0);
        if (mt == 0 && nt + 1 < NT) wf[(nt + 1) & 1] = lds_frag(st + R::kOffB, nw + (nt + 1) * 16 + li, lg);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (kScaled && i > 0) {
        const int j = i - 1, jm = j % ML, jn = j / ML;
        if (jn < 2) sc[jm][jn] = sa[jm] * (jn ? sb1 : sb0);  // at first use
        fma4(acc[jm][jn], t[j & 1], sc[jm][W13 ? (jn & 1) : 0]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // The K loop, one copy per live m-tile count (ML = 0: DMAs and barriers
  // only) and ring.  Two stages: one K step in flight while the other is
  // computed.  Three: two in flight; before step kb a wave waits until only
  // its loads of step kb + 1 are outstanding (dmas per stage; past the last
  // issued stage, none).
  auto kloop = [&](auto ml_tag, auto ring) {
    constexpr int ML = decltype(ml_tag)::value;
    using R = decltype(ring);
    constexpr int NS = R::kNS;
    issue(smem_dyn, 0, ring);
    if constexpr (NS == 3) {
      if (KS > 1) issue(smem_dyn + R::kStage, 1, ring);
    }
    wait_lgkmcnt0();
    int cur = 0;  // stage of step kb
    for (int kb = 0; kb < KS; ++kb) {
      if constexpr (NS == 2) {
        wait_vmcnt<0>();  // this wave's DMAs of step kb have landed
      } else if (kb + 1 < KS) {
        switch (dmas) {  // wave-uniform
          case 4: wait_vmcnt<4>(); break;
          case 5: wait_vmcnt<5>(); break;
          case 6: wait_vmcnt<6>(); break;
          case 7: wait_vmcnt<7>(); break;
          case 8: wait_vmcnt<8>(); break;
          case 9: wait_vmcnt<9>(); break;
          default: wait_vmcnt<0>(); break;
        }
      } else {
        wait_vmcnt<0>();
      }
      barrier_lds();  // ... every wave's, and step kb - 1's buffer is no longer read
      const int nxt = cur + NS - 1 >= NS ? cur - 1 : cur + NS - 1;  // stage of step kb + NS - 1
      if (kb + NS - 1 < KS) issue(smem_dyn + nxt * R::kStage, kb + NS - 1, ring);
      if constexpr (ML > 0) mma(smem_dyn + cur * R::kStage, ml_tag, ring);
      cur = cur + 1 == NS ? 0 : cur + 1;
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using I4 = std::integral_constant<int, 4>;
  using I5 = std::integral_constant<int, 5>;
  static_assert(MT == 4 || MT == 5, "m-tiles per wave");
  auto run = [&](auto ring) {
    if (MT == 5 && mlive >= 5) {
      if constexpr (MT == 5) kloop(I5{}, ring);
    } else if (mlive >= 4) {
      kloop(I4{}, ring);
    } else if (mlive == 3) {
      kloop(I3{}, ring);
    } else if (mlive == 2) {
      kloop(I2{}, ring);
    } else if (mlive == 1) {
      kloop(I1{}, ring);
    } else {
      kloop(I0{}, ring);
    }
  };
  // Padding closes the block, so its live routes fit the three-stage ring's
  // activation slot when row kRows3 is padding (workgroup-uniform).
  bool ring3 = false;
  if constexpr (kScaled && P::kRing3) ring3 = __builtin_amdgcn_readfirstlane(sorted[base + P::kRows3] >= numel ? 1 : 0) != 0;
  if (ring3) {
    if constexpr (kScaled && P::kRing3) run(typename P::R3{});
  } else {
    run(typename P::R2{});
  }
  barrier_lds();  // every wave is done with the stages before LDS is reused

  if constexpr (W13) {
    // route_w (apply_router_weight_on_input): gate/up times the route's weight
    // before their bf16 rounding; without it the factor is 1 (exact).
    float rw[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      rw[mt] = 1.0f;
      if (route_w) {
        const int r = sorted[base + wm * P::WTM + mt * 16 + li];
        rw[mt] = r < numel ? route_w[r] : 0.0f;
      }
    }
    if constexpr (!kScaled) {  // bf16 activation
      uint16_t* a2b = reinterpret_cast<uint16_t*>(a2);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int64_t row = base + wm * P::WTM + mt * 16 + li;
#pragma unroll
        for (int q = 0; q < NT / 2; ++q) {
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r)
            o[r] = swiglu_bf16(bf16r(acc[mt][2 * q][r] * rw[mt]), bf16r(acc[mt][2 * q + 1][r] * rw[mt]), limit);
          const int col = n0 + (4 * wn + q) * 16 + 4 * lg;
          *reinterpret_cast<uint2*>(a2b + row * I + col) = pack_bf16x4(o[0], o[1], o[2], o[3]);
        }
      }
      return;
    }
    // SiLU-and-mul, row amax across the 2 n-waves through LDS, 1x128 quantiser.
    float* red = reinterpret_cast<float*>(smem_dyn);  // [WN][BM]
    float v[MT][NT / 2][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float amax = 0.f;
#pragma unroll
      for (int q = 0; q < NT / 2; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float xv = swiglu_bf16(bf16r(acc[mt][2 * q][r] * rw[mt]), bf16r(acc[mt][2 * q + 1][r] * rw[mt]), limit);
          v[mt][q][r] = xv;
          amax = fmaxf(amax, fabsf(xv));
        }
      amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
      amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
      if (lg == 0) red[wn * BM + wm * P::WTM + mt * 16 + li] = amax;
    }
    __syncthreads();
    const int gpr = I / 128;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int ml = wm * P::WTM + mt * 16 + li;
      const float amax = fmaxf(1e-10f, fmaxf(red[ml], red[BM + ml]));
      const float scale = amax / 448.0f, rs = 1.0f / scale;
      const int64_t row = base + ml;
      if (wn == 0 && lg == 0) {
        if (scale_order & kA2ScalesInRoutes)  // [block, I / 128, BM routes], as the W2 tiles read them
          a2s[(static_cast<int64_t>(mb) * gpr + tn) * BM + ml] = scale;
        else
          a2s[row * gpr + tn] = scale;
      }
#pragma unroll
      for (int q = 0; q < NT / 2; ++q) {
        const int col = n0 + (4 * wn + q) * 16 + 4 * lg;
        *reinterpret_cast<uint32_t*>(a2 + row * I + col) = quant4_e4m3(v[mt][q], scale, rs);
      }
    }
  } else {
    // y = bf16(acc * w) staged through LDS so that each store writes 16 bytes
    // per lane and whole 512-byte tile rows (the 8-byte fragment stores
    // scatter 32-byte pieces over 16 rows per instruction).  Row r of the
    // tile takes 512 bytes, its 16-byte chunk c at slot c ^ (r & 31).
    uint8_t* yt = smem_dyn;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = wm * P::WTM + mt * 16 + li;
      const int r = sorted[base + row];
      const float rw = r < numel && route_w ? route_w[r] : 1.0f;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int col = nw + nt * 16 + 4 * lg;
        const v4f a = acc[mt][nt];
        const int off = row * 512 + (((col >> 3) ^ (row & 31)) << 4) + ((col >> 2) & 1) * 8;
        *reinterpret_cast<uint2*>(yt + off) = pack_bf16x4(a[0] * rw, a[1] * rw, a[2] * rw, a[3] * rw);
      }
    }
    __syncthreads();
    const int c = lane % 32;
    const int n = n0 + c * 8;
#pragma unroll 4
    for (int it = 0; it < BM / 16; ++it) {
      const int row = it * 16 + wave * 2 + lane / 32;
      const int r = sorted[base + row];
      if (r >= numel || n >= N) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(yt + row * 512 + ((c ^ (row & 31)) << 4));
      *reinterpret_cast<uint4*>(y + static_cast<int64_t>(r) * N + n) = v;
    }
  }
}

// ------------------------------------------- w4afp8 prefill GEMMs ---------
// Tile: 128 routes x 256 weight rows, 8 waves as 2 (m) x 4 (n) with 64 x 64
// per wave, on a W4Pipe::NS-deep LDS ring fed by direct global->LDS loads
// (the discipline of tile_pipe.h).  A stage holds one K step (128 elements):
//   [activations 128 x 128 B, w4 order, row r chunk c at w4_act_off(r, c)]
//   [packed weights 256 x 64 B, row r chunk c at w4_lds_off(r, c)]
//   [activation corrections 128 x 16 B, each row's value four times, which is
//    an MFMA accumulator input as read]
//   [weight-scale words 256 x 4 B: the aligned 4 bytes holding row r's bf16
//    scale of the step, next to that of the step before or after it]
//   [256 x 4 B that waves 4-7 fill with one shared word (with transposed
//    scales: a copy of the scale words), so every wave issues the same number
//    of loads per stage (the waits count per wave); nothing reads it]
// The weights cross LDS packed; each wave expands its fragments after the LDS
// read (w4_frag), with the offset correction as the MFMA accumulator input
// and the bf16 weight scale applied per step (acc += p * s, 4 FMAs per MFMA).
// W13: the 256 weight rows are 128 gate + 128 up rows interleaved by 16, the
// epilogue writes the bf16 SwiGLU activation of every padded route row;
// W2: 256 hidden rows, epilogue y[r] = bf16(acc * a2 row scale).
// EVEN: K / 128 is even (a row's scale words never straddle two rows).

struct W4Pipe {
  static constexpr int BM = 128, BN = 256, NS = 4, MT = 4, NT = 4;
  static_assert(NS >= 2, "the ring keeps NS - 1 steps in flight");
  static constexpr int kOffB = BM * 128;
  static constexpr int kOffC = kOffB + BN * 64;
  static constexpr int kOffS = kOffC + BM * 16;
  static constexpr int kOffD = kOffS + BN * 4;
  static constexpr int kStage = kOffD + BN * 4;
  static constexpr int kLds = NS * kStage;
  static constexpr int kIPS = 6;  // loads per stage per wave: 2 activation, 2 weight, 1 correction, 1 scale
};
static_assert(W4Pipe::kLds <= 160 * 1024, "LDS ring exceeds the CU's LDS");

// LDS slots of the W4 tiles.  A lane group reads one 16-byte chunk of 16
// consecutive rows; any 8 consecutive rows of them land in 8 distinct
// 16-byte bank groups of a 128-byte line (the packed weights also in 16
// distinct groups of a 256-byte line: measured 22.7M -> 6.5M bank-conflict
// cycles per W13 launch; the same extension for the 128-byte activation
// rows measured 3.6 % slower).
// Activation chunk c (of 8) of row r: slot c ^ (r & 7), as lds_off.
__device__ __forceinline__ int w4_act_swz(int r) { return r & 7; }
__device__ __forceinline__ int w4_act_off(int r, int c) { return r * 128 + ((c ^ w4_act_swz(r)) << 4); }
// Packed weight chunk c (of 4) of row r: slot c ^ f(r), f a bijection of row
// bits 1-2 (8-row lines) and of bits 2-3 (16-row lines).
__device__ __forceinline__ int w4_wt_swz(int r) { return (((r >> 1) ^ (r >> 3)) & 1) | (((r >> 2) & 1) << 1); }
__device__ __forceinline__ int w4_lds_off(int r, int c) { return r * 64 + ((c ^ w4_wt_swz(r)) << 4); }

// act: W13 the quantised x [T, K] (rows = tokens), W2 a2 [rows, K] in padded
// route order, act_bytes its size (< 2^31); act_scale: W13 the token row
// scales, W2 the a2 row scales; act_corr: [rows, K/128] offset corrections;
// ws: bf16 [E, N, K/128]; SCT (K / 128 even): the same scales as 32-bit
// words of two K steps, transposed to [E, K/256, N] (W4ScalesT, in the
// alignment's launch), so that one stage's 256 rows read consecutive words
// instead of one 128-byte line per row (at K = 4096 the rows lie 64 bytes
// apart).
// out: W13 bf16 activation [padded rows, I]; W2 y [numel, N].
template <bool W13, bool EVEN, bool SCT = false>
__global__ __launch_bounds__(512, 1) void moe_w4_gemm_kernel(
    const uint8_t* __restrict__ act, const float* __restrict__ act_scale,
    const float* __restrict__ act_corr, int act_bytes, int topk, int K,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, const int32_t* __restrict__ eids, int E, int numel, int max_tiles, const uint8_t* __restrict__ w,
    const uint16_t* __restrict__ ws, int N, int I, float limit, uint16_t* __restrict__ out) {
  using P = W4Pipe;
  constexpr int BM = P::BM, BN = P::BN, NS = P::NS, MT = P::MT, NT = P::NT, WN = 4, WTM = 64, WTN = 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  const int TN = W13 ? I / 128 : (N + BN - 1) / BN;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, eids, E, TN, e, mb, tn)) return;
  const int n0 = W13 ? tn * 128 : tn * BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / WN, wn = wave % WN, li = lane % 16, lg = lane / 16;
  const int KS = K / 128;

  auto wrow = [&](int j) -> int {  // weight row of local tile row j
    if constexpr (W13) {
      const int p = j / 32, q = j % 32;
      return q < 16 ? n0 + 16 * p + q : I + n0 + 16 * p + (q - 16);
    } else {
      return min(n0 + j, N - 1);
    }
  };
  auto arow = [&](int r) -> int64_t {  // activation row of tile row r (-1: padding)
    const int rr = mb * BM + r;
    const int s = sorted[rr];
    if (s >= numel) return -1;
    return W13 ? static_cast<int64_t>(s / topk) : rr;
  };

  // Per-lane load sources at K step 0 and wave-uniform LDS offsets in a
  // stage.  Activation rows and corrections are read through buffer
  // descriptors: a padding row's lanes get an offset past the end and fetch
  // nothing (their LDS bytes are left undefined; only padding outputs, which
  // are never stored or used, depend on them).
  const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(act, act_bytes);
  const __amdgpu_buffer_rsrc_t crs = buffer_rsrc(act_corr, act_bytes / 32);
  uint32_t offA[2];
  const uint8_t* srcB[2];
  int ldsA[2], ldsB[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int ga = wave + 8 * j;  // 8-row activation group
    const int64_t ra = arow(ga * 8 + lane / 8);
    const int slot_a = lane % 8;  // lane writes slot lane % 8 of row 8 * ga + lane / 8
    offA[j] = ra >= 0 ? static_cast<uint32_t>(ra * KS * 128 + ((slot_a ^ w4_act_swz(ga * 8 + lane / 8)) << 4))
                      : kBufferOff;
    ldsA[j] = ga * 1024;
    const int rb = ga * 16 + lane / 4;  // 16-row weight group ga
    srcB[j] = w + (static_cast<int64_t>(e) * N + wrow(rb)) * KS * 64 + (((lane % 4) ^ w4_wt_swz(rb)) << 4);
    ldsB[j] = P::kOffB + ga * 1024;
  }
  const int64_t rc = arow(wave * 16 + lane / 4);
  const uint32_t offC = rc >= 0 ? static_cast<uint32_t>(rc * KS * 4) : kBufferOff;
  const int ldsC = P::kOffC + wave * 256;
  static_assert(!SCT || EVEN, "transposed scale words pair two K steps");
  const int64_t rowKS = (static_cast<int64_t>(e) * N + wrow((wave % 4) * 64 + lane)) * KS;
  const uint8_t* wsb = reinterpret_cast<const uint8_t*>(ws);
  // SCT: word (K step pair 0) of the lane's row; pair p is p * N words on.
  const uint8_t* wst = wsb + (static_cast<int64_t>(e) * (KS / 2) * N + wrow((wave % 4) * 64 + lane)) * 4;
  const int ldsS = (wave < 4 ? P::kOffS : P::kOffD) + (wave % 4) * 256;
  auto issue = [&](uint8_t* st, int step) {
#pragma unroll
    for (int j = 0; j < 2; ++j) buffer_dma16(ars, offA[j] + static_cast<uint32_t>(step) * 128, st + ldsA[j]);
#pragma unroll
    for (int j = 0; j < 2; ++j) dma16(srcB[j] + static_cast<int64_t>(step) * 64, st + ldsB[j]);
    buffer_dma4(crs, offC + static_cast<uint32_t>(step) * 4, st + ldsC);
    if constexpr (SCT)
      dma4(wst + static_cast<int64_t>(step / 2) * N * 4, st + ldsS);
    else  // waves 4-7 keep the load count only: one shared word (a copy of the 256
          // scattered words cost 5 % at T=512)
      dma4(wave < 4 ? wsb + ((rowKS + step) & ~static_cast<int64_t>(1)) * 2 : wsb, st + ldsS);
  };
  // Padding routes close a block, so a wave whose first route is padding
  // holds none.
  const bool wave_live = sorted[mb * BM + wm * WTM] < numel;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  // Operand fragments (double-buffered across steps) and the step's
  // corrections and scale words (read in the step that uses them).
  struct Frags {
    v8i x[MT];
    v4i w[NT];
  };
  struct Small {
    v4f c[MT];
    v4i s[NT];
  };
  auto read = [&](const uint8_t* st, Frags& f) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = wm * WTM + mt * 16 + li;
      const v4i lo = lds_load<v4i>(st, w4_act_off(r, 2 * lg));
      const v4i hi = lds_load<v4i>(st, w4_act_off(r, 2 * lg + 1));
      f.x[mt] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) f.w[nt] = lds_load<v4i>(st, P::kOffB + w4_lds_off(wn * WTN + nt * 16 + li, lg));
  };
  // with_s: also the scale words (EVEN: an odd step reuses its even
  // predecessor's words, which hold both steps' scales).
  auto read_small = [&](const uint8_t* st, Small& q, bool with_s) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) q.c[mt] = lds_load<v4f>(st, P::kOffC + (wm * WTM + mt * 16 + li) * 16);
    if (with_s) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) q.s[nt] = lds_load<v4i>(st, P::kOffS + (wn * WTN + nt * 16 + 4 * lg) * 4);
    }
  };
  // MFMAs n-tile by n-tile: the expansion of a weight fragment serves its
  // four MFMAs.  The sequence is software-pipelined in blocks separated by
  // scheduling barriers, so the compiler cannot regroup it: block i issues
  // MFMA i, then the promotion of MFMA i - 1 (acc += p * s, whose result is
  // ready by then) and a quarter of the next fragment's expansion and scale
  // words -- about as many VALU cycles as the MFMA takes, and no VALU
  // instruction waits on the MFMA in flight.  PAR: parity of the K step,
  // which picks each scale word's half.
  auto mma = [&](const Frags& f, const Small& q, auto par_tag) {
    constexpr int PAR = decltype(par_tag)::value;
    if (!wave_live) return;
    auto scale = [&](int nt, int r) {
      const uint32_t wd = static_cast<uint32_t>(q.s[nt][r]);
      const bool hi = EVEN ? PAR != 0 : ((r ^ PAR) & 1) != 0;
      return __uint_as_float(hi ? (wd & 0xFFFF0000u) : (wd << 16));
    };
    auto expand_word = [&](int nt, int j, v8i& dst) {
      const uint32_t wd = static_cast<uint32_t>(f.w[nt][j]);
      dst[2 * j] = static_cast<int>(__builtin_amdgcn_bitop3_b32(wd, 0x88888888u, 0x0F0F0F0Fu, 0x28));
      dst[2 * j + 1] = static_cast<int>(__builtin_amdgcn_bitop3_b32(wd >> 4, 0x88888888u, 0x0F0F0F0Fu, 0x28));
    };
    constexpr int NI = MT * NT;
    v8i wx[2];
    v4f sc[2];
    v4f t[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      expand_word(0, j, wx[0]);
      sc[0][j] = scale(0, j);
    }
#pragma unroll
    for (int i = 0; i <= NI; ++i) {
      const int nt = i / MT, mt = i % MT;
      if (i < NI) t[i & 1] = mfma_fp8(wx[nt & 1], f.x[mt], q.c[mt]);
      __builtin_amdgcn_sched_barrier(0);
      if (i > 0) {
        const int jp = i - 1;
        fma4v(acc[jp % MT][jp / MT], t[jp & 1], sc[(jp / MT) & 1]);
      }
      if (i < NI && nt + 1 < NT) {
        expand_word(nt + 1, mt, wx[(nt + 1) & 1]);
        sc[(nt + 1) & 1][mt] = scale(nt + 1, mt);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using Even = std::integral_constant<int, 0>;
  using Odd = std::integral_constant<int, 1>;
  // Step kb: buffer kb % NS -- step kb, whose fragments and small values
  // every wave read during step kb - 1, as the barrier proves -- is refilled
  // with step kb + NS (NS - 1 steps in flight); step kb + 1's fragments are
  // read while step kb's MFMAs run, and its small values after them.
  auto step = [&](int kb, const Frags& cur, Frags& nxt, Small& q, auto par_tag) {
    wait_lgkmcnt0();
    wait_vmcnt<(NS - 2) * P::kIPS>();
    barrier_lds();
    issue(smem_dyn + (kb % NS) * P::kStage, min(kb + NS, KS - 1));
    read(smem_dyn + ((kb + 1) % NS) * P::kStage, nxt);
    mma(cur, q, par_tag);
    read_small(smem_dyn + ((kb + 1) % NS) * P::kStage, q, !EVEN || decltype(par_tag)::value == 1);
  };
#pragma unroll
  for (int st = 0; st < NS; ++st) issue(smem_dyn + st * P::kStage, min(st, KS - 1));
  wait_vmcnt<(NS - 1) * P::kIPS>();
  barrier_lds();
  Frags f0, f1;
  Small q;
  read(smem_dyn, f0);
  read_small(smem_dyn, q, true);
  for (int kb = 0; kb < KS; kb += 2) {
    step(kb, f0, f1, q, Even{});
    if (kb + 1 < KS) step(kb + 1, f1, f0, q, Odd{});
  }
  wait_lgkmcnt0();
  wait_vmcnt<0>();  // the ring's trailing loads land before LDS is released
  barrier_lds();

  if constexpr (W13) {
    uint16_t* a = out;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int64_t row = static_cast<int64_t>(mb) * BM + wm * WTM + mt * 16 + li;
      const int r = sorted[row];
      const float srow = r < numel ? act_scale[r / topk] * kW4Unit : 0.f;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = swiglu_w4(bf16r(acc[mt][2 * q][j] * srow), bf16r(acc[mt][2 * q + 1][j] * srow), limit);
        const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
        *reinterpret_cast<uint2*>(a + row * I + col) = pack_bf16x4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int64_t row = static_cast<int64_t>(mb) * BM + wm * WTM + mt * 16 + li;
      const int r = sorted[row];
      if (r >= numel) continue;
      const float rs = act_scale[row] * kW4Unit;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int n = n0 + wn * WTN + nt * 16 + 4 * lg;
        if (n >= N) continue;
        const v4f v = acc[mt][nt];
        *reinterpret_cast<uint2*>(out + static_cast<int64_t>(r) * N + n) =
            pack_bf16x4(v[0] * rs, v[1] * rs, v[2] * rs, v[3] * rs);
      }
    }
  }
}

// ------------------------------------------------------------ host side ---
// Split-K factor of the decode GEMVs: enough waves to cover the chip
// (kGemvTargetWaves over the active experts' n-tiles), at least 4 K steps
// per split.
static int moe_splits(int64_t waves_per_split, int KS) {
  int s = static_cast<int>((kGemvTargetWaves + waves_per_split - 1) / waves_per_split);
  return max(1, min(s, max(1, KS / 4)));
}

static int64_t moe_umax(int64_t numel, int E) { return std::min<int64_t>(E, numel); }

static int ksteps(int64_t K, int kind) { return static_cast<int>(K / (kind == kBf16 ? 64 : 128)); }

// kW4 decode GEMVs run 3 waves per SIMD (1024 SIMDs on an MI355X): among
// s = 1 .. KS / 4 the split with the fewest wave rounds x K steps per wave,
// the smallest on ties, so the last round is not a partial one (no split
// once one split's waves fill the GPU).
static int w4_splits(int64_t waves_per_split, int KS) {
  constexpr int64_t kSlots = 1024 * 3;
  if (waves_per_split >= kSlots) return 1;  // one split already fills the GPU
  int best = 1;
  int64_t cost = -1;
  for (int sp = 1; sp <= std::max(1, KS / 4); ++sp) {
    const int64_t rounds = (waves_per_split * sp + kSlots - 1) / kSlots;
    const int64_t c = rounds * ((KS + sp - 1) / sp);
    if (cost < 0 || c < cost) {
      cost = c;
      best = sp;
    }
  }
  return best;
}
static int w13_splits(int64_t numel, int E, int64_t H, int64_t I, int kind) {
  const int64_t wps = moe_umax(numel, E) * (2 * I / 16);
  return kind == kW4 ? w4_splits(wps, ksteps(H, kind)) : moe_splits(wps, ksteps(H, kind));
}
static int w2_splits(int64_t numel, int E, int64_t H, int64_t I, int kind) {
  const int64_t wps = moe_umax(numel, E) * (H / 16);
  return kind == kW4 ? w4_splits(wps, ksteps(I, kind)) : moe_splits(wps, ksteps(I, kind));
}

static size_t al256(size_t x) { return (x + 255) / 256 * 256; }

// Stage scratch: fp32 split-K partials of the decode GEMVs (none for GEMMs).
// Bytes of route_scales_kernel's copy for the fp8 grouped W13 on 128- and
// 256-route blocks (0 where it is not used): cap rows of H / 128 scales.
static size_t route_scales_bytes(int64_t cap, int64_t H, int block_m, int kind) {
  const size_t b = static_cast<size_t>(cap) * (H / 128) * 4;
  return kind == kFp8 && (block_m == kMoeBigBM || block_m == kMoeBM) && (H / 128) % 4 == 0 && b < (1ull << 31) ? b : 0;
}
static size_t w13_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int kind) {
  if (block_m != kGemvBlock) return route_scales_bytes(numel + static_cast<int64_t>(E) * (block_m - 1), H, block_m, kind);
  if (block_m != kGemvBlock) return 0;
  return al256(static_cast<size_t>(w13_splits(numel, E, H, I, kind)) * numel * 2 * I * 4);
}
static size_t w2_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int kind) {
  if (block_m != kGemvBlock) return 0;
  const int s = w2_splits(numel, E, H, I, kind);
  return s > 1 ? al256(static_cast<size_t>(s) * numel * H * 4) : 0;
}
static size_t stage_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int kind) {
  return std::max(w13_scratch(numel, E, H, I, block_m, kind),
                  w2_scratch(numel, E, H, I, block_m, kind));
}

template <bool W13, bool EVEN, bool SCT = false>
static int raise_w4_lds() {
  static bool done = false;
  if (done) return VMAMD_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(moe_w4_gemm_kernel<W13, EVEN, SCT>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, W4Pipe::kLds) != hipSuccess) {
    set_error("w4afp8 moe: cannot raise the LDS limit of the grouped GEMM kernel");
    return VMAMD_ERR_HIP;
  }
  done = true;
  return VMAMD_OK;
}

// True when the w4afp8 GEMMs over K can read their scales transposed (SCT;
// the transposition moves 8 bytes at a time: an even count of word pairs).
static bool w4_sct(int64_t K) { return (K / 128) % 4 == 0; }

// kW4 grouped GEMM launch (W13: N = 2I, out = bf16 activation; W2: N = H,
// out = y).  The scale words are read 4 bytes at a time, so the scale array
// must be 4-byte aligned; wst: the same scales transposed (W4ScalesT), or
// null.
template <bool W13>
static int launch_w4_gemm(const uint8_t* act, int64_t act_rows, const float* act_scale,
                          const float* act_corr, int topk, int K, const int32_t* sorted,
                          const int32_t* offs, const int32_t* ntpp, const int32_t* eids, int E, int numel,
                          int tiles, const uint8_t* w, const void* ws, int N, int I, float limit, uint16_t* out,
                          hipStream_t st, const uint32_t* wst = nullptr) {
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(ws) % 4 == 0,
                "w4afp8 moe: weight scales must be 4-byte aligned for the grouped GEMMs");
  VMAMD_REQUIRE(act_rows * K < (1ll << 31), "w4afp8 moe: the grouped GEMMs take activations below 2 GiB");
  const int act_bytes = static_cast<int>(act_rows * K);
  const uint16_t* wsh = static_cast<const uint16_t*>(ws);
  if (wst && w4_sct(K)) {
    int rc = raise_w4_lds<W13, true, true>();
    if (rc) return rc;
    moe_w4_gemm_kernel<W13, true, true><<<xcd_grid(tiles), 512, W4Pipe::kLds, st>>>(
        act, act_scale, act_corr, act_bytes, topk, K, sorted, offs, ntpp, eids, E, numel, tiles, w,
        reinterpret_cast<const uint16_t*>(wst), N, I, limit, out);
  } else if ((K / 128) % 2 == 0) {
    int rc = raise_w4_lds<W13, true>();
    if (rc) return rc;
    moe_w4_gemm_kernel<W13, true><<<xcd_grid(tiles), 512, W4Pipe::kLds, st>>>(
        act, act_scale, act_corr, act_bytes, topk, K, sorted, offs, ntpp, eids, E, numel, tiles, w, wsh, N, I,
        limit, out);
  } else {
    int rc = raise_w4_lds<W13, false>();
    if (rc) return rc;
    moe_w4_gemm_kernel<W13, false><<<xcd_grid(tiles), 512, W4Pipe::kLds, st>>>(
        act, act_scale, act_corr, act_bytes, topk, K, sorted, offs, ntpp, eids, E, numel, tiles, w, wsh, N, I,
        limit, out);
  }
  return check_launch(W13 ? "w4afp8 moe w13 (gemm)" : "w4afp8 moe w2 (gemm)");
}

template <int KIND, bool W13>
static int raise_dma_lds() {
  static bool done = false;
  if (done) return VMAMD_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(moe_gemm_dma_kernel<KIND, W13>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, MoePipe<KIND>::kLds) != hipSuccess) {
    set_error("moe gemm: cannot raise the LDS limit of the grouped GEMM kernel");
    return VMAMD_ERR_HIP;
  }
  done = true;
  return VMAMD_OK;
}

template <int KIND, bool W13, int MTV>
static int raise_big_lds() {
  static bool done = false;
  if (done) return VMAMD_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(moe_big_kernel<KIND, W13, MTV>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, MoeBigTile<MTV>::kLds) != hipSuccess) {
    set_error("moe gemm: cannot raise the LDS limit of the grouped GEMM kernel");
    return VMAMD_ERR_HIP;
  }
  done = true;
  return VMAMD_OK;
}

// moe_big_kernel with m-tiles of 16 * MTV routes per wave (block size 64 * MTV).
template <int KIND, bool W13, int MTV, typename... Args>
static int launch_big(int tiles, hipStream_t st, Args... args) {
  int rc = raise_big_lds<KIND, W13, MTV>();
  if (rc) return rc;
  moe_big_kernel<KIND, W13, MTV><<<xcd_grid(tiles), MoeBigTile<MTV>::kThreads, MoeBigTile<MTV>::kLds, st>>>(args...);
  return check_launch(W13 ? "moe w13 (gemm)" : "moe w2 (gemm)");
}

// The 256-route kernels read activations, scales and each expert's weights
// through buffer descriptors: all below 2 GiB.
static bool big_fits(int64_t act_rows, int64_t K, int64_t N, int E) {
  return act_rows * K < (1ll << 31) && act_rows * (K / 128) * 4 < (1ll << 31) && N * K < (1ll << 31) &&
         static_cast<int64_t>(E) * ((N + 127) / 128) * (K / 128) * 4 < (1ll << 31);
}

// Bytes of a decode GEMV's activation operand ([rows, K]); the GEMV reads it
// through a buffer descriptor, which the callers keep below 2 GiB.
template <int KIND>
static int gemv_act_bytes(int64_t rows, int64_t K) {
  return static_cast<int>(rows * (K / KindBytes<KIND>::kElems) * KindBytes<KIND>::kAct);
}

// Decode GEMV launch.  one_block: the single-block form (MAXB = 1: fewer
// registers, the pipelined K loop), which still handles an expert with more
// than 16 routes by re-streaming its weights once per block; chosen while
// experts average at most 8 routes (gemv_one_block), where it measured as
// fast or faster than the 4-block form (w4afp8 E=128 at T=32: 366 -> 285 us,
// T=64: 422 -> 338 us; bf16 E=128 T=128 and fp8 E=256 T=64 1-3 % faster).
// vs: the kFp8 scale layout allows one 16-byte load per group of scales.
static bool gemv_one_block(int64_t numel, int E) { return numel <= 8 * static_cast<int64_t>(E); }

template <int KIND, int MODE = kGemvGrouped, typename... Args>
static void launch_gemv(dim3 grid, hipStream_t st, bool one_block, bool vs, Args... args) {
  const int32_t* none = nullptr;
  if constexpr (KIND != kBf16) {
    if (vs) {
      if (one_block)
        moe_gemv_kernel<1, KIND, true, MODE><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args..., none, none, 0, 0, nullptr, nullptr, nullptr, 0.f, 0);
      else
        moe_gemv_kernel<4, KIND, true, MODE><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args..., none, none, 0, 0, nullptr, nullptr, nullptr, 0.f, 0);
      return;
    }
  }
  if (one_block)
    moe_gemv_kernel<1, KIND, false, MODE><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args..., none, none, 0, 0, nullptr, nullptr, nullptr, 0.f, 0);
  else
    moe_gemv_kernel<4, KIND, false, MODE><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args..., none, none, 0, 0, nullptr, nullptr, nullptr, 0.f, 0);
}

// The decode GEMV with direct route slots (kGemvDirect, kGemvDirectAct, the combines).
template <int KIND, int MODE, typename... Args>
static void launch_gemv_direct(dim3 grid, int threads, size_t lds, hipStream_t st, bool vs, Args... args) {
  if constexpr (MODE == kGemvDirectQ) {  // kFp8 / kW4 with vector scales only
    if constexpr (KIND == kFp8 || KIND == kW4) moe_gemv_kernel<1, KIND, true, MODE><<<grid, threads, lds, st>>>(args...);
    return;
  }
  if constexpr (KIND != kBf16 && MODE != kGemvDirectQ) {
    if (vs) {
      moe_gemv_kernel<1, KIND, true, MODE><<<grid, threads, lds, st>>>(args...);
      return;
    }
  }
  if constexpr (MODE != kGemvDirectQ) moe_gemv_kernel<1, KIND, false, MODE><<<grid, threads, lds, st>>>(args...);
}

// True when a GEMV over K may read its scales U at a time: K/128 a multiple
// of U and the scale arrays aligned so that every row is (kFp8: 16 bytes for
// both scale sets; kW4: 8 bytes for the bf16 weight scales, 16 for the
// activation corrections).
template <int KIND>
static bool gemv_vector_scales(int64_t K, const void* act_s, const void* w_s) {
  if constexpr (KIND == kFp8)
    return (K / 128) % kGemvU == 0 && reinterpret_cast<uintptr_t>(act_s) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(w_s) % 16 == 0;
  if constexpr (KIND == kW8A16) return (K / 128) % kGemvU == 0 && reinterpret_cast<uintptr_t>(w_s) % 16 == 0;
  if constexpr (KIND == kW4)
    return (K / 128) % kGemvU == 0 && reinterpret_cast<uintptr_t>(w_s) % 8 == 0 &&
           reinterpret_cast<uintptr_t>(act_s) % 16 == 0;
  return false;
}

// The reference GEMV's activation (moe_act_native_kernel) over numel routes:
// ids (with emap / E) name the dead routes, which get zero rows; null ids
// make every route live.
static int launch_act_native(const float* scratch, int splits, int numel, int I, float limit,
                             const float* route_w, const int32_t* ids, const int32_t* emap,
                             int64_t emap_len, int E, uint16_t* a2, hipStream_t st) {
  const int64_t chunks = static_cast<int64_t>(numel) * (I / 8);
  const int blocks = static_cast<int>((chunks + 255) / 256);
#define VMAMD_ACTN(S)                                                                                 \
  moe_act_native_kernel<S><<<blocks, 256, 0, st>>>(scratch, splits, numel, I, limit, route_w, ids, emap, \
                                                   emap_len, E, a2)
  switch (splits) {
    case 1: VMAMD_ACTN(1); break;
    case 2: VMAMD_ACTN(2); break;
    case 3: VMAMD_ACTN(3); break;
    case 4: VMAMD_ACTN(4); break;
    default: VMAMD_ACTN(0); break;
  }
#undef VMAMD_ACTN
  return check_launch("moe w13 (activation)");
}

// The decode path's activation: split-K sum of the W13 partials, SwiGLU and
// a2 (kFp8: 1x128 quantiser; kW4: per-row quantiser in w4 order; kBf16: the
// bf16 activation; kW8A16, and kBf16 with `native`: the reference GEMV's
// activation, which keeps gate and up in fp32 through the SwiGLU).
template <int KIND>
static int launch_act_decode(const float* scratch, int s13, int numel, int I, float limit,
                             const float* route_w, const float* xs, int topk, uint8_t* a2,
                             float* a2s, float* a2corr, hipStream_t st, bool native = false) {
  if (KIND == kW8A16 || native)
    return launch_act_native(scratch, s13, numel, I, limit, route_w, nullptr, nullptr, 0, 0,
                             reinterpret_cast<uint16_t*>(a2), st);
  if constexpr (KIND == kFp8) {
    const int64_t groups = static_cast<int64_t>(numel) * (I / 128);
    const int blocks = static_cast<int>((groups + 15) / 16);
#define VMAMD_ACTQ(S) \
  moe_act_quant_kernel<S><<<blocks, 256, 0, st>>>(scratch, s13, numel, I, limit, route_w, a2, a2s)
    switch (s13) {
      case 1: VMAMD_ACTQ(1); break;
      case 2: VMAMD_ACTQ(2); break;
      case 3: VMAMD_ACTQ(3); break;
      case 4: VMAMD_ACTQ(4); break;
      default: VMAMD_ACTQ(0); break;
    }
#undef VMAMD_ACTQ
  } else if constexpr (KIND == kW4) {  // a2: fp8 [numel, I], a2s: row scales
    moe_act_rowquant_w4_kernel<<<numel, kRowThreads, 0, st>>>(scratch, s13, numel, I, limit, xs,
                                                              topk, a2, a2s, a2corr);
  } else {
    const int64_t chunks = static_cast<int64_t>(numel) * (I / 8);
    moe_act_bf16_kernel<KIND><<<static_cast<int>((chunks + 255) / 256), 256, 0, st>>>(
        scratch, s13, numel, I, limit, xs, topk, route_w, reinterpret_cast<uint16_t*>(a2));
  }
  return check_launch("moe w13 (activation)");
}

// Launches of the two stages; arguments are validated by the callers.  kBf16:
// xa is x itself, xs / w13_s / a2s unused; kW8A16 (decode path only): xa is
// x itself, xs / a2s unused, a2 bf16.  kW4: xa in w4 order with the
// block corrections xcorr, xs the token row scales; the decode path writes
// a2 (w4 order) with a2s and a2corr, the prefill path the bf16 activation to
// a2 (quantised per row by the caller).
template <int KIND>
static int launch_w13(const uint8_t* xa, const float* xs, const float* xcorr, int T, int H, int topk,
                      const int32_t* sorted, int64_t cap, int block_m, const int32_t* offs,
                      const int32_t* ntpp, const int32_t* active, const int32_t* nact,
                      const uint8_t* w13, const void* w13_s, int E, int I, float limit,
                      const float* route_w, uint8_t* a2, float* a2s, float* a2corr, float* scratch,
                      hipStream_t st, const int32_t* eids = nullptr, bool native = false,
                      const uint32_t* w4st = nullptr, const float* xs_routes = nullptr, bool a2s_routes = false) {
  const int numel = T * topk;
  const float* act_s = KIND == kW4 ? xcorr : xs;  // per-step activation values the GEMV reads
  VMAMD_REQUIRE(KIND != kW8A16 || block_m == kGemvBlock, "moe w13: bf16 x fp8 runs on the decode GEMV only");
  if (KIND == kW8A16 || block_m == kGemvBlock) {
    const int s13 = w13_splits(numel, E, H, I, KIND);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g13((2 * I / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s13);
    launch_gemv<KIND>(g13, st, gemv_one_block(numel, E), gemv_vector_scales<KIND>(H, act_s, w13_s), xa, gemv_act_bytes<KIND>(T, H),
                      act_s, topk, H, sorted, offs, active,
                      nact, w13, w13_s, 2 * I, numel, s13, scratch,
                      static_cast<const float*>(nullptr), static_cast<uint16_t*>(nullptr));
    int rc = check_launch("moe w13 (gemv)");
    if (rc) return rc;
    return launch_act_decode<KIND>(scratch, s13, numel, I, limit, route_w, xs, topk, a2, a2s, a2corr, st,
                                   native);
  }
  if constexpr (KIND == kFp8 || KIND == kBf16) {
    if (block_m == kMoeBigBM || block_m == kMoeBig320) {
      constexpr int eb = KIND == kBf16 ? 2 : 1;  // bytes per element
      VMAMD_REQUIRE(big_fits(T, H * eb, 2ll * I, E), "moe w13: operands past 2 GiB for the 256-route GEMM");
      const int tiles = static_cast<int>((cap + block_m - 1) / block_m) * (I / 128);
      const int abytes = static_cast<int>(static_cast<int64_t>(T) * H * eb);
      const int sbytes = static_cast<int>(static_cast<int64_t>(T) * (H / 128) * 4);
      const float* ws13 = static_cast<const float*>(w13_s);
      if (block_m == kMoeBig320) {
        if constexpr (KIND == kBf16)
          return launch_big<KIND, true, 5>(tiles, st, xa, abytes, xs, sbytes, topk, static_cast<int>(H), sorted, offs,
                                           ntpp, eids, E, numel, tiles, w13, ws13, 2 * I, I, limit, route_w, a2, a2s,
                                           static_cast<uint16_t*>(nullptr));
      }
      // xs_routes: route_scales_kernel's copy of the x scales; a2s_routes:
      // a2s written in route order for a W2 launch with a2s_routes.
      const int order = (xs_routes ? kActScalesInRoutes : 0) | (a2s_routes ? kA2ScalesInRoutes : 0);
      return launch_big<KIND, true, 4>(tiles, st, xa, abytes, xs_routes ? xs_routes : xs,
                                       xs_routes ? static_cast<int>(cap * (H / 128) * 4) : sbytes, topk,
                                       static_cast<int>(H), sorted, offs, ntpp, eids, E, numel, tiles, w13, ws13,
                                       2 * I, I, limit, route_w, a2, a2s, static_cast<uint16_t*>(nullptr), order);
    }
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  const int tiles = max_blocks * (I / 128);
  if constexpr (KIND == kW4) {
    return launch_w4_gemm<true>(xa, T, xs, xcorr, topk, H, sorted, offs, ntpp, eids, E, numel, tiles, w13,
                                w13_s, 2 * I, I, limit, reinterpret_cast<uint16_t*>(a2), st, w4st);
  } else if constexpr (KIND == kFp8 || KIND == kBf16) {
    int rc = raise_dma_lds<KIND, true>();
    if (rc) return rc;
    const int64_t abytes = static_cast<int64_t>(T) * H * KindBytes<KIND>::kAct / KindBytes<KIND>::kElems;
    VMAMD_REQUIRE(abytes < (1ll << 31), "moe w13: activations past 2 GiB for the grouped GEMM");
    const int order = (xs_routes ? kActScalesInRoutes : 0) | (a2s_routes ? kA2ScalesInRoutes : 0);
    moe_gemm_dma_kernel<KIND, true><<<xcd_grid(tiles), 512, MoePipe<KIND>::kLds, st>>>(
        xa, static_cast<int>(abytes), xs_routes ? xs_routes : xs, topk, H, sorted, offs, ntpp, eids, E, numel,
        tiles, w13, static_cast<const float*>(w13_s), 2 * I, I, limit, route_w, a2, a2s, nullptr, order);
  }
  return check_launch("moe w13 (gemm)");
}

// kW4: a2s are the a2 row scales and take the routed weight's place in y;
// a2corr the block corrections of a2 (w4 order).
// combined_out: when given and the decode path splits K, the reduce and the
// top-k combine run as one kernel writing the layer output there (y is not
// written) and *combined is set; otherwise y is written as usual.
template <int KIND>
static int launch_w2(const uint8_t* a2, const float* a2s, const float* a2corr, int T, int topk,
                     const int32_t* sorted,
                     int64_t cap, int block_m, const int32_t* offs, const int32_t* ntpp,
                     const int32_t* active, const int32_t* nact, const uint8_t* w2, const void* w2_s,
                     int E, int H, int I, const float* topk_weights, const float* route_w,
                     const int32_t* topk_ids, const int32_t* emap, int64_t emap_len, uint16_t* y,
                     float* scratch, hipStream_t st, uint16_t* combined_out = nullptr,
                     bool* combined = nullptr, const int32_t* eids = nullptr, const uint32_t* w4st = nullptr,
                     bool a2s_routes = false) {
  const int numel = T * topk;
  const float* yscale = KIND == kW4 ? a2s : route_w;
  const float* act_s = KIND == kW4 ? a2corr : a2s;  // per-step activation values the GEMV reads
  if (combined) *combined = false;
  VMAMD_REQUIRE(KIND != kW8A16 || block_m == kGemvBlock, "moe w2: bf16 x fp8 runs on the decode GEMV only");
  if (KIND == kW8A16 || block_m == kGemvBlock) {
    const int s2 = w2_splits(numel, E, H, I, KIND);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g2((H / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s2);
    if (s2 > 1 && combined_out && combined && H % 8 == 0) {
      launch_gemv<KIND>(g2, st, gemv_one_block(numel, E), gemv_vector_scales<KIND>(I, act_s, w2_s), a2, gemv_act_bytes<KIND>(numel, I), act_s, 1, I, sorted, offs, active,
                        nact, w2, w2_s, H, numel, s2, scratch, static_cast<const float*>(nullptr),
                        static_cast<uint16_t*>(nullptr));
      int rc = check_launch("moe w2 (gemv)");
      if (rc) return rc;
      if constexpr (KIND == kW4)
        launch_w2_combine<true>(scratch, s2, T, topk, H, topk_ids, emap, emap_len, E, yscale,
                                topk_weights, combined_out, st);
      else
        launch_w2_combine<false>(scratch, s2, T, topk, H, topk_ids, emap, emap_len, E, yscale,
                                 nullptr, combined_out, st);
      *combined = true;
      return check_launch("moe w2 (combine)");
    }
    if (s2 == 1) {
      launch_gemv<KIND>(g2, st, gemv_one_block(numel, E), gemv_vector_scales<KIND>(I, act_s, w2_s), a2, gemv_act_bytes<KIND>(numel, I), act_s, 1, I, sorted, offs,
                        active, nact, w2, w2_s, H, numel, 1, static_cast<float*>(nullptr), yscale, y);
      return check_launch("moe w2 (gemv)");
    }
    launch_gemv<KIND>(g2, st, gemv_one_block(numel, E), gemv_vector_scales<KIND>(I, act_s, w2_s), a2, gemv_act_bytes<KIND>(numel, I), act_s, 1, I, sorted, offs, active,
                      nact, w2, w2_s, H, numel, s2, scratch, static_cast<const float*>(nullptr),
                      static_cast<uint16_t*>(nullptr));
    int rc = check_launch("moe w2 (gemv)");
    if (rc) return rc;
    const int64_t mn = static_cast<int64_t>(numel) * H;
    moe_w2_reduce_kernel<false><<<static_cast<int>((mn / 4 + 255) / 256), 256, 0, st>>>(
        scratch, s2, numel, H, topk_ids, emap, emap_len, E, yscale, y);
    return check_launch("moe w2 (reduce)");
  }
  if constexpr (KIND == kFp8 || KIND == kBf16) {
    if (block_m == kMoeBigBM || block_m == kMoeBig320) {
      constexpr int eb = KIND == kBf16 ? 2 : 1;  // bytes per element
      VMAMD_REQUIRE(big_fits(cap, I * eb, H, E), "moe w2: operands past 2 GiB for the 256-route GEMM");
      const int tiles = static_cast<int>((cap + block_m - 1) / block_m) * ((H + 255) / 256);
      const int abytes = static_cast<int>(cap * I * eb), sbytes = static_cast<int>(cap * (I / 128) * 4);
      const float* ws2 = static_cast<const float*>(w2_s);
      uint8_t* const none8 = nullptr;
      float* const nonef = nullptr;
      if (block_m == kMoeBig320) {
        if constexpr (KIND == kBf16)
          return launch_big<KIND, false, 5>(tiles, st, a2, abytes, a2s, sbytes, 1, I, sorted, offs, ntpp, eids, E,
                                            numel, tiles, w2, ws2, H, I, 0.f, route_w, none8, nonef, y);
      }
      return launch_big<KIND, false, 4>(tiles, st, a2, abytes, a2s, sbytes, 1, I, sorted, offs, ntpp, eids, E, numel,
                                        tiles, w2, ws2, H, I, 0.f, route_w, none8, nonef, y,
                                        a2s_routes ? kActScalesInRoutes : 0);
    }
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  if constexpr (KIND == kW4) {
    const int tiles = max_blocks * ((H + W4Pipe::BN - 1) / W4Pipe::BN);
    return launch_w4_gemm<false>(a2, cap, a2s, a2corr, 1, I, sorted, offs, ntpp, eids, E, numel, tiles, w2,
                                 w2_s, H, I, 0.f, y, st, w4st);
  } else if constexpr (KIND == kFp8 || KIND == kBf16) {
    const int tiles = max_blocks * ((H + 255) / 256);
    int rc = raise_dma_lds<KIND, false>();
    if (rc) return rc;
    const int64_t abytes = cap * I * KindBytes<KIND>::kAct / KindBytes<KIND>::kElems;
    VMAMD_REQUIRE(abytes < (1ll << 31), "moe w2: activations past 2 GiB for the grouped GEMM");
    moe_gemm_dma_kernel<KIND, false><<<xcd_grid(tiles), 512, MoePipe<KIND>::kLds, st>>>(
        a2, static_cast<int>(abytes), a2s, 1, I, sorted, offs, ntpp, eids, E, numel, tiles, w2, static_cast<const float*>(w2_s), H,
        I, 0.f, route_w, nullptr, nullptr, y, a2s_routes ? kActScalesInRoutes : 0);
  }
  return check_launch("moe w2 (gemm)");
}

// Workspace carve-up of a fused layer, shared by the size query and the
// launcher.  The two stages run one after the other on one stream, so their
// scratch shares one region.  kFp8 / kW4 add the quantised x and scales; kW4
// also keeps the bf16 activation before its row quantiser.
struct MoeWs {
  size_t xq, xs, xcorr, sorted, eids, ntpp, offs, active, nact, acnt, abf, a2, a2s, a2corr, y, scratch, wst13,
      wst2, xsr, total;
  bool sct13, sct2;  // kW4 grouped GEMMs: the transposed weight scales (W4ScalesT) at wst13 / wst2
};

static MoeWs moe_layout(int64_t T, int topk, int E, int64_t H, int64_t I, int bm, int kind) {
  MoeWs w{};
  const int64_t numel = T * topk;
  const int64_t cap = numel + static_cast<int64_t>(E) * (bm - 1);
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o += al256(bytes); return at; };
  if (kind == kFp8 || kind == kW4) {
    w.xq = take(T * H);
    w.xs = take(kind == kFp8 ? T * (H / 128) * 4 : T * 4);
  }
  if (kind == kW4) w.xcorr = take(T * (H / 128) * 4);
  w.sorted = take(cap * 4);
  w.eids = take(((cap + bm - 1) / bm) * 4);
  w.ntpp = take(4);
  w.offs = take((E + 1) * 4);
  w.active = take(E * 4);
  w.nact = take(4);
  if (kind == kBf16 || kind == kW8A16) w.acnt = take(align_counts_bytes(numel, E));  // align_routes
  const int64_t arows = bm == kGemvBlock ? numel : cap;  // route order (decode) or padded order
  if (kind == kW4) w.abf = take(arows * I * 2);
  w.a2 = take(arows * I * (kind == kBf16 || kind == kW8A16 ? 2 : 1));
  if (kind == kFp8) w.a2s = take(arows * (I / 128) * 4);
  if (kind == kW4) {
    w.a2s = take(arows * 4);
    w.a2corr = take(arows * (I / 128) * 4);
  }
  w.y = take(numel * H * 2);
  w.scratch = take(stage_scratch(numel, E, H, I, bm, kind));
  w.sct13 = kind == kW4 && bm != kGemvBlock && w4_sct(H);
  w.sct2 = kind == kW4 && bm != kGemvBlock && w4_sct(I);
  if (w.sct13) w.wst13 = take(static_cast<size_t>(E) * 2 * I * (H / 128) * 2);
  if (w.sct2) w.wst2 = take(static_cast<size_t>(E) * H * (I / 128) * 2);
  w.xsr = take(route_scales_bytes(cap, H, bm, kind));  // route_scales_kernel
  w.total = o;
  return w;
}

// One token on the decode path (top-k <= kMaxCombineSlots): every route is
// its own GEMV slot, so the alignment is skipped (kFp8 / kW4: x is quantised
// inside the W13 launch), and the W2 GEMV sums the top-k in the same launch.
// Each route reads its expert's weights, so routes that share an expert read
// them again: a token's top-k names distinct experts, but with more tokens a
// batch whose tokens pick the same experts would read each expert's weights
// once per token (measured: DeepSeek-V3 fp8 at T=2 with both tokens on the
// same 8 experts, slower than the grouped GEMMs), which the grouped slots of
// the alignment avoid.  With varied routing the direct slots measured faster
// up to 16 routes (fp8 DeepSeek-V3) and 64 / 96 routes (bf16 / w4afp8 E=128
// layers), but the dispatch has no sight of the routing before the launch.
// kW4: a2s are the a2 row scales (the W2 output scale) and the routed weights
// enter the sum, as in the grouped form.
static bool use_direct_slots(int64_t T, int topk, int kind) { return T == 1 && topk <= combine_slots(kind); }
// The W13 launch writes the activation itself (kGemvDirectAct) when its
// split count fits one workgroup.
static bool direct_act(int kind, int s13) {
  return (kind == kBf16 || kind == kW8A16) && s13 <= gemv_waves(kGemvDirectAct, kind) / 2;
}

// The W2 GEMV of one token with the top-k sum (kGemvCombine), over the K
// splits the grouped W2 GEMV takes for the same routes, so that the sums are
// its bits.
template <int KIND>
static int launch_combine(const uint8_t* a2, const float* a2s, const float* a2corr, int T, int H, int I, int numel,
                          int topk, const uint8_t* w2, const void* w2_s, const float* topk_weights,
                          const int32_t* topk_ids, const int32_t* emap, int64_t emap_len, int E,
                          const float* w2_rw, uint16_t* out, hipStream_t st) {
  const int32_t* none = nullptr;
  const float* a2_act_s = KIND == kW4 ? a2corr : a2s;
  const float* yscale = KIND == kW4 ? a2s : w2_rw;
  launch_gemv_direct<KIND, kGemvCombine>(
      dim3(H / 16, T, 1), topk * kWave, 0, st, gemv_vector_scales<KIND>(I, a2_act_s, w2_s), a2,
      gemv_act_bytes<KIND>(numel, I), a2_act_s, 1, I, none, none, none, none, w2, w2_s, H, numel,
      w2_splits(numel, E, H, I, KIND), static_cast<float*>(nullptr), yscale, static_cast<uint16_t*>(nullptr),
      topk_ids, emap, emap_len, E, out,
      KIND == kW4 ? topk_weights : static_cast<const float*>(nullptr), static_cast<float*>(nullptr), 0.f, 0);
  return check_launch("moe w2 (gemv + top-k sum)");
}

// xa: x as the W13 GEMV reads it (kFp8 / kW4: quantised by the caller, with
// xs the 1x128 scales / the row scales and xcorr the kW4 block corrections);
// qx (kFp8 / kW4): xa is the bf16 x, quantised by each W13 workgroup in LDS
// (kW4: xs receives the row scales from the W13 launch).
template <int KIND>
static int fused_direct(bool qx, const uint8_t* xa, const float* xs, const float* xcorr, int T, int H,
                        const uint8_t* w13, const void* w13_s, const uint8_t* w2, const void* w2_s,
                        int E, int I, int topk, const float* topk_weights, const int32_t* topk_ids,
                        const int32_t* emap, int64_t emap_len, float limit, const float* w13_rw,
                        const float* w2_rw, float* scratch, uint8_t* a2, float* a2s, float* a2corr,
                        uint16_t* out, hipStream_t st, bool native = false) {
  const int numel = T * topk;
  const int32_t* none = nullptr;
  const float* act_s = KIND == kW4 ? xcorr : xs;
  const int s13 = w13_splits(numel, E, H, I, KIND);
  const dim3 g13((2 * I / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, numel, s13);
  int rc = VMAMD_OK;
  if constexpr (KIND == kBf16 || KIND == kW8A16) {
    if (direct_act(KIND, s13)) {
      launch_gemv_direct<KIND, kGemvDirectAct>(
          dim3(I / 16, numel, 1), 2 * s13 * kWave, 0, st, gemv_vector_scales<KIND>(H, act_s, w13_s), xa,
          gemv_act_bytes<KIND>(T, H), act_s, topk, H, none, none, none, none, w13, w13_s, 2 * I, numel, s13,
          static_cast<float*>(nullptr), w13_rw, reinterpret_cast<uint16_t*>(a2), topk_ids, emap, emap_len, E,
          static_cast<uint16_t*>(nullptr), static_cast<const float*>(nullptr), static_cast<float*>(nullptr), limit,
          KIND == kW8A16 || native ? 1 : 0);
      rc = check_launch("moe w13 (gemv + activation)");
      if (rc) return rc;
      return launch_combine<KIND>(a2, a2s, a2corr, T, H, I, numel, topk, w2, w2_s, topk_weights, topk_ids, emap,
                                  emap_len, E, w2_rw, out, st);
    }
  }
  if (qx) {
    launch_gemv_direct<KIND, kGemvDirectQ>(
        g13, kMoeGemvWaves * kWave, static_cast<size_t>(H) + (H / 128) * 4 + (KIND == kW4 ? 32 : 0), st, true,
        xa, static_cast<int>(static_cast<int64_t>(T) * H * 2), static_cast<const float*>(nullptr), topk, H, none,
        none, none, none, w13, w13_s, 2 * I, numel, s13, scratch, static_cast<const float*>(nullptr),
        static_cast<uint16_t*>(nullptr), topk_ids, emap, emap_len, E, static_cast<uint16_t*>(nullptr),
        static_cast<const float*>(nullptr), KIND == kW4 ? const_cast<float*>(xs) : static_cast<float*>(nullptr),
        0.f, 0);
  } else {
    launch_gemv_direct<KIND, kGemvDirect>(
        g13, kMoeGemvWaves * kWave, 0, st, gemv_vector_scales<KIND>(H, act_s, w13_s), xa,
        gemv_act_bytes<KIND>(T, H), act_s, topk, H, none, none, none, none, w13, w13_s, 2 * I, numel, s13,
        scratch, static_cast<const float*>(nullptr), static_cast<uint16_t*>(nullptr), topk_ids, emap, emap_len,
        E, static_cast<uint16_t*>(nullptr), static_cast<const float*>(nullptr), static_cast<float*>(nullptr), 0.f, 0);
  }
  rc = check_launch("moe w13 (gemv)");
  if (rc) return rc;
  rc = launch_act_decode<KIND>(scratch, s13, numel, I, limit, w13_rw, xs, topk, a2, a2s, a2corr, st, native);
  if (rc) return rc;
  return launch_combine<KIND>(a2, a2s, a2corr, T, H, I, numel, topk, w2, w2_s, topk_weights, topk_ids, emap,
                              emap_len, E, w2_rw, out, st);
}

// Path choice of `auto`: the decode kernels (GEMV over 16-route blocks) up to
// a number of routes per expert measured on MI355X, the grouped GEMMs over
// 128- or 256-route blocks above.  Measured crossovers (graph replay, caches
// flushed): fp8 DeepSeek-V3 (E=256, H=7168, I=2048, top-8) between 2 and 3
// routes per expert (T=64 / 96); bf16 (E=128, H=2048, I=768) and w4afp8
// (E=128, H=4096, I=1536) between 8 and 16 (T=128 / 256).
// fp8 and bf16 layers with at least 128 routes per expert take 256-route
// blocks (moe_big_kernel), against 128-route blocks, W13 / W2: fp8
// DeepSeek-V3 (E=256, H=7168, I=2048, top-8) T=3072 +3 % / -3 %, T=4096
// -1 % / -6 %, T=6144 -8 % / -10 %, T=8192 -2 % / -10 %; bf16 (E=128,
// H=2048, I=768, top-8) T=2048 -7 % / -10 %, T=4096 -12 % / 0, T=8192
// -10 % / -17 %.
// bf16 takes 320-route blocks where the expected largest expert, mean +
// 3 sqrt(mean) routes, needs fewer of them than of 256-route blocks, each
// 320-route block counted 1.25x (its share of the work when blocks are
// full).  bf16 (E=128, H=2048, I=768, top-8), W13 + W2 stages, 256 vs 320
// routes per block: T=1024 325 / 354 µs, T=2048 345 / 370, T=3072 364 / 396,
// T=4096 (mean 256) 512 / 423, T=6144 621 / 719, T=8192 (mean 512) 797 /
// 727, T=16384 1367 / 1418: the rule takes 320 at T=4096 and 8192 only.
// Results are bitwise equal either way.
static int bf16_big_block(int64_t routes, int E) {
  const double mean = static_cast<double>(routes) / E;
  const double top = mean + 3.0 * std::sqrt(mean);
  const double b256 = std::ceil(top / kMoeBigBM), b320 = std::ceil(top / kMoeBig320);
  return 1.25 * b320 < b256 ? kMoeBig320 : kMoeBigBM;
}

static int moe_block_m(int64_t T, int topk, int E, int path, int kind) {
  if (path == VMAMD_MOE_PATH_GEMV || path == VMAMD_MOE_PATH_NATIVE_GEMV || kind == kW8A16) return kGemvBlock;
  const int64_t routes = T * topk;
  const int big = kind == kBf16 ? bf16_big_block(routes, E) : kMoeBigBM;
  const int grouped = kind != kW4 && routes >= 128 * static_cast<int64_t>(E) ? big : kMoeBM;
  if (path == VMAMD_MOE_PATH_GEMM) return grouped;
  const int64_t limit = kind == kFp8 ? (5 * static_cast<int64_t>(E)) / 2 : 12 * static_cast<int64_t>(E);
  return routes <= limit ? kGemvBlock : grouped;
}

static int check_stage_common(const char* who, int kind, int64_t T, int topk, int E, int64_t H,
                              int64_t I, int block_m, int64_t cap) {
  VMAMD_REQUIRE(T >= 0 && topk > 0 && E > 0 && E <= 1024, "%s: bad sizes (T=%lld topk=%d E=%d)",
                who, (long long)T, topk, E);
  VMAMD_REQUIRE(H > 0 && I > 0 && H % 128 == 0 && I % 128 == 0,
                "%s: hidden (%lld) and intermediate (%lld) sizes must be multiples of 128", who,
                (long long)H, (long long)I);
  VMAMD_REQUIRE(block_m == kGemvBlock || block_m == kMoeBM || block_m == kMoeBigBM || block_m == kMoeBig320,
                "%s: block_m must be %d, %d, %d or %d (got %d)", who, kGemvBlock, kMoeBM, kMoeBigBM, kMoeBig320,
                block_m);
  VMAMD_REQUIRE(block_m != kMoeBig320 || kind == kBf16, "%s: block_m %d is for bf16 weights only", who,
                kMoeBig320);
  VMAMD_REQUIRE(block_m != kMoeBigBM || kind == kFp8 || kind == kBf16, "%s: block_m %d needs fp8 or bf16 weights",
                who, kMoeBigBM);
  VMAMD_REQUIRE(T * topk < (1ll << 30) && T * H < (1ll << 40), "%s: problem too large", who);
  VMAMD_REQUIRE(block_m != kGemvBlock || (T * H * 2 < (1ll << 31) && T * topk * I * 2 < (1ll << 31)),
                "%s: the decode path (block_m 16) takes activations below 2 GiB", who);
  VMAMD_REQUIRE(cap >= T * topk + static_cast<int64_t>(E) * (block_m - 1) && cap < (1ll << 31),
                "%s: capacity %lld < T*topk + E*(block_m-1)", who, (long long)cap);
  return VMAMD_OK;
}

template <int KIND>
static int fused_layer(const char* who, const void* x, int64_t T, int64_t H, const void* w13,
                       const void* w13_s, const void* w2, const void* w2_s, int E, int64_t I,
                       const float* topk_weights, const int32_t* topk_ids, int topk,
                       const int32_t* expert_map, int64_t expert_map_len, float swiglu_limit,
                       bool weight_on_input, int path, void* out, void* workspace,
                       size_t workspace_bytes, vmamd_stream_t stream) {
  VMAMD_REQUIRE(path >= VMAMD_MOE_PATH_AUTO && path <= VMAMD_MOE_PATH_NATIVE_GEMV, "%s: unknown path %d",
                who, path);
  VMAMD_REQUIRE(KIND != kW4 || !weight_on_input, "%s: apply_router_weight_on_input is not supported",
                who);
  // The reference GEMV's numerics: activations not quantised, gate / up kept
  // in fp32 through the SwiGLU (kW8A16 for fp8 weights, kBf16 with the native
  // activation for bf16 weights).
  const bool native = KIND == kW8A16 || path == VMAMD_MOE_PATH_NATIVE_GEMV;
  VMAMD_REQUIRE(!native || KIND == kW8A16 || KIND == kBf16, "%s: the native GEMV path takes fp8 or bf16 weights",
                who);
  const int bm = moe_block_m(T, topk, E, path, KIND);
  const int64_t cap = T * topk + static_cast<int64_t>(E) * (bm - 1);
  int rc = check_stage_common(who, KIND, T, topk, E, H, I, bm, cap);
  if (rc) return rc;
  VMAMD_REQUIRE(KIND != kW4 || (H <= 16384 && I <= 16384),
                "%s: per-row quantisation supports rows of up to 16384", who);
  VMAMD_REQUIRE(KIND != kW4 || (reinterpret_cast<uintptr_t>(w13_s) % 4 == 0 &&
                                reinterpret_cast<uintptr_t>(w2_s) % 4 == 0),
                "%s: weight scales must be 4-byte aligned", who);
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && w13 && w2 && topk_weights && topk_ids && out &&
                    (KIND == kBf16 || (w13_s && w2_s)),
                "%s: null pointer", who);
  const MoeWs L = moe_layout(T, topk, E, H, I, bm, KIND);
  VMAMD_REQUIRE(workspace && workspace_bytes >= L.total, "%s: workspace of %zu bytes required (got %zu)",
                who, L.total, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0 &&
                    reinterpret_cast<uintptr_t>(x) % 16 == 0,
                "%s: workspace must be 256-byte and x 16-byte aligned", who);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
  int32_t* eids = reinterpret_cast<int32_t*>(ws + L.eids);
  int32_t* ntpp = reinterpret_cast<int32_t*>(ws + L.ntpp);
  int32_t* offs = reinterpret_cast<int32_t*>(ws + L.offs);
  int32_t* active = reinterpret_cast<int32_t*>(ws + L.active);
  int32_t* nact = reinterpret_cast<int32_t*>(ws + L.nact);
  uint8_t* a2 = ws + L.a2;
  float* a2s = KIND == kBf16 || KIND == kW8A16 ? nullptr : reinterpret_cast<float*>(ws + L.a2s);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  float* scratch = reinterpret_cast<float*>(ws + L.scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int numel = static_cast<int>(T * topk);
  const int h = static_cast<int>(H), i = static_cast<int>(I), t = static_cast<int>(T);

  // The routed weight is applied once: on the W13 output before the
  // activation (apply_router_weight_on_input), otherwise in the W2 epilogue.
  const float* w13_rw = weight_on_input ? topk_weights : nullptr;
  const float* w2_rw = weight_on_input ? nullptr : topk_weights;
  if (bm == kGemvBlock && use_direct_slots(T, topk, KIND)) {
    const uint8_t* xd = static_cast<const uint8_t*>(x);
    float* xsd = nullptr;
    float* xcd = nullptr;
    // kFp8 / kW4: each W13 workgroup quantises its token's x row (vector-
    // loaded scales, whole workgroups of 16-row tiles); otherwise the
    // quantiser runs first.
    const bool qx = (KIND == kFp8 || KIND == kW4) && (H / 128) % kGemvU == 0 &&
                    reinterpret_cast<uintptr_t>(w13_s) % (KIND == kFp8 ? 16 : 8) == 0 &&
                    (2 * I) % (16 * kMoeGemvWaves) == 0 && H <= (KIND == kFp8 ? 32768 : 16384);
    if constexpr (KIND == kFp8) {
      if (!qx) {
        xsd = reinterpret_cast<float*>(ws + L.xs);
        rc = vmamd_per_token_group_quant_fp8(x, kBF16, T, H, H, 128, 1e-10f, -448.f, 448.f, ws + L.xq, xsd,
                                             H / 128, 1, st);
        xd = ws + L.xq;
      }
    } else if constexpr (KIND == kW4) {  // the alignment part of this launch sees no routes
      xsd = reinterpret_cast<float*>(ws + L.xs);
      if (!qx) {
        xcd = reinterpret_cast<float*>(ws + L.xcorr);
        rc = align_and_row_quant_fp8(topk_ids, 0, E, bm, expert_map, expert_map_len, sorted, cap, eids,
                                     ntpp, offs, active, nact, x, T, H, ws + L.xq, xsd, xcd, st);
        xd = ws + L.xq;
      }
    }
    if (rc) return rc;
    return fused_direct<KIND>(qx, xd, xsd, xcd, t, h, static_cast<const uint8_t*>(w13), w13_s,
                              static_cast<const uint8_t*>(w2), w2_s, E, i, topk, topk_weights, topk_ids,
                              expert_map, expert_map_len, swiglu_limit, w13_rw, w2_rw, scratch, a2, a2s,
                              KIND == kW4 ? reinterpret_cast<float*>(ws + L.a2corr) : nullptr,
                              static_cast<uint16_t*>(out), st, native);
  }
  const uint8_t* xa = static_cast<const uint8_t*>(x);
  const float* xs = nullptr;
  float* xcorr = KIND == kW4 ? reinterpret_cast<float*>(ws + L.xcorr) : nullptr;
  uint32_t* wst13 = nullptr;  // kW4 grouped GEMMs: the transposed weight scales
  uint32_t* wst2 = nullptr;
  float* xsr = nullptr;  // kFp8 grouped W13: x scales in route order
  float* a2corr = KIND == kW4 ? reinterpret_cast<float*>(ws + L.a2corr) : nullptr;
  if constexpr (KIND == kFp8) {  // quantiser and alignment in one launch
    uint8_t* xq = ws + L.xq;
    float* xsw = reinterpret_cast<float*>(ws + L.xs);
    rc = align_and_group_quant_fp8(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap,
                                   eids, ntpp, offs, active, nact, x, T, H, xq, xsw, st);
    if (rc) return rc;
    xa = xq;
    xs = xsw;
    // 128-route blocks: the copy from 32 routes per expert (fewer: the blocks
    // are mostly padding and the launch costs what the loads save).
    if (route_scales_bytes(cap, H, bm, KIND) > 0 && (bm != kMoeBM || numel >= 32ll * E)) {
      xsr = reinterpret_cast<float*>(ws + L.xsr);
      route_scales_kernel<<<static_cast<int>((cap + 255) / 256), 256, 0, st>>>(xsw, sorted, ntpp, numel, topk,
                                                                             static_cast<int>(H / 128), bm, xsr);
      rc = check_launch("fused_moe (x scales in route order)");
      if (rc) return rc;
    }
  } else if constexpr (KIND == kW4) {  // per-row quantiser and alignment in one launch, with the
                                       // grouped GEMMs' transposed weight scales
    uint8_t* xq = ws + L.xq;
    float* xsw = reinterpret_cast<float*>(ws + L.xs);
    W4ScalesT sct{};
    sct.E = E;
    if (L.sct13) {
      wst13 = reinterpret_cast<uint32_t*>(ws + L.wst13);
      sct.in[0] = static_cast<const uint32_t*>(w13_s);
      sct.out[0] = wst13;
      sct.n[0] = 2 * i;
      sct.kp[0] = h / 256;
    }
    if (L.sct2) {
      wst2 = reinterpret_cast<uint32_t*>(ws + L.wst2);
      sct.in[1] = static_cast<const uint32_t*>(w2_s);
      sct.out[1] = wst2;
      sct.n[1] = h;
      sct.kp[1] = i / 256;
    }
    rc = align_and_row_quant_fp8(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap,
                                 eids, ntpp, offs, active, nact, x, T, H, xq, xsw, xcorr, st, &sct);
    if (rc) return rc;
    xa = xq;
    xs = xsw;
  } else {
    rc = align_routes(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap, eids, ntpp, offs, active,
                      nact, reinterpret_cast<int32_t*>(ws + L.acnt), st);
    if (rc) return rc;
  }
  // kW4 prefill: bf16 activation, quantised per row below (the decode path
  // writes the quantised a2 directly).
  uint8_t* act_out = KIND == kW4 && bm != kGemvBlock ? ws + L.abf : a2;
  // kFp8 grouped GEMMs: W13 writes the a2 scales in route order and W2 reads
  // them so (the a2 scales stay inside this call).
  const bool a2s_routes = KIND == kFp8 && (bm == kMoeBigBM || bm == kMoeBM);
  rc = launch_w13<KIND>(xa, xs, xcorr, t, h, topk, sorted, cap, bm, offs, ntpp, active, nact,
                        static_cast<const uint8_t*>(w13), w13_s, E, i, swiglu_limit, w13_rw, act_out,
                        a2s, a2corr, scratch, st, eids, native, wst13, xsr, a2s_routes);
  if (rc) return rc;
  if constexpr (KIND == kW4) {
    if (bm != kGemvBlock) {  // rows past the last block are skipped on the device
      launch_rowquant_w4(reinterpret_cast<const uint16_t*>(act_out), i, cap, ntpp, a2, a2s, a2corr, st);
      rc = check_launch("w4afp8_moe (a2 quantiser)");
      if (rc) return rc;
    }
  }
  bool combined = false;
  rc = launch_w2<KIND>(a2, a2s, a2corr, t, topk, sorted, cap, bm, offs, ntpp, active, nact,
                       static_cast<const uint8_t*>(w2), w2_s, E, h, i, topk_weights, w2_rw, topk_ids,
                       expert_map, expert_map_len, y, scratch, st, static_cast<uint16_t*>(out),
                       &combined, eids, wst2, a2s_routes);
  if (rc || combined) return rc;
  // Slots of dropped routes (negative ids, or non-local experts) hold no
  // expert output and are skipped by the combine.
  return moe_sum_impl(KIND == kW4 ? "w4afp8_moe (combine)" : "fused_moe (combine)", y, kBF16, T, topk,
                      H, topk_ids, expert_map, expert_map_len, E,
                      KIND == kW4 ? topk_weights : nullptr, out, stream);
}

template <int KIND>
static int stage_w13(const char* who, const void* xa, const float* xs, int64_t T, int64_t H, int topk,
                     const int32_t* sorted, int64_t capacity, int block_m, const int32_t* offs,
                     const int32_t* ntpp, const int32_t* active, const int32_t* nact,
                     const void* w13, const void* w13_s, int E, int64_t I, float limit, void* a2,
                     float* a2s, void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common(who, KIND, T, topk, E, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(xa && sorted && offs && ntpp && w13 && a2 &&
                    (KIND == kBf16 || (xs && w13_s)) && (KIND != kFp8 || a2s),
                "%s: null pointer", who);
  VMAMD_REQUIRE(block_m != kGemvBlock || (active && nact),
                "%s: the decode path (block_m 16) needs active_experts / num_active", who);
  const size_t need = w13_scratch(T * topk, E, H, I, block_m, KIND);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(xa) % 16 == 0 && reinterpret_cast<uintptr_t>(a2) % 16 == 0,
                "%s: activations, a2 and workspace must be 16-byte aligned", who);
  // The fp8 grouped W13 reads its x scales in route order when the
  // workspace holds the copy for this capacity (route_scales_kernel).
  float* xsr = nullptr;
  const size_t rsb = route_scales_bytes(capacity, H, block_m, KIND);
  if (rsb > 0 && workspace_bytes >= rsb) {
    xsr = static_cast<float*>(workspace);
    route_scales_kernel<<<static_cast<int>((capacity + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
        xs, sorted, ntpp, static_cast<int>(T * topk), topk, static_cast<int>(H / 128), block_m, xsr);
    rc = check_launch("moe_fp8_w13 (x scales in route order)");
    if (rc) return rc;
  }
  return launch_w13<KIND>(static_cast<const uint8_t*>(xa), xs, nullptr, static_cast<int>(T), static_cast<int>(H),
                          topk, sorted, capacity, block_m, offs, ntpp, active, nact,
                          static_cast<const uint8_t*>(w13), w13_s, E, static_cast<int>(I), limit,
                          nullptr, static_cast<uint8_t*>(a2), a2s, nullptr, static_cast<float*>(workspace),
                          reinterpret_cast<hipStream_t>(stream), nullptr, false, nullptr, xsr);
}

template <int KIND>
static int stage_w2(const char* who, const void* a2, const float* a2s, int64_t T, int topk,
                    const int32_t* sorted, int64_t capacity, int block_m, const int32_t* offs,
                    const int32_t* ntpp, const int32_t* active, const int32_t* nact, const void* w2,
                    const void* w2_s, int E, int64_t H, int64_t I, const float* topk_weights,
                    const int32_t* topk_ids, const int32_t* emap, int64_t emap_len, void* y,
                    void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common(who, KIND, T, topk, E, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(a2 && sorted && offs && ntpp && w2 && topk_ids && y &&
                    (KIND == kBf16 || (a2s && w2_s)) && (KIND == kW4 || topk_weights),
                "%s: null pointer", who);
  VMAMD_REQUIRE(block_m != kGemvBlock || (active && nact),
                "%s: the decode path (block_m 16) needs active_experts / num_active", who);
  const size_t need = w2_scratch(T * topk, E, H, I, block_m, KIND);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a2) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(y) % (block_m >= kMoeBigBM ? 16 : 8) == 0,
                "%s: a2 and workspace must be 16-byte aligned, y 8-byte (16-byte for block_m %d)", who,
                kMoeBigBM);
  return launch_w2<KIND>(static_cast<const uint8_t*>(a2), a2s, nullptr, static_cast<int>(T), topk, sorted,
                         capacity, block_m, offs, ntpp, active, nact, static_cast<const uint8_t*>(w2),
                         w2_s, E, static_cast<int>(H), static_cast<int>(I), topk_weights,
                         KIND == kW4 ? nullptr : topk_weights, topk_ids,
                         emap, emap_len, static_cast<uint16_t*>(y), static_cast<float*>(workspace),
                         reinterpret_cast<hipStream_t>(stream));
}

// ------------------------------------------------ the reference GEMV ops --
// musa_fused_gemv_moe / musa_fused_gemv (csrc/musa/gemv.mu:723-1170) on the
// decode GEMV.  Route r = row * topk + k of A's rows uses expert topk_ids[r]
// and writes row r of C; without ids (the dense op) every row is a route of
// the one expert.  Up to kMaxCombineSlots routes each route is its own GEMV
// slot (the reference's own grid: one slot per route); more are grouped per
// expert by the alignment, so an expert's weights stream once per 16 routes.
// The GEMV writes fp32 split-K partials and one epilogue launch finishes:
// the reference activation (use_swiglu) or bf16(acc * w), dead routes zero.
struct GemvOpWs {
  size_t sorted, eids, ntpp, offs, active, nact, partial, total;
};

static bool gemv_op_direct(int64_t numel, bool dense) { return !dense && numel <= kMaxCombineSlots; }

// GEMV slots along gridDim.y: 1 (dense), the routes (direct), or the experts
// that can be active (grouped).
static int64_t gemv_op_slots(int64_t numel, int E, bool dense) {
  return dense ? 1 : gemv_op_direct(numel, dense) ? numel : moe_umax(numel, E);
}

static int gemv_op_kind(int a_dtype, int b_dtype) {
  if (b_dtype == VMAMD_DTYPE_E4M3) {
    if (a_dtype == kBF16) return kW8A16;
    if (a_dtype == VMAMD_DTYPE_E4M3) return kFp8;
  } else if (b_dtype == kBF16 && a_dtype == kBF16) {
    return kBf16;
  }
  return -1;
}

static int gemv_op_splits(int64_t numel, int E, int64_t N, int64_t K, int kind, bool dense) {
  return moe_splits(gemv_op_slots(numel, E, dense) * (N / 16), ksteps(K, kind));
}

static GemvOpWs gemv_op_layout(int64_t numel, int E, int64_t N, int64_t K, int kind, bool dense) {
  GemvOpWs w{};
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o += al256(bytes); return at; };
  if (!dense && !gemv_op_direct(numel, dense)) {
    const int64_t cap = numel + static_cast<int64_t>(E) * (kGemvBlock - 1);
    w.sorted = take(cap * 4);
    w.eids = take(((cap + kGemvBlock - 1) / kGemvBlock) * 4);
    w.ntpp = take(4);
    w.offs = take((E + 1) * 4);
    w.active = take(E * 4);
    w.nact = take(4);
  }
  w.partial = take(static_cast<size_t>(gemv_op_splits(numel, E, N, K, kind, dense)) * numel * N * 4);
  w.total = o;
  return w;
}

// Host round to nearest even bf16 (the reference rounds swiglu_limit to the
// activation dtype, gemv.mu:946-951).
static float round_bf16_host(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return f;
  u += 0x7fffu + ((u >> 16) & 1u);
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

template <int KIND>
static int gemv_op_launch(const void* A, const float* A_scale, int64_t rows, int64_t K, const void* B,
                          const float* B_scale, int E, int64_t N, const float* topk_weights,
                          const int32_t* topk_ids, int topk, bool mul_rw, bool swiglu, float limit, void* C,
                          uint8_t* ws, const GemvOpWs& L, hipStream_t st) {
  const bool dense = topk_ids == nullptr;
  const int numel = static_cast<int>(rows * topk);
  const int n = static_cast<int>(N), k = static_cast<int>(K);
  const int splits = gemv_op_splits(numel, E, N, K, KIND, dense);
  const int act_bytes = gemv_act_bytes<KIND>(rows, K);
  const bool vs = gemv_vector_scales<KIND>(K, A_scale, B_scale);
  const uint8_t* act = static_cast<const uint8_t*>(A);
  const uint8_t* w = static_cast<const uint8_t*>(B);
  float* partial = reinterpret_cast<float*>(ws + L.partial);
  const int32_t* none = nullptr;
  const dim3 grid((n / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, static_cast<unsigned>(gemv_op_slots(numel, E, dense)),
                  splits);
  if (dense) {
    launch_gemv<KIND, kGemvDense>(grid, st, numel <= 8, vs, act, act_bytes, A_scale, topk, k, none, none, none,
                                  none, w, static_cast<const void*>(B_scale), n, numel, splits, partial,
                                  static_cast<const float*>(nullptr), static_cast<uint16_t*>(nullptr));
  } else if (gemv_op_direct(numel, dense) && swiglu && direct_act(KIND, splits)) {
    if constexpr (KIND == kBf16 || KIND == kW8A16) {  // the W13 GEMV writes the activation (zeros if dropped)
      launch_gemv_direct<KIND, kGemvDirectAct>(
          dim3(n / 32, numel, 1), 2 * splits * kWave, 0, st, vs, act, act_bytes, A_scale, topk, k, none, none, none,
          none, w, static_cast<const void*>(B_scale), n, numel, splits, static_cast<float*>(nullptr),
          mul_rw ? topk_weights : static_cast<const float*>(nullptr), static_cast<uint16_t*>(C), topk_ids, none,
          int64_t{0}, E, static_cast<uint16_t*>(nullptr), static_cast<const float*>(nullptr),
          static_cast<float*>(nullptr), limit, 1);
    }
    return check_launch("fused_gemv (gemv + activation)");
  } else if (gemv_op_direct(numel, dense)) {
    launch_gemv_direct<KIND, kGemvDirect>(
        grid, kMoeGemvWaves * kWave, 0, st, vs, act, act_bytes, A_scale, topk, k, none, none, none, none, w,
        static_cast<const void*>(B_scale), n, numel, splits, partial, static_cast<const float*>(nullptr),
        static_cast<uint16_t*>(nullptr), topk_ids, none, int64_t{0}, E, static_cast<uint16_t*>(nullptr),
        static_cast<const float*>(nullptr), static_cast<float*>(nullptr), 0.f, 0);
  } else {
    int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
    int32_t* offs = reinterpret_cast<int32_t*>(ws + L.offs);
    int32_t* active = reinterpret_cast<int32_t*>(ws + L.active);
    int32_t* nact = reinterpret_cast<int32_t*>(ws + L.nact);
    const int64_t cap = numel + static_cast<int64_t>(E) * (kGemvBlock - 1);
    int rc = vmamd_moe_align_block_size(topk_ids, numel, E, kGemvBlock, nullptr, 0, sorted, cap,
                                        reinterpret_cast<int32_t*>(ws + L.eids),
                                        reinterpret_cast<int32_t*>(ws + L.ntpp), offs, nullptr, active, nact,
                                        reinterpret_cast<vmamd_stream_t>(st));
    if (rc) return rc;
    launch_gemv<KIND>(grid, st, gemv_one_block(numel, E), vs, act, act_bytes, A_scale, topk, k, sorted, offs,
                      active, nact, w, static_cast<const void*>(B_scale), n, numel, splits, partial,
                      static_cast<const float*>(nullptr), static_cast<uint16_t*>(nullptr));
  }
  int rc = check_launch("fused_gemv (gemv)");
  if (rc) return rc;
  const float* rw = mul_rw ? topk_weights : nullptr;
  if (swiglu)
    return launch_act_native(partial, splits, numel, n / 2, limit, rw, topk_ids, nullptr, 0, E,
                             static_cast<uint16_t*>(C), st);
  const int64_t mn = static_cast<int64_t>(numel) * n;
  moe_w2_reduce_kernel<true><<<static_cast<int>((mn / 4 + 255) / 256), 256, 0, st>>>(
      partial, splits, numel, n, topk_ids, nullptr, 0, E, rw, static_cast<uint16_t*>(C));
  return check_launch("fused_gemv (epilogue)");
}

static int gemv_op(const char* who, const void* A, int a_dtype, const float* A_scale, int64_t rows, int64_t K,
                   const void* B, int b_dtype, const float* B_scale, int E, int64_t N, const float* topk_weights,
                   const int32_t* topk_ids, int topk, bool mul_rw, bool swiglu, float limit, void* C,
                   void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  const int kind = gemv_op_kind(a_dtype, b_dtype);
  VMAMD_REQUIRE(kind >= 0, "%s: takes bf16 x e4m3 (W8A16), e4m3 x e4m3 (with A_scale) or bf16 x bf16 "
                "(A dtype %d, B dtype %d)", who, a_dtype, b_dtype);
  VMAMD_REQUIRE(rows >= 0 && topk > 0 && E > 0 && E <= 1024 && rows * topk < (1ll << 30),
                "%s: bad sizes (rows=%lld topk=%d experts=%d)", who, (long long)rows, topk, E);
  VMAMD_REQUIRE(N > 0 && N % (swiglu ? 32 : 16) == 0 && N < (1ll << 24),
                "%s: output size %lld must be a positive multiple of %d", who, (long long)N, swiglu ? 32 : 16);
  VMAMD_REQUIRE(K > 0 && K % (kind == kBf16 ? 64 : 128) == 0 && K < (1ll << 24),
                "%s: reduction size %lld must be a positive multiple of %d", who, (long long)K,
                kind == kBf16 ? 64 : 128);
  VMAMD_REQUIRE(rows * K * (a_dtype == kBF16 ? 2 : 1) < (1ll << 31) && N * K < (1ll << 31),
                "%s: operands past 2 GiB", who);
  VMAMD_REQUIRE(kind == kBf16 || B_scale, "%s: fp8 weights need their 128x128 block scales", who);
  VMAMD_REQUIRE(kind != kFp8 || A_scale, "%s: fp8 activations need their 1x128 group scales", who);
  VMAMD_REQUIRE(!mul_rw || topk_weights, "%s: mul_routed_weight needs topk_weights", who);
  if (rows == 0) return VMAMD_OK;
  VMAMD_REQUIRE(A && B && C, "%s: null pointer", who);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(C) % 16 == 0 && reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
                "%s: A, B and C must be 16-byte and the workspace 256-byte aligned", who);
  const GemvOpWs L = gemv_op_layout(rows * topk, E, N, K, kind, topk_ids == nullptr);
  VMAMD_REQUIRE(workspace && workspace_bytes >= L.total, "%s: workspace of %zu bytes required (got %zu)", who,
                L.total, workspace_bytes);
  if (a_dtype == kBF16 && limit > 0.f) limit = round_bf16_host(limit);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (kind) {
    case kW8A16:
      return gemv_op_launch<kW8A16>(A, A_scale, rows, K, B, B_scale, E, N, topk_weights, topk_ids, topk, mul_rw,
                                    swiglu, limit, C, ws, L, st);
    case kFp8:
      return gemv_op_launch<kFp8>(A, A_scale, rows, K, B, B_scale, E, N, topk_weights, topk_ids, topk, mul_rw,
                                  swiglu, limit, C, ws, L, st);
    default:
      return gemv_op_launch<kBf16>(A, nullptr, rows, K, B, nullptr, E, N, topk_weights, topk_ids, topk, mul_rw,
                                   swiglu, limit, C, ws, L, st);
  }
}

}  // namespace vmamd

using namespace vmamd;

// ------------------------------------------------------------------ fp8 ---
extern "C" size_t vmamd_moe_fp8_stage_workspace_size(int64_t T, int topk, int num_experts,
                                                     int64_t H, int64_t I, int block_m) {
  return stage_scratch(T * topk, num_experts, H, I, block_m, kFp8);
}

extern "C" int vmamd_moe_fp8_w13(const void* xq, const float* xs, int64_t T, int64_t H, int topk,
                                 const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                 const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                 const int32_t* active_experts, const int32_t* num_active,
                                 const void* w13, const float* w13_s, int num_experts, int64_t I,
                                 float swiglu_limit, void* a2q, float* a2s, void* workspace,
                                 size_t workspace_bytes, vmamd_stream_t stream) {
  return stage_w13<kFp8>("moe_fp8_w13", xq, xs, T, H, topk, sorted_token_ids, capacity, block_m,
                         expert_offsets, num_tokens_post_pad, active_experts, num_active, w13, w13_s,
                         num_experts, I, swiglu_limit, a2q, a2s, workspace, workspace_bytes, stream);
}

extern "C" int vmamd_moe_fp8_w2(const void* a2q, const float* a2s, int64_t T, int topk,
                                const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                const int32_t* active_experts, const int32_t* num_active,
                                const void* w2, const float* w2_s, int num_experts, int64_t H,
                                int64_t I, const float* topk_weights, const int32_t* topk_ids,
                                const int32_t* expert_map, int64_t expert_map_len, void* y,
                                void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  return stage_w2<kFp8>("moe_fp8_w2", a2q, a2s, T, topk, sorted_token_ids, capacity, block_m,
                        expert_offsets, num_tokens_post_pad, active_experts, num_active, w2, w2_s,
                        num_experts, H, I, topk_weights, topk_ids, expert_map, expert_map_len, y,
                        workspace, workspace_bytes, stream);
}

extern "C" size_t vmamd_fused_moe_fp8_workspace_size(int64_t T, int topk, int num_experts,
                                                     int64_t H, int64_t I, int path) {
  const int kind = path == VMAMD_MOE_PATH_NATIVE_GEMV ? kW8A16 : kFp8;
  return moe_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path, kind), kind).total;
}

extern "C" int vmamd_fused_moe_fp8(const void* x, int x_dtype, int64_t T, int64_t H,
                                   const void* w13, const float* w13_s, const void* w2,
                                   const float* w2_s, int num_experts, int64_t I,
                                   const float* topk_weights, const int32_t* topk_ids, int topk,
                                   const int32_t* expert_map, int64_t expert_map_len,
                                   float swiglu_limit, int apply_router_weight_on_input, int path,
                                   void* out, void* workspace, size_t workspace_bytes,
                                   vmamd_stream_t stream) {
  VMAMD_REQUIRE(x_dtype == kBF16, "fused_moe_fp8: hidden states must be bf16");
  if (path == VMAMD_MOE_PATH_NATIVE_GEMV)
    return fused_layer<kW8A16>("fused_moe_fp8 (native gemv)", x, T, H, w13, w13_s, w2, w2_s, num_experts, I,
                               topk_weights, topk_ids, topk, expert_map, expert_map_len, swiglu_limit,
                               apply_router_weight_on_input != 0, path, out, workspace, workspace_bytes,
                               stream);
  return fused_layer<kFp8>("fused_moe_fp8", x, T, H, w13, w13_s, w2, w2_s, num_experts, I,
                           topk_weights, topk_ids, topk, expert_map, expert_map_len, swiglu_limit,
                           apply_router_weight_on_input != 0, path, out, workspace,
                           workspace_bytes, stream);
}

// ----------------------------------------------------------------- bf16 ---
extern "C" size_t vmamd_moe_bf16_stage_workspace_size(int64_t T, int topk, int num_experts,
                                                      int64_t H, int64_t I, int block_m) {
  return stage_scratch(T * topk, num_experts, H, I, block_m, kBf16);
}

extern "C" int vmamd_moe_bf16_w13(const void* x, int64_t T, int64_t H, int topk,
                                  const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                  const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                  const int32_t* active_experts, const int32_t* num_active,
                                  const void* w13, int num_experts, int64_t I, float swiglu_limit,
                                  void* a2, void* workspace, size_t workspace_bytes,
                                  vmamd_stream_t stream) {
  return stage_w13<kBf16>("moe_bf16_w13", x, nullptr, T, H, topk, sorted_token_ids, capacity,
                          block_m, expert_offsets, num_tokens_post_pad, active_experts, num_active,
                          w13, nullptr, num_experts, I, swiglu_limit, a2, nullptr, workspace,
                          workspace_bytes, stream);
}

extern "C" int vmamd_moe_bf16_w2(const void* a2, int64_t T, int topk,
                                 const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                 const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                 const int32_t* active_experts, const int32_t* num_active,
                                 const void* w2, int num_experts, int64_t H, int64_t I,
                                 const float* topk_weights, const int32_t* topk_ids,
                                 const int32_t* expert_map, int64_t expert_map_len, void* y,
                                 void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  return stage_w2<kBf16>("moe_bf16_w2", a2, nullptr, T, topk, sorted_token_ids, capacity, block_m,
                         expert_offsets, num_tokens_post_pad, active_experts, num_active, w2, nullptr,
                         num_experts, H, I, topk_weights, topk_ids, expert_map, expert_map_len, y,
                         workspace, workspace_bytes, stream);
}

extern "C" size_t vmamd_fused_moe_bf16_workspace_size(int64_t T, int topk, int num_experts,
                                                      int64_t H, int64_t I, int path) {
  return moe_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path, kBf16), kBf16).total;
}

extern "C" int vmamd_fused_moe_bf16(const void* x, int64_t T, int64_t H, const void* w13,
                                    const void* w2, int num_experts, int64_t I,
                                    const float* topk_weights, const int32_t* topk_ids, int topk,
                                    const int32_t* expert_map, int64_t expert_map_len,
                                    float swiglu_limit, int apply_router_weight_on_input, int path,
                                    void* out, void* workspace, size_t workspace_bytes,
                                    vmamd_stream_t stream) {
  return fused_layer<kBf16>("fused_moe_bf16", x, T, H, w13, nullptr, w2, nullptr, num_experts, I,
                            topk_weights, topk_ids, topk, expert_map, expert_map_len, swiglu_limit,
                            apply_router_weight_on_input != 0, path, out, workspace,
                            workspace_bytes, stream);
}

// --------------------------------------------------------------- w4afp8 ---
extern "C" size_t vmamd_w4afp8_moe_workspace_size(int64_t T, int topk, int num_experts, int64_t H,
                                                  int64_t I, int path) {
  return moe_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path, kW4), kW4).total;
}

extern "C" int vmamd_w4afp8_moe(const void* x, int64_t T, int64_t H, const void* w13,
                                const void* w13_s, const void* w2, const void* w2_s,
                                int num_experts, int64_t I, const float* topk_weights,
                                const int32_t* topk_ids, int topk, const int32_t* expert_map,
                                int64_t expert_map_len, float swiglu_limit, int path, void* out,
                                void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  return fused_layer<kW4>("w4afp8_moe", x, T, H, w13, w13_s, w2, w2_s, num_experts, I, topk_weights,
                          topk_ids, topk, expert_map, expert_map_len, swiglu_limit, false, path,
                          out, workspace, workspace_bytes, stream);
}

// ------------------------------------------------- reference GEMV ops ---
extern "C" size_t vmamd_fused_gemv_moe_workspace_size(int64_t rows, int topk, int num_experts, int64_t N,
                                                      int64_t K, int a_dtype, int b_dtype) {
  const int kind = gemv_op_kind(a_dtype, b_dtype);
  if (kind < 0 || rows <= 0 || topk <= 0 || num_experts <= 0) return 0;
  return gemv_op_layout(rows * topk, num_experts, N, K, kind, false).total;
}

extern "C" int vmamd_fused_gemv_moe(const void* A, int a_dtype, const float* A_scale, int64_t rows, int64_t K,
                                    const void* B, int b_dtype, const float* B_scale, int num_experts,
                                    int64_t N, const float* topk_weights, const int32_t* topk_ids, int topk,
                                    int mul_routed_weight, int use_swiglu, float swiglu_limit, void* C,
                                    void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  VMAMD_REQUIRE(rows == 0 || topk_ids, "fused_gemv_moe: null topk_ids");
  return gemv_op("fused_gemv_moe", A, a_dtype, A_scale, rows, K, B, b_dtype, B_scale, num_experts, N,
                 topk_weights, topk_ids, topk, mul_routed_weight != 0, use_swiglu != 0, swiglu_limit, C,
                 workspace, workspace_bytes, stream);
}

extern "C" size_t vmamd_fused_gemv_workspace_size(int64_t M, int64_t N, int64_t K, int a_dtype, int b_dtype) {
  const int kind = gemv_op_kind(a_dtype, b_dtype);
  if (kind < 0 || M <= 0) return 0;
  return gemv_op_layout(M, 1, N, K, kind, true).total;
}

extern "C" int vmamd_fused_gemv(const void* A, int a_dtype, const float* A_scale, int64_t M, int64_t K,
                                const void* B, int b_dtype, const float* B_scale, int64_t N, int use_swiglu,
                                void* C, void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  return gemv_op("fused_gemv", A, a_dtype, A_scale, M, K, B, b_dtype, B_scale, 1, N, nullptr, nullptr, 1,
                 false, use_swiglu != 0, 0.f, C, workspace, workspace_bytes, stream);
}
