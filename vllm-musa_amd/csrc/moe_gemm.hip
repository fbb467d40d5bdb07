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
//   w13 rows [0, I) gate, [I, 2I) up; routes r = t * topk + k; sorted /
//   offsets / active come from moe_align_block_size.
//
// Every kind moves K in "steps": 128 K-elements for kFp8 / kW4 (one 16x16x128
// fp8 MFMA; kW4 nibbles are converted to e4m3 codes on the way in, every
// integer in [-8, 7] being exact in e4m3), 64 for kBf16 (two 16x16x32 bf16
// MFMAs).  Per step kFp8 promotes acc += p * sa[m] * sb[n/128], kW4 promotes
// acc += p * sw[n] with the row's own weight scale and applies the activation
// row scale once at the end, kBf16 accumulates directly.
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
#include <type_traits>

#include "quant_dev.h"
#include "mfma_fp8.h"
#include "tile_pipe.h"

namespace vmamd {

constexpr int kFp8 = 0, kBf16 = 1, kW4 = 2;

// Bytes of one K step: activation row, weight row.
template <int KIND> struct KindBytes {
  static constexpr int kAct = 128;
  static constexpr int kW = KIND == kW4 ? 64 : 128;
  static constexpr int kElems = KIND == kBf16 ? 64 : 128;  // K elements per step
};

// --------------------------------------------------------------- helpers --
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

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
  if constexpr (KIND == kW4) return global_frag_int4(p, g);
  else return global_frag(p, g);
}

// ---------------------------------------------------------- decode GEMV ---
constexpr int kMoeGemvWaves = 4;
constexpr int kGemvBlock = 16;  // routes per block (one MFMA column tile)
// K steps each wave keeps in flight (8 KiB of weights per wave; 4 and 8
// measured alike, 4 needs fewer registers), and the number of waves the
// split-K factor aims to launch (16 per CU).
constexpr int kGemvU = 4;
constexpr int kGemvTargetWaves = 4096;

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
// Activation fragment at byte offset off (row + K-block start) of a buffer.
__device__ __forceinline__ v8i buffer_frag(__amdgpu_buffer_rsrc_t rs, uint32_t off, int g) {
  const v4i lo = buffer_ld16(rs, off + 16u * g);
  const v4i hi = buffer_ld16(rs, off + 64u + 16u * g);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// act: [rows, K] activation bytes (rows = numel / act_div), act_bytes its
// size (< 2^31); act_s: kFp8 [rows, K/128] group scales; kW4 / kBf16 unused.
// ws: kFp8 f32 block scales; kW4 bf16 row scales.
//
// Start-up order: the expert id is the only load the weight stream depends
// on, so the first K group of weights is requested before the route list is
// resolved (offsets -> the block's route ids -> activation rows); every wave
// starts at once, so a serial chain of lookups in front of the stream would
// leave HBM idle.  The route ids are read with uniform (scalar) loads, which
// are counted apart from the vector loads, so waiting for them does not wait
// for the weights.  Columns of padding routes fetch no activation bytes.
// Four waves per SIMD hold the whole T = 1 grid of a DeepSeek-V3-sized layer
// at once; the int4 variant fits three and the 4-block variant two.
//
// VS (K/128 a multiple of U and aligned scale rows): kFp8 reads the U block
// scales of a group, and each route's U activation scales, with one 16-byte
// load each instead of U scattered ones; kW4 reads each of the lane's four
// rows' U bf16 scales with one 8-byte load instead of U 2-byte ones.  Splits
// start on group boundaries, so with VS every group lies entirely inside its
// split.
template <int MAXB, int KIND, bool VS = false>
__global__ __launch_bounds__(kMoeGemvWaves * kWave, MAXB == 1 ? (KIND == kW4 ? 3 : 4) : 2) void
moe_gemv_kernel(
    const uint8_t* __restrict__ act, int act_bytes, const float* __restrict__ act_s, int act_div,
    int K, const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ active, const int32_t* __restrict__ num_active,
    const uint8_t* __restrict__ w, const void* __restrict__ ws, int N, int numel, int splits,
    float* __restrict__ partial, const float* __restrict__ route_w, uint16_t* __restrict__ y) {
  using KB_ = KindBytes<KIND>;
  constexpr int U = kGemvU;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const int li = lane % 16, lg = lane / 16;
  const int ntile = blockIdx.x * kMoeGemvWaves + wave;
  if (ntile * 16 >= N) return;  // wave-uniform, no barriers in this kernel
  const int slot = blockIdx.y;
  // The exit test reads both values, so both loads are in flight together;
  // active[] has one entry per expert and gridDim.y never exceeds the expert
  // count, so the read is in bounds.
  const int e = active[slot];
  const int na = num_active[0];
  if (slot >= na || e < 0) return;
  const int split = blockIdx.z;
  const int KS = K / KB_::kElems;                    // K steps
  const int arowb = KS * KB_::kAct;
  const int64_t wrowb = static_cast<int64_t>(KS) * KB_::kW;
  const int NB = (N + 127) / 128;
  const int groups = (KS + kGemvU - 1) / kGemvU;  // splits start on group boundaries
  const int kb0 = split * groups / splits * kGemvU;
  const int kb1 = min((split + 1) * groups / splits * kGemvU, KS);
  const int n = ntile * 16 + 4 * lg;
  const uint8_t* wrow = w + (static_cast<int64_t>(e) * N + ntile * 16 + li) * wrowb;
  const float* wsr = nullptr;                        // kFp8: block scales of the 16 rows
  const uint16_t* wsw[4] = {nullptr, nullptr, nullptr, nullptr};  // kW4: scales of rows n..n+3
  if constexpr (KIND == kFp8)
    wsr = static_cast<const float*>(ws) + (static_cast<int64_t>(e) * NB + (ntile * 16) / 128) * KS;
  if constexpr (KIND == kW4) {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      wsw[r] = static_cast<const uint16_t*>(ws) + (static_cast<int64_t>(e) * N + n + r) * KS;
  }
  // kFp8 block scales of the wave's rows through a descriptor: uniform values
  // read by vector loads, which queue behind the weight loads instead of
  // making the weight stream wait for scalar loads.
  const __amdgpu_buffer_rsrc_t wsrs = buffer_rsrc(wsr, KIND == kFp8 ? KS * 4 : 0);
  const __amdgpu_buffer_rsrc_t ars = buffer_rsrc(act, act_bytes);
  const __amdgpu_buffer_rsrc_t srs = buffer_rsrc(act_s, KIND == kFp8 ? act_bytes / 32 : 0);
  const v4f zero = {0.f, 0.f, 0.f, 0.f};

  // One K group of weights (U steps from kb, clamped to the split's range).
  // kW4 with one route block keeps the weights packed (half the registers:
  // more waves, more bytes in flight) and converts each fragment right before
  // its MFMA; with several blocks a fragment is converted once per group.
  constexpr bool kRawW4 = KIND == kW4 && MAXB == 1;
  v8i wf[kRawW4 ? 1 : U];
  uint4 wraw[kRawW4 ? U : 1];
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
        wraw[u] = global_frag_int4_raw(wrow + static_cast<int64_t>(k) * KB_::kW, lg);
      else
        wf[u] = weight_frag<KIND>(wrow + static_cast<int64_t>(k) * KB_::kW, lg);
      if constexpr (!VS) sb[u] = 0.f;
      sw[u] = zero;
      if constexpr (KIND == kFp8 && !VS)
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
  // Activation loads and MFMAs of the group at kb with the weights in wf.
  // Steps past the split's end take masked (zero) activations, so the group
  // has no branches: their products are exactly zero.
  auto group = [&](int kb, int nb) {
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      if (b < nb) {
        v8i xf[U];
        float as[U];
        if constexpr (VS) {  // scale byte offset = activation byte offset / 32
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
          xf[u] = buffer_frag(ars, off, lg);
          if constexpr (!VS) as[u] = 0.f;
          if constexpr (KIND == kFp8 && !VS)  // scale byte offset = activation byte offset / 32
            as[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  srs, static_cast<int>(live ? off / 32 : kBufferOff), 0, 0));
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if constexpr (KIND == kFp8) {
            fma4(acc[b], mfma_fp8(wf[u], xf[u], zero), as[u] * sb[u]);
          } else if constexpr (KIND == kW4) {
            if constexpr (kRawW4)
              fma4v(acc[b], mfma_fp8(int4_frag_to_fp8(wraw[u]), xf[u], zero), w4_scales(u));
            else
              fma4v(acc[b], mfma_fp8(wf[u], xf[u], zero), w4_scales(u));
          } else {
            acc[b] = mfma_bf16x2(wf[u], xf[u], acc[b]);
          }
        }
      }
    }
  };

  const int seg0 = offsets[e];
  const int nblk = (offsets[e + 1] - seg0) / kGemvBlock;  // >= 1 for an active expert
  int b0 = 0;
  do {
    load_w(kb0);  // first group: in flight while the routes are resolved
    const int nb = min(MAXB, nblk - b0);
    int rr[MAXB];
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      int r = numel;
      if (b < nb) {
        const int32_t* ids = sorted + seg0 + (b0 + b) * kGemvBlock;
        int sid[kGemvBlock];
#pragma unroll
        for (int j = 0; j < kGemvBlock; ++j) sid[j] = ids[j];
        r = sid[0];
#pragma unroll
        for (int j = 1; j < kGemvBlock; ++j) r = li == j ? sid[j] : r;
      }
      const bool valid = r >= 0 && r < numel;
      rr[b] = valid ? r : -1;
      aoff[b] = valid ? static_cast<uint32_t>((r / act_div) * arowb) : kBufferOff;
      acc[b] = zero;
    }
    group(kb0, nb);
    for (int kb = kb0 + U; kb < kb1; kb += U) {
      load_w(kb);
      group(kb, nb);
    }
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      if (b >= nb || rr[b] < 0) continue;
      const int r = rr[b];
      const v4f a = acc[b];
      if (y) {
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
  float q[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = v[j] != v[j] ? -448.0f : fminf(fmaxf(v[j] / scale, -448.0f), 448.0f);
  uint2 out;
  out.x = f32x4_to_fp8x4(q[0], q[1], q[2], q[3]);
  out.y = f32x4_to_fp8x4(q[4], q[5], q[6], q[7]);
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

// kW4 decode: moe_act_bf16_kernel<kW4> and the per-row a2 quantiser in one
// pass, one kRowThreads block per route row: the bf16-rounded activations stay
// in registers for the row maximum and the quantiser (the values the separate
// quantiser would read back), so neither the bf16 activation nor a second
// launch is needed.  I <= kRowThreads * 8 * kRowChunks.
__global__ __launch_bounds__(kRowThreads) void moe_act_rowquant_w4_kernel(
    const float* __restrict__ partial, int splits, int numel, int I, float limit,
    const float* __restrict__ xs, int topk, uint8_t* __restrict__ a2q, float* __restrict__ a2s) {
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
      *reinterpret_cast<uint2*>(a2q + static_cast<int64_t>(r) * I + ch * 8) =
          quant8(v[c], s, -448.0f, 448.0f);
  }
}

// A route's slot is live when its expert id is >= 0 and its local id
// (through expert_map when given) lies in [0, E): the rule of the alignment,
// which places no other route, so no other partial row is ever written.
__device__ __forceinline__ bool route_live(const int32_t* __restrict__ emap, int64_t emap_len, int E,
                                           int e) {
  if (e < 0) return false;
  if (emap) {
    if (e >= emap_len) return false;
    e = emap[e];
  }
  return e >= 0 && e < E;
}

// y[r, n] = bf16(sum_s partial[s, r, n] * w_r) for the W2 split path (kW4:
// w_r is the a2 row scale).
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
  if (!route_live(emap, emap_len, E, ids[r])) return;
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
// workgroups past the used tiles.
__device__ __forceinline__ bool moe_tile(int wg, int max_tiles, const int32_t* __restrict__ offsets,
                                         const int32_t* __restrict__ ntpp, int E, int TN,
                                         int& e_out, int& mb_out, int& tn_out) {
  const int used = min(ntpp[0] / kMoeBM * TN, max_tiles);
  const int per = (used + kXcds - 1) / kXcds;
  const int q = wg / kXcds;
  if (q >= per) return false;
  const int L = (wg % kXcds) * per + q;
  if (L >= used) return false;
  // largest e with offsets[e] / BM * TN <= L (empty experts collapse onto the next)
  int lo = 0, hi = E - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (offsets[mid] / kMoeBM * TN <= L) lo = mid; else hi = mid - 1;
  }
  const int b0 = offsets[lo] / kMoeBM;
  const int nb = offsets[lo + 1] / kMoeBM - b0;
  const int local = L - b0 * TN;
  e_out = lo;
  tn_out = local / nb;
  mb_out = b0 + local % nb;
  return true;
}

// Weight-tile loader of the prefill GEMMs.  One pass moves THREADS/CPR rows;
// kFp8 / kBf16 copy 16-byte chunks (CPR = 8 per 128-byte row step), kW4 reads
// 16 packed bytes (32 elements) per thread (CPR = 4) and writes the two
// 16-byte e4m3 chunks they expand to.
template <int KIND, int THREADS, int BN>
struct WLoader {
  static constexpr int CPR = KIND == kW4 ? 4 : 8;
  static constexpr int RSTEP = THREADS / CPR;
  static constexpr int BCH = BN / RSTEP;
  using Raw = typename std::conditional<KIND == kW4, uint4, v4i>::type;
  int64_t goff[BCH];
  int l0, l1;  // LDS byte offsets (row 0 of the pass) of the chunks written
  Raw raw[BCH];

  __device__ __forceinline__ void load(const uint8_t* __restrict__ w, int step) {
#pragma unroll
    for (int c = 0; c < BCH; ++c) {
      const uint8_t* p = w + goff[c] + static_cast<int64_t>(step) * KindBytes<KIND>::kW;
      if constexpr (KIND == kW4) raw[c] = *reinterpret_cast<const uint4*>(p);
      else raw[c] = ld16(p);
    }
  }
  __device__ __forceinline__ void store(uint8_t* tile) const {
#pragma unroll
    for (int c = 0; c < BCH; ++c) {
      if constexpr (KIND == kW4) {
        st16(tile + l0 + c * RSTEP * 128, int4x16_to_fp8(uint2{raw[c].x, raw[c].y}));
        st16(tile + l1 + c * RSTEP * 128, int4x16_to_fp8(uint2{raw[c].z, raw[c].w}));
      } else {
        st16(tile + l0 + c * RSTEP * 128, raw[c]);
      }
    }
  }
};

// W13: tile = 128 routes x (128 gate + 128 up rows); 8 waves as 2 (m) x 4 (n);
// local weight row j: pair p = j / 32, q = j % 32 -> gate row n0 + 16p + q
// (q < 16) or up row I + n0 + 16p + q - 16.  Dynamic LDS per stage: the two
// tiles, plus (kW4) the fp32 scales of the 256 weight rows.
constexpr int kW13Threads = 512;
constexpr int kW13BN = 256;
template <int KIND>
constexpr int w13_stage_bytes() { return (kMoeBM + kW13BN) * 128 + (KIND == kW4 ? kW13BN * 4 : 0); }

// xs: kFp8 [T, H/128] group scales, kW4 [T] row scales.  w13s: kFp8 f32
// block scales, kW4 bf16 row scales.  a2: kFp8 e4m3 [rows, I] (+ a2s), kBf16 /
// kW4 bf16 [rows, I].
template <int KIND>
__global__ __launch_bounds__(kW13Threads, 1) void moe_w13_gemm_kernel(
    const uint8_t* __restrict__ xa, const float* __restrict__ xs, int topk, int H,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w13, const void* __restrict__ w13s, int I, float limit,
    uint8_t* __restrict__ a2, float* __restrict__ a2s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  using KB_ = KindBytes<KIND>;
  constexpr int BM = kMoeBM, BN = kW13BN, THREADS = kW13Threads;
  constexpr int WN = 4, WTM = 64, WTN = 64, MT = 4, NT = 4;
  constexpr int RSTEP = THREADS / 8;   // activation rows per copy pass
  constexpr int ACH = BM / RSTEP;      // 2
  constexpr int STAGE = w13_stage_bytes<KIND>();

  const int TN = I / 128;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, E, TN, e, mb, tn)) return;
  const int n0 = tn * 128;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane % 16, lg = lane / 16;
  const int KS = H / KB_::kElems;
  const int64_t arowb = static_cast<int64_t>(KS) * KB_::kAct;
  const int64_t wrowb = static_cast<int64_t>(KS) * KB_::kW;
  const int NB2 = (2 * I + 127) / 128;

  const int crow = tid / 8, cch = tid % 8;
  const int la0 = lds_off(crow, cch);
  // Padding rows of the block load row 0 and are zeroed in registers.
  int64_t goff_a[ACH];
  bool aval[ACH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const int r = sorted[mb * BM + crow + c * RSTEP];
    aval[c] = r < numel;
    goff_a[c] = (aval[c] ? static_cast<int64_t>(r / topk) * arowb : 0) + cch * 16;
  }
  auto w13_row = [&](int j) {  // local weight row -> row of w13[e]
    const int p = j / 32, q = j % 32;
    return q < 16 ? n0 + 16 * p + q : I + n0 + 16 * p + (q - 16);
  };
  WLoader<KIND, THREADS, BN> wl;
  {
    using WL = WLoader<KIND, THREADS, BN>;
    const int wr = tid / WL::CPR, wc = tid % WL::CPR;
#pragma unroll
    for (int c = 0; c < WL::BCH; ++c)
      wl.goff[c] = (static_cast<int64_t>(e) * 2 * I + w13_row(wr + c * WL::RSTEP)) * wrowb + wc * 16;
    wl.l0 = BM * 128 + lds_off(wr, KIND == kW4 ? 2 * wc : wc);
    wl.l1 = BM * 128 + lds_off(wr, 2 * wc + 1);
  }
  // kW4: thread j < BN stages the scale of local weight row j.
  const uint16_t* wsc_row = nullptr;
  if constexpr (KIND == kW4)
    wsc_row = tid < BN ? static_cast<const uint16_t*>(w13s) +
                             (static_cast<int64_t>(e) * 2 * I + w13_row(tid)) * KS
                       : nullptr;
  const float* xs_row[MT];
  bool tval[MT];
  float srow[MT];  // kW4: activation row scales
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = sorted[mb * BM + wm * WTM + mt * 16 + li];
    tval[mt] = r < numel;
    const int64_t tok = tval[mt] ? r / topk : 0;
    xs_row[mt] = KIND == kFp8 ? xs + tok * KS : nullptr;
    srow[mt] = KIND == kW4 ? (tval[mt] ? xs[tok] : 0.f) : 0.f;
  }
  const float* sg = nullptr;
  const float* su = nullptr;
  if constexpr (KIND == kFp8) {
    sg = static_cast<const float*>(w13s) + (static_cast<int64_t>(e) * NB2 + n0 / 128) * KS;
    su = static_cast<const float*>(w13s) + (static_cast<int64_t>(e) * NB2 + (I + n0) / 128) * KS;
  }

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  const v4i z4 = {0, 0, 0, 0};
  v4i ra[ACH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const v4i v = ld16(xa + goff_a[c]);
    ra[c] = aval[c] ? v : z4;
  }
  wl.load(w13, 0);
  float wsc = 0.f;
  if constexpr (KIND == kW4)
    if (wsc_row) wsc = bf16_to_f32(wsc_row[0]);
#pragma unroll
  for (int c = 0; c < ACH; ++c) st16(&smem_dyn[la0 + c * RSTEP * 128], ra[c]);
  wl.store(smem_dyn);
  if constexpr (KIND == kW4)
    if (wsc_row) reinterpret_cast<float*>(smem_dyn + (BM + BN) * 128)[tid] = wsc;
  float sa[MT], sbg = 0.f, sbu = 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = 0.f;
  if constexpr (KIND == kFp8) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = tval[mt] ? xs_row[mt][0] : 0.f;
    sbg = sg[0];
    sbu = su[0];
  }
  __syncthreads();

  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < KS; ++kb) {
    const int cur = kb & 1;
    // Prefetch step kb+1 (the last iteration re-reads step KS-1 into the idle
    // buffer; that copy is never used).
    const int kn = min(kb + 1, KS - 1);
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const v4i v = ld16(xa + goff_a[c] + static_cast<int64_t>(kn) * KB_::kAct);
      ra[c] = aval[c] ? v : z4;
    }
    wl.load(w13, kn);
    float san[MT], sbgn = 0.f, sbun = 0.f, wscn = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) san[mt] = 0.f;
    if constexpr (KIND == kFp8) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float v = xs_row[mt][kn];
        san[mt] = tval[mt] ? v : 0.f;
      }
      sbgn = sg[kn];
      sbun = su[kn];
    }
    if constexpr (KIND == kW4)
      if (wsc_row) wscn = bf16_to_f32(wsc_row[kn]);

    const uint8_t* tile = smem_dyn + cur * STAGE;
    v8i xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt] = lds_frag(tile, wm * WTM + mt * 16 + li, lg);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int wrow_l = wn * WTN + nt * 16;
      const v8i wf = lds_frag(tile + BM * 128, wrow_l + li, lg);
      if constexpr (KIND == kFp8) {
        const float sb = (nt & 1) ? sbu : sbg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) fma4(acc[mt][nt], mfma_fp8(wf, xf[mt], zero), sa[mt] * sb);
      } else if constexpr (KIND == kW4) {
        const v4f swv = *reinterpret_cast<const v4f*>(tile + (BM + BN) * 128 + (wrow_l + 4 * lg) * 4);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) fma4v(acc[mt][nt], mfma_fp8(wf, xf[mt], zero), swv);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma_bf16x2(wf, xf[mt], acc[mt][nt]);
      }
    }
    uint8_t* nxt = smem_dyn + (cur ^ 1) * STAGE;
#pragma unroll
    for (int c = 0; c < ACH; ++c) st16(&nxt[la0 + c * RSTEP * 128], ra[c]);
    wl.store(nxt);
    if constexpr (KIND == kW4)
      if (wsc_row) reinterpret_cast<float*>(nxt + (BM + BN) * 128)[tid] = wscn;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = san[mt];
    sbg = sbgn;
    sbu = sbun;
    __syncthreads();
  }

  if constexpr (KIND == kFp8) {
    // Epilogue: activation, row amax across the 4 n-waves through LDS, quantise.
    float* red = reinterpret_cast<float*>(smem_dyn);  // [WN][BM]
    float v[MT][2][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float amax = 0.f;
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = swiglu_bf16(bf16r(acc[mt][2 * q][r]), bf16r(acc[mt][2 * q + 1][r]), limit);
          v[mt][q][r] = x;
          amax = fmaxf(amax, fabsf(x));
        }
      amax = fmaxf(amax, __shfl_xor(amax, 16, kWave));
      amax = fmaxf(amax, __shfl_xor(amax, 32, kWave));
      if (lg == 0) red[wn * BM + wm * WTM + mt * 16 + li] = amax;
    }
    __syncthreads();
    const int gpr = I / 128;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int ml = wm * WTM + mt * 16 + li;
      float amax = 1e-10f;
#pragma unroll
      for (int w = 0; w < WN; ++w) amax = fmaxf(amax, red[w * BM + ml]);
      const float scale = amax / 448.0f;
      const int64_t row = static_cast<int64_t>(mb) * BM + ml;
      if (wn == 0 && lg == 0) a2s[row * gpr + tn] = scale;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = v[mt][q][r];
          o[r] = x != x ? -448.0f : fminf(fmaxf(x / scale, -448.0f), 448.0f);
        }
        const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
        *reinterpret_cast<uint32_t*>(a2 + row * I + col) = f32x4_to_fp8x4(o[0], o[1], o[2], o[3]);
      }
    }
  } else {
    uint16_t* a2b = reinterpret_cast<uint16_t*>(a2);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int64_t row = static_cast<int64_t>(mb) * BM + wm * WTM + mt * 16 + li;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (KIND == kW4)
            o[r] = swiglu_w4(bf16r(acc[mt][2 * q][r] * srow[mt]),
                             bf16r(acc[mt][2 * q + 1][r] * srow[mt]), limit);
          else
            o[r] = swiglu_bf16(bf16r(acc[mt][2 * q][r]), bf16r(acc[mt][2 * q + 1][r]), limit);
        }
        const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
        *reinterpret_cast<uint2*>(a2b + row * I + col) = pack_bf16x4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// W2: tile = 128 routes x 128 hidden rows, 4 waves as 2 x 2, K = I.
// a2s: kFp8 [rows, I/128] group scales, kW4 [rows] row scales.
// y[r] = bf16(acc * route_w[r]) (kFp8 / kBf16) or bf16(acc * a2s[row]) (kW4).
template <int KIND>
__global__ __launch_bounds__(256, 2) void moe_w2_gemm_kernel(
    const uint8_t* __restrict__ a2, const float* __restrict__ a2s, int I,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w2, const void* __restrict__ w2s, int H,
    const float* __restrict__ route_w, uint16_t* __restrict__ y) {
  using KB_ = KindBytes<KIND>;
  constexpr int BM = kMoeBM, BN = 128, THREADS = 256, WN = 2, WTM = 64, WTN = 64, MT = 4, NT = 4;
  constexpr int RSTEP = THREADS / 8, ACH = BM / RSTEP;
  constexpr int STAGE = (BM + BN) * 128 + (KIND == kW4 ? BN * 4 : 0);
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][STAGE];

  const int TN = (H + BN - 1) / BN;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, E, TN, e, mb, tn)) return;
  const int n0 = tn * BN;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane % 16, lg = lane / 16;
  const int KS = I / KB_::kElems;
  const int64_t arowb = static_cast<int64_t>(KS) * KB_::kAct;
  const int64_t wrowb = static_cast<int64_t>(KS) * KB_::kW;
  const int NBH = (H + 127) / 128;

  const int crow = tid / 8, cch = tid % 8;
  const int la0 = lds_off(crow, cch);
  int64_t goff_a[ACH];
#pragma unroll
  for (int c = 0; c < ACH; ++c)
    goff_a[c] = (static_cast<int64_t>(mb) * BM + crow + c * RSTEP) * arowb + cch * 16;
  WLoader<KIND, THREADS, BN> wl;
  {
    using WL = WLoader<KIND, THREADS, BN>;
    const int wr = tid / WL::CPR, wc = tid % WL::CPR;
#pragma unroll
    for (int c = 0; c < WL::BCH; ++c)
      wl.goff[c] = (static_cast<int64_t>(e) * H + min(n0 + wr + c * WL::RSTEP, H - 1)) * wrowb + wc * 16;
    wl.l0 = BM * 128 + lds_off(wr, KIND == kW4 ? 2 * wc : wc);
    wl.l1 = BM * 128 + lds_off(wr, 2 * wc + 1);
  }
  const uint16_t* wsc_row = nullptr;
  if constexpr (KIND == kW4)
    wsc_row = tid < BN ? static_cast<const uint16_t*>(w2s) +
                             (static_cast<int64_t>(e) * H + min(n0 + tid, H - 1)) * KS
                       : nullptr;
  const float* sb_p = nullptr;
  if constexpr (KIND == kFp8)
    sb_p = static_cast<const float*>(w2s) + (static_cast<int64_t>(e) * NBH + n0 / 128) * KS;
  const int64_t arow0 = static_cast<int64_t>(mb) * BM + wm * WTM + li;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  v4i ra[ACH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) ra[c] = ld16(a2 + goff_a[c]);
  wl.load(w2, 0);
  float wsc = 0.f;
  if constexpr (KIND == kW4)
    if (wsc_row) wsc = bf16_to_f32(wsc_row[0]);
#pragma unroll
  for (int c = 0; c < ACH; ++c) st16(&smem[0][la0 + c * RSTEP * 128], ra[c]);
  wl.store(smem[0]);
  if constexpr (KIND == kW4)
    if (wsc_row) reinterpret_cast<float*>(smem[0] + (BM + BN) * 128)[tid] = wsc;
  float sa[MT], sb = 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = 0.f;
  if constexpr (KIND == kFp8) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = a2s[(arow0 + mt * 16) * KS];
    sb = sb_p[0];
  }
  __syncthreads();

  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < KS; ++kb) {
    const int cur = kb & 1;
    const int kn = min(kb + 1, KS - 1);
#pragma unroll
    for (int c = 0; c < ACH; ++c) ra[c] = ld16(a2 + goff_a[c] + static_cast<int64_t>(kn) * KB_::kAct);
    wl.load(w2, kn);
    float san[MT], sbn = 0.f, wscn = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) san[mt] = 0.f;
    if constexpr (KIND == kFp8) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) san[mt] = a2s[(arow0 + mt * 16) * KS + kn];
      sbn = sb_p[kn];
    }
    if constexpr (KIND == kW4)
      if (wsc_row) wscn = bf16_to_f32(wsc_row[kn]);
    const uint8_t* tile = smem[cur];
    v8i xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt] = lds_frag(tile, wm * WTM + mt * 16 + li, lg);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int wrow_l = wn * WTN + nt * 16;
      const v8i wf = lds_frag(tile + BM * 128, wrow_l + li, lg);
      if constexpr (KIND == kFp8) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) fma4(acc[mt][nt], mfma_fp8(wf, xf[mt], zero), sa[mt] * sb);
      } else if constexpr (KIND == kW4) {
        const v4f swv = *reinterpret_cast<const v4f*>(tile + (BM + BN) * 128 + (wrow_l + 4 * lg) * 4);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) fma4v(acc[mt][nt], mfma_fp8(wf, xf[mt], zero), swv);
      } else {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][nt] = mfma_bf16x2(wf, xf[mt], acc[mt][nt]);
      }
    }
#pragma unroll
    for (int c = 0; c < ACH; ++c) st16(&smem[cur ^ 1][la0 + c * RSTEP * 128], ra[c]);
    wl.store(smem[cur ^ 1]);
    if constexpr (KIND == kW4)
      if (wsc_row) reinterpret_cast<float*>(smem[cur ^ 1] + (BM + BN) * 128)[tid] = wscn;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = san[mt];
    sb = sbn;
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = sorted[arow0 + mt * 16];
    if (r >= numel) continue;
    float rw = 1.0f;
    if constexpr (KIND == kW4) rw = a2s[arow0 + mt * 16];
    else rw = route_w ? route_w[r] : 1.0f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = n0 + wn * WTN + nt * 16 + 4 * lg;
      if (n >= H) continue;
      const v4f a = acc[mt][nt];
      *reinterpret_cast<uint2*>(y + static_cast<int64_t>(r) * H + n) =
          pack_bf16x4(a[0] * rw, a[1] * rw, a[2] * rw, a[3] * rw);
    }
  }
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

template <int KIND, bool W13>
__global__ __launch_bounds__(512, 1) void moe_gemm_dma_kernel(
    const uint8_t* __restrict__ act, const float* __restrict__ act_s, int topk, int K,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N, int I, float limit,
    const float* __restrict__ route_w, uint8_t* __restrict__ a2, float* __restrict__ a2s,
    uint16_t* __restrict__ y) {
  using P = MoePipe<KIND>;
  using KB_ = KindBytes<KIND>;
  constexpr int NS = 3, BM = 128, BN = 256, WN = 4, MT = P::MT, NT = P::NT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  const int TN = W13 ? I / 128 : (N + BN - 1) / BN;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, E, TN, e, mb, tn)) return;
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
  auto arow = [&](int r) -> int64_t {  // activation row of tile row r
    const int rr = mb * BM + r;
    if constexpr (W13) {
      const int s = sorted[rr];
      return s < numel ? static_cast<int64_t>(s / topk) : 0;
    } else {
      return rr;
    }
  };

  P p;
#pragma unroll
  for (int j = 0; j < P::kDmaA; ++j) {
    p.srcA[j] = act + arow(P::rowA(wave, lane, j)) * rowb + P::chunk(lane);
    p.ldsA[j] = (wave + j * P::kWaves) * 8 * 128;
  }
#pragma unroll
  for (int j = 0; j < P::kDmaB; ++j) {
    p.srcB[j] = w + (static_cast<int64_t>(e) * N + wrow(P::rowB(wave, lane, j))) * rowb + P::chunk(lane);
    p.ldsB[j] = P::kOffB + (wave + j * P::kWaves) * 8 * 128;
  }
  if constexpr (KIND == kFp8) {
    if (wave < BM / 64) {  // activation group scales of tile rows 64*wave + lane
      p.srcS = reinterpret_cast<const uint8_t*>(act_s + arow(64 * wave + lane) * KS);
      p.ldsS = P::kOffSA + 64 * wave * 4;
    } else {  // weight-block scales: W13 gate / up block, W2 the tile's two 128-row blocks
      const int slot = min(lane, 1);
      const int brow = W13 ? (slot ? (I + n0) / 128 : n0 / 128) : min(n0 / 128 + slot, NB - 1);
      p.srcS = reinterpret_cast<const uint8_t*>(ws + (static_cast<int64_t>(e) * NB + brow) * KS);
      p.ldsS = P::kOffSB;
    }
    p.stepS = 4;
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
  auto step = [&](int kb, const Frags& cur, Frags& nxt) {
    wait_lgkmcnt0();
    wait_vmcnt<(NS - 2) * P::kIPS>();
    barrier_lds();
    p.issue(smem_dyn + (kb % NS) * P::kStage, min(kb + NS, KS - 1));
    read(smem_dyn + ((kb + 1) % NS) * P::kStage, nxt);
    mma(cur);
  };
#pragma unroll
  for (int s = 0; s < NS; ++s) p.issue(smem_dyn + s * P::kStage, min(s, KS - 1));
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
        const float scale = amax / 448.0f;
        const int64_t row = static_cast<int64_t>(mb) * BM + ml;
        if (wn == 0 && lg == 0) a2s[row * gpr + tn] = scale;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          float o[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = v[mt][q][r];
            o[r] = x != x ? -448.0f : fminf(fmaxf(x / scale, -448.0f), 448.0f);
          }
          const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
          *reinterpret_cast<uint32_t*>(a2 + row * I + col) = f32x4_to_fp8x4(o[0], o[1], o[2], o[3]);
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
static size_t w13_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int kind) {
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

template <int KIND>
static int raise_w13_lds() {
  static bool done = false;
  if (done) return VMAMD_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(moe_w13_gemm_kernel<KIND>),
                          hipFuncAttributeMaxDynamicSharedMemorySize,
                          2 * w13_stage_bytes<KIND>()) != hipSuccess) {
    set_error("moe w13: cannot raise the LDS limit of the W13 kernel");
    return VMAMD_ERR_HIP;
  }
  done = true;
  return VMAMD_OK;
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

// Bytes of a decode GEMV's activation operand ([rows, K]); the GEMV reads it
// through a buffer descriptor, which the callers keep below 2 GiB.
template <int KIND>
static int gemv_act_bytes(int64_t rows, int64_t K) {
  return static_cast<int>(rows * (K / KindBytes<KIND>::kElems) * KindBytes<KIND>::kAct);
}

// Decode GEMV launch: an expert holds at most T routes when each token's
// top-k ids are distinct, so T <= 16 needs one 16-route block per pass
// (MAXB = 1, fewer registers); more blocks are still handled, by re-streaming
// the expert's weights once per block.
// vs: the kFp8 scale layout allows one 16-byte load per group of scales.
template <int KIND, typename... Args>
static void launch_gemv(dim3 grid, hipStream_t st, int T, bool vs, Args... args) {
  if constexpr (KIND != kBf16) {
    if (vs) {
      if (T <= kGemvBlock)
        moe_gemv_kernel<1, KIND, true><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args...);
      else
        moe_gemv_kernel<4, KIND, true><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args...);
      return;
    }
  }
  if (T <= kGemvBlock)
    moe_gemv_kernel<1, KIND><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args...);
  else
    moe_gemv_kernel<4, KIND><<<grid, kMoeGemvWaves * kWave, 0, st>>>(args...);
}

// True when a GEMV over K may read its scales U at a time: K/128 a multiple
// of U and the scale arrays aligned so that every row is (kFp8: 16 bytes for
// both scale sets; kW4: 8 bytes for the bf16 weight scales).
template <int KIND>
static bool gemv_vector_scales(int64_t K, const void* act_s, const void* w_s) {
  if constexpr (KIND == kFp8)
    return (K / 128) % kGemvU == 0 && reinterpret_cast<uintptr_t>(act_s) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(w_s) % 16 == 0;
  if constexpr (KIND == kW4) return (K / 128) % kGemvU == 0 && reinterpret_cast<uintptr_t>(w_s) % 8 == 0;
  return false;
}

// Launches of the two stages; arguments are validated by the callers.  kBf16:
// xa is x itself, xs / w13_s / a2s unused.  kW4: xs are the token row scales,
// a2 receives the bf16 activation (quantised per row by the caller).
template <int KIND>
static int launch_w13(const uint8_t* xa, const float* xs, int T, int H, int topk,
                      const int32_t* sorted, int64_t cap, int block_m, const int32_t* offs,
                      const int32_t* ntpp, const int32_t* active, const int32_t* nact,
                      const uint8_t* w13, const void* w13_s, int E, int I, float limit,
                      const float* route_w, uint8_t* a2, float* a2s, float* scratch, hipStream_t st) {
  const int numel = T * topk;
  if (block_m == kGemvBlock) {
    const int s13 = w13_splits(numel, E, H, I, KIND);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g13((2 * I / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s13);
    launch_gemv<KIND>(g13, st, T, gemv_vector_scales<KIND>(H, xs, w13_s), xa, gemv_act_bytes<KIND>(T, H),
                      xs, topk, H, sorted, offs, active,
                      nact, w13, w13_s, 2 * I, numel, s13, scratch,
                      static_cast<const float*>(nullptr), static_cast<uint16_t*>(nullptr));
    int rc = check_launch("moe w13 (gemv)");
    if (rc) return rc;
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
                                                                topk, a2, a2s);
    } else {
      const int64_t chunks = static_cast<int64_t>(numel) * (I / 8);
      moe_act_bf16_kernel<KIND><<<static_cast<int>((chunks + 255) / 256), 256, 0, st>>>(
          scratch, s13, numel, I, limit, xs, topk, route_w, reinterpret_cast<uint16_t*>(a2));
    }
    return check_launch("moe w13 (activation)");
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  const int tiles = max_blocks * (I / 128);
  if constexpr (KIND == kW4) {
    int rc = raise_w13_lds<KIND>();
    if (rc) return rc;
    moe_w13_gemm_kernel<KIND><<<xcd_grid(tiles), kW13Threads, 2 * w13_stage_bytes<KIND>(), st>>>(
        xa, xs, topk, H, sorted, offs, ntpp, E, numel, tiles, w13, w13_s, I, limit, a2, a2s);
  } else {
    int rc = raise_dma_lds<KIND, true>();
    if (rc) return rc;
    moe_gemm_dma_kernel<KIND, true><<<xcd_grid(tiles), 512, MoePipe<KIND>::kLds, st>>>(
        xa, xs, topk, H, sorted, offs, ntpp, E, numel, tiles, w13,
        static_cast<const float*>(w13_s), 2 * I, I, limit, route_w, a2, a2s, nullptr);
  }
  return check_launch("moe w13 (gemm)");
}

// kW4: a2s are the a2 row scales and take the routed weight's place in y.
// combined_out: when given and the decode path splits K, the reduce and the
// top-k combine run as one kernel writing the layer output there (y is not
// written) and *combined is set; otherwise y is written as usual.
template <int KIND>
static int launch_w2(const uint8_t* a2, const float* a2s, int T, int topk, const int32_t* sorted,
                     int64_t cap, int block_m, const int32_t* offs, const int32_t* ntpp,
                     const int32_t* active, const int32_t* nact, const uint8_t* w2, const void* w2_s,
                     int E, int H, int I, const float* topk_weights, const float* route_w,
                     const int32_t* topk_ids, const int32_t* emap, int64_t emap_len, uint16_t* y,
                     float* scratch, hipStream_t st, uint16_t* combined_out = nullptr,
                     bool* combined = nullptr) {
  const int numel = T * topk;
  const float* yscale = KIND == kW4 ? a2s : route_w;
  if (combined) *combined = false;
  if (block_m == kGemvBlock) {
    const int s2 = w2_splits(numel, E, H, I, KIND);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g2((H / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s2);
    if (s2 > 1 && combined_out && combined && H % 8 == 0) {
      launch_gemv<KIND>(g2, st, T, gemv_vector_scales<KIND>(I, a2s, w2_s), a2, gemv_act_bytes<KIND>(numel, I), a2s, 1, I, sorted, offs, active,
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
      launch_gemv<KIND>(g2, st, T, gemv_vector_scales<KIND>(I, a2s, w2_s), a2, gemv_act_bytes<KIND>(numel, I), a2s, 1, I, sorted, offs,
                        active, nact, w2, w2_s, H, numel, 1, static_cast<float*>(nullptr), yscale, y);
      return check_launch("moe w2 (gemv)");
    }
    launch_gemv<KIND>(g2, st, T, gemv_vector_scales<KIND>(I, a2s, w2_s), a2, gemv_act_bytes<KIND>(numel, I), a2s, 1, I, sorted, offs, active,
                      nact, w2, w2_s, H, numel, s2, scratch, static_cast<const float*>(nullptr),
                      static_cast<uint16_t*>(nullptr));
    int rc = check_launch("moe w2 (gemv)");
    if (rc) return rc;
    const int64_t mn = static_cast<int64_t>(numel) * H;
    moe_w2_reduce_kernel<<<static_cast<int>((mn / 4 + 255) / 256), 256, 0, st>>>(
        scratch, s2, numel, H, topk_ids, emap, emap_len, E, yscale, y);
    return check_launch("moe w2 (reduce)");
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  if constexpr (KIND == kW4) {
    const int tiles = max_blocks * ((H + 127) / 128);
    moe_w2_gemm_kernel<KIND><<<xcd_grid(tiles), 256, 0, st>>>(a2, a2s, I, sorted, offs, ntpp, E,
                                                              numel, tiles, w2, w2_s, H,
                                                              topk_weights, y);
  } else {
    const int tiles = max_blocks * ((H + 255) / 256);
    int rc = raise_dma_lds<KIND, false>();
    if (rc) return rc;
    moe_gemm_dma_kernel<KIND, false><<<xcd_grid(tiles), 512, MoePipe<KIND>::kLds, st>>>(
        a2, a2s, 1, I, sorted, offs, ntpp, E, numel, tiles, w2, static_cast<const float*>(w2_s), H,
        I, 0.f, route_w, nullptr, nullptr, y);
  }
  return check_launch("moe w2 (gemm)");
}

// Workspace carve-up of a fused layer, shared by the size query and the
// launcher.  The two stages run one after the other on one stream, so their
// scratch shares one region.  kFp8 / kW4 add the quantised x and scales; kW4
// also keeps the bf16 activation before its row quantiser.
struct MoeWs {
  size_t xq, xs, sorted, eids, ntpp, offs, active, nact, abf, a2, a2s, y, scratch, total;
};

static MoeWs moe_layout(int64_t T, int topk, int E, int64_t H, int64_t I, int bm, int kind) {
  MoeWs w{};
  const int64_t numel = T * topk;
  const int64_t cap = numel + static_cast<int64_t>(E) * (bm - 1);
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o += al256(bytes); return at; };
  if (kind != kBf16) {
    w.xq = take(T * H);
    w.xs = take(kind == kFp8 ? T * (H / 128) * 4 : T * 4);
  }
  w.sorted = take(cap * 4);
  w.eids = take(((cap + bm - 1) / bm) * 4);
  w.ntpp = take(4);
  w.offs = take((E + 1) * 4);
  w.active = take(E * 4);
  w.nact = take(4);
  const int64_t arows = bm == kGemvBlock ? numel : cap;  // route order (decode) or padded order
  if (kind == kW4) w.abf = take(arows * I * 2);
  w.a2 = take(arows * I * (kind == kBf16 ? 2 : 1));
  if (kind == kFp8) w.a2s = take(arows * (I / 128) * 4);
  if (kind == kW4) w.a2s = take(arows * 4);
  w.y = take(numel * H * 2);
  w.scratch = take(stage_scratch(numel, E, H, I, bm, kind));
  w.total = o;
  return w;
}

// Path choice of `auto`: the decode kernels (GEMV over 16-route blocks) up to
// a number of routes per expert measured on MI355X, the grouped GEMMs over
// 128-route blocks above.  Measured crossovers (graph replay, caches
// flushed): fp8 DeepSeek-V3 (E=256, H=7168, I=2048, top-8) between 2 and 3
// routes per expert (T=64 / 96); bf16 (E=128, H=2048, I=768) and w4afp8
// (E=128, H=4096, I=1536) between 8 and 16 (T=128 / 256).
static int moe_block_m(int64_t T, int topk, int E, int path, int kind) {
  if (path == VMAMD_MOE_PATH_GEMV) return kGemvBlock;
  if (path == VMAMD_MOE_PATH_GEMM) return kMoeBM;
  const int64_t routes = T * topk;
  const int64_t limit = kind == kFp8 ? (5 * static_cast<int64_t>(E)) / 2 : 12 * static_cast<int64_t>(E);
  return routes <= limit ? kGemvBlock : kMoeBM;
}

static int check_stage_common(const char* who, int64_t T, int topk, int E, int64_t H, int64_t I,
                              int block_m, int64_t cap) {
  VMAMD_REQUIRE(T >= 0 && topk > 0 && E > 0 && E <= 1024, "%s: bad sizes (T=%lld topk=%d E=%d)",
                who, (long long)T, topk, E);
  VMAMD_REQUIRE(H > 0 && I > 0 && H % 128 == 0 && I % 128 == 0,
                "%s: hidden (%lld) and intermediate (%lld) sizes must be multiples of 128", who,
                (long long)H, (long long)I);
  VMAMD_REQUIRE(block_m == kGemvBlock || block_m == kMoeBM, "%s: block_m must be %d or %d (got %d)",
                who, kGemvBlock, kMoeBM, block_m);
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
  VMAMD_REQUIRE(path >= VMAMD_MOE_PATH_AUTO && path <= VMAMD_MOE_PATH_GEMM, "%s: unknown path %d",
                who, path);
  VMAMD_REQUIRE(KIND != kW4 || !weight_on_input, "%s: apply_router_weight_on_input is not supported",
                who);
  const int bm = moe_block_m(T, topk, E, path, KIND);
  const int64_t cap = T * topk + static_cast<int64_t>(E) * (bm - 1);
  int rc = check_stage_common(who, T, topk, E, H, I, bm, cap);
  if (rc) return rc;
  VMAMD_REQUIRE(KIND != kW4 || (H <= 16384 && I <= 16384),
                "%s: per-row quantisation supports rows of up to 16384", who);
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
  float* a2s = KIND == kBf16 ? nullptr : reinterpret_cast<float*>(ws + L.a2s);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  float* scratch = reinterpret_cast<float*>(ws + L.scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int numel = static_cast<int>(T * topk);
  const int h = static_cast<int>(H), i = static_cast<int>(I), t = static_cast<int>(T);

  const uint8_t* xa = static_cast<const uint8_t*>(x);
  const float* xs = nullptr;
  if constexpr (KIND == kFp8) {  // quantiser and alignment in one launch
    uint8_t* xq = ws + L.xq;
    float* xsw = reinterpret_cast<float*>(ws + L.xs);
    rc = align_and_group_quant_fp8(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap,
                                   eids, ntpp, offs, active, nact, x, T, H, xq, xsw, st);
    if (rc) return rc;
    xa = xq;
    xs = xsw;
  } else if constexpr (KIND == kW4) {  // per-row quantiser and alignment in one launch
    uint8_t* xq = ws + L.xq;
    float* xsw = reinterpret_cast<float*>(ws + L.xs);
    rc = align_and_row_quant_fp8(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap,
                                 eids, ntpp, offs, active, nact, x, T, H, xq, xsw, st);
    if (rc) return rc;
    xa = xq;
    xs = xsw;
  } else {
    rc = vmamd_moe_align_block_size(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap,
                                    eids, ntpp, offs, nullptr, active, nact, stream);
    if (rc) return rc;
  }
  // kW4 prefill: bf16 activation, quantised per row below (the decode path
  // writes the quantised a2 directly).
  uint8_t* act_out = KIND == kW4 && bm != kGemvBlock ? ws + L.abf : a2;
  // The routed weight is applied once: on the W13 output before the
  // activation (apply_router_weight_on_input), otherwise in the W2 epilogue.
  const float* w13_rw = weight_on_input ? topk_weights : nullptr;
  const float* w2_rw = weight_on_input ? nullptr : topk_weights;
  rc = launch_w13<KIND>(xa, xs, t, h, topk, sorted, cap, bm, offs, ntpp, active, nact,
                        static_cast<const uint8_t*>(w13), w13_s, E, i, swiglu_limit, w13_rw, act_out,
                        a2s, scratch, st);
  if (rc) return rc;
  if constexpr (KIND == kW4) {
    if (bm != kGemvBlock) {
      rc = vmamd_per_token_quant_fp8(act_out, cap, I, I, 1e-4f, -448.f, 448.f, a2, a2s, stream);
      if (rc) return rc;
    }
  }
  bool combined = false;
  rc = launch_w2<KIND>(a2, a2s, t, topk, sorted, cap, bm, offs, ntpp, active, nact,
                       static_cast<const uint8_t*>(w2), w2_s, E, h, i, topk_weights, w2_rw, topk_ids,
                       expert_map, expert_map_len, y, scratch, st, static_cast<uint16_t*>(out),
                       &combined);
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
  int rc = check_stage_common(who, T, topk, E, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(xa && sorted && offs && ntpp && w13 && a2 &&
                    (KIND == kBf16 || (xs && w13_s)) && (KIND != kFp8 || a2s),
                "%s: null pointer", who);
  VMAMD_REQUIRE(block_m == kMoeBM || (active && nact),
                "%s: the decode path (block_m 16) needs active_experts / num_active", who);
  const size_t need = w13_scratch(T * topk, E, H, I, block_m, KIND);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(xa) % 16 == 0 && reinterpret_cast<uintptr_t>(a2) % 16 == 0,
                "%s: activations, a2 and workspace must be 16-byte aligned", who);
  return launch_w13<KIND>(static_cast<const uint8_t*>(xa), xs, static_cast<int>(T), static_cast<int>(H),
                          topk, sorted, capacity, block_m, offs, ntpp, active, nact,
                          static_cast<const uint8_t*>(w13), w13_s, E, static_cast<int>(I), limit,
                          nullptr, static_cast<uint8_t*>(a2), a2s, static_cast<float*>(workspace),
                          reinterpret_cast<hipStream_t>(stream));
}

template <int KIND>
static int stage_w2(const char* who, const void* a2, const float* a2s, int64_t T, int topk,
                    const int32_t* sorted, int64_t capacity, int block_m, const int32_t* offs,
                    const int32_t* ntpp, const int32_t* active, const int32_t* nact, const void* w2,
                    const void* w2_s, int E, int64_t H, int64_t I, const float* topk_weights,
                    const int32_t* topk_ids, const int32_t* emap, int64_t emap_len, void* y,
                    void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common(who, T, topk, E, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(a2 && sorted && offs && ntpp && w2 && topk_ids && y &&
                    (KIND == kBf16 || (a2s && w2_s)) && (KIND == kW4 || topk_weights),
                "%s: null pointer", who);
  VMAMD_REQUIRE(block_m == kMoeBM || (active && nact),
                "%s: the decode path (block_m 16) needs active_experts / num_active", who);
  const size_t need = w2_scratch(T * topk, E, H, I, block_m, KIND);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a2) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0,
                "%s: a2 and workspace must be 16-byte and y 8-byte aligned", who);
  return launch_w2<KIND>(static_cast<const uint8_t*>(a2), a2s, static_cast<int>(T), topk, sorted,
                         capacity, block_m, offs, ntpp, active, nact, static_cast<const uint8_t*>(w2),
                         w2_s, E, static_cast<int>(H), static_cast<int>(I), topk_weights,
                         KIND == kW4 ? nullptr : topk_weights, topk_ids,
                         emap, emap_len, static_cast<uint16_t*>(y), static_cast<float*>(workspace),
                         reinterpret_cast<hipStream_t>(stream));
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
  return moe_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path, kFp8), kFp8).total;
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
