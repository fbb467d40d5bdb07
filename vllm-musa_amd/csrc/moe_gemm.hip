// Fused-MoE expert GEMMs (W13 gate/up, W2 down) for 128x128 block-fp8 and
// for bf16 expert weights.
//
// Layouts (row-major):
//   fp8:  xq [T, H] e4m3, xs [T, H/128] f32 (1x128 activation groups)
//         w13 [E, 2I, H] e4m3, w13_s [E, 2I/128, H/128]; w2 [E, H, I], w2_s [E, H/128, I/128]
//   bf16: x [T, H] bf16; w13 [E, 2I, H] bf16; w2 [E, H, I] bf16
//   w13 rows [0, I) gate, [I, 2I) up; routes r = t * topk + k; sorted /
//   offsets / active come from moe_align_block_size.
//
// Both operand kinds move 128-byte row chunks: for fp8 a chunk is one
// 128-wide K-block (one 16x16x128 MFMA, then the scale promotion
// acc += p * sa[m] * sb[n/128]); for bf16 it is 64 K-elements (two chained
// 16x16x32 bf16 MFMAs, no scales).
//
// Decode path (few routes per expert): moe_gemv_kernel.  A wave owns 16
// weight rows of one active expert and a K range; it streams the rows from
// HBM once (no LDS) and applies each 16-row fragment to every 16-route block
// of that expert.  W13 writes fp32 split-K partials per route; the act kernel
// sums them in a fixed order, rounds gate/up to bf16, applies SiLU-and-mul
// and (fp8) quantises a2 per 1x128 group.  W2 writes bf16(acc * routed
// weight) per route, or fp32 partials reduced by moe_w2_reduce_kernel.
//
// Prefill path (many routes per expert): grouped MFMA GEMMs over 128-route
// blocks.  Tiles are ordered expert-major -- all blocks of one (expert,
// n-tile) are consecutive -- and each XCD takes a contiguous tile range, so
// the blocks of an expert that share a weight tile run together on one XCD
// and the tile is fetched from HBM once.  W13 covers 128 gate + 128 up rows
// per tile (interleaved by 16 so each lane holds matching gate/up values) and
// fuses SiLU-and-mul (and the fp8 a2 quantiser) into its epilogue.
#include <algorithm>

#include "mfma_fp8.h"

namespace vmamd {

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

// One 128-byte chunk of both operands into an accumulator.
template <bool FP8>
__device__ __forceinline__ void chunk_mma(v4f& acc, const v8i& w, const v8i& x, float s) {
  if constexpr (FP8) {
    fma4(acc, mfma_fp8(w, x, v4f{0.f, 0.f, 0.f, 0.f}), s);
  } else {
    acc = mfma_bf16x2(w, x, acc);
  }
}

// ---------------------------------------------------------- decode GEMV ---
constexpr int kMoeGemvWaves = 4;
constexpr int kGemvBlock = 16;  // routes per block (one MFMA column tile)

template <int MAXB, bool FP8>
__global__ __launch_bounds__(kMoeGemvWaves * kWave) void moe_gemv_kernel(
    const uint8_t* __restrict__ act, const float* __restrict__ act_s, int act_div, int K,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ active, const int32_t* __restrict__ num_active,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N, int numel, int splits,
    float* __restrict__ partial, const float* __restrict__ route_w, uint16_t* __restrict__ y) {
  constexpr int EB = FP8 ? 1 : 2;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int li = lane % 16, lg = lane / 16;
  const int ntile = blockIdx.x * kMoeGemvWaves + wave;
  if (ntile * 16 >= N) return;  // wave-uniform, no barriers in this kernel
  const int slot = blockIdx.y;
  if (slot >= num_active[0]) return;
  const int e = active[slot];
  const int seg0 = offsets[e];
  const int nblk = (offsets[e + 1] - seg0) / kGemvBlock;
  const int split = blockIdx.z;
  const int64_t rowb = static_cast<int64_t>(K) * EB;
  const int KC = static_cast<int>(rowb / 128);  // 128-byte chunks (== scale blocks for fp8)
  const int NB = (N + 127) / 128;
  const int kb0 = split * KC / splits, kb1 = (split + 1) * KC / splits;
  const uint8_t* wrow = w + (static_cast<int64_t>(e) * N + ntile * 16 + li) * rowb;
  const float* wsr = nullptr;
  if constexpr (FP8) wsr = ws + (static_cast<int64_t>(e) * NB + (ntile * 16) / 128) * KC;
  const int n = ntile * 16 + 4 * lg;

  for (int b0 = 0; b0 < nblk; b0 += MAXB) {
    const int nb = min(MAXB, nblk - b0);
    int rr[MAXB];
    const uint8_t* arow[MAXB];
    const float* asr[MAXB];
#pragma unroll
    for (int b = 0; b < MAXB; ++b) {
      const int r = sorted[seg0 + (b0 + min(b, nb - 1)) * kGemvBlock + li];
      const bool valid = r < numel;
      rr[b] = valid ? r : -1;
      const int64_t row = valid ? r / act_div : 0;
      arow[b] = act + row * rowb;
      asr[b] = FP8 ? act_s + row * KC : nullptr;
    }
    v4f acc[MAXB];
#pragma unroll
    for (int b = 0; b < MAXB; ++b) acc[b] = v4f{0.f, 0.f, 0.f, 0.f};

    constexpr int U = 4;
    int kb = kb0;
    for (; kb + U <= kb1; kb += U) {
      v8i wf[U];
      float sb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        wf[u] = global_frag(wrow + (kb + u) * 128, lg);
        sb[u] = 0.f;
        if constexpr (FP8) sb[u] = wsr[kb + u];
      }
#pragma unroll
      for (int b = 0; b < MAXB; ++b) {
        if (b < nb) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const v8i xf = global_frag(arow[b] + (kb + u) * 128, lg);
            float s = 0.f;
            if constexpr (FP8) s = asr[b][kb + u] * sb[u];
            chunk_mma<FP8>(acc[b], wf[u], xf, s);
          }
        }
      }
    }
    for (; kb < kb1; ++kb) {
      const v8i wf = global_frag(wrow + kb * 128, lg);
      float sb = 0.f;
      if constexpr (FP8) sb = wsr[kb];
#pragma unroll
      for (int b = 0; b < MAXB; ++b) {
        if (b < nb) {
          float s = 0.f;
          if constexpr (FP8) s = asr[b][kb] * sb;
          chunk_mma<FP8>(acc[b], wf, global_frag(arow[b] + kb * 128, lg), s);
        }
      }
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
  }
}

// Gate/up of 8 consecutive columns c0.. of route r, split partials summed in
// a fixed order, each rounded to bf16 and combined by SiLU-and-mul.
__device__ __forceinline__ void act8(const float* __restrict__ partial, int splits, int numel, int I,
                                     int r, int c0, float limit, float (&v)[8]) {
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
    v[j + 0] = swiglu_bf16(bf16r(gs.x), bf16r(us.x), limit);
    v[j + 1] = swiglu_bf16(bf16r(gs.y), bf16r(us.y), limit);
    v[j + 2] = swiglu_bf16(bf16r(gs.z), bf16r(us.z), limit);
    v[j + 3] = swiglu_bf16(bf16r(gs.w), bf16r(us.w), limit);
  }
}

// fp8: activation then a2 quantisation per 1x128 group (one 16-lane segment
// per group, 8 columns per lane).  NaN activations (clamped variant) quantise
// to fp8_min.
__global__ __launch_bounds__(256) void moe_act_quant_kernel(const float* __restrict__ partial,
                                                            int splits, int numel, int I,
                                                            float limit, uint8_t* __restrict__ a2q,
                                                            float* __restrict__ a2s) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * 16 + threadIdx.x / 16;
  const int sub = threadIdx.x % 16;
  const int gpr = I / 128;
  if (g >= static_cast<int64_t>(numel) * gpr) return;
  const int r = static_cast<int>(g / gpr);
  const int c0 = static_cast<int>(g % gpr) * 128 + sub * 8;
  float v[8];
  act8(partial, splits, numel, I, r, c0, limit, v);
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

// bf16: a2[r, c] = the bf16 activation, 8 columns per thread (16-byte store).
__global__ __launch_bounds__(256) void moe_act_bf16_kernel(const float* __restrict__ partial,
                                                           int splits, int numel, int I,
                                                           float limit, uint16_t* __restrict__ a2) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int cpr = I / 8;
  if (idx >= static_cast<int64_t>(numel) * cpr) return;
  const int r = static_cast<int>(idx / cpr);
  const int c0 = static_cast<int>(idx % cpr) * 8;
  float v[8];
  act8(partial, splits, numel, I, r, c0, limit, v);
  uint4 o;
  o.x = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  o.y = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
  o.z = static_cast<uint32_t>(f32_to_bf16(v[4])) | (static_cast<uint32_t>(f32_to_bf16(v[5])) << 16);
  o.w = static_cast<uint32_t>(f32_to_bf16(v[6])) | (static_cast<uint32_t>(f32_to_bf16(v[7])) << 16);
  *reinterpret_cast<uint4*>(a2 + static_cast<int64_t>(r) * I + c0) = o;
}

// y[r, n] = bf16(sum_s partial[s, r, n] * w_r) for the W2 split path.
__global__ __launch_bounds__(256) void moe_w2_reduce_kernel(const float* __restrict__ partial,
                                                            int splits, int numel, int N,
                                                            const int32_t* __restrict__ ids,
                                                            const int32_t* __restrict__ emap,
                                                            int64_t emap_len,
                                                            const float* __restrict__ route_w,
                                                            uint16_t* __restrict__ y) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  const int64_t mn = static_cast<int64_t>(numel) * N;
  if (i4 >= mn) return;
  const int r = static_cast<int>(i4 / N);
  if (emap) {
    const int e = ids[r];
    if (e < 0 || e >= emap_len || emap[e] < 0) return;
  }
  float4 acc = *reinterpret_cast<const float4*>(partial + i4);
  for (int s = 1; s < splits; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(partial + s * mn + i4);
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  const float rw = route_w ? route_w[r] : 1.0f;
  *reinterpret_cast<uint2*>(y + i4) = pack_bf16x4(acc.x * rw, acc.y * rw, acc.z * rw, acc.w * rw);
}

// ------------------------------------------------------ prefill GEMMs -----
constexpr int kMoeBM = 128;

// Expert-major decode of a logical tile index: all blocks of (expert, tn)
// are consecutive.  Returns false past the used tiles.
__device__ __forceinline__ bool moe_tile(int wg, int max_tiles, const int32_t* __restrict__ offsets,
                                         const int32_t* __restrict__ ntpp, int E, int TN,
                                         int& e_out, int& mb_out, int& tn_out) {
  const int per = (max_tiles + kXcds - 1) / kXcds;
  const int L = (wg % kXcds) * per + wg / kXcds;
  const int used = ntpp[0] / kMoeBM * TN;
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

// W13: tile = 128 routes x (128 gate + 128 up rows); 8 waves as 2 (m) x 4 (n);
// local weight row j: pair p = j / 32, q = j % 32 -> gate row n0 + 16p + q
// (q < 16) or up row I + n0 + 16p + q - 16.  Dynamic LDS: 2 x 48 KiB.
constexpr int kW13Threads = 512;
constexpr int kW13Lds = 2 * (kMoeBM + 256) * 128;

template <bool FP8>
__global__ __launch_bounds__(kW13Threads, 1) void moe_w13_gemm_kernel(
    const uint8_t* __restrict__ xa, const float* __restrict__ xs, int topk, int H,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w13, const float* __restrict__ w13s, int I, float limit,
    uint8_t* __restrict__ a2, float* __restrict__ a2s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  constexpr int EB = FP8 ? 1 : 2;
  constexpr int BM = kMoeBM, BN = 256, THREADS = kW13Threads;
  constexpr int WN = 4, WTM = 64, WTN = 64, MT = 4, NT = 4;
  constexpr int RSTEP = THREADS / 8;                 // 64 rows per copy pass
  constexpr int ACH = BM / RSTEP, BCH = BN / RSTEP;  // 2, 4
  constexpr int STAGE = (BM + BN) * 128;

  const int TN = I / 128;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, E, TN, e, mb, tn)) return;
  const int n0 = tn * 128;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane % 16, lg = lane / 16;
  const int64_t rowb = static_cast<int64_t>(H) * EB;
  const int KC = static_cast<int>(rowb / 128);  // chunks; == scale blocks for fp8
  const int NB2 = (2 * I + 127) / 128;

  const int crow = tid / 8, cch = tid % 8;
  const int l0 = lds_off(crow, cch);
  // Padding rows of the block load row 0 and are zeroed in registers.
  int64_t goff_a[ACH];
  bool aval[ACH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const int r = sorted[mb * BM + crow + c * RSTEP];
    aval[c] = r < numel;
    goff_a[c] = (aval[c] ? static_cast<int64_t>(r / topk) * rowb : 0) + cch * 16;
  }
  int64_t goff_b[BCH];
#pragma unroll
  for (int c = 0; c < BCH; ++c) {
    const int j = crow + c * RSTEP, p = j / 32, q = j % 32;
    const int row = q < 16 ? n0 + 16 * p + q : I + n0 + 16 * p + (q - 16);
    goff_b[c] = (static_cast<int64_t>(e) * 2 * I + row) * rowb + cch * 16;
  }
  const float* xs_row[MT];
  bool tval[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = sorted[mb * BM + wm * WTM + mt * 16 + li];
    tval[mt] = r < numel;
    xs_row[mt] = FP8 ? xs + (tval[mt] ? static_cast<int64_t>(r / topk) * KC : 0) : nullptr;
  }
  const float* sg = FP8 ? w13s + (static_cast<int64_t>(e) * NB2 + n0 / 128) * KC : nullptr;
  const float* su = FP8 ? w13s + (static_cast<int64_t>(e) * NB2 + (I + n0) / 128) * KC : nullptr;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  const v4i z4 = {0, 0, 0, 0};
  v4i ra[ACH], rb[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const v4i v = ld16(xa + goff_a[c]);
    ra[c] = aval[c] ? v : z4;
  }
#pragma unroll
  for (int c = 0; c < BCH; ++c) rb[c] = ld16(w13 + goff_b[c]);
#pragma unroll
  for (int c = 0; c < ACH; ++c) st16(&smem_dyn[l0 + c * RSTEP * 128], ra[c]);
#pragma unroll
  for (int c = 0; c < BCH; ++c) st16(&smem_dyn[BM * 128 + l0 + c * RSTEP * 128], rb[c]);
  float sa[MT], sbg = 0.f, sbu = 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = 0.f;
  if constexpr (FP8) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = tval[mt] ? xs_row[mt][0] : 0.f;
    sbg = sg[0];
    sbu = su[0];
  }
  __syncthreads();

  for (int kb = 0; kb < KC; ++kb) {
    const int cur = kb & 1;
    // Prefetch chunk kb+1 (the last iteration re-reads chunk KC-1 into the
    // idle buffer; that copy is never used).
    const int kn = min(kb + 1, KC - 1);
    const int off = kn * 128;
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const v4i v = ld16(xa + goff_a[c] + off);
      ra[c] = aval[c] ? v : z4;
    }
#pragma unroll
    for (int c = 0; c < BCH; ++c) rb[c] = ld16(w13 + goff_b[c] + off);
    float san[MT], sbgn = 0.f, sbun = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) san[mt] = 0.f;
    if constexpr (FP8) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float v = xs_row[mt][kn];
        san[mt] = tval[mt] ? v : 0.f;
      }
      sbgn = sg[kn];
      sbun = su[kn];
    }

    const uint8_t* tile = smem_dyn + cur * STAGE;
    v8i xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt] = lds_frag(tile, wm * WTM + mt * 16 + li, lg);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const v8i wf = lds_frag(tile + BM * 128, wn * WTN + nt * 16 + li, lg);
      const float sb = (nt & 1) ? sbu : sbg;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) chunk_mma<FP8>(acc[mt][nt], wf, xf[mt], sa[mt] * sb);
    }
    uint8_t* nxt = smem_dyn + (cur ^ 1) * STAGE;
#pragma unroll
    for (int c = 0; c < ACH; ++c) st16(&nxt[l0 + c * RSTEP * 128], ra[c]);
#pragma unroll
    for (int c = 0; c < BCH; ++c) st16(&nxt[BM * 128 + l0 + c * RSTEP * 128], rb[c]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = san[mt];
    sbg = sbgn;
    sbu = sbun;
    __syncthreads();
  }

  if constexpr (FP8) {
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
        for (int r = 0; r < 4; ++r)
          o[r] = swiglu_bf16(bf16r(acc[mt][2 * q][r]), bf16r(acc[mt][2 * q + 1][r]), limit);
        const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
        *reinterpret_cast<uint2*>(a2b + row * I + col) = pack_bf16x4(o[0], o[1], o[2], o[3]);
      }
    }
  }
}

// W2: tile = 128 routes x 128 hidden rows, 4 waves as 2 x 2, K = I.
template <bool FP8>
__global__ __launch_bounds__(256, 2) void moe_w2_gemm_kernel(
    const uint8_t* __restrict__ a2, const float* __restrict__ a2s, int I,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w2, const float* __restrict__ w2s, int H,
    const float* __restrict__ route_w, uint16_t* __restrict__ y) {
  constexpr int EB = FP8 ? 1 : 2;
  constexpr int BM = kMoeBM, BN = 128, THREADS = 256, WN = 2, WTM = 64, WTN = 64, MT = 4, NT = 4;
  constexpr int RSTEP = THREADS / 8, ACH = BM / RSTEP, BCH = BN / RSTEP;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][(BM + BN) * 128];

  const int TN = (H + BN - 1) / BN;
  int e, mb, tn;
  if (!moe_tile(blockIdx.x, max_tiles, offsets, ntpp, E, TN, e, mb, tn)) return;
  const int n0 = tn * BN;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane % 16, lg = lane / 16;
  const int64_t rowb = static_cast<int64_t>(I) * EB;
  const int KC = static_cast<int>(rowb / 128);
  const int NBH = (H + 127) / 128;

  const int crow = tid / 8, cch = tid % 8;
  const int l0 = lds_off(crow, cch);
  int64_t goff_a[ACH], goff_b[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c)
    goff_a[c] = (static_cast<int64_t>(mb) * BM + crow + c * RSTEP) * rowb + cch * 16;
#pragma unroll
  for (int c = 0; c < BCH; ++c)
    goff_b[c] = (static_cast<int64_t>(e) * H + min(n0 + crow + c * RSTEP, H - 1)) * rowb + cch * 16;
  const float* sb_p = FP8 ? w2s + (static_cast<int64_t>(e) * NBH + n0 / 128) * KC : nullptr;
  const int64_t arow0 = static_cast<int64_t>(mb) * BM + wm * WTM + li;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  v4i ra[ACH], rb[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) ra[c] = ld16(a2 + goff_a[c]);
#pragma unroll
  for (int c = 0; c < BCH; ++c) rb[c] = ld16(w2 + goff_b[c]);
#pragma unroll
  for (int c = 0; c < ACH; ++c) st16(&smem[0][l0 + c * RSTEP * 128], ra[c]);
#pragma unroll
  for (int c = 0; c < BCH; ++c) st16(&smem[0][BM * 128 + l0 + c * RSTEP * 128], rb[c]);
  float sa[MT], sb = 0.f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = 0.f;
  if constexpr (FP8) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = a2s[(arow0 + mt * 16) * KC];
    sb = sb_p[0];
  }
  __syncthreads();

  for (int kb = 0; kb < KC; ++kb) {
    const int cur = kb & 1;
    const int kn = min(kb + 1, KC - 1);
    const int off = kn * 128;
#pragma unroll
    for (int c = 0; c < ACH; ++c) ra[c] = ld16(a2 + goff_a[c] + off);
#pragma unroll
    for (int c = 0; c < BCH; ++c) rb[c] = ld16(w2 + goff_b[c] + off);
    float san[MT], sbn = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) san[mt] = 0.f;
    if constexpr (FP8) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) san[mt] = a2s[(arow0 + mt * 16) * KC + kn];
      sbn = sb_p[kn];
    }
    const uint8_t* tile = smem[cur];
    v8i xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt] = lds_frag(tile, wm * WTM + mt * 16 + li, lg);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const v8i wf = lds_frag(tile + BM * 128, wn * WTN + nt * 16 + li, lg);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) chunk_mma<FP8>(acc[mt][nt], wf, xf[mt], sa[mt] * sb);
    }
#pragma unroll
    for (int c = 0; c < ACH; ++c) st16(&smem[cur ^ 1][l0 + c * RSTEP * 128], ra[c]);
#pragma unroll
    for (int c = 0; c < BCH; ++c) st16(&smem[cur ^ 1][BM * 128 + l0 + c * RSTEP * 128], rb[c]);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) sa[mt] = san[mt];
    sb = sbn;
    __syncthreads();
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = sorted[arow0 + mt * 16];
    if (r >= numel) continue;
    const float rw = route_w ? route_w[r] : 1.0f;
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

// ------------------------------------------------------------ host side ---
// Split-K factor of the decode GEMVs: enough waves to cover the chip
// (>= 4096 over the active experts' n-tiles), at least 4 chunks per split.
static int moe_splits(int64_t waves_per_split, int KC) {
  int s = static_cast<int>((4096 + waves_per_split - 1) / waves_per_split);
  return max(1, min(s, max(1, KC / 4)));
}

static int64_t moe_umax(int64_t numel, int E) { return std::min<int64_t>(E, numel); }

// eb = operand bytes per element (1 fp8, 2 bf16).
static int w13_splits(int64_t numel, int E, int64_t H, int64_t I, int eb) {
  return moe_splits(moe_umax(numel, E) * (2 * I / 16), static_cast<int>(H * eb / 128));
}
static int w2_splits(int64_t numel, int E, int64_t H, int64_t I, int eb) {
  return moe_splits(moe_umax(numel, E) * (H / 16), static_cast<int>(I * eb / 128));
}

static size_t al256(size_t x) { return (x + 255) / 256 * 256; }

// Stage scratch: fp32 split-K partials of the decode GEMVs (none for GEMMs).
static size_t w13_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int eb) {
  if (block_m != kGemvBlock) return 0;
  return al256(static_cast<size_t>(w13_splits(numel, E, H, I, eb)) * numel * 2 * I * 4);
}
static size_t w2_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int eb) {
  if (block_m != kGemvBlock) return 0;
  const int s = w2_splits(numel, E, H, I, eb);
  return s > 1 ? al256(static_cast<size_t>(s) * numel * H * 4) : 0;
}
static size_t stage_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m, int eb) {
  return std::max(w13_scratch(numel, E, H, I, block_m, eb), w2_scratch(numel, E, H, I, block_m, eb));
}

template <bool FP8>
static int raise_w13_lds() {
  static bool done = false;
  if (done) return VMAMD_OK;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(moe_w13_gemm_kernel<FP8>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, kW13Lds) != hipSuccess) {
    set_error("moe w13: cannot raise the LDS limit of the W13 kernel");
    return VMAMD_ERR_HIP;
  }
  done = true;
  return VMAMD_OK;
}

// Launches of the two stages; arguments are validated by the callers.  For
// bf16 `xa` is x itself and xs / w13_s / a2s are unused.
template <bool FP8>
static int launch_w13(const uint8_t* xa, const float* xs, int T, int H, int topk,
                      const int32_t* sorted, int64_t cap, int block_m, const int32_t* offs,
                      const int32_t* ntpp, const int32_t* active, const int32_t* nact,
                      const uint8_t* w13, const float* w13_s, int E, int I, float limit,
                      uint8_t* a2, float* a2s, float* scratch, hipStream_t st) {
  constexpr int EB = FP8 ? 1 : 2;
  const int numel = T * topk;
  if (block_m == kGemvBlock) {
    const int s13 = w13_splits(numel, E, H, I, EB);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g13((2 * I / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s13);
    moe_gemv_kernel<4, FP8><<<g13, kMoeGemvWaves * kWave, 0, st>>>(
        xa, xs, topk, H, sorted, offs, active, nact, w13, w13_s, 2 * I, numel, s13, scratch,
        nullptr, nullptr);
    int rc = check_launch("moe w13 (gemv)");
    if (rc) return rc;
    if constexpr (FP8) {
      const int64_t groups = static_cast<int64_t>(numel) * (I / 128);
      moe_act_quant_kernel<<<static_cast<int>((groups + 15) / 16), 256, 0, st>>>(
          scratch, s13, numel, I, limit, a2, a2s);
    } else {
      const int64_t chunks = static_cast<int64_t>(numel) * (I / 8);
      moe_act_bf16_kernel<<<static_cast<int>((chunks + 255) / 256), 256, 0, st>>>(
          scratch, s13, numel, I, limit, reinterpret_cast<uint16_t*>(a2));
    }
    return check_launch("moe w13 (activation)");
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  const int tiles = max_blocks * (I / 128);
  int rc = raise_w13_lds<FP8>();
  if (rc) return rc;
  moe_w13_gemm_kernel<FP8><<<xcd_grid(tiles), kW13Threads, kW13Lds, st>>>(
      xa, xs, topk, H, sorted, offs, ntpp, E, numel, tiles, w13, w13_s, I, limit, a2, a2s);
  return check_launch("moe w13 (gemm)");
}

template <bool FP8>
static int launch_w2(const uint8_t* a2, const float* a2s, int T, int topk, const int32_t* sorted,
                     int64_t cap, int block_m, const int32_t* offs, const int32_t* ntpp,
                     const int32_t* active, const int32_t* nact, const uint8_t* w2, const float* w2_s,
                     int E, int H, int I, const float* topk_weights, const int32_t* topk_ids,
                     const int32_t* emap, int64_t emap_len, uint16_t* y, float* scratch,
                     hipStream_t st) {
  constexpr int EB = FP8 ? 1 : 2;
  const int numel = T * topk;
  if (block_m == kGemvBlock) {
    const int s2 = w2_splits(numel, E, H, I, EB);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g2((H / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s2);
    if (s2 == 1) {
      moe_gemv_kernel<4, FP8><<<g2, kMoeGemvWaves * kWave, 0, st>>>(
          a2, a2s, 1, I, sorted, offs, active, nact, w2, w2_s, H, numel, 1, nullptr, topk_weights, y);
      return check_launch("moe w2 (gemv)");
    }
    moe_gemv_kernel<4, FP8><<<g2, kMoeGemvWaves * kWave, 0, st>>>(
        a2, a2s, 1, I, sorted, offs, active, nact, w2, w2_s, H, numel, s2, scratch, nullptr, nullptr);
    int rc = check_launch("moe w2 (gemv)");
    if (rc) return rc;
    const int64_t mn = static_cast<int64_t>(numel) * H;
    moe_w2_reduce_kernel<<<static_cast<int>((mn / 4 + 255) / 256), 256, 0, st>>>(
        scratch, s2, numel, H, topk_ids, emap, emap_len, topk_weights, y);
    return check_launch("moe w2 (reduce)");
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  const int tiles = max_blocks * ((H + 127) / 128);
  moe_w2_gemm_kernel<FP8><<<xcd_grid(tiles), 256, 0, st>>>(a2, a2s, I, sorted, offs, ntpp, E, numel,
                                                           tiles, w2, w2_s, H, topk_weights, y);
  return check_launch("moe w2 (gemm)");
}

// Workspace carve-up of a fused layer, shared by the size query and the
// launcher.  The two stages run one after the other on one stream, so their
// scratch shares one region.  fp8 adds the quantised x and a2 scales.
struct MoeWs {
  size_t xq, xs, sorted, eids, ntpp, offs, active, nact, a2, a2s, y, scratch, total;
};

static MoeWs moe_layout(int64_t T, int topk, int E, int64_t H, int64_t I, int bm, bool fp8) {
  MoeWs w{};
  const int eb = fp8 ? 1 : 2;
  const int64_t numel = T * topk;
  const int64_t cap = numel + static_cast<int64_t>(E) * (bm - 1);
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o += al256(bytes); return at; };
  if (fp8) {
    w.xq = take(T * H);
    w.xs = take(T * (H / 128) * 4);
  }
  w.sorted = take(cap * 4);
  w.eids = take(((cap + bm - 1) / bm) * 4);
  w.ntpp = take(4);
  w.offs = take((E + 1) * 4);
  w.active = take(E * 4);
  w.nact = take(4);
  const int64_t arows = bm == kGemvBlock ? numel : cap;  // route order (decode) or padded order
  w.a2 = take(arows * I * eb);
  if (fp8) w.a2s = take(arows * (I / 128) * 4);
  w.y = take(numel * H * 2);
  w.scratch = take(stage_scratch(numel, E, H, I, bm, eb));
  w.total = o;
  return w;
}

// Decode kernels (GEMV over 16-route blocks) while an expert receives about
// one block of routes on average (or up to 64 tokens), the grouped GEMM over
// 128-route blocks above: below that the 128-row tiles are mostly padding.
static int moe_block_m(int64_t T, int topk, int E, int path) {
  if (path == VMAMD_MOE_PATH_GEMV) return kGemvBlock;
  if (path == VMAMD_MOE_PATH_GEMM) return kMoeBM;
  return (T <= 64 || T * topk <= static_cast<int64_t>(kGemvBlock) * E) ? kGemvBlock : kMoeBM;
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
  VMAMD_REQUIRE(cap >= T * topk + static_cast<int64_t>(E) * (block_m - 1) && cap < (1ll << 31),
                "%s: capacity %lld < T*topk + E*(block_m-1)", who, (long long)cap);
  return VMAMD_OK;
}

template <bool FP8>
static int fused_layer(const char* who, const void* x, int64_t T, int64_t H, const void* w13,
                       const float* w13_s, const void* w2, const float* w2_s, int E, int64_t I,
                       const float* topk_weights, const int32_t* topk_ids, int topk,
                       const int32_t* expert_map, int64_t expert_map_len, float swiglu_limit,
                       int path, void* out, void* workspace, size_t workspace_bytes,
                       vmamd_stream_t stream) {
  VMAMD_REQUIRE(path >= VMAMD_MOE_PATH_AUTO && path <= VMAMD_MOE_PATH_GEMM, "%s: unknown path %d",
                who, path);
  const int bm = moe_block_m(T, topk, E, path);
  const int64_t cap = T * topk + static_cast<int64_t>(E) * (bm - 1);
  int rc = check_stage_common(who, T, topk, E, H, I, bm, cap);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && w13 && w2 && topk_weights && topk_ids && out && (!FP8 || (w13_s && w2_s)),
                "%s: null pointer", who);
  const MoeWs L = moe_layout(T, topk, E, H, I, bm, FP8);
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
  float* a2s = FP8 ? reinterpret_cast<float*>(ws + L.a2s) : nullptr;
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  float* scratch = reinterpret_cast<float*>(ws + L.scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int numel = static_cast<int>(T * topk);
  const int h = static_cast<int>(H), i = static_cast<int>(I), t = static_cast<int>(T);

  const uint8_t* xa = static_cast<const uint8_t*>(x);
  const float* xs = nullptr;
  if constexpr (FP8) {
    uint8_t* xq = ws + L.xq;
    float* xsw = reinterpret_cast<float*>(ws + L.xs);
    rc = vmamd_per_token_group_quant_fp8(x, kBF16, T, H, H, 128, 1e-10f, -448.f, 448.f, xq, xsw,
                                         H / 128, 1, stream);
    if (rc) return rc;
    xa = xq;
    xs = xsw;
  }
  rc = vmamd_moe_align_block_size(topk_ids, numel, E, bm, expert_map, expert_map_len, sorted, cap,
                                  eids, ntpp, offs, nullptr, active, nact, stream);
  if (rc) return rc;
  rc = launch_w13<FP8>(xa, xs, t, h, topk, sorted, cap, bm, offs, ntpp, active, nact,
                       static_cast<const uint8_t*>(w13), w13_s, E, i, swiglu_limit, a2, a2s, scratch,
                       st);
  if (rc) return rc;
  rc = launch_w2<FP8>(a2, a2s, t, topk, sorted, cap, bm, offs, ntpp, active, nact,
                      static_cast<const uint8_t*>(w2), w2_s, E, h, i, topk_weights, topk_ids,
                      expert_map, expert_map_len, y, scratch, st);
  if (rc) return rc;
  // Slots of dropped routes (negative ids, or non-local experts) hold no
  // expert output and are skipped by the combine.
  return vmamd_moe_sum(y, kBF16, T, topk, H, topk_ids, expert_map, expert_map_len, out, stream);
}

template <bool FP8>
static int stage_w13(const char* who, const void* xa, const float* xs, int64_t T, int64_t H, int topk,
                     const int32_t* sorted, int64_t capacity, int block_m, const int32_t* offs,
                     const int32_t* ntpp, const int32_t* active, const int32_t* nact,
                     const void* w13, const float* w13_s, int E, int64_t I, float limit, void* a2,
                     float* a2s, void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common(who, T, topk, E, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(xa && sorted && offs && ntpp && w13 && a2 && (!FP8 || (xs && w13_s && a2s)),
                "%s: null pointer", who);
  VMAMD_REQUIRE(block_m == kMoeBM || (active && nact),
                "%s: the decode path (block_m 16) needs active_experts / num_active", who);
  const size_t need = w13_scratch(T * topk, E, H, I, block_m, FP8 ? 1 : 2);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(xa) % 16 == 0 && reinterpret_cast<uintptr_t>(a2) % 16 == 0,
                "%s: activations, a2 and workspace must be 16-byte aligned", who);
  return launch_w13<FP8>(static_cast<const uint8_t*>(xa), xs, static_cast<int>(T), static_cast<int>(H),
                         topk, sorted, capacity, block_m, offs, ntpp, active, nact,
                         static_cast<const uint8_t*>(w13), w13_s, E, static_cast<int>(I), limit,
                         static_cast<uint8_t*>(a2), a2s, static_cast<float*>(workspace),
                         reinterpret_cast<hipStream_t>(stream));
}

template <bool FP8>
static int stage_w2(const char* who, const void* a2, const float* a2s, int64_t T, int topk,
                    const int32_t* sorted, int64_t capacity, int block_m, const int32_t* offs,
                    const int32_t* ntpp, const int32_t* active, const int32_t* nact, const void* w2,
                    const float* w2_s, int E, int64_t H, int64_t I, const float* topk_weights,
                    const int32_t* topk_ids, const int32_t* emap, int64_t emap_len, void* y,
                    void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common(who, T, topk, E, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(a2 && sorted && offs && ntpp && w2 && topk_ids && y && (!FP8 || (a2s && w2_s)),
                "%s: null pointer", who);
  VMAMD_REQUIRE(block_m == kMoeBM || (active && nact),
                "%s: the decode path (block_m 16) needs active_experts / num_active", who);
  const size_t need = w2_scratch(T * topk, E, H, I, block_m, FP8 ? 1 : 2);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "%s: workspace of %zu bytes required (got %zu)", who, need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a2) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0,
                "%s: a2 and workspace must be 16-byte and y 8-byte aligned", who);
  return launch_w2<FP8>(static_cast<const uint8_t*>(a2), a2s, static_cast<int>(T), topk, sorted,
                        capacity, block_m, offs, ntpp, active, nact, static_cast<const uint8_t*>(w2),
                        w2_s, E, static_cast<int>(H), static_cast<int>(I), topk_weights, topk_ids,
                        emap, emap_len, static_cast<uint16_t*>(y), static_cast<float*>(workspace),
                        reinterpret_cast<hipStream_t>(stream));
}

}  // namespace vmamd

using namespace vmamd;

// ------------------------------------------------------------------ fp8 ---
extern "C" size_t vmamd_moe_fp8_stage_workspace_size(int64_t T, int topk, int num_experts,
                                                     int64_t H, int64_t I, int block_m) {
  return stage_scratch(T * topk, num_experts, H, I, block_m, 1);
}

extern "C" int vmamd_moe_fp8_w13(const void* xq, const float* xs, int64_t T, int64_t H, int topk,
                                 const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                 const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                 const int32_t* active_experts, const int32_t* num_active,
                                 const void* w13, const float* w13_s, int num_experts, int64_t I,
                                 float swiglu_limit, void* a2q, float* a2s, void* workspace,
                                 size_t workspace_bytes, vmamd_stream_t stream) {
  return stage_w13<true>("moe_fp8_w13", xq, xs, T, H, topk, sorted_token_ids, capacity, block_m,
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
  return stage_w2<true>("moe_fp8_w2", a2q, a2s, T, topk, sorted_token_ids, capacity, block_m,
                        expert_offsets, num_tokens_post_pad, active_experts, num_active, w2, w2_s,
                        num_experts, H, I, topk_weights, topk_ids, expert_map, expert_map_len, y,
                        workspace, workspace_bytes, stream);
}

extern "C" size_t vmamd_fused_moe_fp8_workspace_size(int64_t T, int topk, int num_experts,
                                                     int64_t H, int64_t I, int path) {
  return moe_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path), true).total;
}

extern "C" int vmamd_fused_moe_fp8(const void* x, int x_dtype, int64_t T, int64_t H,
                                   const void* w13, const float* w13_s, const void* w2,
                                   const float* w2_s, int num_experts, int64_t I,
                                   const float* topk_weights, const int32_t* topk_ids, int topk,
                                   const int32_t* expert_map, int64_t expert_map_len,
                                   float swiglu_limit, int path, void* out, void* workspace,
                                   size_t workspace_bytes, vmamd_stream_t stream) {
  VMAMD_REQUIRE(x_dtype == kBF16, "fused_moe_fp8: hidden states must be bf16");
  return fused_layer<true>("fused_moe_fp8", x, T, H, w13, w13_s, w2, w2_s, num_experts, I,
                           topk_weights, topk_ids, topk, expert_map, expert_map_len, swiglu_limit,
                           path, out, workspace, workspace_bytes, stream);
}

// ----------------------------------------------------------------- bf16 ---
extern "C" size_t vmamd_moe_bf16_stage_workspace_size(int64_t T, int topk, int num_experts,
                                                      int64_t H, int64_t I, int block_m) {
  return stage_scratch(T * topk, num_experts, H, I, block_m, 2);
}

extern "C" int vmamd_moe_bf16_w13(const void* x, int64_t T, int64_t H, int topk,
                                  const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                  const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                  const int32_t* active_experts, const int32_t* num_active,
                                  const void* w13, int num_experts, int64_t I, float swiglu_limit,
                                  void* a2, void* workspace, size_t workspace_bytes,
                                  vmamd_stream_t stream) {
  return stage_w13<false>("moe_bf16_w13", x, nullptr, T, H, topk, sorted_token_ids, capacity,
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
  return stage_w2<false>("moe_bf16_w2", a2, nullptr, T, topk, sorted_token_ids, capacity, block_m,
                         expert_offsets, num_tokens_post_pad, active_experts, num_active, w2, nullptr,
                         num_experts, H, I, topk_weights, topk_ids, expert_map, expert_map_len, y,
                         workspace, workspace_bytes, stream);
}

extern "C" size_t vmamd_fused_moe_bf16_workspace_size(int64_t T, int topk, int num_experts,
                                                      int64_t H, int64_t I, int path) {
  return moe_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path), false).total;
}

extern "C" int vmamd_fused_moe_bf16(const void* x, int64_t T, int64_t H, const void* w13,
                                    const void* w2, int num_experts, int64_t I,
                                    const float* topk_weights, const int32_t* topk_ids, int topk,
                                    const int32_t* expert_map, int64_t expert_map_len,
                                    float swiglu_limit, int path, void* out, void* workspace,
                                    size_t workspace_bytes, vmamd_stream_t stream) {
  return fused_layer<false>("fused_moe_bf16", x, T, H, w13, nullptr, w2, nullptr, num_experts, I,
                            topk_weights, topk_ids, topk, expert_map, expert_map_len, swiglu_limit,
                            path, out, workspace, workspace_bytes, stream);
}
