// Fused-MoE expert GEMMs for 128x128 block-fp8 weights (W13 gate/up, W2 down).
//
// Layouts (row-major):
//   xq  [T, H] e4m3, xs [T, H/128] f32        (1x128 activation groups)
//   w13 [E, 2I, H] e4m3, w13_s [E, 2I/128, H/128]; rows [0, I) gate, [I, 2I) up
//   w2  [E, H, I] e4m3, w2_s [E, H/128, I/128]
//   routes r = t * topk + k; sorted/offsets/active come from moe_align_block_size
//
// Decode path (few routes per expert): moe_gemv_fp8_kernel.  A wave owns 16
// weight rows of one active expert and a K range; it streams the rows from
// HBM once (no LDS) and applies each 16x128 fragment to every 16-route block
// of that expert.  W13 writes fp32 split-K partials per route; a second
// kernel (moe_act_quant_kernel) sums them in a fixed order, rounds to bf16,
// applies SiLU-and-mul and quantises a2 per 1x128 group.  W2 writes
// bf16(acc * routed weight) per route (or fp32 partials when split).
//
// Prefill path (many routes per expert): grouped MFMA GEMMs over 128-route
// blocks.  Tiles are ordered expert-major -- all blocks of one (expert,
// n-tile) are consecutive -- and each XCD takes a contiguous tile range, so
// the blocks of an expert that share a weight tile run together on one XCD
// and the tile is fetched from HBM once.  W13 covers 128 gate + 128 up rows
// per tile (interleaved by 16 so each lane holds matching gate/up values) and
// fuses SiLU-and-mul and the a2 quantiser into its epilogue.
#include <algorithm>

#include "mfma_fp8.h"

namespace vmamd {

// --------------------------------------------------------------- helpers --
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// SiLU-and-mul on bf16-materialised gate/up; limit > 0 applies the clamped
// variant (gate <= L, up in [-L, L], sigmoid / silu / product each rounded to
// bf16).  Returns the bf16-rounded activation, or NaN for the clamped
// variant's exceptional inputs (quantised to fp8_min by the caller).
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

// ---------------------------------------------------------- decode GEMV ---
constexpr int kMoeGemvWaves = 4;
constexpr int kGemvBlock = 16;  // routes per block (one MFMA column tile)

template <int MAXB>
__global__ __launch_bounds__(kMoeGemvWaves * kWave) void moe_gemv_fp8_kernel(
    const uint8_t* __restrict__ act, const float* __restrict__ act_s, int act_div, int K,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ active, const int32_t* __restrict__ num_active,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N, int numel, int splits,
    float* __restrict__ partial, const float* __restrict__ route_w, uint16_t* __restrict__ y) {
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
  const int KB = K / 128, NB = (N + 127) / 128;
  const int kb0 = split * KB / splits, kb1 = (split + 1) * KB / splits;
  const uint8_t* wrow = w + (static_cast<int64_t>(e) * N + ntile * 16 + li) * K;
  const float* wsr = ws + (static_cast<int64_t>(e) * NB + (ntile * 16) / 128) * KB;
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
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
      arow[b] = act + row * K;
      asr[b] = act_s + row * KB;
    }
    v4f acc[MAXB];
#pragma unroll
    for (int b = 0; b < MAXB; ++b) acc[b] = zero;

    constexpr int U = 4;
    int kb = kb0;
    for (; kb + U <= kb1; kb += U) {
      v8i wf[U];
      float sb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        wf[u] = global_frag(wrow + (kb + u) * 128, lg);
        sb[u] = wsr[kb + u];
      }
#pragma unroll
      for (int b = 0; b < MAXB; ++b) {
        if (b < nb) {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const v8i xf = global_frag(arow[b] + (kb + u) * 128, lg);
            fma4(acc[b], mfma_fp8(wf[u], xf, zero), asr[b][kb + u] * sb[u]);
          }
        }
      }
    }
    for (; kb < kb1; ++kb) {
      const v8i wf = global_frag(wrow + kb * 128, lg);
      const float sb = wsr[kb];
#pragma unroll
      for (int b = 0; b < MAXB; ++b)
        if (b < nb) fma4(acc[b], mfma_fp8(wf, global_frag(arow[b] + kb * 128, lg), zero), asr[b][kb] * sb);
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

// Sum W13 split partials (fixed order), round gate/up to bf16, SiLU-and-mul,
// quantise a2 per 1x128 group: one 16-lane segment per group, 8 columns per lane.
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
  const int64_t plane = static_cast<int64_t>(numel) * 2 * I;
  const float* src = partial + static_cast<int64_t>(r) * 2 * I + c0;
  float v[8];
  float amax = 1e-10f;
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
#pragma unroll
  for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
  amax = group_max<16>(amax);
  const float scale = amax / 448.0f;
  if (sub == 0) a2s[static_cast<int64_t>(r) * gpr + c0 / 128] = scale;
  float q[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) q[j] = fminf(fmaxf(v[j] / scale, -448.0f), 448.0f);
  uint2 out;
  out.x = f32x4_to_fp8x4(q[0], q[1], q[2], q[3]);
  out.y = f32x4_to_fp8x4(q[4], q[5], q[6], q[7]);
  *reinterpret_cast<uint2*>(a2q + static_cast<int64_t>(r) * I + c0) = out;
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

__global__ __launch_bounds__(kW13Threads, 1) void moe_w13_gemm_fp8_kernel(
    const uint8_t* __restrict__ xq, const float* __restrict__ xs, int topk, int H,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w13, const float* __restrict__ w13s, int I, float limit,
    uint8_t* __restrict__ a2q, float* __restrict__ a2s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
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
  const int KB = H / 128;
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
    goff_a[c] = (aval[c] ? static_cast<int64_t>(r / topk) * H : 0) + cch * 16;
  }
  int64_t goff_b[BCH];
#pragma unroll
  for (int c = 0; c < BCH; ++c) {
    const int j = crow + c * RSTEP, p = j / 32, q = j % 32;
    const int row = q < 16 ? n0 + 16 * p + q : I + n0 + 16 * p + (q - 16);
    goff_b[c] = (static_cast<int64_t>(e) * 2 * I + row) * H + cch * 16;
  }
  const float* xs_row[MT];
  bool tval[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = sorted[mb * BM + wm * WTM + mt * 16 + li];
    tval[mt] = r < numel;
    xs_row[mt] = xs + (tval[mt] ? static_cast<int64_t>(r / topk) * KB : 0);
  }
  const float* sg = w13s + (static_cast<int64_t>(e) * NB2 + n0 / 128) * KB;
  const float* su = w13s + (static_cast<int64_t>(e) * NB2 + (I + n0) / 128) * KB;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  const v4i z4 = {0, 0, 0, 0};
  v4i ra[ACH], rb[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const v4i v = ld16(xq + goff_a[c]);
    ra[c] = aval[c] ? v : z4;
  }
#pragma unroll
  for (int c = 0; c < BCH; ++c) rb[c] = ld16(w13 + goff_b[c]);
#pragma unroll
  for (int c = 0; c < ACH; ++c) st16(&smem_dyn[l0 + c * RSTEP * 128], ra[c]);
#pragma unroll
  for (int c = 0; c < BCH; ++c) st16(&smem_dyn[BM * 128 + l0 + c * RSTEP * 128], rb[c]);
  float sa[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = tval[mt] ? xs_row[mt][0] : 0.f;
  float sbg = sg[0], sbu = su[0];
  __syncthreads();

  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < KB; ++kb) {
    const int cur = kb & 1;
    // Prefetch K-block kb+1 (the last iteration re-reads block KB-1 into the
    // idle buffer; that copy is never used).
    const int kn = min(kb + 1, KB - 1);
    const int off = kn * 128;
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      const v4i v = ld16(xq + goff_a[c] + off);
      ra[c] = aval[c] ? v : z4;
    }
#pragma unroll
    for (int c = 0; c < BCH; ++c) rb[c] = ld16(w13 + goff_b[c] + off);
    float san[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float v = xs_row[mt][kn];
      san[mt] = tval[mt] ? v : 0.f;
    }
    const float sbgn = sg[kn], sbun = su[kn];

    const uint8_t* tile = smem_dyn + cur * STAGE;
    v8i xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt] = lds_frag(tile, wm * WTM + mt * 16 + li, lg);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const v8i wf = lds_frag(tile + BM * 128, wn * WTN + nt * 16 + li, lg);
      const float sb = (nt & 1) ? sbu : sbg;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) fma4(acc[mt][nt], mfma_fp8(wf, xf[mt], zero), sa[mt] * sb);
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
      for (int r = 0; r < 4; ++r) o[r] = fminf(fmaxf(v[mt][q][r] / scale, -448.0f), 448.0f);
      const int col = n0 + (wn * 2 + q) * 16 + 4 * lg;
      *reinterpret_cast<uint32_t*>(a2q + row * I + col) = f32x4_to_fp8x4(o[0], o[1], o[2], o[3]);
    }
  }
}

// W2: tile = 128 routes x 128 hidden rows, 4 waves as 2 x 2, K = I.
__global__ __launch_bounds__(256, 2) void moe_w2_gemm_fp8_kernel(
    const uint8_t* __restrict__ a2q, const float* __restrict__ a2s, int I,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ ntpp, int E, int numel, int max_tiles,
    const uint8_t* __restrict__ w2, const float* __restrict__ w2s, int H,
    const float* __restrict__ route_w, uint16_t* __restrict__ y) {
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
  const int KB = I / 128;
  const int NBH = (H + 127) / 128;

  const int crow = tid / 8, cch = tid % 8;
  const int l0 = lds_off(crow, cch);
  int64_t goff_a[ACH], goff_b[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c)
    goff_a[c] = (static_cast<int64_t>(mb) * BM + crow + c * RSTEP) * I + cch * 16;
#pragma unroll
  for (int c = 0; c < BCH; ++c)
    goff_b[c] = (static_cast<int64_t>(e) * H + min(n0 + crow + c * RSTEP, H - 1)) * I + cch * 16;
  const float* sb_p = w2s + (static_cast<int64_t>(e) * NBH + n0 / 128) * KB;
  const int64_t arow0 = static_cast<int64_t>(mb) * BM + wm * WTM + li;

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  v4i ra[ACH], rb[BCH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) ra[c] = ld16(a2q + goff_a[c]);
#pragma unroll
  for (int c = 0; c < BCH; ++c) rb[c] = ld16(w2 + goff_b[c]);
#pragma unroll
  for (int c = 0; c < ACH; ++c) st16(&smem[0][l0 + c * RSTEP * 128], ra[c]);
#pragma unroll
  for (int c = 0; c < BCH; ++c) st16(&smem[0][BM * 128 + l0 + c * RSTEP * 128], rb[c]);
  float sa[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) sa[mt] = a2s[(arow0 + mt * 16) * KB];
  float sb = sb_p[0];
  __syncthreads();

  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < KB; ++kb) {
    const int cur = kb & 1;
    const int kn = min(kb + 1, KB - 1);
    const int off = kn * 128;
#pragma unroll
    for (int c = 0; c < ACH; ++c) ra[c] = ld16(a2q + goff_a[c] + off);
#pragma unroll
    for (int c = 0; c < BCH; ++c) rb[c] = ld16(w2 + goff_b[c] + off);
    float san[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) san[mt] = a2s[(arow0 + mt * 16) * KB + kn];
    const float sbn = sb_p[kn];
    const uint8_t* tile = smem[cur];
    v8i xf[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xf[mt] = lds_frag(tile, wm * WTM + mt * 16 + li, lg);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const v8i wf = lds_frag(tile + BM * 128, wn * WTN + nt * 16 + li, lg);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) fma4(acc[mt][nt], mfma_fp8(wf, xf[mt], zero), sa[mt] * sb);
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
// (>= 4096 over the active experts' n-tiles), at least 4 K-blocks per split.
static int moe_splits(int64_t waves_per_split, int KB) {
  int s = static_cast<int>((4096 + waves_per_split - 1) / waves_per_split);
  return max(1, min(s, max(1, KB / 4)));
}

static int64_t moe_umax(int64_t numel, int E) { return std::min<int64_t>(E, numel); }

static int w13_splits(int64_t numel, int E, int64_t H, int64_t I) {
  return moe_splits(moe_umax(numel, E) * (2 * I / 16), static_cast<int>(H / 128));
}
static int w2_splits(int64_t numel, int E, int64_t H, int64_t I) {
  return moe_splits(moe_umax(numel, E) * (H / 16), static_cast<int>(I / 128));
}

static size_t al256(size_t x) { return (x + 255) / 256 * 256; }

// Stage scratch: fp32 split-K partials of the decode GEMVs (none for GEMMs).
static size_t w13_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m) {
  if (block_m != kGemvBlock) return 0;
  return al256(static_cast<size_t>(w13_splits(numel, E, H, I)) * numel * 2 * I * 4);
}
static size_t w2_scratch(int64_t numel, int E, int64_t H, int64_t I, int block_m) {
  if (block_m != kGemvBlock) return 0;
  const int s = w2_splits(numel, E, H, I);
  return s > 1 ? al256(static_cast<size_t>(s) * numel * H * 4) : 0;
}

static bool g_w13_lds_raised = false;

// Launches of the two stages; arguments are validated by the callers.
static int launch_w13(const uint8_t* xq, const float* xs, int T, int H, int topk, const int32_t* sorted,
                      int64_t cap, int block_m, const int32_t* offs, const int32_t* ntpp,
                      const int32_t* active, const int32_t* nact, const uint8_t* w13,
                      const float* w13_s, int E, int I, float limit, uint8_t* a2q, float* a2s,
                      float* scratch, hipStream_t st) {
  const int numel = T * topk;
  if (block_m == kGemvBlock) {
    const int s13 = w13_splits(numel, E, H, I);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g13((2 * I / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s13);
    moe_gemv_fp8_kernel<4><<<g13, kMoeGemvWaves * kWave, 0, st>>>(
        xq, xs, topk, H, sorted, offs, active, nact, w13, w13_s, 2 * I, numel, s13, scratch,
        nullptr, nullptr);
    int rc = check_launch("moe_fp8_w13(gemv)");
    if (rc) return rc;
    const int64_t groups = static_cast<int64_t>(numel) * (I / 128);
    moe_act_quant_kernel<<<static_cast<int>((groups + 15) / 16), 256, 0, st>>>(scratch, s13, numel, I,
                                                                               limit, a2q, a2s);
    return check_launch("moe_fp8_w13(act quant)");
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  const int tiles = max_blocks * (I / 128);
  if (!g_w13_lds_raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(moe_w13_gemm_fp8_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kW13Lds) != hipSuccess) {
      set_error("moe_fp8_w13: cannot raise the LDS limit of the W13 kernel");
      return VMAMD_ERR_HIP;
    }
    g_w13_lds_raised = true;
  }
  moe_w13_gemm_fp8_kernel<<<xcd_grid(tiles), kW13Threads, kW13Lds, st>>>(
      xq, xs, topk, H, sorted, offs, ntpp, E, numel, tiles, w13, w13_s, I, limit, a2q, a2s);
  return check_launch("moe_fp8_w13(gemm)");
}

static int launch_w2(const uint8_t* a2q, const float* a2s, int T, int topk, const int32_t* sorted,
                     int64_t cap, int block_m, const int32_t* offs, const int32_t* ntpp,
                     const int32_t* active, const int32_t* nact, const uint8_t* w2, const float* w2_s,
                     int E, int H, int I, const float* topk_weights, const int32_t* topk_ids,
                     const int32_t* emap, int64_t emap_len, uint16_t* y, float* scratch,
                     hipStream_t st) {
  const int numel = T * topk;
  if (block_m == kGemvBlock) {
    const int s2 = w2_splits(numel, E, H, I);
    const int umax = static_cast<int>(moe_umax(numel, E));
    dim3 g2((H / 16 + kMoeGemvWaves - 1) / kMoeGemvWaves, umax, s2);
    if (s2 == 1) {
      moe_gemv_fp8_kernel<4><<<g2, kMoeGemvWaves * kWave, 0, st>>>(
          a2q, a2s, 1, I, sorted, offs, active, nact, w2, w2_s, H, numel, 1, nullptr, topk_weights, y);
      return check_launch("moe_fp8_w2(gemv)");
    }
    moe_gemv_fp8_kernel<4><<<g2, kMoeGemvWaves * kWave, 0, st>>>(
        a2q, a2s, 1, I, sorted, offs, active, nact, w2, w2_s, H, numel, s2, scratch, nullptr, nullptr);
    int rc = check_launch("moe_fp8_w2(gemv)");
    if (rc) return rc;
    const int64_t mn = static_cast<int64_t>(numel) * H;
    moe_w2_reduce_kernel<<<static_cast<int>((mn / 4 + 255) / 256), 256, 0, st>>>(
        scratch, s2, numel, H, topk_ids, emap, emap_len, topk_weights, y);
    return check_launch("moe_fp8_w2(reduce)");
  }
  const int max_blocks = static_cast<int>((cap + kMoeBM - 1) / kMoeBM);
  const int tiles = max_blocks * ((H + 127) / 128);
  moe_w2_gemm_fp8_kernel<<<xcd_grid(tiles), 256, 0, st>>>(a2q, a2s, I, sorted, offs, ntpp, E, numel,
                                                          tiles, w2, w2_s, H, topk_weights, y);
  return check_launch("moe_fp8_w2(gemm)");
}

// Workspace carve-up of the fused layer, shared by the size query and the
// launcher.  The two stages run one after the other on one stream, so their
// scratch shares one region.
struct MoeFp8Ws {
  size_t xq, xs, sorted, eids, ntpp, offs, active, nact, a2q, a2s, y, scratch, total;
};

static MoeFp8Ws moe_fp8_layout(int64_t T, int topk, int E, int64_t H, int64_t I, int bm) {
  MoeFp8Ws w{};
  const int64_t numel = T * topk;
  const int64_t cap = numel + static_cast<int64_t>(E) * (bm - 1);
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o += al256(bytes); return at; };
  w.xq = take(T * H);
  w.xs = take(T * (H / 128) * 4);
  w.sorted = take(cap * 4);
  w.eids = take(((cap + bm - 1) / bm) * 4);
  w.ntpp = take(4);
  w.offs = take((E + 1) * 4);
  w.active = take(E * 4);
  w.nact = take(4);
  const int64_t arows = bm == kGemvBlock ? numel : cap;  // route order (decode) or padded order
  w.a2q = take(arows * I);
  w.a2s = take(arows * (I / 128) * 4);
  w.y = take(numel * H * 2);
  w.scratch = take(std::max(w13_scratch(numel, E, H, I, bm), w2_scratch(numel, E, H, I, bm)));
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

}  // namespace vmamd

using namespace vmamd;

extern "C" size_t vmamd_moe_fp8_stage_workspace_size(int64_t T, int topk, int num_experts,
                                                     int64_t H, int64_t I, int block_m) {
  const int64_t numel = T * topk;
  return std::max(w13_scratch(numel, num_experts, H, I, block_m),
                  w2_scratch(numel, num_experts, H, I, block_m));
}

extern "C" int vmamd_moe_fp8_w13(const void* xq, const float* xs, int64_t T, int64_t H, int topk,
                                 const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                 const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                 const int32_t* active_experts, const int32_t* num_active,
                                 const void* w13, const float* w13_s, int num_experts, int64_t I,
                                 float swiglu_limit, void* a2q, float* a2s, void* workspace,
                                 size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common("moe_fp8_w13", T, topk, num_experts, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(xq && xs && sorted_token_ids && expert_offsets && num_tokens_post_pad && w13 &&
                    w13_s && a2q && a2s,
                "moe_fp8_w13: null pointer");
  VMAMD_REQUIRE(block_m == kMoeBM || (active_experts && num_active),
                "moe_fp8_w13: the decode path (block_m 16) needs active_experts / num_active");
  const size_t need = w13_scratch(T * topk, num_experts, H, I, block_m);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "moe_fp8_w13: workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(xq) % 16 == 0 && reinterpret_cast<uintptr_t>(a2q) % 16 == 0,
                "moe_fp8_w13: xq, a2q and workspace must be 16-byte aligned");
  return launch_w13(static_cast<const uint8_t*>(xq), xs, static_cast<int>(T), static_cast<int>(H), topk,
                    sorted_token_ids, capacity, block_m, expert_offsets, num_tokens_post_pad,
                    active_experts, num_active, static_cast<const uint8_t*>(w13), w13_s, num_experts,
                    static_cast<int>(I), swiglu_limit, static_cast<uint8_t*>(a2q), a2s,
                    static_cast<float*>(workspace), reinterpret_cast<hipStream_t>(stream));
}

extern "C" int vmamd_moe_fp8_w2(const void* a2q, const float* a2s, int64_t T, int topk,
                                const int32_t* sorted_token_ids, int64_t capacity, int block_m,
                                const int32_t* expert_offsets, const int32_t* num_tokens_post_pad,
                                const int32_t* active_experts, const int32_t* num_active,
                                const void* w2, const float* w2_s, int num_experts, int64_t H,
                                int64_t I, const float* topk_weights, const int32_t* topk_ids,
                                const int32_t* expert_map, int64_t expert_map_len, void* y,
                                void* workspace, size_t workspace_bytes, vmamd_stream_t stream) {
  int rc = check_stage_common("moe_fp8_w2", T, topk, num_experts, H, I, block_m, capacity);
  if (rc) return rc;
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(a2q && a2s && sorted_token_ids && expert_offsets && num_tokens_post_pad && w2 &&
                    w2_s && topk_ids && y,
                "moe_fp8_w2: null pointer");
  VMAMD_REQUIRE(block_m == kMoeBM || (active_experts && num_active),
                "moe_fp8_w2: the decode path (block_m 16) needs active_experts / num_active");
  const size_t need = w2_scratch(T * topk, num_experts, H, I, block_m);
  VMAMD_REQUIRE(workspace_bytes >= need && (need == 0 || workspace),
                "moe_fp8_w2: workspace of %zu bytes required (got %zu)", need, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a2q) % 16 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0,
                "moe_fp8_w2: a2q and workspace must be 16-byte and y 8-byte aligned");
  return launch_w2(static_cast<const uint8_t*>(a2q), a2s, static_cast<int>(T), topk, sorted_token_ids,
                   capacity, block_m, expert_offsets, num_tokens_post_pad, active_experts, num_active,
                   static_cast<const uint8_t*>(w2), w2_s, num_experts, static_cast<int>(H),
                   static_cast<int>(I), topk_weights, topk_ids, expert_map, expert_map_len,
                   static_cast<uint16_t*>(y), static_cast<float*>(workspace),
                   reinterpret_cast<hipStream_t>(stream));
}

extern "C" size_t vmamd_fused_moe_fp8_workspace_size(int64_t T, int topk, int num_experts,
                                                     int64_t H, int64_t I, int path) {
  return moe_fp8_layout(T, topk, num_experts, H, I, moe_block_m(T, topk, num_experts, path)).total;
}

extern "C" int vmamd_fused_moe_fp8(const void* x, int x_dtype, int64_t T, int64_t H,
                                   const void* w13, const float* w13_s, const void* w2,
                                   const float* w2_s, int num_experts, int64_t I,
                                   const float* topk_weights, const int32_t* topk_ids, int topk,
                                   const int32_t* expert_map, int64_t expert_map_len,
                                   float swiglu_limit, int path, void* out, void* workspace,
                                   size_t workspace_bytes, vmamd_stream_t stream) {
  VMAMD_REQUIRE(path >= VMAMD_MOE_PATH_AUTO && path <= VMAMD_MOE_PATH_GEMM,
                "fused_moe_fp8: unknown path %d", path);
  const int bm = moe_block_m(T, topk, num_experts, path);
  const int64_t cap = T * topk + static_cast<int64_t>(num_experts) * (bm - 1);
  int rc = check_stage_common("fused_moe_fp8", T, topk, num_experts, H, I, bm, cap);
  if (rc) return rc;
  VMAMD_REQUIRE(x_dtype == kBF16, "fused_moe_fp8: hidden states must be bf16");
  if (T == 0) return VMAMD_OK;
  VMAMD_REQUIRE(x && w13 && w13_s && w2 && w2_s && topk_weights && topk_ids && out,
                "fused_moe_fp8: null pointer");
  const MoeFp8Ws L = moe_fp8_layout(T, topk, num_experts, H, I, bm);
  VMAMD_REQUIRE(workspace && workspace_bytes >= L.total,
                "fused_moe_fp8: workspace of %zu bytes required (got %zu)", L.total, workspace_bytes);
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0,
                "fused_moe_fp8: workspace must be 256-byte aligned");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint8_t* xq = ws + L.xq;
  float* xs = reinterpret_cast<float*>(ws + L.xs);
  int32_t* sorted = reinterpret_cast<int32_t*>(ws + L.sorted);
  int32_t* eids = reinterpret_cast<int32_t*>(ws + L.eids);
  int32_t* ntpp = reinterpret_cast<int32_t*>(ws + L.ntpp);
  int32_t* offs = reinterpret_cast<int32_t*>(ws + L.offs);
  int32_t* active = reinterpret_cast<int32_t*>(ws + L.active);
  int32_t* nact = reinterpret_cast<int32_t*>(ws + L.nact);
  uint8_t* a2q = ws + L.a2q;
  float* a2s = reinterpret_cast<float*>(ws + L.a2s);
  uint16_t* y = reinterpret_cast<uint16_t*>(ws + L.y);
  float* scratch = reinterpret_cast<float*>(ws + L.scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int numel = static_cast<int>(T * topk);
  const int h = static_cast<int>(H), i = static_cast<int>(I), t = static_cast<int>(T);

  rc = vmamd_per_token_group_quant_fp8(x, kBF16, T, H, H, 128, 1e-10f, -448.f, 448.f, xq, xs,
                                       H / 128, 1, stream);
  if (rc) return rc;
  rc = vmamd_moe_align_block_size(topk_ids, numel, num_experts, bm, expert_map, expert_map_len,
                                  sorted, cap, eids, ntpp, offs, nullptr, active, nact, stream);
  if (rc) return rc;
  rc = launch_w13(xq, xs, t, h, topk, sorted, cap, bm, offs, ntpp, active, nact,
                  static_cast<const uint8_t*>(w13), w13_s, num_experts, i, swiglu_limit, a2q, a2s,
                  scratch, st);
  if (rc) return rc;
  rc = launch_w2(a2q, a2s, t, topk, sorted, cap, bm, offs, ntpp, active, nact,
                 static_cast<const uint8_t*>(w2), w2_s, num_experts, h, i, topk_weights, topk_ids,
                 expert_map, expert_map_len, y, scratch, st);
  if (rc) return rc;
  // Slots of dropped routes (negative ids, or non-local experts) hold no
  // expert output and are skipped by the combine.
  return vmamd_moe_sum(y, kBF16, T, topk, H, topk_ids, expert_map, expert_map_len, out, stream);
}
