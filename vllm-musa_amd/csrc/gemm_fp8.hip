// Dense w8a8 block-fp8 GEMM:  C[M,N] = bf16( sum_kb (A_kb . B_kb^T) * As[m,kb] * Bs[n/128,kb] )
//   A  [M, K] e4m3 (1x128 activation groups, scales As[m*as_sm + kb*as_sk])
//   B  [N, K] e4m3 (128x128 weight blocks, scales Bs[ceil(N/128), K/128])
//
// Three kernels:
//  * gemm_fp8_dma_kernel -- 128 x 256 workgroup tile, 8 waves, K-block of 128
//    per step, 3-stage LDS ring fed by direct global->LDS loads (one barrier
//    per K-block), XCD-aware tile order, optional split K.  For M > 64.
//  * gemm_fp8_big_kernel -- 256 x 256 tile, 2 LDS stages, for large M where
//    it needs fewer rounds of workgroups (fewer bytes moved per flop).
//  * gemv_fp8_bs_kernel  -- decode-sized M (<= 64): one workgroup per NT x 16
//    weight rows, its waves split K and stream the rows straight from HBM
//    into registers; each 16x128 weight fragment multiplies every 16-row
//    activation tile and each activation fragment the NT weight tiles, so
//    weights are read exactly once and activations once per NT x 16 rows.
//    The waves' partial sums meet in LDS and are added in wave order
//    (deterministic), one rounding, in the same kernel.
#include "mfma_fp8.h"
#include "tile_pipe.h"

#include <atomic>
#include <mutex>

namespace vmamd {

// ------------------------------------------- tiled GEMM on the DMA ring ---
// 128 x 256 output tile per workgroup (8 waves as 2 (m) x 4 (n), 64 x 64 per
// wave), 3-stage LDS ring fed by direct global->LDS loads: two K steps are in
// flight while the current one runs on MFMA.  Rows past M / N are clamped to
// the last row (their results are not stored).  Split K: workgroup row
// blockIdx.y takes K steps [blockIdx.y * kper, +kper) and, with `partial`
// set, stores its fp32 tile at partial[blockIdx.y][M][N] for
// splitk_reduce_kernel; without it, the bf16 tile at C.
// DensePipeN: the same kernel on 128 x 128 tiles (8 waves of 64 x 32), for
// mid-size M on small N, where 128 x 256 tiles are too few for the CUs.
using DensePipe = TilePipe<true, 128, 256, 2, 4, 3>;
using DensePipeN = TilePipe<true, 128, 128, 2, 4, 3>;

template <typename P>
__global__ __launch_bounds__(P::kThreads, 1) void gemm_fp8_dma_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, int64_t as_sm, int64_t as_sk,
    const uint8_t* __restrict__ B, const float* __restrict__ Bs, uint16_t* __restrict__ C, int M,
    int N, int K, int TM, int TN, int kper, float* __restrict__ partial) {
  constexpr int NS = 3, BM = P::kBM, BN = P::kBN, WN = P::kWN;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  int tm, tn;
  if (!xcd_tile(blockIdx.x, TM, TN, tm, tn)) return;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane % 16, lg = lane / 16;
  const int KS = K / 128, NB = (N + 127) / 128;
  const int kb0 = blockIdx.y * kper, KL = min(kper, KS - kb0);  // the host keeps KL >= 1

  P p;
#pragma unroll
  for (int j = 0; j < P::kDmaA; ++j) {
    const int m = min(m0 + P::rowA(wave, lane, j), M - 1);
    p.srcA[j] = A + static_cast<int64_t>(m) * K + P::chunk(lane);
    p.ldsA[j] = (wave + j * P::kWaves) * 8 * 128;
  }
#pragma unroll
  for (int j = 0; j < P::kDmaB; ++j) {
    const int n = min(n0 + P::rowB(wave, lane, j), N - 1);
    p.srcB[j] = B + static_cast<int64_t>(n) * K + P::chunk(lane);
    p.ldsB[j] = P::kOffB + (wave + j * P::kWaves) * 8 * 128;
  }
  if (wave < BM / 64) {  // activation scales of tile rows 64*wave + lane
    const int m = min(m0 + 64 * wave + lane, M - 1);
    p.srcS = reinterpret_cast<const uint8_t*>(As + static_cast<int64_t>(m) * as_sm);
    p.stepS = static_cast<int>(as_sk * 4);
    p.ldsS = P::kOffSA + 64 * wave * 4;
  } else {  // weight-block scales of the tile's two 128-row blocks (slots 0, 1)
    const int nb = min(n0 / 128 + min(lane, 1), NB - 1);
    p.srcS = reinterpret_cast<const uint8_t*>(Bs + static_cast<int64_t>(nb) * KS);
    p.stepS = 4;
    p.ldsS = P::kOffSB;
  }
  if (kb0 > 0) {  // this split's first K step becomes step 0 of the ring
#pragma unroll
    for (int j = 0; j < P::kDmaA; ++j) p.srcA[j] += static_cast<int64_t>(kb0) * 128;
#pragma unroll
    for (int j = 0; j < P::kDmaB; ++j) p.srcB[j] += static_cast<int64_t>(kb0) * 128;
    p.srcS += static_cast<int64_t>(kb0) * p.stepS;
  }

  v4f acc[P::MT][P::NT];
#pragma unroll
  for (int mt = 0; mt < P::MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < P::NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

  // Fragments of one K step in registers; the next step's are read from LDS
  // while this step's MFMAs run.
  struct Frags {
    v8i x[P::MT], w[P::NT];
    float sa[P::MT], sb;
  };
  auto read = [&](const uint8_t* st, Frags& f) {
    f.sb = lds_load<float>(st, P::kOffSB + (wn * P::WTN / 128) * 4);  // the wave's 128-row scale block
#pragma unroll
    for (int mt = 0; mt < P::MT; ++mt) {
      f.sa[mt] = lds_load<float>(st, P::kOffSA + (wm * P::WTM + mt * 16 + li) * 4);
      f.x[mt] = lds_frag(st, wm * P::WTM + mt * 16 + li, lg);
    }
#pragma unroll
    for (int nt = 0; nt < P::NT; ++nt) f.w[nt] = lds_frag(st + P::kOffB, wn * P::WTN + nt * 16 + li, lg);
  };
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  // The per-K-block scale promotion (acc += p * sa * sb, 4 FMAs) of MFMA i-1
  // runs while MFMA i executes: products rotate through two registers, and the
  // schedule is pinned to MFMA, 4 FMAs, MFMA, ... so the matrix core is not
  // left waiting for the promotion of its own last result.
  auto mma = [&](const Frags& f) {
    constexpr int NI = P::MT * P::NT;
    float sab[P::MT];
#pragma unroll
    for (int mt = 0; mt < P::MT; ++mt) sab[mt] = f.sa[mt] * f.sb;
    v4f t[2];
#pragma unroll
    for (int i = 0; i <= NI; ++i) {
      if (i < NI) {
        t[i & 1] = mfma_fp8(f.w[i % P::NT], f.x[i / P::NT], zero);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two of the next step's LDS reads
      }
      if (i > 0) {
        const int j = i - 1;
        fma4(acc[j / P::NT][j % P::NT], t[j & 1], sab[j / P::NT]);
        __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // its predecessor's 4 FMAs
      }
    }
  };
  // Step kb: its fragments are in `cur`; buffer kb % NS (read into `cur` by
  // every wave before the barrier) is refilled with step kb + NS first, which
  // gives the DMA almost two steps to land, then step kb + 1 is read into
  // `nxt`, two LDS reads after each MFMA (refill first measured 0-2 % faster
  // than after the MFMAs at M = 512 and 4096 on the DeepSeek-V3 shapes).
  auto step = [&](int kb, const Frags& cur, Frags& nxt) {
    wait_lgkmcnt0();  // this wave's reads of the buffer refilled below are done
    wait_vmcnt<(NS - 2) * P::kIPS>();
    barrier_lds();
    p.issue(smem_dyn + (kb % NS) * P::kStage, min(kb + NS, KL - 1));
    read(smem_dyn + ((kb + 1) % NS) * P::kStage, nxt);
    mma(cur);
  };

#pragma unroll
  for (int s = 0; s < NS; ++s) p.issue(smem_dyn + s * P::kStage, min(s, KL - 1));
  wait_vmcnt<(NS - 1) * P::kIPS>();
  barrier_lds();
  Frags f0, f1;
  read(smem_dyn, f0);
  for (int kb = 0; kb < KL; kb += 2) {
    step(kb, f0, f1);
    if (kb + 1 < KL) step(kb + 1, f1, f0);
  }
  wait_vmcnt<0>();  // the ring's trailing DMAs must land before the workgroup's LDS is released

#pragma unroll
  for (int mt = 0; mt < P::MT; ++mt) {
    const int m = m0 + wm * P::WTM + mt * 16 + li;
    if (m >= M) continue;
#pragma unroll
    for (int nt = 0; nt < P::NT; ++nt) {
      const int n = n0 + wn * P::WTN + nt * 16 + 4 * lg;
      if (n >= N) continue;
      const v4f a = acc[mt][nt];
      if (partial)
        *reinterpret_cast<float4*>(partial + (static_cast<int64_t>(blockIdx.y) * M + m) * N + n) =
            float4{a[0], a[1], a[2], a[3]};
      else
        *reinterpret_cast<uint2*>(C + static_cast<int64_t>(m) * N + n) = pack_bf16x4(a[0], a[1], a[2], a[3]);
    }
  }
}

// Raw buffer loads (gfx9 descriptor: base, no stride, num_records bytes); a
// lane whose byte offset is past num_records reads zeros and fetches nothing,
// which masks rows past M and K-blocks past a split without branches.
constexpr int kGemvBufferFlags = 0x00020000;
constexpr uint32_t kGemvMasked = 0x80000000u;  // offset of a masked lane (buffers are < 2 GiB)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemv_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, kGemvBufferFlags);
}

// ------------------------------------------- 256-row tiled GEMM ---------
// For large M.  A CU's loads stream at the rate its vector cache keeps
// requests in flight (measured: the 128 x 256 kernel's DMA ring alone, with
// no MFMA, runs at the same speed as with them), so the bytes a workgroup
// moves per flop set the pace: a 256 x 256 tile moves 64 KiB per K step for
// 16.8 MFLOP, the 128 x 256 tile 48 KiB for 8.4 MFLOP.  8 waves as 4 (m) x
// 2 (n), 64 x 128 per wave (128 accumulator registers a lane; the wave's 128
// weight rows are one 128-row scale block).  Two LDS stages: the DMA of step
// kb + 1 lands while step kb runs.  Each wave reads its step's 4 activation
// fragments when the step starts and streams its 8 weight fragments, two
// register sets deep, under the MFMAs.  Rows past M / N come from the buffer
// descriptors' range check (no fetch) and are not stored.  (A 256 x 224 tile,
// which gives 7168-row weights 32 column tiles -- two full rounds of 256 CUs
// at M = 4096 instead of 1.75 -- measured 3 % slower there.)
using BigPipe = BigTile;
static_assert(BigTile::BM * 512 <= BigTile::kLds, "the bf16 output tile is staged in the stages' LDS");

// as_bytes: the extent of As in bytes (< 2 GiB); the host keeps (M + 256) K
// and (N + 256) K below 2^31.
__global__ __launch_bounds__(BigPipe::kThreads, 1) void gemm_fp8_big_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, int64_t as_sm, int64_t as_sk,
    int as_bytes, const uint8_t* __restrict__ B, const float* __restrict__ Bs, uint16_t* __restrict__ C,
    int M, int N, int K, int TM, int TN, int kper, float* __restrict__ partial, int row_store) {
  using P = BigPipe;
  constexpr int NT = P::NT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  int tm, tn;
  if (!xcd_tile(blockIdx.x, TM, TN, tm, tn)) return;
  const int m0 = tm * P::BM, n0 = tn * P::BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / P::WN, wn = wave % P::WN;
  const int li = lane % 16, lg = lane / 16;
  const int KS = K / 128, NB = (N + 127) / 128;

  // Lane L of DMA j fills LDS row (wave + 8 j) * 8 + L / 8, slot L % 8, from
  // global chunk (L % 8) ^ (L / 8) (the tile's row swizzle).
  const __amdgpu_buffer_rsrc_t ra = gemv_rsrc(A, M * K), rb = gemv_rsrc(B, N * K);
  const uint32_t chunk = static_cast<uint32_t>(((lane % 8) ^ (lane / 8)) * 16);
  const uint32_t offA = static_cast<uint32_t>(m0 + wave * 8 + lane / 8) * K + chunk;
  const uint32_t offB = static_cast<uint32_t>(n0 + wave * 8 + lane / 8) * K + chunk;
  const uint32_t rows64 = 64u * static_cast<uint32_t>(K);
  // Scales through buffer descriptors too (a global->LDS load in the loop
  // makes the compiler wait for every LDS read at once).  Waves 0-3: the
  // activation scales of tile rows 64 * wave + lane; wave 4: the weight-block
  // scales of the tile's two 128-row blocks.
  uint32_t offS, stepS;
  int ldsS;
  __amdgpu_buffer_rsrc_t rs;
  if (wave < P::BM / 64) {
    const int m = min(m0 + 64 * wave + lane, M - 1);
    rs = gemv_rsrc(As, as_bytes);
    offS = static_cast<uint32_t>((m * as_sm) * 4);
    stepS = static_cast<uint32_t>(as_sk * 4);
    ldsS = P::kOffSA + 64 * wave * 4;
  } else {
    const int nb = min(n0 / 128 + min(lane, 1), NB - 1);
    rs = gemv_rsrc(Bs, NB * KS * 4);
    offS = static_cast<uint32_t>(nb * KS * 4);
    stepS = 4;
    ldsS = P::kOffSB;
  }
  auto issue = [&](uint8_t* stage, int step) {
    const uint32_t ks = static_cast<uint32_t>(step) * 128;
#pragma unroll
    for (int j = 0; j < 4; ++j) buffer_dma16(ra, offA + ks + j * rows64, stage + (wave + 8 * j) * 8 * 128);
#pragma unroll
    for (int j = 0; j < 4; ++j) buffer_dma16(rb, offB + ks + j * rows64, stage + P::kOffB + (wave + 8 * j) * 8 * 128);
    if (wave <= P::BM / 64) buffer_dma4(rs, offS + step * stepS, stage + ldsS);
  };

  v4f acc[P::MT][NT];
#pragma unroll
  for (int mt = 0; mt < P::MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  const int nw = wn * 16 * NT;  // the wave's first weight row in the tile

  // One K step from LDS stage `st`: the MFMAs in (n tile, m tile) order, the
  // promotion of MFMA i - 1 (acc += p * sa * sb, 4 FMAs) issued after MFMA i,
  // and weight fragment nt + 1 read under the MFMAs of nt.  The order is
  // pinned (the scheduler otherwise moves each promotion next to its own
  // MFMA and waits for it).
  auto mma = [&](const uint8_t* st) {
    const float sb = lds_load<float>(st, P::kOffSB + 4 * wn);
    float sc[P::MT];
#pragma unroll
    for (int mt = 0; mt < P::MT; ++mt) sc[mt] = lds_load<float>(st, P::kOffSA + (wm * 64 + mt * 16 + li) * 4);
    v8i w[2], x[P::MT];
    w[0] = lds_frag(st + P::kOffB, nw + li, lg);
#pragma unroll
    for (int mt = 0; mt < P::MT; ++mt) x[mt] = lds_frag(st, wm * 64 + mt * 16 + li, lg);
    __builtin_amdgcn_sched_barrier(0);
    v4f t[2];
    constexpr int NI = P::MT * NT;
#pragma unroll
    for (int i = 0; i <= NI; ++i) {
      const int nt = i / P::MT, mt = i % P::MT;
      if (i < NI) {
        t[i & 1] = mfma_fp8(w[nt & 1], x[mt], zero);
        __builtin_amdgcn_sched_barrier(0);
        if (mt == 0 && nt + 1 < NT) w[(nt + 1) & 1] = lds_frag(st + P::kOffB, nw + (nt + 1) * 16 + li, lg);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (i > 0) {
        const int j = i - 1;
        if (j < P::MT) sc[j] *= sb;  // activation row scale x weight-block scale, at first use
        fma4(acc[j % P::MT][j / P::MT], t[j & 1], sc[j % P::MT]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // K steps [kb0, kb1) of split blockIdx.y (all of K without a split).
  const int kb0 = blockIdx.y * kper, kb1 = min(KS, kb0 + kper);
  issue(smem_dyn, kb0);
  wait_lgkmcnt0();
  for (int kb = kb0; kb < kb1; ++kb) {
    const int j = kb - kb0;
    wait_vmcnt<0>();  // this wave's DMAs of step kb have landed
    barrier_lds();    // ... every wave's, and step kb - 1's buffer is no longer read
    if (kb + 1 < kb1) issue(smem_dyn + ((j + 1) & 1) * P::kStage, kb + 1);
    mma(smem_dyn + (j & 1) * P::kStage);
  }

  if (row_store) {
    // bf16 C through LDS: tile row r takes 512 bytes, its 16-byte chunk c at
    // slot c ^ (r & 31); then each half-wave stores one whole 512-byte tile
    // row (the fragment stores below write 32-byte pieces of 16 rows per
    // instruction).  The host sets row_store for N % 8 == 0, a 16-byte aligned
    // C and no split.
    uint8_t* ct = smem_dyn;
    __syncthreads();  // every wave is done with the stages
#pragma unroll
    for (int mt = 0; mt < P::MT; ++mt) {
      const int row = wm * 64 + mt * 16 + li;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int col = nw + nt * 16 + 4 * lg;
        const v4f a = acc[mt][nt];
        const int off = row * 512 + (((col >> 3) ^ (row & 31)) << 4) + ((col >> 2) & 1) * 8;
        *reinterpret_cast<uint2*>(ct + off) = pack_bf16x4(a[0], a[1], a[2], a[3]);
      }
    }
    __syncthreads();
    const int c = lane % 32, n = n0 + c * 8;
#pragma unroll 4
    for (int it = 0; it < P::BM / 16; ++it) {
      const int row = it * 16 + wave * 2 + lane / 32;
      const int m = m0 + row;
      if (m >= M || n >= N) continue;
      const uint4 v = *reinterpret_cast<const uint4*>(ct + row * 512 + ((c ^ (row & 31)) << 4));
      *reinterpret_cast<uint4*>(C + static_cast<int64_t>(m) * N + n) = v;
    }
    return;
  }
#pragma unroll
  for (int mt = 0; mt < P::MT; ++mt) {
    const int m = m0 + wm * 64 + mt * 16 + li;
    if (m >= M) continue;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int n = n0 + nw + nt * 16 + 4 * lg;
      if (n >= N) continue;
      const v4f a = acc[mt][nt];
      if (partial)  // split-K: this split's fp32 tile, partial[split][M][N]
        *reinterpret_cast<float4*>(partial + (static_cast<int64_t>(blockIdx.y) * M + m) * N + n) =
            float4{a[0], a[1], a[2], a[3]};
      else
        *reinterpret_cast<uint2*>(C + static_cast<int64_t>(m) * N + n) = pack_bf16x4(a[0], a[1], a[2], a[3]);
    }
  }
}

static int device_cus();

// Whether the 256 x 256 GEMM beats the 128 x 256 one for an M x N product.
// Time is modelled as rounds of resident workgroups (one per CU) times the
// bytes a workgroup moves per K step, (rows + cols) x 128: over the
// DeepSeek-V3 dense shapes at M = 1024..4096 this picks the faster kernel in
// every measured case where they differ by more than 3 %.  The 256-row
// kernel also needs its buffer offsets below 2 GiB.
static bool use_big_gemm(int M, int N, int K, int64_t as_extent) {
  if (M < 512) return false;
  const int64_t cus = device_cus();
  auto cost = [&](int64_t bm, int64_t bn) {
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    return (tiles + cus - 1) / cus * (bm + bn);
  };
  return cost(256, 256) < cost(128, 256) && static_cast<int64_t>(M + 256) * K < (1ll << 31) &&
         static_cast<int64_t>(N + 256) * K < (1ll << 31) && as_extent < (1ll << 31);
}

static void splitk_reduce(const float* partial, int splits, int64_t mn, uint16_t* c, hipStream_t st);

static int launch_big(const uint8_t* a, const float* As, int64_t as_sm, int64_t as_sk, int as_bytes,
                      const uint8_t* b, const float* Bs, uint16_t* c, int m, int n, int k, hipStream_t st,
                      int splits = 1, int kper = 0, float* partial = nullptr) {
  using P = BigPipe;
  static bool raised = false;
  if (!raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_fp8_big_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, P::kLds) != hipSuccess) {
      set_error("w8a8_block_fp8_matmul: cannot raise the LDS limit of the GEMM kernel");
      return VMAMD_ERR_HIP;
    }
    raised = true;
  }
  const int TM = (m + P::BM - 1) / P::BM, TN = (n + P::BN - 1) / P::BN;
  if (splits <= 1) kper = k / 128;
  const int row_store = splits <= 1 && n % 8 == 0 &&
                        reinterpret_cast<uintptr_t>(c) % 16 == 0;
  gemm_fp8_big_kernel<<<dim3(xcd_grid(TM * TN), splits), P::kThreads, P::kLds, st>>>(
      a, As, as_sm, as_sk, as_bytes, b, Bs, c, m, n, k, TM, TN, kper, splits > 1 ? partial : nullptr,
      row_store);
  int rc = check_launch("w8a8_block_fp8_matmul(gemm)");
  if (rc || splits <= 1) return rc;
  splitk_reduce(partial, splits, static_cast<int64_t>(m) * n, c, st);
  return check_launch("w8a8_block_fp8_matmul(reduce)");
}

// C = bf16(sum_s partial[s]) over the S split-K partials of an M x N output,
// added in split order (deterministic), 4 elements per lane (M * N is a
// multiple of 16).  All S loads of a lane are issued before its first add,
// so a lane costs one memory round trip.
template <int S>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial, int64_t mn,
                                                            uint16_t* __restrict__ C) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x * 4;
  for (int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4; i < mn; i += stride) {
    float4 v[S];
#pragma unroll
    for (int sp = 0; sp < S; ++sp) v[sp] = *reinterpret_cast<const float4*>(partial + sp * mn + i);
    float4 a = v[0];
#pragma unroll
    for (int sp = 1; sp < S; ++sp) {
      a.x += v[sp].x; a.y += v[sp].y; a.z += v[sp].z; a.w += v[sp].w;
    }
    *reinterpret_cast<uint2*>(C + i) = pack_bf16x4(a.x, a.y, a.z, a.w);
  }
}

template <int S>
static void launch_splitk_reduce(const float* partial, int64_t mn, uint16_t* c, hipStream_t st) {
  const int64_t blocks = (mn / 4 + 255) / 256;
  splitk_reduce_kernel<S><<<static_cast<int>(blocks < 8192 ? blocks : 8192), 256, 0, st>>>(partial, mn, c);
}

static void splitk_reduce(const float* partial, int splits, int64_t mn, uint16_t* c, hipStream_t st) {
  switch (splits) {
#define VMAMD_RED(S) \
  case S: launch_splitk_reduce<S>(partial, mn, c, st); break;
    VMAMD_RED(2) VMAMD_RED(3) VMAMD_RED(4) VMAMD_RED(5) VMAMD_RED(6) VMAMD_RED(7) VMAMD_RED(8)
    VMAMD_RED(9) VMAMD_RED(10) VMAMD_RED(11) VMAMD_RED(12) VMAMD_RED(13) VMAMD_RED(14) VMAMD_RED(15)
    VMAMD_RED(16)
#undef VMAMD_RED
    default: break;  // gemm_kper plans 2..16 splits
  }
}

// ------------------------------------------------------------ split-K GEMV --
constexpr int kGemvU = 4;  // K-blocks of weights per pass (8 KiB per wave)

__device__ __forceinline__ v8i gemv_buffer_frag(__amdgpu_buffer_rsrc_t rs, uint32_t off, int g) {
  const v4i lo = __builtin_bit_cast(
      v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off + 16u * g), 0, 0));
  const v4i hi = __builtin_bit_cast(
      v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off + 64u + 16u * g), 0, 0));
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}
// U consecutive f32 scales at byte offset off (U = 2 or 4, 8- or 16-byte aligned).
template <int U>
__device__ __forceinline__ void gemv_buffer_scales(__amdgpu_buffer_rsrc_t rs, uint32_t off, float (&out)[U]) {
  static_assert(U == 2 || U == 4, "scale vector width");
  if constexpr (U == 4) {
    const v4f v = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0));
    for (int u = 0; u < 4; ++u) out[u] = v[u];
  } else {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, static_cast<int>(off), 0, 0));
    out[0] = v[0];
    out[1] = v[1];
  }
}
__device__ __forceinline__ float gemv_buffer_f32(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, static_cast<int>(off), 0, 0));
}

// One workgroup per NT x 16 weight rows; its W waves (W = blockDim.x / 64)
// split K by interleaved groups of U K-blocks: at pass r wave w reads blocks
// [(r*W + w)*U, +U), so the workgroup streams W*U*128 contiguous bytes of
// each of its rows per pass.  Every 16x128 weight fragment multiplies every
// 16-row activation tile (MT of them, M <= 16 * MT) and every activation
// fragment multiplies the NT weight fragments of its K-block, so the weights
// are read exactly once and the activations once per NT x 16 weight rows.
// Weights, both scale sets and activations are raw buffer loads: blocks past
// K and activation rows past M are masked lanes (zeros, no fetch), so the
// loop has no tail and no branches, and the first pass's weights are
// requested before anything else.  The W partial sums meet in LDS and wave 0
// adds them in wave order (deterministic) and rounds once.
// a_bytes = M * K and as_bytes cover A and As (both < 2 GiB);
// NT * 16 * K < 2 GiB; NT * 16 divides 128, so a workgroup's rows share one
// row of weight-block scales.
constexpr int gemv_max_threads(int MT, int NT, int U) {
  // 1024 threads (16 waves) only where the pass fits 128 VGPRs
  return 8 * U * (MT + NT) + 4 * MT * NT + U * (MT + 1) + 24 <= 128 ? 1024 : 512;
}

template <int MT, int NT, int U, bool VS>
__global__ __launch_bounds__(gemv_max_threads(MT, NT, U)) void gemv_fp8_bs_kernel(
    const uint8_t* __restrict__ A, int a_bytes, const float* __restrict__ As, int as_bytes,
    int64_t as_sm, int64_t as_sk, const uint8_t* __restrict__ B, const float* __restrict__ Bs,
    int M, int N, int K, uint16_t* __restrict__ C) {
  static_assert(128 % (16 * NT) == 0, "a workgroup's rows must share one weight-scale row");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  const int W = blockDim.x / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), lane = threadIdx.x % kWave;
  const int li = lane % 16, lg = lane / 16;
  const int n0 = blockIdx.x * NT * 16;  // the grid is exactly N / (NT * 16) workgroups
  const int KB = K / 128;
  const __amdgpu_buffer_rsrc_t wrs = gemv_rsrc(B + static_cast<int64_t>(n0) * K, NT * 16 * K);
  const __amdgpu_buffer_rsrc_t bsrs = gemv_rsrc(Bs + static_cast<int64_t>(n0 / 128) * KB, KB * 4);
  const __amdgpu_buffer_rsrc_t ars = gemv_rsrc(A, a_bytes);
  const __amdgpu_buffer_rsrc_t asrs = gemv_rsrc(As, as_bytes);
  const uint32_t woff = static_cast<uint32_t>(li) * static_cast<uint32_t>(K);
  const uint32_t wtile = 16u * static_cast<uint32_t>(K);  // bytes between weight tiles
  uint32_t aoff[MT], soff[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    aoff[mt] = m < M ? static_cast<uint32_t>(m) * static_cast<uint32_t>(K) : kGemvMasked;
    soff[mt] = m < M ? static_cast<uint32_t>(m * as_sm * 4) : kGemvMasked;
  }
  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};

  // One pass: U K-blocks of the NT weight tiles and of every activation
  // tile, with their scales.  VS: the U scales of a group are contiguous in
  // both scale arrays (As rows with unit K stride, K / 128 a multiple of U,
  // 8- or 16-byte aligned rows), so each set is one wide load instead of U
  // scattered ones; a group is then entirely inside or entirely past K.
  struct Pass {
    v8i wf[NT][U];
    float sb[U];
    v8i xf[MT][U];
    float sa[MT][U];
  };
  auto load = [&](Pass& p, int kb) {
    if constexpr (VS) gemv_buffer_scales<U>(bsrs, kb < KB ? static_cast<uint32_t>(kb * 4) : kGemvMasked, p.sb);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = kb + u < KB;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        p.wf[nt][u] = gemv_buffer_frag(
            wrs, live ? nt * wtile + woff + static_cast<uint32_t>((kb + u) * 128) : kGemvMasked, lg);
      if constexpr (!VS) p.sb[u] = gemv_buffer_f32(bsrs, live ? static_cast<uint32_t>(kb + u) * 4u : kGemvMasked);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (VS) {
        const bool live = aoff[mt] != kGemvMasked && kb < KB;
        gemv_buffer_scales<U>(asrs, live ? soff[mt] + static_cast<uint32_t>(kb * 4) : kGemvMasked, p.sa[mt]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool live = aoff[mt] != kGemvMasked && kb + u < KB;
        p.xf[mt][u] =
            gemv_buffer_frag(ars, live ? aoff[mt] + static_cast<uint32_t>((kb + u) * 128) : kGemvMasked, lg);
        if constexpr (!VS)
          p.sa[mt][u] = gemv_buffer_f32(asrs, live ? soff[mt] + static_cast<uint32_t>((kb + u) * as_sk * 4)
                                                   : kGemvMasked);
      }
    }
  };
  auto compute = [&](const Pass& p) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int u = 0; u < U; ++u)
          fma4(acc[mt][nt], mfma_fp8(p.wf[nt][u], p.xf[mt][u], zero), p.sa[mt][u] * p.sb[u]);
  };
  // Every load of a pass ahead of its first MFMA (the group barriers), so a
  // pass costs one memory round trip.  Measured: two passes in flight per
  // wave (half-size passes, double-buffered registers) is slower; there are
  // enough waves per CU to cover the latency.  The host sizes
  // W <= ceil(KB / U), so every wave owns at least one pass.
  constexpr int kScaleLoads = VS ? 1 : U;
  constexpr int kLoads = (2 * U * NT + kScaleLoads) + MT * (2 * U + kScaleLoads), kMfmas = U * MT * NT;
  const int step = W * U;
  int kb = wave * U;
  do {
    Pass p;
    load(p, kb);
    compute(p);
    __builtin_amdgcn_sched_group_barrier(0x020, kLoads, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, kMfmas, 0);
    kb += step;
  } while (kb < KB);

  if (W > 1) {  // uniform over the grid
    float4* red = reinterpret_cast<float4*>(smem_dyn);
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const v4f& a = acc[mt][nt];
          red[(((wave - 1) * MT + mt) * NT + nt) * kWave + lane] = float4{a[0], a[1], a[2], a[3]};
        }
    }
    __syncthreads();
    if (wave > 0) return;
    for (int w = 1; w < W; ++w) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float4 v = red[(((w - 1) * MT + mt) * NT + nt) * kWave + lane];
          acc[mt][nt][0] += v.x; acc[mt][nt][1] += v.y; acc[mt][nt][2] += v.z; acc[mt][nt][3] += v.w;
        }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    if (m < M) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int n = n0 + nt * 16 + 4 * lg;
        const v4f& a = acc[mt][nt];
        *reinterpret_cast<uint2*>(C + static_cast<int64_t>(m) * N + n) = pack_bf16x4(a[0], a[1], a[2], a[3]);
      }
    }
  }
}

// ------------------------------------------------------------ dispatch ------
constexpr int kGemvMaxM = 64;

// The (MT, NT, U) instances gemv_shape can pick.
#define VMAMD_GEMV_SHAPES(X) \
  X(1, 1, 4) X(1, 2, 2) X(2, 1, 4) X(2, 2, 2) X(2, 4, 2) X(4, 1, 4) X(4, 2, 2) X(4, 4, 2)

struct GemvShape {
  int mt, nt, u, w;  // activation tiles, weight tiles per wave, K-blocks per pass, waves
};

// Workgroups of `kernel` resident per CU at W waves (register, LDS and wave
// limits), cached per W; every instance is built for the same gfx950.
template <int MT, int NT, int U>
static int gemv_blocks_per_cu(int w) {
  static std::atomic<int> cache[17];
  int v = cache[w].load(std::memory_order_relaxed);
  if (v == 0) {
    const size_t lds = static_cast<size_t>(w - 1) * MT * NT * kWave * sizeof(float4);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &v, reinterpret_cast<const void*>(gemv_fp8_bs_kernel<MT, NT, U, true>), w * kWave, lds) != hipSuccess ||
        v < 1)
      v = 1;
    cache[w].store(v, std::memory_order_relaxed);
  }
  return v;
}

static int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

// K splits of the tiled GEMM: where its 128 x 256 tiles are too few to give
// every CU a workgroup (small N, M of a few hundred), workgroups of one tile
// take disjoint K ranges, write fp32 partials and a second kernel adds them.
// Chosen by a time model fitted on MI355X: rounds x K steps per workgroup x
// a step time that grows with the workgroups streaming at once (they share
// HBM: 1.08 us for 28 workgroups, 1.87 us for 224 at 7168 x 18432), plus,
// when split, the partials' round trip at 4 TB/s and 3 us for the extra
// launch.  A round is what one XCD holds at one workgroup per CU; each split
// row of the grid spreads its tiles over the XCDs in blocks of
// ceil(tiles / 8) (xcd_tile).  At most 16 splits of at least 4 K steps each
// and 256 MiB of partials.  Over 80 measured cases (10 shapes, M = 65..2048)
// the picks sum to 5595 us (the nearest measured split count where the pick
// was not measured), the best split of each case to 5573 us, no split to
// 8091 us.  Returns the K steps per split.
constexpr int64_t kSplitKMaxBytes = 256ll << 20;
// step: the modelled time of one K step of the tile relative to the 128 x 256
// tile's (the 256 x 256 tile: kBigStep, the 128 x 128 tile: kNarrowStep);
// min_per: K steps a split keeps at least; bn: the tile's columns.
// *cost_out: the model's time (us).
static int gemm_kper(int M, int N, int K, int bm = 128, double step = 1.0, double* cost_out = nullptr,
                     int min_per = 4, int bn = 256) {
  const int64_t T = static_cast<int64_t>((M + bm - 1) / bm) * ((N + bn - 1) / bn), KS = K / 128;
  const int64_t cus = device_cus(), xcd_cus = max(1, static_cast<int>(cus / kXcds));
  const int64_t per_xcd = (T + kXcds - 1) / kXcds;
  auto gemm_us = [&](int64_t se, int64_t per) {
    const double active = static_cast<double>(min(T * se, cus));
    return static_cast<double>((per_xcd * se + xcd_cus - 1) / xcd_cus * per) * step * (1.0 + 0.004 * active);
  };
  int best = static_cast<int>(KS);
  double cost = gemm_us(1, KS);
  // Tiles that alone occupy more than half the CUs: splitting gained at most
  // 5 % in the fit and lost up to 16 % where the model missed.
  if (2 * T <= cus) {
    for (int64_t s = 2; s <= 16 && s * min_per <= KS; ++s) {
      const int64_t per = (KS + s - 1) / s, se = (KS + per - 1) / per;
      const int64_t bytes = se * static_cast<int64_t>(M) * N * 4;
      if (bytes > kSplitKMaxBytes) break;
      const double c = gemm_us(se, per) + (bytes + 2.0 * M * N) / 4e6 + 3.0;
      if (c < cost) {
        cost = c;
        best = static_cast<int>(per);
      }
    }
  }
  if (cost_out) *cost_out = cost;
  return best;
}

// K step of the 256 x 256 tile against the 128 x 256 tile's: the bytes it
// moves per step, (256 + 256) / (128 + 256).  Its splits keep at least
// kBigMinSteps K steps: with fewer, each workgroup's fixed costs (first load,
// a 256 KiB fp32 partial tile) outweigh the shorter loop (measured on MI355X
// at M = 512: 7168 x 18432 102.9 -> 92.2 us and 7168 x 16384 97.4 -> 86.1 us
// with 4 splits of 36 / 32 steps; 2112 x 7168 32.7 -> 37.0 us and 4096 x 7168
// 37.1 -> 44.0 us with splits of 4-8 steps).
constexpr double kBigStep = 512.0 / 384.0;
constexpr int kBigMinSteps = 32;
// K step of the 128 x 128 tile (DensePipeN) against the 128 x 256 tile's:
// (128 + 128) / (128 + 256).  With it the model takes the narrow tiles
// where they measured faster on MI355X (7 shapes x M = 64..2048, none
// slower: 7168 x 2048 at M = 128 / 256 / 512 21.5 / 24.2 / 28.4 -> 17.4 /
// 18.9 / 19.7 µs, 24576 x 1536 at M = 128 25.0 -> 18.5, 2112 x 7168 at
// M = 128 / 256 23.6 / 26.5 -> 19.2 / 22.3, 4096 x 7168 at M = 128
// 26.0 -> 21.4), and leaves long K (7168 x 16384 / 18432) and large M on
// 128 x 256 tiles, where those measured faster; a smaller factor (0.6)
// also takes 24576 x 1536 at M = 512, measured 30 % slower there.
constexpr double kNarrowStep = 256.0 / 384.0;

// The dense path for an M x N x K product: the GEMV up to M = 16, and up to
// M = 32 / 64 unless the split GEMM is faster there -- weights of 96 MiB and
// more from M = 17, rows of K >= 4096 from M = 33 (measured on MI355X over
// the DeepSeek-V3 linear shapes: e.g. 7168 x 18432 at M = 64, 61 us GEMV,
// 39 us split GEMM).  `splits` > 1 needs splits * M * N * 4 bytes of
// workspace.
// big: the 256 x 256 kernel with K splits, where the 128 x 256 tiles would
// split K too (too few tiles for the CUs) and the model prices the 256-row
// tiles' splits lower (M >= 512).  Without a split the choice between the
// two tile kernels is use_big_gemm's.
struct DensePlan {
  bool gemv, big;
  int kper, splits;
  int bn;  // column width of the 128-row tiles: 256, or 128 (DensePipeN)
};
static DensePlan dense_plan(int M, int N, int K) {
  DensePlan d;
  const int KS = K / 128;
  const bool heavy = static_cast<int64_t>(N) * K >= (96ll << 20);
  d.gemv = M <= 16 || (M <= 32 && !heavy) || (M <= kGemvMaxM && K < 4096 && !heavy);
  d.big = false;
  d.bn = 256;
  double cost = 0.0;
  d.kper = d.gemv ? KS : gemm_kper(M, N, K, 128, 1.0, &cost);
  if (!d.gemv && d.kper < KS && M >= 512) {
    double cost_big = 0.0;
    const int kper_big = gemm_kper(M, N, K, 256, kBigStep, &cost_big, kBigMinSteps);
    if (kper_big < KS && cost_big < cost) {
      d.big = true;
      d.kper = kper_big;
      cost = cost_big;
    }
  }
  if (!d.gemv) {
    double cost_n = 0.0;
    const int kper_n = gemm_kper(M, N, K, 128, kNarrowStep, &cost_n, 4, 128);
    if (cost_n < cost) {
      d.big = false;
      d.bn = 128;
      d.kper = kper_n;
    }
  }
  d.splits = (KS + d.kper - 1) / d.kper;
  return d;
}

// Waves per workgroup: the fewest that minimise rounds x passes, where a
// round is one set of workgroups resident together on every CU and a wave
// makes ceil(groups / W) passes of U K-blocks.  At most 16 (the kernel's
// thread limit may say 8), at most one per group, and the reduction buffer
// within 64 KiB of LDS.  The VS = true instance sizes both scale layouts, so
// the summation order never depends on the scale layout.
template <int MT, int NT, int U>
static int gemv_waves(int tiles, int groups) {
  const int wmax = min(min(gemv_max_threads(MT, NT, U) / kWave, groups), 1 + 64 / (MT * NT));
  const int64_t cus = device_cus();
  int best = 1;
  int64_t cost = -1;
  for (int w = 1; w <= wmax; ++w) {
    const int64_t resident = cus * gemv_blocks_per_cu<MT, NT, U>(w);
    const int64_t c = (tiles + resident - 1) / resident * ((groups + w - 1) / w);
    if (cost < 0 || c < cost) {
      cost = c;
      best = w;
    }
  }
  return best;
}

// Activation tiles cover M; each wave takes NT weight tiles, reusing every
// activation fragment NT times, where the weight matrix has enough 16-row
// tiles to keep every CU busy with fewer, wider workgroups: two from
// N = 7168, four for M > 16 from N = 12288 with K >= 4096 (shorter rows
// leave too few passes to hide the wider pass).  Wider tiles take passes of
// 2 K-blocks (their registers; measured no slower at M <= 16).  Measured on
// MI355X over the DeepSeek-V3 linear shapes and 12288 x 4096,
// 16384 x 7168 at M = 1..64.
static GemvShape gemv_shape(int M, int N, int K) {
  GemvShape g;
  g.mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  g.nt = 1;
  if (N >= 7168 && N % 32 == 0) g.nt = 2;
  if (g.mt >= 2 && N >= 12288 && K >= 4096 && N % 64 == 0) g.nt = 4;
  g.u = g.nt > 1 ? 2 : kGemvU;
  const int tiles = N / (16 * g.nt), groups = (K / 128 + g.u - 1) / g.u;
  g.w = 0;
#define VMAMD_GEMV(MT, NT, U) \
  if (g.mt == MT && g.nt == NT && g.u == U) g.w = gemv_waves<MT, NT, U>(tiles, groups);
  VMAMD_GEMV_SHAPES(VMAMD_GEMV)
#undef VMAMD_GEMV
  return g;
}

template <int MT, int NT, int U>
static void launch_gemv(bool vs, int w, const uint8_t* a, int a_bytes, const float* As, int as_bytes,
                        int64_t as_sm, int64_t as_sk, const uint8_t* b, const float* Bs, int m, int n,
                        int k, uint16_t* c, hipStream_t st) {
  const size_t lds = static_cast<size_t>(w - 1) * MT * NT * kWave * sizeof(float4);
  const int grid = n / (16 * NT);
  if (vs)
    gemv_fp8_bs_kernel<MT, NT, U, true><<<grid, w * kWave, lds, st>>>(a, a_bytes, As, as_bytes, as_sm, as_sk, b,
                                                                     Bs, m, n, k, c);
  else
    gemv_fp8_bs_kernel<MT, NT, U, false><<<grid, w * kWave, lds, st>>>(a, a_bytes, As, as_bytes, as_sm, as_sk, b,
                                                                      Bs, m, n, k, c);
}

// The GEMM's split-K partials (none for the GEMV or an unsplit GEMM).
size_t w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K < 128 || M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31)) return 0;
  const DensePlan d = dense_plan(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K));
  return d.splits > 1 ? static_cast<size_t>(d.splits * M * N * 4) : 0;
}

}  // namespace vmamd

using namespace vmamd;

extern "C" size_t vmamd_w8a8_block_fp8_matmul_workspace_size(int64_t M, int64_t N, int64_t K) {
  return w8a8_workspace_bytes(M, N, K);
}

namespace vmamd {
// gemm_fp8_dma_kernel on pipe P: TM x TN tiles, `splits` K ranges of kper steps.
template <typename P>
static int launch_tile(const uint8_t* a, const float* As, int64_t as_sm, int64_t as_sk, const uint8_t* b,
                       const float* Bs, uint16_t* c, int m, int n, int k, int kper, int splits, float* partial,
                       hipStream_t st) {
  static bool lds_raised = false;
  if (!lds_raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_fp8_dma_kernel<P>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, P::kLds) != hipSuccess) {
      set_error("w8a8_block_fp8_matmul: cannot raise the LDS limit of the GEMM kernel");
      return VMAMD_ERR_HIP;
    }
    lds_raised = true;
  }
  const int TM = (m + P::kBM - 1) / P::kBM, TN = (n + P::kBN - 1) / P::kBN;
  gemm_fp8_dma_kernel<P><<<dim3(xcd_grid(TM * TN), splits), P::kThreads, P::kLds, st>>>(
      a, As, as_sm, as_sk, b, Bs, c, m, n, k, TM, TN, kper, partial);
  return VMAMD_OK;
}
}  // namespace vmamd

extern "C" int vmamd_w8a8_block_fp8_matmul(const void* A, const float* As, int64_t as_stride_m,
                                           int64_t as_stride_k, const void* B, const float* Bs,
                                           void* C, int64_t M, int64_t N, int64_t K, int block_n,
                                           int block_k, void* workspace, size_t workspace_bytes,
                                           vmamd_stream_t stream) {
  VMAMD_REQUIRE(block_n == 128 && block_k == 128,
                "w8a8_block_fp8_matmul: only 128x128 weight blocks are supported (got %dx%d)",
                block_n, block_k);
  VMAMD_REQUIRE(M >= 0 && N > 0 && K > 0, "w8a8_block_fp8_matmul: bad sizes");
  VMAMD_REQUIRE(K % 128 == 0, "w8a8_block_fp8_matmul: K (%lld) must be a multiple of 128",
                (long long)K);
  VMAMD_REQUIRE(N % 16 == 0, "w8a8_block_fp8_matmul: N (%lld) must be a multiple of 16",
                (long long)N);
  VMAMD_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31),
                "w8a8_block_fp8_matmul: sizes must fit in int32");
  if (M == 0) return VMAMD_OK;
  VMAMD_REQUIRE(A && As && B && Bs && C, "w8a8_block_fp8_matmul: null pointer");
  VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(B) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(C) % 8 == 0,
                "w8a8_block_fp8_matmul: A and B must be 16-byte and C 8-byte aligned");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  uint16_t* c = static_cast<uint16_t*>(C);
  const uint8_t* a = static_cast<const uint8_t*>(A);
  const uint8_t* b = static_cast<const uint8_t*>(B);
  // Without the workspace a split plan needs, M <= 64 takes the GEMV and
  // larger M the unsplit GEMM (same result up to the order of the fp32 sums).
  DensePlan plan = dense_plan(m, n, k);
  if (plan.splits > 1 && (workspace == nullptr ||
                          workspace_bytes < static_cast<size_t>(plan.splits) * m * n * 4 ||
                          reinterpret_cast<uintptr_t>(workspace) % 16 != 0)) {
    plan.gemv = m <= kGemvMaxM;
    plan.kper = k / 128;
    plan.splits = 1;
  }
  if (plan.gemv) {
    // A, As and each 16-row weight tile are read through buffer descriptors:
    // all must stay below 2 GiB.
    const int64_t as_elems = (m - 1) * as_stride_m + (k / 128 - 1) * as_stride_k + 1;
    VMAMD_REQUIRE(as_stride_m >= 0 && as_stride_k >= 0 && static_cast<int64_t>(m) * k < (1ll << 31) &&
                      as_elems * 4 < (1ll << 31) && 16ll * k < (1ll << 31),
                  "w8a8_block_fp8_matmul: activations, their scales and 16 weight rows must stay "
                  "below 2 GiB");
    const int a_bytes = m * k, as_bytes = static_cast<int>(as_elems * 4);
    const GemvShape g = gemv_shape(m, n, k);
    VMAMD_REQUIRE(16ll * g.nt * k < (1ll << 31), "w8a8_block_fp8_matmul: weight tile of %d rows past 2 GiB",
                  16 * g.nt);
    const bool vs = as_stride_k == 1 && as_stride_m % g.u == 0 && (k / 128) % g.u == 0 &&
                    reinterpret_cast<uintptr_t>(As) % (4 * g.u) == 0 &&
                    reinterpret_cast<uintptr_t>(Bs) % (4 * g.u) == 0;
    VMAMD_REQUIRE(g.w >= 1, "w8a8_block_fp8_matmul: no GEMV instance for %d x %d x %d", g.mt, g.nt, g.u);
#define VMAMD_GEMV(MT, NT, U)                                                                   \
  if (g.mt == MT && g.nt == NT && g.u == U)                                                     \
    launch_gemv<MT, NT, U>(vs, g.w, a, a_bytes, As, as_bytes, as_stride_m, as_stride_k, b, Bs, m, n, k, c, \
                           st);                                                                 \
  else
    VMAMD_GEMV_SHAPES(VMAMD_GEMV)
    VMAMD_REQUIRE(false, "w8a8_block_fp8_matmul: no GEMV instance for %d x %d x %d", g.mt, g.nt, g.u);
#undef VMAMD_GEMV
    return check_launch("w8a8_block_fp8_matmul(gemv)");
  }
  if (as_stride_m >= 0 && as_stride_k >= 0) {
    const int64_t as_extent = ((m - 1) * as_stride_m + (k / 128 - 1) * as_stride_k + 1) * 4;
    const bool big_ok = static_cast<int64_t>(m + 256) * k < (1ll << 31) &&
                        static_cast<int64_t>(n + 256) * k < (1ll << 31) && as_extent < (1ll << 31);
    if (plan.splits == 1 && plan.bn == 256 && use_big_gemm(m, n, k, as_extent))
      return launch_big(a, As, as_stride_m, as_stride_k, static_cast<int>(as_extent), b, Bs, c, m, n, k, st);
    if (plan.splits > 1 && plan.big && big_ok)
      return launch_big(a, As, as_stride_m, as_stride_k, static_cast<int>(as_extent), b, Bs, c, m, n, k, st,
                        plan.splits, plan.kper, static_cast<float*>(workspace));
  }
  // A split planned for the 256 x 256 kernel that it cannot take (an operand
  // past its 2 GiB descriptors, or negative scale strides) runs on the
  // 128 x 256 kernel with the split its own model prices for 128-row tiles,
  // capped so that the partials fit the workspace sized for the plan.
  if (plan.big && plan.splits > 1) {
    const int KS = k / 128;
    const int64_t max_splits = static_cast<int64_t>(workspace_bytes / (static_cast<size_t>(m) * n * 4));
    int64_t kper = gemm_kper(m, n, k);
    kper = max_splits < 2 ? KS : std::max<int64_t>(kper, (KS + max_splits - 1) / max_splits);
    plan.kper = static_cast<int>(kper);
    plan.splits = static_cast<int>((KS + kper - 1) / kper);
  }
  const int kper = plan.kper, splits = plan.splits;
  VMAMD_REQUIRE(splits >= 1 && splits <= 16, "w8a8_block_fp8_matmul: %d K splits planned", splits);
  float* partial = splits > 1 ? static_cast<float*>(workspace) : nullptr;
  const int rc = plan.bn == 128 ? launch_tile<DensePipeN>(a, As, as_stride_m, as_stride_k, b, Bs, c, m, n, k, kper,
                                                          splits, partial, st)
                                : launch_tile<DensePipe>(a, As, as_stride_m, as_stride_k, b, Bs, c, m, n, k, kper,
                                                         splits, partial, st);
  if (rc) return rc;
  if (splits > 1) splitk_reduce(partial, splits, static_cast<int64_t>(m) * n, c, st);
  return check_launch("w8a8_block_fp8_matmul(gemm)");
}

// ------------------------------------------------- allocation-free variant --
// vmamd_w8a8_block_fp8_matmul_noalloc keeps the split-K partials in one fixed
// device-resident array per GPU instead of a caller workspace.  In host code
// the array's name denotes a host-side stand-in, not device memory, so it is
// never handed to a kernel: its device address comes from
// hipGetSymbolAddress, taken once per device with that device current, and
// only that address is used.  The device is the one the call's stream
// belongs to (the kernels run there), which need not be the current one.
// Every split writes its whole partial slab before the reduce reads it, so
// nothing needs clearing between calls.
namespace vmamd {

constexpr size_t kNoAllocScratchBytes = VMAMD_W8A8_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

static int noalloc_scratch(hipStream_t stream, void** out) {
  static std::mutex mu;
  static void* per_device[64] = {};
  int dev = 0;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= 64) {
    set_error("w8a8_block_fp8_matmul_noalloc: the stream's device is unknown or not below 64");
    return VMAMD_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (per_device[dev] == nullptr) {
    int cur = 0;
    if (hipGetDevice(&cur) != hipSuccess || (cur != dev && hipSetDevice(dev) != hipSuccess)) {
      set_error("w8a8_block_fp8_matmul_noalloc: cannot make device %d current", dev);
      return VMAMD_ERR_HIP;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || p == nullptr) {
      set_error("w8a8_block_fp8_matmul_noalloc: hipGetSymbolAddress of the scratch array failed: %s",
                hipGetErrorString(e));
      return VMAMD_ERR_HIP;
    }
    per_device[dev] = p;
  }
  *out = per_device[dev];
  return VMAMD_OK;
}

}  // namespace vmamd

extern "C" int vmamd_w8a8_block_fp8_matmul_noalloc(const void* A, const float* As,
                                                   int64_t as_stride_m, int64_t as_stride_k,
                                                   const void* B, const float* Bs, void* C,
                                                   int64_t M, int64_t N, int64_t K, int block_n,
                                                   int block_k, vmamd_stream_t stream) {
  const size_t need = w8a8_workspace_bytes(M, N, K);
  VMAMD_REQUIRE(need <= kNoAllocScratchBytes,
                "w8a8_block_fp8_matmul_noalloc: the plan for %lld x %lld x %lld needs %zu bytes of "
                "split-K partials; the fixed scratch holds %zu (call vmamd_w8a8_block_fp8_matmul "
                "with a workspace)",
                (long long)M, (long long)N, (long long)K, need, kNoAllocScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = noalloc_scratch(reinterpret_cast<hipStream_t>(stream), &ws);
    if (rc) return rc;
  }
  return vmamd_w8a8_block_fp8_matmul(A, As, as_stride_m, as_stride_k, B, Bs, C, M, N, K, block_n,
                                     block_k, ws, need > 0 ? kNoAllocScratchBytes : 0, stream);
}
