// Dense w8a8 block-fp8 GEMM:  C[M,N] = bf16( sum_kb (A_kb . B_kb^T) * As[m,kb] * Bs[n/128,kb] )
//   A  [M, K] e4m3 (1x128 activation groups, scales As[m*as_sm + kb*as_sk])
//   B  [N, K] e4m3 (128x128 weight blocks, scales Bs[ceil(N/128), K/128])
//
// Two kernels:
//  * gemm_fp8_dma_kernel -- 128 x 256 workgroup tile, 8 waves, K-block of 128
//    per step, 3-stage LDS ring fed by direct global->LDS loads (one barrier
//    per K-block), XCD-aware tile order.  For M > 64.
//  * gemv_fp8_bs_kernel  -- decode-sized M (<= 64): one wave per 16 weight rows
//    streams its rows straight from HBM (no LDS), each 16x128 weight fragment
//    multiplies every 16-row activation tile held in registers, so weights are
//    read exactly once.  Split-K over blockIdx.y writes fp32 partials that
//    splitk_reduce_kernel sums in a fixed order (deterministic), one rounding.
#include "mfma_fp8.h"
#include "tile_pipe.h"

namespace vmamd {

// ------------------------------------------- tiled GEMM on the DMA ring ---
// 128 x 256 output tile per workgroup (8 waves as 2 (m) x 4 (n), 64 x 64 per
// wave), 3-stage LDS ring fed by direct global->LDS loads: two K steps are in
// flight while the current one runs on MFMA.  Rows past M / N are clamped to
// the last row (their results are not stored).
using DensePipe = TilePipe<true, 128, 256, 2, 4, 3>;

__global__ __launch_bounds__(DensePipe::kThreads, 1) void gemm_fp8_dma_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, int64_t as_sm, int64_t as_sk,
    const uint8_t* __restrict__ B, const float* __restrict__ Bs, uint16_t* __restrict__ C, int M,
    int N, int K, int TM, int TN) {
  using P = DensePipe;
  constexpr int NS = 3, BM = 128, BN = 256, WN = 4;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem_dyn[];
  int tm, tn;
  if (!xcd_tile(blockIdx.x, TM, TN, tm, tn)) return;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane % 16, lg = lane / 16;
  const int KS = K / 128, NB = (N + 127) / 128;

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
    f.sb = lds_load<float>(st, P::kOffSB + (wn / 2) * 4);
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
  // Step kb: its fragments are in `cur`; step kb + 1 is read into `nxt`, two
  // LDS reads after each MFMA, and buffer kb % NS (read into `cur` by every
  // wave before the barrier) is refilled with step kb + NS after the MFMAs
  // are issued -- a wave whose DMA issue waits behind the other waves' in the
  // address unit would otherwise start its MFMAs late.
  auto step = [&](int kb, const Frags& cur, Frags& nxt) {
    wait_lgkmcnt0();  // this wave's reads of the buffer refilled below are done
    wait_vmcnt<(NS - 2) * P::kIPS>();
    barrier_lds();
    read(smem_dyn + ((kb + 1) % NS) * P::kStage, nxt);
    mma(cur);
    p.issue(smem_dyn + (kb % NS) * P::kStage, min(kb + NS, KS - 1));
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
      *reinterpret_cast<uint2*>(C + static_cast<int64_t>(m) * N + n) = pack_bf16x4(a[0], a[1], a[2], a[3]);
    }
  }
}

// ------------------------------------------------------------ split-K GEMV --
constexpr int kGemvWaves = 4;

template <int MT>
__global__ __launch_bounds__(kGemvWaves * kWave) void gemv_fp8_bs_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ As, int64_t as_sm, int64_t as_sk,
    const uint8_t* __restrict__ B, const float* __restrict__ Bs, int M, int N, int K, int splits,
    float* __restrict__ partial, uint16_t* __restrict__ C) {
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int li = lane % 16, lg = lane / 16;
  const int ntile = blockIdx.x * kGemvWaves + wave;
  if (ntile * 16 >= N) return;  // wave-uniform; this kernel has no barriers
  const int split = blockIdx.y;
  const int KB = K / 128;
  const int kb0 = static_cast<int>(static_cast<int64_t>(split) * KB / splits);
  const int kb1 = static_cast<int>(static_cast<int64_t>(split + 1) * KB / splits);
  const uint8_t* wrow = B + static_cast<int64_t>(ntile * 16 + li) * K;
  const float* bs = Bs + static_cast<int64_t>((ntile * 16) / 128) * KB;
  const uint8_t* xrow[MT];
  const float* as[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(mt * 16 + li, M - 1);
    xrow[mt] = A + static_cast<int64_t>(m) * K;
    as[mt] = As + static_cast<int64_t>(m) * as_sm;
  }
  v4f acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
  const v4f zero = {0.f, 0.f, 0.f, 0.f};

  constexpr int U = 4;  // K-blocks in flight per wave
  int kb = kb0;
  for (; kb + U <= kb1; kb += U) {
    v8i w[U];
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = global_frag(wrow + (kb + u) * 128, lg);
    float sbv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) sbv[u] = bs[kb + u];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      v8i x[U];
      float sav[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        x[u] = global_frag(xrow[mt] + (kb + u) * 128, lg);
        sav[u] = as[mt][(kb + u) * as_sk];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) fma4(acc[mt], mfma_fp8(w[u], x[u], zero), sav[u] * sbv[u]);
    }
  }
  for (; kb < kb1; ++kb) {
    const v8i w = global_frag(wrow + kb * 128, lg);
    const float sb = bs[kb];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      fma4(acc[mt], mfma_fp8(w, global_frag(xrow[mt] + kb * 128, lg), zero), as[mt][kb * as_sk] * sb);
  }

  const int n = ntile * 16 + 4 * lg;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + li;
    if (m >= M) continue;
    const v4f a = acc[mt];
    if (splits == 1) {
      *reinterpret_cast<uint2*>(C + static_cast<int64_t>(m) * N + n) = pack_bf16x4(a[0], a[1], a[2], a[3]);
    } else {
      float4 v = {a[0], a[1], a[2], a[3]};
      *reinterpret_cast<float4*>(partial + (static_cast<int64_t>(split) * M + m) * N + n) = v;
    }
  }
}

// C[m, n] = bf16(sum_{s < splits} partial[s, m, n]) in split order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial,
                                                            int splits, int64_t mn,
                                                            uint16_t* __restrict__ C) {
  const int64_t i4 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (i4 >= mn) return;
  float4 acc = *reinterpret_cast<const float4*>(partial + i4);
  for (int s = 1; s < splits; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(partial + s * mn + i4);
    acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
  }
  *reinterpret_cast<uint2*>(C + i4) = pack_bf16x4(acc.x, acc.y, acc.z, acc.w);
}

// ------------------------------------------------------------ dispatch ------
constexpr int kGemvMaxM = 64;

static int gemv_splits(int M, int N, int K) {
  const int tiles = N / 16;
  const int KB = K / 128;
  int s = (2048 + tiles - 1) / tiles;  // aim for >= 2048 waves (8 per CU)
  s = max(1, min(s, KB / 2 > 0 ? KB / 2 : 1));
  (void)M;
  return s;
}

size_t w8a8_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M > kGemvMaxM || M <= 0) return 0;
  const int s = gemv_splits(static_cast<int>(M), static_cast<int>(N), static_cast<int>(K));
  return s > 1 ? static_cast<size_t>(s) * M * N * sizeof(float) : 0;
}

}  // namespace vmamd

using namespace vmamd;

extern "C" size_t vmamd_w8a8_block_fp8_matmul_workspace_size(int64_t M, int64_t N, int64_t K) {
  return w8a8_workspace_bytes(M, N, K);
}

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
  if (m <= kGemvMaxM) {
    const int splits = gemv_splits(m, n, k);
    float* part = nullptr;
    if (splits > 1) {
      const size_t need = static_cast<size_t>(splits) * m * n * sizeof(float);
      VMAMD_REQUIRE(workspace && workspace_bytes >= need,
                    "w8a8_block_fp8_matmul: workspace of %zu bytes required (got %zu)", need,
                    workspace_bytes);
      VMAMD_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 16 == 0,
                    "w8a8_block_fp8_matmul: workspace must be 16-byte aligned");
      part = static_cast<float*>(workspace);
    }
    dim3 grid((n / 16 + kGemvWaves - 1) / kGemvWaves, splits);
    if (m <= 16)
      gemv_fp8_bs_kernel<1><<<grid, kGemvWaves * kWave, 0, st>>>(a, As, as_stride_m, as_stride_k, b, Bs,
                                                                m, n, k, splits, part, c);
    else if (m <= 32)
      gemv_fp8_bs_kernel<2><<<grid, kGemvWaves * kWave, 0, st>>>(a, As, as_stride_m, as_stride_k, b, Bs,
                                                                m, n, k, splits, part, c);
    else
      gemv_fp8_bs_kernel<4><<<grid, kGemvWaves * kWave, 0, st>>>(a, As, as_stride_m, as_stride_k, b, Bs,
                                                                m, n, k, splits, part, c);
    if (splits > 1) {
      const int64_t mn = static_cast<int64_t>(m) * n;
      splitk_reduce_kernel<<<static_cast<int>((mn / 4 + 255) / 256), 256, 0, st>>>(part, splits, mn, c);
    }
    return check_launch("w8a8_block_fp8_matmul(gemv)");
  }
  static bool lds_raised = false;
  if (!lds_raised) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_fp8_dma_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, DensePipe::kLds) != hipSuccess) {
      set_error("w8a8_block_fp8_matmul: cannot raise the LDS limit of the GEMM kernel");
      return VMAMD_ERR_HIP;
    }
    lds_raised = true;
  }
  const int TM = (m + 127) / 128, TN = (n + 255) / 256;
  gemm_fp8_dma_kernel<<<xcd_grid(TM * TN), DensePipe::kThreads, DensePipe::kLds, st>>>(
      a, As, as_stride_m, as_stride_k, b, Bs, c, m, n, k, TM, TN);
  return check_launch("w8a8_block_fp8_matmul(gemm)");
}
