// Multi-stage LDS pipeline of the tiled MFMA GEMMs, fed by direct
// global->LDS loads (global_load_lds_dwordx4: each lane's 16 bytes land at
// M0 + lane * 16, no VGPR staging).
//
// A workgroup computes a BM x BN tile (A rows x B rows, K contiguous in both)
// in K steps of one 128-byte chunk per row.  Stage s of the LDS ring holds
//   [A tile BM x 128 B][B tile BN x 128 B][A scales BM x f32][B scales 64 x f32]
// (scales only for block-scaled fp8).  A row is 8 chunks of 16 bytes with
// chunk c of row r at slot c ^ (r & 7); one DMA instruction of a wave fills 8
// consecutive rows (1 KiB), lane L writing slot L % 8 of row L / 8 and
// therefore reading global chunk (L % 8) ^ (L / 8) of that row.
//
// Ring discipline (NS stages, NS - 1 K steps in flight): before step kb each
// wave waits until its own DMAs of stage kb have landed (vmcnt, counting the
// NS - 2 younger stages it has issued), then a barrier makes every wave's
// stage kb visible and proves that step kb - 1 -- whose buffer is refilled
// next -- has been consumed by all waves.  Every iteration issues exactly one
// stage (past the end it re-reads the last K step into the idle buffer), so
// the vmcnt arithmetic is the same in every iteration.  No other vector
// memory load may be issued inside the loop.
#pragma once

#include "mfma_fp8.h"

namespace vmamd {

typedef __attribute__((address_space(3))) void* lds_void_ptr;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// 16 (or 4) bytes per lane from g to the wave's LDS block at lds + lane * 16 (4).
__device__ __forceinline__ void dma16(const uint8_t* g, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_ptr)((lds_u8*)lds), 16, 0, 0);
}
__device__ __forceinline__ void dma4(const uint8_t* g, uint8_t* lds) {
  __builtin_amdgcn_global_load_lds(g, (lds_void_ptr)((lds_u8*)lds), 4, 0, 0);
}

// Buffer-descriptor forms of dma16 / dma4: a lane whose byte offset lies
// past the buffer's end fetches nothing.  (Unlike the global forms, these
// also leave the compiler free to wait for LDS reads one at a time.)
__device__ __forceinline__ void buffer_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint8_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_ptr)((lds_u8*)lds), 16, static_cast<int>(off), 0, 0, 0);
}
__device__ __forceinline__ void buffer_dma4(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint8_t* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_ptr)((lds_u8*)lds), 4, static_cast<int>(off), 0, 0, 0);
}

// Wait until at most N of this wave's vector-memory loads are outstanding
// (gfx9 s_waitcnt encoding: vmcnt in [3:0] and [15:14], expcnt and lgkmcnt
// left at their no-wait maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x70 | 0xF00);
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Workgroup barrier that the compiler may not move LDS accesses across, and
// that (unlike __syncthreads) does not wait for outstanding DMA loads.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// The 256 x 256 tile of the large-M GEMMs (dense and grouped): 8 waves as
// 4 (m) x 2 (n), 64 x 128 per wave, two LDS stages of
//   [A 256 x 128 B][B 256 x 128 B][A scales 256 x f32][B scales 64 x f32]
// filled by 4 + 4 row-group DMAs per wave (rows (wave + 8 j) * 8 + L / 8)
// and one scale DMA from waves 0-4.
struct BigTile {
  static constexpr int BM = 256, BN = 256, WM = 4, WN = 2, MT = 4, NT = 8, kWaves = 8;
  static constexpr int kThreads = kWaves * kWave;
  static constexpr int kOffB = BM * 128;
  static constexpr int kOffSA = (BM + BN) * 128;
  static constexpr int kOffSB = kOffSA + BM * 4;
  static constexpr int kStage = kOffSB + 256;  // the B-scale DMA writes 64 lanes x 4 bytes
  static constexpr int kLds = 2 * kStage;
  static_assert(BM / 8 == 4 * kWaves && BN / 8 == 4 * kWaves, "4 DMAs of 8 rows per wave and operand");
  static_assert(BN == 2 * 16 * NT && BM == 4 * 16 * MT, "wave tiles");
  static_assert(kLds <= 160 * 1024, "LDS stages exceed the CU's LDS");
};

template <bool SCALED, int BM, int BN, int WM, int WN, int NS>
struct TilePipe {
  static constexpr int kBM = BM, kBN = BN, kWN = WN;  // the tile and the waves across N
  static constexpr int kWaves = WM * WN, kThreads = kWaves * kWave;
  static constexpr int WTM = BM / WM, WTN = BN / WN, MT = WTM / 16, NT = WTN / 16;
  static constexpr int kOffB = BM * 128;
  static constexpr int kOffSA = (BM + BN) * 128;
  static constexpr int kOffSB = kOffSA + BM * 4;
  static constexpr int kStage = (BM + BN) * 128 + (SCALED ? BM * 4 + 64 * 4 : 0);
  static constexpr int kLds = NS * kStage;
  static constexpr int kGroupsA = BM / 8, kGroupsB = BN / 8;
  static_assert(kGroupsA % kWaves == 0 && kGroupsB % kWaves == 0, "row groups per wave");
  static constexpr int kDmaA = kGroupsA / kWaves, kDmaB = kGroupsB / kWaves;
  static constexpr int kScaleDma = SCALED ? 1 : 0;
  static constexpr int kIPS = kDmaA + kDmaB + kScaleDma;  // DMA instructions per stage per wave
  static_assert(!SCALED || BM / 64 < kWaves, "one wave must be left for the B scales");

  // Per lane: source of each of this wave's tile DMAs at K step 0, and of its
  // scale DMA (advanced by the per-step strides below).
  const uint8_t* srcA[kDmaA];
  const uint8_t* srcB[kDmaB];
  const uint8_t* srcS;
  int ldsA[kDmaA], ldsB[kDmaB], ldsS;  // wave-uniform LDS offsets inside a stage
  int stepS;                           // scale bytes per K step of this wave's scale DMA

  // Rows of the tile this lane fetches: A row (wave + j*kWaves)*8 + lane/8, etc.
  __device__ __forceinline__ static int rowA(int wave, int lane, int j) { return (wave + j * kWaves) * 8 + lane / 8; }
  __device__ __forceinline__ static int rowB(int wave, int lane, int j) { return (wave + j * kWaves) * 8 + lane / 8; }
  __device__ __forceinline__ static int chunk(int lane) { return ((lane % 8) ^ (lane / 8)) * 16; }

  __device__ __forceinline__ void issue(uint8_t* stage, int step) const {
#pragma unroll
    for (int j = 0; j < kDmaA; ++j) dma16(srcA[j] + static_cast<int64_t>(step) * 128, stage + ldsA[j]);
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) dma16(srcB[j] + static_cast<int64_t>(step) * 128, stage + ldsB[j]);
    if constexpr (SCALED) dma4(srcS + static_cast<int64_t>(step) * stepS, stage + ldsS);
  }
};

}  // namespace vmamd
