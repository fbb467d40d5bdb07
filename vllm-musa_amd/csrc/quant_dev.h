// Device parts of the 1x128 group quantiser, shared by its own kernel and by
// the fused align + quantise launch of the MoE layer:
//   s = max(eps, amax of the group) / qmax,  q = e4m3fn(clamp(x / s, qmin, qmax)),
// one 16-lane segment per 128-column group, 8 columns per lane.
#pragma once

#include "common.h"

namespace vmamd {

constexpr int kGroup = 128;
constexpr int kLanesPerGroup = 16;
constexpr int kElemsPerLane = kGroup / kLanesPerGroup;  // 8
constexpr int kQuantThreads = 256;
constexpr int kGroupsPerBlock = kQuantThreads / kLanesPerGroup;  // 16

template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::T* p, bool vec, float (&v)[8]) {
  using T = typename Elem<DT>::T;
  if constexpr (sizeof(T) == 2) {
    if (vec) {
      uint4 raw = *reinterpret_cast<const uint4*>(p);
      const uint16_t* h = reinterpret_cast<const uint16_t*>(&raw);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = Elem<DT>::to_f(h[i]);
      return;
    }
  } else {
    if (vec) {
      float4 a = reinterpret_cast<const float4*>(p)[0];
      float4 b = reinterpret_cast<const float4*>(p)[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = Elem<DT>::load(p, i);
}

__device__ __forceinline__ uint2 quant8(const float (&v)[8], float s, float qmin, float qmax) {
  float q[8];
  if (s < __builtin_inff()) {  // one division for the eight quotients (div_rn)
    const float r = 1.0f / s;
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = fminf(fmaxf(div_rn(v[i], s, r), qmin), qmax);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = fminf(fmaxf(v[i] / s, qmin), qmax);
  }
  uint2 out;
  out.x = f32x4_to_fp8x4(q[0], q[1], q[2], q[3]);
  out.y = f32x4_to_fp8x4(q[4], q[5], q[6], q[7]);
  return out;
}

// Group g (row g / groups_per_row) by the 16 lanes of one segment; sub is
// the lane's index in the segment.  Every lane of the segment must call it.
template <int DT>
__device__ __forceinline__ void group_quant_group(
    const typename Elem<DT>::T* __restrict__ x, int64_t x_row_stride, int64_t groups_per_row,
    int64_t g, int sub, bool vec, float eps, float qmin, float qmax, uint8_t* __restrict__ q,
    int64_t q_row_stride, float* __restrict__ s, int64_t s_stride_row, int64_t s_stride_group) {
  const int64_t row = g / groups_per_row;
  const int64_t grp = g - row * groups_per_row;
  const int64_t col = grp * kGroup + sub * kElemsPerLane;

  float v[8];
  load8<DT>(x + row * x_row_stride + col, vec, v);
  float amax = eps;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = group_max<kLanesPerGroup>(amax);
  const float scale = amax / qmax;
  if (sub == 0) s[row * s_stride_row + grp * s_stride_group] = scale;
  *reinterpret_cast<uint2*>(q + row * q_row_stride + col) = quant8(v, scale, qmin, qmax);
}

// ------------------------------------------------- per-row quantiser -----
// s[r] = max(eps, max_c |x[r,c]|) / qmax over the whole row,
// q[r,c] = e4m3(clamp(x[r,c] / s[r], qmin, qmax)).  One 256-thread block per
// row, 8 columns per thread per pass; up to kRowChunks passes stay in
// registers between the amax and the quantise steps.
constexpr int kRowThreads = 256;
constexpr int kRowChunks = 8;  // rows of up to 256 * 8 * 8 = 16384 columns

// w4afp8 activation chunk (8 consecutive columns 8ch.., ch = a chunk index
// of the row): quantised with `scale`, stored in w4 order ([0, 2, 4, 6, 1, 3,
// 5, 7], the order the int4 weight fragments take), and the row's offset
// correction of each 128-column block, corr[ch / 16] = -(sum of the block's
// 128 e4m3 values) / 64, written by the chunk's first lane.  The 16 chunks of
// a block must sit in 16 consecutive lanes (chunk index = lane + a multiple
// of 16) that all call this; the block sum is taken in a fixed order (8
// values in sequence, then an xor butterfly over the 16 lanes).
__device__ __forceinline__ void w4_store_chunk(uint8_t* __restrict__ qrow, float* __restrict__ corr_row,
                                               int ch, const float (&v)[8], float scale, float qmin,
                                               float qmax) {
  const float o[8] = {v[0], v[2], v[4], v[6], v[1], v[3], v[5], v[7]};
  const uint2 b = quant8(o, scale, qmin, qmax);
  *reinterpret_cast<uint2*>(qrow + ch * 8) = b;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) s += fp8_to_f32((b.x >> (8 * j)) & 0xFFu);
#pragma unroll
  for (int j = 0; j < 4; ++j) s += fp8_to_f32((b.y >> (8 * j)) & 0xFFu);
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) s += __shfl_xor(s, m, kWave);
  if ((ch & 15) == 0) corr_row[ch / 16] = s * (-1.0f / 64.0f);
}

// Per-row quantiser (w4afp8 activations): s = max(eps, amax of the row) /
// qmax, q = e4m3fn(clamp(x / s, qmin, qmax)).  A part of kRowThreads threads
// (t = 0 .. kRowThreads - 1 within it) handles one bf16 row; red holds the
// part's kRowThreads / 64 wave maxima.  Every thread of the block must call
// it (it synchronises the block); live = false parts only take part in the
// barrier.  W4: q in w4 order plus the block corrections corr [rows,
// cols / 128] (w4_store_chunk; cols a multiple of 128).
template <bool W4 = false>
__device__ __forceinline__ void row_quant_part(const uint16_t* __restrict__ x, int64_t x_row_stride,
                                               int cols, float eps, float qmin, float qmax,
                                               uint8_t* __restrict__ q, float* __restrict__ s,
                                               int64_t row, bool live, int t, float* red,
                                               float* __restrict__ corr = nullptr) {
  const uint16_t* xr = x + row * x_row_stride;
  const int nchunk = live ? cols / 8 : 0;
  float v[kRowChunks][8];
  float amax = eps;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int ch = t + c * kRowThreads;
    if (ch < nchunk) {
      load8<kBF16>(xr + ch * 8, true, v[c]);
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
    }
  }
  amax = wave_max(amax);
  if (lane_id() == 0) red[t / kWave] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kRowThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
  const float scale = amax / qmax;
  if (live && t == 0) s[row] = scale;
#pragma unroll
  for (int c = 0; c < kRowChunks; ++c) {
    const int ch = t + c * kRowThreads;
    if (ch < nchunk) {
      if constexpr (W4)
        w4_store_chunk(q + row * cols, corr + row * (cols / 128), ch, v[c], scale, qmin, qmax);
      else
        *reinterpret_cast<uint2*>(q + row * cols + ch * 8) = quant8(v[c], scale, qmin, qmax);
    }
  }
}

// The per-row quantiser with one wave per row (no block barrier; several rows
// per workgroup): lane l takes chunks l, l + 64, ... (CPL of them, cols <=
// 512 * CPL), the same maximum (order-independent) and the same bytes as
// row_quant_part.  Every lane of the wave must call it; rows past the end
// (live = false) return before any cross-lane step, wave-uniformly.
template <bool W4, int CPL>
__device__ __forceinline__ void row_quant_wave(const uint16_t* __restrict__ x, int64_t x_row_stride,
                                               int cols, float eps, float qmin, float qmax,
                                               uint8_t* __restrict__ q, float* __restrict__ s,
                                               int64_t row, bool live, float* __restrict__ corr) {
  if (!live) return;
  const int lane = lane_id();
  const uint16_t* xr = x + row * x_row_stride;
  const int nchunk = cols / 8;
  float v[CPL][8];
  float amax = eps;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + c * kWave;
    if (ch < nchunk) {
      load8<kBF16>(xr + ch * 8, true, v[c]);
#pragma unroll
      for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[c][j]));
    }
  }
  amax = wave_max(amax);
  const float scale = amax / qmax;
  if (lane == 0) s[row] = scale;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = lane + c * kWave;
    if (ch < nchunk) {
      if constexpr (W4)
        w4_store_chunk(q + row * cols, corr + row * (cols / 128), ch, v[c], scale, qmin, qmax);
      else
        *reinterpret_cast<uint2*>(q + row * cols + ch * 8) = quant8(v[c], scale, qmin, qmax);
    }
  }
}

}  // namespace vmamd
