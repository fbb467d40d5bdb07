// Building blocks of the fp8 block-scaled and bf16 GEMMs on CDNA4 MFMA.
//
// MFMA shape: v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3 -> f32), one K-block of
// the 128x128 scale grid per instruction.  The weight tile is the "A" operand
// (16 output rows n) and the activation tile the "B" operand (16 columns m),
// so lane (i = lane % 16, g = lane / 16) ends up holding
//     C[n = 4g + r][m = i],  r = 0..3
// -- four consecutive n of one row m: one activation scale and one weight-
// block scale per lane and K-block, and an 8-byte bf16 store per tile.
//
// Operand bytes: lane (i, g) supplies row i, bytes [16g, 16g+16) and
// [64+16g, 64+16g+16) of the 128-byte K-block, for both operands (any
// bijection of K that is the same for both operands gives the same dot
// product; this one makes every 16-lane group read 64 contiguous bytes).
//
// LDS tiles store a row as 8 chunks of 16 bytes with chunk c of row r at
// slot c ^ (r & 7), so the 8 lanes served per LDS cycle hit 8 distinct
// chunk slots (all banks) when reading the same chunk of 8 consecutive rows.
#pragma once

#include "common.h"

namespace vmamd {

__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * 128 + ((chunk ^ (row & 7)) << 4);
}

// Two chained v_mfma_f32_16x16x32_bf16 over one 128-byte row chunk (64 bf16
// of K): the low halves of the fragments (chunk g) are K-slice 0, the high
// halves (chunk g + 4) K-slice 1.  Both operands use the same K order, so the
// sum is the chunk's dot product.
__device__ __forceinline__ v4f mfma_bf16x2(const v8i& a, const v8i& b, v4f c) {
  const v4i alo = {a[0], a[1], a[2], a[3]}, ahi = {a[4], a[5], a[6], a[7]};
  const v4i blo = {b[0], b[1], b[2], b[3]}, bhi = {b[4], b[5], b[6], b[7]};
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, alo),
                                               __builtin_bit_cast(v8bf, blo), c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ahi),
                                               __builtin_bit_cast(v8bf, bhi), c, 0, 0, 0);
  return c;
}

// bf16 activations against fp8 weights (the W8A16 GEMVs).  The lane's fp8
// weight fragment (32 bytes in the layout above: K = 16g + e for byte e < 16,
// K = 64 + 16g + e - 16 above) becomes 32 bf16 values with
// v_cvt_scalef32_pk_bf16_fp8 at scale 1.0, which is exact: every e4m3 value,
// subnormals included, is a bf16 value.  The activation fragment holds the
// 32 bf16 activations of the same K positions in the same order, and four
// chained v_mfma_f32_16x16x32_bf16 take elements [8j, 8j + 8) of both, so the
// products (a bf16 times an e4m3 value: at most 12 significant bits) are exact
// and only the fp32 accumulation rounds.
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
__device__ __forceinline__ v4f mfma_w8a16(const v8i& w, const v16i& x, v4f c) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w0 = static_cast<uint32_t>(w[2 * j]), w1 = static_cast<uint32_t>(w[2 * j + 1]);
    const v4i a = {__builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, false)),
                   __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, 1.0f, true)),
                   __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, false)),
                   __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, 1.0f, true))};
    const v4i b = {x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3]};
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c,
                                                 0, 0, 0);
  }
  return c;
}

// w4afp8 weight operands.  A signed int4 weight x (two per byte, element 2j
// in the low nibble of byte j) enters the MFMA as the e4m3 code u = x + 8,
// which is the nibble with its top bit flipped.  Codes 0..15 are the e4m3
// subnormals and the first normal binade, which are evenly spaced: code u has
// the value u * 2^-9 exactly, and the fp8 MFMA takes subnormal inputs at their
// value.  So a weight costs one XOR and one mask (the odd elements one shift
// more) instead of a table lookup.  The offset leaves the accumulator input:
// with c = -(sum_k a_k) / 64 for the activation row and K block (8 * 2^-9 =
// 2^-6),
//     mfma(u, a, c) = 2^-9 * sum_k a_k * x_k,
// so every block product carries a factor 2^-9, which the epilogues undo
// (times kW4Unit = 512, exact).
//
// The even elements of a 32-bit word of packed weights become one byte plane
// and the odd elements another, so within every 8 K-elements the weight bytes
// run [0, 2, 4, 6, 1, 3, 5, 7].  The activations are stored in that order by
// their quantisers ("w4 order"), and lane group g of a fragment takes the 32
// contiguous elements [32g, 32g + 32) of the K block: packed weight bytes
// [16g, 16g + 16), activation bytes [32g, 32g + 32).
constexpr float kW4Unit = 512.0f;

// 16 packed bytes (32 int4 in K order) -> the 32 e4m3 codes x + 8, w4 order.
// v_bitop3_b32 with table 0x28 computes (s0 ^ s1) & s2.
__device__ __forceinline__ v8i w4_frag(const v4i& raw) {
  v8i f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t w = static_cast<uint32_t>(raw[j]);
    f[2 * j] = static_cast<int>(__builtin_amdgcn_bitop3_b32(w, 0x88888888u, 0x0F0F0F0Fu, 0x28));
    f[2 * j + 1] = static_cast<int>(__builtin_amdgcn_bitop3_b32(w >> 4, 0x88888888u, 0x0F0F0F0Fu, 0x28));
  }
  return f;
}

// The accumulator input {c, c, c, c} of one MFMA (c: the activation row's
// offset correction for the K block).
__device__ __forceinline__ v4f splat4(float c) { return v4f{c, c, c, c}; }

// Loads from LDS through address-space-3 pointers, so the compiler knows
// they touch LDS (a read through a generic pointer makes it wait for every
// outstanding global->LDS DMA first).
template <typename T>
__device__ __forceinline__ T lds_load(const uint8_t* base, int off) {
  typedef __attribute__((address_space(3))) const T lds_t;
  return *(lds_t*)((const __attribute__((address_space(3))) uint8_t*)base + off);
}

// Operand fragment of `row` from an LDS tile.
__device__ __forceinline__ v8i lds_frag(const uint8_t* tile, int row, int g) {
  const v4i lo = lds_load<v4i>(tile, lds_off(row, g));
  const v4i hi = lds_load<v4i>(tile, lds_off(row, g + 4));
  v8i f;
  f[0] = lo[0]; f[1] = lo[1]; f[2] = lo[2]; f[3] = lo[3];
  f[4] = hi[0]; f[5] = hi[1]; f[6] = hi[2]; f[7] = hi[3];
  return f;
}

// Operand fragment straight from global memory (row start + K-block start).
__device__ __forceinline__ v8i global_frag(const uint8_t* p, int g) {
  const uint4 lo = *reinterpret_cast<const uint4*>(p + 16 * g);
  const uint4 hi = *reinterpret_cast<const uint4*>(p + 64 + 16 * g);
  v8i f;
  f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
  f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
  return f;
}

// 16-byte global / LDS moves in a native vector type (keeps prefetch arrays in
// registers: the compiler can scalarise them, which it does not do reliably
// for the HIP uint4 struct).
__device__ __forceinline__ v4i ld16(const uint8_t* p) { return *reinterpret_cast<const v4i*>(p); }
__device__ __forceinline__ void st16(uint8_t* p, const v4i& v) { *reinterpret_cast<v4i*>(p) = v; }

// acc += p * s, element-wise (the per-K-block scale promotion).
__device__ __forceinline__ void fma4(v4f& acc, const v4f& p, float s) {
  acc[0] = fmaf(p[0], s, acc[0]);
  acc[1] = fmaf(p[1], s, acc[1]);
  acc[2] = fmaf(p[2], s, acc[2]);
  acc[3] = fmaf(p[3], s, acc[3]);
}

// acc[r] += p[r] * s[r] (per-row weight scales of the w4afp8 kernels).
__device__ __forceinline__ void fma4v(v4f& acc, const v4f& p, const v4f& s) {
  acc[0] = fmaf(p[0], s[0], acc[0]);
  acc[1] = fmaf(p[1], s[1], acc[1]);
  acc[2] = fmaf(p[2], s[2], acc[2]);
  acc[3] = fmaf(p[3], s[3], acc[3]);
}

__device__ __forceinline__ uint2 pack_bf16x4(float a, float b, float c, float d) {
  uint2 r;
  r.x = f32x2_to_bf16x2(a, b);
  r.y = f32x2_to_bf16x2(c, d);
  return r;
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2).  Give each XCD a contiguous range of logical tiles and walk that
// range in bands of kGroupM row-tiles, so the tiles resident on one XCD at a
// time share activation rows and weight columns in its L2.  Returns false for
// the (at most 7) padding workgroups of a grid rounded up to a multiple of 8.
constexpr int kXcds = 8;
constexpr int kGroupM = 8;

__host__ __device__ inline int xcd_grid(int total) { return (total + kXcds - 1) / kXcds * kXcds; }

__device__ __forceinline__ bool xcd_tile(int wg, int TM, int TN, int& tm, int& tn) {
  const int total = TM * TN;
  const int per = (total + kXcds - 1) / kXcds;
  const int L = (wg % kXcds) * per + wg / kXcds;
  if (L >= total) return false;
  const int band = L / (kGroupM * TN);
  const int first = band * kGroupM;
  const int gsz = min(TM - first, kGroupM);
  const int in = L - band * kGroupM * TN;
  tm = first + in % gsz;
  tn = in / gsz;
  return true;
}

}  // namespace vmamd
