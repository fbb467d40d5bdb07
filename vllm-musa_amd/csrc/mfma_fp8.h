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

// 8 signed int4 values (element 2j in the low nibble of byte j of `x`, 2j+1
// in the high nibble) -> their 8 e4m3 codes, in element order.  Every integer
// in [-8, 7] is exact in e4m3.  The even and the odd elements are taken as
// two byte planes; in each, a byte-permute lookup on the nibble's low three
// bits reads the codes of 0..7 and another those of -8..-1, and the nibble's
// sign (bit 3) selects between them through a per-byte mask that v_perm_b32
// itself builds (selectors 8..11 replicate bit 7 of bytes 1 and 3 of either
// source dword: the mask of x needs the sign bits at bit 7 of every byte,
// which x has for the odd plane and x << 4 for the even one, and x << 8 moves
// bytes 0 and 2 into the positions the selectors read).  Two more permutes
// re-interleave the planes.  16 VALU operations per 8 elements.
__device__ __forceinline__ uint2 int4x8_to_fp8(uint32_t x) {
  constexpr uint32_t kPosLo = 0x44403800u, kPosHi = 0x4E4C4A48u;  // e4m3 of 0..7
  constexpr uint32_t kNegLo = 0xCACCCED0u, kNegHi = 0xB8C0C4C8u;  // e4m3 of -8..-1
  constexpr uint32_t kSignSel = 0x090B080Au;  // byte i <- bit 7 of byte i of q, from {q << 8, q}
  const uint32_t se = x & 0x07070707u, so = (x >> 4) & 0x07070707u;
  const uint32_t qe = x << 4;  // bit 7 of byte i: sign of the even element i
  const uint32_t me = __builtin_amdgcn_perm(qe << 8, qe, kSignSel);
  const uint32_t mo = __builtin_amdgcn_perm(x << 8, x, kSignSel);
  const uint32_t ce = (__builtin_amdgcn_perm(kNegHi, kNegLo, se) & me) |
                      (__builtin_amdgcn_perm(kPosHi, kPosLo, se) & ~me);
  const uint32_t co = (__builtin_amdgcn_perm(kNegHi, kNegLo, so) & mo) |
                      (__builtin_amdgcn_perm(kPosHi, kPosLo, so) & ~mo);
  return uint2{__builtin_amdgcn_perm(co, ce, 0x05010400u), __builtin_amdgcn_perm(co, ce, 0x07030602u)};
}
__device__ __forceinline__ v4i int4x16_to_fp8(uint2 p) {
  const uint2 a = int4x8_to_fp8(p.x), b = int4x8_to_fp8(p.y);
  return v4i{static_cast<int>(a.x), static_cast<int>(a.y), static_cast<int>(b.x), static_cast<int>(b.y)};
}

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

// Operand fragment of one 128-element K-block of a packed int4 row (64 bytes
// at p), converted to e4m3 in the same K order as global_frag: lane group g
// takes elements [16g, 16g+16) and [64+16g, 64+16g+16).
// The packed bytes of such a fragment (16 bytes per lane, kept packed until
// the MFMA needs them), and their conversion.
__device__ __forceinline__ uint4 global_frag_int4_raw(const uint8_t* p, int g) {
  const uint2 lo = *reinterpret_cast<const uint2*>(p + 8 * g);
  const uint2 hi = *reinterpret_cast<const uint2*>(p + 32 + 8 * g);
  return uint4{lo.x, lo.y, hi.x, hi.y};
}
__device__ __forceinline__ v8i int4_frag_to_fp8(const uint4& raw) {
  const v4i a = int4x16_to_fp8(uint2{raw.x, raw.y}), b = int4x16_to_fp8(uint2{raw.z, raw.w});
  v8i f;
  f[0] = a[0]; f[1] = a[1]; f[2] = a[2]; f[3] = a[3];
  f[4] = b[0]; f[5] = b[1]; f[6] = b[2]; f[7] = b[3];
  return f;
}
__device__ __forceinline__ v8i global_frag_int4(const uint8_t* p, int g) {
  return int4_frag_to_fp8(global_frag_int4_raw(p, g));
}

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
  r.x = static_cast<uint32_t>(f32_to_bf16(a)) | (static_cast<uint32_t>(f32_to_bf16(b)) << 16);
  r.y = static_cast<uint32_t>(f32_to_bf16(c)) | (static_cast<uint32_t>(f32_to_bf16(d)) << 16);
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
