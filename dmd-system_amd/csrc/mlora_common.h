// Shared device/host helpers for the gfx950 multi-LoRA kernels.
//
// Conventions used by every kernel in this library:
//   * bf16 values travel as raw uint16_t bit patterns; MFMA operands are
//     8 x bf16 = 16 bytes per lane, loaded as one uint4.
//   * An LDS tile row holds 64 contraction elements = 8 chunks of 16 bytes.
//     Chunk c of row r is stored at chunk position c ^ swz(r) so that the 32
//     (or 16) lanes of one fragment read hit distinct banks.
//   * Segment/adapter routing arrives in kernel arguments (SegTable), copied
//     from the host arrays of the C ABI; no device-side metadata buffers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mlora.h"

namespace mlora {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxSeg = MLORA_MAX_SEGMENTS;
constexpr int kMaxAdapters = MLORA_MAX_ADAPTERS;
constexpr int kMaxRank = MLORA_MAX_RANK;

// Routing for one call. off[] are row offsets (int32: one call covers < 2^31 rows).
struct SegTable {
  int32_t n;
  int32_t off[kMaxSeg + 1];
  int32_t aid[kMaxSeg];
};

// Per-adapter operand table (device pointers) plus ranks and scales.
struct AdapterTable {
  const uint16_t *ptr[kMaxAdapters];
  int32_t rank[kMaxAdapters];
  float scale[kMaxAdapters];
};

// ---------------------------------------------------------------- conversions

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  return (uint32_t)f32_to_bf16_rne(lo) | ((uint32_t)f32_to_bf16_rne(hi) << 16);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// Split 8 fp32 values into hi = bf16(v) and lo = bf16(v - hi): hi + lo carries
// ~16 significant bits, so one bf16 MFMA per part keeps fp32-class accuracy
// for the adapter-gradient reductions.
__device__ __forceinline__ void split_hi_lo(const float (&v)[8], uint4 &hi, uint4 &lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint16_t h0 = f32_to_bf16_rne(v[2 * i]);
    uint16_t h1 = f32_to_bf16_rne(v[2 * i + 1]);
    float r0 = v[2 * i] - bf16_to_f32(h0);
    float r1 = v[2 * i + 1] - bf16_to_f32(h1);
    h[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    l[i] = pack2_bf16(r0, r1);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// Transpose an 8x8 block of 16-bit values held as 8 rows of uint4
// (row e = 8 consecutive columns). Output t holds column t as 8 values
// (element e = row e).
__device__ __forceinline__ uint32_t word_of(const uint4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ void transpose8x8_b16(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    uint32_t o[4];
    const int word = t >> 1;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t a = word_of(in[2 * q], word), b = word_of(in[2 * q + 1], word);
      // element t of rows 2q (low half) and 2q+1 (high half)
      o[q] = (t & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
    }
    out[t] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---------------------------------------------------------------- LDS layout

// Chunk swizzle for a tile with 8 chunks (128 bytes) per row.
__device__ __forceinline__ int swz(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int lds_chunk_offset(int row, int chunk) { return row * 8 + (chunk ^ swz(row)); }

// ---------------------------------------------------------------- routing

// First segment s with off[s+1] > row (segments are nondecreasing).
__device__ __forceinline__ int seg_of_row(const SegTable &seg, int row) {
  int lo = 0, hi = seg.n - 1;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (seg.off[mid + 1] > row) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// Map a linear workgroup id so that consecutive logical ids run on the same
// XCD (workgroups are dealt round-robin over the 8 XCDs of MI355X).
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  constexpr int kXcd = 8;
  if (nblocks % kXcd != 0) return bid;
  return (bid % kXcd) * (nblocks / kXcd) + bid / kXcd;
}

}  // namespace mlora
