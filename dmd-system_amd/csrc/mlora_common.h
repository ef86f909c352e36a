// Shared device/host helpers for the gfx950 multi-LoRA kernels.
//
// Conventions used by every kernel in this library:
//   * bf16 values travel as raw uint16_t bit patterns; MFMA operands are
//     8 x bf16 = 16 bytes per lane, loaded as one u32x4.
//   * An LDS tile row holds 64 contraction elements = 8 chunks of 16 bytes.
//     Chunk c of row r is stored at chunk position c ^ swz(r) so that the 32
//     (or 16) lanes of one fragment read hit distinct banks.
//   * Segment/adapter routing arrives in kernel arguments (SegTable), copied
//     from the host arrays of the C ABI; no device-side metadata buffers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "../../include/mlora.h"

namespace mlora {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Explicit address spaces: LDS pointers stay ds_* instructions and global
// traffic goes through buffer resources (never generic flat accesses).
#define MLORA_LDS __attribute__((address_space(3)))
#define MLORA_GLOBAL __attribute__((address_space(1)))
typedef MLORA_LDS u32x4 lds_u4;
typedef MLORA_LDS f32x4 lds_f4;

template <class T>
__device__ __forceinline__ MLORA_GLOBAL T *gp(T *p) {
  return (MLORA_GLOBAL T *)p;
}

// Raw buffer resource over [base, base + bytes); loads at offsets >= bytes
// return zeros, which is how every loader masks rows/columns out of range.
constexpr uint32_t kBufFlags = 0x00020000u;  // gfx9 raw buffer, dword data format
constexpr int32_t kOOB = 0x7ffffff0;         // an offset past every buffer we build

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, int64_t bytes) {
  const int32_t n = bytes > (int64_t)kOOB ? kOOB : (bytes < 0 ? 0 : (int32_t)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, (int)kBufFlags);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, int32_t off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ float buf_load4f(__amdgpu_buffer_rsrc_t r, int32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

__device__ __forceinline__ void buf_store8(__amdgpu_buffer_rsrc_t r, int32_t off, uint2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned, v), r, off, 0, 0);
}

__device__ __forceinline__ void buf_store16(__amdgpu_buffer_rsrc_t r, int32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}

// The same store with the non-temporal cache policy (nt). For large outputs the
// next kernel then does not pay for the write-back of dirty L2 lines: a 201 MB
// streaming read right after a GEMM that wrote 201 MB took 36 us instead of
// 47-57 us on MI355X, and the GEMM itself was unchanged.
__device__ __forceinline__ void buf_store16_nt(__amdgpu_buffer_rsrc_t r, int32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 2);
}

constexpr int kMaxSeg = MLORA_MAX_SEGMENTS;
constexpr int kMaxAdapters = MLORA_MAX_ADAPTERS;
constexpr int kMaxRank = MLORA_MAX_RANK;
constexpr int kMaxGemmRank = MLORA_MAX_GEMM_RANK;

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

// fp32 -> bf16, round to nearest even (subnormals kept), with the gfx950
// conversion v_cvt_pk_bf16_f32 (one instruction for two values; the integer
// restatement of RNE took ~6 VALU operations per value in every epilogue).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ uint32_t pack2_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, bf16x2{(__bf16)lo, (__bf16)hi});
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Split 8 fp32 values into hi = bf16(v) and lo = bf16(v - hi): hi + lo carries
// ~16 significant bits, so one bf16 MFMA per part keeps fp32-class accuracy
// for the adapter-gradient reductions.
__device__ __forceinline__ void split_hi_lo(const float (&v)[8], u32x4 &hi, u32x4 &lo) {
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
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}

// Transpose an 8x8 block of 16-bit values held as 8 rows of u32x4
// (row e = 8 consecutive columns). Output t holds column t as 8 values
// (element e = row e).
__device__ __forceinline__ uint32_t word_of(const u32x4 &v, int i) {
  return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ void transpose8x8_b16(const u32x4 (&in)[8], u32x4 (&out)[8]) {
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
    out[t] = u32x4{o[0], o[1], o[2], o[3]};
  }
}

// Wave index within the workgroup, as a value the compiler knows is uniform
// (threadIdx.x >> 6 alone is treated as divergent, which would force
// waterfall loops around scalar buffer operands and M0 writes).
// Four pairs of ds_read_b64_tr_b16 (gfx950 transposing LDS read) followed by a
// wait for their data, as one inline-assembly block: pair t reads at a[t] and
// a[t] + OFF2 bytes. Within each 16-lane group, lane j of a read receives
// element (j & 3) of the 8 bytes addressed by lanes 4e + (j >> 2), e = 0..3.
// The compiler's builtin for this instruction carries no memory-operand
// information, so the compiler makes it wait for every direct-to-LDS load
// still in flight (vmcnt(0)), which drains the load pipelines; in assembly the
// reads see only the LDS stage they name (the caller's barriers order it), and
// the trailing lgkmcnt(0) makes the outputs valid where the compiler uses them.
template <int OFF2>
__device__ __forceinline__ void lds_read_tr16_x4(const MLORA_LDS char *base, const int32_t (&a)[4], u32x4 (&out)[4]) {
  u32x2 r0, r1, r2, r3, r4, r5, r6, r7;
  const uint32_t b = (uint32_t)(uintptr_t)base;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %2, %9\n\t"
      "ds_read_b64_tr_b16 %3, %9 offset:%12\n\t"
      "ds_read_b64_tr_b16 %4, %10\n\t"
      "ds_read_b64_tr_b16 %5, %10 offset:%12\n\t"
      "ds_read_b64_tr_b16 %6, %11\n\t"
      "ds_read_b64_tr_b16 %7, %11 offset:%12\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4), "=&v"(r5), "=&v"(r6), "=&v"(r7)
      : "v"(b + a[0]), "v"(b + a[1]), "v"(b + a[2]), "v"(b + a[3]), "i"(OFF2)
      : "memory");
  out[0] = u32x4{r0[0], r0[1], r1[0], r1[1]};
  out[1] = u32x4{r2[0], r2[1], r3[0], r3[1]};
  out[2] = u32x4{r4[0], r4[1], r5[0], r5[1]};
  out[3] = u32x4{r6[0], r6[1], r7[0], r7[1]};
}

// The same for two pairs.
template <int OFF2>
__device__ __forceinline__ void lds_read_tr16_x2(const MLORA_LDS char *base, const int32_t (&a)[2], u32x4 (&out)[2]) {
  u32x2 r0, r1, r2, r3;
  const uint32_t b = (uint32_t)(uintptr_t)base;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4\n\t"
      "ds_read_b64_tr_b16 %1, %4 offset:%6\n\t"
      "ds_read_b64_tr_b16 %2, %5\n\t"
      "ds_read_b64_tr_b16 %3, %5 offset:%6\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(b + a[0]), "v"(b + a[1]), "i"(OFF2)
      : "memory");
  out[0] = u32x4{r0[0], r0[1], r1[0], r1[1]};
  out[1] = u32x4{r2[0], r2[1], r3[0], r3[1]};
}

// One pair.
template <int OFF2>
__device__ __forceinline__ void lds_read_tr16_x1(const MLORA_LDS char *base, int32_t a, u32x4 &out) {
  u32x2 r0, r1;
  const uint32_t b = (uint32_t)(uintptr_t)base;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %2\n\t"
      "ds_read_b64_tr_b16 %1, %2 offset:%3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1)
      : "v"(b + a), "i"(OFF2)
      : "memory");
  out = u32x4{r0[0], r0[1], r1[0], r1[1]};
}

// N pairs (N = 1, 2, 4 or 8), each pair at a[t] and a[t] + OFF2 bytes.
template <int N, int OFF2>
__device__ __forceinline__ void lds_read_tr16(const MLORA_LDS char *base, const int32_t (&a)[N], u32x4 (&out)[N]) {
  if constexpr (N == 1) {
    lds_read_tr16_x1<OFF2>(base, a[0], out[0]);
  } else if constexpr (N == 2) {
    lds_read_tr16_x2<OFF2>(base, a, out);
  } else if constexpr (N == 4) {
    lds_read_tr16_x4<OFF2>(base, a, out);
  } else {
    static_assert(N == 8, "1, 2, 4 or 8 pairs");
    const int32_t lo[4] = {a[0], a[1], a[2], a[3]}, hi[4] = {a[4], a[5], a[6], a[7]};
    u32x4 o0[4], o1[4];
    lds_read_tr16_x4<OFF2>(base, lo, o0);
    lds_read_tr16_x4<OFF2>(base, hi, o1);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      out[t] = o0[t];
      out[t + 4] = o1[t];
    }
  }
}

// Workgroup barrier for LDS pipelines fed by direct-to-LDS loads: waits for
// this wave's LDS reads, then s_barrier, with compiler-level memory fences on
// both sides. __syncthreads() would also wait for every direct-to-LDS load in
// flight (its release fence covers LDS writes), so callers wait explicitly,
// with vmcnt, for just the loads the next stage needs.
__device__ __forceinline__ void lds_pipeline_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// f(integral_constant<int, 0>), f(..1), ... f(..N-1), stopping at the first false.
template <class F, int... K>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, K...>) {
  (void)(f(std::integral_constant<int, K>{}) && ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// vmcnt(n) with the other counters left alone (gfx9 s_waitcnt encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// ---------------------------------------------------------------- LDS layout

// Chunk swizzle for a tile with 8 chunks (128 bytes) per row: chunk c of row r
// sits at slot c ^ swz(r). Any 16 consecutive rows read at one chunk then cover
// 16 distinct 16-byte bank groups (slot bits from r%8, parity from r/8), and
// the swizzle of row r depends only on r mod 16, so every MFMA fragment row
// (32-aligned base + lane) has a lane-constant swizzle.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
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

// The same for any grid size: XCD x (bids x, x + 8, ...) takes the contiguous logical ids
// [x·q + min(x, m), ...) of its share (q = nblocks / 8, m = nblocks % 8; the first m XCDs take
// one more). A bijection on [0, nblocks).
__device__ __forceinline__ int xcd_contiguous(int bid, int nblocks) {
  constexpr int kXcd = 8;
  const int x = bid % kXcd, q = nblocks / kXcd, m = nblocks % kXcd;
  return x * q + (x < m ? x : m) + bid / kXcd;
}

}  // namespace mlora
