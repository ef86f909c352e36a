// e4m3 (OCP E4M3FN: bias 7, max 448, no infinities) conversions for the
// quantised-base variant of the multi-LoRA linear:
//
//   mlora_quantize_rows_fp8 : per-row absmax scaling of a bf16 matrix, each
//                             column optionally multiplied by an fp32 factor
//                             first, to e4m3 (activations X before the fp8 base
//                             GEMM; dY·w_scale before the fp8 dX GEMM)
//   mlora_dequant_rows_fp8  : e4m3 rows times a per-row fp32 scale back to bf16
//                             (the frozen base W for the bf16 dX GEMM)
//   mlora_div_rows_bf16     : bf16 rows divided by a per-row fp32 value
//                             (lora_b / w_scale for the e4m3 forward); the
//                             _batch form divides several such matrices (every
//                             adapter's lora_b) in one launch
//
// Quantisation of row m: v[k] = x[m,k] (times col_scale[k] when given, one
// fp32 product); amax = max_k |v[k]|; scale[m] = amax / 448 and
// q = e4m3_rne(v * (448 / amax)) (both divisions IEEE fp32; an all-zero row
// gets scale 1). Round to nearest even on the 3 mantissa bits, subnormals in
// steps of 2^-9; |x·(448/amax)| <= 448 so nothing saturates.
//
// One wave per row. Rows of up to 9216 elements are loaded once into
// registers (all 16-byte loads of the row in flight together), reduced to the
// absmax and written back as 8 bytes per lane; longer rows take two passes
// (the second re-reads the row, an L2 hit). Memory-bound: 3 bytes of HBM
// traffic per element.
#include "mlora_common.h"
#include "mlora_host.h"

namespace mlora {

// Four values (each |v| <= 448) to e4m3 bytes 0..3 of a dword with the gfx950
// packed conversion (v_cvt_pk_fp8_f32: OCP e4m3, round to nearest even, the
// subnormal grid included).
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  const uint32_t sign = (c & 0x80u) << 24, e = (c >> 3) & 15u, m = c & 7u;
  if (e == 0) return __uint_as_float(sign | __float_as_uint((float)m * 0.001953125f));  // m * 2^-9
  return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

struct QuantArgs {
  const uint16_t *x;
  const float *cs;  // per-column factor or nullptr
  uint8_t *q;
  float *scale;
  int64_t ldx, ldq;
  int32_t M, K;
};

// The 8 values of bf16 chunk v (columns k..k+7), times the column factors when CS.
template <bool CS>
__device__ __forceinline__ void chunk_values(const u32x4 &v, const QuantArgs &a, int k, float (&o)[8]) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    o[2 * w] = bf16_to_f32(v[w] & 0xffff);
    o[2 * w + 1] = bf16_to_f32(v[w] >> 16);
  }
  if constexpr (CS) {
    if (k < a.K) {  // K is a multiple of 8: a chunk is all in range or all past K
      const f32x4 c0 = *(const MLORA_GLOBAL f32x4 *)(a.cs + k), c1 = *(const MLORA_GLOBAL f32x4 *)(a.cs + k + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] *= c0[e];
        o[4 + e] *= c1[e];
      }
    }
  }
}

template <bool CS>
__global__ __launch_bounds__(256) void quantize_rows_kernel(const QuantArgs a) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + wave_id();
  if (m >= a.M) return;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (int64_t)m * a.ldx, (int64_t)a.K * 2);
  float amax = 0.f;
  for (int k = 8 * lane; k < a.K; k += 512) {
    float f[8];
    chunk_values<CS>(buf_load16(rx, 2 * k), a, k, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
  }
  amax = wave_max(amax);
  const float inv = amax > 0.f ? 448.f / amax : 1.f;
  if (lane == 0) a.scale[m] = amax > 0.f ? amax / 448.f : 1.f;
  uint8_t *qrow = a.q + (int64_t)m * a.ldq;
  for (int k = 8 * lane; k < a.K; k += 512) {
    float f[8];
    chunk_values<CS>(buf_load16(rx, 2 * k), a, k, f);
    const uint32_t o0 = pack4_e4m3(f[0] * inv, f[1] * inv, f[2] * inv, f[3] * inv);
    const uint32_t o1 = pack4_e4m3(f[4] * inv, f[5] * inv, f[6] * inv, f[7] * inv);
    *(MLORA_GLOBAL u32x2 *)(qrow + k) = u32x2{o0, o1};
  }
}

// Row held in registers: NI 16-byte chunks per lane (K <= 512 * NI). With
// column factors (CS) the products are formed once, in the absmax pass, and
// kept as fp32 for the conversion pass; the factors are first copied to LDS by
// the whole workgroup (its four rows share them), so the absmax pass reads
// them at LDS latency instead of waiting on a global load per chunk.
template <int NI, bool CS>
__global__ __launch_bounds__(256) void quantize_rows_reg_kernel(const QuantArgs a) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + wave_id();
  __shared__ f32x4 cs_lds[CS ? 128 * NI : 1];  // K <= 512 * NI factors
  if constexpr (CS) {
    for (int i = (int)threadIdx.x; i < a.K / 4; i += 256) cs_lds[i] = *(const MLORA_GLOBAL f32x4 *)(a.cs + 4 * i);
    __syncthreads();  // before any wave leaves: every wave of the workgroup reaches it
  }
  if (m >= a.M) return;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x + (int64_t)m * a.ldx, (int64_t)a.K * 2);
  u32x4 v[NI];
#pragma unroll
  for (int it = 0; it < NI; ++it) v[it] = buf_load16(rx, 2 * (8 * lane + 512 * it));  // past K: reads zero
  float amax = 0.f;
  float f[CS ? NI : 1][8];
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    float t[8];
    const int k = 8 * lane + 512 * it;
    chunk_values<false>(v[it], a, k, t);
    if constexpr (CS) {
      if (k < a.K) {  // K is a multiple of 8: a chunk is all in range or all past K
        const f32x4 c0 = cs_lds[k / 4], c1 = cs_lds[k / 4 + 1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          t[e] *= c0[e];
          t[4 + e] *= c1[e];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      amax = fmaxf(amax, fabsf(t[e]));
      if constexpr (CS) f[it][e] = t[e];
    }
  }
  amax = wave_max(amax);
  const float inv = amax > 0.f ? 448.f / amax : 1.f;
  if (lane == 0) a.scale[m] = amax > 0.f ? amax / 448.f : 1.f;
  uint8_t *qrow = a.q + (int64_t)m * a.ldq;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int k = 8 * lane + 512 * it;
    if (k >= a.K) break;
    float t[8];
    if constexpr (CS) {
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = f[it][e];
    } else {
      chunk_values<false>(v[it], a, k, t);
    }
    const uint32_t o0 = pack4_e4m3(t[0] * inv, t[1] * inv, t[2] * inv, t[3] * inv);
    const uint32_t o1 = pack4_e4m3(t[4] * inv, t[5] * inv, t[6] * inv, t[7] * inv);
    *(MLORA_GLOBAL u32x2 *)(qrow + k) = u32x2{o0, o1};
  }
}

struct DequantArgs {
  const uint8_t *q;
  const float *scale;
  uint16_t *y;
  int64_t ldq, ldy;
  int32_t M, K;
};

__global__ __launch_bounds__(256) void dequant_rows_kernel(const DequantArgs a) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + wave_id();
  if (m >= a.M) return;
  const float s = a.scale[m];
  const uint8_t *qrow = a.q + (int64_t)m * a.ldq;
  uint16_t *yrow = a.y + (int64_t)m * a.ldy;
  for (int k = 8 * lane; k < a.K; k += 512) {
    const u32x2 v = *(const MLORA_GLOBAL u32x2 *)(qrow + k);
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t word = v[w >> 1] >> (16 * (w & 1));
      o[w] = pack2_bf16(e4m3_to_f32(word & 0xff) * s, e4m3_to_f32((word >> 8) & 0xff) * s);
    }
    *(MLORA_GLOBAL u32x4 *)(yrow + k) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

struct DivArgs {
  const uint16_t *x;
  const float *div;
  uint16_t *y;
  int64_t ldx, ldy;
  int32_t M, K;
};

// One row divided by d, a wave per row (K a multiple of 8).
__device__ __forceinline__ void div_row(const uint16_t *xrow, uint16_t *yrow, float d, int K, int lane) {
  for (int k = 8 * lane; k < K; k += 512) {
    const u32x4 v = *(const MLORA_GLOBAL u32x4 *)(xrow + k);
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = pack2_bf16(bf16_to_f32(v[w] & 0xffff) / d, bf16_to_f32(v[w] >> 16) / d);
    *(MLORA_GLOBAL u32x4 *)(yrow + k) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

__global__ __launch_bounds__(256) void div_rows_kernel(const DivArgs a) {
  const int m = blockIdx.x * 4 + wave_id();
  if (m >= a.M) return;
  div_row(a.x + (int64_t)m * a.ldx, a.y + (int64_t)m * a.ldy, a.div[m], a.K, threadIdx.x & 63);
}

// Several matrices of M rows divided by the same per-row values (the lora_b of every adapter by
// w_scale): matrix blockIdx.y, four rows per workgroup.
struct DivBatchArgs {
  const uint16_t *x[kMaxAdapters];
  uint16_t *y[kMaxAdapters];
  int64_t ldx[kMaxAdapters], ldy[kMaxAdapters];
  int32_t K[kMaxAdapters];
  const float *div;
  int32_t M;
};

__global__ __launch_bounds__(256) void div_rows_batch_kernel(const DivBatchArgs a) {
  const int i = blockIdx.y;
  const int m = blockIdx.x * 4 + wave_id();
  if (m >= a.M) return;
  div_row(a.x[i] + (int64_t)m * a.ldx[i], a.y[i] + (int64_t)m * a.ldy[i], a.div[m], a.K[i], threadIdx.x & 63);
}

}  // namespace mlora

using namespace mlora;

template <bool CS>
static void launch_quantize(const QuantArgs &a, int64_t K, hipStream_t s) {
  const dim3 grid((unsigned)((a.M + 3) / 4)), block(256);
  const int64_t ni = (K + 511) / 512;  // 16-byte chunks per lane
  if (ni <= 2) hipLaunchKernelGGL((quantize_rows_reg_kernel<2, CS>), grid, block, 0, s, a);
  else if (ni <= 4) hipLaunchKernelGGL((quantize_rows_reg_kernel<4, CS>), grid, block, 0, s, a);
  else if (ni <= 8) hipLaunchKernelGGL((quantize_rows_reg_kernel<8, CS>), grid, block, 0, s, a);
  else if (ni <= 18) hipLaunchKernelGGL((quantize_rows_reg_kernel<18, CS>), grid, block, 0, s, a);
  else hipLaunchKernelGGL(quantize_rows_kernel<CS>, grid, block, 0, s, a);
}

extern "C" int mlora_quantize_rows_fp8(const void *x, int64_t ldx, int64_t M, int64_t K, const float *col_scale,
                                       void *xq, int64_t ldq, float *scale, void *stream) {
  if (M < 0 || K < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 4 || K > INT32_MAX / 2) return MLORA_ERR_LIMIT;
  int st = check_bf16_matrix(x, ldx, M, K);
  if (st) return st;
  if ((st = check_fp8_matrix(xq, ldq, M, K))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  if (scale == nullptr) return MLORA_ERR_INVALID;
  if (col_scale != nullptr && !aligned16(col_scale)) return MLORA_ERR_UNSUPPORTED;
  QuantArgs a{static_cast<const uint16_t *>(x), col_scale, static_cast<uint8_t *>(xq), scale, ldx, ldq, (int32_t)M,
              (int32_t)K};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (col_scale != nullptr) launch_quantize<true>(a, K, s);
  else launch_quantize<false>(a, K, s);
  return launch_status();
}

extern "C" int mlora_dequant_rows_fp8(const void *q, int64_t ldq, const float *scale, int64_t M, int64_t K, void *y,
                                      int64_t ldy, void *stream) {
  if (M < 0 || K < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 4 || K > INT32_MAX / 2) return MLORA_ERR_LIMIT;
  int st = check_fp8_matrix(q, ldq, M, K);
  if (st) return st;
  if ((st = check_bf16_matrix(y, ldy, M, K))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  if (scale == nullptr) return MLORA_ERR_INVALID;
  DequantArgs a{static_cast<const uint8_t *>(q), scale, static_cast<uint16_t *>(y), ldq, ldy, (int32_t)M, (int32_t)K};
  hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

extern "C" int mlora_div_rows_bf16(const void *x, int64_t ldx, const float *div, int64_t M, int64_t K, void *y,
                                   int64_t ldy, void *stream) {
  if (M < 0 || K < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 4 || K > INT32_MAX / 2) return MLORA_ERR_LIMIT;
  int st = check_bf16_matrix(x, ldx, M, K);
  if (st) return st;
  if ((st = check_bf16_matrix(y, ldy, M, K))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  if (div == nullptr) return MLORA_ERR_INVALID;
  DivArgs a{static_cast<const uint16_t *>(x), div, static_cast<uint16_t *>(y), ldx, ldy, (int32_t)M, (int32_t)K};
  hipLaunchKernelGGL(div_rows_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return launch_status();
}

extern "C" int mlora_div_rows_bf16_batch(const void *const *x, const int64_t *ldx, const float *div, int64_t M,
                                         const int64_t *K, void *const *y, const int64_t *ldy, int32_t n,
                                         void *stream) {
  if (n < 0 || M < 0) return MLORA_ERR_INVALID;
  if (n > kMaxAdapters || M > INT32_MAX - 4) return MLORA_ERR_LIMIT;
  if (n == 0 || M == 0) return MLORA_OK;
  if (x == nullptr || ldx == nullptr || K == nullptr || y == nullptr || ldy == nullptr) return MLORA_ERR_INVALID;
  DivBatchArgs a{};
  bool work = false;
  for (int i = 0; i < n; ++i) {
    if (K[i] < 0) return MLORA_ERR_INVALID;
    if (K[i] > INT32_MAX / 2) return MLORA_ERR_LIMIT;
    int st = check_bf16_matrix(x[i], ldx[i], M, K[i]);
    if (st) return st;
    if ((st = check_bf16_matrix(y[i], ldy[i], M, K[i]))) return st;
    a.x[i] = static_cast<const uint16_t *>(x[i]);
    a.y[i] = static_cast<uint16_t *>(y[i]);
    a.ldx[i] = ldx[i];
    a.ldy[i] = ldy[i];
    a.K[i] = (int32_t)K[i];
    work = work || K[i] > 0;
  }
  if (!work) return MLORA_OK;
  if (div == nullptr) return MLORA_ERR_INVALID;
  a.div = div;
  a.M = (int32_t)M;
  hipLaunchKernelGGL(div_rows_batch_kernel, dim3((unsigned)((M + 3) / 4), (unsigned)n), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}
