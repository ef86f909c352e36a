// Modulated LayerNorm that opens a DiT sublayer, i.e. the input of the block's
// next linear, written straight to bf16:
//
//   v[f]   = (x[f] - mean) · (1 / sqrt(var + eps))     affine-free LayerNorm of the row
//            (fp32, two passes: mean = Σx / W, var = Σ(x - mean)² / W),
//            or x[f] itself when x is already normalized (float32)
//   s[f]   = RN(scale_row[f] + scale[b, t, f])          with a scale-shift table,
//            or scale[b, t, f]                          without
//   h[f]   = RN(shift_row[f] + shift[b, t, f])  or  shift[b, t, f]
//   out[f] = bf16_rne(RN(RN(v[f] · RN(1 + s[f])) + h[f]))
//
// These are the reference's three forward forms:
//   * the exact epilogue after PyTorch's fp32 LayerNorm
//     (runtime/wan13b_modulated_norm_kernel.py:26-97: add.rn 1 + scale, mul.rn, add.rn shift, BF16 store);
//   * its materialization form, the table rows added to the per-token components first (:100-204);
//   * the fused LayerNorm + modulation (runtime/wan13b_fused_layernorm_kernel.py:22-132).
// The elementwise steps are separate fp32 operations rounded to nearest, with
// contraction off, so they match the reference bit for bit given the same v.
// The LayerNorm sums in a fixed order: each lane sums its own chunks in order,
// then a butterfly over the wave.
//
// x is bf16 (the reference's hidden state) or float32 (the Wan block's float32
// residual stream, which the gated-residual GEMM epilogue writes). One wave per
// row holds the row in registers: W ≤ 8192 features (Wan-1.3B 1536, Helios
// 5120), up to 16 chunks of 8 per lane. Loads and stores are 16 bytes, and the
// kernel is HBM-bound.
#include "mlora_common.h"
#include "mlora_host.h"

namespace mlora {

constexpr int kNormMaxWidth = 8192;
constexpr int kNormRowsPerBlock = 4;

struct NormArgs {
  const void *x;
  const void *scale_row, *shift_row;  // both or neither (table_dtype)
  const void *scale, *shift;          // scale_f32 / shift_f32: float32, else bf16
  uint16_t *out;
  int64_t x_sb, x_st, scale_sb, scale_st, shift_sb, shift_st, out_sb, out_st;  // element strides
  int32_t rows, tokens, width;
  int32_t table_f32, scale_f32, shift_f32;
  float eps;
};

// Eight consecutive values at element offset e of a bf16 or float32 array.
__device__ __forceinline__ void load8(const void *base, bool f32, int64_t e, float (&v)[8]) {
  if (f32) {
    const float *p = static_cast<const float *>(base) + e;
    const f32x4 a = *(const MLORA_GLOBAL f32x4 *)p, b = *(const MLORA_GLOBAL f32x4 *)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = a[i], v[i + 4] = b[i];
  } else {
    const u32x4 u = *(const MLORA_GLOBAL u32x4 *)(static_cast<const uint16_t *>(base) + e);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = bf16_to_f32((uint16_t)(i % 2 ? u[i / 2] >> 16 : u[i / 2] & 0xffff));
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// RN(RN(v · RN(1 + s)) + h): three roundings, no fused multiply-add.
__device__ __forceinline__ float modulate(float v, float s, float h) {
#pragma clang fp contract(off)
  const float ops = 1.0f + s;
  const float p = v * ops;
  return p + h;
}

__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// One row's LayerNorm (LN) in place on the lane's chunks x; padded chunks hold zeros.
template <int NCH, bool LN>
__device__ __forceinline__ void normalize_row(float (&x)[NCH][8], int lane, int nchunks, float width, float eps) {
  if constexpr (LN) {
    float s1 = 0.f;
#pragma unroll
    for (int k = 0; k < NCH; ++k)
#pragma unroll
      for (int i = 0; i < 8; ++i) s1 += x[k][i];
    const float mean = wave_sum(s1) / width;
    float s2 = 0.f;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const bool live = lane + 64 * k < nchunks;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float c = x[k][i] - mean;
        x[k][i] = c;
        if (live) s2 += c * c;
      }
    }
    const float var = wave_sum(s2) / width;
    const float rstd = 1.0f / __fsqrt_rn(var + eps);
#pragma unroll
    for (int k = 0; k < NCH; ++k)
#pragma unroll
      for (int i = 0; i < 8; ++i) x[k][i] *= rstd;
  }
}

template <int NCH, bool XF32>
__device__ __forceinline__ void load_row(const NormArgs &a, int64_t xo, int lane, int nchunks, float (&x)[NCH][8]) {
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nchunks) load8(a.x, XF32, xo + 8 * c, x[k]);
    else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[k][i] = 0.f;
    }
  }
}

// The scale and shift of chunk c of row (b, t), with the table rows added.
__device__ __forceinline__ void load_mod(const NormArgs &a, int64_t so, int64_t ho, int c, float (&s)[8], float (&h)[8]) {
  load8(a.scale, a.scale_f32, so + 8 * c, s);
  load8(a.shift, a.shift_f32, ho + 8 * c, h);
  if (a.scale_row != nullptr) {
    float ts[8], th[8];
    load8(a.scale_row, a.table_f32, 8 * c, ts);
    load8(a.shift_row, a.table_f32, 8 * c, th);
#pragma unroll
    for (int i = 0; i < 8; ++i) s[i] = add_rn(ts[i], s[i]), h[i] = add_rn(th[i], h[i]);
  }
}

__device__ __forceinline__ void store8(uint16_t *orow, int c, const float (&x)[8], const float (&s)[8],
                                       const float (&h)[8]) {
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    o[i] = pack2_bf16(modulate(x[2 * i], s[2 * i], h[2 * i]), modulate(x[2 * i + 1], s[2 * i + 1], h[2 * i + 1]));
  *(MLORA_GLOBAL u32x4 *)(orow + 8 * c) = u32x4{o[0], o[1], o[2], o[3]};
}

// RW == 1: one row per wave. RW > 1 (scale and shift broadcast over the tokens of a batch,
// token stride 0): a wave takes RW consecutive rows of one batch and materializes their common
// scale and shift once, in registers, instead of reading them again for every row.
template <int NCH, bool XF32, bool LN, int RW>
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void modulated_norm_kernel(const NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int nchunks = a.width / 8;
  const float width = (float)a.width;
  if constexpr (RW == 1) {
    const int r = blockIdx.x * kNormRowsPerBlock + wave_id();
    if (r >= a.rows) return;
    const int64_t b = r / a.tokens, t = r % a.tokens;
    float x[NCH][8];
    load_row<NCH, XF32>(a, b * a.x_sb + t * a.x_st, lane, nchunks, x);
    normalize_row<NCH, LN>(x, lane, nchunks, width, a.eps);
    const int64_t so = b * a.scale_sb + t * a.scale_st, ho = b * a.shift_sb + t * a.shift_st;
    uint16_t *orow = a.out + b * a.out_sb + t * a.out_st;
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = lane + 64 * k;
      if (c >= nchunks) break;
      float s[8], h[8];
      load_mod(a, so, ho, c, s, h);
      store8(orow, c, x[k], s, h);
    }
  } else {
    const int groups = (a.tokens + RW - 1) / RW;  // row groups per batch
    const int gi = blockIdx.x * kNormRowsPerBlock + wave_id();
    if (gi >= (a.rows / a.tokens) * groups) return;
    const int64_t b = gi / groups;
    const int t0 = (gi % groups) * RW;
    float s[NCH][8], h[NCH][8];
#pragma unroll
    for (int k = 0; k < NCH; ++k) {
      const int c = lane + 64 * k;
      if (c < nchunks) load_mod(a, b * a.scale_sb, b * a.shift_sb, c, s[k], h[k]);
    }
    for (int t = t0; t < t0 + RW && t < a.tokens; ++t) {
      float x[NCH][8];
      load_row<NCH, XF32>(a, b * a.x_sb + t * a.x_st, lane, nchunks, x);
      normalize_row<NCH, LN>(x, lane, nchunks, width, a.eps);
      uint16_t *orow = a.out + b * a.out_sb + t * a.out_st;
#pragma unroll
      for (int k = 0; k < NCH; ++k) {
        const int c = lane + 64 * k;
        if (c >= nchunks) break;
        store8(orow, c, x[k], s[k], h[k]);
      }
    }
  }
}

// Chunks per lane are rounded up to one of these instances (the extra chunks are
// masked off). Broadcast scale and shift (token stride 0) up to 2048 features take
// kNormGroupRows rows per wave.
constexpr int kNormGroupRows = 8;

template <bool XF32, bool LN, int RW>
static void launch_norm_rw(const NormArgs &a, int nch, int64_t waves, hipStream_t s) {
  const dim3 grid((unsigned)((waves + kNormRowsPerBlock - 1) / kNormRowsPerBlock)), block(64 * kNormRowsPerBlock);
  if (nch <= 1) hipLaunchKernelGGL((modulated_norm_kernel<1, XF32, LN, RW>), grid, block, 0, s, a);
  else if (nch <= 2) hipLaunchKernelGGL((modulated_norm_kernel<2, XF32, LN, RW>), grid, block, 0, s, a);
  else if (nch <= 3) hipLaunchKernelGGL((modulated_norm_kernel<3, XF32, LN, RW>), grid, block, 0, s, a);
  else if (nch <= 4) hipLaunchKernelGGL((modulated_norm_kernel<4, XF32, LN, RW>), grid, block, 0, s, a);
  else if constexpr (RW == 1) {
    if (nch <= 6) hipLaunchKernelGGL((modulated_norm_kernel<6, XF32, LN, 1>), grid, block, 0, s, a);
    else if (nch <= 8) hipLaunchKernelGGL((modulated_norm_kernel<8, XF32, LN, 1>), grid, block, 0, s, a);
    else if (nch <= 10) hipLaunchKernelGGL((modulated_norm_kernel<10, XF32, LN, 1>), grid, block, 0, s, a);
    else if (nch <= 12) hipLaunchKernelGGL((modulated_norm_kernel<12, XF32, LN, 1>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((modulated_norm_kernel<16, XF32, LN, 1>), grid, block, 0, s, a);
  }
}

template <bool XF32, bool LN>
static void launch_norm(const NormArgs &a, int nch, bool grouped, hipStream_t s) {
  if (grouped) {
    const int64_t groups = (a.tokens + kNormGroupRows - 1) / kNormGroupRows;
    launch_norm_rw<XF32, LN, kNormGroupRows>(a, nch, (int64_t)(a.rows / a.tokens) * groups, s);
  } else {
    launch_norm_rw<XF32, LN, 1>(a, nch, a.rows, s);
  }
}

// Rows of 16-byte chunks: every row start 16-byte aligned.
static bool rows_aligned(const void *p, int64_t sb, int64_t st) {
  return aligned16(p) && sb >= 0 && st >= 0 && sb % 8 == 0 && st % 8 == 0;
}

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_modulated_norm(const void *x, int x_dtype, int64_t x_sb, int64_t x_st, int apply_ln, float eps,
                                    const void *scale_row, const void *shift_row, int table_dtype,
                                    const void *scale, int scale_dtype, const void *shift, int shift_dtype,
                                    int64_t scale_sb, int64_t scale_st, int64_t shift_sb, int64_t shift_st,
                                    void *out, int64_t out_sb, int64_t out_st,
                                    int64_t batches, int64_t tokens, int64_t width, void *stream) {
  if (batches < 0 || tokens < 0 || width < 0) return MLORA_ERR_INVALID;
  if (x_dtype != MLORA_BF16 && x_dtype != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  for (int d : {scale_dtype, shift_dtype})
    if (d != MLORA_BF16 && d != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  if (!apply_ln && x_dtype != MLORA_F32) return MLORA_ERR_UNSUPPORTED;  // normalized input is float32
  if (apply_ln && !(eps > 0.f && eps < INFINITY)) return MLORA_ERR_INVALID;
  if ((scale_row == nullptr) != (shift_row == nullptr)) return MLORA_ERR_INVALID;
  if (scale_row != nullptr && table_dtype != MLORA_BF16 && table_dtype != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  if (width > 0 && (width % 8 != 0 || width > kNormMaxWidth)) return MLORA_ERR_UNSUPPORTED;
  if (batches > 0 && tokens > INT32_MAX / batches) return MLORA_ERR_LIMIT;
  const int64_t rows = batches * tokens;
  if (rows > INT32_MAX - kNormRowsPerBlock) return MLORA_ERR_LIMIT;
  if (rows == 0 || width == 0) return MLORA_OK;
  if (x == nullptr || scale == nullptr || shift == nullptr || out == nullptr) return MLORA_ERR_INVALID;
  if (tokens > 1 && (x_st < width || out_st < width)) return MLORA_ERR_INVALID;  // rows of one batch overlap
  if (!rows_aligned(x, x_sb, x_st) || !rows_aligned(out, out_sb, out_st) || !rows_aligned(scale, scale_sb, scale_st) ||
      !rows_aligned(shift, shift_sb, shift_st))
    return MLORA_ERR_UNSUPPORTED;
  if (scale_row != nullptr && (!aligned16(scale_row) || !aligned16(shift_row))) return MLORA_ERR_UNSUPPORTED;
  NormArgs a{x, scale_row, shift_row, scale, shift, static_cast<uint16_t *>(out),
             x_sb, x_st, scale_sb, scale_st, shift_sb, shift_st, out_sb, out_st,
             (int32_t)rows, (int32_t)tokens, (int32_t)width,
             table_dtype == MLORA_F32 ? 1 : 0, scale_dtype == MLORA_F32 ? 1 : 0, shift_dtype == MLORA_F32 ? 1 : 0,
             eps};
  const int nch = (int)((width / 8 + 63) / 64);
  const bool grouped = scale_st == 0 && shift_st == 0 && nch <= 4 && tokens > 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!apply_ln) launch_norm<true, false>(a, nch, grouped, s);
  else if (x_dtype == MLORA_F32) launch_norm<true, true>(a, nch, grouped, s);
  else launch_norm<false, true>(a, nch, grouped, s);
  return launch_status();
}
