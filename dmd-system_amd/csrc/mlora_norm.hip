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
//
// Backward (the reference's fused backward, runtime/wan13b_fused_layernorm_backward_kernel.py):
//   hidden gradient (:27-134): per row, with n = LN(x), gn = RN(g · RN(1 + s)),
//       dx = ((gn - Σgn / W) - n · (Σ(gn·n) / W)) · rstd,  plus the row's mean and rstd;
//   reduced component gradient (:137-212): per sample and feature, Σ_t g·n (the scale slot)
//       and Σ_t g (the shift slot), with n = (x - mean) · rstd from the stored statistics;
//       here as per-chunk partial sums over 64-token chunks, added in a fixed order;
//   per-token component gradient (:215-270): g·n and g at every token.
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

// ------------------------------------------------------------------ backward

constexpr int kNormBwdMaxWidth = 5120;  // the row and its gradient stay in registers
constexpr int kNormTokenChunk = 64;     // tokens per partial sum of the reduced component gradient

struct NormBwdArgs {
  const void *x, *g;
  const void *scale_row;  // nullptr: no table
  const void *scale;
  void *dx;
  float *mean, *rstd;  // [batches * tokens]
  int64_t x_sb, x_st, g_sb, g_st, scale_sb, scale_st, dx_sb, dx_st;
  int32_t rows, tokens, width;
  int32_t x_f32, g_f32, table_f32, scale_f32, dx_f32;
  float eps;
};

__device__ __forceinline__ void store8_any(void *base, bool f32, int64_t e, const float (&v)[8]) {
  if (f32) {
    float *p = static_cast<float *>(base) + e;
    *(MLORA_GLOBAL f32x4 *)p = f32x4{v[0], v[1], v[2], v[3]};
    *(MLORA_GLOBAL f32x4 *)(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
  } else {
    *(MLORA_GLOBAL u32x4 *)(static_cast<uint16_t *>(base) + e) =
        u32x4{pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]), pack2_bf16(v[4], v[5]), pack2_bf16(v[6], v[7])};
  }
}

// ((gn - gsum_w) - n · gnn_w) · rstd, each operation rounded (no fused multiply-add).
__device__ __forceinline__ float ln_input_grad(float gn, float n, float gsum_w, float gnn_w, float rstd) {
#pragma clang fp contract(off)
  const float a = gn - gsum_w;
  const float b = n * gnn_w;
  return (a - b) * rstd;
}

__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

template <int NCH>
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void norm_backward_kernel(const NormBwdArgs a) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * kNormRowsPerBlock + wave_id();
  if (r >= a.rows) return;
  const int64_t b = r / a.tokens, t = r % a.tokens;
  const int nchunks = a.width / 8;
  const float width = (float)a.width;
  float x[NCH][8];
  const int64_t xo = b * a.x_sb + t * a.x_st;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c < nchunks) load8(a.x, a.x_f32, xo + 8 * c, x[k]);
    else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[k][i] = 0.f;
    }
  }
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
  const float rstd = 1.0f / __fsqrt_rn(var + a.eps);
  // x -> n; gn = RN(g · RN(1 + s)) into g; the two row sums over live chunks
  float g[NCH][8];
  float sg = 0.f, sgn = 0.f;
  const int64_t go = b * a.g_sb + t * a.g_st, so = b * a.scale_sb + t * a.scale_st;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
#pragma unroll
    for (int i = 0; i < 8; ++i) x[k][i] = mul_rn(x[k][i], rstd);
    if (c < nchunks) {
      float sc[8];
      load8(a.g, a.g_f32, go + 8 * c, g[k]);
      load8(a.scale, a.scale_f32, so + 8 * c, sc);
      if (a.scale_row != nullptr) {
        float ts[8];
        load8(a.scale_row, a.table_f32, 8 * c, ts);
#pragma unroll
        for (int i = 0; i < 8; ++i) sc[i] = add_rn(ts[i], sc[i]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        g[k][i] = mul_rn(g[k][i], add_rn(1.0f, sc[i]));
        sg += g[k][i];
        sgn += g[k][i] * x[k][i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) g[k][i] = 0.f;
    }
  }
  const float gsum_w = wave_sum(sg) / width, gnn_w = wave_sum(sgn) / width;
  const int64_t dxo = b * a.dx_sb + t * a.dx_st;
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = lane + 64 * k;
    if (c >= nchunks) break;
    float d[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) d[i] = ln_input_grad(g[k][i], x[k][i], gsum_w, gnn_w, rstd);
    store8_any(a.dx, a.dx_f32, dxo + 8 * c, d);
  }
  if (lane == 0) {
    a.mean[r] = mean;
    a.rstd[r] = rstd;
  }
}

struct NormCompArgs {
  const void *x, *g;
  const float *mean, *rstd;  // [batches * tokens]
  float *partial;            // reduced: [batches, n_tchunks, 2, width]
  void *out;
  int64_t x_sb, x_st, g_sb, g_st, out_sb, out_st, out_sc;
  int32_t batches, tokens, width, n_tchunks;
  int32_t x_f32, g_f32, out_f32, si, hi;
};

// One workgroup per (sample, 64-token chunk): thread j owns feature chunks j, j + 256, ...
// (CPT of them) and sums g·n and g over the chunk's tokens in token order.
constexpr int kCompMaxChunksPerThread = kNormMaxWidth / 8 / 256;

template <int CPT>
__global__ __launch_bounds__(256) void norm_component_partial_kernel(const NormCompArgs a) {
  const int b = blockIdx.x / a.n_tchunks, tc = blockIdx.x % a.n_tchunks;
  const int t0 = tc * kNormTokenChunk, t1 = min(t0 + kNormTokenChunk, a.tokens);
  const int nchunks = a.width / 8;
  float sgn[CPT][8], sg[CPT][8];
#pragma unroll
  for (int q = 0; q < CPT; ++q)
#pragma unroll
    for (int i = 0; i < 8; ++i) sgn[q][i] = 0.f, sg[q][i] = 0.f;
#pragma unroll 4
  for (int t = t0; t < t1; ++t) {
    const int64_t r = (int64_t)b * a.tokens + t;
    const float mean = a.mean[r], rstd = a.rstd[r];
#pragma unroll
    for (int q = 0; q < CPT; ++q) {
      const int c = threadIdx.x + 256 * q;
      if (c >= nchunks) break;
      float xv[8], gv[8];
      load8(a.x, a.x_f32, b * a.x_sb + t * a.x_st + 8 * c, xv);
      load8(a.g, a.g_f32, b * a.g_sb + t * a.g_st + 8 * c, gv);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float n = mul_rn(xv[i] - mean, rstd);
        sgn[q][i] += gv[i] * n;
        sg[q][i] += gv[i];
      }
    }
  }
  float *p = a.partial + ((int64_t)b * a.n_tchunks + tc) * 2 * a.width;
#pragma unroll
  for (int q = 0; q < CPT; ++q) {
    const int c = threadIdx.x + 256 * q;
    if (c >= nchunks) break;
    store8_any(p, true, 8 * c, sgn[q]);
    store8_any(p + a.width, true, 8 * c, sg[q]);
  }
}

// out[b, si, 8c..8c+7] = Σ_tc partial[b, tc, 0, 8c..], out[b, hi, ...] = Σ_tc partial[b, tc, 1, ...]:
// one wave per (sample, slot, 8-feature chunk). Lane l adds chunks tc = l, l + 64, ... in order,
// then a butterfly adds the lanes: a fixed order.
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void norm_component_reduce_kernel(const NormCompArgs a) {
  const int lane = threadIdx.x & 63;
  const int nchunks = a.width / 8;
  const int64_t wv = (int64_t)blockIdx.x * kNormRowsPerBlock + wave_id();
  if (wv >= (int64_t)a.batches * 2 * nchunks) return;
  const int b = (int)(wv / (2 * nchunks)), k = (int)((wv / nchunks) % 2), c = (int)(wv % nchunks);
  const int64_t per = 2 * (int64_t)a.width;
  const float *p = a.partial + (int64_t)b * a.n_tchunks * per + (int64_t)k * a.width + 8 * c;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  for (int tc = lane; tc < a.n_tchunks; tc += 64) {
    float v[8];
    load8(p + (int64_t)tc * per, true, 0, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += v[i];
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = wave_sum(acc[i]);
  if (lane < 8) {
    const int64_t o = b * a.out_sb + (int64_t)(k == 0 ? a.si : a.hi) * a.out_sc + 8 * c + lane;
    float mine = acc[0];
#pragma unroll
    for (int i = 1; i < 8; ++i) mine = lane == i ? acc[i] : mine;
    if (a.out_f32) static_cast<float *>(a.out)[o] = mine;
    else static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_rne(mine);
  }
}

// Per token: out[b, t, si, :] = RN(g·n), out[b, t, hi, :] = g. One wave per row.
__global__ __launch_bounds__(64 * kNormRowsPerBlock) void norm_component_token_kernel(const NormCompArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kNormRowsPerBlock + wave_id();
  if (r >= (int64_t)a.batches * a.tokens) return;
  const int64_t b = r / a.tokens, t = r % a.tokens;
  const float mean = a.mean[r], rstd = a.rstd[r];
  const int nchunks = a.width / 8;
  const int64_t ob = b * a.out_sb + t * a.out_st;
  for (int c = lane; c < nchunks; c += 64) {
    float xv[8], gv[8], sn[8];
    load8(a.x, a.x_f32, b * a.x_sb + t * a.x_st + 8 * c, xv);
    load8(a.g, a.g_f32, b * a.g_sb + t * a.g_st + 8 * c, gv);
#pragma unroll
    for (int i = 0; i < 8; ++i) sn[i] = mul_rn(gv[i], mul_rn(xv[i] - mean, rstd));
    store8_any(a.out, a.out_f32, ob + (int64_t)a.si * a.out_sc + 8 * c, sn);
    store8_any(a.out, a.out_f32, ob + (int64_t)a.hi * a.out_sc + 8 * c, gv);
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
  if (batches > 1 && out_sb < (tokens - 1) * out_st + width) return MLORA_ERR_INVALID;  // batches overlap
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

extern "C" int mlora_modulated_norm_backward(const void *x, int x_dtype, int64_t x_sb, int64_t x_st,
                                             const void *g, int g_dtype, int64_t g_sb, int64_t g_st,
                                             const void *scale_row, int table_dtype,
                                             const void *scale, int scale_dtype, int64_t scale_sb, int64_t scale_st,
                                             void *dx, int dx_dtype, int64_t dx_sb, int64_t dx_st,
                                             float *mean, float *rstd, float eps,
                                             int64_t batches, int64_t tokens, int64_t width, void *stream) {
  if (batches < 0 || tokens < 0 || width < 0) return MLORA_ERR_INVALID;
  for (int d : {x_dtype, g_dtype, scale_dtype, dx_dtype})
    if (d != MLORA_BF16 && d != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  if (scale_row != nullptr && table_dtype != MLORA_BF16 && table_dtype != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  if (!(eps > 0.f && eps < INFINITY)) return MLORA_ERR_INVALID;
  if (width > 0 && (width % 8 != 0 || width > kNormBwdMaxWidth)) return MLORA_ERR_UNSUPPORTED;
  if (batches > 0 && tokens > INT32_MAX / batches) return MLORA_ERR_LIMIT;
  const int64_t rows = batches * tokens;
  if (rows > INT32_MAX - kNormRowsPerBlock) return MLORA_ERR_LIMIT;
  if (rows == 0 || width == 0) return MLORA_OK;
  if (x == nullptr || g == nullptr || scale == nullptr || dx == nullptr || mean == nullptr || rstd == nullptr)
    return MLORA_ERR_INVALID;
  if (tokens > 1 && dx_st < width) return MLORA_ERR_INVALID;  // rows of one batch overlap
  if (batches > 1 && dx_sb < (tokens - 1) * dx_st + width) return MLORA_ERR_INVALID;  // batches overlap
  if (!rows_aligned(x, x_sb, x_st) || !rows_aligned(g, g_sb, g_st) || !rows_aligned(scale, scale_sb, scale_st) ||
      !rows_aligned(dx, dx_sb, dx_st))
    return MLORA_ERR_UNSUPPORTED;
  if (scale_row != nullptr && !aligned16(scale_row)) return MLORA_ERR_UNSUPPORTED;
  NormBwdArgs a{x, g, scale_row, scale, dx, mean, rstd, x_sb, x_st, g_sb, g_st, scale_sb, scale_st, dx_sb, dx_st,
                (int32_t)rows, (int32_t)tokens, (int32_t)width,
                x_dtype == MLORA_F32, g_dtype == MLORA_F32, table_dtype == MLORA_F32, scale_dtype == MLORA_F32,
                dx_dtype == MLORA_F32, eps};
  const int nch = (int)((width / 8 + 63) / 64);
  const dim3 grid((unsigned)((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock)), block(64 * kNormRowsPerBlock);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (nch <= 1) hipLaunchKernelGGL(norm_backward_kernel<1>, grid, block, 0, s, a);
  else if (nch <= 2) hipLaunchKernelGGL(norm_backward_kernel<2>, grid, block, 0, s, a);
  else if (nch <= 3) hipLaunchKernelGGL(norm_backward_kernel<3>, grid, block, 0, s, a);
  else if (nch <= 4) hipLaunchKernelGGL(norm_backward_kernel<4>, grid, block, 0, s, a);
  else if (nch <= 6) hipLaunchKernelGGL(norm_backward_kernel<6>, grid, block, 0, s, a);
  else if (nch <= 8) hipLaunchKernelGGL(norm_backward_kernel<8>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(norm_backward_kernel<10>, grid, block, 0, s, a);
  return launch_status();
}

extern "C" int64_t mlora_modulated_norm_component_workspace_bytes(int64_t batches, int64_t tokens, int64_t width) {
  if (batches < 0 || tokens < 0 || width < 0) return MLORA_ERR_INVALID;
  const int64_t n_tchunks = (tokens + kNormTokenChunk - 1) / kNormTokenChunk;
  return batches * n_tchunks * 2 * width * (int64_t)sizeof(float);
}

extern "C" int mlora_modulated_norm_component_grad(const void *x, int x_dtype, int64_t x_sb, int64_t x_st,
                                                   const void *g, int g_dtype, int64_t g_sb, int64_t g_st,
                                                   const float *mean, const float *rstd,
                                                   void *out, int out_dtype, int64_t out_sb, int64_t out_st,
                                                   int64_t out_sc, int scale_index, int shift_index, int reduce,
                                                   void *workspace, int64_t workspace_bytes,
                                                   int64_t batches, int64_t tokens, int64_t width, void *stream) {
  if (batches < 0 || tokens < 0 || width < 0) return MLORA_ERR_INVALID;
  for (int d : {x_dtype, g_dtype, out_dtype})
    if (d != MLORA_BF16 && d != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  if (scale_index < 0 || scale_index >= 6 || shift_index < 0 || shift_index >= 6 || scale_index == shift_index)
    return MLORA_ERR_INVALID;
  if (width > 0 && (width % 8 != 0 || width > kNormMaxWidth)) return MLORA_ERR_UNSUPPORTED;
  if (batches > 0 && tokens > INT32_MAX / batches) return MLORA_ERR_LIMIT;
  if (batches * tokens > INT32_MAX - kNormRowsPerBlock) return MLORA_ERR_LIMIT;
  if (batches == 0 || width == 0) return MLORA_OK;
  if (out == nullptr) return MLORA_ERR_INVALID;
  if (out_sb < 0 || out_st < 0 || out_sc < width) return MLORA_ERR_INVALID;  // the six slots do not overlap
  NormCompArgs a{x, g, mean, rstd, static_cast<float *>(workspace), out, x_sb, x_st, g_sb, g_st, out_sb, out_st, out_sc,
                 (int32_t)batches, (int32_t)tokens, (int32_t)width,
                 (int32_t)((tokens + kNormTokenChunk - 1) / kNormTokenChunk),
                 x_dtype == MLORA_F32, g_dtype == MLORA_F32, out_dtype == MLORA_F32, scale_index, shift_index};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (reduce) {
    if (out_sb < 6 * out_sc) return MLORA_ERR_INVALID;  // samples do not overlap
    if (tokens == 0) {  // nothing to sum: zero gradients, written by the reduce kernel
      a.n_tchunks = 0;
    } else {
      if (x == nullptr || g == nullptr || mean == nullptr || rstd == nullptr) return MLORA_ERR_INVALID;
      if (!rows_aligned(x, x_sb, x_st) || !rows_aligned(g, g_sb, g_st)) return MLORA_ERR_UNSUPPORTED;
      const int64_t need = mlora_modulated_norm_component_workspace_bytes(batches, tokens, width);
      if (workspace == nullptr || workspace_bytes < need) return MLORA_ERR_WORKSPACE;
      if (!aligned16(workspace)) return MLORA_ERR_UNSUPPORTED;
      const dim3 grid((unsigned)(batches * a.n_tchunks));
      const int cpt = (int)((width / 8 + 255) / 256);
      if (cpt <= 1) hipLaunchKernelGGL(norm_component_partial_kernel<1>, grid, dim3(256), 0, s, a);
      else if (cpt <= 2) hipLaunchKernelGGL(norm_component_partial_kernel<2>, grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL(norm_component_partial_kernel<kCompMaxChunksPerThread>, grid, dim3(256), 0, s, a);
      int st = launch_status();
      if (st) return st;
    }
    const int64_t waves = batches * 2 * (width / 8);
    hipLaunchKernelGGL(norm_component_reduce_kernel, dim3((unsigned)((waves + kNormRowsPerBlock - 1) / kNormRowsPerBlock)),
                       dim3(64 * kNormRowsPerBlock), 0, s, a);
    return launch_status();
  }
  if (tokens == 0) return MLORA_OK;
  if (x == nullptr || g == nullptr || mean == nullptr || rstd == nullptr) return MLORA_ERR_INVALID;
  if (out_sc < width || out_st < 6 * out_sc) return MLORA_ERR_INVALID;  // [B, T, 6, W] rows do not overlap
  if (batches > 1 && out_sb < (tokens - 1) * out_st + 6 * out_sc) return MLORA_ERR_INVALID;  // nor batches
  if (!rows_aligned(x, x_sb, x_st) || !rows_aligned(g, g_sb, g_st) || !aligned16(out) || out_sb % 8 != 0 ||
      out_st % 8 != 0 || out_sc % 8 != 0)
    return MLORA_ERR_UNSUPPORTED;
  const int64_t rows = batches * tokens;
  hipLaunchKernelGGL(norm_component_token_kernel, dim3((unsigned)((rows + kNormRowsPerBlock - 1) / kNormRowsPerBlock)),
                     dim3(64 * kNormRowsPerBlock), 0, s, a);
  return launch_status();
}
