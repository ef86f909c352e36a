/*
 * mlora.h — C ABI of the MI355X (gfx950) batched multi-LoRA linear.
 *
 * Computes, for a frozen base W shared by several low-rank adapters,
 *
 *   Y = X·Wᵀ (+b) + Σ_seg s_a·(X_seg·A_aᵀ)·B_aᵀ          forward
 *   dX = dY·W + Σ_seg (s_a·dY_seg·B_a)·A_a                backward (W frozen: no dW)
 *   dB_a = s_a·Σ_{m∈a} dY[m]ᵀ·h[m]      dA_a = Σ_{m∈a} g[m]ᵀ·X[m]
 *
 * where rows of X are split into contiguous segments [seg_offsets[s],
 * seg_offsets[s+1]) and segment s uses adapter adapter_ids[s] (-1 = base only,
 * the teacher / "LoRA disabled" role).
 *
 * It replaces, for one call, the per-role modules of the reference
 * (DMD-System, sliortega295-ops):
 *   src/distillschedule/training/low_rank.py:26-28   TrainableLowRankLinear.forward
 *   src/distillschedule/native/models.py:44-51       LoRALinear.forward (fp32 LoRA)
 *   src/distillschedule/reference/livewan_wan21/wanstreamer/lora.py:22-27,65-74
 *       LoRALinear.forward / lora_enabled(model, False) (null adapter)
 * and the Triton LoRA kernels those modules call:
 *   src/distillschedule/runtime/wan13b_lora_epilogue.py:55-92   (epilogue add)
 *   src/distillschedule/runtime/helios_lora_b_gemm_kernel.py:53-131 (LoRA-B GEMM + residual)
 *   src/distillschedule/backends/training/minimax_h3/triton_lora_epilogue.py:143-178
 *
 * Conventions (all entry points):
 *   - Every tensor pointer is a device pointer; every array documented as
 *     "host" is read on the host during the call and may be freed after it.
 *   - Matrices are row-major with an explicit leading dimension (elements).
 *   - Nothing is allocated, nothing synchronises the host; work is enqueued on
 *     `stream` (a hipStream_t, passed as void* so this header needs no HIP).
 *   - Return MLORA_OK (0) or a negative mlora_status; no exceptions cross the
 *     ABI. Argument errors are detected before any launch.
 *   - Reentrant: no global mutable state; safe to call from several host
 *     threads on different streams. The one exception is
 *     mlora_seg_outer_noalloc: it keeps its partial sums in one file-scope
 *     device array per GPU, so its calls on one GPU must be serialised.
 *   - Results are deterministic: fixed-order reductions, no float atomics.
 */
#ifndef MLORA_H_
#define MLORA_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLORA_ABI_VERSION 9

/* Limits of one call (kernel-argument tables). Callers with more segments
 * split the rows into several calls; the Python host layer does this. */
#define MLORA_MAX_SEGMENTS 128
#define MLORA_MAX_ADAPTERS 32
#define MLORA_MAX_RANK 256
#define MLORA_MAX_STACKED 8   /* linears in one stacked call (mlora_gemm_fwd_stacked / _dx_stacked) */
/* The GEMM entry points take adapter ranks up to this: the LoRA term of stacked linears that read
 * one input is the side-by-side h (or g) of up to MLORA_MAX_STACKED members, each of rank at most
 * MLORA_MAX_RANK (the GEMM runs the LoRA term as extra k-tiles, so any length fits). */
#define MLORA_MAX_GEMM_RANK (MLORA_MAX_RANK * MLORA_MAX_STACKED)

typedef enum mlora_dtype {
  MLORA_F32 = 0,
  MLORA_BF16 = 1,
  MLORA_FP8_E4M3 = 2 /* OCP e4m3fn, as gfx950 MFMA consumes it */
} mlora_dtype;

typedef enum mlora_status {
  MLORA_OK = 0,
  MLORA_ERR_INVALID = -1,     /* null pointer, bad shape, bad stride, bad routing */
  MLORA_ERR_UNSUPPORTED = -2, /* dtype/alignment combination not implemented */
  MLORA_ERR_WORKSPACE = -3,   /* workspace missing or too small */
  MLORA_ERR_LAUNCH = -4,      /* hipLaunchKernel reported an error */
  MLORA_ERR_LIMIT = -5,       /* more segments/adapters/rank than one call takes */
  MLORA_ERR_DEVICE = -6       /* no current device, or the library's device set-up failed */
} mlora_status;

/* Segment routing shared by all entry points (host arrays).
 *   seg_offsets[n_segments+1]: seg_offsets[0] == 0, nondecreasing,
 *                              seg_offsets[n_segments] == M.
 *   adapter_ids[n_segments]:   -1 (base only) or 0 <= id < n_adapters.
 * Adapter table (host arrays, length n_adapters):
 *   ranks[i] in {0} ∪ [8, MLORA_MAX_RANK], multiple of 8 (GEMM entry points: up to
 *   MLORA_MAX_GEMM_RANK); scales[i] = alpha_i / rank_i.
 * The reference builds one role per module call (training/dmd.py:301-353);
 * here each role is a segment of one call over the shared frozen base
 * (training/construction_sharing.py:105-118). */

int mlora_abi_version(void);
const char *mlora_status_string(int status);
/* SHA-256 (hex) of the sources this library was built from (csrc/ and include/), so a
 * loader can refuse a library built from other sources with the same ABI version. */
const char *mlora_source_hash(void);

/* Shrink: for each row m of a segment with adapter a (rank r_a),
 *   h[m, j] = s_a · Σ_k P[m, k] · Op_a(j, k),   j < r_a
 * and writes it twice:
 *   h_rows  bf16 [M, ldh]   (row-major; round-to-nearest-even of the fp32 value)
 *   h_frag  (may be NULL)   h split into bf16 hi + lo parts (hi = bf16(h),
 *           lo = bf16(h - hi)) in the per-lane operand order of the gfx950
 *           16x16x32 bf16 MFMA, for mlora_seg_outer. Blocks of 32 rows are
 *           counted from each segment's first row; segment s starts at padded
 *           row Σ_{s'<s} roundup(len_s', 32). Block B, j-tile t (16 j), part p
 *           (0 hi, 1 lo), lane L, element e holds h[32·B' + 8·(L/16) + e][16·t + L%16]
 *           (B' = block within its segment) at 16-byte index ((B·frag_jtiles + t)·2 + p)·64 + L.
 *           Size: mlora_frag_bytes(). frag_jtiles >= ceil(max rank / 16).
 * op_layout 0: Op_a stored [r_a, K] (K contiguous, e.g. lora_a, low_rank.py:21)
 * op_layout 1: Op_a stored [K, r_a] (r contiguous, e.g. lora_b [N, r] for the
 *              backward g = s·dY·B, low_rank.py:22)
 * op_lo_ptrs (may be NULL): the adapter operands as two bf16 parts, op_ptrs[i] =
 *           hi = bf16(v) and op_lo_ptrs[i] = lo = bf16(v - hi) of an fp32 master v
 *           (same shape and layout); h then uses hi + lo (~16 significant bits of v)
 *           instead of bf16(v). This is the fp32 LoRA compute of
 *           native/models.py:44-51 (update = F.linear(F.linear(x.float(), a), b) with
 *           fp32 masters, models.py:150-156) over bf16 activations.
 * row_div (may be NULL): per-row divisors [M]; h_rows (not h_frag) then holds
 *           h[m, j] / row_div[m]. The e4m3 forward passes its activation scales
 *           here (see mlora_gemm_fwd_fp8).
 * Rows of base-only segments are not written.
 * Reference: F.linear(value, lora_a) in low_rank.py:28 (forward shrink) and the
 * autograd LinearBackward of F.linear(h, lora_b) (dH = g·B, as written out in
 * runtime/helios_lora_b_gemm_kernel.py:105). */
int mlora_shrink(const void *p, int64_t ldp, int64_t M, int64_t K,
                 const void *const *op_ptrs, const void *const *op_lo_ptrs, int op_layout,
                 const int32_t *ranks, const float *scales, int32_t n_adapters,
                 const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                 void *h_rows, int64_t ldh, void *h_frag, int32_t frag_jtiles,
                 const float *row_div,
                 void *stream);
/* Bytes of the h_frag buffer for this routing and frag_jtiles (< 0: status). */
int64_t mlora_frag_bytes(int64_t M, int32_t frag_jtiles, const int64_t *seg_offsets,
                         const int32_t *adapter_ids, int32_t n_segments);

/* Base GEMM with the LoRA expand fused into its epilogue:
 *   Y[m, n] = bf16( Σ_k X[m,k]·W[n,k] + bias[n] + Σ_j h_rows[m,j]·B_a[n,j] )
 * (h_rows already carries s_a, see mlora_shrink). W is bf16 [N, K] (ldw).
 * bias: NULL, or bias_dtype MLORA_BF16 / MLORA_F32, length N.
 * b_ptrs[i]: bf16 [N, r_i] contiguous (lora_b). h_rows may be NULL when no
 * segment has an adapter.
 * If accumulate != 0, Y is read and the result added to it (Y += ...), which
 * with K == 0 gives the standalone expand of the reference's LoRA-B GEMM +
 * residual kernels (helios_lora_b_gemm_kernel.py:25-50).
 * Reference: low_rank.py:28 (base(value) + scale·F.linear(F.linear(value, A), B)). */
int mlora_gemm_fwd(const void *x, int64_t ldx, int64_t M, int64_t K,
                   const void *w, int64_t ldw, int64_t N,
                   const void *bias, int bias_dtype,
                   const void *h_rows, int64_t ldh,
                   const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                   const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                   void *y, int64_t ldy, int accumulate,
                   void *stream);

/* Several linears that read one input X, as one GEMM (the q / k / v projections of a DiT block,
 * which the reference only shares one fp32 cast of X between: runtime/wan13b_lora_cast.py:265-300):
 * the G = N / group_cols linears' frozen weights stacked by rows into w [N, K], their LoRA terms
 * from one stacked shrink: linear g's h rows in h_rows columns [g·group_ecols, g·group_ecols + r_a)
 * (mlora_shrink of X by [A_0,a; A_1,a; ...]) and b_ptrs[a] = [B_0,a; B_1,a; ...] ([N, r_a]):
 *   Y_g[m, n'] = bf16( Σ_k X[m,k]·W[n,k] + bias[n] + Σ_j h_rows[m, g·group_ecols + j]·B_a[n, j] ),
 *                n = g·group_cols + n'
 * written to y_ptrs[g] ([M, group_cols] each, pitch ldy). group_cols a multiple of 256, N a multiple
 * of group_cols, G <= MLORA_MAX_STACKED, r_a <= group_ecols (a multiple of 8). Each output equals
 * mlora_gemm_fwd of its own linear bit for bit. */
int mlora_gemm_fwd_stacked(const void *x, int64_t ldx, int64_t M, int64_t K,
                           const void *w, int64_t ldw, int64_t N, int64_t group_cols,
                           const void *bias, int bias_dtype,
                           const void *h_rows, int64_t ldh, int64_t group_ecols,
                           const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                           const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                           void *const *y_ptrs, int64_t ldy,
                           void *stream);

/* The input gradient of those G linears as one GEMM whose contraction runs over their dY in turn:
 *   dX[m, k] = bf16( Σ_g Σ_n' dY_g[m, n']·W_cat[g·group_cols + n', k] + Σ_j g_rows[m, j]·A_a[j, k] )
 * with w_t = W_catᵀ ([K, groups·group_cols], the stacked frozen weights transposed, pitch ldw),
 * dy_ptrs[g] = dY_g ([M, group_cols], pitch lddy), g_rows [M, groups·R] the G shrinks of dY side by
 * side (linear g's g = s·dY_g·B_g,a in columns [g·R, (g+1)·R)) and a_ptrs[a] = the stacked
 * [A_0,a; A_1,a; ...] transposed ([K, groups·R]). One rounding of the whole sum (autograd sums the
 * G linears' dX in bf16). Reference: the autograd of low_rank.py:28 for each linear, summed over
 * the linears that read X. */
int mlora_gemm_dx_stacked(const void *const *dy_ptrs, int64_t lddy, int64_t M, int64_t group_cols, int64_t groups,
                          const void *w_t, int64_t ldw, int64_t K,
                          const void *g_rows, int64_t ldg,
                          const void *const *a_ptrs, const int32_t *ranks, int32_t n_adapters,
                          const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                          void *dx, int64_t lddx,
                          void *stream);

/* mlora_gemm_fwd with the DiT block's gated residual fused into the epilogue: the linear
 * closes a branch (attention out-projection, FFN down-projection) whose output y enters
 * the residual stream as x' = x + y·gate (reference/livewan_wan21/wan/modules/model.py:305-313;
 * the exact contract of runtime/helios_residual_kernel.py:66-86):
 *   stream_dtype MLORA_BF16: out[m, n] = bf16( RN( res[m, n] + RN( bf16(Y[m, n]) · gate[m / gate_rows, n] ) ) )
 *   stream_dtype MLORA_F32:  out[m, n] =       RN( res[m, n] + RN( bf16(Y[m, n]) · gate[m / gate_rows, n] ) )
 * with Y the value mlora_gemm_fwd would store, fp32 multiply then fp32 add, each rounded to
 * nearest (no fused multiply-add). The float32 stream is the Wan block's: x is float32 and
 * `x = x + y * e[2]` runs under float32 autocast (model.py:305-306,312-313), so the bf16 y is
 * promoted and the sum is not rounded to bf16. res (x) and out are [M, N] of the stream dtype
 * (float32 rows: pitch a multiple of 4, 16-byte aligned, N a multiple of 8) and may be the same
 * matrix (in-place update of x); gate is fp32 with ⌈M / gate_rows⌉ rows of pitch ldgate
 * (ldgate a multiple of 4, 16-byte aligned): gate_rows = tokens per sample for a per-sample
 * gate [B, 1, N], 1 for a per-token gate. Y itself is not written. */
int mlora_gemm_fwd_gated(const void *x, int64_t ldx, int64_t M, int64_t K,
                         const void *w, int64_t ldw, int64_t N,
                         const void *bias, int bias_dtype,
                         const void *h_rows, int64_t ldh,
                         const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                         const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                         const void *res, int64_t ldres, const float *gate, int64_t ldgate, int64_t gate_rows,
                         void *out, int64_t ldout, int stream_dtype,
                         void *stream);
/* Backward of that gated residual for a frozen gate: dY[m, n] = bf16(dOut[m, n] · gate[m / gate_rows, n])
 * (one fp32 multiply rounded to nearest: runtime/helios_residual_kernel.py:90-133); the
 * gradient of x is dOut. dOut is bf16 or float32 (dout_dtype, the stream's dtype); gate as in
 * mlora_gemm_fwd_gated. */
int mlora_gate_scale_rows(const void *dout, int64_t ldout, int64_t M, int64_t N,
                          const float *gate, int64_t ldgate, int64_t gate_rows,
                          void *dy, int64_t lddy, int dout_dtype,
                          void *stream);

/* Modulated LayerNorm that opens a DiT sublayer (the input of its next linear), bf16 out:
 *   v[f]   = apply_ln ? (x[f] - mean)·(1 / sqrt(var + eps))   affine-free LayerNorm of the row
 *                       (fp32, mean = Σx / W, var = Σ(x - mean)² / W)
 *                     : x[f]                                   (x already normalized: float32)
 *   s[f]   = scale_row ? RN(scale_row[f] + scale[b,t,f]) : scale[b,t,f]   (likewise shift)
 *   out[f] = bf16_rne(RN(RN(v[f]·RN(1 + s[f])) + shift'[f]))
 * for rows (b, t), b < batches, t < tokens, features f < width; every operand is addressed
 * as base + b·stride_b + t·stride_t + f (element strides; stride_t 0 broadcasts one row over
 * the tokens of a batch). Replaces, by apply_ln and scale_row:
 *   apply_ln 0, no table: fused_modulated_norm_epilogue (runtime/wan13b_modulated_norm_kernel.py:207-263,
 *                         kernel :26-97), the exact epilogue after PyTorch's fp32 LayerNorm;
 *   apply_ln 0, table:    fused_modulated_norm_materialization (:266-353, kernel :100-204), the
 *                         scale-shift table rows [width] added to the per-token components first;
 *   apply_ln 1, table:    fused_bf16_layernorm_modulation (runtime/wan13b_fused_layernorm_kernel.py:135-222,
 *                         kernel :22-132); x may also be float32 (the Wan block's residual stream).
 * The elementwise steps are separate fp32 operations rounded to nearest (bit-exact given v).
 * x_dtype MLORA_BF16 or MLORA_F32 (float32 when apply_ln is 0); table_dtype, scale_dtype and
 * shift_dtype MLORA_BF16 or MLORA_F32; eps > 0 when apply_ln. width a multiple of 8 up to 8192; every
 * pointer 16-byte aligned, strides nonnegative multiples of 8. */
int mlora_modulated_norm(const void *x, int x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                         int apply_ln, float eps,
                         const void *scale_row, const void *shift_row, int table_dtype,
                         const void *scale, int scale_dtype, const void *shift, int shift_dtype,
                         int64_t scale_stride_b, int64_t scale_stride_t,
                         int64_t shift_stride_b, int64_t shift_stride_t,
                         void *out, int64_t out_stride_b, int64_t out_stride_t,
                         int64_t batches, int64_t tokens, int64_t width,
                         void *stream);

/* Backward of mlora_modulated_norm with apply_ln (the reference's fused backward,
 * runtime/wan13b_fused_layernorm_backward_kernel.py), for the upstream gradient g of out:
 *   fused_bf16_layernorm_modulation_hidden_backward (:337-393, kernel :27-134): per row,
 *     n = LN(x), s' = RN(1 + (scale_row ? RN(scale_row + scale) : scale)), gn = RN(g·s'),
 *     dx = RN(RN(RN(gn - Σgn / W) - RN(n·(Σ(gn·n) / W)))·rstd), and the row's mean and rstd
 *     (float32 [batches·tokens], row b·tokens + t).
 * x, g, scale and dx are bf16 or float32 (dx in dx_dtype); width a multiple of 8 up to 5120. */
int mlora_modulated_norm_backward(const void *x, int x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                                  const void *g, int g_dtype, int64_t g_stride_b, int64_t g_stride_t,
                                  const void *scale_row, int table_dtype,
                                  const void *scale, int scale_dtype, int64_t scale_stride_b, int64_t scale_stride_t,
                                  void *dx, int dx_dtype, int64_t dx_stride_b, int64_t dx_stride_t,
                                  float *mean, float *rstd, float eps,
                                  int64_t batches, int64_t tokens, int64_t width,
                                  void *stream);
/* Gradients of the two modulation components from the same x, g and the row statistics
 * above, with n = RN(RN(x - mean)·rstd):
 *   reduce 1: fused_reduced_component_gradient (:396-447, kernel :137-212):
 *             out[b, scale_index, f] = Σ_t g·n, out[b, shift_index, f] = Σ_t g  (out [batches, 6, width]
 *             with strides out_stride_b, out_stride_c; float32 partial sums over 64-token chunks,
 *             added in a fixed order, in a caller workspace of
 *             mlora_modulated_norm_component_workspace_bytes(batches, tokens, width) bytes);
 *   reduce 0: fused_tensor4d_component_gradient (:450-502, kernel :215-270):
 *             out[b, t, scale_index, :] = RN(g·n), out[b, t, shift_index, :] = g  (out [batches, tokens, 6,
 *             width]; no workspace).
 * The other four component slots are not written. out_dtype MLORA_BF16 or MLORA_F32. */
int64_t mlora_modulated_norm_component_workspace_bytes(int64_t batches, int64_t tokens, int64_t width);
int mlora_modulated_norm_component_grad(const void *x, int x_dtype, int64_t x_stride_b, int64_t x_stride_t,
                                        const void *g, int g_dtype, int64_t g_stride_b, int64_t g_stride_t,
                                        const float *mean, const float *rstd,
                                        void *out, int out_dtype, int64_t out_stride_b, int64_t out_stride_t,
                                        int64_t out_stride_c, int scale_index, int shift_index, int reduce,
                                        void *workspace, int64_t workspace_bytes,
                                        int64_t batches, int64_t tokens, int64_t width,
                                        void *stream);

/* Input gradient with the LoRA term fused into its epilogue:
 *   dX[m, k] = bf16( Σ_n dY[m,n]·W[n,k] + Σ_j g_rows[m,j]·A_a[j,k] )
 * g_rows = s_a·dY·B_a from mlora_shrink(op_layout=1). a_ptrs[i]: bf16 [r_i, K].
 * If accumulate != 0, dX is read and the result added to it (dX += ...): the
 * dX of linears that read one input, summed in fp32 before one rounding per
 * call instead of autograd's separate bf16 additions (the q/k/v projections fed
 * one tensor, runtime/wan13b_lora_cast.py:265-300).
 * Reference: autograd of low_rank.py:28 — dX = dY·W + (s·dY·B)·A. */
int mlora_gemm_dx(const void *dy, int64_t lddy, int64_t M, int64_t N,
                  const void *w, int64_t ldw, int64_t K,
                  const void *g_rows, int64_t ldg,
                  const void *const *a_ptrs, const int32_t *ranks, int32_t n_adapters,
                  const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                  void *dx, int64_t lddx, int accumulate,
                  void *stream);

/* Segmented outer-product reduction (adapter gradients):
 *   D_a[c, j] = Σ_{m in segments of adapter a} P[m, c] · h[m, j]
 * P bf16 [M, C] (ldp); h given as the h_frag fragments of mlora_shrink (same
 * routing and frag_jtiles), used as hi + lo, so h enters at ~16-bit precision. Written as out_dtype (MLORA_F32 or MLORA_BF16) to
 * out_ptrs[a], layout out_layout 0: [C, r_a] (dB_a = s·dYᵀ·h, lora_b shape),
 * out_layout 1: [r_a, C] (dA_a = gᵀ·X, lora_a shape). Adapters with no rows
 * get zeros. Deterministic two-stage reduction through `workspace`
 * (size from mlora_seg_outer_workspace_bytes).
 * Reference: autograd of low_rank.py:28 (dB = s·dYᵀ·h, dA = gᵀ·x);
 * runtime/helios_lora_b_gemm_kernel.py:106 (d_b = g.T @ h). */
int mlora_seg_outer(const void *p, int64_t ldp, int64_t M, int64_t C,
                    const void *h_frag, int32_t frag_jtiles,
                    void *const *out_ptrs, int out_layout, int out_dtype,
                    const int32_t *ranks, int32_t n_adapters,
                    const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                    void *workspace, int64_t workspace_bytes,
                    void *stream);
int64_t mlora_seg_outer_workspace_bytes(int64_t M, int64_t C,
                                        const int32_t *ranks, int32_t n_adapters,
                                        const int64_t *seg_offsets, const int32_t *adapter_ids,
                                        int32_t n_segments);

/* Bytes of the device array that holds mlora_seg_outer_noalloc's partial sums (per GPU). */
#define MLORA_NOALLOC_SCRATCH_BYTES (64 << 20)

/* mlora_seg_outer with no workspace argument and no allocation of any kind. It has no
 * counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * partial sums live in a device array of MLORA_NOALLOC_SCRATCH_BYTES inside this library,
 * one per GPU, held from the library's first use on that GPU until the process ends; its
 * address is looked up on the first call on each device (the current device, which must be
 * the stream's device). It runs mlora_seg_outer's kernels with mlora_seg_outer's plan, so the
 * results are the same bit for bit; a call whose workspace (mlora_seg_outer_workspace_bytes)
 * exceeds the array returns MLORA_ERR_LIMIT before any device work (the Wan-1.3B shapes need
 * ~34 MB). Every call on one GPU uses that GPU's one array and
 * nothing carries over between calls (each call writes every partial it reads), but calls
 * that overlap in time on one GPU (different streams, or host threads) race on the array. */
int mlora_seg_outer_noalloc(const void *p, int64_t ldp, int64_t M, int64_t C,
                            const void *h_frag, int32_t frag_jtiles,
                            void *const *out_ptrs, int out_layout, int out_dtype,
                            const int32_t *ranks, int32_t n_adapters,
                            const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                            void *stream);

/* ---- Quantised frozen base (OCP e4m3 / float8_e4m3fn, per-row fp32 scale).
 * The reference keeps its frozen base in bf16/fp32 (low_rank.py:20, native/models.py:150-156);
 * these three entry points serve the variant whose frozen W is stored as e4m3 with one fp32
 * scale per output channel, with the same LoRA semantics (low_rank.py:28) on top. */

/* Per-row absmax quantisation of a bf16 matrix, optionally after a per-column fp32 factor:
 * v[m,k] = x[m,k] · col_scale[k] (col_scale may be NULL: factor 1; else 16-byte aligned, [K]),
 * scale[m] = max_k |v[m,k]| / 448 (1 for an all-zero row), q[m,k] = e4m3_rne(v[m,k] · (448 /
 * max_k |v[m,k]|)), saturating at 448. q: [M, K] bytes (ldq and K multiples of 16, 16-byte
 * aligned). Used for activations (per token), for dY·w_scale before the e4m3 dX GEMM, and to
 * produce the per-output-channel weight format. */
int mlora_quantize_rows_fp8(const void *x, int64_t ldx, int64_t M, int64_t K,
                            const float *col_scale,
                            void *q, int64_t ldq, float *scale,
                            void *stream);

/* y[m, k] = bf16( e4m3(q[m,k]) · scale[m] ): the frozen e4m3 W back in bf16 for the dX GEMM. */
int mlora_dequant_rows_fp8(const void *q, int64_t ldq, const float *scale, int64_t M, int64_t K,
                           void *y, int64_t ldy,
                           void *stream);

/* y[m, k] = bf16( x[m,k] / div[m] ) for a bf16 matrix (the lora_b operand of the e4m3 forward). */
int mlora_div_rows_bf16(const void *x, int64_t ldx, const float *div, int64_t M, int64_t K,
                        void *y, int64_t ldy,
                        void *stream);

/* mlora_div_rows_bf16 over n <= MLORA_MAX_ADAPTERS matrices of M rows in one launch:
 * y[i][m, k] = bf16( x[i][m,k] / div[m] ), matrix i [M, K[i]] with pitches ldx[i] / ldy[i]
 * (every adapter's lora_b / w_scale for one e4m3 forward, the same values bit for bit).
 * x, ldx, K, y and ldy are host arrays of n entries; div [M] is a device array.
 * No counterpart in the reference: it replaces n launches of mlora_div_rows_bf16. */
int mlora_div_rows_bf16_batch(const void *const *x, const int64_t *ldx, const float *div, int64_t M,
                              const int64_t *K, void *const *y, const int64_t *ldy, int32_t n,
                              void *stream);

/* mlora_gemm_fwd with an e4m3 base contraction (v_mfma_scale_f32_32x32x64_f8f6f4):
 *   Y[m, n] = bf16( x_scale[m]·w_scale[n]·( Σ_k xq[m,k]·wq[n,k] + Σ_j h_rows[m,j]·B_a[n,j] ) + bias[n] )
 * xq [M, K] and wq [N, K] e4m3 bytes (mlora_quantize_rows_fp8 layout, K >= 16); x_scale [M],
 * w_scale [N] fp32 (16-byte aligned; NULL: all 1). The LoRA operands are bf16 and enter the same
 * fp32 accumulators as the e4m3 products, so the caller passes them divided by the scales:
 * h_rows = h / x_scale[m] (mlora_shrink with row_div = x_scale) and B_a = lora_b / w_scale[n]
 * (mlora_div_rows_bf16); one scaling in the epilogue then restores both terms.
 * Reference semantics: low_rank.py:28 with base weight w_scale[n]·wq[n,k].
 * The same entry point computes the e4m3 dX of that linear (dX = dY·W + g·A, the transposed
 * GEMM of the reference's autograd backward): xq = dY·w_scale quantised per row (scale
 * dy_scale), wq = the frozen e4m3 W transposed ([K, N]), w_scale = NULL, no bias,
 * h_rows = g / dy_scale[m] (mlora_shrink with row_div = dy_scale) and b_ptrs = A_aᵀ ([K, r]). */
int mlora_gemm_fwd_fp8(const void *xq, int64_t ldx, const float *x_scale, int64_t M, int64_t K,
                       const void *wq, int64_t ldw, const float *w_scale, int64_t N,
                       const void *bias, int bias_dtype,
                       const void *h_rows, int64_t ldh,
                       const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                       const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                       void *y, int64_t ldy, int accumulate,
                       void *stream);

/* ---- fp32 arithmetic (the reference's precision='fp32' mode: no autocast,
 * training/single_device.py:77-80, so TrainableLowRankLinear computes
 * base(x) + s·F.linear(F.linear(x, A), B) and its autograd backward in fp32,
 * training/low_rank.py:26-28). Every operand, product and sum is IEEE float32 on the
 * gfx950 fp32 matrix core (v_mfma_f32_32x32x2_f32); sums run in a fixed order
 * (deterministic). Matrices are float32 row-major, 4-byte aligned, any shape; ranks are
 * any value in [0, MLORA_MAX_RANK] (no padding). Routing as above. */

/* h[m, j] = s_a · Σ_k P[m, k]·Op_a(j, k) for the rows of adapter segments (op_layout as
 * mlora_shrink), j < width; other entries of h [M, width] are written as 0.
 * Reference: F.linear(value, lora_a) (low_rank.py:28) and dH = s·dY·B of its backward. */
int mlora_f32_shrink(const void *p, int64_t ldp, int64_t M, int64_t K,
                     const void *const *op_ptrs, int op_layout,
                     const int32_t *ranks, const float *scales, int32_t n_adapters,
                     const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                     void *h, int64_t ldh, int64_t width,
                     void *stream);

/* Y[m, n] = Σ_k X[m,k]·W[n,k] + bias[n] + Σ_j h[m,j]·B_a[n,j] (h from mlora_f32_shrink, it
 * carries s_a); W [N, K], B_a [N, r_a] contiguous, bias NULL or [N].
 * Reference: low_rank.py:28, base(value) + scale·F.linear(F.linear(value, A), B). */
int mlora_f32_gemm_fwd(const void *x, int64_t ldx, int64_t M, int64_t K,
                       const void *w, int64_t ldw, int64_t N, const void *bias,
                       const void *h_rows, int64_t ldh,
                       const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                       const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                       void *y, int64_t ldy,
                       void *stream);

/* dX[m, k] = Σ_n dY[m,n]·W[n,k] + Σ_j g[m,j]·A_a[j,k] (g = s_a·dY·B_a from
 * mlora_f32_shrink with op_layout 1); A_a [r_a, K] contiguous.
 * Reference: autograd of low_rank.py:28, dX = dY·W + (s·dY·B)·A. */
int mlora_f32_gemm_dx(const void *dy, int64_t lddy, int64_t M, int64_t N,
                      const void *w, int64_t ldw, int64_t K,
                      const void *g_rows, int64_t ldg,
                      const void *const *a_ptrs, const int32_t *ranks, int32_t n_adapters,
                      const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                      void *dx, int64_t lddx,
                      void *stream);

/* D_a[c, j] = Σ_{m in segments of a} P[m, c]·H[m, j] (segments summed in routing order),
 * written to out_ptrs[a] as [C, r_a] (out_layout 0: dB_a = dYᵀ·h with P = dY, H = h) or
 * [r_a, C] (out_layout 1: dA_a = gᵀ·X with P = X, H = g). Adapters without rows get zeros.
 * Reference: autograd of low_rank.py:28 (dB = s·dYᵀ·(x·Aᵀ), dA = (s·dY·B)ᵀ·x). */
int mlora_f32_seg_outer(const void *p, int64_t ldp, int64_t M, int64_t C,
                        const void *h, int64_t ldh,
                        void *const *out_ptrs, int out_layout,
                        const int32_t *ranks, int32_t n_adapters,
                        const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                        void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MLORA_H_ */
