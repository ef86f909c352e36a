"""Autograd function of the batched multi-LoRA linear.

Forward (per row m of a segment with adapter a, rank r_a, scale s_a):
    Y[m] = X[m]·Wᵀ + b + s_a·(X[m]·A_aᵀ)·B_aᵀ
Backward (W and b frozen, as in the reference, training/low_rank.py:20):
    g[m]  = s_a·dY[m]·B_a                 (shrink of dY)
    dX[m] = dY[m]·W + g[m]·A_a            (transposed GEMM, LoRA term fused)
    dB_a  = s_a·Σ_{m∈a} dY[m]ᵀ·h[m]       (segmented reduction, h = X·A_aᵀ)
    dA_a  = Σ_{m∈a} g[m]ᵀ·X[m]            (segmented reduction)
which is the autograd of the reference's per-adapter forward
``base(value) + scale·F.linear(F.linear(value, lora_a), lora_b)``
(training/low_rank.py:26-28) applied to each segment.

Kernels: shrink -> fused GEMM forward; shrink(dY) -> fused dX GEMM and two
segmented reductions. Arithmetic by input type:
  * bf16 activations and base (or bf16 autocast, training/single_device.py:88): bf16
    MFMA with fp32 accumulation; under autocast the adapters are rounded to bf16 as
    autocast rounds F.linear's operands (low_rank.py:28 under autocast);
  * bf16 activations and base with fp32 adapter masters outside autocast (the
    fp32 LoRA compute of native/models.py:44-51,150-156): the shrinks multiply by the
    masters split into two bf16 parts (hi + lo, ~16 significant bits), so h, g and
    the adapter gradients are fp32-class; Y and dX stay bf16;
  * fp32 activations, base and adapters outside autocast (precision='fp32',
    training/single_device.py:77-80): MultiLoRAF32Function, every operation in
    float32 on the fp32 MFMA.
The adapter gradients come back in the parameters' dtype (fp32 masters stay fp32).
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as F

from . import _lib, kernels
from .routing import SegmentRouting


def _as_operand(t: torch.Tensor, rows_pad: int | None = None, cols_pad: int | None = None) -> torch.Tensor:
    """bf16 contiguous copy/view of an adapter matrix, zero-padded to a multiple of 8 ranks."""
    t = t.detach().to(torch.bfloat16).contiguous()
    if rows_pad is not None and rows_pad != t.shape[0]:
        t = F.pad(t, (0, 0, 0, rows_pad - t.shape[0]))
    if cols_pad is not None and cols_pad != t.shape[1]:
        t = F.pad(t, (0, cols_pad - t.shape[1]))
    return t


def _prepare(ctx, x, N: int, ab, scales, routing: SegmentRouting, grad0: int, row_div=None, split: bool = False):
    """Validate adapters, build padded bf16 operands and run the forward shrink.

    grad0 is the index of the first lora_a among the autograd inputs. split: the adapters
    are fp32 masters used at fp32-class precision (hi + lo bf16 parts in the shrinks).
    Returns (A_ops, B_ops, A_lo, B_lo, h_rows, h_frag); A_lo / B_lo are empty lists unless
    split. Records the routing and shapes on ctx.
    """
    n = len(ab) // 2
    if len(ab) != 2 * n or len(scales) != n:
        raise ValueError("multi-LoRA: one lora_a, one lora_b and one scale per adapter")
    As, Bs = ab[:n], ab[n:]
    M, K = x.shape
    routing.validate_for(M, n)
    ranks = [int(a.shape[0]) for a in As]
    for a, b, r in zip(As, Bs, ranks):
        if a.shape != (r, K) or b.shape != (N, r):
            raise ValueError(f"multi-LoRA: lora_a {tuple(a.shape)} / lora_b {tuple(b.shape)} do not match "
                             f"rank {r}, in {K}, out {N}")
    pranks = [(r + 7) // 8 * 8 for r in ranks]
    if split:
        A_ops, A_lo = zip(*[kernels.split_hi_lo(_as_operand_f32(a, rows_pad=p)) for a, p in zip(As, pranks)])
        B_ops, B_lo = zip(*[kernels.split_hi_lo(_as_operand_f32(b, cols_pad=p)) for b, p in zip(Bs, pranks)])
        A_ops, A_lo, B_ops, B_lo = list(A_ops), list(A_lo), list(B_ops), list(B_lo)
    else:
        A_ops = [_as_operand(a, rows_pad=p) for a, p in zip(As, pranks)]
        B_ops = [_as_operand(b, cols_pad=p) for b, p in zip(Bs, pranks)]
        A_lo, B_lo = [], []
    width = kernels.padded_rank(pranks)
    need_b_grad = any(ctx.needs_input_grad[grad0 + n + i] for i in range(n))
    h_rows, h_frag = (None, [])
    if width > 0:
        h_rows, h_frag = kernels.shrink(x, A_ops, 0, scales, routing, want_frag=need_b_grad, width=width,
                                        row_div=row_div, ops_lo=A_lo if split else None)
    ctx.routing, ctx.scales, ctx.n, ctx.grad0 = routing, tuple(float(s) for s in scales), n, grad0
    ctx.ranks, ctx.pranks, ctx.width, ctx.split = ranks, pranks, width, split
    ctx.a_dtypes = [a.dtype for a in As]
    ctx.b_dtypes = [b.dtype for b in Bs]
    return A_ops, B_ops, A_lo, B_lo, h_rows, list(h_frag or [])


def _as_operand_f32(t: torch.Tensor, rows_pad: int | None = None, cols_pad: int | None = None) -> torch.Tensor:
    """float32 copy/view of an adapter matrix, zero-padded to a multiple of 8 ranks."""
    t = t.detach().to(torch.float32)
    if rows_pad is not None and rows_pad != t.shape[0]:
        t = F.pad(t, (0, 0, 0, rows_pad - t.shape[0]))
    if cols_pad is not None and cols_pad != t.shape[1]:
        t = F.pad(t, (0, cols_pad - t.shape[1]))
    return t


def _save(ctx, *tensors, frag=()):
    """save_for_backward of the call's tensors followed by the h fragments (one per call group)."""
    ctx.n_frag = len(frag)
    ctx.save_for_backward(*tensors, *frag)


def _saved(ctx):
    """(tensors, h fragments) as _save stored them."""
    saved = list(ctx.saved_tensors)
    k = len(saved) - ctx.n_frag
    return saved[:k], saved[k:]


def _backward(ctx, dy, x, dx_gemm, A_ops, B_ops, h_frag, B_lo=None, row_div=None):
    """dX (dx_gemm(g_rows)), dA_i, dB_i; returns (dx, dAs, dBs).

    dy is bf16 contiguous; g_rows (the LoRA term of dX) are divided by row_div
    when given (the e4m3 dX folds dY's row scale into them). B_lo: the lo parts of
    split fp32 masters (g then uses hi + lo)."""
    n, g0, routing = ctx.n, ctx.grad0, ctx.routing
    need_x = ctx.needs_input_grad[0]
    need_a = [ctx.needs_input_grad[g0 + i] for i in range(n)]
    need_b = [ctx.needs_input_grad[g0 + n + i] for i in range(n)]
    dx = None
    g_rows = g_frag = None
    if ctx.width > 0 and (need_x or any(need_a)):
        g_rows, g_frag = kernels.shrink(dy, B_ops, 1, ctx.scales, routing, want_frag=any(need_a), width=ctx.width,
                                        row_div=row_div, ops_lo=B_lo or None)
    dAs: list = [None] * n
    dBs: list = [None] * n
    # dB right after the dY shrink, while dY is still in the last-level cache (0.15% per step at
    # the Wan shape against running it after the dX GEMM)
    if any(need_b):
        outs = kernels.seg_outer(dy, h_frag, ctx.width, ctx.pranks, routing, 0,
                                 [ctx.b_dtypes[i] for i in range(n)])
        dBs = [o[:, :r] if nb else None for o, r, nb in zip(outs, ctx.ranks, need_b)]
    if need_x:
        dx = dx_gemm(g_rows)
    if any(need_a):
        outs = kernels.seg_outer(x, g_frag, ctx.width, ctx.pranks, routing, 1,
                                 [ctx.a_dtypes[i] for i in range(n)])
        dAs = [o[:r] if na else None for o, r, na in zip(outs, ctx.ranks, need_a)]
    return dx, dAs, dBs


def _dx_gemm(dy, weight, weight_t, A_ops, routing):
    """dX = dY·W + g·A_a. With the frozen base also held transposed (weight_t [K, N]) it runs
    on the NT kernel against A_aᵀ ([K, r], transposed per call): 3-5% faster than the NN
    kernel that reads W's rows as the contraction (measured at the Wan shapes)."""
    if weight_t is not None:
        a_t = [a.t().contiguous() for a in A_ops]
        return lambda g_rows: kernels.gemm_fwd(dy, weight_t, None, g_rows, a_t, routing)
    return lambda g_rows: kernels.gemm_dx(dy, weight, g_rows, A_ops, routing)


class MultiLoRAFunction(torch.autograd.Function):
    """``apply(x, weight, weight_t, bias, routing, scales, split, *lora_as, *lora_bs)``.

    x [M, K] bf16 contiguous, weight [N, K] bf16 (frozen), weight_t None or weight
    transposed ([K, N] contiguous, frozen: dX then runs on the NT GEMM), bias [N] or None
    (frozen), routing a SegmentRouting over the M rows, scales one float per adapter;
    lora_as[i] [r_i, K], lora_bs[i] [N, r_i] of any float dtype. split: fp32 adapters are
    used at fp32-class precision (hi + lo bf16 parts) instead of rounded to bf16.
    """

    @staticmethod
    def forward(ctx, x, weight, weight_t, bias, routing: SegmentRouting, scales: Sequence[float], split: bool, *ab):
        if any(ctx.needs_input_grad[1:4]):
            raise RuntimeError("multi-LoRA: the base weight and bias are frozen (requires_grad=False)")
        A_ops, B_ops, A_lo, B_lo, h_rows, h_frag = _prepare(ctx, x, weight.shape[0], ab, scales, routing, grad0=7,
                                                            split=bool(split))
        y = kernels.gemm_fwd(x, weight, bias, h_rows, B_ops, routing)
        ctx.has_wt = weight_t is not None
        _save(ctx, x, weight, weight_t, *A_ops, *B_ops, *B_lo, frag=h_frag)
        return y

    @staticmethod
    def backward(ctx, dy):
        n = ctx.n
        (x, weight, weight_t, *ops), h_frag = _saved(ctx)
        dy = dy.to(torch.bfloat16).contiguous()
        dx_gemm = _dx_gemm(dy, weight, weight_t if ctx.has_wt else None, ops[:n], ctx.routing)
        dx, dAs, dBs = _backward(ctx, dy, x, dx_gemm, ops[:n], ops[n:2 * n], h_frag, B_lo=ops[2 * n:])
        return (dx, None, None, None, None, None, None, *dAs, *dBs)


class MultiLoRAF32Function(torch.autograd.Function):
    """``apply(x, weight, bias, routing, scales, *lora_as, *lora_bs)`` with every tensor float32: the
    reference's precision='fp32' mode (training/single_device.py:77-80), where
    TrainableLowRankLinear runs base(x) + s·F.linear(F.linear(x, A), B) (low_rank.py:26-28) and
    its autograd backward in float32. Every product and sum is float32 on the fp32 MFMA, in a
    fixed order: h = s·X·A_aᵀ, Y = X·Wᵀ + b + h·B_aᵀ; g = s·dY·B_a, dX = dY·W + g·A_a,
    dA_a = gᵀ·X, dB_a = dYᵀ·h over each adapter's rows.
    """

    @staticmethod
    def forward(ctx, x, weight, bias, routing: SegmentRouting, scales: Sequence[float], *ab):
        if any(ctx.needs_input_grad[1:3]):
            raise RuntimeError("multi-LoRA: the base weight and bias are frozen (requires_grad=False)")
        n = len(ab) // 2
        if len(ab) != 2 * n or len(scales) != n:
            raise ValueError("multi-LoRA: one lora_a, one lora_b and one scale per adapter")
        As, Bs = [a.detach().contiguous() for a in ab[:n]], [b.detach().contiguous() for b in ab[n:]]
        M, K = x.shape
        N = weight.shape[0]
        routing.validate_for(M, n)
        ranks = [int(a.shape[0]) for a in As]
        for a, b, r in zip(As, Bs, ranks):
            if a.shape != (r, K) or b.shape != (N, r):
                raise ValueError(f"multi-LoRA: lora_a {tuple(a.shape)} / lora_b {tuple(b.shape)} do not match "
                                 f"rank {r}, in {K}, out {N}")
        width = max([0, *ranks])
        h = kernels.f32_shrink(x, As, 0, scales, routing, width) if width else None
        y = kernels.f32_gemm_fwd(x, weight, bias, h, Bs, routing)
        ctx.routing, ctx.scales, ctx.n, ctx.ranks, ctx.width = routing, tuple(float(v) for v in scales), n, ranks, width
        ctx.save_for_backward(x, weight, h, *As, *Bs)
        return y

    @staticmethod
    def backward(ctx, dy):
        n, routing = ctx.n, ctx.routing
        x, weight, h, *ops = ctx.saved_tensors
        As, Bs = ops[:n], ops[n:]
        dy = dy.to(torch.float32).contiguous()
        need_x = ctx.needs_input_grad[0]
        need_a = any(ctx.needs_input_grad[5:5 + n])
        need_b = any(ctx.needs_input_grad[5 + n:])
        g = kernels.f32_shrink(dy, Bs, 1, ctx.scales, routing, ctx.width) if ctx.width and (need_x or need_a) else None
        dx = kernels.f32_gemm_dx(dy, weight, g, As, routing) if need_x else None
        dAs = kernels.f32_seg_outer(x, g, ctx.ranks, routing, 1) if need_a else [None] * n
        dBs = kernels.f32_seg_outer(dy, h, ctx.ranks, routing, 0) if need_b else [None] * n
        dAs = [d if ctx.needs_input_grad[5 + i] else None for i, d in enumerate(dAs)]
        dBs = [d if ctx.needs_input_grad[5 + n + i] else None for i, d in enumerate(dBs)]
        return (dx, None, None, None, None, *dAs, *dBs)


class MultiLoRAGatedResidualFunction(torch.autograd.Function):
    """``apply(x, weight, weight_t, bias, routing, scales, residual, gate, *lora_as, *lora_bs)``: the linear
    that closes a DiT block branch, with the block's gated residual fused into its epilogue:

        out = residual + bf16(Y)·gate[row group],   Y = the multi-LoRA linear of x

    (reference/livewan_wan21/wan/modules/model.py:305-313, rounding as
    runtime/helios_residual_kernel.py:66-86: fp32 multiply, fp32 add), in the residual
    stream's dtype: bf16 (the sum rounded to bf16) or float32 (the Wan block's stream, not
    rounded). residual [M, N], gate [G, N] fp32 frozen (M / G consecutive rows per gate row:
    the tokens of one sample). Backward (frozen gate, helios_residual_kernel.py:90-133):
    d residual = dOut; dY = bf16(dOut·gate), then the linear's own backward.
    """

    @staticmethod
    def forward(ctx, x, weight, weight_t, bias, routing: SegmentRouting, scales: Sequence[float], residual, gate,
                *ab):
        if any(ctx.needs_input_grad[1:4]):
            raise RuntimeError("multi-LoRA: the base weight and bias are frozen (requires_grad=False)")
        if ctx.needs_input_grad[7]:
            raise RuntimeError("gated residual: the gate is frozen (a trainable modulation is not fused)")
        A_ops, B_ops, _, _, h_rows, h_frag = _prepare(ctx, x, weight.shape[0], ab, scales, routing, grad0=8)
        out = kernels.gemm_fwd_gated(x, weight, bias, h_rows, B_ops, routing, residual, gate)
        ctx.has_wt = weight_t is not None
        _save(ctx, x, weight, weight_t, gate, *A_ops, *B_ops, frag=h_frag)
        return out

    @staticmethod
    def backward(ctx, dout):
        n = ctx.n
        (x, weight, weight_t, gate, *ops), h_frag = _saved(ctx)
        dout = dout.contiguous()
        dy = kernels.gate_scale_rows(dout, gate)
        dx_gemm = _dx_gemm(dy, weight, weight_t if ctx.has_wt else None, ops[:n], ctx.routing)
        dx, dAs, dBs = _backward(ctx, dy, x, dx_gemm, ops[:n], ops[n:], h_frag)
        d_res = dout if ctx.needs_input_grad[6] else None
        return (dx, None, None, None, None, None, d_res, None, *dAs, *dBs)


class MultiLoRAFP8Function(torch.autograd.Function):
    """``apply(x, wq, w_scale, wq_t, bias, routing, scales, dx_bf16, *lora_as, *lora_bs)``:
    the same linear with the frozen base stored as e4m3 ``wq`` [N, K] and one
    fp32 scale per output channel ``w_scale`` [N] (base weight =
    w_scale[n]·wq[n, k]); ``wq_t`` is wq transposed ([K, N], for dX).

    Forward: X is quantised per token to e4m3 (mlora_quantize_rows_fp8) and the
    base product runs on the e4m3 MFMA with fp32 accumulation; the LoRA shrink
    and expand stay bf16 on the unquantised X. Backward: dX = dY·W + g·A runs
    on the e4m3 MFMA as well — dY·w_scale[n] quantised per row (scale
    dy_scale), times wq_t, plus the bf16 LoRA term g/dy_scale times A_aᵀ, all
    scaled by dy_scale[m] in the epilogue; dA, dB as in the bf16 path. With
    ``dx_bf16`` the dX runs instead on the bf16 MFMA against the base dequantised
    to bf16 (bf16(w_scale[n]·wq[n, k]), made per call): dY is not quantised, so dX
    carries bf16 rounding only (2.3e-3 rel-L2 against 2.6e-2 at config 5), at the cost of
    a slower dX (+16-17% per fwd+bwd step at config 5).
    """

    @staticmethod
    def forward(ctx, x, wq, w_scale, wq_t, bias, routing: SegmentRouting, scales: Sequence[float], dx_bf16: bool,
                *ab):
        if any(ctx.needs_input_grad[1:5]):
            raise RuntimeError("multi-LoRA: the base weight, its scale and the bias are frozen")
        xq, x_scale = kernels.quantize_rows_fp8(x)
        # the LoRA operands enter the e4m3 accumulators divided by the scales the
        # epilogue multiplies back: h / x_scale[m] (shrink) and lora_b / w_scale[n]
        A_ops, B_ops, _, _, h_rows, h_frag = _prepare(ctx, x, wq.shape[0], ab, scales, routing, grad0=8,
                                                      row_div=x_scale)
        B_div = kernels.div_rows_bf16_many(B_ops, w_scale)
        y = kernels.gemm_fwd_fp8(xq, x_scale, wq, w_scale, bias, h_rows, B_div, routing)
        ctx.dx_bf16 = bool(dx_bf16)
        _save(ctx, x, wq if ctx.dx_bf16 else wq_t, w_scale, *A_ops, *B_ops, frag=h_frag)
        return y

    @staticmethod
    def backward(ctx, dy):
        n = ctx.n
        (x, wq_or_t, w_scale, *ops), h_frag = _saved(ctx)
        dy = dy.to(torch.bfloat16).contiguous()
        if ctx.dx_bf16:
            def dx_gemm(g_rows):
                w_deq = kernels.dequant_rows_fp8(wq_or_t, w_scale)  # bf16 [N, K]
                return kernels.gemm_dx(dy, w_deq, g_rows, ops[:n], ctx.routing)

            dx, dAs, dBs = _backward(ctx, dy, x, dx_gemm, ops[:n], ops[n:], h_frag)
        else:
            dyq = dy_scale = None
            if ctx.needs_input_grad[0]:
                dyq, dy_scale = kernels.quantize_rows_fp8(dy, col_scale=w_scale)

            def dx_gemm(g_rows):
                a_t = [a.t().contiguous() for a in ops[:n]]  # A_aᵀ [K, r]: the NT form of the LoRA term
                return kernels.gemm_fwd_fp8(dyq, dy_scale, wq_or_t, None, None, g_rows, a_t, ctx.routing)

            dx, dAs, dBs = _backward(ctx, dy, x, dx_gemm, ops[:n], ops[n:], h_frag, row_div=dy_scale)
        return (dx, None, None, None, None, None, None, None, *dAs, *dBs)


def _stack_slices(G: int, R: int) -> list[tuple[int, int]]:
    """Member ranges [g0, g1) of G stacked linears of rank R whose side-by-side LoRA rows fit one
    shrink / reduction call (at most MAX_RANK columns: 2 members of rank 128, 1 of rank 256); the
    GEMMs take all G·R columns at once (MAX_GEMM_RANK)."""
    per = max(1, _lib.MAX_RANK // R)
    return [(g0, min(G, g0 + per)) for g0 in range(0, G, per)]


def _stacked_operand(mats: Sequence[torch.Tensor], split: bool) -> tuple[torch.Tensor, torch.Tensor | None]:
    """The matrices stacked by rows as one bf16 operand: (hi, None), or with ``split`` (fp32
    masters at fp32-class precision) the (hi, lo) parts of the fp32 stack."""
    if split:
        return kernels.split_hi_lo(torch.cat([m.detach().to(torch.float32) for m in mats]))
    if len(mats) == 1:
        return _as_operand(mats[0]), None
    return torch.cat([_as_operand(m) for m in mats]), None


def _stacked_shrink(x, A_hi, A_lo, scales, routing: SegmentRouting, G: int, R: int, want_frag: bool):
    """h [M, G·R] of G stacked linears (linear g at columns g·R) from the stacked A ([G·R, K] per
    adapter), by one shrink per member slice (_stack_slices); returns (h_rows, the fragments of
    each slice, or empty lists)."""
    h_rows = torch.empty((x.shape[0], G * R), dtype=torch.bfloat16, device=x.device)
    frags = []
    for g0, g1 in _stack_slices(G, R):
        c = slice(g0 * R, g1 * R)
        _, f = kernels.shrink(x, [a[c] for a in A_hi], 0, scales, routing, want_frag=want_frag, width=(g1 - g0) * R,
                              h_out=h_rows[:, c], ops_lo=None if A_lo is None else [a[c] for a in A_lo])
        frags.append(list(f or []))
    return h_rows, frags


def _save_stacked(ctx, tensors, frags) -> None:
    """save_for_backward of the call's tensors and the per-slice fragments."""
    ctx.frag_counts = [len(f) for f in frags]
    _save(ctx, *tensors, frag=[t for f in frags for t in f])


def _saved_stacked(ctx):
    tensors, flat = _saved(ctx)
    frags, k = [], 0
    for c in ctx.frag_counts:
        frags.append(flat[k:k + c])
        k += c
    return tensors, frags


def _stacked_grads(ctx, x, dys, b_hi, b_lo, h_frags, dx_fn, a0: int, b0: int):
    """Backward of G stacked linears of rank R (ctx.G, ctx.R, ctx.n adapters): g_g = s·dY_g·B_g
    side by side into g [M, G·R] (fragments per member slice), dX = dx_fn(g_rows), dA of each
    slice's members from one reduction over X, dB_g from one reduction over dY_g. b_hi[g] /
    b_lo[g]: linear g's B operands ([N_g, R] per adapter; lo None unless split); a0 / b0: the
    autograd input index of the first lora_a / lora_b."""
    G, R, n, routing = ctx.G, ctx.R, ctx.n, ctx.routing
    need_x = ctx.needs_input_grad[0]
    need_a = [[ctx.needs_input_grad[a0 + g * n + i] for i in range(n)] for g in range(G)]
    need_b = [[ctx.needs_input_grad[b0 + g * n + i] for i in range(n)] for g in range(G)]
    any_a = any(map(any, need_a))
    slices = _stack_slices(G, R)
    g_rows, g_frags = None, [None] * len(slices)
    dA = [[None] * n for _ in range(G)]
    dB = [[None] * n for _ in range(G)]
    if need_x or any_a:
        g_rows = torch.empty((x.shape[0], G * R), dtype=torch.bfloat16, device=x.device)
    for s, (g0, g1) in enumerate(slices):
        w = (g1 - g0) * R
        if need_x or any_a:
            g_frags[s] = kernels.alloc_frags(routing, w // 16, x.device) if any_a else None
        for g in range(g0, g1):
            if need_x or any_a:
                kernels.shrink(dys[g], b_hi[g], 1, ctx.scales, routing, want_frag=any_a, width=w,
                               h_out=g_rows[:, g * R:(g + 1) * R], frag_out=g_frags[s], frag_jt=w // 16,
                               frag_t0=(g - g0) * R // 16, ops_lo=b_lo[g])
            if any(need_b[g]):  # right after the shrink of dY_g, while dY_g is still cached
                outs = kernels.seg_outer(dys[g], h_frags[s], w, [R] * n, routing, 0, ctx.b_dtypes[g],
                                         frag_jt=w // 16, frag_t0=(g - g0) * R // 16)
                dB[g] = [o if need_b[g][i] else None for i, o in enumerate(outs)]
    dx = dx_fn(g_rows) if need_x else None
    for s, (g0, g1) in enumerate(slices):
        w = (g1 - g0) * R
        if any(any(need_a[g]) for g in range(g0, g1)):
            outs = kernels.seg_outer(x, g_frags[s], w, [w] * n, routing, 1, [torch.float32] * n)
            for g in range(g0, g1):
                dA[g] = [outs[i][(g - g0) * R:(g - g0 + 1) * R].to(ctx.a_dtypes[g][i]) if need_a[g][i] else None
                         for i in range(n)]
    return dx, dA, dB


def _check_stack(what: str, As, Bs, K: int, widths: Sequence[int]) -> int:
    """One rank R (a multiple of 16) for every linear and adapter; returns R."""
    R = int(As[0][0].shape[0])
    if R % 16 or R > _lib.MAX_RANK:
        raise ValueError(f"{what}: the rank must be a multiple of 16, at most {_lib.MAX_RANK} (got {R})")
    for g, N in enumerate(widths):
        for a, b in zip(As[g], Bs[g]):
            if a.shape != (R, K) or b.shape != (N, R):
                raise ValueError(f"{what}: lora_a {tuple(a.shape)} / lora_b {tuple(b.shape)} of linear {g} do not "
                                 f"match rank {R}, in {K}, out {N}")
    return R


class SharedInputMultiLoRAFunction(torch.autograd.Function):
    """``apply(x, routing, scales, groups, weights, biases, split, *lora_as, *lora_bs)``: G =
    ``groups`` multi-LoRA linears that read the same input x [M, K].

    weights / biases: tuples of the G frozen bases ([N_g, K] bf16; bias [N_g] or None);
    lora_as = [A_g,i for g < G for i < n] ([R, K] each), lora_bs likewise ([N_g, R]): one rank R
    (a multiple of 16, at most 256) for every linear and adapter, adapter i's scale scales[i] in
    every linear. split: fp32 adapter masters used at fp32-class precision (hi + lo bf16 parts in
    the shrinks), as MultiLoRAFunction does. Returns the G outputs [M, N_g], each equal to its own
    multi-LoRA linear's.

    Forward: shrinks of X by the stacked [A_0,i; …; A_{G-1},i], 256 columns per call (X read once
    per call instead of once per linear), then each linear's fused GEMM reading its R columns of
    the stacked h. Backward: the G shrinks g_g = s·dY_g·B_g write side by side into one g
    [M, G·R] and its fragments; dX accumulates the G linears' dY_g·W_g + g_g·A_g in the dX GEMM's
    epilogue (fp32 sum, one bf16 rounding per call, instead of autograd's G-1 separate bf16
    additions); dA of the linears of one 256-column slice is one reduction over X; dB_g one
    reduction per dY_g.
    """

    @staticmethod
    def forward(ctx, x, routing: SegmentRouting, scales: Sequence[float], groups: int, weights, biases, split: bool,
                *ab):
        G = int(groups)
        n = len(ab) // (2 * G) if G > 0 else 0
        if G < 2 or n == 0 or len(ab) != 2 * G * n or len(scales) != n or len(weights) != G or len(biases) != G:
            raise ValueError("shared-input multi-LoRA: G >= 2 linears, G·n lora_a and G·n lora_b, one scale per adapter")
        if any(w.requires_grad for w in weights) or any(b is not None and b.requires_grad for b in biases):
            raise RuntimeError("multi-LoRA: the base weight and bias are frozen (requires_grad=False)")
        M, K = x.shape
        As = [list(ab[g * n:(g + 1) * n]) for g in range(G)]
        Bs = [list(ab[G * n + g * n:G * n + (g + 1) * n]) for g in range(G)]
        routing.validate_for(M, n)
        for g in range(G):
            if weights[g].shape[1] != K:
                raise ValueError(f"shared-input multi-LoRA: linear {g} has in_features {weights[g].shape[1]}, "
                                 f"the input has {K}")
        R = _check_stack("shared-input multi-LoRA", As, Bs, K, [w.shape[0] for w in weights])
        split = bool(split)
        A_hi, A_lo = zip(*[_stacked_operand([As[g][i] for g in range(G)], split) for i in range(n)])  # [G·R, K]
        B_parts = [[_stacked_operand([b], split) for b in Bs[g]] for g in range(G)]
        B_hi = [[p[0] for p in bp] for bp in B_parts]
        B_lo = [[p[1] for p in bp] for bp in B_parts] if split else []
        need_b_grad = any(ctx.needs_input_grad[7 + G * n:])
        h_rows, frags = _stacked_shrink(x, A_hi, A_lo if split else None, scales, routing, G, R, need_b_grad)
        ys = [kernels.gemm_fwd(x, weights[g], biases[g], h_rows[:, g * R:(g + 1) * R], B_hi[g], routing)
              for g in range(G)]
        _save_stacked(ctx, [x, *weights, *A_hi, *[b for bg in B_hi for b in bg], *[b for bg in B_lo for b in bg]],
                      frags)
        ctx.routing, ctx.scales, ctx.n, ctx.G, ctx.R = routing, tuple(float(v) for v in scales), n, G, R
        ctx.split = split
        ctx.a_dtypes = [[a.dtype for a in As[g]] for g in range(G)]
        ctx.b_dtypes = [[b.dtype for b in Bs[g]] for g in range(G)]
        return tuple(ys)

    @staticmethod
    def backward(ctx, *dys):
        n, G, R, routing = ctx.n, ctx.G, ctx.R, ctx.routing
        (x, *ops), h_frags = _saved_stacked(ctx)
        ws, ops = ops[:G], ops[G:]
        A_hi = ops[:n]
        B_hi = [ops[n + g * n:n + (g + 1) * n] for g in range(G)]
        B_lo = ([ops[n + G * n + g * n:n + G * n + (g + 1) * n] for g in range(G)] if ctx.split
                else [None] * G)
        M = x.shape[0]
        # an output nobody used has no gradient: it contributes zeros
        dys = [torch.zeros((M, ws[g].shape[0]), dtype=torch.bfloat16, device=x.device) if d is None
               else d.to(torch.bfloat16).contiguous() for g, d in enumerate(dys)]

        def dx_fn(g_rows):
            dx = None
            for g in range(G):
                dx = kernels.gemm_dx(dys[g], ws[g], g_rows[:, g * R:(g + 1) * R],
                                     [a[g * R:(g + 1) * R] for a in A_hi], routing, out=dx, accumulate=g > 0)
            return dx

        dx, dA, dB = _stacked_grads(ctx, x, dys, B_hi, B_lo, h_frags, dx_fn, a0=7, b0=7 + G * n)
        return (dx, None, None, None, None, None, None, *[d for dg in dA for d in dg], *[d for dg in dB for d in dg])


class StackedLinearsFunction(torch.autograd.Function):
    """``apply(x, routing, scales, groups, w_cat, b_cat, w_cat_t, split, *lora_as, *lora_bs)``: G
    multi-LoRA linears that read x [M, K], as one stacked call. w_cat [G·N, K] bf16 = their frozen
    weights stacked by rows (b_cat [G·N] or None, w_cat_t = w_cat transposed [K, G·N] or None, all
    frozen); lora_as = [A_g,i for g < G for i < n] ([R, K] each), lora_bs likewise ([N, R]); one
    rank R (a multiple of 16, at most 256) and one output width N (a multiple of 256) for every
    linear. split: fp32 adapter masters at fp32-class precision (hi + lo bf16 parts in the
    shrinks). Returns the G outputs [M, N], each bit-identical to that linear's own call.

    Forward: shrinks of X by the stacked [A_0,i; ...; A_{G-1},i], 256 columns per call (X read
    once per call), and one GEMM over the stacked weights (mlora_gemm_fwd_stacked: X's row tiles
    feed all G linears' column tiles). Backward: the G shrinks g_g = s·dY_g·B_g side by side into
    g [M, G·R]; dX = Σ_g dY_g·W_g + g·A_cat as ONE GEMM whose contraction runs over the G dY in
    turn and then the G·R columns of g (mlora_gemm_dx_stacked: no concatenated dY, no per-linear
    dX, one rounding of the sum); dA of each 256-column slice's linears from one reduction over
    X; dB_g one reduction over dY_g.
    """

    @staticmethod
    def forward(ctx, x, routing: SegmentRouting, scales: Sequence[float], groups: int, w_cat, b_cat, w_cat_t,
                split: bool, *ab):
        G = int(groups)
        n = len(ab) // (2 * G) if G > 0 else 0
        if G < 2 or n == 0 or len(ab) != 2 * G * n or len(scales) != n:
            raise ValueError("stacked multi-LoRA: G >= 2 linears, G·n lora_a and G·n lora_b, one scale per adapter")
        if w_cat.requires_grad or (b_cat is not None and b_cat.requires_grad):
            raise RuntimeError("multi-LoRA: the base weight and bias are frozen (requires_grad=False)")
        M, K = x.shape
        NT = w_cat.shape[0]
        N = NT // G
        As = [list(ab[g * n:(g + 1) * n]) for g in range(G)]
        Bs = [list(ab[G * n + g * n:G * n + (g + 1) * n]) for g in range(G)]
        routing.validate_for(M, n)
        if NT != G * N or N % 256 or G > _lib.MAX_STACKED or w_cat.shape[1] != K:
            raise ValueError(f"stacked multi-LoRA: {G} linears (at most {_lib.MAX_STACKED}) of width {N} (a multiple "
                             f"of 256) over in_features {K}")
        R = _check_stack("stacked multi-LoRA", As, Bs, K, [N] * G)
        split = bool(split)
        A_hi, A_lo = zip(*[_stacked_operand([As[g][i] for g in range(G)], split) for i in range(n)])  # [G·R, K]
        B_hi, B_lo = zip(*[_stacked_operand([Bs[g][i] for g in range(G)], split) for i in range(n)])  # [G·N, R]
        need_b_grad = any(ctx.needs_input_grad[8 + G * n:])
        h_rows, frags = _stacked_shrink(x, A_hi, A_lo if split else None, scales, routing, G, R, need_b_grad)
        ys = kernels.gemm_fwd_stacked(x, w_cat, b_cat, h_rows, B_hi, routing, N, R)
        _save_stacked(ctx, [x, w_cat, w_cat_t, *A_hi, *B_hi, *(B_lo if split else ())], frags)
        ctx.routing, ctx.scales, ctx.n, ctx.G, ctx.R, ctx.N = routing, tuple(float(v) for v in scales), n, G, R, N
        ctx.has_wt, ctx.split = w_cat_t is not None, split
        ctx.a_dtypes = [[a.dtype for a in As[g]] for g in range(G)]
        ctx.b_dtypes = [[b.dtype for b in Bs[g]] for g in range(G)]
        return tuple(ys)

    @staticmethod
    def backward(ctx, *dys):
        n, G, N, routing = ctx.n, ctx.G, ctx.N, ctx.routing
        (x, w_cat, w_cat_t, *ops), h_frags = _saved_stacked(ctx)
        A_hi, B_hi, B_lo = ops[:n], ops[n:2 * n], ops[2 * n:]
        M = x.shape[0]
        # an output nobody used has no gradient: it contributes zeros
        dys = [torch.zeros((M, N), dtype=torch.bfloat16, device=x.device) if d is None
               else d.to(torch.bfloat16).contiguous() for d in dys]
        member = lambda parts, g: [b[g * N:(g + 1) * N] for b in parts]  # noqa: E731

        def dx_fn(g_rows):
            if ctx.has_wt:  # one GEMM over the G dY against the stacked base held transposed
                return kernels.gemm_dx_stacked(dys, w_cat_t, g_rows, [a.t().contiguous() for a in A_hi], routing)
            # NN form over the stacked base: the dY side by side
            return kernels.gemm_dx(torch.cat(dys, dim=1), w_cat, g_rows, list(A_hi), routing)

        dx, dA, dB = _stacked_grads(ctx, x, dys, [member(B_hi, g) for g in range(G)],
                                    [member(B_lo, g) if ctx.split else None for g in range(G)], h_frags, dx_fn,
                                    a0=8, b0=8 + G * n)
        return (dx, None, None, None, None, None, None, None, *[d for dg in dA for d in dg],
                *[d for dg in dB for d in dg])


def _bf16_rows(x: torch.Tensor, weight_dtype: torch.dtype) -> torch.Tensor:
    """x [..., K] as contiguous bf16 rows [M, K] (under bf16 autocast the cast is done here)."""
    x2 = x.reshape(-1, x.shape[-1])
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
        weight_dtype = torch.bfloat16
    if x2.dtype != torch.bfloat16 or weight_dtype != torch.bfloat16:
        raise RuntimeError("multi-LoRA linear computes in bfloat16: pass bf16 input and base weight, "
                           "or call it under torch.autocast('cuda', dtype=torch.bfloat16)")
    if not x2.is_cuda:
        raise RuntimeError("multi-LoRA linear runs on the ROCm device only (HIP kernels, no CPU path)")
    return x2.contiguous()


def shared_input_multi_lora(x: torch.Tensor, weights: Sequence[torch.Tensor], biases: Sequence[torch.Tensor | None],
                            lora_as: Sequence[Sequence[torch.Tensor]], lora_bs: Sequence[Sequence[torch.Tensor]],
                            scales: Sequence[float], routing: SegmentRouting,
                            transposed_base_for_dx: bool = True) -> tuple[torch.Tensor, ...]:
    """Functional form over x [..., K]: the G linears' outputs [..., N_g]; lora_as[g][i] / lora_bs[g][i]
    are linear g's adapter i (one rank, a multiple of 16, for all). Linears of one width (a multiple
    of 256, at most MAX_STACKED of them) run as one stacked call (StackedLinearsFunction) over a
    cached stacked copy of their frozen bases; other widths run SharedInputMultiLoRAFunction (shared
    shrinks, per-linear GEMMs). Arithmetic as multi_lora_linear's for bf16 x: under bf16 autocast
    the adapters are rounded to bf16; outside it fp32 adapter masters are used at fp32-class
    precision."""
    from .low_rank import stacked_bases
    lead = x.shape[:-1]
    G = len(weights)
    x2 = _bf16_rows(x, weights[0].dtype)
    flat_a = [a for g in range(G) for a in lora_as[g]]
    flat_b = [b for g in range(G) for b in lora_bs[g]]
    split = not _autocast_bf16() and any(t.dtype == torch.float32 for t in (*flat_a, *flat_b))
    widths = {int(w.shape[0]) for w in weights}
    if len(widths) == 1 and next(iter(widths)) % 256 == 0 and G <= _lib.MAX_STACKED:
        N = next(iter(widths))
        want_t = transposed_base_for_dx and torch.is_grad_enabled() and x.requires_grad
        w_cat, b_cat, w_cat_t = stacked_bases(list(weights), list(biases), want_t)
        with torch.autocast("cuda", enabled=False):
            ys = StackedLinearsFunction.apply(x2, routing, tuple(scales), G, w_cat, b_cat, w_cat_t if want_t else None,
                                              split, *flat_a, *flat_b)
        return tuple(v.reshape(*lead, N) for v in ys)
    ws = tuple(w.detach().to(torch.bfloat16) for w in weights)  # a no-op unless autocast runs fp32 bases
    bs = tuple(None if b is None else b.detach() for b in biases)
    with torch.autocast("cuda", enabled=False):
        ys = SharedInputMultiLoRAFunction.apply(x2, routing, tuple(scales), G, ws, bs, split, *flat_a, *flat_b)
    return tuple(y.reshape(*lead, w.shape[0]) for y, w in zip(ys, ws))


def _autocast_bf16() -> bool:
    return torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16


def multi_lora_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                      lora_as: Sequence[torch.Tensor], lora_bs: Sequence[torch.Tensor],
                      scales: Sequence[float], routing: SegmentRouting,
                      weight_t: torch.Tensor | None = None) -> torch.Tensor:
    """Functional form over x of shape [..., K]; returns [..., N]. weight_t: the frozen
    weight transposed ([K, N] bf16 contiguous, made once by the caller) for the faster dX.

    Arithmetic follows the inputs, as the reference's F.linear calls would (see the module doc):
    under bf16 autocast, or with bf16 x and weight, bf16 out (fp32 adapters outside autocast are
    used at fp32-class precision); with float32 x, weight and adapters outside autocast, float32
    out computed in float32 (MultiLoRAF32Function). Other combinations raise."""
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    split = f32 = False
    if _autocast_bf16():
        x2 = x2.to(torch.bfloat16)
        weight = weight.to(torch.bfloat16)
    elif x2.dtype == torch.float32 and weight.dtype == torch.float32:
        tensors = [*lora_as, *lora_bs] + ([bias] if bias is not None else [])
        if any(t.dtype != torch.float32 for t in tensors):
            raise RuntimeError("multi-LoRA linear in float32: the bias and the adapters must be float32 too "
                               "(as F.linear requires one dtype outside autocast)")
        f32 = True
    elif x2.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16:
        split = any(t.dtype == torch.float32 for t in [*lora_as, *lora_bs])
    else:
        raise RuntimeError("multi-LoRA linear computes in bfloat16 or float32: pass bf16 (or float32) input and "
                           "base weight, or call it under torch.autocast('cuda', dtype=torch.bfloat16)")
    if not x2.is_cuda:
        raise RuntimeError("multi-LoRA linear runs on the ROCm device only (HIP kernels, no CPU path)")
    with torch.autocast("cuda", enabled=False):
        if f32:
            y = MultiLoRAF32Function.apply(x2.contiguous(), weight.detach().contiguous(), bias, routing,
                                           tuple(scales), *lora_as, *lora_bs)
        else:
            y = MultiLoRAFunction.apply(x2.contiguous(), weight, weight_t, bias, routing, tuple(scales), split,
                                        *lora_as, *lora_bs)
    return y.reshape(*lead, weight.shape[0])


def multi_lora_linear_gated(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                            lora_as: Sequence[torch.Tensor], lora_bs: Sequence[torch.Tensor],
                            scales: Sequence[float], routing: SegmentRouting, residual: torch.Tensor,
                            gate: torch.Tensor, weight_t: torch.Tensor | None = None) -> torch.Tensor:
    """residual + linear(x)·gate, fused (MultiLoRAGatedResidualFunction). x [..., K]; residual
    [..., N] bf16 or float32 (the Wan block's stream) with x's leading shape; gate fp32 [B, 1, N]
    (one row per sample of a [B, L, ...] batch), [B, L, N] (per token) or [G, N]. Returns
    [..., N] in the residual's dtype."""
    K, N = x.shape[-1], weight.shape[0]
    lead = x.shape[:-1]
    x2 = _bf16_rows(x, weight.dtype)
    weight = weight.to(torch.bfloat16)
    if residual.dtype not in (torch.bfloat16, torch.float32) or residual.shape != (*lead, N):
        raise RuntimeError("gated residual: the residual stream must be bf16 or float32 with the output's shape")
    if gate.dtype != torch.float32 or gate.shape[-1] != N:
        raise RuntimeError("gated residual: the gate must be float32 with out_features columns")
    g2 = gate.reshape(-1, N)
    if g2.stride(1) != 1 or g2.stride(0) % 4 or g2.data_ptr() % 16:
        g2 = g2.contiguous()
    with torch.autocast("cuda", enabled=False):
        out = MultiLoRAGatedResidualFunction.apply(x2, weight, weight_t, bias, routing, tuple(scales),
                                                   residual.reshape(-1, N).contiguous(), g2, *lora_as, *lora_bs)
    return out.reshape(*lead, N)


def multi_lora_linear_fp8(x: torch.Tensor, wq: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None,
                          lora_as: Sequence[torch.Tensor], lora_bs: Sequence[torch.Tensor],
                          scales: Sequence[float], routing: SegmentRouting,
                          wq_t: torch.Tensor | None = None, dx_bf16: bool = False) -> torch.Tensor:
    """Functional form with an e4m3 base (wq [N, K] float8_e4m3fn, w_scale [N] fp32); bf16 out.

    wq_t: wq transposed ([K, N], contiguous) for the e4m3 dX; made here when not given (a frozen
    base keeps it, see MultiLoRALinear.quantize_base_fp8). dx_bf16: dX on the bf16 MFMA against
    the dequantised base (no quantisation of dY; +16-17% per fwd+bwd step at config 5)."""
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
    if x2.dtype != torch.bfloat16:
        raise RuntimeError("multi-LoRA linear computes in bfloat16: pass a bf16 input, "
                           "or call it under torch.autocast('cuda', dtype=torch.bfloat16)")
    if not x2.is_cuda:
        raise RuntimeError("multi-LoRA linear runs on the ROCm device only (HIP kernels, no CPU path)")
    if wq_t is None and not dx_bf16:
        wq_t = wq.t().contiguous()
    with torch.autocast("cuda", enabled=False):
        y = MultiLoRAFP8Function.apply(x2.contiguous(), wq, w_scale, wq_t, bias, routing, tuple(scales),
                                       bool(dx_bf16), *lora_as, *lora_bs)
    return y.reshape(*lead, wq.shape[0])
