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
segmented reductions. Compute is bf16 with fp32 accumulation; the adapter
gradients come back in the parameters' dtype (fp32 masters stay fp32).
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as F

from . import kernels
from .routing import SegmentRouting


def _as_operand(t: torch.Tensor, rows_pad: int | None = None, cols_pad: int | None = None) -> torch.Tensor:
    """bf16 contiguous copy/view of an adapter matrix, zero-padded to a multiple of 8 ranks."""
    t = t.detach().to(torch.bfloat16).contiguous()
    if rows_pad is not None and rows_pad != t.shape[0]:
        t = F.pad(t, (0, 0, 0, rows_pad - t.shape[0]))
    if cols_pad is not None and cols_pad != t.shape[1]:
        t = F.pad(t, (0, cols_pad - t.shape[1]))
    return t


class MultiLoRAFunction(torch.autograd.Function):
    """``apply(x, weight, bias, routing, scales, *lora_as, *lora_bs)``.

    x [M, K] bf16 contiguous, weight [N, K] bf16 (frozen), bias [N] or None
    (frozen), routing a SegmentRouting over the M rows, scales one float per
    adapter; lora_as[i] [r_i, K], lora_bs[i] [N, r_i] of any float dtype.
    """

    @staticmethod
    def forward(ctx, x, weight, bias, routing: SegmentRouting, scales: Sequence[float], *ab):
        n = len(ab) // 2
        if len(ab) != 2 * n or len(scales) != n:
            raise ValueError("multi-LoRA: one lora_a, one lora_b and one scale per adapter")
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            raise RuntimeError("multi-LoRA: the base weight and bias are frozen (requires_grad=False)")
        As, Bs = ab[:n], ab[n:]
        M, K = x.shape
        N = weight.shape[0]
        routing.validate_for(M, n)
        ranks = [int(a.shape[0]) for a in As]
        for a, b, r in zip(As, Bs, ranks):
            if a.shape != (r, K) or b.shape != (N, r):
                raise ValueError(f"multi-LoRA: lora_a {tuple(a.shape)} / lora_b {tuple(b.shape)} do not match "
                                 f"rank {r}, in {K}, out {N}")
        pranks = [(r + 7) // 8 * 8 for r in ranks]
        A_ops = [_as_operand(a, rows_pad=p) for a, p in zip(As, pranks)]
        B_ops = [_as_operand(b, cols_pad=p) for b, p in zip(Bs, pranks)]
        width = kernels.padded_rank(pranks)
        need_b_grad = any(ctx.needs_input_grad[5 + n + i] for i in range(n))
        h_rows, h_frag = (None, None)
        if width > 0:
            h_rows, h_frag = kernels.shrink(x, A_ops, 0, scales, routing, want_frag=need_b_grad, width=width)
        y = kernels.gemm_fwd(x, weight, bias, h_rows, B_ops, routing)
        ctx.routing, ctx.scales, ctx.n = routing, tuple(float(s) for s in scales), n
        ctx.ranks, ctx.pranks, ctx.width = ranks, pranks, width
        ctx.a_dtypes = [a.dtype for a in As]
        ctx.b_dtypes = [b.dtype for b in Bs]
        ctx.h_frag = h_frag  # per call group; plain tensors produced and consumed here
        ctx.save_for_backward(x, weight, *A_ops, *B_ops)
        return y

    @staticmethod
    def backward(ctx, dy):
        n = ctx.n
        x, weight, *ops = ctx.saved_tensors
        h_frag = ctx.h_frag
        A_ops, B_ops = ops[:n], ops[n:]
        routing = ctx.routing
        need_x = ctx.needs_input_grad[0]
        need_a = [ctx.needs_input_grad[5 + i] for i in range(n)]
        need_b = [ctx.needs_input_grad[5 + n + i] for i in range(n)]
        dy = dy.to(torch.bfloat16).contiguous()
        dx = None
        g_rows = g_frag = None
        if ctx.width > 0 and (need_x or any(need_a)):
            g_rows, g_frag = kernels.shrink(dy, B_ops, 1, ctx.scales, routing, want_frag=any(need_a), width=ctx.width)
        if need_x:
            dx = kernels.gemm_dx(dy, weight, g_rows, A_ops, routing)
        dAs: list = [None] * n
        dBs: list = [None] * n
        if any(need_b):
            outs = kernels.seg_outer(dy, h_frag, ctx.width, ctx.pranks, routing, 0,
                                     [ctx.b_dtypes[i] for i in range(n)])
            dBs = [o[:, :r] if nb else None for o, r, nb in zip(outs, ctx.ranks, need_b)]
        if any(need_a):
            outs = kernels.seg_outer(x, g_frag, ctx.width, ctx.pranks, routing, 1,
                                     [ctx.a_dtypes[i] for i in range(n)])
            dAs = [o[:r] if na else None for o, r, na in zip(outs, ctx.ranks, need_a)]
        return (dx, None, None, None, None, *dAs, *dBs)


def multi_lora_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                      lora_as: Sequence[torch.Tensor], lora_bs: Sequence[torch.Tensor],
                      scales: Sequence[float], routing: SegmentRouting) -> torch.Tensor:
    """Functional form over x of shape [..., K]; returns [..., N] bf16."""
    K = x.shape[-1]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        x2 = x2.to(torch.bfloat16)
        weight = weight.to(torch.bfloat16)
    if x2.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise RuntimeError("multi-LoRA linear computes in bfloat16: pass bf16 input and base weight, "
                           "or call it under torch.autocast('cuda', dtype=torch.bfloat16)")
    if not x2.is_cuda:
        raise RuntimeError("multi-LoRA linear runs on the ROCm device only (HIP kernels, no CPU path)")
    with torch.autocast("cuda", enabled=False):
        y = MultiLoRAFunction.apply(x2.contiguous(), weight, bias, routing, tuple(scales), *lora_as, *lora_bs)
    return y.reshape(*lead, weight.shape[0])
