"""Modulated LayerNorm of a DiT block on the HIP kernel (``mlora_modulated_norm``).

The reference's three forward entry points, with the same names, argument meaning and
error type (RuntimeError on any contract violation):

* ``fused_modulated_norm_epilogue(normalized, scale, shift, output)``:
  ``output = bf16(RN(RN(normalized · RN(1 + scale)) + shift))`` after PyTorch's fp32
  LayerNorm (runtime/wan13b_modulated_norm_kernel.py:207-263, kernel :26-97).
* ``fused_modulated_norm_materialization(normalized, scale_shift_table, scale_index,
  shift_index, scale_component, shift_component, output)``: the same, with
  ``scale = RN(table[0, scale_index] + scale_component)`` and ``shift`` alike
  (:266-353, kernel :100-204).
* ``fused_bf16_layernorm_modulation(hidden, ..., output, *, eps)``: the affine-free
  LayerNorm of the bf16 hidden state fused in front
  (runtime/wan13b_fused_layernorm_kernel.py:135-222, kernel :22-132).

and the reference's fused backward (runtime/wan13b_fused_layernorm_backward_kernel.py):

* ``fused_bf16_layernorm_modulation_hidden_backward(hidden, grad_output, scale_shift_table,
  scale_index, scale_component, hidden_gradient, mean, rstd, *, eps)`` (:337-393);
* ``fused_reduced_component_gradient(hidden, grad_output, mean, rstd, component_gradient,
  scale_index, shift_index)`` into [B, 6, W] (:396-447);
* ``fused_tensor4d_component_gradient(...)`` into [B, T, 6, W] (:450-502).

``ModulatedLayerNormFunction`` / ``modulated_layer_norm`` put the fused forward and these
backward kernels into one autograd op, with the gradients of the hidden state, the table and
the components.

Generalized here: any batch count and any width the kernel takes (a multiple of 8 up to
8192; 5120 for the backward), where the reference accepts its registered B1/B3 layouts at one
width (1536 for Wan-1.3B, 5120 for Helios). The ``fused_layernorm_modulation*`` forms also
take a float32 hidden state and gradient: the Wan block's residual stream, as the
gated-residual GEMM epilogue writes it.

The elementwise steps are bit-exact given the same normalized values. The fused
LayerNorm sums in its own fixed order, so it agrees with another LayerNorm to fp32
rounding (rarely one bf16 ulp in the output).
"""
from __future__ import annotations

import torch

from . import kernels

_TABLE_DTYPES = (torch.bfloat16, torch.float32)


def _fail(message: str) -> None:
    raise RuntimeError("modulated norm: " + message)


def _check_common(lead: torch.Tensor, output: torch.Tensor, others) -> None:
    for name, t in (("input", lead), ("output", output), *others):
        if not t.is_cuda:
            _fail(f"{name} must be a ROCm device tensor")
        if t.dim() != 3:
            _fail(f"{name} must be [batch, tokens, width], got {tuple(t.shape)}")
        if any(st < 0 for st in t.stride()):
            _fail(f"{name} has a negative stride")
    if output.dtype is not torch.bfloat16:
        _fail("output must be bfloat16")
    if output.shape != lead.shape:
        _fail(f"output shape {tuple(output.shape)} != input shape {tuple(lead.shape)}")


def _table_rows(table: torch.Tensor, scale_index: int, shift_index: int, width: int):
    if not table.is_cuda or table.dtype not in _TABLE_DTYPES:
        _fail("scale-shift table must be a bfloat16 or float32 device tensor")
    if table.dim() != 3 or tuple(table.shape[:2]) != (1, 6) or table.shape[2] != width:
        _fail(f"scale-shift table must be [1, 6, {width}], got {tuple(table.shape)}")
    if table.stride(2) != 1:
        _fail("scale-shift table must have unit feature stride")
    si, hi = int(scale_index), int(shift_index)
    if not (0 <= si < 6 and 0 <= hi < 6):
        _fail(f"component indices must be in [0, 6), got {si}, {hi}")
    return table[0, si], table[0, hi]


def _check_components(lead: torch.Tensor, scale_component: torch.Tensor, shift_component: torch.Tensor) -> None:
    for name, t in (("scale_component", scale_component), ("shift_component", shift_component)):
        if t.dtype not in _TABLE_DTYPES:
            _fail(f"{name} must be bfloat16 or float32")
        if t.shape != lead.shape:
            _fail(f"{name} shape {tuple(t.shape)} != {tuple(lead.shape)}")


def fused_modulated_norm_epilogue(normalized: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                                  output: torch.Tensor) -> torch.Tensor:
    """output = bf16(RN(RN(normalized · RN(1 + scale)) + shift)), all float32 inputs."""
    _check_common(normalized, output, (("scale", scale), ("shift", shift)))
    for name, t in (("normalized", normalized), ("scale", scale), ("shift", shift)):
        if t.dtype is not torch.float32:
            _fail(f"{name} must be float32")
        if t.shape != normalized.shape:
            _fail(f"{name} shape {tuple(t.shape)} != {tuple(normalized.shape)}")
    if output.numel() == 0:
        return output
    return kernels.modulated_norm(normalized, scale, shift, output)


def fused_modulated_norm_materialization(normalized: torch.Tensor, scale_shift_table: torch.Tensor,
                                         scale_index: int, shift_index: int, scale_component: torch.Tensor,
                                         shift_component: torch.Tensor, output: torch.Tensor) -> torch.Tensor:
    """The epilogue with scale = RN(table[0, scale_index] + scale_component) and
    shift = RN(table[0, shift_index] + shift_component)."""
    _check_common(normalized, output, (("scale_component", scale_component), ("shift_component", shift_component)))
    if normalized.dtype is not torch.float32:
        _fail("normalized must be float32")
    _check_components(normalized, scale_component, shift_component)
    srow, hrow = _table_rows(scale_shift_table, scale_index, shift_index, normalized.shape[2])
    if output.numel() == 0:
        return output
    return kernels.modulated_norm(normalized, scale_component, shift_component, output,
                                  scale_row=srow, shift_row=hrow)


def fused_layernorm_modulation(hidden: torch.Tensor, scale_shift_table: torch.Tensor, scale_index: int,
                               shift_index: int, scale_component: torch.Tensor, shift_component: torch.Tensor,
                               output: torch.Tensor, *, eps: float) -> torch.Tensor:
    """Affine-free LayerNorm of each row of `hidden` (bf16 or float32), then the
    materialized modulation, written to the bf16 output in one pass."""
    _check_common(hidden, output, (("scale_component", scale_component), ("shift_component", shift_component)))
    if hidden.dtype not in (torch.bfloat16, torch.float32):
        _fail("hidden must be bfloat16 or float32")
    if not float(eps) > 0:
        _fail("LayerNorm epsilon must be positive")
    _check_components(hidden, scale_component, shift_component)
    srow, hrow = _table_rows(scale_shift_table, scale_index, shift_index, hidden.shape[2])
    if output.numel() == 0:
        return output
    return kernels.modulated_norm(hidden, scale_component, shift_component, output, eps=float(eps),
                                  scale_row=srow, shift_row=hrow)


def fused_bf16_layernorm_modulation(hidden: torch.Tensor, scale_shift_table: torch.Tensor, scale_index: int,
                                    shift_index: int, scale_component: torch.Tensor,
                                    shift_component: torch.Tensor, output: torch.Tensor, *,
                                    eps: float) -> torch.Tensor:
    """fused_layernorm_modulation for the reference's bf16 hidden state."""
    if hidden.dtype is not torch.bfloat16:
        _fail("hidden must be bfloat16")
    return fused_layernorm_modulation(hidden, scale_shift_table, scale_index, shift_index, scale_component,
                                      shift_component, output, eps=eps)


def _check_stats(lead: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor) -> None:
    for name, t in (("mean", mean), ("rstd", rstd)):
        if not t.is_cuda or t.dtype is not torch.float32:
            _fail(f"row statistic {name} must be a float32 device tensor")
        if tuple(t.shape) != tuple(lead.shape[:2]) or not t.is_contiguous():
            _fail(f"row statistic {name} must be contiguous [{lead.shape[0]}, {lead.shape[1]}]")


def fused_layernorm_modulation_hidden_backward(hidden: torch.Tensor, grad_output: torch.Tensor,
                                               scale_shift_table: torch.Tensor, scale_index: int,
                                               scale_component: torch.Tensor, hidden_gradient: torch.Tensor,
                                               mean: torch.Tensor, rstd: torch.Tensor, *, eps: float) -> torch.Tensor:
    """Gradient of fused_layernorm_modulation's output with respect to `hidden` (bf16 or
    float32, as are grad_output and hidden_gradient), plus the rows' mean and rstd."""
    for name, t in (("hidden", hidden), ("grad_output", grad_output), ("hidden_gradient", hidden_gradient)):
        if not t.is_cuda or t.dim() != 3:
            _fail(f"{name} must be a [batch, tokens, width] device tensor")
        if t.dtype not in (torch.bfloat16, torch.float32):
            _fail(f"{name} must be bfloat16 or float32")
        if t.shape != hidden.shape:
            _fail(f"{name} shape {tuple(t.shape)} != {tuple(hidden.shape)}")
    if scale_component.dtype not in _TABLE_DTYPES or scale_component.shape != hidden.shape:
        _fail("scale_component must be bfloat16 or float32 with the hidden state's shape")
    if not float(eps) > 0:
        _fail("LayerNorm epsilon must be positive")
    srow, _ = _table_rows(scale_shift_table, scale_index, 0, hidden.shape[2])
    _check_stats(hidden, mean, rstd)
    if hidden.numel() == 0:
        return hidden_gradient
    return kernels.modulated_norm_backward(hidden, grad_output, scale_component, hidden_gradient, mean, rstd,
                                           eps=float(eps), scale_row=srow)


def fused_bf16_layernorm_modulation_hidden_backward(hidden: torch.Tensor, grad_output: torch.Tensor,
                                                    scale_shift_table: torch.Tensor, scale_index: int,
                                                    scale_component: torch.Tensor, hidden_gradient: torch.Tensor,
                                                    mean: torch.Tensor, rstd: torch.Tensor, *,
                                                    eps: float) -> torch.Tensor:
    """The hidden backward for the reference's bf16 hidden state, upstream gradient and output."""
    for name, t in (("hidden", hidden), ("grad_output", grad_output), ("hidden_gradient", hidden_gradient)):
        if t.dtype is not torch.bfloat16:
            _fail(f"{name} must be bfloat16")
    return fused_layernorm_modulation_hidden_backward(hidden, grad_output, scale_shift_table, scale_index,
                                                      scale_component, hidden_gradient, mean, rstd, eps=eps)


def _component_gradient(hidden, grad_output, mean, rstd, component_gradient, scale_index, shift_index, rank):
    if not component_gradient.is_cuda or component_gradient.dtype not in _TABLE_DTYPES:
        _fail("component gradient must be a bfloat16 or float32 device tensor")
    B, T, W = hidden.shape
    want = (B, 6, W) if rank == 3 else (B, T, 6, W)
    if tuple(component_gradient.shape) != want:
        _fail(f"component gradient must be {list(want)}, got {tuple(component_gradient.shape)}")
    si, hi = int(scale_index), int(shift_index)
    if not (0 <= si < 6 and 0 <= hi < 6) or si == hi:
        _fail(f"component indices must be two different values in [0, 6), got {si}, {hi}")
    if hidden.dtype not in _TABLE_DTYPES or grad_output.dtype not in _TABLE_DTYPES:
        _fail("hidden and grad_output must be bfloat16 or float32")
    if grad_output.shape != hidden.shape:
        _fail("grad_output shape differs from the hidden state's")
    _check_stats(hidden, mean, rstd)
    if B == 0 or T == 0:  # nothing to sum: the buffer is returned untouched (as the reference does
        return component_gradient  # for an empty token interval, so earlier intervals' sums survive)
    return kernels.modulated_norm_component_grad(hidden, grad_output, mean, rstd, component_gradient, si, hi)


def fused_reduced_component_gradient(hidden: torch.Tensor, grad_output: torch.Tensor, mean: torch.Tensor,
                                     rstd: torch.Tensor, component_gradient: torch.Tensor, scale_index: int,
                                     shift_index: int) -> torch.Tensor:
    """component_gradient[b, scale_index] = Σ_t grad_output·n, [b, shift_index] = Σ_t grad_output
    ([B, 6, W]; n = (hidden - mean)·rstd; summed in a fixed order)."""
    return _component_gradient(hidden, grad_output, mean, rstd, component_gradient, scale_index, shift_index, 3)


def fused_tensor4d_component_gradient(hidden: torch.Tensor, grad_output: torch.Tensor, mean: torch.Tensor,
                                      rstd: torch.Tensor, component_gradient: torch.Tensor, scale_index: int,
                                      shift_index: int) -> torch.Tensor:
    """component_gradient[b, t, scale_index] = grad_output·n, [b, t, shift_index] = grad_output
    ([B, T, 6, W])."""
    return _component_gradient(hidden, grad_output, mean, rstd, component_gradient, scale_index, shift_index, 4)


class ModulatedLayerNormFunction(torch.autograd.Function):
    """``apply(hidden, table, component, scale_index, shift_index, eps)`` ->
    bf16(LN(hidden)·RN(1 + RN(table[0, si] + c_si)) + RN(table[0, hi] + c_hi)).

    hidden [B, T, W] bf16 or float32; table [1, 6, W]; component [B, 6, W] (one modulation per
    sample, Wan's time embedding) or [B, T, 6, W] (per token). Gradients: hidden (its dtype),
    table and component (float32 sums, in their dtypes), from the fused backward kernels."""

    @staticmethod
    def forward(ctx, hidden, table, component, scale_index: int, shift_index: int, eps: float):
        if hidden.dim() != 3:
            _fail(f"hidden must be [batch, tokens, width], got {tuple(hidden.shape)}")
        if int(scale_index) == int(shift_index):
            _fail("scale and shift must be two different components")
        B, T, W = hidden.shape
        if component.dim() == 3:
            scale_c = component[:, scale_index].unsqueeze(1).expand(B, T, W)
            shift_c = component[:, shift_index].unsqueeze(1).expand(B, T, W)
        elif component.dim() == 4:
            scale_c, shift_c = component[:, :, scale_index], component[:, :, shift_index]
        else:
            _fail("component must be [B, 6, W] or [B, T, 6, W]")
        out = torch.empty(B, T, W, dtype=torch.bfloat16, device=hidden.device)
        fused_layernorm_modulation(hidden, table, scale_index, shift_index, scale_c, shift_c, out, eps=eps)
        ctx.save_for_backward(hidden, table, component)
        ctx.idx, ctx.eps = (int(scale_index), int(shift_index)), float(eps)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        hidden, table, component = ctx.saved_tensors
        si, hi = ctx.idx
        B, T, W = hidden.shape
        g = grad_out.contiguous()
        scale_c = (component[:, si].unsqueeze(1).expand(B, T, W) if component.dim() == 3
                   else component[:, :, si])
        dx = torch.empty_like(hidden)
        mean = torch.empty(B, T, dtype=torch.float32, device=hidden.device)
        rstd = torch.empty_like(mean)
        fused_layernorm_modulation_hidden_backward(hidden, g, table, si, scale_c, dx, mean, rstd, eps=ctx.eps)
        d_table = d_comp = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dc = torch.zeros(component.shape, dtype=torch.float32, device=hidden.device)
            if component.dim() == 3:
                fused_reduced_component_gradient(hidden, g, mean, rstd, dc, si, hi)
                dt = dc.sum(dim=0, keepdim=True)
            else:
                fused_tensor4d_component_gradient(hidden, g, mean, rstd, dc, si, hi)
                dt = dc.sum(dim=(0, 1)).unsqueeze(0)
            if ctx.needs_input_grad[1]:
                d_table = dt.to(table.dtype)
            if ctx.needs_input_grad[2]:
                d_comp = dc.to(component.dtype)
        return dx, d_table, d_comp, None, None, None


def modulated_layer_norm(hidden: torch.Tensor, table: torch.Tensor, component: torch.Tensor, scale_index: int,
                         shift_index: int, eps: float = 1e-6) -> torch.Tensor:
    """The Wan block's ``norm(x).float() * (1 + e[si]) + e[hi]`` with ``e = modulation + e_time``
    (wan/modules/model.py:298-311), cast to bf16 for the next linear, as one autograd op."""
    return ModulatedLayerNormFunction.apply(hidden, table, component, scale_index, shift_index, eps)
