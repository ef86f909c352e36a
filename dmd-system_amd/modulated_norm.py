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

Generalized here: any batch count and any width the kernel takes (a multiple of 8 up to
8192), where the reference accepts its registered B1/B3 layouts at one width (1536 for
Wan-1.3B, 5120 for Helios). ``fused_layernorm_modulation`` also takes a float32 hidden
state: the Wan block's residual stream, as the gated-residual GEMM epilogue writes it.

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
