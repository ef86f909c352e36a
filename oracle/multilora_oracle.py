"""CPU oracle of the batched multi-LoRA linear — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker / the timed CPU baseline.
The product path (``dmd-system_amd``) never imports it and has no CPU path.

It restates, in numpy, the reference's per-adapter LoRA linear
(sliortega295-ops/DMD-System):

  * training/low_rank.py:26-28   ``base(value) + scale * F.linear(F.linear(value, lora_a), lora_b)``
    applied to each role's rows — the roles are the segments here
    (training/dmd.py:301-353 calls each role module on its own batch);
  * its autograd backward (W frozen, low_rank.py:20):
    g_u = s·dY, dB = g_uᵀ·h, g_h = g_u·B, dA = g_hᵀ·X, dX = dY·W + g_h·A;
  * reference/livewan_wan21/wanstreamer/lora.py:22-27,65-74: a disabled
    adapter (``lora_enabled(model, False)``) is the base alone -> adapter id -1;
  * the rounding points of three reference variants, for comparison only:
      - autocast bf16 (low_rank.py:28 under training/single_device.py:88):
        every F.linear output rounded to bf16, then bf16 mul and bf16 add;
      - fp32 LoRA update (native/models.py:44-51):
        bf16(f32(base) + f32(update)·s);
      - LiveWan (wanstreamer/lora.py:27): base + bf16(update)·s in bf16.

How each function is pinned (tests/test_oracle.py): brute-force loops on
tiny inputs, central finite differences for the backward, torch.autograd as
an independent library routine, the reference's own construction fixture
(tests/test_training_construction.py:24-38: 4x4 linears filled with 0.25,
rank 2, alpha 2, B = 0 -> base only), invariants (segment permutation,
concatenation of per-role calls, linearity in the scale), and torch's bf16
conversion for ``bf16_round``.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np


# ------------------------------------------------------------------ bf16

def bf16_round(a) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32.

    Same rule as IEEE round-to-nearest-even on the top 16 bits; NaN stays NaN.
    """
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = (rounded & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    nan = np.isnan(f)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out)
    return out.reshape(f.shape)


# ------------------------------------------------------------------ e4m3 (OCP E4M3FN)
#
# The quantised-base variant stores the frozen W as OCP 8-bit E4M3 (bias 7,
# 3 mantissa bits, subnormals 2^-9 apart, max 448, 0x7F/0xFF NaN, no
# infinities; the format torch calls float8_e4m3fn) with one fp32 scale per
# output channel, and quantises activations per row. The reference has no
# such path (its base is bf16/fp32, low_rank.py:20); these functions define
# the variant's arithmetic. Pinned in tests/test_oracle.py against torch's
# float8_e4m3fn conversions (all 256 codes; random, tie and subnormal values)
# and against a brute-force nearest-representable search.

def e4m3_decode(q) -> np.ndarray:
    """float32 value of each e4m3 byte (NaN for 0x7F / 0xFF)."""
    q = np.asarray(q, dtype=np.uint8).astype(np.int64)
    sign = np.where(q & 0x80, -1.0, 1.0)
    e = (q >> 3) & 15
    m = q & 7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (sign * mag).astype(np.float32)
    return np.where((q & 0x7F) == 0x7F, np.float32(np.nan), out)


def e4m3_encode(a) -> np.ndarray:
    """Nearest e4m3 byte of float32 values (ties to even), saturating at ±448.

    Normal range (|a| >= 2^-6): round the fp32 mantissa to 3 bits; below it,
    round |a|·2^9 to an integer (the subnormal grid); |a| >= 464 (which rounds
    past 448) and NaN give 0x7E with the sign of a.
    """
    f = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    bits = f.view(np.uint32).astype(np.uint64)
    sign = (bits >> 24) & 0x80
    mag = np.abs(f)
    v = mag.view(np.uint32).astype(np.uint64)
    v = v + 0x7FFFF + ((v >> 20) & 1)
    normal = ((((v >> 23) - 120) << 3) | ((v >> 20) & 7)) & 0xFF
    with np.errstate(invalid="ignore"):
        sub = np.rint(mag * np.float32(512)).astype(np.float64)
        code = np.where(mag < np.float32(2.0 ** -6), np.nan_to_num(sub), normal)
        code = np.where(mag < np.float32(464), code, 0x7E)
    code = np.where(np.isnan(f), 0x7E, code)
    return (code.astype(np.uint64) | sign).astype(np.uint8).reshape(f.shape)


def quantize_rows_e4m3(x, col_scale=None):
    """Per-row absmax quantisation -> (q uint8 [M, K], scale float32 [M]).

    With col_scale, each column is first multiplied by its factor (one fp32
    product). scale = amax / 448 and q = e4m3(x · (448 / amax)), both quotients
    in fp32; an all-zero row gets scale 1 (and q = 0).
    """
    x = np.asarray(x, dtype=np.float32)
    if col_scale is not None:
        x = (x * np.asarray(col_scale, np.float32)[None, :]).astype(np.float32)
    amax = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    pos = amax > 0
    safe = np.where(pos, amax, np.float32(1)).astype(np.float32)
    inv = np.where(pos, np.float32(448) / safe, np.float32(1)).astype(np.float32)
    scale = np.where(pos, safe / np.float32(448), np.float32(1)).astype(np.float32)
    q = e4m3_encode((x * inv[:, None]).astype(np.float32))
    return q, scale


def dequant_rows_e4m3(q, scale) -> np.ndarray:
    """fp32 e4m3(q)·scale per row (before any bf16 rounding)."""
    return (e4m3_decode(q) * np.asarray(scale, np.float32)[:, None]).astype(np.float32)


def forward_fp8_base(x, wq, w_scale, b, As, Bs, scales, seg_offsets, adapter_ids) -> np.ndarray:
    """Reference semantics with the e4m3 base: forward() with W = w_scale[n]·e4m3(wq[n, k]), exact."""
    w = e4m3_decode(wq).astype(np.float64) * np.asarray(w_scale, np.float64)[:, None]
    return forward(x, w, b, As, Bs, scales, seg_offsets, adapter_ids)


def forward_fp8_quantized_x(x, wq, w_scale, b, As, Bs, scales, seg_offsets, adapter_ids) -> np.ndarray:
    """The e4m3 kernel's arithmetic, exactly: the base product uses X quantised
    per row (quantize_rows_e4m3), the LoRA term the unquantised X; fp64 sums
    (the kernel's e4m3 products are exact in fp32, only the summation order
    and the final bf16 rounding differ)."""
    x = np.asarray(x, np.float64)
    xq, xs = quantize_rows_e4m3(x.astype(np.float32))
    base = (e4m3_decode(xq).astype(np.float64) @ e4m3_decode(wq).astype(np.float64).T)
    base = base * xs.astype(np.float64)[:, None] * np.asarray(w_scale, np.float64)[None, :]
    if b is not None:
        base = base + np.asarray(b, np.float64)[None, :]
    lora = forward(x, np.zeros((base.shape[1], x.shape[1])), None, As, Bs, scales, seg_offsets, adapter_ids)
    return base + lora


def dx_fp8_quantized_dy(dy, wq, w_scale, As, Bs, scales, seg_offsets, adapter_ids) -> np.ndarray:
    """The e4m3 dX arithmetic, exactly: dX = dY·W + Σ_seg s·(dY·B_a)·A_a with
    W = w_scale[n]·e4m3(wq[n, k]), where the base product uses dY·w_scale
    quantised per row (quantize_rows_e4m3 with col_scale = w_scale) times e4m3(wq)
    and the row scale, and the LoRA term the unquantised dY; fp64 sums."""
    dy = np.asarray(dy, np.float64)
    dq, ds = quantize_rows_e4m3(dy.astype(np.float32), col_scale=w_scale)
    base = (e4m3_decode(dq).astype(np.float64) @ e4m3_decode(wq).astype(np.float64)) * ds.astype(np.float64)[:, None]
    lora = dx_rows(np.arange(dy.shape[0]), np.zeros((dy.shape[1], base.shape[1])), As, Bs, scales, seg_offsets,
                   adapter_ids, dy)
    return base + lora


# ------------------------------------------------------------------ routing

def row_adapters(seg_offsets: Sequence[int], adapter_ids: Sequence[int]) -> np.ndarray:
    """Adapter id of each row (int64), -1 for base-only rows."""
    off = [int(v) for v in seg_offsets]
    ids = [int(v) for v in adapter_ids]
    if len(off) != len(ids) + 1 or off[0] != 0 or any(b < a for a, b in zip(off, off[1:])):
        raise ValueError("oracle: malformed segment offsets")
    out = np.empty(off[-1], dtype=np.int64)
    for s, a in enumerate(ids):
        out[off[s]:off[s + 1]] = a
    return out


def _segments(seg_offsets, adapter_ids):
    for s, a in enumerate(adapter_ids):
        lo, hi = int(seg_offsets[s]), int(seg_offsets[s + 1])
        yield lo, hi, int(a)


# ------------------------------------------------------------------ exact path

def forward(x, w, b, As, Bs, scales, seg_offsets, adapter_ids, dtype=np.float64) -> np.ndarray:
    """Y for every segment, evaluated per segment like one reference module call each."""
    x = np.asarray(x, dtype)
    w = np.asarray(w, dtype)
    y = x @ w.T
    if b is not None:
        y = y + np.asarray(b, dtype)
    for lo, hi, a in _segments(seg_offsets, adapter_ids):
        if a < 0 or hi == lo:
            continue
        h = x[lo:hi] @ np.asarray(As[a], dtype).T
        y[lo:hi] += dtype(scales[a]) * (h @ np.asarray(Bs[a], dtype).T)
    return y


def backward(x, w, As, Bs, scales, seg_offsets, adapter_ids, dy, dtype=np.float64):
    """(dX, [dA_i], [dB_i]) of sum(Y * dY); W and bias are frozen."""
    x = np.asarray(x, dtype)
    w = np.asarray(w, dtype)
    dy = np.asarray(dy, dtype)
    dx = dy @ w
    dAs = [np.zeros(np.shape(A), dtype) for A in As]
    dBs = [np.zeros(np.shape(B), dtype) for B in Bs]
    for lo, hi, a in _segments(seg_offsets, adapter_ids):
        if a < 0 or hi == lo:
            continue
        A = np.asarray(As[a], dtype)
        B = np.asarray(Bs[a], dtype)
        s = dtype(scales[a])
        xs, gu = x[lo:hi], s * dy[lo:hi]
        h = xs @ A.T
        dBs[a] += gu.T @ h
        gh = gu @ B
        dAs[a] += gh.T @ xs
        dx[lo:hi] += gh @ A
    return dx, dAs, dBs


def forward_rows(rows, x, w, b, As, Bs, scales, seg_offsets, adapter_ids, dtype=np.float64) -> np.ndarray:
    """Y restricted to the given row indices (rows are independent in the forward)."""
    rows = np.asarray(rows, dtype=np.int64)
    ad = row_adapters(seg_offsets, adapter_ids)[rows]
    xr = np.asarray(x[rows], dtype)
    y = xr @ np.asarray(w, dtype).T
    if b is not None:
        y = y + np.asarray(b, dtype)
    for a in np.unique(ad):
        if a < 0:
            continue
        sel = ad == a
        h = xr[sel] @ np.asarray(As[a], dtype).T
        y[sel] += dtype(scales[a]) * (h @ np.asarray(Bs[a], dtype).T)
    return y


def dx_rows(rows, w, As, Bs, scales, seg_offsets, adapter_ids, dy, dtype=np.float64) -> np.ndarray:
    """dX restricted to the given rows (rows are independent in dX)."""
    rows = np.asarray(rows, dtype=np.int64)
    ad = row_adapters(seg_offsets, adapter_ids)[rows]
    dyr = np.asarray(dy[rows], dtype)
    dx = dyr @ np.asarray(w, dtype)
    for a in np.unique(ad):
        if a < 0:
            continue
        sel = ad == a
        gh = dtype(scales[a]) * (dyr[sel] @ np.asarray(Bs[a], dtype))
        dx[sel] += gh @ np.asarray(As[a], dtype)
    return dx


# ------------------------------------------------------------------ reference rounding variants

def _mm_f32(a, b_t):
    """fp32-accumulated product a @ b_tᵀ of float32 operands."""
    return np.asarray(a, np.float32) @ np.asarray(b_t, np.float32).T


def forward_autocast_bf16(x, w, b, As, Bs, scales, seg_offsets, adapter_ids) -> np.ndarray:
    """low_rank.py:28 under bf16 autocast: operands and every op result rounded to bf16."""
    xq, wq = bf16_round(x), bf16_round(w)
    base = _mm_f32(xq, wq)
    if b is not None:
        base = base + bf16_round(b)
    base = bf16_round(base)
    y = base.copy()
    for lo, hi, a in _segments(seg_offsets, adapter_ids):
        if a < 0 or hi == lo:
            continue
        h = bf16_round(_mm_f32(xq[lo:hi], bf16_round(As[a])))
        u = bf16_round(_mm_f32(h, bf16_round(Bs[a])))
        su = bf16_round(np.float32(scales[a]) * u)
        y[lo:hi] = bf16_round(base[lo:hi] + su)
    return y


def forward_fp32_update(x, w, b, As, Bs, scales, seg_offsets, adapter_ids) -> np.ndarray:
    """native/models.py:44-51: bf16 base, fp32 update, (base.float() + update*s).to(bf16)."""
    xq, wq = bf16_round(x), bf16_round(w)
    base = _mm_f32(xq, wq)
    if b is not None:
        base = base + bf16_round(b)
    base = bf16_round(base)
    y = base.copy()
    x32 = np.asarray(xq, np.float32)
    for lo, hi, a in _segments(seg_offsets, adapter_ids):
        if a < 0 or hi == lo:
            continue
        upd = _mm_f32(_mm_f32(x32[lo:hi], As[a]), Bs[a])
        y[lo:hi] = bf16_round(base[lo:hi] + (upd * np.float32(scales[a])).astype(np.float32))
    return y


def forward_livewan(x, w, b, As, Bs, scales, seg_offsets, adapter_ids) -> np.ndarray:
    """wanstreamer/lora.py:22-27: y + linear(linear(x.f32, a), b).to(bf16) * scale, in bf16."""
    xq, wq = bf16_round(x), bf16_round(w)
    base = _mm_f32(xq, wq)
    if b is not None:
        base = base + bf16_round(b)
    base = bf16_round(base)
    y = base.copy()
    for lo, hi, a in _segments(seg_offsets, adapter_ids):
        if a < 0 or hi == lo:
            continue
        upd = bf16_round(_mm_f32(_mm_f32(xq[lo:hi], As[a]), Bs[a]))
        y[lo:hi] = bf16_round(base[lo:hi] + bf16_round(upd * np.float32(scales[a])))
    return y


# ------------------------------------------------------------------ metrics

def gated_residual(x, y, gate, gate_rows: int) -> np.ndarray:
    """The DiT block's residual update x' = x + y·gate with the rounding contract of
    runtime/helios_residual_kernel.py:66-86 (the Wan block: model.py:305-313):
    bf16( RN_f32( f32(x) + RN_f32( f32(y) · gate[m // gate_rows] ) ) ) — a float32
    multiply, then a float32 add (numpy rounds each operation; no fused multiply-add),
    then bf16 round-to-nearest-even. x, y: bf16 values [M, N]; gate: float32 [G, N]."""
    x = np.asarray(x, dtype=np.float32)
    y = np.asarray(y, dtype=np.float32)
    g = np.repeat(np.asarray(gate, dtype=np.float32), gate_rows, axis=0)[: x.shape[0]]
    p = np.multiply(y, g, dtype=np.float32)
    return bf16_round(np.add(x, p, dtype=np.float32))


def gated_residual_f32(x, y, gate, gate_rows: int) -> np.ndarray:
    """The Wan block's float32 residual stream (reference/livewan_wan21/wan/modules/model.py:
    305-306,312-313: ``x = x + y * e[2]`` under float32 autocast, x and e float32, y bf16):
    RN_f32( x + RN_f32( f32(y) · gate[m // gate_rows] ) ) — two float32 operations, no final
    rounding. x: float32 [M, N]; y: bf16 values; gate: float32 [G, N]."""
    x = np.asarray(x, dtype=np.float32)
    y = np.asarray(y, dtype=np.float32)
    g = np.repeat(np.asarray(gate, dtype=np.float32), gate_rows, axis=0)[: x.shape[0]]
    return np.add(x, np.multiply(y, g, dtype=np.float32), dtype=np.float32)


def gate_scale(dout, gate, gate_rows: int) -> np.ndarray:
    """Frozen-gate backward of gated_residual / gated_residual_f32 (helios_residual_kernel.py:90-133):
    dY = bf16(RN_f32(f32(dOut) · gate[m // gate_rows])); dX = dOut (dOut bf16 or float32)."""
    d = np.asarray(dout, dtype=np.float32)
    g = np.repeat(np.asarray(gate, dtype=np.float32), gate_rows, axis=0)[: d.shape[0]]
    return bf16_round(np.multiply(d, g, dtype=np.float32))


# ------------------------------------------------------------------ modulated LayerNorm

def layer_norm(x, eps: float) -> np.ndarray:
    """Affine-free LayerNorm over the last axis (mean, biased variance), evaluated in float64
    and rounded once to float32: the normalized values the reference's fused kernel computes in
    float32 (runtime/wan13b_fused_layernorm_kernel.py:55-60: mean = Σx / W,
    var = Σ(x - mean)² / W, (x - mean)·rsqrt(var + eps)), without their rounding."""
    x = np.asarray(x, dtype=np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    c = x - mean
    var = (c * c).mean(axis=-1, keepdims=True)
    return (c / np.sqrt(var + eps)).astype(np.float32)


def modulated_norm(v, scale, shift, scale_row=None, shift_row=None) -> np.ndarray:
    """bf16( RN(RN(v · RN(1 + s)) + h) ): runtime/wan13b_modulated_norm_kernel.py:70-97
    (add.rn 1 + scale, mul.rn, add.rn shift, BF16 store). With table rows
    (the materialization form, :158-174) s = RN(scale_row + scale), h = RN(shift_row + shift).
    Inputs are float32 values (bf16 components converted exactly); numpy rounds each
    float32 operation and never fuses a multiply-add."""
    v = np.asarray(v, dtype=np.float32)
    s = np.asarray(scale, dtype=np.float32)
    h = np.asarray(shift, dtype=np.float32)
    if scale_row is not None:
        s = np.add(np.asarray(scale_row, dtype=np.float32), s, dtype=np.float32)
        h = np.add(np.asarray(shift_row, dtype=np.float32), h, dtype=np.float32)
    ops = np.add(np.float32(1.0), s, dtype=np.float32)
    p = np.multiply(v, ops, dtype=np.float32)
    return bf16_round(np.add(p, h, dtype=np.float32))


def modulated_norm_backward(x, g, scale, eps: float, scale_row=None):
    """Closed-form gradients of out = LN(x)·(1 + s) + h (s = scale_row + scale) for the upstream
    gradient g, in float64 — what the reference's fused backward evaluates in float32
    (runtime/wan13b_fused_layernorm_backward_kernel.py:27-270):
      n = (x - mean)·rstd, gn = g·(1 + s),
      dx = (gn - mean_f(gn) - n·mean_f(gn·n))·rstd,   d_scale = g·n,   d_shift = g
    (per element; the reduced component gradient sums d_scale and d_shift over tokens).
    Returns (dx, d_scale, d_shift, mean, rstd)."""
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    s = np.asarray(scale, dtype=np.float64)
    if scale_row is not None:
        s = np.asarray(scale_row, dtype=np.float64) + s
    mean = x.mean(axis=-1, keepdims=True)
    c = x - mean
    rstd = 1.0 / np.sqrt((c * c).mean(axis=-1, keepdims=True) + eps)
    n = c * rstd
    gn = g * (1.0 + s)
    dx = (gn - gn.mean(axis=-1, keepdims=True) - n * (gn * n).mean(axis=-1, keepdims=True)) * rstd
    return dx, g * n, g, mean[..., 0], rstd[..., 0]


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    den = np.linalg.norm(want.ravel())
    num = np.linalg.norm((got - want).ravel())
    return float(num / den) if den > 0 else float(num)
