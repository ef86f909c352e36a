"""Torch-tensor front end of the C ABI: checks, output allocation, streams.

Every function here launches HIP kernels from ``libmlora.so`` on the current
stream of the tensors' device. There is no CPU path: non-ROCm tensors or a
missing library raise.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib
from .routing import SegmentRouting

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError("multi-LoRA kernel contract: " + message)


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_rows(name: str, t: torch.Tensor, cols: int | None = None) -> None:
    _require(t.is_cuda, f"{name} must be a ROCm device tensor")
    _require(t.dtype == torch.bfloat16, f"{name} must be bfloat16, got {t.dtype}")
    _require(t.dim() == 2 and t.stride(1) == 1, f"{name} must be a 2-D row-major matrix")
    if cols is not None:
        _require(t.shape[1] == cols, f"{name} has {t.shape[1]} columns, expected {cols}")


def _routing_arrays(off, ids):
    return _lib.i64_array(off), _lib.i32_array(ids), len(ids)


def padded_rank(ranks: Sequence[int]) -> int:
    r = max([0, *ranks])
    return (r + 7) // 8 * 8


def frag_jtiles(width: int) -> int:
    """j-tiles (16 ranks each) of the hi/lo fragment layout for row width `width`."""
    return (width + 15) // 16


_FRAG_TILE_BYTES = 2 * 64 * 16  # one j-tile (hi + lo) of one 32-row block in the fragment layout


def alloc_frags(routing: SegmentRouting, jtiles: int, device) -> list:
    """Empty hi/lo fragment buffers (one per call group of `routing`) of `jtiles` j-tiles."""
    lib = _lib.load()
    out = []
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        o, i, n = _routing_arrays(off, ids)
        nbytes = lib.mlora_frag_bytes(r1 - r0, jtiles, o, i, n)
        _lib.check("mlora_frag_bytes", nbytes if nbytes < 0 else 0)
        out.append(torch.empty(max(nbytes, 16) // 2, dtype=torch.bfloat16, device=device))
    return out


def shrink(p: torch.Tensor, ops: Sequence[torch.Tensor], op_layout: int, scales: Sequence[float],
           routing: SegmentRouting, want_frag: bool, width: int,
           row_div: torch.Tensor | None = None, h_out: torch.Tensor | None = None,
           frag_out: list | None = None, frag_jt: int | None = None,
           frag_t0: int = 0, ops_lo: Sequence[torch.Tensor] | None = None) -> tuple[torch.Tensor, list | None]:
    """h = s·P·Op_aᵀ per segment -> (h_rows bf16 [M, width], per-call-group hi/lo fragments or None).

    row_div [M] fp32 (optional) divides the rows of h_rows only (the row scales of the e4m3 forward's X
    and of the e4m3 dX's dY).

    ops_lo (optional): the lo parts of fp32 adapter operands split as ops = bf16(v), ops_lo =
    bf16(v - ops) (split_hi_lo); h then uses both (~16 significant bits of v).

    Writing into a part of larger buffers (the stacked LoRA operands of linears that share
    an input): h_out is a row-major view [M, >= r] whose row stride is the buffer's (rows
    get their r_a values at its first columns), frag_out fragment buffers of `frag_jt`
    j-tiles per block (alloc_frags) that receive h's j-tiles at j-tile `frag_t0` on.
    """
    M, K = p.shape
    _check_rows("P", p)
    ranks = [int(o.shape[0] if op_layout == 0 else o.shape[1]) for o in ops]
    for o, r in zip(ops, ranks):
        _check_rows("adapter operand", o)
        _require(o.is_contiguous(), "adapter operands must be contiguous")
        _require(o.shape == ((r, K) if op_layout == 0 else (K, r)), "adapter operand shape")
    if ops_lo is not None:
        _require(len(ops_lo) == len(ops), "one lo part per adapter operand")
        for o, lo in zip(ops, ops_lo):
            _check_rows("adapter operand lo part", lo)
            _require(lo.is_contiguous() and lo.shape == o.shape, "lo part has its hi part's shape")
    if row_div is not None:
        _check_scale("row_div", row_div, M)
    if h_out is not None:
        _check_rows("h_out", h_out)
        _require(h_out.shape[0] == M and h_out.shape[1] >= max([0, *ranks]), "h_out is [M, >= max rank]")
    h_rows = h_out if h_out is not None else torch.empty((M, width), dtype=torch.bfloat16, device=p.device)
    lib = _lib.load()
    ptrs, rk, sc = _lib.ptr_array([_ptr(o) for o in ops]), _lib.i32_array(ranks), _lib.f32_array(scales)
    lo_ptrs = None if ops_lo is None else _lib.ptr_array([_ptr(o) for o in ops_lo])
    jt = frag_jtiles(width) if frag_jt is None else frag_jt
    _require(0 <= frag_t0 and frag_t0 * 16 + max([0, *ranks]) <= jt * 16, "fragment j-tiles out of range")
    stream = _stream(p)
    frags = None
    if want_frag:
        frags = frag_out if frag_out is not None else alloc_frags(routing, jt, p.device)
        _require(len(frags) == len(list(routing.groups(_lib.MAX_SEGMENTS))), "one fragment buffer per call group")
    for g, (r0, r1, off, ids) in enumerate(routing.groups(_lib.MAX_SEGMENTS)):
        o, i, n = _routing_arrays(off, ids)
        fptr = None if frags is None else frags[g].data_ptr() + frag_t0 * _FRAG_TILE_BYTES
        if r1 == r0:
            continue
        _lib.check("mlora_shrink", lib.mlora_shrink(
            p[r0:r1].data_ptr(), p.stride(0), r1 - r0, K, ptrs, lo_ptrs, op_layout, rk, sc, len(ops),
            o, i, n, h_rows[r0:r1].data_ptr(), h_rows.stride(0), fptr, jt,
            None if row_div is None else row_div[r0:r1].data_ptr(), stream))
    return h_rows, frags


def gemm_fwd(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, h_rows: torch.Tensor | None,
             bs: Sequence[torch.Tensor], routing: SegmentRouting, out: torch.Tensor | None = None,
             accumulate: bool = False) -> torch.Tensor:
    """Y = X·Wᵀ + bias + per-segment h_rows·B_aᵀ, bf16 out. h_rows may be a column slice of a
    wider buffer (its row stride is passed)."""
    M, K = x.shape
    N = w.shape[0]
    _check_rows("X", x, K)
    _check_rows("W", w, K)
    if bias is not None:
        _require(bias.is_cuda and bias.dtype in _DT and bias.is_contiguous() and bias.shape == (N,), "bias")
    ranks = [int(b.shape[1]) for b in bs]
    for b in bs:
        _check_rows("lora_b", b)
        _require(b.is_contiguous() and b.shape[0] == N, "lora_b must be contiguous [N, r]")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _check_rows("Y", y, N)
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(b) for b in bs]), _lib.i32_array(ranks)
    ldh = h_rows.stride(0) if h_rows is not None else 0
    stream = _stream(x)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        hr = None if h_rows is None else h_rows[r0:r1].data_ptr()
        _lib.check("mlora_gemm_fwd", lib.mlora_gemm_fwd(
            x[r0:r1].data_ptr(), x.stride(0), r1 - r0, K, w.data_ptr(), w.stride(0), N,
            _ptr(bias), _DT[bias.dtype] if bias is not None else 0, hr, ldh,
            ptrs, rk, len(bs), o, i, n, y[r0:r1].data_ptr(), y.stride(0), int(accumulate), stream))
    return y


def gemm_fwd_stacked(x: torch.Tensor, w_cat: torch.Tensor, bias_cat: torch.Tensor | None, h_rows: torch.Tensor | None,
                     bs_cat: Sequence[torch.Tensor], routing: SegmentRouting, group_cols: int,
                     group_ecols: int) -> list[torch.Tensor]:
    """G linears that read x as one GEMM: w_cat [G·N, K] (their weights stacked by rows), bias_cat
    [G·N] or None, bs_cat[a] = [B_0,a; ...; B_{G-1},a] ([G·N, r_a]); linear g's LoRA rows are h_rows
    columns [g·group_ecols, g·group_ecols + r_a). Returns the G outputs [M, N] (each its own tensor)."""
    M, K = x.shape
    NT = w_cat.shape[0]
    G = NT // group_cols
    _check_rows("X", x, K)
    _check_rows("W", w_cat, K)
    if bias_cat is not None:
        _require(bias_cat.is_cuda and bias_cat.dtype in _DT and bias_cat.is_contiguous() and bias_cat.shape == (NT,),
                 "bias")
    ranks = [int(b.shape[1]) for b in bs_cat]
    for b in bs_cat:
        _check_rows("lora_b", b)
        _require(b.is_contiguous() and b.shape[0] == NT, "stacked lora_b must be contiguous [G·N, r]")
    ys = [torch.empty((M, group_cols), dtype=torch.bfloat16, device=x.device) for _ in range(G)]
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(b) for b in bs_cat]), _lib.i32_array(ranks)
    ldh = h_rows.stride(0) if h_rows is not None else 0
    stream = _stream(x)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        hr = None if h_rows is None else h_rows[r0:r1].data_ptr()
        _lib.check("mlora_gemm_fwd_stacked", lib.mlora_gemm_fwd_stacked(
            x[r0:r1].data_ptr(), x.stride(0), r1 - r0, K, w_cat.data_ptr(), w_cat.stride(0), NT, group_cols,
            _ptr(bias_cat), _DT[bias_cat.dtype] if bias_cat is not None else 0, hr, ldh, group_ecols,
            ptrs, rk, len(bs_cat), o, i, n, _lib.ptr_array([y[r0:r1].data_ptr() for y in ys]), group_cols, stream))
    return ys


def gemm_dx_stacked(dys: Sequence[torch.Tensor], w_cat_t: torch.Tensor, g_rows: torch.Tensor | None,
                    a_t_cat: Sequence[torch.Tensor], routing: SegmentRouting) -> torch.Tensor:
    """dX of G stacked linears as one GEMM: Σ_g dY_g·W_g + g_rows·A_cat,a, with w_cat_t = the stacked
    weights transposed [K, G·N], dys the G gradients [M, N] (contiguous), a_t_cat[a] = the stacked
    [A_0,a; ...] transposed ([K, G·R]) and g_rows [M, G·R]."""
    G = len(dys)
    M, N = dys[0].shape
    K = w_cat_t.shape[0]
    for d in dys:
        _check_rows("dY", d, N)
        _require(d.shape[0] == M and d.stride(0) == dys[0].stride(0), "the dY of the stacked linears share a shape")
    _check_rows("W_cat^T", w_cat_t, G * N)
    ranks = [int(a.shape[1]) for a in a_t_cat]
    for a in a_t_cat:
        _check_rows("stacked lora_a^T", a)
        _require(a.is_contiguous() and a.shape[0] == K, "stacked lora_a^T must be contiguous [K, G·R]")
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dys[0].device)
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(a) for a in a_t_cat]), _lib.i32_array(ranks)
    ldg = g_rows.stride(0) if g_rows is not None else 0
    stream = _stream(dys[0])
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        _lib.check("mlora_gemm_dx_stacked", lib.mlora_gemm_dx_stacked(
            _lib.ptr_array([d[r0:r1].data_ptr() for d in dys]), dys[0].stride(0), r1 - r0, N, G,
            w_cat_t.data_ptr(), w_cat_t.stride(0), K, None if g_rows is None else g_rows[r0:r1].data_ptr(), ldg,
            ptrs, rk, len(a_t_cat), o, i, n, dx[r0:r1].data_ptr(), dx.stride(0), stream))
    return dx


def _gate_rows(gate: torch.Tensor, M: int, N: int) -> int:
    """Rows of Y per gate row for a gate [G, N] (fp32, row pitch a multiple of 4) over M rows."""
    _require(gate.is_cuda and gate.dtype == torch.float32 and gate.dim() == 2 and gate.shape[1] == N
             and gate.stride(1) == 1 and gate.stride(0) % 4 == 0 and gate.data_ptr() % 16 == 0,
             "gate must be a float32 [G, N] matrix with 16-byte rows")
    G = gate.shape[0]
    _require(G >= 1 and M % G == 0, f"{M} rows do not split evenly over {G} gate rows")
    return M // G


def _check_stream(name: str, t: torch.Tensor, cols: int) -> None:
    """A residual-stream matrix: bf16 rows, or float32 rows of 16-byte chunks."""
    _require(t.is_cuda, f"{name} must be a ROCm device tensor")
    _require(t.dtype in (torch.bfloat16, torch.float32), f"{name} must be bfloat16 or float32, got {t.dtype}")
    _require(t.dim() == 2 and t.stride(1) == 1 and t.shape[1] == cols, f"{name} must be a row-major [M, {cols}] matrix")


def gemm_fwd_gated(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, h_rows: torch.Tensor | None,
                   bs: Sequence[torch.Tensor], routing: SegmentRouting, res: torch.Tensor, gate: torch.Tensor,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """out = res + bf16(X·Wᵀ + bias + h_rows·B_aᵀ)·gate[row group] (the block's gated residual; gate
    [G, N] fp32, M / G consecutive rows per gate row), in the residual stream's dtype: bf16 (the sum
    rounded to bf16) or float32 (not rounded). out may be res (in place)."""
    M, K = x.shape
    N = w.shape[0]
    _check_rows("X", x, K)
    _check_rows("W", w, K)
    _check_stream("residual", res, N)
    _require(res.shape[0] == M, "residual has the rows of X")
    per = _gate_rows(gate, M, N)
    if bias is not None:
        _require(bias.is_cuda and bias.dtype in _DT and bias.is_contiguous() and bias.shape == (N,), "bias")
    ranks = [int(b.shape[1]) for b in bs]
    for b in bs:
        _check_rows("lora_b", b)
        _require(b.is_contiguous() and b.shape[0] == N, "lora_b must be contiguous [N, r]")
    y = out if out is not None else torch.empty((M, N), dtype=res.dtype, device=x.device)
    _check_stream("out", y, N)
    _require(y.dtype == res.dtype, "out has the residual stream's dtype")
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(b) for b in bs]), _lib.i32_array(ranks)
    ldh = h_rows.stride(0) if h_rows is not None else 0
    stream = _stream(x)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        _require(r0 % per == 0, "a call group must start at a gate-row boundary")
        o, i, n = _routing_arrays(off, ids)
        hr = None if h_rows is None else h_rows[r0:r1].data_ptr()
        _lib.check("mlora_gemm_fwd_gated", lib.mlora_gemm_fwd_gated(
            x[r0:r1].data_ptr(), x.stride(0), r1 - r0, K, w.data_ptr(), w.stride(0), N,
            _ptr(bias), _DT[bias.dtype] if bias is not None else 0, hr, ldh,
            ptrs, rk, len(bs), o, i, n, res[r0:r1].data_ptr(), res.stride(0),
            gate[r0 // per:].data_ptr(), gate.stride(0), per, y[r0:r1].data_ptr(), y.stride(0), _DT[res.dtype],
            stream))
    return y


def gate_scale_rows(dout: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """dY = bf16(dOut · gate[row group]): the frozen-gate derivative of the gated residual
    (dOut bf16 or float32, the residual stream's dtype)."""
    M, N = dout.shape
    _check_stream("dOut", dout, N)
    per = _gate_rows(gate, M, N)
    dy = torch.empty((M, N), dtype=torch.bfloat16, device=dout.device)
    lib = _lib.load()
    _lib.check("mlora_gate_scale_rows", lib.mlora_gate_scale_rows(
        dout.data_ptr(), dout.stride(0), M, N, gate.data_ptr(), gate.stride(0), per, dy.data_ptr(), dy.stride(0),
        _DT[dout.dtype], _stream(dout)))
    return dy


def _rows3(name: str, t: torch.Tensor, dtypes, shape) -> None:
    _require(t.is_cuda, f"{name} must be a ROCm device tensor")
    _require(t.dtype in dtypes, f"{name} must be one of {[str(d) for d in dtypes]}, got {t.dtype}")
    _require(tuple(t.shape) == tuple(shape), f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    _require(t.stride(2) == 1 or t.shape[2] <= 1, f"{name} must have unit feature stride")


def modulated_norm(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, out: torch.Tensor, *,
                   eps: float | None = None, scale_row: torch.Tensor | None = None,
                   shift_row: torch.Tensor | None = None) -> torch.Tensor:
    """out[b,t,f] = bf16(RN(RN(v · RN(1 + s)) + h)) over [B, T, W] operands, where
    v = LayerNorm(x) (affine-free, when eps is given; x bf16 or float32) or x itself (float32,
    already normalized), and s / h are scale / shift, each first added (RN) to a table row
    [W] when scale_row / shift_row are given. Operands may broadcast over tokens (stride 0)."""
    B, T, W = x.shape
    _rows3("x", x, (torch.bfloat16, torch.float32) if eps is not None else (torch.float32,), (B, T, W))
    _rows3("scale", scale, (torch.bfloat16, torch.float32), (B, T, W))
    _rows3("shift", shift, (torch.bfloat16, torch.float32), (B, T, W))
    _rows3("output", out, (torch.bfloat16,), (B, T, W))
    _require((scale_row is None) == (shift_row is None), "scale_row and shift_row come together")
    if scale_row is not None:
        for name, r in (("scale_row", scale_row), ("shift_row", shift_row)):
            _require(r.is_cuda and r.dim() == 1 and r.shape[0] == W and r.stride(0) == 1,
                     f"{name} must be a contiguous device vector of {W}")
            _require(r.dtype in (torch.bfloat16, torch.float32), f"{name} must be bfloat16 or float32")
        _require(scale_row.dtype == shift_row.dtype, "scale_row and shift_row share a dtype")
    _require(eps is None or eps > 0, "LayerNorm epsilon must be positive")
    lib = _lib.load()
    tdt = _DT[scale_row.dtype] if scale_row is not None else _lib.BF16
    _lib.check("mlora_modulated_norm", lib.mlora_modulated_norm(
        x.data_ptr(), _DT[x.dtype], x.stride(0), x.stride(1), int(eps is not None), float(eps or 0.0),
        _ptr(scale_row), _ptr(shift_row), tdt, scale.data_ptr(), _DT[scale.dtype], shift.data_ptr(), _DT[shift.dtype],
        scale.stride(0), scale.stride(1), shift.stride(0), shift.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), B, T, W, _stream(x)))
    return out


def modulated_norm_backward(x: torch.Tensor, g: torch.Tensor, scale: torch.Tensor, dx: torch.Tensor,
                            mean: torch.Tensor, rstd: torch.Tensor, *, eps: float,
                            scale_row: torch.Tensor | None = None) -> torch.Tensor:
    """dx of out = bf16(LN(x)·RN(1 + s) + h) for the upstream gradient g ([B, T, W] each; s =
    RN(scale_row + scale) with a table row); writes the rows' mean and rstd ([B, T] float32)."""
    B, T, W = x.shape
    fl = (torch.bfloat16, torch.float32)
    _rows3("hidden", x, fl, (B, T, W))
    _rows3("grad_output", g, fl, (B, T, W))
    _rows3("scale_component", scale, fl, (B, T, W))
    _rows3("hidden_gradient", dx, fl, (B, T, W))
    for name, t in (("mean", mean), ("rstd", rstd)):
        _require(t.is_cuda and t.dtype == torch.float32 and tuple(t.shape) == (B, T) and t.is_contiguous(),
                 f"{name} must be a contiguous float32 [{B}, {T}] device tensor")
    if scale_row is not None:
        _require(scale_row.is_cuda and scale_row.dim() == 1 and scale_row.shape[0] == W and scale_row.stride(0) == 1
                 and scale_row.dtype in fl, f"scale_row must be a contiguous device vector of {W}")
    _require(eps > 0, "LayerNorm epsilon must be positive")
    lib = _lib.load()
    _lib.check("mlora_modulated_norm_backward", lib.mlora_modulated_norm_backward(
        x.data_ptr(), _DT[x.dtype], x.stride(0), x.stride(1), g.data_ptr(), _DT[g.dtype], g.stride(0), g.stride(1),
        _ptr(scale_row), _DT[scale_row.dtype] if scale_row is not None else _lib.BF16,
        scale.data_ptr(), _DT[scale.dtype], scale.stride(0), scale.stride(1),
        dx.data_ptr(), _DT[dx.dtype], dx.stride(0), dx.stride(1), mean.data_ptr(), rstd.data_ptr(), float(eps),
        B, T, W, _stream(x)))
    return dx


def modulated_norm_component_grad(x: torch.Tensor, g: torch.Tensor, mean: torch.Tensor, rstd: torch.Tensor,
                                  out: torch.Tensor, scale_index: int, shift_index: int) -> torch.Tensor:
    """Scale / shift component gradients into out: [B, 6, W] (summed over tokens: Σ g·n, Σ g)
    or [B, T, 6, W] (per token: g·n, g); n from the row statistics. Other slots untouched."""
    B, T, W = x.shape
    fl = (torch.bfloat16, torch.float32)
    _rows3("hidden", x, fl, (B, T, W))
    _rows3("grad_output", g, fl, (B, T, W))
    for name, t in (("mean", mean), ("rstd", rstd)):
        _require(t.is_cuda and t.dtype == torch.float32 and tuple(t.shape) == (B, T) and t.is_contiguous(),
                 f"{name} must be a contiguous float32 [{B}, {T}] device tensor")
    _require(out.is_cuda and out.dtype in fl, "component gradient must be a bfloat16 or float32 device tensor")
    reduce = out.dim() == 3
    _require(tuple(out.shape) == ((B, 6, W) if reduce else (B, T, 6, W)),
             f"component gradient must be [{B}, 6, {W}] or [{B}, {T}, 6, {W}], got {tuple(out.shape)}")
    _require(out.stride(-1) == 1, "component gradient must have unit feature stride")
    lib = _lib.load()
    if reduce:
        sb, st, sc = out.stride(0), 0, out.stride(1)
        nbytes = lib.mlora_modulated_norm_component_workspace_bytes(B, T, W)
        _lib.check("mlora_modulated_norm_component_workspace_bytes", nbytes if nbytes < 0 else 0)
        ws = torch.empty((max(nbytes, 16) + 15) // 16 * 4, dtype=torch.float32, device=x.device)
    else:
        sb, st, sc = out.stride(0), out.stride(1), out.stride(2)
        ws, nbytes = None, 0
    _lib.check("mlora_modulated_norm_component_grad", lib.mlora_modulated_norm_component_grad(
        x.data_ptr(), _DT[x.dtype], x.stride(0), x.stride(1), g.data_ptr(), _DT[g.dtype], g.stride(0), g.stride(1),
        mean.data_ptr(), rstd.data_ptr(), out.data_ptr(), _DT[out.dtype], sb, st, sc, int(scale_index),
        int(shift_index), int(reduce), _ptr(ws), nbytes, B, T, W, _stream(x)))
    return out


def gemm_dx(dy: torch.Tensor, w: torch.Tensor, g_rows: torch.Tensor | None, as_: Sequence[torch.Tensor],
            routing: SegmentRouting, out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """dX = dY·W + per-segment g_rows·A_a, bf16 out (accumulate: dX += ..., into `out`).
    g_rows may be a column slice of a wider buffer (its row stride is passed)."""
    M, N = dy.shape
    K = w.shape[1]
    _check_rows("dY", dy, N)
    _check_rows("W", w, K)
    ranks = [int(a.shape[0]) for a in as_]
    for a in as_:
        _check_rows("lora_a", a, K)
        _require(a.is_contiguous(), "lora_a must be contiguous [r, K]")
    _require(not accumulate or out is not None, "accumulate needs the dX to add to")
    dx = out if out is not None else torch.empty((M, K), dtype=torch.bfloat16, device=dy.device)
    _check_rows("dX", dx, K)
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(a) for a in as_]), _lib.i32_array(ranks)
    ldg = g_rows.stride(0) if g_rows is not None else 0
    stream = _stream(dy)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        gr = None if g_rows is None else g_rows[r0:r1].data_ptr()
        _lib.check("mlora_gemm_dx", lib.mlora_gemm_dx(
            dy[r0:r1].data_ptr(), dy.stride(0), r1 - r0, N, w.data_ptr(), w.stride(0), K, gr, ldg,
            ptrs, rk, len(as_), o, i, n, dx[r0:r1].data_ptr(), dx.stride(0), int(accumulate), stream))
    return dx


def seg_outer(p: torch.Tensor, frags: list, width: int, ranks: Sequence[int], routing: SegmentRouting,
              out_layout: int, out_dtypes: Sequence[torch.dtype], frag_jt: int | None = None,
              frag_t0: int = 0) -> list[torch.Tensor]:
    """Per-adapter Σ_m P[m,c]·h[m,j] -> [C, r_a] (layout 0) or [r_a, C] (layout 1).

    `frags` are the hi/lo fragments written by `shrink` for the same routing and width; with
    frag_jt / frag_t0, h is the part of fragments of frag_jt j-tiles that starts at j-tile frag_t0.
    """
    M, C = p.shape
    _check_rows("P", p, C)
    lib = _lib.load()
    groups = list(routing.groups(_lib.MAX_SEGMENTS))
    _require(frags is not None and len(frags) == len(groups), "h fragments from shrink() of the same routing")
    dtypes = list(out_dtypes)
    _require(all(d in _DT for d in dtypes), "adapter gradients are float32 or bfloat16")
    jt = frag_jtiles(width) if frag_jt is None else frag_jt
    _require(0 <= frag_t0 and frag_t0 * 16 + max([0, *ranks]) <= jt * 16, "fragment j-tiles out of range")
    outs: list[torch.Tensor | None] = [None] * len(ranks)
    stream = _stream(p)
    shape = (lambda r: (C, r)) if out_layout == 0 else (lambda r: (r, C))
    single = len(groups) == 1
    # Adapters are reduced per output dtype (normally one dtype for all).
    for dt in sorted(set(dtypes), key=str):
        sel = [a for a in range(len(ranks)) if dtypes[a] == dt]
        mask_ranks = _lib.i32_array([r if dtypes[a] == dt else 0 for a, r in enumerate(ranks)])
        # several row groups: reduce each into fp32, then add in group order
        for (r0, r1, off, ids), frag in zip(groups, frags):
            o, i, n = _routing_arrays(off, ids)
            ws_bytes = lib.mlora_seg_outer_workspace_bytes(r1 - r0, C, mask_ranks, len(ranks), o, i, n)
            _lib.check("mlora_seg_outer_workspace_bytes", ws_bytes if ws_bytes < 0 else 0)
            ws = torch.empty((max(ws_bytes, 16) + 15) // 16 * 4, dtype=torch.float32, device=p.device)
            part = [torch.empty(shape(ranks[a]), dtype=dt if single else torch.float32, device=p.device)
                    if a in sel else None for a in range(len(ranks))]
            _lib.check("mlora_seg_outer", lib.mlora_seg_outer(
                p[r0:r1].data_ptr(), p.stride(0), r1 - r0, C, frag.data_ptr() + frag_t0 * _FRAG_TILE_BYTES, jt,
                _lib.ptr_array([_ptr(t) for t in part]), out_layout, _DT[dt if single else torch.float32],
                mask_ranks, len(ranks), o, i, n, ws.data_ptr(), ws.numel() * 4, stream))
            for a in sel:
                outs[a] = part[a] if outs[a] is None else outs[a] + part[a]
        if not single:
            for a in sel:
                outs[a] = outs[a].to(dt)
    return outs  # type: ignore[return-value]


# ------------------------------------------------------------ quantised base (e4m3)

_FP8_STORAGE = (torch.uint8, torch.float8_e4m3fn)


def _check_fp8_rows(name: str, t: torch.Tensor, cols: int | None = None) -> None:
    _require(t.is_cuda, f"{name} must be a ROCm device tensor")
    _require(t.dtype in _FP8_STORAGE, f"{name} must be float8_e4m3fn (or its uint8 bytes), got {t.dtype}")
    _require(t.dim() == 2 and t.stride(1) == 1, f"{name} must be a 2-D row-major matrix")
    if cols is not None:
        _require(t.shape[1] == cols, f"{name} has {t.shape[1]} columns, expected {cols}")


def _check_scale(name: str, s: torch.Tensor, n: int) -> None:
    _require(s.is_cuda and s.dtype == torch.float32 and s.is_contiguous() and s.shape == (n,),
             f"{name} must be a contiguous float32 vector of length {n}")


def quantize_rows_fp8(x: torch.Tensor, col_scale: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row absmax e4m3 quantisation of x (times col_scale[k] per column when given):
    (q float8_e4m3fn [M, K], scale float32 [M]), x·col_scale ≈ q·scale."""
    M, K = x.shape
    _check_rows("X", x, K)
    if col_scale is not None:
        _check_scale("col_scale", col_scale, K)
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x.device)
    scale = torch.empty((M,), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    _lib.check("mlora_quantize_rows_fp8", lib.mlora_quantize_rows_fp8(
        x.data_ptr(), x.stride(0), M, K, _ptr(col_scale), q.data_ptr(), q.stride(0), scale.data_ptr(), _stream(x)))
    return q, scale


def dequant_rows_fp8(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """bf16(e4m3(q[m, k]) · scale[m])."""
    M, K = q.shape
    _check_fp8_rows("q", q, K)
    _check_scale("scale", scale, M)
    y = torch.empty((M, K), dtype=torch.bfloat16, device=q.device)
    lib = _lib.load()
    _lib.check("mlora_dequant_rows_fp8", lib.mlora_dequant_rows_fp8(
        q.data_ptr(), q.stride(0), scale.data_ptr(), M, K, y.data_ptr(), y.stride(0), _stream(q)))
    return y


def div_rows_bf16(x: torch.Tensor, div: torch.Tensor) -> torch.Tensor:
    """bf16(x[m, k] / div[m])."""
    M, K = x.shape
    _check_rows("x", x, K)
    _check_scale("div", div, M)
    y = torch.empty((M, K), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    _lib.check("mlora_div_rows_bf16", lib.mlora_div_rows_bf16(
        x.data_ptr(), x.stride(0), div.data_ptr(), M, K, y.data_ptr(), y.stride(0), _stream(x)))
    return y


def div_rows_bf16_many(xs: Sequence[torch.Tensor], div: torch.Tensor) -> list[torch.Tensor]:
    """[bf16(x[m, k] / div[m]) for x in xs]: matrices of one row count, MAX_ADAPTERS per launch."""
    if not xs:
        return []
    M = xs[0].shape[0]
    for x in xs:
        _check_rows("x", x)
        _require(x.shape[0] == M, "the matrices share their row count")
    _check_scale("div", div, M)
    ys = [torch.empty(x.shape, dtype=torch.bfloat16, device=x.device) for x in xs]
    lib = _lib.load()
    for i0 in range(0, len(xs), _lib.MAX_ADAPTERS):
        xb, yb = xs[i0:i0 + _lib.MAX_ADAPTERS], ys[i0:i0 + _lib.MAX_ADAPTERS]
        _lib.check("mlora_div_rows_bf16_batch", lib.mlora_div_rows_bf16_batch(
            _lib.ptr_array([x.data_ptr() for x in xb]), _lib.i64_array([x.stride(0) for x in xb]), div.data_ptr(),
            M, _lib.i64_array([x.shape[1] for x in xb]), _lib.ptr_array([y.data_ptr() for y in yb]),
            _lib.i64_array([y.stride(0) for y in yb]), len(xb), _stream(xs[0])))
    return ys


def gemm_fwd_fp8(xq: torch.Tensor, x_scale: torch.Tensor, wq: torch.Tensor, w_scale: torch.Tensor | None,
                 bias: torch.Tensor | None, h_rows: torch.Tensor | None, bs: Sequence[torch.Tensor],
                 routing: SegmentRouting) -> torch.Tensor:
    """Y = (Xq·Wqᵀ + per-segment h_rows·B_aᵀ)·x_scale[m]·w_scale[n] + bias, bf16 out (e4m3 MFMA base).

    h_rows and bs are the LoRA operands divided by the scales: shrink(..., row_div=x_scale) and
    div_rows_bf16(lora_b, w_scale); w_scale None means 1. The e4m3 dX is the same product:
    xq = dY·w_scale quantised per row, wq = Wqᵀ [K, N], w_scale None, bs = A_aᵀ [K, r].
    """
    M, K = xq.shape
    N = wq.shape[0]
    _check_fp8_rows("Xq", xq, K)
    _check_fp8_rows("Wq", wq, K)
    _check_scale("x_scale", x_scale, M)
    if w_scale is not None:
        _check_scale("w_scale", w_scale, N)
    if bias is not None:
        _require(bias.is_cuda and bias.dtype in _DT and bias.is_contiguous() and bias.shape == (N,), "bias")
    ranks = [int(b.shape[1]) for b in bs]
    for b in bs:
        _check_rows("lora_b", b)
        _require(b.is_contiguous() and b.shape[0] == N, "lora_b must be contiguous [N, r]")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=xq.device)
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(b) for b in bs]), _lib.i32_array(ranks)
    ldh = h_rows.stride(0) if h_rows is not None else 0
    stream = _stream(xq)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        hr = None if h_rows is None else h_rows[r0:r1].data_ptr()
        _lib.check("mlora_gemm_fwd_fp8", lib.mlora_gemm_fwd_fp8(
            xq[r0:r1].data_ptr(), xq.stride(0), x_scale[r0:r1].data_ptr(), r1 - r0, K,
            wq.data_ptr(), wq.stride(0), _ptr(w_scale), N,
            _ptr(bias), _DT[bias.dtype] if bias is not None else 0, hr, ldh,
            ptrs, rk, len(bs), o, i, n, y[r0:r1].data_ptr(), y.stride(0), 0, stream))
    return y


# ------------------------------------------------------------ fp32 arithmetic

def split_hi_lo(t: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(hi, lo) bf16 parts of a float matrix: hi = bf16(t), lo = bf16(t - hi), both contiguous.
    hi + lo carries ~16 significant bits of t (relative error <= 2^-16)."""
    t32 = t.detach().to(torch.float32)
    hi = t32.to(torch.bfloat16)
    lo = (t32 - hi.to(torch.float32)).to(torch.bfloat16)
    return hi.contiguous(), lo.contiguous()


def _check_f32(name: str, t: torch.Tensor, cols: int | None = None) -> None:
    _require(t.is_cuda, f"{name} must be a ROCm device tensor")
    _require(t.dtype == torch.float32, f"{name} must be float32, got {t.dtype}")
    _require(t.dim() == 2 and t.stride(1) == 1, f"{name} must be a 2-D row-major matrix")
    if cols is not None:
        _require(t.shape[1] == cols, f"{name} has {t.shape[1]} columns, expected {cols}")


def f32_shrink(p: torch.Tensor, ops: Sequence[torch.Tensor], op_layout: int, scales: Sequence[float],
               routing: SegmentRouting, width: int) -> torch.Tensor:
    """fp32 h = s_a·P·Op_aᵀ per segment -> h [M, width] float32 (zeros outside adapter rows / ranks)."""
    M, K = p.shape
    _check_f32("P", p)
    ranks = [int(o.shape[0] if op_layout == 0 else o.shape[1]) for o in ops]
    for o, r in zip(ops, ranks):
        _check_f32("adapter operand", o)
        _require(o.is_contiguous() and o.shape == ((r, K) if op_layout == 0 else (K, r)), "adapter operand shape")
    h = torch.empty((M, width), dtype=torch.float32, device=p.device)
    lib = _lib.load()
    ptrs, rk, sc = _lib.ptr_array([_ptr(o) for o in ops]), _lib.i32_array(ranks), _lib.f32_array(scales)
    stream = _stream(p)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        _lib.check("mlora_f32_shrink", lib.mlora_f32_shrink(
            p[r0:r1].data_ptr(), p.stride(0), r1 - r0, K, ptrs, op_layout, rk, sc, len(ops), o, i, n,
            h[r0:r1].data_ptr(), h.stride(0), width, stream))
    return h


def f32_gemm_fwd(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, h: torch.Tensor | None,
                 bs: Sequence[torch.Tensor], routing: SegmentRouting) -> torch.Tensor:
    """fp32 Y = X·Wᵀ + bias + per-segment h·B_aᵀ."""
    M, K = x.shape
    N = w.shape[0]
    _check_f32("X", x, K)
    _check_f32("W", w, K)
    if bias is not None:
        _require(bias.is_cuda and bias.dtype == torch.float32 and bias.is_contiguous() and bias.shape == (N,), "bias")
    ranks = [int(b.shape[1]) for b in bs]
    for b in bs:
        _check_f32("lora_b", b)
        _require(b.is_contiguous() and b.shape[0] == N, "lora_b must be contiguous [N, r]")
    y = torch.empty((M, N), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(b) for b in bs]), _lib.i32_array(ranks)
    ldh = h.stride(0) if h is not None else 0
    stream = _stream(x)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        _lib.check("mlora_f32_gemm_fwd", lib.mlora_f32_gemm_fwd(
            x[r0:r1].data_ptr(), x.stride(0), r1 - r0, K, w.data_ptr(), w.stride(0), N, _ptr(bias),
            None if h is None else h[r0:r1].data_ptr(), ldh, ptrs, rk, len(bs), o, i, n,
            y[r0:r1].data_ptr(), y.stride(0), stream))
    return y


def f32_gemm_dx(dy: torch.Tensor, w: torch.Tensor, g: torch.Tensor | None, as_: Sequence[torch.Tensor],
                routing: SegmentRouting) -> torch.Tensor:
    """fp32 dX = dY·W + per-segment g·A_a."""
    M, N = dy.shape
    K = w.shape[1]
    _check_f32("dY", dy, N)
    _check_f32("W", w, K)
    ranks = [int(a.shape[0]) for a in as_]
    for a in as_:
        _check_f32("lora_a", a, K)
        _require(a.is_contiguous(), "lora_a must be contiguous [r, K]")
    dx = torch.empty((M, K), dtype=torch.float32, device=dy.device)
    lib = _lib.load()
    ptrs, rk = _lib.ptr_array([_ptr(a) for a in as_]), _lib.i32_array(ranks)
    ldg = g.stride(0) if g is not None else 0
    stream = _stream(dy)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        if r1 == r0:
            continue
        o, i, n = _routing_arrays(off, ids)
        _lib.check("mlora_f32_gemm_dx", lib.mlora_f32_gemm_dx(
            dy[r0:r1].data_ptr(), dy.stride(0), r1 - r0, N, w.data_ptr(), w.stride(0), K,
            None if g is None else g[r0:r1].data_ptr(), ldg, ptrs, rk, len(as_), o, i, n,
            dx[r0:r1].data_ptr(), dx.stride(0), stream))
    return dx


def f32_seg_outer(p: torch.Tensor, h: torch.Tensor, ranks: Sequence[int], routing: SegmentRouting,
                  out_layout: int) -> list[torch.Tensor]:
    """fp32 per-adapter Σ_m P[m,c]·h[m,j] -> [C, r_a] (layout 0) or [r_a, C] (layout 1); row groups of
    more than one call are added in group order."""
    M, C = p.shape
    _check_f32("P", p)
    _check_f32("h", h)
    lib = _lib.load()
    shape = (lambda r: (C, r)) if out_layout == 0 else (lambda r: (r, C))
    outs: list[torch.Tensor | None] = [None] * len(ranks)
    stream = _stream(p)
    for r0, r1, off, ids in routing.groups(_lib.MAX_SEGMENTS):
        o, i, n = _routing_arrays(off, ids)
        part = [torch.zeros(shape(r), dtype=torch.float32, device=p.device) for r in ranks]
        _lib.check("mlora_f32_seg_outer", lib.mlora_f32_seg_outer(
            p[r0:r1].data_ptr(), p.stride(0), r1 - r0, C, h[r0:r1].data_ptr(), h.stride(0),
            _lib.ptr_array([t.data_ptr() for t in part]), out_layout, _lib.i32_array(list(ranks)), len(ranks),
            o, i, n, stream))
        outs = [t if acc is None else acc + t for acc, t in zip(outs, part)]
    return outs  # type: ignore[return-value]
