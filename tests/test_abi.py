"""The C-ABI library loads, exports every symbol include/mlora.h declares, and
rejects bad arguments with the documented status codes before any launch
(so these run without a GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mlora.h"


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._lib.load()


def declared_symbols():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(mlora_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    syms = declared_symbols()
    for name in ("mlora_abi_version", "mlora_status_string", "mlora_shrink", "mlora_gemm_fwd", "mlora_gemm_dx",
                 "mlora_seg_outer", "mlora_seg_outer_workspace_bytes"):
        assert name in syms


def test_library_exports_every_declared_symbol(lib, pkg):
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in pkg._lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_status_strings(lib, pkg):
    assert lib.mlora_abi_version() == pkg._lib.ABI_VERSION == 9
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.mlora_status_string(code)
    assert b"unknown" in lib.mlora_status_string(-99)


def test_header_limits_match_python(pkg):
    text = HEADER.read_text()
    for name, val in (("MLORA_MAX_SEGMENTS", pkg._lib.MAX_SEGMENTS), ("MLORA_MAX_ADAPTERS", pkg._lib.MAX_ADAPTERS),
                      ("MLORA_MAX_RANK", pkg._lib.MAX_RANK), ("MLORA_ABI_VERSION", pkg._lib.ABI_VERSION),
                      ("MLORA_MAX_STACKED", pkg._lib.MAX_STACKED)):
        assert re.search(rf"#define {name} {val}\b", text), name
    assert "#define MLORA_MAX_GEMM_RANK (MLORA_MAX_RANK * MLORA_MAX_STACKED)" in text
    assert pkg._lib.MAX_GEMM_RANK == pkg._lib.MAX_RANK * pkg._lib.MAX_STACKED


def _gemm_fwd(lib, L, *, M=64, K=64, N=64, x=0x1000, w=0x2000, y=0x3000, ldx=None, off=None, ids=None,
              ranks=(8,), bptr=(0x4000,), h=0x5000, ldh=8, bias=None, bias_dtype=1):
    off = off if off is not None else [0, M]
    ids = ids if ids is not None else [0]
    return lib.mlora_gemm_fwd(x, ldx or K, M, K, w, K, N, bias, bias_dtype, h, ldh,
                              L.ptr_array(list(bptr)), L.i32_array(list(ranks)), len(ranks),
                              L.i64_array(off), L.i32_array(ids), len(ids), y, N, 0, None)


def test_gemm_fwd_rejects_bad_routing_and_layout(lib, pkg):
    L = pkg._lib
    assert _gemm_fwd(lib, L, off=[0, 32]) == L.ERR_INVALID            # offsets do not cover M
    assert _gemm_fwd(lib, L, off=[1, 64]) == L.ERR_INVALID            # does not start at 0
    assert _gemm_fwd(lib, L, off=[0, 40, 30, 64], ids=[0, 0, 0]) == L.ERR_INVALID  # decreasing
    assert _gemm_fwd(lib, L, ids=[1]) == L.ERR_INVALID                # adapter id out of range
    assert _gemm_fwd(lib, L, ids=[-2]) == L.ERR_INVALID
    assert _gemm_fwd(lib, L, x=0x1008) == L.ERR_UNSUPPORTED           # misaligned X
    assert _gemm_fwd(lib, L, K=60, ldx=60) == L.ERR_UNSUPPORTED       # K not a multiple of 8
    assert _gemm_fwd(lib, L, ranks=(5,)) == L.ERR_INVALID             # rank not a multiple of 8
    assert _gemm_fwd(lib, L, ranks=(L.MAX_GEMM_RANK + 8,)) == L.ERR_LIMIT  # rank above the GEMM limit
    # a stacked rank above the shrink's limit is a GEMM rank: validated against h's width
    assert _gemm_fwd(lib, L, ranks=(L.MAX_RANK + 8,), ldh=8) == L.ERR_INVALID
    assert _gemm_fwd(lib, L, bptr=(0,)) == L.ERR_INVALID              # used adapter without B
    assert _gemm_fwd(lib, L, h=0) == L.ERR_INVALID                    # adapter rows without h
    assert _gemm_fwd(lib, L, bias=0x6000, bias_dtype=2) == L.ERR_UNSUPPORTED
    n = L.MAX_SEGMENTS + 1
    assert _gemm_fwd(lib, L, M=n, off=list(range(n + 1)), ids=[0] * n) == L.ERR_LIMIT


def test_gemm_fwd_empty_problem_is_a_no_op(lib, pkg):
    L = pkg._lib
    assert _gemm_fwd(lib, L, M=0, off=[0, 0], x=0, y=0, h=0) == L.OK


def test_seg_outer_workspace_and_validation(lib, pkg):
    L = pkg._lib
    off, ids = L.i64_array([0, 1000, 3000]), L.i32_array([0, 1])
    ranks = L.i32_array([64, 128])
    ws = lib.mlora_seg_outer_workspace_bytes(3000, 1536, ranks, 2, off, ids, 2)
    assert ws > 0 and ws % (1536 * 4) == 0
    # adapters without rows need no workspace
    assert lib.mlora_seg_outer_workspace_bytes(3000, 1536, ranks, 2, L.i64_array([0, 3000]),
                                               L.i32_array([-1]), 1) == 0
    outs = L.ptr_array([0x7000, 0x8000])
    st = lib.mlora_seg_outer(0x1000, 1536, 3000, 1536, 0x2000, 8, outs, 0, L.F32, ranks, 2, off, ids, 2,
                             0x9000, ws - 16, None)
    assert st == L.ERR_WORKSPACE
    st = lib.mlora_seg_outer(0x1000, 1536, 3000, 1536, 0x2000, 8, outs, 2, L.F32, ranks, 2, off, ids, 2,
                             0x9000, ws, None)
    assert st == L.ERR_INVALID  # bad layout
    st = lib.mlora_seg_outer(0x1000, 1536, 3000, 1536, 0x2000, 4, outs, 0, L.F32, ranks, 2, off, ids, 2,
                             0x9000, ws, None)
    assert st == L.ERR_INVALID  # fragments narrower than rank 128


def test_frag_bytes(lib, pkg):
    L = pkg._lib
    # segments of 40 and 0 and 70 rows -> padded 64 + 0 + 96 rows = 5 blocks of 32
    n = lib.mlora_frag_bytes(110, 4, L.i64_array([0, 40, 40, 110]), L.i32_array([0, -1, 1]), 3)
    assert n == 5 * 4 * 2048
    assert lib.mlora_frag_bytes(110, 99, L.i64_array([0, 110]), L.i32_array([0]), 1) == L.ERR_INVALID


def test_shrink_validation(lib, pkg):
    L = pkg._lib
    off, ids = L.i64_array([0, 64]), L.i32_array([0])
    args = lambda layout, ranks, h, lo=None: lib.mlora_shrink(  # noqa: E731
        0x1000, 64, 64, 64, L.ptr_array([0x2000]), lo, layout, L.i32_array(ranks), L.f32_array([1.0]), 1,
        off, ids, 1, h, 64, None, 0, None, None)
    assert args(3, [8], 0x3000) == L.ERR_INVALID
    assert args(0, [12], 0x3000) == L.ERR_INVALID
    assert args(0, [L.MAX_RANK + 8], 0x3000) == L.ERR_LIMIT  # the shrink's rank limit stays 256
    assert args(0, [8], 0) == L.ERR_INVALID
    # split (fp32-master) operands: every used operand needs an aligned lo part
    assert args(0, [8], 0x3000, lo=L.ptr_array([0])) == L.ERR_INVALID
    assert args(0, [8], 0x3000, lo=L.ptr_array([0x4008])) == L.ERR_UNSUPPORTED


def test_library_matches_its_sources(lib, pkg):
    """The library reports the hash of the sources it was built from; the loader refuses a
    library whose hash differs from the sources beside it (a stale prebuilt library)."""
    built = lib.mlora_source_hash().decode()
    assert len(built) == 64 and built == pkg._lib.expected_source_hash()
    saved = pkg._lib._LIB
    orig = pkg._lib.expected_source_hash
    try:
        pkg._lib._LIB = None
        pkg._lib.expected_source_hash = lambda: "0" * 64
        with pytest.raises(RuntimeError, match="other sources"):
            pkg._lib.load()
    finally:
        pkg._lib.expected_source_hash = orig
        pkg._lib._LIB = saved


def test_f32_entry_points_validate_before_launch(lib, pkg):
    L = pkg._lib
    off, ids = L.i64_array([0, 64]), L.i32_array([0])
    ptr, rk, sc = L.ptr_array([0x2000]), L.i32_array([5]), L.f32_array([1.0])
    sh = lambda layout=0, h=0x3000, width=5, p=0x1000, o=off: lib.mlora_f32_shrink(  # noqa: E731
        p, 64, 64, 64, ptr, layout, rk, sc, 1, o, ids, 1, h, width, width, None)
    assert sh(layout=2) == L.ERR_INVALID
    assert sh(width=4) == L.ERR_INVALID                 # narrower than the rank
    assert sh(p=0x1002) == L.ERR_UNSUPPORTED            # float rows are 4-byte aligned
    assert sh(h=0) == L.ERR_INVALID
    assert sh(o=L.i64_array([0, 60])) == L.ERR_INVALID  # routing covers M rows
    fwd = lambda ldw=64, h=0x5000, bias=None: lib.mlora_f32_gemm_fwd(  # noqa: E731
        0x1000, 64, 64, 64, 0x2000, ldw, 48, bias, h, 8, ptr, rk, 1, off, ids, 1, 0x3000, 48, None)
    assert fwd(ldw=32) == L.ERR_INVALID                 # ld < K
    assert fwd(h=0) == L.ERR_INVALID                    # adapter rows need h
    assert fwd(bias=0x6002) == L.ERR_UNSUPPORTED
    dx = lambda g=0x5000: lib.mlora_f32_gemm_dx(  # noqa: E731
        0x1000, 48, 64, 48, 0x2000, 64, 64, g, 8, ptr, rk, 1, off, ids, 1, 0x3000, 64, None)
    assert dx(g=0) == L.ERR_INVALID
    so = lambda layout=0, outs=(0x7000,): lib.mlora_f32_seg_outer(  # noqa: E731
        0x1000, 64, 64, 64, 0x2000, 8, L.ptr_array(list(outs)), layout, rk, 1, off, ids, 1, None)
    assert so(layout=3) == L.ERR_INVALID
    assert so(outs=(0,)) == L.ERR_INVALID
    assert lib.mlora_f32_shrink(0x1000, 64, 0, 64, ptr, 0, rk, sc, 1, L.i64_array([0, 0]), ids, 1, 0x3000, 5,
                                5, None) == L.OK


def test_fp8_entry_points_validate_before_launch(lib, pkg):
    L = pkg._lib
    # quantize: K must be a multiple of 16 for the e4m3 rows, ld >= K, non-null scale,
    # a column-factor vector (optional) 16-byte aligned
    assert lib.mlora_quantize_rows_fp8(0x1000, 40, 4, 40, None, 0x2000, 48, 0x3000, None) == L.ERR_UNSUPPORTED
    assert lib.mlora_quantize_rows_fp8(0x1000, 32, 4, 32, None, 0x2000, 16, 0x3000, None) == L.ERR_INVALID
    assert lib.mlora_quantize_rows_fp8(0x1000, 32, 4, 32, None, 0x2000, 32, None, None) == L.ERR_INVALID
    assert lib.mlora_quantize_rows_fp8(0x1000, 32, 4, 32, 0x5004, 0x2000, 32, 0x3000, None) == L.ERR_UNSUPPORTED
    assert lib.mlora_quantize_rows_fp8(0x1000, 32, 0, 32, None, 0x2000, 32, None, None) == L.OK
    assert lib.mlora_dequant_rows_fp8(0x1001, 32, 0x3000, 4, 32, 0x2000, 32, None) == L.ERR_UNSUPPORTED
    assert lib.mlora_dequant_rows_fp8(0x1000, 32, None, 4, 32, 0x2000, 32, None) == L.ERR_INVALID
    assert lib.mlora_div_rows_bf16(0x1000, 32, None, 4, 32, 0x2000, 32, None) == L.ERR_INVALID
    assert lib.mlora_div_rows_bf16(0x1000, 4, 0x3000, 4, 8, 0x2000, 8, None) == L.ERR_INVALID

    def div_batch(xs=(0x1000, 0x4000), lds=(64, 32), div=0x3000, M=4, ks=(64, 32), ys=(0x2000, 0x5000),
                  ldys=None, n=None):
        n = len(xs) if n is None else n
        return lib.mlora_div_rows_bf16_batch(L.ptr_array(list(xs)), L.i64_array(list(lds)), div, M,
                                             L.i64_array(list(ks)), L.ptr_array(list(ys)),
                                             L.i64_array(list(ldys or lds)), n, None)
    assert div_batch(div=None) == L.ERR_INVALID                       # rows to divide, no divisors
    assert div_batch(div=None, ks=(0, 0)) == L.OK                     # nothing to divide
    assert div_batch(M=0, div=None) == L.OK
    assert div_batch(lds=(64, 16)) == L.ERR_INVALID                   # pitch below the width
    assert div_batch(xs=(0x1000, 0x4008)) == L.ERR_UNSUPPORTED        # 16-byte rows
    assert div_batch(ks=(64, 36), lds=(64, 40)) == L.ERR_UNSUPPORTED  # widths in 8-element chunks
    assert div_batch(ks=(64, -8)) == L.ERR_INVALID
    assert div_batch(n=-1) == L.ERR_INVALID
    assert div_batch(xs=[0x1000] * (L.MAX_ADAPTERS + 1), lds=[64] * (L.MAX_ADAPTERS + 1),
                     ks=[64] * (L.MAX_ADAPTERS + 1), ys=[0x2000] * (L.MAX_ADAPTERS + 1)) == L.ERR_LIMIT
    assert div_batch(n=0) == L.OK

    def fwd8(M=64, K=64, N=64, ldx=64, xs=0x6000, ws=0x7000, off=None, ids=None):
        off = off if off is not None else [0, M]
        ids = ids if ids is not None else [-1]
        return lib.mlora_gemm_fwd_fp8(0x1000, ldx, xs, M, K, 0x2000, K, ws, N, None, 1, None, 0,
                                      L.ptr_array([0x4000]), L.i32_array([8]), 1,
                                      L.i64_array(off), L.i32_array(ids), len(ids), 0x3000, N, 0, None)
    assert fwd8(K=40, ldx=48) == L.ERR_UNSUPPORTED       # K not a multiple of 16
    assert fwd8(ldx=72) == L.ERR_UNSUPPORTED             # ld not a multiple of 16
    assert fwd8(ldx=32) == L.ERR_INVALID                 # ld < K
    assert fwd8(xs=None) == L.ERR_INVALID                # the row scales are required
    assert fwd8(ws=0x7004) == L.ERR_UNSUPPORTED          # w_scale 16-byte aligned
    assert fwd8(K=0, ldx=0) == L.ERR_UNSUPPORTED         # an e4m3 contraction is required
    assert fwd8(off=[0, 60]) == L.ERR_INVALID            # routing must cover M rows
    assert fwd8(M=0, off=[0, 0]) == L.OK
    assert fwd8(M=0, off=[0, 0], ws=None) == L.OK        # w_scale may be NULL (all 1: the e4m3 dX)



def test_gated_residual_entry_points_validate(lib, pkg):
    L = pkg._lib
    off, ids = L.i64_array([0, 64]), L.i32_array([-1])
    b, rk = L.ptr_array([0x4000]), L.i32_array([8])

    def fwd(res=0x7000, gate=0x8000, ldgate=64, gate_rows=16, out=0x9000, M=64, dt=L.BF16):
        o = L.i64_array([0, M])
        return lib.mlora_gemm_fwd_gated(0x1000, 64, M, 64, 0x2000, 64, 64, None, 1, None, 0, b, rk, 1, o, ids, 1,
                                        res, 64, gate, ldgate, gate_rows, out, 64, dt, None)

    assert fwd(res=None) == L.ERR_INVALID
    assert fwd(gate=None) == L.ERR_INVALID
    assert fwd(gate_rows=0) == L.ERR_INVALID
    assert fwd(ldgate=60) == L.ERR_UNSUPPORTED                 # gate rows shorter than N
    assert fwd(ldgate=66) == L.ERR_UNSUPPORTED                 # gate rows are 16-byte chunks
    assert fwd(gate=0x8004) == L.ERR_UNSUPPORTED
    assert fwd(res=0x7008) == L.ERR_UNSUPPORTED
    assert fwd(M=0) == L.OK
    assert fwd(dt=L.FP8_E4M3) == L.ERR_UNSUPPORTED           # the stream is bf16 or float32
    assert fwd(dt=L.F32, res=0x7008) == L.ERR_UNSUPPORTED    # float32 rows are 16-byte aligned
    assert fwd(dt=L.F32, out=None) == L.ERR_INVALID

    def gs(dout=0x1000, gate=0x8000, ldgate=64, gate_rows=4, dy=0x3000, M=8, N=64, dt=L.BF16):
        return lib.mlora_gate_scale_rows(dout, 64, M, N, gate, ldgate, gate_rows, dy, 64, dt, None)

    assert gs(gate=None) == L.ERR_INVALID
    assert gs(gate_rows=0) == L.ERR_INVALID
    assert gs(ldgate=62) == L.ERR_UNSUPPORTED
    assert gs(dy=0x3002) == L.ERR_UNSUPPORTED
    assert gs(M=0) == L.OK
    assert gs(M=-1) == L.ERR_INVALID
    assert gs(dt=L.F32, dout=0x1004) == L.ERR_UNSUPPORTED
    assert gs(dt=2) == L.ERR_UNSUPPORTED


def test_stacked_gemm_validates_before_launch(lib, pkg):
    L = pkg._lib
    off, ids = L.i64_array([0, 64]), L.i32_array([0])
    b, rk = L.ptr_array([0x4000]), L.i32_array([64])

    def st(N=768, group_cols=256, group_ecols=64, ldh=192, M=64):
        o = L.i64_array([0, M])
        ys = L.ptr_array([0x3000, 0x6000, 0x9000])
        return lib.mlora_gemm_fwd_stacked(0x1000, 64, M, 64, 0x2000, 64, N, group_cols, None, 1, 0x5000, ldh,
                                          group_ecols, b, rk, 1, o, ids, 1, ys, group_cols, None)

    assert st(group_cols=128) == L.ERR_UNSUPPORTED   # a whole number of 256-wide tiles per linear
    assert st(N=640) == L.ERR_UNSUPPORTED            # N a multiple of group_cols
    assert st(group_ecols=32) == L.ERR_INVALID       # rank 64 does not fit 32 columns per linear
    assert st(ldh=128) == L.ERR_INVALID              # h rows hold every linear's columns
    assert st(N=9 * 256, group_cols=256) == L.ERR_UNSUPPORTED   # more than MLORA_MAX_STACKED linears
    assert st(M=0) == L.OK

    def dx(groups=3, ldw=768, dys=(0x1000, 0x2000, 0x3000)):
        return lib.mlora_gemm_dx_stacked(L.ptr_array(list(dys)), 256, 64, 256, groups, 0x4000, ldw, 64, 0x5000, 192,
                                         b, rk, 1, off, ids, 1, 0x6000, 64, None)
    assert dx(groups=9) == L.ERR_UNSUPPORTED
    assert dx(ldw=512) == L.ERR_INVALID             # W_cat^T rows hold the three linears' columns
    assert dx(dys=(0x1000, 0x2008, 0x3000)) == L.ERR_UNSUPPORTED


def _mnorm(lib, *, x=0x1000, x_dtype=1, apply_ln=1, eps=1e-6, srow=None, hrow=None, tdt=1,
           scale=0x2000, sdt=0, shift=0x3000, hdt=0, out=0x4000, B=1, T=4, W=64, xst=None, ost=None, osb=None):
    xst = W if xst is None else xst
    ost = W if ost is None else ost
    osb = T * ost if osb is None else osb
    return lib.mlora_modulated_norm(x, x_dtype, T * xst, xst, apply_ln, eps, srow, hrow, tdt,
                                    scale, sdt, shift, hdt, 0, 0, 0, 0, out, osb, ost, B, T, W, None)


def test_modulated_norm_rejects_bad_arguments(lib, pkg):
    L = pkg._lib
    assert _mnorm(lib, W=60) == L.ERR_UNSUPPORTED                      # width not a multiple of 8
    assert _mnorm(lib, W=8200) == L.ERR_UNSUPPORTED                    # wider than 8192
    assert _mnorm(lib, eps=0.0) == L.ERR_INVALID                       # LayerNorm epsilon
    assert _mnorm(lib, eps=float("nan")) == L.ERR_INVALID
    assert _mnorm(lib, apply_ln=0, x_dtype=1) == L.ERR_UNSUPPORTED     # normalized input is float32
    assert _mnorm(lib, x_dtype=2) == L.ERR_UNSUPPORTED                 # e4m3 hidden state
    assert _mnorm(lib, sdt=2) == L.ERR_UNSUPPORTED
    assert _mnorm(lib, srow=0x5000) == L.ERR_INVALID                   # table rows come in pairs
    assert _mnorm(lib, srow=0x5000, hrow=0x6000, tdt=2) == L.ERR_UNSUPPORTED
    assert _mnorm(lib, x=None) == L.ERR_INVALID
    assert _mnorm(lib, out=None) == L.ERR_INVALID
    assert _mnorm(lib, x=0x1008) == L.ERR_UNSUPPORTED                  # 16-byte alignment
    assert _mnorm(lib, xst=68) == L.ERR_UNSUPPORTED                    # row stride not a multiple of 8
    assert _mnorm(lib, ost=32) == L.ERR_INVALID                        # output rows overlap
    assert _mnorm(lib, B=2, osb=3 * 64) == L.ERR_INVALID               # the two samples' rows overlap
    assert _mnorm(lib, B=-1) == L.ERR_INVALID
    assert _mnorm(lib, B=0) == L.OK                                    # nothing to do, no launch
    assert _mnorm(lib, W=0) == L.OK


def test_modulated_norm_backward_rejects_bad_arguments(lib, pkg):
    L = pkg._lib

    def bwd(x=0x1000, g=0x2000, sc=0x3000, dx=0x4000, mean=0x5000, rstd=0x6000, eps=1e-6, W=64, T=4, dt=1, B=1,
            dxsb=None):
        dxsb = T * W if dxsb is None else dxsb
        return lib.mlora_modulated_norm_backward(x, dt, T * W, W, g, dt, T * W, W, None, 1, sc, 0, 0, 0,
                                                 dx, dt, dxsb, W, mean, rstd, eps, B, T, W, None)

    assert bwd(W=5128) == L.ERR_UNSUPPORTED          # the backward keeps rows up to 5120 in registers
    assert bwd(W=12) == L.ERR_UNSUPPORTED
    assert bwd(eps=0.0) == L.ERR_INVALID
    assert bwd(dt=2) == L.ERR_UNSUPPORTED
    assert bwd(mean=None) == L.ERR_INVALID
    assert bwd(g=0x2004) == L.ERR_UNSUPPORTED        # 16-byte alignment
    assert bwd(T=0) == L.OK
    assert bwd(B=2, dxsb=3 * 64) == L.ERR_INVALID    # the two samples' dx rows overlap

    def comp(reduce=1, si=4, hi=3, ws=None, wsb=0, out=0x7000, sb=6 * 64, st=0, sc=64, W=64, T=4, B=1):
        return lib.mlora_modulated_norm_component_grad(0x1000, 1, T * W, W, 0x2000, 1, T * W, W, 0x5000, 0x6000,
                                                       out, 0, sb, st, sc, si, hi, reduce, ws, wsb, B, T, W, None)

    need = lib.mlora_modulated_norm_component_workspace_bytes(1, 4, 64)
    assert need == 1 * 1 * 2 * 64 * 4
    assert comp() == L.ERR_WORKSPACE                 # the reduced form needs its partial-sum workspace
    assert comp(ws=0x8000, wsb=need - 4) == L.ERR_WORKSPACE
    assert comp(si=3, hi=3) == L.ERR_INVALID         # two different slots
    assert comp(si=6) == L.ERR_INVALID
    assert comp(sc=32) == L.ERR_INVALID              # slots overlap
    assert comp(out=None) == L.ERR_INVALID
    assert comp(reduce=0, st=100) == L.ERR_INVALID   # [B, T, 6, W] rows overlap
    assert comp(reduce=0, st=6 * 64, sb=3 * 6 * 64, B=2) == L.ERR_INVALID  # the two samples overlap
    assert comp(reduce=0, sb=4 * 6 * 64, st=6 * 64, out=0x7004) == L.ERR_UNSUPPORTED


# ---------------------------------------------------------------- host-side sizing, random routings

from hypothesis import given, settings, strategies as st  # noqa: E402

_segments = st.lists(st.tuples(st.integers(0, 300), st.integers(-1, 3)), min_size=1, max_size=128)


@settings(max_examples=300, deadline=None)
@given(segs=_segments, jt=st.integers(0, 16))
def test_frag_bytes_is_padded_blocks_times_jtiles(lib, pkg, segs, jt):
    """One 2 KB fragment tile per 32-row block of every segment (each padded to whole blocks) and
    j-tile, whatever the routing."""
    L = pkg._lib
    off = [0]
    for n, _ in segs:
        off.append(off[-1] + n)
    got = lib.mlora_frag_bytes(off[-1], jt, L.i64_array(off), L.i32_array([a for _, a in segs]), len(segs))
    assert got == sum((n + 31) // 32 for n, _ in segs) * jt * 2048


@settings(max_examples=200, deadline=None)
@given(segs=_segments, bad=st.sampled_from(["start", "decrease", "end", "id"]))
def test_malformed_routings_are_rejected(lib, pkg, segs, bad):
    L = pkg._lib
    off = [0]
    for n, _ in segs:
        off.append(off[-1] + n)
    ids = [a for _, a in segs]
    M = off[-1]
    if bad == "start":
        off[0] = 1
    elif bad == "decrease":
        if len(off) < 3:
            off.insert(1, 5)
            ids.append(0)
        off[1] = off[2] + 1
    elif bad == "end":
        M += 1
    else:
        ids[0] = -2
    assert lib.mlora_frag_bytes(M, 4, L.i64_array(off), L.i32_array(ids), len(ids)) == L.ERR_INVALID


@settings(max_examples=200, deadline=None)
@given(segs=_segments, C=st.sampled_from([8, 72, 1536, 8960]))
def test_seg_outer_workspace_follows_the_adapter_rows(lib, pkg, segs, C):
    """fp32 partials of whole C-wide rows; none at all when no adapter owns a row."""
    L = pkg._lib
    off = [0]
    for n, _ in segs:
        off.append(off[-1] + n)
    ids = [a for _, a in segs]
    ranks = L.i32_array([64, 16, 128, 8])
    ws = lib.mlora_seg_outer_workspace_bytes(off[-1], C, ranks, 4, L.i64_array(off), L.i32_array(ids), len(ids))
    assert ws >= 0 and ws % (C * 4) == 0
    assert (ws > 0) == any(n > 0 and a >= 0 for n, a in segs)
