"""Grids of 256x256 output tiles a little over whole rounds of the 256 CUs.

Such a grid (1284 tiles at 27280 x 3072: five rounds and four tiles) runs its whole rounds as
256x256 tiles and its last few tiles (at most 64) as 128x128 quarters (8 waves) in a second
launch. Every output keeps its k order and MFMA sequence in all tile sizes, so the GEMMs must
give the same bits as calls on row blocks of 1024 rows (fewer than 256 tiles: 128x128 tiles
throughout), and the fp64 oracle's result within the bf16 tolerance. Covered: the forward
GEMM with bias and three rank-128 segments (config 3's routing), the NN dX, a tail of 64 tiles
(5000 x 4096: 256 quarters), one of 104 tiles (27280 x 14336, run as 256x256 tiles), quarters
wholly past the matrix (a last row tile of 100 rows and a last column tile of 128 columns), the
stacked forward and dX of three linears that read one input, the gated-residual epilogue on bf16
and float32 streams, and the e4m3 forward (which runs its tail as 256x256 tiles).
"""
import math

import pytest
import torch

from oracle import multilora_oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3
CFG3_SEGS = (8054, 11878, 7348)  # config 3's three segments (27280 rows)


def f64(t):
    return t.detach().double().cpu().numpy()


def _sub_routing(pkg, routing, r0, r1):
    """The segments of rows [r0, r1), renumbered from 0."""
    lengths, ids = [], []
    off = routing.seg_offsets
    for s, a in enumerate(routing.adapter_ids):
        lo, hi = max(off[s], r0), min(off[s + 1], r1)
        if lo < hi:
            lengths.append(hi - lo)
            ids.append(a)
    return pkg.SegmentRouting.from_lengths(lengths, ids)


def _operands(dev, M, K, N, rank, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    b = (torch.randn(N, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    h = (torch.randn(M, rank, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    bs = [(torch.randn(N, rank, generator=g) * 0.05).to(torch.bfloat16).to(dev) for _ in range(3)]
    return x, w, b, h, bs


def _row_blocks(M, rows=1024):
    return [(r0, min(r0 + rows, M)) for r0 in range(0, M, rows)]


@pytest.mark.parametrize("M,K,N,lengths,ids", [
    (27280, 320, 3072, CFG3_SEGS, (0, 1, 2)),            # 1284 tiles: a tail of 4
    (5000, 256, 4096, (2100, 2900), (0, 2)),             # 20 x 16 tiles: a tail of 64
    (27280, 192, 14336, CFG3_SEGS, (2, -1, 0)),          # 5992 tiles: a tail of 104 (not split)
    (4964, 200, 3200, (2000, 2964), (1, 0)),              # 20 x 13 tiles: quarters past M and N
], ids=["tail4", "tail64", "tail104", "narrow_edges"])
def test_forward_tail_equals_row_blocks(pkg, dev, M, K, N, lengths, ids):
    from dmd_system_amd import kernels
    print(f"tail forward M={M} K={K} N={N}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    x, w, b, h, bs = _operands(dev, M, K, N, 128, seed=M + N)
    y = kernels.gemm_fwd(x, w, b, h, bs, routing)
    torch.cuda.synchronize()
    for r0, r1 in _row_blocks(M):
        yb = kernels.gemm_fwd(x[r0:r1], w, b, h[r0:r1], bs, _sub_routing(pkg, routing, r0, r1))
        torch.cuda.synchronize()
        assert torch.equal(y[r0:r1], yb), (r0, r1)
    # sampled rows (every 29th, and the last 300: the tail's row tiles) against the fp64 product
    # (h given: Y = X·Wᵀ + b + h·B_aᵀ per segment)
    rows = sorted(set(range(0, M, 29)) | set(range(M - 300, M)))
    idx = torch.tensor(rows, device=dev)
    ref = f64(x[idx]) @ f64(w).T + f64(b)
    hf = f64(h[idx])
    off = routing.seg_offsets
    for s, a in enumerate(routing.adapter_ids):
        sel = [i for i, m in enumerate(rows) if off[s] <= m < off[s + 1]]
        if a >= 0 and sel:
            ref[sel] += hf[sel] @ f64(bs[a]).T
    assert O.rel_l2(f64(y[idx]), ref) <= TOL


def test_nn_dx_tail_equals_row_blocks(pkg, dev):
    from dmd_system_amd import kernels
    M, N, K = 27280, 320, 3072  # dX [M, K]: 1284 tiles
    print(f"tail dX NN M={M} N={N} K={K}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(CFG3_SEGS, (1, 0, 2))
    g = torch.Generator().manual_seed(5)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    gr = (torch.randn(M, 128, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    As = [((torch.rand(128, K, generator=g) * 2 - 1) / math.sqrt(K)).to(torch.bfloat16).to(dev) for _ in range(3)]
    dx = kernels.gemm_dx(dy, w, gr, As, routing)
    torch.cuda.synchronize()
    for r0, r1 in _row_blocks(M):
        db = kernels.gemm_dx(dy[r0:r1], w, gr[r0:r1], As, _sub_routing(pkg, routing, r0, r1))
        torch.cuda.synchronize()
        assert torch.equal(dx[r0:r1], db), (r0, r1)


def test_fp8_forward_tail_equals_row_blocks(pkg, dev):
    from dmd_system_amd import kernels
    M, K, N = 27280, 256, 3072
    print(f"tail e4m3 forward M={M} K={K} N={N}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(CFG3_SEGS, (0, 2, 1))
    x, w, b, h, bs = _operands(dev, M, K, N, 64, seed=9)
    xq, xs = kernels.quantize_rows_fp8(x)
    wq, ws = kernels.quantize_rows_fp8(w)
    y = kernels.gemm_fwd_fp8(xq, xs, wq, ws, b, h, bs, routing)
    torch.cuda.synchronize()
    for r0, r1 in _row_blocks(M):
        yb = kernels.gemm_fwd_fp8(xq[r0:r1], xs[r0:r1], wq, ws, b, h[r0:r1], bs, _sub_routing(pkg, routing, r0, r1))
        torch.cuda.synchronize()
        assert torch.equal(y[r0:r1], yb), (r0, r1)


def test_stacked_forward_tail_equals_row_blocks(pkg, dev):
    """Three linears that read one input as one GEMM (27280 x 3 x 3072: 3852 tiles, a tail of 12):
    each quarter stores into its own linear's output."""
    from dmd_system_amd import kernels
    M, K, N, G, R = 27280, 256, 3072, 3, 128
    print(f"tail stacked forward M={M} K={K} N={G}x{N}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(CFG3_SEGS, (0, 1, 2))
    g = torch.Generator().manual_seed(11)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(G * N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    b = (torch.randn(G * N, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    h = (torch.randn(M, G * R, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    bs = [(torch.randn(G * N, R, generator=g) * 0.05).to(torch.bfloat16).to(dev) for _ in range(3)]
    ys = kernels.gemm_fwd_stacked(x, w, b, h, bs, routing, N, R)
    torch.cuda.synchronize()
    for r0, r1 in _row_blocks(M):
        yb = kernels.gemm_fwd_stacked(x[r0:r1], w, b, h[r0:r1], bs, _sub_routing(pkg, routing, r0, r1), N, R)
        torch.cuda.synchronize()
        for y, y1 in zip(ys, yb):
            assert torch.equal(y[r0:r1], y1), (r0, r1)


def test_stacked_dx_tail_equals_row_blocks(pkg, dev):
    """dX of three stacked linears (27280 x 3072 output: 1284 tiles, a tail of 4)."""
    from dmd_system_amd import kernels
    M, K, N, G, R = 27280, 3072, 256, 3, 64
    print(f"tail stacked dX M={M} K={K} N={G}x{N}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(CFG3_SEGS, (2, 0, 1))
    g = torch.Generator().manual_seed(12)
    dys = [torch.randn(M, N, generator=g).to(torch.bfloat16).to(dev) for _ in range(G)]
    w_t = (torch.randn(K, G * N, generator=g) / math.sqrt(G * N)).to(torch.bfloat16).to(dev)
    gr = (torch.randn(M, G * R, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    a_t = [((torch.rand(K, G * R, generator=g) * 2 - 1) / math.sqrt(K)).to(torch.bfloat16).to(dev) for _ in range(3)]
    dx = kernels.gemm_dx_stacked(dys, w_t, gr, a_t, routing)
    torch.cuda.synchronize()
    for r0, r1 in _row_blocks(M):
        db = kernels.gemm_dx_stacked([d[r0:r1] for d in dys], w_t, gr[r0:r1], a_t, _sub_routing(pkg, routing, r0, r1))
        torch.cuda.synchronize()
        assert torch.equal(dx[r0:r1], db), (r0, r1)


@pytest.mark.parametrize("stream_dtype", [torch.bfloat16, torch.float32], ids=["bf16_stream", "f32_stream"])
def test_gated_forward_tail_equals_row_blocks(pkg, dev, stream_dtype):
    """The gated-residual epilogue (16 gate rows of 1705 rows) on a grid with a tail of 4."""
    from dmd_system_amd import kernels
    M, K, N = 27280, 256, 3072
    print(f"tail gated forward M={M} K={K} N={N} {stream_dtype}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(CFG3_SEGS, (1, 2, 0))
    x, w, b, h, bs = _operands(dev, M, K, N, 128, seed=13)
    g = torch.Generator().manual_seed(14)
    res = torch.randn(M, N, generator=g).to(stream_dtype).to(dev)
    gate = torch.randn(16, N, generator=g).to(dev)
    per = M // 16
    y = kernels.gemm_fwd_gated(x, w, b, h, bs, routing, res, gate)
    torch.cuda.synchronize()
    for r0 in range(0, M, 2 * per):  # row blocks on gate-row boundaries
        r1 = min(r0 + 2 * per, M)
        yb = kernels.gemm_fwd_gated(x[r0:r1], w, b, h[r0:r1], bs, _sub_routing(pkg, routing, r0, r1), res[r0:r1],
                                    gate[r0 // per:r1 // per].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(y[r0:r1], yb), (r0, r1)
