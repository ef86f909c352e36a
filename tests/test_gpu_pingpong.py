"""Edge cases of the 256x256 NT GEMM's ping-pong schedule, against the other tile shapes.

A grid of 20480 x 4096 outputs is 1280 tiles of 256x256, whole rounds of the 256 CUs, so the
whole launch runs the ping-pong tile (N = 4000 adds a last column of partial 256x256 tiles, 16 x 80
tiles); calls on row blocks of 1024 rows (at most 256 tiles of 128x128) run the interleaved 128x128
tile. Every output keeps its k order and MFMA sequence in both, so
they must agree bit for bit. Covered: contractions shorter than two k-tiles (the walk runs from
the first step), a partial last k-tile, the LoRA-only product (K = 0), LoRA ranks that are not a
whole number of k-tiles, segment boundaries inside a tile (rows of another segment masked), a
null segment, the bias, and the accumulating store. Sampled rows are also checked against the
fp64 product.
"""
import math

import pytest
import torch

from oracle import multilora_oracle as O

pytestmark = pytest.mark.gpu

TOL = 2e-3
M = 20480
SEGS = (7001, 6479, 3000, 4000)   # boundaries inside 256-row tiles
IDS = (0, 1, -1, 2)               # ranks 128, 64 and 96 (not a whole number of 64-wide k-tiles)
RANKS = (128, 64, 96)


def f64(t):
    return t.detach().double().cpu().numpy()


def _sub_routing(pkg, routing, r0, r1):
    lengths, ids = [], []
    off = routing.seg_offsets
    for s, a in enumerate(routing.adapter_ids):
        lo, hi = max(off[s], r0), min(off[s + 1], r1)
        if lo < hi:
            lengths.append(hi - lo)
            ids.append(a)
    return pkg.SegmentRouting.from_lengths(lengths, ids)


def _operands(dev, K, N, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(N, K, generator=g) / math.sqrt(max(K, 1))).to(torch.bfloat16).to(dev)
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).to(dev)
    h = (torch.randn(M, max(RANKS), generator=g) * 0.3).to(torch.bfloat16).to(dev)
    bs = [(torch.randn(N, r, generator=g) * 0.05).to(torch.bfloat16).to(dev) for r in RANKS]
    return x, w, b, h, bs


@pytest.mark.parametrize("K,N", [(0, 4096), (64, 4096), (104, 4096), (136, 4096), (1000, 4096), (1600, 4096),
                                 (136, 4000), (1000, 4000)])
@pytest.mark.parametrize("accumulate", [False, True], ids=["store", "accumulate"])
def test_pingpong_equals_row_blocks(pkg, dev, K, N, accumulate):
    from dmd_system_amd import kernels
    print(f"ping-pong forward M={M} K={K} N={N} accumulate={accumulate}", flush=True)
    routing = pkg.SegmentRouting.from_lengths(SEGS, IDS)
    x, w, b, h, bs = _operands(dev, K, N, seed=K + N + 7 * accumulate)
    bias = None if K == 0 else b
    y0 = (torch.randn(M, N, generator=torch.Generator().manual_seed(3)) * 0.5).to(torch.bfloat16).to(dev)
    y = y0.clone() if accumulate else None
    y = kernels.gemm_fwd(x, w, bias, h, bs, routing, out=y, accumulate=accumulate)
    torch.cuda.synchronize()
    for r0 in range(0, M, 1024):
        r1 = min(r0 + 1024, M)
        yb = y0[r0:r1].clone() if accumulate else None
        yb = kernels.gemm_fwd(x[r0:r1], w, bias, h[r0:r1], bs, _sub_routing(pkg, routing, r0, r1), out=yb,
                              accumulate=accumulate)
        torch.cuda.synchronize()
        assert torch.equal(y[r0:r1], yb), (r0, r1)
    # sampled rows (every 37th, and both sides of every segment boundary) against fp64
    off = routing.seg_offsets
    rows = set(range(0, M, 37))
    for o in off[1:-1]:
        rows |= set(range(max(o - 3, 0), min(o + 3, M)))
    rows = sorted(rows)
    idx = torch.tensor(rows, device=dev)
    ref = f64(x[idx]) @ f64(w).T if K else 0.0 * f64(y[idx])
    if bias is not None:
        ref = ref + f64(bias)
    if accumulate:
        ref = ref + f64(y0[idx])
    hf = f64(h[idx])
    for s, a in enumerate(routing.adapter_ids):
        sel = [i for i, m in enumerate(rows) if off[s] <= m < off[s + 1]]
        if a >= 0 and sel:
            ref[sel] += hf[sel][:, :RANKS[a]] @ f64(bs[a]).T
    assert O.rel_l2(f64(y[idx]), ref) <= TOL
