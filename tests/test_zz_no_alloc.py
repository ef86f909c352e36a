"""mlora_seg_outer_noalloc (the segmented reduction with its partial sums in the library's
device array, no allocation) against mlora_seg_outer (caller workspace), through the C ABI.

Two calls in a row on one GPU, the second with a smaller input, each bit-identical to the
workspace entry point; and a call whose workspace would exceed the array, rejected with
MLORA_ERR_LIMIT before any device work.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(pkg, dev, M, K, C, ranks, lengths, ids, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
    p = torch.randn(M, C, generator=g, device=dev).to(torch.bfloat16)
    A = [((torch.rand(r, K, generator=g, device=dev) * 2 - 1) / K ** 0.5).to(torch.bfloat16) for r in ranks]
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    width = pkg.kernels.padded_rank(ranks)
    _, frags = pkg.kernels.shrink(x, A, 0, [1.0] * len(ranks), routing, True, width)
    assert len(frags) == 1
    return p, frags[0], pkg.kernels.frag_jtiles(width), routing


def _run(pkg, lib, p, frag, jt, ranks, routing, out_dtype, noalloc):
    L = pkg._lib
    M, C = p.shape
    dt = torch.float32 if out_dtype == L.F32 else torch.bfloat16
    outs = [torch.full((C, r), float("nan"), dtype=dt, device=p.device) for r in ranks]
    off, ids = L.i64_array(routing.seg_offsets), L.i32_array(routing.adapter_ids)
    rk = L.i32_array(list(ranks))
    ptrs = L.ptr_array([o.data_ptr() for o in outs])
    stream = torch.cuda.current_stream(p.device).cuda_stream
    if noalloc:
        st = lib.mlora_seg_outer_noalloc(p.data_ptr(), p.stride(0), M, C, frag.data_ptr(), jt, ptrs, 0, out_dtype,
                                         rk, len(ranks), off, ids, len(routing.adapter_ids), stream)
        ws_bytes = None
    else:
        ws_bytes = lib.mlora_seg_outer_workspace_bytes(M, C, rk, len(ranks), off, ids, len(routing.adapter_ids))
        ws = torch.empty(max(ws_bytes, 16) // 4 + 4, dtype=torch.float32, device=p.device)
        st = lib.mlora_seg_outer(p.data_ptr(), p.stride(0), M, C, frag.data_ptr(), jt, ptrs, 0, out_dtype, rk,
                                 len(ranks), off, ids, len(routing.adapter_ids), ws.data_ptr(), ws.numel() * 4,
                                 stream)
    assert st == L.OK, lib.mlora_status_string(st)
    torch.cuda.synchronize()
    return outs, ws_bytes


def test_noalloc_matches_workspace_entry_twice(pkg, dev):
    lib = pkg._lib.load()
    L = pkg._lib
    cases = [  # the Wan-1.3B reduction shape, then a smaller, ragged one
        dict(M=65520, K=256, C=1536, ranks=(64, 64), lengths=(32760, 32760), ids=(0, 1), seed=61, dt=L.BF16),
        dict(M=1000, K=136, C=200, ranks=(24, 8, 40), lengths=(77, 301, 250, 372), ids=(2, 0, -1, 1), seed=62,
             dt=L.F32),
    ]
    for c in cases:
        print("case", {k: v for k, v in c.items() if k not in ("ids",)}, flush=True)
        p, frag, jt, routing = _case(pkg, dev, c["M"], c["K"], c["C"], c["ranks"], c["lengths"], c["ids"], c["seed"])
        want, ws_bytes = _run(pkg, lib, p, frag, jt, c["ranks"], routing, c["dt"], noalloc=False)
        assert 0 < ws_bytes <= L.NOALLOC_SCRATCH_BYTES  # the default plan fits: bit-identical expected
        got, _ = _run(pkg, lib, p, frag, jt, c["ranks"], routing, c["dt"], noalloc=True)
        for a, b in zip(got, want):
            assert not torch.isnan(a).any()
            assert torch.equal(a, b)


def test_noalloc_rejects_a_workspace_larger_than_the_array(pkg, dev):
    """16 segments of 1024 rows at C = 12288 (the FLUX FFN width), ranks up to 128: the partial
    sums (~100 MB) exceed the 64 MiB array: MLORA_ERR_LIMIT, nothing launched."""
    lib = pkg._lib.load()
    L = pkg._lib
    n = 16
    off = L.i64_array([1024 * i for i in range(n + 1)])
    ids = L.i32_array(list(range(n)))
    rk = L.i32_array([16, 32, 64, 128] * 4)
    assert lib.mlora_seg_outer_workspace_bytes(1024 * n, 12288, rk, n, off, ids, n) > L.NOALLOC_SCRATCH_BYTES
    outs = L.ptr_array([0x10000 * (i + 1) for i in range(n)])
    st = lib.mlora_seg_outer_noalloc(0x1000, 12288, 1024 * n, 12288, 0x2000, 8, outs, 0, L.F32, rk, n, off, ids, n,
                                     None)
    assert st == L.ERR_LIMIT
