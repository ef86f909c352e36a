"""The multi-LoRA op captured in a HIP graph (torch.cuda.graph): forward and backward captured
once, then replayed. Every entry point of the library only launches kernels on the caller's
stream (no allocation, memset or host synchronisation inside), so a capture holds the same
kernels as the eager step. Each replay must equal the eager step bit for bit, with eager work
and synchronisations between the replays, and again after the captured inputs are overwritten.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _tensors(dev, seed, M=4096, K=512, N=768, ranks=(64, 32)):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    As = [((torch.rand(r, K, generator=g) * 2 - 1) / math.sqrt(K)).to(torch.bfloat16) for r in ranks]
    Bs = [(torch.randn(N, r, generator=g) * 0.05).to(torch.bfloat16) for r in ranks]
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    return [t.to(dev) for t in (x, *As, *Bs, dy)]


def _eager(op, x, As, Bs, dy):
    """y, dX, dA, dB of one eager step on fresh leaves holding the given values."""
    xl = x.detach().clone().requires_grad_(True)
    Al = [a.detach().clone().requires_grad_(True) for a in As]
    Bl = [v.detach().clone().requires_grad_(True) for v in Bs]
    y = op(xl, Al, Bl)
    y.backward(dy)
    torch.cuda.synchronize()
    return [y.detach(), xl.grad] + [a.grad for a in Al] + [v.grad for v in Bl]


@pytest.mark.parametrize("path", ["bf16_dx_nn", "bf16_dx_nt", "e4m3", "e4m3_dx_bf16"])
def test_graph_replays_equal_eager(pkg, dev, path):
    """bf16 base (dX on the NN kernel or against the transposed base) and e4m3 base (e4m3 dX, or
    bf16 dX against the dequantised base): forward, backward and the per-row quantisations."""
    M, K, N = 4096, 512, 768
    g = torch.Generator().manual_seed(30)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    b = (torch.randn(N, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(dev)
    routing = pkg.SegmentRouting.from_lengths((1500, 96, 2500), (0, -1, 1))
    if path.startswith("bf16"):
        wt = w.t().contiguous() if path == "bf16_dx_nt" else None

        def op(x, As, Bs):
            return pkg.multi_lora_linear(x, w, b, As, Bs, [1.0, 0.5], routing, weight_t=wt)
    else:
        from dmd_system_amd import kernels
        wq, ws = kernels.quantize_rows_fp8(w)
        wqt = wq.t().contiguous()

        def op(x, As, Bs):
            return pkg.multi_lora_linear_fp8(x, wq, ws, b, As, Bs, [1.0, 0.5], routing, wq_t=wqt,
                                             dx_bf16=path == "e4m3_dx_bf16")

    x0, a0, a1, b0, b1, dy0 = _tensors(dev, 31)
    x = x0.clone().requires_grad_(True)
    As = [a0.clone().requires_grad_(True), a1.clone().requires_grad_(True)]
    Bs = [b0.clone().requires_grad_(True), b1.clone().requires_grad_(True)]
    dy = dy0.clone()
    leaves = [x, *As, *Bs]

    def step():
        y = op(x, As, Bs)
        y.backward(dy)
        return y

    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            for t in leaves:
                t.grad = None
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in leaves:
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static = step()

    def outputs():
        return [y_static, x.grad] + [t.grad for t in As] + [t.grad for t in Bs]

    want = _eager(op, x0, [a0, a1], [b0, b1], dy0)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outputs(), want)):
            assert torch.equal(got, ref), (rep, i)
        assert torch.randn(1000, device=dev).abs().sum().item() > 0  # eager work between replays

    # new values in the captured inputs: the replay reads them
    x1, c0, c1, d0, d1, dy1 = _tensors(dev, 32)
    with torch.no_grad():
        for t, v in zip([x, *As, *Bs, dy], [x1, c0, c1, d0, d1, dy1]):
            t.copy_(v)
    want = _eager(op, x1, [c0, c1], [d0, d1], dy1)
    for rep in range(2):
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, ref) in enumerate(zip(outputs(), want)):
            assert torch.equal(got, ref), ("new inputs", rep, i)
