"""GPU parity of the gated residual fused into the GEMM epilogue (downstream
epilogue fusion): out = bf16(x + bf16(Y)·gate) with the rounding contract of
runtime/helios_residual_kernel.py:66-86, and its frozen-gate backward (:90-133).

Oracle: ``oracle.multilora_oracle.gated_residual`` / ``gate_scale`` applied to this
library's own unfused output Y (the same kernels without the fusion). Bar: bit-exact —
the fused epilogue rounds Y to bf16 exactly as the unfused store does, then the same two
float32 operations. Backward: bit-exact against torch autograd of the unfused composition
(the same dY = bf16(dOut·gate) reaches the same kernels).
"""
import math

import numpy as np
import pytest
import torch

from oracle import multilora_oracle as O

pytestmark = pytest.mark.gpu


def _case(dev, M, K, N, ranks, lengths, ids, seed, samples):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dev, torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(dev, torch.bfloat16)
    b = (torch.randn(N, generator=g) * 0.1).to(dev, torch.bfloat16)
    As = [((torch.rand(r, K, generator=g) * 2 - 1) / math.sqrt(K)).to(dev, torch.bfloat16) for r in ranks]
    Bs = [(torch.randn(N, r, generator=g) * 0.05).to(dev, torch.bfloat16) for r in ranks]
    hidden = torch.randn(M, N, generator=g).to(dev, torch.bfloat16)
    gate = (torch.randn(samples, N, generator=g) * 0.5).to(dev)  # fp32, one row per sample
    return x, w, b, As, Bs, hidden, gate


def _np(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("M,K,N,samples", [(1000, 320, 256, 4), (1000, 320, 256, 1000), (16384, 1536, 1536, 2)])
def test_fused_gated_residual_is_bit_exact(pkg, dev, M, K, N, samples):
    print(f"gated residual M={M} K={K} N={N} gate rows {samples}", flush=True)
    lengths = (M // 2, M // 4, M - M // 2 - M // 4)
    ids = (0, -1, 1)
    x, w, b, As, Bs, hidden, gate = _case(dev, M, K, N, (32, 16), lengths, ids, seed=M + samples, samples=samples)
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    scales = [2.0, 0.5]
    with torch.no_grad():
        y = pkg.multi_lora_linear(x, w, b, As, Bs, scales, routing)
        out = pkg.multi_lora_linear_gated(x, w, b, As, Bs, scales, routing, hidden, gate)
    want = O.gated_residual(_np(hidden), _np(y), _np(gate), M // samples)
    assert np.array_equal(_np(out), want)
    # the same in place on the residual stream, through the kernel wrapper
    A_ops = [a.contiguous() for a in As]
    h_rows, _ = pkg.kernels.shrink(x, A_ops, 0, scales, routing, False, 32)
    res = hidden.clone()
    pkg.kernels.gemm_fwd_gated(x, w, b, h_rows, Bs, routing, res, gate, out=res)
    assert torch.equal(res, out)


def test_fused_gated_residual_backward_matches_unfused(pkg, dev):
    print("gated residual backward", flush=True)
    M, K, N = 2048, 512, 512
    lengths, ids = (1024, 700, 324), (1, 0, -1)
    x, w, b, As, Bs, hidden, gate = _case(dev, M, K, N, (16, 48), lengths, ids, seed=77, samples=4)
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    scales = [1.0, 0.25]
    dout = torch.randn(M, N, generator=torch.Generator().manual_seed(78)).to(dev, torch.bfloat16)

    def run(fused):
        xi = x.clone().requires_grad_(True)
        hi = hidden.clone().requires_grad_(True)
        Ai = [a.clone().requires_grad_(True) for a in As]
        Bi = [v.clone().requires_grad_(True) for v in Bs]
        if fused:
            out = pkg.multi_lora_linear_gated(xi, w, b, Ai, Bi, scales, routing, hi, gate)
        else:
            y = pkg.multi_lora_linear(xi, w, b, Ai, Bi, scales, routing)
            g = gate.repeat_interleave(M // gate.shape[0], dim=0)
            out = (hi.float() + y.float() * g).to(torch.bfloat16)
        out.backward(dout)
        return out.detach(), xi.grad, hi.grad, [a.grad for a in Ai], [v.grad for v in Bi]

    f, u = run(True), run(False)
    assert torch.equal(f[0], u[0])
    assert torch.equal(f[1], u[1]) and torch.equal(f[2], u[2]) and torch.equal(f[2], dout)
    for a, c in zip(f[3] + f[4], u[3] + u[4]):
        assert torch.equal(a, c)
    dy = pkg.kernels.gate_scale_rows(dout, gate)
    assert np.array_equal(_np(dy), O.gate_scale(_np(dout), _np(gate), M // 4))


def test_module_gated_residual_under_roles(pkg, dev):
    """MultiLoRALinear.gated_residual inside a role batch (the block's o-projection)."""
    print("module gated residual", flush=True)
    from toy_dit import make_roles
    teacher, fake, gen = make_roles(pkg, hidden=256, ffn=512, heads=4, rank=16, device=dev, dtype=torch.bfloat16)
    fused = pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})
    B, L = 3, 40
    g = torch.Generator().manual_seed(5)
    attn = torch.randn(B, L, 256, generator=g).to(dev, torch.bfloat16)
    xres = torch.randn(B, L, 256, generator=g).to(dev, torch.bfloat16)
    e2 = torch.randn(B, 1, 256, generator=g).to(dev)  # Wan's per-sample gate e[2]
    rb = pkg.RoleBatch([("teacher", 1), ("fake", 1), ("gen", 1)])
    with torch.no_grad(), pkg.roles_active(fused, rb):
        y = fused.o(attn)
        out = fused.o.gated_residual(attn, xres, e2)
        # the role's own module gives the same for its sample
        out_fake = fake.o.gated_residual(attn[1:2], xres[1:2], e2[1:2])
    want = O.gated_residual(_np(xres.reshape(-1, 256)), _np(y.reshape(-1, 256)), _np(e2.reshape(B, 256)), L)
    assert np.array_equal(_np(out.reshape(-1, 256)), want)
    assert torch.equal(out_fake, out[1:2])


@pytest.mark.parametrize("M,K,N,samples", [(1000, 320, 256, 4), (16384, 1536, 1536, 2)])
def test_fused_gated_residual_float32_stream(pkg, dev, M, K, N, samples):
    """The Wan block's float32 residual stream (model.py:305-306,312-313): out = x + bf16(Y)·gate
    in float32, bit-exact against oracle.gated_residual_f32 on the unfused Y; in place too; and
    the backward (d x = dOut float32, dY = bf16(dOut·gate)) bit-exact against torch autograd of
    the unfused float32 composition."""
    print(f"float32-stream gated residual M={M} K={K} N={N} gate rows {samples}", flush=True)
    lengths = (M // 2, M // 4, M - M // 2 - M // 4)
    ids = (0, -1, 1)
    x, w, b, As, Bs, hidden, gate = _case(dev, M, K, N, (32, 16), lengths, ids, seed=7 * M + samples,
                                          samples=samples)
    g = torch.Generator().manual_seed(M)
    stream = torch.randn(M, N, generator=g).to(dev)  # float32 residual stream
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    scales = [2.0, 0.5]
    with torch.no_grad():
        y = pkg.multi_lora_linear(x, w, b, As, Bs, scales, routing)
        out = pkg.multi_lora_linear_gated(x, w, b, As, Bs, scales, routing, stream, gate)
    assert out.dtype == torch.float32
    want = O.gated_residual_f32(_np(stream), _np(y), _np(gate), M // samples)
    assert np.array_equal(_np(out), want)
    A_ops = [a.contiguous() for a in As]
    h_rows, _ = pkg.kernels.shrink(x, A_ops, 0, scales, routing, False, 32)
    res = stream.clone()
    pkg.kernels.gemm_fwd_gated(x, w, b, h_rows, Bs, routing, res, gate, out=res)
    assert torch.equal(res, out)
    # backward against autograd of the unfused composition, same kernels underneath
    xs = [x.clone().requires_grad_(True) for _ in range(2)]
    ss = [stream.clone().requires_grad_(True) for _ in range(2)]
    Ag = [[a.clone().requires_grad_(True) for a in As] for _ in range(2)]
    Bg = [[v.clone().requires_grad_(True) for v in Bs] for _ in range(2)]
    dout = torch.randn(M, N, generator=g).to(dev)
    fused = pkg.multi_lora_linear_gated(xs[0], w, b, Ag[0], Bg[0], scales, routing, ss[0], gate)
    fused.backward(dout)
    yy = pkg.multi_lora_linear(xs[1], w, b, Ag[1], Bg[1], scales, routing)
    unfused = ss[1] + yy.float() * gate.repeat_interleave(M // samples, dim=0)
    unfused.backward(dout)
    assert torch.equal(fused.detach(), unfused.detach())
    assert ss[0].grad.dtype == torch.float32 and torch.equal(ss[0].grad, ss[1].grad)
    assert torch.equal(xs[0].grad, xs[1].grad)
    for p0, p1 in zip(Ag[0] + Bg[0], Ag[1] + Bg[1]):
        assert torch.equal(p0.grad, p1.grad)
