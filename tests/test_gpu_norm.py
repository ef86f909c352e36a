"""GPU parity of the modulated LayerNorm that opens a DiT sublayer (the downstream
fusion on the linear's output), through the reference-named host functions in ``modulated_norm.py``.

Oracle: ``oracle.multilora_oracle.modulated_norm`` and ``layer_norm``. Bars:

* epilogue and materialization forms (the normalized input is given): bit-exact. Both are
  float32 operations rounded one at a time, then a bf16 store
  (runtime/wan13b_modulated_norm_kernel.py:70-97, :158-174);
* fused LayerNorm (runtime/wan13b_fused_layernorm_kernel.py:22-132): the kernel's float32
  LayerNorm sums in its own fixed order. Against the oracle's float64 LayerNorm, every output
  is within one bf16 ulp and at least 99% are equal.
"""
import numpy as np
import pytest
import torch

from oracle import multilora_oracle as O

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


def _bf16_ulp(a):
    return np.spacing(np.abs(a).astype(np.float32)).astype(np.float64) * 65536  # one bf16 ulp (normal values)


def _check_layernorm_output(got, want, one_plus_s):
    """got and want round two float32 values that differ only by the LayerNorm's summation
    order: |Δv| is a few 1e-7 for unit-variance rows, so the outputs differ by at most one
    bf16 ulp, plus |Δv|·|1 + s| where the shift nearly cancels the product (there the
    output's own ulp is tiny)."""
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = _bf16_ulp(np.maximum(np.abs(got), np.abs(want))) + 1e-5 * np.abs(one_plus_s)
    exact = float((got == want).mean())
    assert (diff <= bound).all(), f"max excess {float((diff - bound).max()):.3g}, exact {exact:.5f}"
    assert exact >= 0.99, f"only {exact:.5f} of the outputs are equal"


def _components(g, dev, B, T, W, dtype, layout):
    """(scale, shift) views [B, T, W]: 'full' (token stride W), 'broadcast' (token stride 0:
    one row per batch, as Wan's per-sample time embedding) or 'six' (token stride 6W: two of
    the six chunks of a [B, T, 6, W] tensor)."""
    if layout == "full":
        return [(0.1 * torch.randn(B, T, W, generator=g)).to(dev, dtype) for _ in range(2)]
    if layout == "broadcast":
        return [(0.1 * torch.randn(B, 1, W, generator=g)).to(dev, dtype).expand(B, T, W) for _ in range(2)]
    e = (0.1 * torch.randn(B, T, 6, W, generator=g)).to(dev, dtype)
    return e[:, :, 1], e[:, :, 0]


@pytest.mark.parametrize("B,T,W", [(1, 4096, 1536), (3, 1000, 1536), (2, 333, 5120), (1, 50, 8)])
@pytest.mark.parametrize("layout", ["full", "broadcast"])
def test_epilogue_is_bit_exact(pkg, dev, B, T, W, layout):
    print(f"modulated-norm epilogue B={B} T={T} W={W} {layout}", flush=True)
    g = torch.Generator().manual_seed(B * T + W)
    normalized = torch.randn(B, T, W, generator=g).to(dev)
    scale, shift = _components(g, dev, B, T, W, torch.float32, layout)
    out = torch.empty(B, T, W, dtype=torch.bfloat16, device=dev)
    pkg.fused_modulated_norm_epilogue(normalized, scale, shift, out)
    want = O.modulated_norm(_np(normalized), _np(scale), _np(shift))
    assert np.array_equal(_np(out), want)


@pytest.mark.parametrize("table_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("comp", [(torch.bfloat16, "six"), (torch.float32, "broadcast"), (torch.float32, "full")])
def test_materialization_is_bit_exact(pkg, dev, table_dtype, comp):
    comp_dtype, layout = comp
    B, T, W = 3, 777, 1536
    print(f"modulated-norm materialization table {table_dtype} components {comp_dtype} {layout}", flush=True)
    g = torch.Generator().manual_seed(7)
    normalized = torch.randn(B, T, W, generator=g).to(dev)
    table = (0.1 * torch.randn(1, 6, W, generator=g)).to(dev, table_dtype)
    scale_c, shift_c = _components(g, dev, B, T, W, comp_dtype, layout)
    out = torch.empty(B, T, W, dtype=torch.bfloat16, device=dev)
    pkg.fused_modulated_norm_materialization(normalized, table, 1, 0, scale_c, shift_c, out)
    want = O.modulated_norm(_np(normalized), _np(scale_c), _np(shift_c), _np(table[0, 1]), _np(table[0, 0]))
    assert np.array_equal(_np(out), want)
    # scale and shift components of different dtypes
    shift_f = shift_c.float()
    pkg.fused_modulated_norm_materialization(normalized, table, 4, 3, scale_c, shift_f, out)
    want = O.modulated_norm(_np(normalized), _np(scale_c), _np(shift_f), _np(table[0, 4]), _np(table[0, 3]))
    assert np.array_equal(_np(out), want)


@pytest.mark.parametrize("hidden_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,T,W", [(1, 2048, 1536), (3, 300, 5120), (2, 100, 520), (1, 64, 8192), (1, 33, 8)])
def test_fused_layernorm_within_one_ulp(pkg, dev, hidden_dtype, B, T, W):
    print(f"fused layernorm modulation {hidden_dtype} B={B} T={T} W={W}", flush=True)
    g = torch.Generator().manual_seed(W + T)
    hidden = (3 + 2 * torch.randn(B, T, W, generator=g)).to(dev, hidden_dtype)
    table = (0.1 * torch.randn(1, 6, W, generator=g)).to(dev)
    scale_c, shift_c = _components(g, dev, B, T, W, torch.float32, "broadcast")
    out = torch.empty(B, T, W, dtype=torch.bfloat16, device=dev)
    if hidden_dtype == torch.bfloat16:
        pkg.fused_bf16_layernorm_modulation(hidden, table, 1, 0, scale_c, shift_c, out, eps=1e-6)
    else:
        pkg.fused_layernorm_modulation(hidden, table, 1, 0, scale_c, shift_c, out, eps=1e-6)
    v = O.layer_norm(_np(hidden), 1e-6)
    want = O.modulated_norm(v, _np(scale_c), _np(shift_c), _np(table[0, 1]), _np(table[0, 0]))
    _check_layernorm_output(_np(out), want, 1 + _np(table[0, 1]) + _np(scale_c))


def test_wan_block_float32_stream_at_full_size(pkg, dev):
    """The Wan-1.3B shape: 2 samples of 32760 tokens, width 1536. The float32 residual stream
    from the gated-residual GEMM epilogue goes through the norm of the next sublayer, with
    Wan's modulation table [1, 6, W] and per-sample time embedding [B, 6, W]
    (token stride 0). Checked against the oracle on every 16th row."""
    print("fused layernorm modulation, Wan-1.3B float32 stream", flush=True)
    B, T, W, eps = 2, 32760, 1536, 1e-6
    g = torch.Generator().manual_seed(13)
    M, K = B * T, 1536
    x = torch.randn(M, K, generator=g).to(dev, torch.bfloat16)
    w = (torch.randn(W, K, generator=g) / K ** 0.5).to(dev, torch.bfloat16)
    b = (0.1 * torch.randn(W, generator=g)).to(dev, torch.bfloat16)
    As = [((torch.rand(64, K, generator=g) * 2 - 1) / K ** 0.5).to(dev, torch.bfloat16) for _ in range(2)]
    Bs = [(0.02 * torch.randn(W, 64, generator=g)).to(dev, torch.bfloat16) for _ in range(2)]
    stream = torch.randn(M, W, generator=g).to(dev)
    gate = (0.5 * torch.randn(B, W, generator=g)).to(dev)
    routing = pkg.SegmentRouting.from_lengths((T, T), (0, 1))
    with torch.no_grad():
        xs = pkg.multi_lora_linear_gated(x, w, b, As, Bs, [1.0, 1.0], routing, stream, gate)
    assert xs.dtype == torch.float32
    table = (0.1 * torch.randn(1, 6, W, generator=g)).to(dev)
    e = (0.1 * torch.randn(B, 6, W, generator=g)).to(dev)
    scale_c = e[:, 1:2].expand(B, T, W)
    shift_c = e[:, 0:1].expand(B, T, W)
    hidden = xs.view(B, T, W)
    out = torch.empty(B, T, W, dtype=torch.bfloat16, device=dev)
    pkg.fused_layernorm_modulation(hidden, table, 1, 0, scale_c, shift_c, out, eps=eps)
    rows = slice(None, None, 16)
    hs = _np(hidden)[:, rows]
    v = O.layer_norm(hs, eps)
    want = O.modulated_norm(v, _np(scale_c)[:, rows], _np(shift_c)[:, rows], _np(table[0, 1]), _np(table[0, 0]))
    _check_layernorm_output(_np(out)[:, rows], want, 1 + _np(table[0, 1]) + _np(scale_c)[:, rows])


def test_contract_violations_raise(pkg, dev):
    print("modulated norm contract checks", flush=True)
    B, T, W = 1, 8, 64
    f32 = torch.zeros(B, T, W, device=dev)
    bf = torch.zeros(B, T, W, device=dev, dtype=torch.bfloat16)
    table = torch.zeros(1, 6, W, device=dev)
    with pytest.raises(RuntimeError):
        pkg.fused_modulated_norm_epilogue(bf.float().bfloat16(), f32, f32, bf)  # normalized must be float32
    with pytest.raises(RuntimeError):
        pkg.fused_modulated_norm_epilogue(f32, f32, f32, f32)  # output must be bfloat16
    with pytest.raises(RuntimeError):
        pkg.fused_modulated_norm_epilogue(f32, f32[:, :4], f32, bf)  # shape mismatch
    with pytest.raises(RuntimeError):
        pkg.fused_modulated_norm_materialization(f32, table[:, :5], 1, 0, f32, f32, bf)  # table layout
    with pytest.raises(RuntimeError):
        pkg.fused_modulated_norm_materialization(f32, table, 6, 0, f32, f32, bf)  # component index
    with pytest.raises(RuntimeError):
        pkg.fused_bf16_layernorm_modulation(f32, table, 1, 0, f32, f32, bf, eps=1e-6)  # hidden must be bf16
    with pytest.raises(RuntimeError):
        pkg.fused_layernorm_modulation(bf, table, 1, 0, f32, f32, bf, eps=0.0)  # epsilon
    with pytest.raises(RuntimeError):
        odd = torch.zeros(B, T, 60, device=dev)
        pkg.fused_modulated_norm_epilogue(odd, odd, odd, torch.zeros(B, T, 60, device=dev, dtype=torch.bfloat16))
    empty = torch.zeros(0, T, W, device=dev)
    assert pkg.fused_modulated_norm_epilogue(empty, empty, empty, empty.bfloat16()).numel() == 0


# ------------------------------------------------------------------ backward

def _bwd_case(dev, B, T, W, hidden_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    hidden = (3 + 2 * torch.randn(B, T, W, generator=g)).to(dev, hidden_dtype)
    grad = torch.randn(B, T, W, generator=g).to(dev, hidden_dtype)
    table = (0.1 * torch.randn(1, 6, W, generator=g)).to(dev)
    e = (0.1 * torch.randn(B, 6, W, generator=g)).to(dev)
    return hidden, grad, table, e


def _rel(got, want):
    return O.rel_l2(got, want)


@pytest.mark.parametrize("hidden_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,T,W", [(3, 700, 1536), (2, 129, 5120), (1, 64, 520), (1, 5, 8)])
def test_hidden_backward_matches_closed_form(pkg, dev, hidden_dtype, B, T, W):
    """dx and the row statistics against the oracle's float64 closed form. float32 dx: rel-L2
    ≤ 1e-5 (fp32 evaluation); bf16 dx: every element within one bf16 ulp plus 1e-4·|dx|max
    (the cancellation in gn - mean(gn) - n·mean(gn·n) is evaluated in fp32)."""
    print(f"modulated-norm hidden backward {hidden_dtype} B={B} T={T} W={W}", flush=True)
    hidden, grad, table, e = _bwd_case(dev, B, T, W, hidden_dtype, seed=B * T + W)
    scale_c = e[:, 1:2].expand(B, T, W)
    dx = torch.empty_like(hidden)
    mean = torch.empty(B, T, device=dev)
    rstd = torch.empty(B, T, device=dev)
    if hidden_dtype == torch.bfloat16:
        pkg.fused_bf16_layernorm_modulation_hidden_backward(hidden, grad, table, 1, scale_c, dx, mean, rstd, eps=1e-6)
    else:
        pkg.fused_layernorm_modulation_hidden_backward(hidden, grad, table, 1, scale_c, dx, mean, rstd, eps=1e-6)
    want, _, _, wmean, wrstd = O.modulated_norm_backward(_np(hidden), _np(grad), _np(scale_c), 1e-6, _np(table[0, 1]))
    np.testing.assert_allclose(_np(mean), wmean, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(_np(rstd), wrstd, rtol=1e-5)
    got = _np(dx)
    if hidden_dtype == torch.float32:
        assert _rel(got, want) <= 1e-5
    else:
        bound = _bf16_ulp(want) + 1e-4 * np.abs(want).max()
        assert (np.abs(got - want) <= bound).all()


@pytest.mark.parametrize("hidden_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_component_gradients(pkg, dev, hidden_dtype, out_dtype):
    """Reduced [B, 6, W] (Σ_t g·n, Σ_t g) and per-token [B, T, 6, W] (g·n, g) gradients against
    the oracle; the four other slots stay untouched. float32 out: rel-L2 ≤ 1e-5 (sums of 1000
    tokens in float32); bf16 out: ≤ 4e-3 (one rounding)."""
    print(f"modulated-norm component gradients {hidden_dtype} -> {out_dtype}", flush=True)
    B, T, W = 2, 1000, 1536
    hidden, grad, table, e = _bwd_case(dev, B, T, W, hidden_dtype, seed=99)
    scale_c = e[:, 4:5].expand(B, T, W)
    dx = torch.empty_like(hidden)
    mean = torch.empty(B, T, device=dev)
    rstd = torch.empty(B, T, device=dev)
    pkg.fused_layernorm_modulation_hidden_backward(hidden, grad, table, 4, scale_c, dx, mean, rstd, eps=1e-6)
    _, ds, dh, _, _ = O.modulated_norm_backward(_np(hidden), _np(grad), _np(scale_c), 1e-6, _np(table[0, 4]))
    tol = 1e-5 if out_dtype == torch.float32 else 4e-3
    red = torch.full((B, 6, W), 7.0, device=dev, dtype=out_dtype)
    pkg.fused_reduced_component_gradient(hidden, grad, mean, rstd, red, 4, 3)
    assert _rel(_np(red[:, 4]), ds.sum(axis=1)) <= tol
    assert _rel(_np(red[:, 3]), dh.sum(axis=1)) <= tol
    assert (_np(red[:, [0, 1, 2, 5]]) == 7.0).all()
    # an empty token interval leaves the reduced buffer untouched (wan13b_fused_layernorm_backward_kernel.py:420-421)
    kept = red.clone()
    pkg.fused_reduced_component_gradient(hidden[:, :0], grad[:, :0], torch.empty(B, 0, device=dev),
                                         torch.empty(B, 0, device=dev), red, 4, 3)
    torch.cuda.synchronize()
    assert torch.equal(red, kept)
    per = torch.full((B, T, 6, W), 7.0, device=dev, dtype=out_dtype)
    pkg.fused_tensor4d_component_gradient(hidden, grad, mean, rstd, per, 4, 3)
    assert _rel(_np(per[:, :, 4]), ds) <= tol
    assert _rel(_np(per[:, :, 3]), dh) <= (0 if out_dtype == hidden_dtype else tol)
    assert (_np(per[:, :, [0, 1, 2, 5]]) == 7.0).all()


@pytest.mark.parametrize("per_token", [False, True])
def test_autograd_op_matches_torch_float64(pkg, dev, per_token):
    """modulated_layer_norm (fused forward + fused backward) against torch autograd of
    layer_norm(x)·(1 + (table + e)[si]) + (table + e)[hi] in float64: the gradients of the
    float32 hidden state, the table and the time embedding. Two backward passes are
    bit-identical (fixed-order reductions)."""
    print(f"modulated layer norm autograd, per_token={per_token}", flush=True)
    B, T, W, eps = 2, 512, 1536, 1e-6
    g = torch.Generator().manual_seed(5)
    hidden = (3 + 2 * torch.randn(B, T, W, generator=g)).to(dev).requires_grad_(True)
    table = (0.1 * torch.randn(1, 6, W, generator=g)).to(dev).requires_grad_(True)
    shape = (B, T, 6, W) if per_token else (B, 6, W)
    e = (0.1 * torch.randn(*shape, generator=g)).to(dev).requires_grad_(True)
    up = torch.randn(B, T, W, generator=g).to(dev, torch.bfloat16)
    out = pkg.modulated_layer_norm(hidden, table, e, 4, 3, eps)
    assert out.dtype == torch.bfloat16
    out.backward(up)
    grads = [t.grad.clone() for t in (hidden, table, e)]
    for t in (hidden, table, e):
        t.grad = None
    pkg.modulated_layer_norm(hidden, table, e, 4, 3, eps).backward(up)
    for a, t in zip(grads, (hidden, table, e)):
        assert torch.equal(a, t.grad)
    # float64 reference on the CPU
    h64 = hidden.detach().double().cpu().requires_grad_(True)
    t64 = table.detach().double().cpu().requires_grad_(True)
    e64 = e.detach().double().cpu().requires_grad_(True)
    mod = t64.unsqueeze(1) + e64 if per_token else t64 + e64  # [B, (T,) 6, W]
    s_ = mod[..., 4, :] if per_token else mod[:, 4:5, :]
    h_ = mod[..., 3, :] if per_token else mod[:, 3:4, :]
    ref = torch.nn.functional.layer_norm(h64, (W,), eps=eps) * (1 + s_) + h_
    assert O.rel_l2(_np(out), ref.detach().numpy()) <= 4e-3  # one bf16 rounding
    ref.backward(up.double().cpu())
    assert O.rel_l2(_np(grads[0]), h64.grad.numpy()) <= 1e-5
    assert O.rel_l2(_np(grads[1]), t64.grad.numpy()) <= 1e-5
    assert O.rel_l2(_np(grads[2]), e64.grad.numpy()) <= 1e-5


def test_wan_block_chain_forward_and_backward(pkg, dev):
    """One Wan-style block built from this library's ops on the float32 residual stream
    (wan/modules/model.py:298-313): norm1 + modulation -> stacked q, k, v -> attention (torch)
    -> o with the gated residual -> norm2 + modulation -> ffn.0 -> tanh-GELU -> ffn.2 with
    the gated residual; two roles (segments) with their own adapters over one frozen base.
    Forward and the gradients of x and of the adapters against the same block in float64
    torch ops (no intermediate bf16 rounding): rel-L2 ≤ 3e-2, the bf16 pipeline's scale."""
    print("Wan block chain: modulated norm + stacked qkv + gated residual", flush=True)
    from tests.toy_dit import _attention
    B, T, C, F, heads, r = 2, 256, 256, 512, 4, 16
    g = torch.Generator().manual_seed(21)
    routing = pkg.SegmentRouting.from_lengths((T, T), (0, 1))
    scales = [1.0, 1.0]

    def lin(k, n):
        w = (torch.randn(n, k, generator=g) / k ** 0.5).to(dev, torch.bfloat16)
        b = (0.02 * torch.randn(n, generator=g)).to(dev, torch.bfloat16)
        As = [((torch.rand(r, k, generator=g) * 2 - 1) / k ** 0.5).to(dev).requires_grad_(True) for _ in range(2)]
        Bs = [(0.05 * torch.randn(n, r, generator=g)).to(dev).requires_grad_(True) for _ in range(2)]
        return w, b, As, Bs

    q, k, v, o, f0, f2 = lin(C, C), lin(C, C), lin(C, C), lin(C, C), lin(C, F), lin(F, C)
    modulation = (0.1 * torch.randn(1, 6, C, generator=g)).to(dev)
    e_time = (0.1 * torch.randn(B, 6, C, generator=g)).to(dev)
    x0 = torch.randn(B, T, C, generator=g).to(dev).requires_grad_(True)
    up = torch.randn(B, T, C, generator=g).to(dev)
    e = modulation + e_time  # [B, 6, C]; the gates e[2], e[5] one row per sample

    def ours(x):
        y = pkg.modulated_layer_norm(x, modulation, e_time, 1, 0)
        qq, kk, vv = pkg.shared_input_multi_lora(y, [q[0], k[0], v[0]], [q[1], k[1], v[1]],
                                                 [q[2], k[2], v[2]], [q[3], k[3], v[3]], scales, routing)
        att = _attention(qq, kk, vv, heads)
        x = pkg.multi_lora_linear_gated(att, *o[:2], o[2], o[3], scales, routing, x, e[:, 2:3].contiguous())
        y = pkg.modulated_layer_norm(x, modulation, e_time, 4, 3)
        h = torch.nn.functional.gelu(pkg.multi_lora_linear(y, *f0[:2], f0[2], f0[3], scales, routing),
                                     approximate="tanh")
        return pkg.multi_lora_linear_gated(h, *f2[:2], f2[2], f2[3], scales, routing, x, e[:, 5:6].contiguous())

    def ref_lin(x, p):
        w, b, As, Bs = p
        xd = x.reshape(2, T, -1)
        ys = [xd[i] @ w.double().t() + b.double() + (xd[i] @ As[i].double().t()) @ Bs[i].double().t() for i in range(2)]
        return torch.stack(ys)

    def ref(x):
        ed = e.double()
        ln = lambda t: torch.nn.functional.layer_norm(t, (C,), eps=1e-6)
        y = ln(x) * (1 + ed[:, 1:2]) + ed[:, 0:1]
        att = _attention(ref_lin(y, q), ref_lin(y, k), ref_lin(y, v), heads)
        x = x + ref_lin(att, o) * ed[:, 2:3]
        y = ln(x) * (1 + ed[:, 4:5]) + ed[:, 3:4]
        h = torch.nn.functional.gelu(ref_lin(y, f0), approximate="tanh")
        return x + ref_lin(h, f2) * ed[:, 5:6]

    out = ours(x0)
    assert out.dtype == torch.float32
    out.backward(up)
    params = [t for p in (q, k, v, o, f0, f2) for t in (*p[2], *p[3])]
    got = [x0.grad.clone()] + [t.grad.clone() for t in params]
    for t in [x0, *params]:
        t.grad = None
    xd = x0.detach().double().requires_grad_(True)
    pd = [t.detach().double().requires_grad_(True) for t in params]
    it = iter(pd)
    for p in (q, k, v, o, f0, f2):
        p[2][:] = [next(it) for _ in range(2)]
        p[3][:] = [next(it) for _ in range(2)]
    want = ref(xd)
    want.backward(up.double())
    assert O.rel_l2(_np(out), want.detach().cpu().numpy()) <= 3e-2
    assert O.rel_l2(_np(got[0]), xd.grad.cpu().numpy()) <= 3e-2
    for a, t in zip(got[1:], pd):
        assert O.rel_l2(_np(a), t.grad.cpu().numpy()) <= 3e-2
