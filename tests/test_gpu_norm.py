"""GPU parity of the modulated LayerNorm that opens a DiT sublayer (the
modulated norm), through the reference-named host functions in ``modulated_norm.py``.

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
