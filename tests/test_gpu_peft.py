"""PEFT LoRA layers (W1 / H3 call site) on the HIP path vs the fp64 oracle and PEFT's own operator
order. The layers are tests/peft_layout.PeftLoraLinear (PEFT's attribute layout; peft itself is
not installed, so parity against the real library stays unpinned).

Bars: bf16 outputs within rel-L2 2e-3 of the exact result; fp32 LoRA masters' gradients within
5e-5 of the exact gradients of the unrounded masters; routing (disabled adapters, mixed batches,
role batches) bit-exact against the same op called per role.
"""
import numpy as np
import pytest
import torch

from oracle import multilora_oracle as O
from peft_layout import peft_model

pytestmark = pytest.mark.gpu

TOL = 2e-3
TOL_MASTER = 5e-5


def f64(t):
    return t.detach().double().cpu().numpy()


def _fill_b(model, std=0.05, seed=0):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if hasattr(m, "lora_B"):
                for name in m.lora_B:
                    w = m.lora_B[name].weight
                    w.copy_(torch.randn(w.shape, generator=g) * std)


def test_w1_layout_fp32_masters_over_bf16_base(pkg, dev):
    """W1 (training/wan_public.py:213): one adapter 'default', r = alpha, fp32 masters (the
    trainables are made float), bf16 base and activations, no autocast around the LoRA."""
    from dmd_system_amd import peft_site as P
    model = peft_model([(256, 384)], {"default": (32, 32.0)}, dtype=torch.float32, seed=1)
    _fill_b(model, seed=1)
    model = model.to(dev)
    P.install_peft_multi_lora(model)
    layer = model[0]
    x = torch.randn(3, 100, 256, device=dev).to(torch.bfloat16).requires_grad_(True)
    y = layer(x)
    assert y.dtype == torch.bfloat16 and y.shape == (3, 100, 384)
    dy = torch.randn_like(y)
    y.backward(dy)
    A, B = layer.lora_A["default"].weight, layer.lora_B["default"].weight
    base = layer.base_layer
    xr, dyr = f64(x.reshape(-1, 256)), f64(dy.reshape(-1, 384))
    off, ids = [0, 300], [0]
    exact = O.forward(xr, f64(base.weight), f64(base.bias), [f64(A)], [f64(B)], [1.0], off, ids)
    dx_ref, dA_ref, dB_ref = O.backward(xr, f64(base.weight), [f64(A)], [f64(B)], [1.0], off, ids, dyr)
    assert O.rel_l2(f64(y.reshape(-1, 384)), exact) <= TOL
    # PEFT's own rounding: bf16 base, fp32 update, fp32 sum, one cast (two roundings in all)
    peft = O.forward_fp32_update(xr, f64(base.weight), f64(base.bias), [f64(A)], [f64(B)], [1.0], off, ids)
    assert O.rel_l2(f64(y.reshape(-1, 384)), peft) <= 2 * TOL
    assert O.rel_l2(f64(x.grad.reshape(-1, 256)), dx_ref) <= TOL
    assert A.grad.dtype == torch.float32
    assert O.rel_l2(f64(A.grad), dA_ref[0]) <= TOL_MASTER
    assert O.rel_l2(f64(B.grad), dB_ref[0]) <= TOL_MASTER
    assert base.weight.grad is None


def test_named_adapters_under_autocast(pkg, dev):
    """H3-style named adapters (backends/training/minimax_h3/model.py:286-330) under bf16 autocast:
    set_adapter switches the role; the adapters are rounded to bf16 as autocast rounds F.linear's
    operands; the result matches the oracle on those rounded operands."""
    from dmd_system_amd import peft_site as P
    model = peft_model([(192, 256)], {"student": (16, 16.0), "fake": (32, 64.0)}, base_dtype=torch.float32, seed=2)
    _fill_b(model, seed=2)
    model = model.to(dev)
    P.install_peft_multi_lora(model)
    layer = model[0]
    x = torch.randn(4, 50, 192, device=dev)
    for name, scale in (("student", 1.0), ("fake", 2.0)):
        layer.set_adapter(name)
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            y = layer(x)
        assert y.dtype == torch.bfloat16
        q = lambda t: f64(t.to(torch.bfloat16))  # noqa: E731
        want = O.forward(q(x.reshape(-1, 192)), q(layer.base_layer.weight), f64(layer.base_layer.bias),
                         [q(layer.lora_A[name].weight)], [q(layer.lora_B[name].weight)], [scale], [0, 200], [0])
        assert O.rel_l2(f64(y.reshape(-1, 256)), want) <= TOL


def test_mixed_batch_disabled_and_roles_are_bit_exact(pkg, dev):
    """adapter_names per sample, disable_adapters, and a role batch (teacher base-only + critic) in
    one launch equal the same op called once per role, bit for bit; gradients reach only the
    adapters whose rows are in the batch."""
    from dmd_system_amd import peft_site as P
    model = peft_model([(128, 192)], {"generator": (16, 16.0), "critic": (8, 16.0)}, dtype=torch.float32, seed=3)
    _fill_b(model, seed=3)
    model = model.to(dev)
    P.install_peft_multi_lora(model)
    layer = model[0]
    x = torch.randn(5, 40, 128, device=dev).to(torch.bfloat16)

    def single(name, xs):
        if name == "__base__":
            layer.enable_adapters(False)
        else:
            layer.enable_adapters(True)
            layer.set_adapter(name)
        with torch.no_grad():
            out = layer(xs)
        layer.enable_adapters(True)
        return out

    names = ["generator", "generator", "__base__", "critic", "generator"]
    with torch.no_grad():
        mixed = layer(x, adapter_names=names)
    for i, n in enumerate(names):
        assert torch.equal(mixed[i], single(n, x[i:i + 1])[0]), (i, n)
    # the base alone equals the plain linear to bf16 rounding
    base_only = single("__base__", x)
    ref = torch.nn.functional.linear(x.float(), layer.base_layer.weight.float(), layer.base_layer.bias.float())
    assert O.rel_l2(f64(base_only), f64(ref)) <= TOL
    # role batch: teacher (2 samples, base only) + critic (3 samples), forward and backward
    batch = pkg.RoleBatch([("teacher", 2), ("critic", 3)])
    xg = x.clone().requires_grad_(True)
    with P.peft_roles_active(model, batch, base_roles=("teacher",)):
        out = layer(xg)
    assert torch.equal(out[:2].detach(), single("__base__", x[:2]))
    assert torch.equal(out[2:].detach(), single("critic", x[2:]))
    out.float().square().mean().backward()
    assert layer.lora_A["critic"].weight.grad is not None
    assert layer.lora_A["generator"].weight.grad is None
    assert torch.isfinite(xg.grad).all()
