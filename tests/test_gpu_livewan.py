"""LiveWan's critic LoRA (reference/livewan_wan21/wanstreamer/lora.py:8-27) on the HIP path.

* A module of the reference's layout (rank 32, fp32 a / b over a bf16 base, the layout
  inject_lora leaves on the bf16 critic, runtime/livewan_crossscale_worker.py:1587,1594), run
  through install_livewan_multi_lora: Y and dX within rel-L2 2e-3 of the fp64 oracle (one bf16
  rounding), da / db within 5e-5 of the exact gradients of the unrounded fp32 masters. The
  reference's own operator order (base and update rounded to bf16, bf16 multiply, bf16 add) is
  farther from the oracle than these outputs, and within two roundings of them.
* ``enabled = False`` is the base alone: bit-exact against an adapter-free launch, and a / b
  get no gradient (they are outside the graph, as in the reference).
* The teacher + critic batch of livewan_crossscale_worker.py:2614-2645 (the teacher's
  conditional and unconditional passes with the adapters off, the critic's with them on) run as
  one call per linear through fuse_roles(..., base_roles=('teacher',)): every linear bit-exact
  against the per-role calls, the whole model's forward and the critic's adapter gradients
  within 1e-3 (the torch attention in between runs at another batch size).
"""
import numpy as np
import pytest
import torch

from livewan_layout import TARGETS, WanLike, wrap_reference_layout
from oracle import multilora_oracle as O

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-3
TOL_MASTER_GRAD = 5e-5


def f64(t):
    return t.detach().double().cpu().numpy()


def _model(pkg, dev, hidden=256, ffn=512, layers=2, rank=32):
    model = WanLike(hidden=hidden, ffn=ffn, heads=4, layers=layers).to(torch.bfloat16)
    wrap_reference_layout(model, rank=rank)
    model = model.to(dev)
    pkg.install_livewan_multi_lora(model)
    return model


@pytest.mark.parametrize("K,N", [(1536, 1536), (1536, 8960), (8960, 1536)])
def test_reference_layout_matches_oracle(pkg, dev, K, N):
    print(f"livewan layout K={K} N={N}", flush=True)
    from livewan_layout import RefLayoutLoRA
    g = torch.Generator().manual_seed(61)
    base = torch.nn.Linear(K, N).to(torch.bfloat16)
    with torch.no_grad():
        base.weight.copy_(torch.randn(N, K, generator=g) / K ** 0.5)
        base.bias.copy_(torch.randn(N, generator=g) / K ** 0.5)
    torch.manual_seed(62)
    m = RefLayoutLoRA(base, rank=32)
    with torch.no_grad():
        m.b.copy_(torch.randn(N, 32, generator=g) * 0.02)
    m = m.to(dev)
    model = torch.nn.ModuleDict({"lin": m})
    pkg.install_livewan_multi_lora(model)
    M = 4096
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    xg = x.to(dev).requires_grad_(True)
    y = m(xg)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and m.a.grad.dtype == torch.float32 and m.b.grad.dtype == torch.float32
    assert m.base.weight.grad is None
    off, ids = [0, M], [0]
    W, bias, A, B = f64(m.base.weight), f64(m.base.bias), [f64(m.a)], [f64(m.b)]
    y_ref = O.forward(f64(x), W, bias, A, B, [1.0], off, ids)
    dx_ref, dA_ref, dB_ref = O.backward(f64(x), W, A, B, [1.0], off, ids, f64(dy))
    errs = {"y": O.rel_l2(f64(y), y_ref), "dx": O.rel_l2(f64(xg.grad), dx_ref),
            "da": O.rel_l2(f64(m.a.grad), dA_ref[0]), "db": O.rel_l2(f64(m.b.grad), dB_ref[0])}
    print("rel-L2", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["y"] <= TOL_BF16 and errs["dx"] <= TOL_BF16, errs
    assert errs["da"] <= TOL_MASTER_GRAD and errs["db"] <= TOL_MASTER_GRAD, errs
    # the reference's operator order (base, update and sum each rounded to bf16) sits farther from
    # the exact result (2.4e-3 at 1536x1536) than the single rounding here, and within two
    # roundings of it
    y_lw = O.forward_livewan(f64(x), W, bias, A, B, [1.0], off, ids)
    assert errs["y"] < O.rel_l2(y_lw, y_ref)
    assert O.rel_l2(f64(y), y_lw) <= 2 * TOL_BF16


def test_disabled_is_the_base_alone(pkg, dev):
    print("livewan disabled", flush=True)
    model = _model(pkg, dev, hidden=256, ffn=512, layers=1)
    lin = model.blocks[0].ffn[0]
    x = torch.randn(3, 100, 256, device=dev).to(torch.bfloat16).requires_grad_(True)
    with pkg.livewan.lora_enabled(model, False):
        y = lin(x)
    with torch.no_grad():
        y_free = pkg.multi_lora_linear(x, lin.base.weight, lin.base.bias, [], [], [],
                                       pkg.SegmentRouting.single(300, pkg.BASE_ONLY))
    assert torch.equal(y, y_free)
    y.float().sum().backward()
    assert lin.a.grad is None and lin.b.grad is None and x.grad is not None
    want = O.forward(f64(x.reshape(-1, 256)), f64(lin.base.weight), f64(lin.base.bias), [], [], [], [0, 300], [-1])
    assert O.rel_l2(f64(y.reshape(-1, 512)), want) <= TOL_BF16
    with torch.no_grad():
        assert not torch.equal(lin(x), y)  # enabled again on exit: the adapter acts


@pytest.mark.parametrize("name", TARGETS)
def test_teacher_critic_linear_bit_exact(pkg, dev, name):
    print(f"livewan teacher+critic linear {name}", flush=True)
    model = _model(pkg, dev)
    fused = pkg.fuse_roles({"teacher": model, "critic": model}, base_roles=("teacher",))
    lin, own = fused.blocks[1].get_submodule(name), model.blocks[1].get_submodule(name)
    B, L = 2, 96
    z = torch.randn(B, L, own.base.in_features, device=dev).to(torch.bfloat16)
    rb = pkg.RoleBatch([("teacher", 2 * B), ("critic", B)])
    with torch.no_grad():
        with pkg.roles_active(fused, rb):
            yt, yc = rb.split(lin(torch.cat([z, z, z])))
        with pkg.livewan.lora_enabled(model, False):
            rt = own(torch.cat([z, z]))
        with pkg.livewan.lora_enabled(model, True):
            rc = own(z)
    assert torch.equal(yt, rt) and torch.equal(yc, rc)
    assert not torch.equal(yc, yt[:B])  # the critic's adapter acts


def test_teacher_critic_model_forward_and_backward(pkg, dev):
    """The whole model: teacher (2B samples, adapters off) and critic (B samples) in one pass;
    the critic's adapter gradients from one backward equal those of its own call."""
    print("livewan teacher+critic model", flush=True)
    model = _model(pkg, dev)
    fused = pkg.fuse_roles({"teacher": model, "critic": model}, base_roles=("teacher",))
    B, L, H = 2, 64, 256
    gen = torch.Generator().manual_seed(63)
    z = torch.randn(B, L, H, generator=gen).to(dev, torch.bfloat16)
    w = torch.randn(B, L, H, generator=gen).to(dev, torch.bfloat16)
    adapters = [p for p in model.parameters() if p.requires_grad]
    rb = pkg.RoleBatch([("teacher", 2 * B), ("critic", B)])
    with pkg.roles_active(fused, rb):
        yt, yc = rb.split(fused(torch.cat([z, z, z])))
    (yc.float() * w.float()).sum().backward()
    batched = [p.grad.clone() for p in adapters]
    for p in adapters:
        p.grad = None
    with torch.no_grad(), pkg.livewan.lora_enabled(model, False):
        rt = model(torch.cat([z, z]))
    with pkg.livewan.lora_enabled(model, True):
        rc = model(z)
    (rc.float() * w.float()).sum().backward()
    separate = [p.grad for p in adapters]

    def rel(a, b):
        return float((a.double() - b.double()).norm() / b.double().norm())

    assert rel(yt.detach(), rt) <= 1e-3 and rel(yc.detach(), rc.detach()) <= 1e-3
    assert all(rel(a, b) <= 1e-3 for a, b in zip(batched, separate))
    assert all(float(a.abs().sum()) > 0 for a in batched)
    assert np.isfinite(f64(yc)).all()
