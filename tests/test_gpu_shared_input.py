"""GPU parity of shared-input stacking: linears that read one tensor, run as one stacked
call, give what each gives alone (forward), and the adapters and the input get the
gradients of the separate calls (backward).

Oracle: the exact fp64 product of the stacked linears, Σ_g over the members for dX
(autograd's sum of the members' dX), per row segment (oracle/multilora_oracle.py
restates it per linear). Tolerances: forward bit-exact against the same kernels called
per member (each member's GEMM reads its own R columns of the stacked h, which the
stacked shrink computes in the same order as the member's own); backward: dX, a sum over the G linears, within √G·2e-3 rel-L2 of the
fp64 reference (one bf16 rounding per accumulating call) and no worse than the per-member
path's (which rounds each member's dX and each bf16 addition), the adapters' gradients
within 2e-3 of the per-member calls'.
"""
import pytest
import torch
from torch import nn

from toy_dit import inputs, make_roles, rel_l2

pytestmark = pytest.mark.gpu


def _members(pkg, dev, G=3, K=512, N=256, ranks=(32, 32), seed=0):
    g = torch.Generator().manual_seed(seed)
    mods = []
    for _ in range(G):
        base = nn.Linear(K, N)
        with torch.no_grad():
            base.weight.copy_(torch.randn(N, K, generator=g) / K ** 0.5)
            base.bias.copy_(torch.randn(N, generator=g) * 0.1)
        m = pkg.MultiLoRALinear(base, ranks=list(ranks), alphas=[2.0 * r for r in ranks])
        with torch.no_grad():
            for b in m.lora_b:
                b.copy_(torch.randn(b.shape, generator=g) * 0.05)
        mods.append(m.to(dev, torch.bfloat16))
    holder = nn.Module()
    for i, m in enumerate(mods):
        holder.add_module(f"m{i}", m)
    return holder, mods


def _reference(x, mods, routing, dys):
    """fp64: per member Y_g, and dX = Σ_g dY_g·W_g + s·(dY_g·B_g)·A_g per segment."""
    xd = x.double()
    ys, dx = [], torch.zeros_like(xd)
    for m, dy in zip(mods, dys):
        W, b = m.base.weight.double(), m.base.bias.double()
        y = xd @ W.T + b
        dyd = dy.double()
        dx += dyd @ W
        for (r0, r1), a in zip(zip(routing.seg_offsets, routing.seg_offsets[1:]), routing.adapter_ids):
            if a < 0 or r1 == r0:
                continue
            A, B, s = m.lora_a[a].double(), m.lora_b[a].double(), m.scales[a]
            y[r0:r1] += s * (xd[r0:r1] @ A.T) @ B.T
            dx[r0:r1] += s * (dyd[r0:r1] @ B) @ A
        ys.append(y)
    return ys, dx


@pytest.mark.parametrize("lengths,ids,ranks", [((300, 212, 100), (0, 1, -1), (32, 32)), ((1000,), (1,), (32, 32)),
                                               ((64, 64), (-1, 0), (32, 32)), ((400, 111), (1, 0), (64, 64))])
def test_stacked_call_matches_members(pkg, dev, lengths, ids, ranks):
    print(f"stacked q/k/v lengths {lengths} ids {ids} ranks {ranks}", flush=True)
    holder, mods = _members(pkg, dev, ranks=ranks)
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    M = sum(lengths)
    x = torch.randn(M, 512, generator=torch.Generator().manual_seed(1)).to(dev, torch.bfloat16)
    dys = [torch.randn(M, 256, generator=torch.Generator().manual_seed(2 + i)).to(dev, torch.bfloat16)
           for i in range(3)]
    params = [p for m in mods for p in (*m.lora_a, *m.lora_b)]

    def run(fused):
        for p in params:
            p.grad = None
        if fused:
            pkg.fuse_shared_inputs(holder, [["m0", "m1", "m2"]])
        xi = x.clone().requires_grad_(True)
        ys = [m(xi, routing) for m in mods]
        torch.autograd.backward(ys, dys)
        if fused:
            assert mods[0].shared_input.launches == 1
            pkg.release_shared_inputs(holder)
        return [y.detach() for y in ys], xi.grad, [None if p.grad is None else p.grad.clone() for p in params]

    ys_f, dx_f, gr_f = run(True)
    ys_s, dx_s, gr_s = run(False)
    for a, b in zip(ys_f, ys_s):
        assert torch.equal(a, b)
    ref_y, ref_dx = _reference(x, mods, routing, dys)
    for a, r in zip(ys_f, ref_y):
        assert rel_l2(a, r) <= 2e-3
    # dX sums G linears' products: the stacked path rounds once per accumulating call (G
    # roundings), the separate path (autograd, as the reference runs it) rounds every member's
    # dX and then each bf16 addition (2G-1 roundings, ~3e-3 here). The bound is the bf16 one
    # per rounded partial sum, and the stacked dX must be no worse than the separate one.
    G = len(mods)
    assert rel_l2(dx_f, ref_dx) <= 2e-3 * G ** 0.5
    assert rel_l2(dx_f, ref_dx) <= rel_l2(dx_s, ref_dx)
    for a, b in zip(gr_f, gr_s):
        assert (a is None) == (b is None)
        if a is not None:
            assert rel_l2(a, b) <= 2e-3


def test_dit_block_with_roles_and_shared_inputs(pkg, dev):
    """q/k/v and cross-attention k/v stacked inside the multi-role module tree: the block's
    outputs and every adapter's gradients match the same tree without stacking."""
    print("dit block roles + shared inputs", flush=True)
    teacher, fake, gen = make_roles(pkg, hidden=256, ffn=512, heads=4, rank=16, device=dev, dtype=torch.bfloat16)
    fused = pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})
    x, c = inputs(4, 48, 12, 256, dev, torch.bfloat16, seed=9)
    w = torch.randn(4, 48, 256, generator=torch.Generator().manual_seed(10)).to(dev, torch.bfloat16)
    rb = pkg.RoleBatch([("teacher", 1), ("fake", 2), ("gen", 1)])
    params = [p for p in fused.parameters() if p.requires_grad]

    def run(stacked):
        for p in params:
            p.grad = None
        groups = pkg.fuse_shared_inputs(fused, [["q", "k", "v"], ["cross.k", "cross.v"]]) if stacked else []
        with pkg.roles_active(fused, rb):
            y = fused(x, c)
        (y.float() * w.float()).sum().backward()
        launches = [g.launches for g in groups]
        pkg.release_shared_inputs(fused)
        return y.detach(), [p.grad.clone() for p in params], launches

    y_s, g_s, launches = run(True)
    y_u, g_u, _ = run(False)
    assert launches == [1, 1]
    assert rel_l2(y_s, y_u) <= 1e-3
    for a, b in zip(g_s, g_u):
        assert rel_l2(a, b) <= 2e-3


def test_reuse_only_for_the_same_unmodified_input(pkg, dev):
    print("shared input reuse keys", flush=True)
    holder, mods = _members(pkg, dev, G=2, ranks=(16,))
    pkg.fuse_shared_inputs(holder, [["m0", "m1"]])
    routing = pkg.SegmentRouting.single(256, 0)
    x = torch.randn(256, 512, generator=torch.Generator().manual_seed(3)).to(dev, torch.bfloat16)
    x0 = x.clone()
    with torch.no_grad():
        y0 = mods[0](x, routing)
        x.add_(1.0)                      # in place: m1 must not reuse the stacked result
        y1 = mods[1](x, routing)
        assert mods[0].shared_input.launches == 2
        y0b = mods[0](x0, routing)       # another tensor: a new stacked call, then m1 reuses it
        y1b = mods[1](x0, routing)
        assert mods[0].shared_input.launches == 3
        pkg.release_shared_inputs(holder)
        assert torch.equal(y0, mods[0](x0, routing)) and torch.equal(y0b, y0)
        assert torch.equal(y1, mods[1](x, routing))
        assert torch.equal(y1b, mods[1](x0, routing))


@pytest.mark.parametrize("transposed", [True, False], ids=["dx_nt", "dx_nn"])
def test_stacked_qkv_at_the_wan_shape(pkg, dev, transposed):
    """q / k / v of the Wan-1.3B block (1536 -> 1536, rank 64, generator + fake critic) as one stacked
    GEMM: each output bit-identical to the member's own call; dX (one GEMM over the three dY) within
    2e-3 of the fp64 sum of the members' dX; adapter gradients within 2e-3 of the per-member calls'."""
    print(f"stacked qkv wan shape, transposed={transposed}", flush=True)
    holder, mods = _members(pkg, dev, G=3, K=1536, N=1536, ranks=(64, 64), seed=5)
    for m in mods:
        m.transposed_base_for_dx = transposed
    lengths, ids = (4096, 4096), (0, 1)
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    M = sum(lengths)
    x = torch.randn(M, 1536, generator=torch.Generator().manual_seed(6)).to(dev, torch.bfloat16)
    dys = [torch.randn(M, 1536, generator=torch.Generator().manual_seed(7 + i)).to(dev, torch.bfloat16)
           for i in range(3)]
    params = [p for m in mods for p in (*m.lora_a, *m.lora_b)]

    def run(fused):
        for p in params:
            p.grad = None
        if fused:
            pkg.fuse_shared_inputs(holder, [["m0", "m1", "m2"]])
        xi = x.clone().requires_grad_(True)
        ys = [m(xi, routing) for m in mods]
        torch.autograd.backward(ys, dys)
        if fused:
            assert mods[0].shared_input.launches == 1
            pkg.release_shared_inputs(holder)
        return [y.detach() for y in ys], xi.grad, [p.grad.clone() for p in params]

    ys_f, dx_f, gr_f = run(True)
    ys_s, dx_s, gr_s = run(False)
    for a, b in zip(ys_f, ys_s):
        assert torch.equal(a, b)
    rows = torch.arange(0, M, 13, device=dev)
    ref_y, ref_dx = _reference(x[rows], mods, pkg.SegmentRouting.from_lengths(
        (int((rows < 4096).sum()), int((rows >= 4096).sum())), ids), [d[rows] for d in dys])
    for a, r in zip(ys_f, ref_y):
        assert rel_l2(a[rows], r) <= 2e-3
    assert rel_l2(dx_f[rows], ref_dx) <= 2e-3
    for a, b in zip(gr_f, gr_s):
        assert rel_l2(a, b) <= 2e-3


def _wan_qkv(pkg, dev, family, rank, seed):
    """q / k / v of the Wan-1.3B block (1536 -> 1536, bf16 base). family 'multi': MultiLoRALinear with
    two bf16 adapters (generator, fake critic); 'peft': PEFT layers of the W1 layout (one adapter
    'default', r = alpha, fp32 masters, training/wan_public.py:213) after install_peft_multi_lora."""
    from peft_layout import PeftLoraLinear
    g = torch.Generator().manual_seed(seed)
    holder = nn.Module()
    for name in ("q", "k", "v"):
        base = nn.Linear(1536, 1536)
        with torch.no_grad():
            base.weight.copy_(torch.randn(1536, 1536, generator=g) / 1536 ** 0.5)
            base.bias.copy_(torch.randn(1536, generator=g) * 0.1)
        if family == "multi":
            m = pkg.MultiLoRALinear(base, ranks=[rank, rank], alphas=[rank, rank])
            with torch.no_grad():
                for b in m.lora_b:
                    b.copy_(torch.randn(b.shape, generator=g) * 0.02)
            m = m.to(dev, torch.bfloat16)
        else:
            m = PeftLoraLinear(base.to(torch.bfloat16), {"default": (rank, float(rank))}, dtype=torch.float32)
            with torch.no_grad():
                m.lora_B["default"].weight.copy_(torch.randn(1536, rank, generator=g) * 0.02)
            m = m.to(dev)
        holder.add_module(name, m)
    if family == "peft":
        pkg.install_peft_multi_lora(holder)
    return holder, [holder.q, holder.k, holder.v]


def _adapters(m):
    if hasattr(m, "lora_A"):
        return [m.lora_A["default"].weight], [m.lora_B["default"].weight], [float(m.scaling["default"])]
    return list(m.lora_a), list(m.lora_b), list(m.scales)


@pytest.mark.parametrize("family,rank", [("multi", 128), ("peft", 256)], ids=["bf16_r128", "peft_fp32_r256"])
def test_stacked_qkv_at_the_reference_ranks(pkg, dev, family, rank):
    """q / k / v at the Wan shape (65520 tokens, 1536 -> 1536) and the reference's ranks: rank 128
    (two bf16 adapters on the generator / critic segments; the shrinks run two members, then one)
    and rank 256 with fp32 masters in the PEFT layout (one member per shrink, hi + lo parts).
    Forward: each output bit-identical to the member's own call, and within 2e-3 of the fp64
    oracle on 512 sampled rows; dX (one GEMM over the three dY and the 3·rank LoRA columns)
    within 2e-3 of the fp64 oracle's sum of the members' dX; adapter gradients against fp64
    products of the whole batch: 2e-3 for bf16 adapters (their bf16 rounding), 5e-5 for fp32
    masters (fp32-class)."""
    import numpy as np
    from oracle import multilora_oracle as O
    print(f"stacked qkv at the reference ranks: {family} rank {rank}", flush=True)
    holder, mods = _wan_qkv(pkg, dev, family, rank, seed=41)
    M = 65520
    if family == "multi":
        lengths, ids = (32760, 32760), (0, 1)
    else:
        lengths, ids = (M,), (0,)
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    gen = torch.Generator().manual_seed(42)
    x = torch.randn(M, 1536, generator=gen).to(dev, torch.bfloat16)
    dys = [torch.randn(M, 1536, generator=gen).to(dev, torch.bfloat16) for _ in range(3)]
    params = [p for m in mods for ab in _adapters(m)[:2] for p in ab]

    def run(fused):
        for p in params:
            p.grad = None
        if fused:
            pkg.fuse_shared_inputs(holder, [["q", "k", "v"]])
        xi = x.clone().requires_grad_(True)
        ys = [m(xi, routing) if family == "multi" else m(xi) for m in mods]
        torch.autograd.backward(ys, dys)
        if fused:
            assert mods[0].shared_input.launches == 1
            pkg.release_shared_inputs(holder)
        torch.cuda.synchronize()
        return [y.detach() for y in ys], xi.grad, [p.grad.clone() for p in params]

    ys_f, dx_f, gr_f = run(True)
    ys_s, _, _ = run(False)
    for a, b in zip(ys_f, ys_s):
        assert torch.equal(a, b)
    rows = np.sort(np.random.default_rng(43).choice(M, 512, replace=False))
    rows[0], rows[-1] = 0, M - 1
    ad = O.row_adapters(routing.seg_offsets, routing.adapter_ids)[rows]
    loff = [0] + [i for i in range(1, len(ad)) if ad[i] != ad[i - 1]] + [len(ad)]
    lids = [int(ad[i]) for i in loff[:-1]]
    f64 = lambda t: t.detach().double().cpu().numpy()  # noqa: E731
    xr, dx_ref = f64(x[rows]), 0.0
    for m, y, dy in zip(mods, ys_f, dys):
        As, Bs, scales = _adapters(m)
        base = m.base_layer if hasattr(m, "base_layer") else m.base
        Af, Bf = [f64(a) for a in As], [f64(b) for b in Bs]
        y_ref = O.forward_rows(np.arange(len(rows)), xr, f64(base.weight), f64(base.bias), Af, Bf, scales, loff, lids)
        assert O.rel_l2(f64(y[rows]), y_ref) <= 2e-3
        dx_ref = dx_ref + O.dx_rows(np.arange(len(rows)), f64(base.weight), Af, Bf, scales, loff, lids,
                                    f64(dy[rows]))
    assert O.rel_l2(f64(dx_f[rows]), dx_ref) <= 2e-3
    # adapter gradients against fp64 products over the whole batch (on the device)
    tol = 5e-5 if family == "peft" else 2e-3
    k = 0
    xd = x.double()
    for m, dy in zip(mods, dys):
        As, Bs, scales = _adapters(m)
        n = len(As)
        got_a, got_b = gr_f[k:k + n], gr_f[k + n:k + 2 * n]
        k += 2 * n
        for (lo, hi), a in zip(zip(routing.seg_offsets, routing.seg_offsets[1:]), routing.adapter_ids):
            xs, gu = xd[lo:hi], scales[a] * dy[lo:hi].double()
            dB_ref = gu.T @ (xs @ As[a].detach().double().T)
            dA_ref = (gu @ Bs[a].detach().double()).T @ xs
            assert got_a[a].dtype == As[a].dtype and got_b[a].dtype == Bs[a].dtype
            assert float((got_b[a].double() - dB_ref).norm() / dB_ref.norm()) <= tol
            assert float((got_a[a].double() - dA_ref).norm() / dA_ref.norm()) <= tol


def test_stacked_peft_roles_and_disabled_members(pkg, dev):
    """PEFT layers in a group: members on different active adapters (of one rank and scaling) still
    stack, each with its own adapter; with the adapters disabled every member runs the base alone
    on its own (bit-exact with an adapter-free launch). Every output equals the member's own call."""
    from peft_layout import PeftLoraLinear
    print("stacked peft disabled / different adapters", flush=True)
    holder = nn.Module()
    g = torch.Generator().manual_seed(44)
    for name in ("q", "k"):
        m = PeftLoraLinear(nn.Linear(256, 256).to(torch.bfloat16), {"a": (16, 16.0), "b": (16, 16.0)},
                           dtype=torch.bfloat16)
        with torch.no_grad():
            for n in ("a", "b"):
                m.lora_B[n].weight.copy_(torch.randn(256, 16, generator=g) * 0.05)
        holder.add_module(name, m.to(dev))
    pkg.install_peft_multi_lora(holder)
    group = pkg.fuse_shared_inputs(holder, [["q", "k"]])[0]
    x = torch.randn(2, 64, 256, generator=g).to(dev, torch.bfloat16)
    with torch.no_grad():
        yq, yk = holder.q(x), holder.k(x)
        assert group.launches == 1
        holder.k.set_adapter("b")
        yq2, yk2 = holder.q(x), holder.k(x)
        assert group.launches == 2  # q on 'a', k on 'b': one stacked call, each member its adapter
        for m in (holder.q, holder.k):
            m.enable_adapters(False)
        zq = holder.q(x)
        assert group.launches == 2  # disabled: the base alone, per member
        pkg.release_shared_inputs(holder)
        assert torch.equal(zq, pkg.multi_lora_linear(x, holder.q.base_layer.weight, holder.q.base_layer.bias,
                                                     [], [], [], pkg.SegmentRouting.single(128, pkg.BASE_ONLY)))
        for m in (holder.q, holder.k):
            m.enable_adapters(True)
        holder.k.set_adapter("a")
        assert torch.equal(yq, holder.q(x)) and torch.equal(yk, holder.k(x)) and torch.equal(yq2, yq)
        holder.k.set_adapter("b")
        assert torch.equal(yk2, holder.k(x)) and not torch.equal(yk2, yk)


def _grads_close(a, b, tol):
    for x, y in zip(a, b):
        assert float((x.double() - y.double()).norm() / y.double().norm()) <= tol


def test_livewan_self_attention_group(pkg, dev):
    """LiveWan's layout (the reference's module after install_livewan_multi_lora, fp32 a / b over the
    bf16 critic) with self_attn.q / k / v stacked: the model's output bit-identical to the unstacked
    model's, every adapter gradient within 1e-4 (the stacked reductions sum in another order);
    with the adapters off (lora_enabled(model, False)) every member runs the base alone on its own."""
    from livewan_layout import WanLike, wrap_reference_layout
    print("livewan self-attention group", flush=True)
    model = WanLike(hidden=256, ffn=512, heads=4, layers=1).to(torch.bfloat16)
    wrap_reference_layout(model, rank=32)
    model = model.to(dev)
    pkg.install_livewan_multi_lora(model)
    gen = torch.Generator().manual_seed(71)
    x = torch.randn(2, 64, 256, generator=gen).to(dev, torch.bfloat16)
    w = torch.randn(2, 64, 256, generator=gen).to(dev, torch.bfloat16)
    params = [p for p in model.parameters() if p.requires_grad]
    names = [["blocks.0.self_attn.q", "blocks.0.self_attn.k", "blocks.0.self_attn.v"]]

    def run(stacked):
        for p in params:
            p.grad = None
        groups = pkg.fuse_shared_inputs(model, names) if stacked else []
        y = model(x)
        (y.float() * w.float()).sum().backward()
        with torch.no_grad(), pkg.livewan.lora_enabled(model, False):
            y_off = model(x)
        launches = [g.launches for g in groups]
        pkg.release_shared_inputs(model)
        return y.detach(), y_off, [p.grad.clone() for p in params], launches

    y_s, off_s, g_s, launches = run(True)
    y_u, off_u, g_u, _ = run(False)
    assert launches == [1]  # the disabled pass ran its members on their own
    assert torch.equal(y_s, y_u) and torch.equal(off_s, off_u) and not torch.equal(y_s, off_s)
    _grads_close(g_s, g_u, 1e-4)


def test_native_lora_linear_group(pkg, dev):
    """The native LoRALinear (install_lora: fp32 masters over a bf16 base) at rank 128, q / k / v
    stacked: outputs bit-identical to the members' own calls, gradients within 1e-4."""
    from types import SimpleNamespace
    print("native LoRALinear group rank 128", flush=True)
    holder = nn.Module()
    gen = torch.Generator().manual_seed(72)
    for name in ("q", "k", "v"):
        lin = nn.Linear(512, 512)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(512, 512, generator=gen) / 512 ** 0.5)
        setattr(holder, name, lin.to(torch.bfloat16))
    pkg.install_lora(holder, SimpleNamespace(lora_rank=128, lora_alpha=64, target_modules=["q", "k", "v"]))
    for name in ("q", "k", "v"):
        with torch.no_grad():
            m = getattr(holder, name)
            m.b.copy_(torch.randn(m.b.shape, generator=gen) * 0.02)
    holder = holder.to(dev)
    mods = [holder.q, holder.k, holder.v]
    x = torch.randn(4096, 512, generator=gen).to(dev, torch.bfloat16)
    dys = [torch.randn(4096, 512, generator=gen).to(dev, torch.bfloat16) for _ in range(3)]
    params = [p for m in mods for p in (m.a, m.b)]

    def run(stacked):
        for p in params:
            p.grad = None
        group = pkg.fuse_shared_inputs(holder, [["q", "k", "v"]])[0] if stacked else None
        xi = x.clone().requires_grad_(True)
        ys = [m(xi) for m in mods]
        torch.autograd.backward(ys, dys)
        if stacked:
            assert group.launches == 1
            pkg.release_shared_inputs(holder)
        return [y.detach() for y in ys], xi.grad, [p.grad.clone() for p in params]

    ys_s, dx_s, g_s = run(True)
    ys_u, dx_u, g_u = run(False)
    assert all(torch.equal(a, b) for a, b in zip(ys_s, ys_u))
    assert all(g.dtype == torch.float32 for g in g_s)
    _grads_close(g_s, g_u, 1e-4)
    assert float((dx_s.double() - dx_u.double()).norm() / dx_u.double().norm()) <= 4e-3


def test_peft_role_batch_group(pkg, dev):
    """PEFT layers routed by a role batch (peft_roles_active: the teacher's rows on the base alone,
    the critic's on its adapter, H3's pattern) with q / k / v stacked: outputs bit-identical to the
    unstacked layers', adapter gradients within 2e-3 (bf16 adapters)."""
    from peft_layout import PeftLoraLinear
    print("peft role batch group", flush=True)
    holder = nn.Module()
    gen = torch.Generator().manual_seed(73)
    for name in ("q", "k", "v"):
        m = PeftLoraLinear(nn.Linear(512, 512).to(torch.bfloat16), {"critic": (64, 64.0)}, dtype=torch.bfloat16)
        with torch.no_grad():
            m.lora_B["critic"].weight.copy_(torch.randn(512, 64, generator=gen) * 0.05)
        holder.add_module(name, m.to(dev))
    pkg.install_peft_multi_lora(holder)
    mods = [holder.q, holder.k, holder.v]
    x = torch.randn(3, 200, 512, generator=gen).to(dev, torch.bfloat16)
    dys = [torch.randn(3, 200, 512, generator=gen).to(dev, torch.bfloat16) for _ in range(3)]
    params = [p for m in mods for p in (m.lora_A["critic"].weight, m.lora_B["critic"].weight)]
    rb = pkg.RoleBatch([("teacher", 2), ("critic", 1)])

    def run(stacked):
        for p in params:
            p.grad = None
        group = pkg.fuse_shared_inputs(holder, [["q", "k", "v"]])[0] if stacked else None
        xi = x.clone().requires_grad_(True)
        with pkg.peft_roles_active(holder, rb, base_roles=("teacher",)):
            ys = [m(xi) for m in mods]
        torch.autograd.backward(ys, dys)
        if stacked:
            assert group.launches == 1
            pkg.release_shared_inputs(holder)
        return [y.detach() for y in ys], [p.grad.clone() for p in params]

    ys_s, g_s = run(True)
    ys_u, g_u = run(False)
    assert all(torch.equal(a, b) for a, b in zip(ys_s, ys_u))
    _grads_close(g_s, g_u, 2e-3)


@pytest.mark.parametrize("split", [False, True], ids=["bf16", "fp32_masters"])
@pytest.mark.parametrize("widths", [(256, 512, 768), (512, 512, 512)], ids=["mixed_widths", "stacked"])
def test_rank128_many_segments(pkg, dev, split, widths):
    """Rank 128 with 131 segments (two calls of the kernels' 128-segment tables, base-only segments
    between), for members of different widths (SharedInputMultiLoRAFunction: the shared shrinks in
    256-column slices, one GEMM per member, the members' dX accumulated in the dX GEMMs'
    epilogues) and of one width (StackedLinearsFunction): each output bit-identical to the
    member's own call; dX within 2e-3 (one stacked GEMM) or √G·2e-3 (G accumulating GEMMs) of the
    fp64 sum of the members' dX; adapter gradients within 2e-3 (bf16) / 1e-4 (fp32 masters) of
    the per-member calls'."""
    print(f"rank 128, 131 segments, widths {widths}, split={split}", flush=True)
    g = torch.Generator().manual_seed(74)
    holder = nn.Module()
    mods = []
    for i, N in enumerate(widths):
        base = nn.Linear(512, N)
        with torch.no_grad():
            base.weight.copy_(torch.randn(N, 512, generator=g) / 512 ** 0.5)
        m = pkg.MultiLoRALinear(base, ranks=[128, 128], alphas=[64, 256])
        with torch.no_grad():
            for b in m.lora_b:
                b.copy_(torch.randn(b.shape, generator=g) * 0.03)
        m = m.to(dev, torch.bfloat16)
        if split:
            for p in (*m.lora_a, *m.lora_b):
                p.data = p.data.float()
        holder.add_module(f"m{i}", m)
        mods.append(m)
    lengths = tuple(32 + (7 * i) % 50 for i in range(131))
    ids = tuple(-1 if i % 5 == 4 else i % 2 for i in range(131))
    routing = pkg.SegmentRouting.from_lengths(lengths, ids)
    M = sum(lengths)
    x = torch.randn(M, 512, generator=g).to(dev, torch.bfloat16)
    dys = [torch.randn(M, N, generator=g).to(dev, torch.bfloat16) for N in widths]
    params = [p for m in mods for p in (*m.lora_a, *m.lora_b)]

    def run(fused):
        for p in params:
            p.grad = None
        if fused:
            pkg.fuse_shared_inputs(holder, [["m0", "m1", "m2"]])
        xi = x.clone().requires_grad_(True)
        ys = [m(xi, routing) for m in mods]
        torch.autograd.backward(ys, dys)
        if fused:
            assert mods[0].shared_input.launches == 1
            pkg.release_shared_inputs(holder)
        return [y.detach() for y in ys], xi.grad, [p.grad.clone() for p in params]

    ys_f, dx_f, gr_f = run(True)
    ys_s, dx_s, gr_s = run(False)
    for a, b in zip(ys_f, ys_s):
        assert torch.equal(a, b)
    with torch.no_grad():
        dx_ref = torch.zeros(M, 512, dtype=torch.float64, device=dev)
        for m, dy in zip(mods, dys):
            dyd = dy.double()
            dx_ref += dyd @ m.base.weight.double()
            for (r0, r1), a in zip(zip(routing.seg_offsets, routing.seg_offsets[1:]), routing.adapter_ids):
                if a >= 0 and r1 > r0:
                    dx_ref[r0:r1] += m.scales[a] * (dyd[r0:r1] @ m.lora_b[a].double()) @ m.lora_a[a].double()
    # one rounding of the sum in the stacked dX GEMM; one per accumulating call (G of them) when
    # the members' widths differ
    tol = 2e-3 if len(set(widths)) == 1 else 2e-3 * len(widths) ** 0.5
    assert float((dx_f.double() - dx_ref).norm() / dx_ref.norm()) <= tol
    _grads_close(gr_f, gr_s, 1e-4 if split else 2e-3)
    assert all(p.dtype == (torch.float32 if split else torch.bfloat16) for p in gr_f)
