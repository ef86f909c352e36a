"""GPU parity of the multi-role call site: the roles' samples concatenated and run once
through ``fuse_roles``' module tree give what each role's own model gives on its own
samples (the reference's per-role calls, training/dmd.py:324-345 and
runtime/livewan_crossscale_worker.py:2614-2645), forward and backward.

Tolerances: a fused linear against the same kernel called per role is bit-exact (a row's
result does not depend on the other segments of its call); whole blocks with adapter
roles within 1e-3 rel-L2 (the torch attention in between runs at another batch size);
the teacher, whose own model uses torch's bf16 nn.Linear, within the bf16 bound 2e-3.
"""
import pytest
import torch

from toy_dit import inputs, make_roles, rel_l2

pytestmark = pytest.mark.gpu

H, FFN, HEADS, RANK = 256, 512, 4, 16


def _roles(pkg, dev, **kw):
    teacher, fake, gen = make_roles(pkg, hidden=H, ffn=FFN, heads=HEADS, rank=RANK, device=dev,
                                    dtype=torch.bfloat16, **kw)
    return teacher, fake, gen, pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})


@pytest.mark.parametrize("name,tokens", [("q", 77), ("cross.k", 13), ("ffn.0", 64), ("ffn.2", 5)])
def test_fused_linear_is_bit_exact_per_role(pkg, dev, name, tokens):
    print(f"fused linear {name} tokens {tokens}", flush=True)
    teacher, fake, gen, fused = _roles(pkg, dev)
    lin = fused.get_submodule(name)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(4, tokens, lin.base.in_features, generator=g).to(dev, torch.bfloat16)
    rb = pkg.RoleBatch([("teacher", 2), ("fake", 1), ("gen", 1)])
    with torch.no_grad():
        with pkg.roles_active(fused, rb):
            y = lin(x)
        yt, yf, yg = rb.split(y)
        rows = 2 * tokens
        base_only = lin(x[:2], pkg.SegmentRouting.single(rows, pkg.BASE_ONLY))
        assert torch.equal(yt, base_only)
        assert torch.equal(yf, fake.get_submodule(name)(x[2:3]))
        assert torch.equal(yg, gen.get_submodule(name)(x[3:4]))
        assert rel_l2(yt, teacher.get_submodule(name)(x[:2])) <= 2e-3
        # the adapters act: every role's rows differ from the others'
        assert not torch.equal(yf, lin(x[2:3], pkg.SegmentRouting.single(tokens, pkg.BASE_ONLY)))


def test_fused_block_forward_matches_roles(pkg, dev):
    print("fused block forward", flush=True)
    teacher, fake, gen, fused = _roles(pkg, dev)
    x, c = inputs(5, 64, 16, H, dev, torch.bfloat16, seed=3)
    rb = pkg.RoleBatch([("teacher", 2), ("fake", 2), ("gen", 1)])
    with torch.no_grad():
        with pkg.roles_active(fused, rb):
            yt, yf, yg = rb.split(fused(x, c))
        rt = teacher(x[:2], c[:2])
        rf = fake(x[2:4], c[2:4])
        rg = gen(x[4:], c[4:])
    assert rel_l2(yf, rf) <= 1e-3 and rel_l2(yg, rg) <= 1e-3
    assert rel_l2(yt, rt) <= 2e-3
    assert rel_l2(yf, rt[:1].expand_as(yf)) > 1e-2  # different samples, different adapters


def test_fused_block_partial_targets(pkg, dev):
    print("fused block partial targets", flush=True)
    teacher, fake, gen, fused = _roles(pkg, dev, fake_targets=["q", "cross.v", "ffn.2"], gen_targets=["k", "o"])
    x, c = inputs(3, 32, 8, H, dev, torch.bfloat16, seed=4)
    rb = pkg.RoleBatch([("gen", 1), ("teacher", 1), ("fake", 1)])
    with torch.no_grad():
        with pkg.roles_active(fused, rb):
            yg, yt, yf = rb.split(fused(x, c))
        assert rel_l2(yg, gen(x[:1], c[:1])) <= 1e-3
        assert rel_l2(yt, teacher(x[1:2], c[1:2])) <= 2e-3
        assert rel_l2(yf, fake(x[2:], c[2:])) <= 1e-3


def test_fused_block_backward_matches_roles(pkg, dev):
    """One backward through the batched call gives each role's adapters the gradients its
    own call gives them; the teacher's rows give the adapters nothing."""
    print("fused block backward", flush=True)
    teacher, fake, gen, fused = _roles(pkg, dev)
    x, c = inputs(4, 48, 12, H, dev, torch.bfloat16, seed=6)
    w = torch.randn(4, 48, H, generator=torch.Generator().manual_seed(7)).to(dev, torch.bfloat16)
    rb = pkg.RoleBatch([("teacher", 1), ("fake", 2), ("gen", 1)])
    adapters = [p for role in (fake, gen) for p in role.parameters() if p.requires_grad]

    def grads():
        out = [p.grad.clone() for p in adapters]
        for p in adapters:
            p.grad = None
        return out

    xb = x.clone().requires_grad_(True)
    with pkg.roles_active(fused, rb):
        y = fused(xb, c)
    (y.float() * w.float()).sum().backward()
    batched, dx_batched = grads(), xb.grad

    dxs = []
    for role, sl in ((teacher, slice(0, 1)), (fake, slice(1, 3)), (gen, slice(3, 4))):
        xr = x[sl].clone().requires_grad_(True)
        (role(xr, c[sl]).float() * w[sl].float()).sum().backward()
        dxs.append(xr.grad)
    separate = grads()
    for a, b in zip(batched, separate):
        assert rel_l2(a, b) <= 2e-3
    assert all(a.abs().sum() > 0 for a in batched)
    assert rel_l2(dx_batched[1:], torch.cat(dxs[1:])) <= 2e-3
    assert rel_l2(dx_batched[:1], dxs[0]) <= 2e-3


@pytest.mark.parametrize("fmt", ["peft", "diffsynth"])
def test_exported_adapters_reload_bit_exact(pkg, dev, fmt):
    """A role's adapters exported from the fused tree and imported into a fresh copy of the
    role give the same outputs through the HIP path (power-of-two scale: exact in both formats)."""
    print(f"adapter round trip {fmt}", flush=True)
    teacher, fake, gen, fused = _roles(pkg, dev)
    state, config = pkg.export_adapters(fused, role="fake", fmt=fmt)
    teacher2, fake2, _ = make_roles(pkg, hidden=H, ffn=FFN, heads=HEADS, rank=RANK, device=dev,
                                    dtype=torch.bfloat16, seed=7)
    pkg.import_adapters(fake2, state, config, fmt=fmt)
    x, c = inputs(2, 32, 8, H, dev, torch.bfloat16, seed=11)
    with torch.no_grad():
        for p, q in zip(teacher.parameters(), teacher2.parameters()):
            q.copy_(p)  # the same frozen base (seed 7 drew another one)
        assert torch.equal(fake(x, c), fake2(x, c))
