"""Host-side logic of the multi-role call site on CPU: RoleBatch routing, fuse_roles'
aliasing checks (the shared frozen construction's invariants,
tests/test_training_construction.py:79-94) and the active-batch context. No kernel runs."""
import copy

import pytest
import torch
from torch import nn

from toy_dit import TARGETS, make_roles


# ---------------------------------------------------------------- RoleBatch

def test_role_batch_routing_scales_rows_per_sample(pkg):
    rb = pkg.RoleBatch([("teacher", 2), ("fake", 1), ("gen", 1)])
    assert rb.samples == 4
    for per in (1, 7, 77):
        r = rb.routing(4 * per, {"fake": 0, "gen": 1})
        assert r.seg_offsets == (0, 2 * per, 3 * per, 4 * per)
        assert r.adapter_ids == (-1, 0, 1)
    # a role without an adapter at this linear is base-only; equal neighbours form one segment
    r = rb.routing(40, {"gen": 0})
    assert r.seg_offsets == (0, 30, 40) and r.adapter_ids == (-1, 0)
    r = pkg.RoleBatch([("fake", 1), ("fake", 2), ("teacher", 0), ("gen", 1)]).routing(8, {"fake": 1, "gen": 1})
    assert r.seg_offsets == (0, 8) and r.adapter_ids == (1,)
    assert rb.routing(0, {}).num_rows == 0


def test_role_batch_rejects_bad_shapes(pkg):
    rb = pkg.RoleBatch([("teacher", 2), ("fake", 1)])
    with pytest.raises(ValueError, match="do not split into 3 samples"):
        rb.routing(10, {})
    with pytest.raises(ValueError):
        pkg.RoleBatch([])
    with pytest.raises(ValueError):
        pkg.RoleBatch([("a", -1)])
    a, b = torch.zeros(2, 5), torch.ones(1, 5)
    t = rb.cat([a, b])
    assert t.shape == (3, 5)
    u, v = rb.split(t)
    assert torch.equal(u, a) and torch.equal(v, b)
    with pytest.raises(ValueError, match="role 'fake' has 1 samples"):
        rb.cat([a, torch.ones(2, 5)])
    with pytest.raises(ValueError):
        rb.split(torch.zeros(4, 5))


# ---------------------------------------------------------------- fuse_roles

def test_fuse_roles_shares_every_tensor(pkg):
    teacher, fake, gen = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=4)
    fused = pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})
    assert fused.role_names == ("teacher", "fake", "gen")
    for t in TARGETS:
        m = fused.get_submodule(t)
        assert isinstance(m, pkg.MultiLoRALinear)
        assert m.role_ids == {"fake": 0, "gen": 1}
        assert m.base.weight is teacher.get_submodule(t).weight
        assert m.base.bias is fake.get_submodule(t).base.bias
        assert m.lora_a[0] is fake.get_submodule(t).lora_a and m.lora_b[1] is gen.get_submodule(t).lora_b
        assert m.scales == [fake.get_submodule(t).scale, gen.get_submodule(t).scale]
    assert fused.norm1.weight is teacher.norm1.weight and fused.shift is teacher.shift
    frozen = {id(p) for p in teacher.parameters()}
    lora = {id(p) for role in (fake, gen) for p in role.parameters() if p.requires_grad}
    assert {id(p) for p in fused.parameters()} == frozen | lora
    assert all(p.requires_grad == (id(p) in lora) for p in fused.parameters())
    # the roles themselves are untouched
    assert isinstance(fake.q, pkg.TrainableLowRankLinear) and type(teacher.q) is nn.Linear


def test_fuse_roles_partial_targets(pkg):
    teacher, fake, gen = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=4, fake_targets=["q", "ffn.2"],
                                    gen_targets=["q", "v"])
    fused = pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})
    assert fused.q.role_ids == {"fake": 0, "gen": 1}
    assert fused.v.role_ids == {"gen": 0} and fused.ffn[2].role_ids == {"fake": 0}
    assert type(fused.k) is nn.Linear and fused.k.weight is teacher.k.weight
    rb = pkg.RoleBatch([("teacher", 1), ("fake", 1), ("gen", 1)])
    assert fused.v.active_roles is None
    assert rb.routing(30, fused.v.role_ids).adapter_ids == (-1, 0)


def test_fuse_roles_fails_closed(pkg):
    teacher, fake, gen = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=4)
    unshared = copy.deepcopy(teacher)  # same values, separate frozen storage
    with pytest.raises(ValueError, match="multi-role call: frozen parameter 'norm1.weight' of role 'copy' is not shared"):
        pkg.fuse_roles({"teacher": teacher, "copy": unshared})
    trains = copy.deepcopy(teacher, {id(p): p for p in teacher.parameters() if p is not teacher.norm1.weight})
    trains.norm1.weight.requires_grad_(True)
    with pytest.raises(ValueError, match="trains 'norm1.weight', which is not a LoRA adapter"):
        pkg.fuse_roles({"teacher": teacher, "x": trains})
    other_buf = copy.deepcopy(teacher, {id(p): p for p in teacher.parameters()})
    other_buf.shift.add_(1)
    with pytest.raises(ValueError, match="buffer 'shift' of role 'x' differs"):
        pkg.fuse_roles({"teacher": teacher, "x": other_buf})
    other = copy.deepcopy(teacher, {id(p): p for p in teacher.parameters()})
    other.extra = nn.Identity()
    with pytest.raises(ValueError, match="different module structure"):
        pkg.fuse_roles({"teacher": teacher, "x": other})
    with pytest.raises(ValueError):
        pkg.fuse_roles({})


def test_roles_active_sets_and_restores(pkg):
    teacher, fake, gen = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=4)
    fused = pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})
    rb = pkg.RoleBatch([("teacher", 2), ("fake", 1)])
    inner = pkg.RoleBatch([("gen", 3)])
    mods = [m for m in fused.modules() if isinstance(m, pkg.MultiLoRALinear)]
    with pkg.roles_active(fused, rb):
        assert all(m.active_roles is rb for m in mods)
        with pkg.roles_active(fused, inner):
            assert all(m.active_roles is inner for m in mods)
        assert all(m.active_roles is rb for m in mods)
    assert all(m.active_roles is None for m in mods)
    with pytest.raises(ValueError, match="unknown role 'critic'"):
        with pkg.roles_active(fused, pkg.RoleBatch([("critic", 1)])):
            pass
    with pytest.raises(ValueError, match="no routing given and no role batch active"):
        fused.q(torch.zeros(1, 4, 32))
    with pytest.raises(ValueError, match="no fused multi-role linear"):
        with pkg.roles_active(teacher, rb):
            pass
