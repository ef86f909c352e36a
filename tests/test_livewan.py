"""LiveWan's critic LoRA on the CPU: the module layout and initialisation, inject_lora's
contract (wanstreamer/lora.py:34-56), lora_enabled / set_lora / lora_state_dict, installing on
modules of the reference's layout, fuse_roles with a base-only teacher role, the restore
identity, and that no CPU path exists. No kernel runs."""
import pytest
import torch
from torch import nn

from livewan_layout import RefLayoutLoRA, WanLike, wrap_reference_layout


def test_module_layout_and_init(pkg):
    L = pkg.livewan
    torch.manual_seed(0)
    m = L.LiveWanLoRALinear(nn.Linear(512, 384), rank=32)
    assert m.rank == 32 and m.scale == 1.0 and m.enabled is True
    assert m.a.shape == (32, 512) and m.b.shape == (384, 32)
    assert m.a.dtype == torch.float32 and not m.b.any()
    assert abs(float(m.a.detach().std()) - 1 / 32) < 0.1 / 32  # N(0, 1/rank) std, as wanstreamer/lora.py:19
    assert not m.base.weight.requires_grad and not m.base.bias.requires_grad
    assert L.LiveWanLoRALinear(nn.Linear(8, 8), rank=4, alpha=8).scale == 2.0
    assert set(m.state_dict()) == {"base.weight", "base.bias", "a", "b"}
    assert L.is_livewan_lora_linear(m) and L.is_livewan_lora_linear(RefLayoutLoRA(nn.Linear(8, 8), 4))
    assert not L.is_livewan_lora_linear(nn.Linear(8, 8))
    assert not L.is_livewan_lora_linear(pkg.TrainableLowRankLinear(nn.Linear(8, 8), rank=4, alpha=4))


def test_inject_lora_contract(pkg):
    L = pkg.livewan
    model = WanLike(hidden=64, ffn=128, heads=2, layers=3).to(torch.bfloat16)
    params, n, total = L.inject_lora(model, rank=8)
    assert n == 3 * 6
    assert total == sum(p.numel() for p in params) == 3 * (4 * 2 * 64 * 8 + 64 * 8 + 128 * 8 + 128 * 8 + 64 * 8)
    assert all(p.dtype == torch.float32 for p in params)
    assert isinstance(model.blocks[0].ffn[0], L.LiveWanLoRALinear)
    assert model.blocks[0].ffn[0].base.weight.dtype == torch.bfloat16
    assert not any(p.requires_grad for name, p in model.named_parameters() if ".base." in name)
    # a second call wraps nothing more
    assert L.inject_lora(model, rank=8)[1] == 0
    keys = set(L.lora_state_dict(model))
    assert "blocks.1.self_attn.q.a" in keys and "blocks.2.ffn.2.b" in keys and len(keys) == 2 * 18


def test_lora_enabled_restores_each_flag(pkg):
    L = pkg.livewan
    model = wrap_reference_layout(WanLike(hidden=32, ffn=64, heads=2, layers=2), rank=4)
    mods = [m for m in model.modules() if isinstance(m, RefLayoutLoRA)]
    mods[3].enabled = False
    with L.lora_enabled(model, False):
        assert not any(m.enabled for m in mods)
    assert [m.enabled for m in mods] == [i != 3 for i in range(len(mods))]
    L.set_lora(model, True)
    assert all(m.enabled for m in mods)


def test_install_on_reference_layout_and_uninstall(pkg):
    L = pkg.livewan
    model = wrap_reference_layout(WanLike(hidden=32, ffn=64, heads=2, layers=2).to(torch.bfloat16), rank=4)
    names = pkg.install_livewan_multi_lora(model)
    assert len(names) == 12 and names[0] == "blocks.0.self_attn.q"
    lin = model.blocks[0].self_attn.q
    assert isinstance(lin, RefLayoutLoRA) and lin.forward.__func__ is L.livewan_forward
    with pytest.raises(RuntimeError, match="ROCm device only"):  # no CPU path
        lin(torch.randn(3, 32, dtype=torch.bfloat16))
    pkg.uninstall_livewan_multi_lora(model)
    assert "forward" not in lin.__dict__
    assert lin(torch.randn(3, 32, dtype=torch.bfloat16)).shape == (3, 32)  # the module's own forward again
    with pytest.raises(ValueError, match="no LiveWan LoRA modules"):
        pkg.install_livewan_multi_lora(nn.Sequential(nn.Linear(2, 2)))


def test_fuse_roles_with_base_only_teacher(pkg):
    model = wrap_reference_layout(WanLike(hidden=32, ffn=64, heads=2, layers=2), rank=8)
    fused = pkg.fuse_roles({"teacher": model, "critic": model}, base_roles=("teacher",))
    lin = fused.blocks[1].ffn[2]
    assert isinstance(lin, pkg.MultiLoRALinear)
    assert lin.role_ids == {"critic": 0}
    assert lin.lora_a[0] is model.blocks[1].ffn[2].a and lin.base.weight is model.blocks[1].ffn[2].base.weight
    rb = pkg.RoleBatch([("teacher", 2), ("critic", 1)])
    lin.active_roles = rb
    r = lin.role_routing(3 * 5)
    assert r.seg_offsets == (0, 10, 15) and r.adapter_ids == (-1, 0)
    model.blocks[1].ffn[2].enabled = False  # lora_enabled(critic, False) at call time: base only
    assert lin.role_routing(15).adapter_ids == (-1,)
    with pytest.raises(ValueError, match="two adapter roles"):
        pkg.fuse_roles({"a": model, "b": model})
    with pytest.raises(ValueError, match="base roles"):
        pkg.fuse_roles({"critic": model}, base_roles=("teacher",))
    # a teacher with its own plain Linears over the same frozen tensors fuses as before
    teacher = WanLike(hidden=32, ffn=64, heads=2, layers=2)
    for blk_t, blk_c in zip(teacher.blocks, model.blocks):
        for name in ("self_attn.q", "self_attn.k", "self_attn.v", "self_attn.o", "ffn.0", "ffn.2"):
            parent, _, leaf = name.rpartition(".")
            src = blk_c.get_submodule(name).base
            dst_parent = blk_t.get_submodule(parent)
            if leaf.isdigit():
                dst_parent[int(leaf)] = src
            else:
                setattr(dst_parent, leaf, src)
    teacher.requires_grad_(False)
    fused2 = pkg.fuse_roles({"teacher": teacher, "critic": model})
    assert fused2.blocks[0].self_attn.q.role_ids == {"critic": 0}


def test_restore_identity(pkg):
    ident = pkg.restore_identity()["mi355x_multi_lora"]
    assert ident["abi_version"] == pkg._lib.ABI_VERSION
    assert ident["kernel_source_sha256"] == pkg._lib.expected_source_hash()
    assert len(ident["python_source_sha256"]) == 64 and ident["arch"] == "gfx950"
    import json
    json.dumps(ident)  # the reference digests model metadata as JSON
