"""The PEFT call site on the CPU: layer recognition, install / uninstall, routing of mixed
batches and role batches, and the fail-closed checks (all raise before any device work)."""
import pytest
import torch
from torch import nn

from peft_layout import PeftLoraLinear, peft_model


def test_install_finds_peft_layers_and_restores(pkg):
    from dmd_system_amd import peft_site as P
    model = peft_model([(16, 32), (32, 16)], {"generator": (4, 4.0), "critic": (8, 16.0)})
    assert P.is_peft_lora_linear(model[0]) and not P.is_peft_lora_linear(model[1])
    names = P.install_peft_multi_lora(model)
    assert names == ["0", "2"]
    assert model[0].forward.__func__ is P._peft_forward
    P.uninstall_peft_multi_lora(model)
    assert "forward" not in model[0].__dict__
    with pytest.raises(ValueError, match="no PEFT LoRA Linear layers"):
        P.install_peft_multi_lora(nn.Sequential(nn.Linear(2, 2)))


def test_mixed_batch_routing(pkg):
    from dmd_system_amd import peft_site as P
    x = torch.zeros(5, 7, 16)
    names, r = P._mixed_routing(x, ["b", "b", "__base__", "a", "b"])
    assert names == ["b", "a"]
    assert r.seg_offsets == (0, 14, 21, 28, 35) and r.adapter_ids == (0, -1, 1, 0)
    with pytest.raises(RuntimeError, match="4 entries for a batch of 5"):
        P._mixed_routing(x, ["a"] * 4)


def test_fail_closed_before_any_device_work(pkg):
    from dmd_system_amd import peft_site as P
    model = peft_model([(16, 16)], {"generator": (4, 4.0), "critic": (4, 4.0)})
    P.install_peft_multi_lora(model)
    layer = model[0]
    x = torch.randn(2, 3, 16, dtype=torch.bfloat16)
    layer.set_adapter(["generator", "critic"])
    with pytest.raises(RuntimeError, match="one active adapter"):
        layer(x)
    layer.set_adapter("generator")
    layer.merged_adapters = ["generator"]
    with pytest.raises(RuntimeError, match="merged"):
        layer(x)
    layer.merged_adapters = []
    layer.lora_variant["generator"] = object()
    with pytest.raises(RuntimeError, match="variant"):
        layer(x)
    layer.lora_variant.clear()
    layer.lora_dropout["generator"] = nn.Dropout(0.1)
    with pytest.raises(RuntimeError, match="dropout"):
        layer(x)
    layer.lora_dropout["generator"].eval()  # inactive dropout is the identity: allowed (then: no CPU path)
    with pytest.raises(RuntimeError, match="ROCm device only"):
        layer(x)
    layer.lora_dropout["generator"] = nn.Identity()
    with pytest.raises(RuntimeError, match="variant keyword"):
        layer(x, alora_offsets=[1])
    layer.enable_adapters(False)
    with pytest.raises(RuntimeError, match="disabled"):
        layer(x, adapter_names=["generator", "critic"])
    # disabled AND merged: the base weight carries the adapter, so the base-only branch would
    # silently include it; the merged check comes first (wan13b_lora_cast.py:185-189)
    layer.merged_adapters = ["generator"]
    with pytest.raises(RuntimeError, match="merged"):
        layer(x)


def test_roles_need_known_names(pkg):
    from dmd_system_amd import peft_site as P
    model = peft_model([(16, 16)], {"generator": (4, 4.0), "critic": (4, 4.0)})
    with pytest.raises(ValueError, match="install_peft_multi_lora first"):
        with P.peft_roles_active(model, pkg.RoleBatch([("critic", 1)])):
            pass
    P.install_peft_multi_lora(model)
    with pytest.raises(ValueError, match="'teacher' is neither"):
        with P.peft_roles_active(model, pkg.RoleBatch([("teacher", 1), ("critic", 1)])):
            pass
    with P.peft_roles_active(model, pkg.RoleBatch([("teacher", 2), ("critic", 1)]), base_roles=("teacher",)):
        assert model[0].__dict__["peft_roles"][1] == ("teacher",)
    assert "peft_roles" not in model[0].__dict__
