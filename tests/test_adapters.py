"""Adapter state formats on CPU: PEFT (a PeftModel's get_peft_model_state_dict layout,
scaling in the config), PEFT's in-module keys (training/wan_public.py:213), the diffusers
conversion H3 saves (backends/training/minimax_h3/model.py:441-449) and DiffSynth (scale baked
into B; reference/diffsynth_h3_cached/h3_dmd2.py:177-183): round trips, per-role export of a
multi-role tree, the fail-closed checks, and what each format means numerically. No kernel
runs."""
import math

import pytest
import torch
from torch import nn

from toy_dit import TARGETS, make_roles


def _model(pkg, rank=4, alpha=8.0, seed=0):
    torch.manual_seed(seed)
    m = nn.Sequential()
    m.add_module("q", nn.Linear(16, 24))
    m.add_module("ffn", nn.Linear(24, 16))
    pkg.trainable_scope(m, {"mode": "lora", "rank": rank, "alpha": alpha, "targets": ["q", "ffn"]})
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, pkg.TrainableLowRankLinear):
                mod.lora_b.normal_(0, 0.1)
    return m


@pytest.mark.parametrize("fmt", ["peft", "diffsynth"])
def test_round_trip_is_exact(pkg, fmt):
    src, dst = _model(pkg, seed=0), _model(pkg, seed=1)
    state, config = pkg.export_adapters(src, fmt=fmt)
    if fmt == "peft":
        assert set(state) == {f"base_model.model.{n}.lora_{p}.weight" for n in ("q", "ffn") for p in "AB"}
        assert config["r"] == 4 and config["lora_alpha"] == 8.0 and config["target_modules"] == ["ffn", "q"]
    else:
        assert set(state) == {f"{n}.lora_{p}.weight" for n in ("q", "ffn") for p in "AB"}
    assert sorted(pkg.import_adapters(dst, state, config, fmt=fmt)) == ["ffn", "q"]
    for a, b in zip(src.parameters(), dst.parameters()):
        if a.requires_grad:
            assert torch.equal(a, b)


def test_formats_mean_what_their_loaders_compute(pkg):
    """PEFT: y = base(x) + (alpha/r)·B(A(x)); DiffSynth: y = base(x) + B'(A(x)), B' = B·alpha/r."""
    m = _model(pkg, rank=4, alpha=6.0)
    x = torch.randn(5, 16, dtype=torch.float64)
    mod = m.q
    want = x @ mod.base.weight.double().T + mod.base.bias.double() \
        + mod.scale * (x @ mod.lora_a.double().T) @ mod.lora_b.double().T
    peft, cfg = pkg.export_adapters(m, fmt="peft")
    A, B = peft["base_model.model.q.lora_A.weight"].double(), peft["base_model.model.q.lora_B.weight"].double()
    y = x @ mod.base.weight.double().T + mod.base.bias.double() + cfg["lora_alpha"] / cfg["r"] * (x @ A.T) @ B.T
    assert torch.allclose(y, want, rtol=0, atol=1e-12)
    ds, _ = pkg.export_adapters(m, fmt="diffsynth")
    A, B = ds["q.lora_A.weight"].double(), ds["q.lora_B.weight"].double()
    y = x @ mod.base.weight.double().T + mod.base.bias.double() + (x @ A.T) @ B.T
    assert torch.allclose(y, want, rtol=1e-6, atol=1e-7)


def test_multi_role_tree_exports_each_role(pkg):
    teacher, fake, gen = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=4, fake_targets=["q", "k", "ffn.2"])
    fused = pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})
    sf, cf = pkg.export_adapters(fused, role="fake")
    sg, _ = pkg.export_adapters(fused, role="gen")
    assert cf["target_modules"] == ["ffn.2", "k", "q"] and cf["role"] == "fake"
    assert len(sg) == 2 * len(TARGETS)
    assert torch.equal(sf["base_model.model.k.lora_B.weight"], fake.k.lora_b.detach())
    with pytest.raises(ValueError, match="pass role="):
        pkg.export_adapters(fused)
    with pytest.raises(ValueError, match="no LoRA adapter for role 'teacher'"):
        pkg.export_adapters(fused, role="teacher")
    # the per-role state loads into the role's own (unfused) model and back into the tree
    teacher2, fake2, gen2 = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=4, seed=5, fake_targets=["q", "k", "ffn.2"])
    pkg.import_adapters(fake2, sf, cf)
    assert torch.equal(fake2.ffn[2].lora_a, fake.ffn[2].lora_a)
    fused2 = pkg.fuse_roles({"teacher": teacher2, "fake": fake2, "gen": gen2})
    pkg.import_adapters(fused2, sg, role="gen")
    assert torch.equal(gen2.cross.v.lora_b, gen.cross.v.lora_b)


def test_import_fails_closed(pkg):
    m = _model(pkg)
    state, config = pkg.export_adapters(m)
    bad = dict(state)
    bad["base_model.model.q.lora_A.weight"] = torch.zeros(5, 16)
    with pytest.raises(ValueError, match="adapter state: 'q': lora_A"):
        pkg.import_adapters(m, bad, config)
    bad = {k: v for k, v in state.items() if ".q." not in k}
    with pytest.raises(ValueError, match="missing"):
        pkg.import_adapters(m, bad, config)
    assert pkg.import_adapters(m, bad, config, strict=False) == ["ffn"]
    with pytest.raises(ValueError, match="unused keys"):
        pkg.import_adapters(m, {**state, "base_model.model.other.lora_A.weight": torch.zeros(1)}, config)
    with pytest.raises(ValueError, match="config scaling"):
        pkg.import_adapters(m, state, {**config, "lora_alpha": 4.0})
    with pytest.raises(ValueError, match="config rank"):
        pkg.import_adapters(m, state, {**config, "r": 8, "lora_alpha": 16.0})
    bad = dict(state)
    bad["base_model.model.ffn.lora_B.weight"] = torch.full((16, 4), math.inf)
    with pytest.raises(ValueError, match="non-finite"):
        pkg.import_adapters(m, bad, config)
    with pytest.raises(ValueError, match="format"):
        pkg.export_adapters(m, fmt="lycoris")


@pytest.mark.parametrize("fmt", ["peft", "diffsynth"])
def test_safetensors_files(pkg, tmp_path, fmt):
    src, dst = _model(pkg, seed=2), _model(pkg, seed=3)
    pkg.save_adapters(str(tmp_path), src, fmt=fmt)
    assert (tmp_path / "adapter_model.safetensors").exists() and (tmp_path / "adapter_config.json").exists()
    assert sorted(pkg.load_adapters(str(tmp_path), dst)) == ["ffn", "q"]
    assert torch.equal(src.q.lora_b, dst.q.lora_b) and torch.equal(src.ffn.lora_a, dst.ffn.lora_a)


# ------------------------------------------------------------ PEFT in-module and diffusers layouts

def test_peft_module_round_trip_and_real_layout(pkg):
    """"peft_module": the keys PEFT's layers hold inside the model (wan_public.py:213, adapter
    'default'); a state dict taken from a PEFT-layout model (tests/peft_layout.py) imports into the
    drop-in modules over the same base, and the imported module computes what the PEFT layer does."""
    from peft_layout import PeftLoraLinear
    src, dst = _model(pkg, seed=0), _model(pkg, seed=1)
    state, config = pkg.export_adapters(src, fmt="peft_module", with_base=True)
    assert set(state) >= {"q.lora_A.default.weight", "q.lora_B.default.weight", "q.base_layer.weight",
                          "q.base_layer.bias", "ffn.lora_A.default.weight"}
    assert config["adapter_name"] == "default" and config["r"] == 4
    with pytest.raises(ValueError, match="differs from the module's frozen base"):
        pkg.import_adapters(dst, state, config, fmt="peft_module")  # dst has another base (seed 1)
    with torch.no_grad():
        for n in ("q", "ffn"):
            dst.get_submodule(n).base.weight.copy_(src.get_submodule(n).base.weight)
            dst.get_submodule(n).base.bias.copy_(src.get_submodule(n).base.bias)
    assert sorted(pkg.import_adapters(dst, state, config, fmt="peft_module")) == ["ffn", "q"]
    for a, b in zip(src.parameters(), dst.parameters()):
        assert torch.equal(a, b)
    # a PEFT-layout layer's own state dict, with a named adapter
    torch.manual_seed(5)
    peft = PeftLoraLinear(nn.Linear(16, 24), {"critic": (4, 8.0)})
    with torch.no_grad():
        peft.lora_B["critic"].weight.normal_(0, 0.1)
    holder = nn.Module()
    holder.q = peft
    sd = holder.state_dict()
    assert set(sd) == {"q.base_layer.weight", "q.base_layer.bias", "q.lora_A.critic.weight", "q.lora_B.critic.weight"}
    mine = nn.Sequential()
    mine.add_module("q", nn.Linear(16, 24))
    with torch.no_grad():
        mine.q.weight.copy_(peft.base_layer.weight)
        mine.q.bias.copy_(peft.base_layer.bias)
    pkg.trainable_scope(mine, {"mode": "lora", "rank": 4, "alpha": 8.0, "targets": ["q"]})
    assert pkg.import_adapters(mine, sd, None, fmt="peft_module", adapter="critic") == ["q"]
    x = torch.randn(5, 16)
    m = mine.q
    want = peft(x)
    got = torch.nn.functional.linear(x, m.base.weight, m.base.bias) + m.scale * (x @ m.lora_a.T) @ m.lora_b.T
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_diffusers_key_renames_and_round_trip(pkg, tmp_path):
    """"diffusers" (the H3 backend's pytorch_lora_weights.safetensors, minimax_h3/model.py:441-449):
    diffusers 0.34's PEFT -> diffusers renames, first match only, applied after ".processor." -> ".";
    names with none of the patterns (Wan's q/k/v/o) are unchanged. Parity with diffusers itself is
    unpinned (not installed)."""
    from dmd_system_amd.adapters import diffusers_key
    assert diffusers_key("blocks.0.attn1.to_q.lora_A.weight") == "blocks.0.attn1.to_q.lora.down.weight"
    assert diffusers_key("blocks.0.attn1.to_out.0.lora_B.weight") == "blocks.0.attn1.to_out.0.lora.up.weight"
    assert diffusers_key("text_model.layers.1.self_attn.q_proj.lora_A.weight") == \
        "text_model.layers.1.self_attn.q_proj.lora_linear_layer.down.weight"
    assert diffusers_key("blocks.0.self_attn.q.lora_A.weight") == "blocks.0.self_attn.q.lora_A.weight"
    assert diffusers_key("a.processor.to_k.lora_B.weight") == "a.to_k.lora.up.weight"
    src, dst = _model(pkg, seed=0), _model(pkg, seed=1)
    pkg.save_adapters(str(tmp_path / "role"), src, fmt="diffusers")
    assert sorted(p.name for p in (tmp_path / "role").iterdir()) == ["pytorch_lora_weights.safetensors"]
    assert sorted(pkg.load_adapters(str(tmp_path / "role"), dst)) == ["ffn", "q"]
    for a, b in zip(src.parameters(), dst.parameters()):
        if a.requires_grad:
            assert torch.equal(a, b)
