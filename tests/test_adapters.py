"""Adapter state formats on CPU: PEFT (get_peft_model_state_dict layout, scaling in the
config; backends/training/minimax_h3/model.py:442-451) and DiffSynth (scale baked into B;
reference/diffsynth_h3_cached/h3_dmd2.py:177-183) round trips, per-role export of a
multi-role tree, the fail-closed checks, and what each format means numerically. No
kernel runs."""
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
