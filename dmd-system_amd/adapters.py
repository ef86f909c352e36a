"""Adapter state in the reference's exchange formats: export and import of trained LoRA.

The drop-in modules keep the reference's own parameter names, so the reference's
checkpoints (``training/checkpoint.py:177``, module ``state_dict`` with ``<target>.lora_a`` /
``<target>.lora_b`` / ``<target>.base.weight``) load unchanged. Trained adapters also leave
the reference in two other layouts, which this module writes and reads:

* ``"peft"`` — PEFT's adapter state dict, as ``get_peft_model_state_dict`` returns it and
  the minimax-H3 backend saves it (``backends/training/minimax_h3/model.py:442-451``):
  ``base_model.model.<target>.lora_A.weight`` [r, in] and ``...lora_B.weight`` [out, r],
  with ``r`` / ``lora_alpha`` (scaling alpha / r, applied at run time) in the adapter
  config (``training/wan_public.py:213-214``; ``rank_pattern`` / ``alpha_pattern`` when
  targets differ).
* ``"diffsynth"`` — the DiffSynth export of ``reference/diffsynth_h3_cached/h3_dmd2.py:177-183``:
  ``<target>.lora_A.weight`` = A and ``<target>.lora_B.weight`` = B·(alpha / r), the
  scale baked into B for a loader that applies none.

A ``MultiLoRALinear`` built by ``fuse_roles`` holds several roles' adapters; ``role`` picks
one (a role without an adapter at a target exports nothing for it). Import writes into the
existing Parameters in place (their dtype and device), so optimizers keep owning them.
Every mismatch fails closed with ``ValueError('adapter state: …')``.
"""
from __future__ import annotations

import json
import os
from typing import Mapping

import torch
from torch import nn

from .low_rank import MultiLoRALinear, TrainableLowRankLinear

PEFT_PREFIX = "base_model.model."
FORMATS = ("peft", "diffsynth")
ADAPTER_FILE = "adapter_model.safetensors"
CONFIG_FILE = "adapter_config.json"


def _require(value, message):
    if not value:
        raise ValueError('adapter state: ' + message)


def _slots(model: nn.Module, role: str | None) -> dict[str, tuple[nn.Parameter, nn.Parameter, float]]:
    """target name -> (lora_a, lora_b, scale) of the chosen role."""
    out = {}
    for name, m in model.named_modules():
        if isinstance(m, TrainableLowRankLinear):
            _require(role is None, f'{name!r} holds one adapter: no role to select')
            out[name] = (m.lora_a, m.lora_b, m.scale)
        elif isinstance(m, MultiLoRALinear):
            if role is None:
                _require(m.num_adapters == 1, f'{name!r} holds {m.num_adapters} adapters: pass role=')
                i = 0
            elif role in m.role_ids:
                i = m.role_ids[role]
            else:
                _require(m.role_ids, f'{name!r} has no role names (build it with fuse_roles)')
                continue  # this role has no adapter at this target
            out[name] = (m.lora_a[i], m.lora_b[i], m.scales[i])
    _require(out, 'the model has no LoRA adapter' + (f' for role {role!r}' if role else ''))
    return out


def _keys(name: str, fmt: str, prefix: str) -> tuple[str, str]:
    if fmt == "peft":
        return f"{prefix}{name}.lora_A.weight", f"{prefix}{name}.lora_B.weight"
    return f"{name}.lora_A.weight", f"{name}.lora_B.weight"


def export_adapters(model: nn.Module, *, role: str | None = None, fmt: str = "peft",
                    prefix: str = PEFT_PREFIX) -> tuple[dict[str, torch.Tensor], dict]:
    """(state, config): the adapters of ``model`` (of ``role``) as CPU tensors in ``fmt``."""
    _require(fmt in FORMATS, f'format {fmt!r} is not one of {FORMATS}')
    slots = _slots(model, role)
    state: dict[str, torch.Tensor] = {}
    ranks, alphas = {}, {}
    for name, (a, b, s) in slots.items():
        ka, kb = _keys(name, fmt, prefix)
        state[ka] = a.detach().to("cpu").contiguous()
        bb = b.detach().to("cpu")
        state[kb] = (bb * s if fmt == "diffsynth" else bb).contiguous()
        ranks[name] = int(a.shape[0])
        alphas[name] = float(s) * int(a.shape[0])
    targets = sorted(slots)
    if fmt == "peft":
        r = max(set(ranks.values()), key=list(ranks.values()).count)
        alpha = max(set(alphas.values()), key=list(alphas.values()).count)
        config = {"peft_type": "LORA", "r": r, "lora_alpha": alpha, "lora_dropout": 0.0, "bias": "none",
                  "target_modules": targets,
                  "rank_pattern": {n: v for n, v in ranks.items() if v != r},
                  "alpha_pattern": {n: v for n, v in alphas.items() if v != alpha}}
    else:
        config = {"format": "diffsynth", "scale_baked_into_lora_B": True, "target_modules": targets,
                  "ranks": ranks}
    if role is not None:
        config["role"] = role
    return state, config


def import_adapters(model: nn.Module, state: Mapping[str, torch.Tensor], config: Mapping | None = None, *,
                    role: str | None = None, fmt: str = "peft", prefix: str = PEFT_PREFIX,
                    strict: bool = True) -> list[str]:
    """Copy adapters from ``state`` (``fmt``) into the model's Parameters; returns the targets
    loaded. ``strict``: every target of the model (role) must be present and every key used.
    A PEFT ``config`` is checked against each target's rank and scale; a DiffSynth state's B
    is divided by the target's scale."""
    _require(fmt in FORMATS, f'format {fmt!r} is not one of {FORMATS}')
    slots = _slots(model, role)
    used, loaded = set(), []
    for name, (a, b, s) in slots.items():
        ka, kb = _keys(name, fmt, prefix)
        if ka not in state or kb not in state:
            _require(not strict, f'missing {ka!r} / {kb!r}')
            continue
        ta, tb = state[ka], state[kb]
        _require(tuple(ta.shape) == tuple(a.shape) and tuple(tb.shape) == tuple(b.shape),
                 f'{name!r}: lora_A {tuple(ta.shape)} / lora_B {tuple(tb.shape)} do not match '
                 f'{tuple(a.shape)} / {tuple(b.shape)}')
        _require(bool(torch.isfinite(ta).all()) and bool(torch.isfinite(tb).all()), f'{name!r}: non-finite values')
        if fmt == "peft" and config is not None:
            r = int(config.get("rank_pattern", {}).get(name, config.get("r", a.shape[0])))
            alpha = float(config.get("alpha_pattern", {}).get(name, config.get("lora_alpha", r)))
            _require(r == a.shape[0], f'{name!r}: config rank {r} != module rank {a.shape[0]}')
            _require(abs(alpha / r - s) <= 1e-6 * max(1.0, abs(s)),
                     f'{name!r}: config scaling {alpha}/{r} != module scale {s}')
        with torch.no_grad():
            a.copy_(ta.to(device=a.device, dtype=a.dtype))
            tb = tb.to(device=b.device, dtype=torch.float64 if fmt == "diffsynth" else b.dtype)
            b.copy_(tb / s if fmt == "diffsynth" else tb)
        used.update((ka, kb))
        loaded.append(name)
    if strict:
        extra = sorted(set(state) - used)
        _require(not extra, f'unused keys {extra[:4]}{"…" if len(extra) > 4 else ""}')
    return loaded


def save_adapters(directory: str, model: nn.Module, *, role: str | None = None, fmt: str = "peft",
                  prefix: str = PEFT_PREFIX) -> None:
    """``directory``/adapter_model.safetensors + adapter_config.json (PEFT's file names)."""
    from safetensors.torch import save_file
    state, config = export_adapters(model, role=role, fmt=fmt, prefix=prefix)
    os.makedirs(directory, exist_ok=True)
    save_file(state, os.path.join(directory, ADAPTER_FILE))
    with open(os.path.join(directory, CONFIG_FILE), "w") as f:
        json.dump(config, f, indent=1, sort_keys=True)


def load_adapters(directory: str, model: nn.Module, *, role: str | None = None, prefix: str = PEFT_PREFIX,
                  strict: bool = True) -> list[str]:
    """Read what save_adapters wrote (the format comes from the config) into the model."""
    from safetensors.torch import load_file
    with open(os.path.join(directory, CONFIG_FILE)) as f:
        config = json.load(f)
    fmt = "diffsynth" if config.get("format") == "diffsynth" else "peft"
    state = load_file(os.path.join(directory, ADAPTER_FILE))
    return import_adapters(model, state, config, role=role, fmt=fmt, prefix=prefix, strict=strict)
