"""Adapter state in the reference's exchange formats: export and import of trained LoRA.

The drop-in modules keep the reference's own parameter names, so the reference's
checkpoints (``training/checkpoint.py:177``, module ``state_dict`` with ``<target>.lora_a`` /
``<target>.lora_b`` / ``<target>.base.weight``) load unchanged. Trained adapters also leave
the reference in other layouts, which this module writes and reads:

* ``"peft"`` — a PeftModel's adapter state dict, as ``get_peft_model_state_dict`` returns it
  for a model wrapped by ``get_peft_model``: ``base_model.model.<target>.lora_A.weight``
  [r, in] and ``...lora_B.weight`` [out, r], with ``r`` / ``lora_alpha`` (scaling alpha / r,
  applied at run time) in ``adapter_config.json`` (``rank_pattern`` / ``alpha_pattern`` when
  targets differ), weights in ``adapter_model.safetensors``.
* ``"peft_module"`` — PEFT's layers inside the model itself, as ``model.add_adapter(config)``
  leaves them (``training/wan_public.py:213``, adapter ``'default'``; H3's per-role adapters,
  ``backends/training/minimax_h3/model.py:286-330``): the model's own state dict holds
  ``<target>.lora_A.<adapter>.weight``, ``<target>.lora_B.<adapter>.weight`` and the frozen base
  as ``<target>.base_layer.weight`` / ``.bias`` (``wan_public.py:498`` loads such a state dict).
  Import takes the adapter's keys and, with ``check_base``, checks each ``base_layer`` tensor
  against the module's frozen base; other keys of the model are not adapter state.
* ``"diffusers"`` — what the H3 backend saves per role (``minimax_h3/model.py:441-449``):
  ``get_peft_model_state_dict(denoiser, adapter_name=role)`` (``<target>.lora_A.weight``, no
  wrapper prefix) converted by diffusers' ``convert_state_dict_to_diffusers`` (diffusers
  0.34.0, pinned for H3 in pyproject.toml:71) into ``pytorch_lora_weights.safetensors``: its
  PEFT-to-diffusers key renames (``to_q/k/v.lora_A`` -> ``.lora.down``, ``lora_B`` -> ``.lora.up``,
  ``to_out.0.*`` likewise, ``.q/k/v/out_proj.lora_A`` -> ``.lora_linear_layer.down``, ...; first
  match only; ``.processor.`` -> ``.``) are restated in ``_DIFFUSERS_RENAMES``; the scale is
  not stored. diffusers is not installed here and the reference holds no file of this layout:
  parity of this format with diffusers is unpinned (round trips and the renames are tested).
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
FORMATS = ("peft", "peft_module", "diffusers", "diffsynth")
ADAPTER_FILE = "adapter_model.safetensors"
DIFFUSERS_FILE = "pytorch_lora_weights.safetensors"
CONFIG_FILE = "adapter_config.json"

# diffusers 0.34.0 PEFT -> diffusers key renames (state_dict_utils.PEFT_TO_DIFFUSERS), applied to
# each key after the always-applied ".processor." -> "."; the first pattern contained in the
# key is replaced and no other.
_DIFFUSERS_ALWAYS = ((".processor.", "."),)
_DIFFUSERS_RENAMES = (
    (".q_proj.lora_B", ".q_proj.lora_linear_layer.up"), (".q_proj.lora_A", ".q_proj.lora_linear_layer.down"),
    (".k_proj.lora_B", ".k_proj.lora_linear_layer.up"), (".k_proj.lora_A", ".k_proj.lora_linear_layer.down"),
    (".v_proj.lora_B", ".v_proj.lora_linear_layer.up"), (".v_proj.lora_A", ".v_proj.lora_linear_layer.down"),
    (".out_proj.lora_B", ".out_proj.lora_linear_layer.up"), (".out_proj.lora_A", ".out_proj.lora_linear_layer.down"),
    ("to_k.lora_A", "to_k.lora.down"), ("to_k.lora_B", "to_k.lora.up"),
    ("to_q.lora_A", "to_q.lora.down"), ("to_q.lora_B", "to_q.lora.up"),
    ("to_v.lora_A", "to_v.lora.down"), ("to_v.lora_B", "to_v.lora.up"),
    ("to_out.0.lora_A", "to_out.0.lora.down"), ("to_out.0.lora_B", "to_out.0.lora.up"),
)


def diffusers_key(peft_key: str) -> str:
    """The key convert_state_dict_to_diffusers gives a PEFT adapter-state key."""
    for pat, new in _DIFFUSERS_ALWAYS:
        if pat in peft_key:
            peft_key = peft_key.replace(pat, new)
    for pat, new in _DIFFUSERS_RENAMES:
        if pat in peft_key:
            return peft_key.replace(pat, new)
    return peft_key


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


def _keys(name: str, fmt: str, prefix: str, adapter: str = "default") -> tuple[str, str]:
    if fmt == "peft":
        return f"{prefix}{name}.lora_A.weight", f"{prefix}{name}.lora_B.weight"
    if fmt == "peft_module":
        return f"{name}.lora_A.{adapter}.weight", f"{name}.lora_B.{adapter}.weight"
    if fmt == "diffusers":
        return diffusers_key(f"{name}.lora_A.weight"), diffusers_key(f"{name}.lora_B.weight")
    return f"{name}.lora_A.weight", f"{name}.lora_B.weight"


def _base_of(model: nn.Module, name: str) -> nn.Linear:
    m = model.get_submodule(name)
    return m.base


def export_adapters(model: nn.Module, *, role: str | None = None, fmt: str = "peft",
                    prefix: str = PEFT_PREFIX, adapter: str = "default",
                    with_base: bool = False) -> tuple[dict[str, torch.Tensor], dict]:
    """(state, config): the adapters of ``model`` (of ``role``) as CPU tensors in ``fmt``
    (``adapter``: the PEFT adapter name of ``"peft_module"``; ``with_base`` adds each target's
    frozen base as ``<target>.base_layer.*`` there, as a PEFT model's own state dict holds it)."""
    _require(fmt in FORMATS, f'format {fmt!r} is not one of {FORMATS}')
    slots = _slots(model, role)
    state: dict[str, torch.Tensor] = {}
    ranks, alphas = {}, {}
    for name, (a, b, s) in slots.items():
        ka, kb = _keys(name, fmt, prefix, adapter)
        if fmt == "peft_module" and with_base:
            base = _base_of(model, name)
            state[f"{name}.base_layer.weight"] = base.weight.detach().to("cpu").contiguous()
            if base.bias is not None:
                state[f"{name}.base_layer.bias"] = base.bias.detach().to("cpu").contiguous()
        state[ka] = a.detach().to("cpu").contiguous()
        bb = b.detach().to("cpu")
        state[kb] = (bb * s if fmt == "diffsynth" else bb).contiguous()
        ranks[name] = int(a.shape[0])
        alphas[name] = float(s) * int(a.shape[0])
    targets = sorted(slots)
    if fmt in ("peft", "peft_module", "diffusers"):
        r = max(set(ranks.values()), key=list(ranks.values()).count)
        alpha = max(set(alphas.values()), key=list(alphas.values()).count)
        config = {"peft_type": "LORA", "r": r, "lora_alpha": alpha, "lora_dropout": 0.0, "bias": "none",
                  "target_modules": targets,
                  "rank_pattern": {n: v for n, v in ranks.items() if v != r},
                  "alpha_pattern": {n: v for n, v in alphas.items() if v != alpha}}
        if fmt == "peft_module":
            config["adapter_name"] = adapter
    else:
        config = {"format": "diffsynth", "scale_baked_into_lora_B": True, "target_modules": targets,
                  "ranks": ranks}
    if role is not None:
        config["role"] = role
    return state, config


def import_adapters(model: nn.Module, state: Mapping[str, torch.Tensor], config: Mapping | None = None, *,
                    role: str | None = None, fmt: str = "peft", prefix: str = PEFT_PREFIX,
                    strict: bool = True, adapter: str = "default", check_base: bool = True) -> list[str]:
    """Copy adapters from ``state`` (``fmt``) into the model's Parameters; returns the targets
    loaded. ``strict``: every target of the model (role) must be present and every adapter key
    used (for ``"peft_module"``: every ``lora_A`` / ``lora_B`` key of ``adapter``; the rest of a
    model state dict is not adapter state). A PEFT-style ``config`` is checked against each
    target's rank and scale; a DiffSynth state's B is divided by the target's scale;
    ``check_base`` (``"peft_module"``): a ``<target>.base_layer.*`` tensor present in ``state``
    must equal the module's frozen base."""
    _require(fmt in FORMATS, f'format {fmt!r} is not one of {FORMATS}')
    slots = _slots(model, role)
    used, loaded = set(), []
    for name, (a, b, s) in slots.items():
        ka, kb = _keys(name, fmt, prefix, adapter)
        if ka not in state or kb not in state:
            _require(not strict, f'missing {ka!r} / {kb!r}')
            continue
        ta, tb = state[ka], state[kb]
        _require(tuple(ta.shape) == tuple(a.shape) and tuple(tb.shape) == tuple(b.shape),
                 f'{name!r}: lora_A {tuple(ta.shape)} / lora_B {tuple(tb.shape)} do not match '
                 f'{tuple(a.shape)} / {tuple(b.shape)}')
        _require(bool(torch.isfinite(ta).all()) and bool(torch.isfinite(tb).all()), f'{name!r}: non-finite values')
        if fmt in ("peft", "peft_module", "diffusers") and config is not None:
            r = int(config.get("rank_pattern", {}).get(name, config.get("r", a.shape[0])))
            alpha = float(config.get("alpha_pattern", {}).get(name, config.get("lora_alpha", r)))
            _require(r == a.shape[0], f'{name!r}: config rank {r} != module rank {a.shape[0]}')
            _require(abs(alpha / r - s) <= 1e-6 * max(1.0, abs(s)),
                     f'{name!r}: config scaling {alpha}/{r} != module scale {s}')
        if fmt == "peft_module" and check_base:
            base = _base_of(model, name)
            for key, t in ((f"{name}.base_layer.weight", base.weight), (f"{name}.base_layer.bias", base.bias)):
                if key in state:
                    _require(t is not None and tuple(state[key].shape) == tuple(t.shape)
                             and torch.equal(state[key].to(device=t.device, dtype=t.dtype), t.detach()),
                             f'{key!r} differs from the module\'s frozen base')
        with torch.no_grad():
            a.copy_(ta.to(device=a.device, dtype=a.dtype))
            tb = tb.to(device=b.device, dtype=torch.float64 if fmt == "diffsynth" else b.dtype)
            b.copy_(tb / s if fmt == "diffsynth" else tb)
        used.update((ka, kb))
        loaded.append(name)
    if strict:
        if fmt == "peft_module":
            tag = f".{adapter}.weight"
            extra = sorted(k for k in state if (".lora_A." in k or ".lora_B." in k) and k.endswith(tag) and k not in used)
        else:
            extra = sorted(set(state) - used)
        _require(not extra, f'unused keys {extra[:4]}{"…" if len(extra) > 4 else ""}')
    return loaded


def save_adapters(directory: str, model: nn.Module, *, role: str | None = None, fmt: str = "peft",
                  prefix: str = PEFT_PREFIX) -> None:
    """``directory``/adapter_model.safetensors + adapter_config.json (PEFT's file names), or for
    ``"diffusers"`` the H3 backend's ``pytorch_lora_weights.safetensors`` alone (diffusers keeps no
    config beside it)."""
    from safetensors.torch import save_file
    _require(fmt != "peft_module", 'a "peft_module" state is part of a model state dict, not an adapter file')
    state, config = export_adapters(model, role=role, fmt=fmt, prefix=prefix)
    os.makedirs(directory, exist_ok=True)
    if fmt == "diffusers":
        save_file(state, os.path.join(directory, DIFFUSERS_FILE))
        return
    save_file(state, os.path.join(directory, ADAPTER_FILE))
    with open(os.path.join(directory, CONFIG_FILE), "w") as f:
        json.dump(config, f, indent=1, sort_keys=True)


def load_adapters(directory: str, model: nn.Module, *, role: str | None = None, prefix: str = PEFT_PREFIX,
                  strict: bool = True) -> list[str]:
    """Read what save_adapters wrote into the model: the format comes from the config, or is
    ``"diffusers"`` for a directory holding only pytorch_lora_weights.safetensors."""
    from safetensors.torch import load_file
    if not os.path.exists(os.path.join(directory, CONFIG_FILE)) and os.path.exists(
            os.path.join(directory, DIFFUSERS_FILE)):
        state = load_file(os.path.join(directory, DIFFUSERS_FILE))
        return import_adapters(model, state, None, role=role, fmt="diffusers", strict=strict)
    with open(os.path.join(directory, CONFIG_FILE)) as f:
        config = json.load(f)
    fmt = "diffsynth" if config.get("format") == "diffsynth" else "peft"
    state = load_file(os.path.join(directory, ADAPTER_FILE))
    return import_adapters(model, state, config, role=role, fmt=fmt, prefix=prefix, strict=strict)
