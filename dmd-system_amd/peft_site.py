"""PEFT LoRA layers on the HIP path (the W1 / H3 call site of the LoRA linear).

The reference installs PEFT adapters on its DiTs: the W1 factory calls
``model.add_adapter(LoraConfig(r=rank, lora_alpha=rank, lora_dropout=0., ...))``
(training/wan_public.py:213, adapter ``'default'``), and H3 adds one named adapter per role,
switching with ``set_adapter(role)`` and running the teacher with ``disable_adapters()``
(backends/training/minimax_h3/model.py:286-330). A PEFT LoRA ``Linear`` layer holds

    base_layer (nn.Linear), lora_A[name] (nn.Linear in -> r, no bias), lora_B[name]
    (nn.Linear r -> out), lora_dropout[name], scaling[name], active_adapters, merged,
    disable_adapters

and computes, for its active adapter (operator order replayed at
runtime/wan13b_lora_cast.py:204-229):

    result = base_layer(x); x = cast(x, lora_A.weight.dtype)
    result = result + lora_B(lora_A(dropout(x))) * scaling; result.to(result dtype)

``install_peft_multi_lora(model)`` replaces the forward of every such layer with the batched
multi-LoRA op (the same arithmetic rules as the other modules: bf16 autocast rounds the
adapters like autocast rounds F.linear's operands; fp32 masters over a bf16 base outside
autocast are used at fp32-class precision; float32 everything runs in float32):

* one active adapter: one segment; ``disable_adapters``: the base alone (adapter id -1);
* ``adapter_names=[...]`` (PEFT's mixed batch: one name per sample, ``'__base__'`` for no
  adapter): one segment per run of equal names, all in one launch;
* ``peft_roles_active(model, RoleBatch(...), base_roles=...)``: every installed layer routes the
  batch's roles to the adapters of the same name (H3's roles are adapter names) and the
  ``base_roles`` (the teacher) to the base alone — several roles' forwards in one pass.

It fails closed (RuntimeError, nothing launched) where the reference's installed forward does
(runtime/wan13b_lora_cast.py:526-560): merged adapters, more than one active adapter, an active
adapter missing from lora_A, LoRA variants (DoRA, ...), variant keyword arguments; and where the
op would differ from PEFT: an active dropout (p > 0 in training mode) and a LoRA-B bias.

peft itself is not importable in this environment: layers are recognised by their attribute
layout, and parity against the real library is unpinned (the tests use a module with PEFT's
attribute layout and the operator order above).
"""
from __future__ import annotations

import types
from contextlib import contextmanager
from typing import Iterable, Sequence

import torch
from torch import nn

from .function import multi_lora_linear
from .low_rank import transposed_base
from .roles import RoleBatch
from .routing import BASE_ONLY, SegmentRouting

BASE_NAME = "__base__"  # PEFT's name for "no adapter" in a mixed batch
_ATTRS = ("base_layer", "lora_A", "lora_B", "lora_dropout", "scaling")


def is_peft_lora_linear(m: nn.Module) -> bool:
    """A PEFT LoRA Linear layer: the attribute layout above over an nn.Linear base."""
    return (all(hasattr(m, a) for a in _ATTRS) and isinstance(m.base_layer, nn.Linear)
            and isinstance(m.lora_A, nn.ModuleDict) and isinstance(m.lora_B, nn.ModuleDict))


def _fail(message: str):
    raise RuntimeError("PEFT LoRA on the multi-LoRA op: " + message)


def _active_adapters(m: nn.Module) -> list[str]:
    a = getattr(m, "active_adapters", None)
    if a is None:
        a = getattr(m, "active_adapter", None)
    if isinstance(a, str):
        a = [a]
    return list(a or [])


def _check_adapter(m: nn.Module, name: str) -> None:
    if name not in m.lora_A:
        _fail(f"adapter {name!r} is absent from lora_A")
    if name in (getattr(m, "lora_variant", None) or {}) or (getattr(m, "use_dora", None) or {}).get(name, False):
        _fail(f"adapter {name!r} is a LoRA variant (DoRA, ...): outside the fused contract")
    if getattr(m.lora_B[name], "bias", None) is not None:
        _fail(f"adapter {name!r} has a LoRA-B bias, which the op does not apply")
    drop = m.lora_dropout[name] if name in m.lora_dropout else nn.Identity()
    if isinstance(drop, nn.Dropout) and drop.p > 0 and drop.training:
        _fail(f"adapter {name!r} has active dropout (p={drop.p}) on its input: set lora_dropout=0 or eval()")


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0


def _mixed_routing(x: torch.Tensor, adapter_names: Sequence[str]) -> tuple[list[str], SegmentRouting]:
    """PEFT's mixed batch: one adapter name per sample (dimension 0) -> adapters and routing."""
    samples = x.shape[0] if x.dim() > 1 else 0
    if len(adapter_names) != samples:
        _fail(f"adapter_names has {len(adapter_names)} entries for a batch of {samples} samples")
    per = _rows(x) // samples if samples else 0
    names: list[str] = []
    lengths: list[int] = []
    ids: list[int] = []
    for n in adapter_names:
        a = BASE_ONLY
        if n != BASE_NAME:
            if n not in names:
                names.append(n)
            a = names.index(n)
        if ids and ids[-1] == a:
            lengths[-1] += per
        else:
            lengths.append(per)
            ids.append(a)
    if not ids:
        lengths, ids = [0], [BASE_ONLY]
    return names, SegmentRouting.from_lengths(lengths, ids)


def peft_plan(self: nn.Module, x: torch.Tensor, adapter_names: Sequence[str] | None = None):
    """(adapter names, routing) of one installed layer's call on x, with the fail-closed checks of
    the module doc: the disabled layer routes every row to the base alone, a mixed batch by
    sample, an active role batch by role, otherwise the one active adapter over every row."""
    roles = self.__dict__.get("peft_roles")
    # merged first: a merged base carries the adapter, so even the disabled (base-only) branch
    # would include it; the reference's installed forward rejects merged layers whatever
    # disable_adapters says (runtime/wan13b_lora_cast.py:185-189)
    if getattr(self, "merged", False):
        _fail("merged adapters (the base already carries them): unmerge first")
    if getattr(self, "disable_adapters", False):
        if adapter_names is not None:
            _fail("adapter_names cannot be used while the adapters are disabled")
        names, routing = [], SegmentRouting.single(_rows(x), BASE_ONLY)
    elif adapter_names is not None:
        names, routing = _mixed_routing(x, adapter_names)
    elif roles is not None:
        batch, base_roles = roles
        names = [r for r, _ in batch.parts if r not in base_roles]
        names = list(dict.fromkeys(names))
        routing = batch.routing(_rows(x), {n: i for i, n in enumerate(names)})
    else:
        act = [a for a in _active_adapters(self)]
        if len(act) != 1:
            _fail(f"one active adapter is required (active: {act})")
        names, routing = act, SegmentRouting.single(_rows(x), 0)
    for n in names:
        _check_adapter(self, n)
    return names, routing


def _peft_single(self: nn.Module, x: torch.Tensor, adapter_names: Sequence[str] | None = None) -> torch.Tensor:
    """One layer's own call on the multi-LoRA op."""
    names, routing = peft_plan(self, x, adapter_names)
    base = self.base_layer
    As = [self.lora_A[n].weight for n in names]
    Bs = [self.lora_B[n].weight for n in names]
    scales = [float(self.scaling[n]) for n in names]
    return multi_lora_linear(x, base.weight, base.bias, As, Bs, scales, routing,
                             weight_t=transposed_base(base.weight, x, getattr(self, "transposed_base_for_dx", True)))


def _peft_forward(self: nn.Module, x: torch.Tensor, *args, **kwargs) -> torch.Tensor:
    """The installed forward (a method of each layer). A layer in a shared-input group
    (fuse_shared_inputs) runs stacked with the group's other linears when its adapters are on
    and no mixed batch is given."""
    adapter_names = kwargs.pop("adapter_names", None)
    if args or any(v is not None for v in kwargs.values()):
        _fail("extra forward arguments (variant keyword arguments) are outside the fused contract")
    group = self.__dict__.get("shared_input")
    if group is not None and adapter_names is None and not getattr(self, "disable_adapters", False):
        return group(self, x)
    return _peft_single(self, x, adapter_names)


def is_installed(m: nn.Module) -> bool:
    """The layer's forward is the multi-LoRA one (install_peft_multi_lora)."""
    return "_peft_original_forward" in m.__dict__


def install_peft_multi_lora(model: nn.Module) -> list[str]:
    """Route every PEFT LoRA Linear layer of ``model`` through the multi-LoRA op; returns their
    names. ValueError if there is none (nothing would run on the HIP path)."""
    found = [(name, m) for name, m in model.named_modules() if is_peft_lora_linear(m)]
    if not found:
        raise ValueError("no PEFT LoRA Linear layers (base_layer / lora_A / lora_B) in the model")
    for _, m in found:
        if "_peft_original_forward" not in m.__dict__:
            m.__dict__["_peft_original_forward"] = m.__dict__.get("forward")
            m.forward = types.MethodType(_peft_forward, m)
    return [name for name, _ in found]


def uninstall_peft_multi_lora(model: nn.Module) -> None:
    """Give every installed layer its own forward back."""
    for m in model.modules():
        if "_peft_original_forward" in m.__dict__:
            orig = m.__dict__.pop("_peft_original_forward")
            if orig is None:
                del m.forward
            else:
                m.forward = orig
            m.__dict__.pop("peft_roles", None)


def _installed(model: nn.Module) -> Iterable[nn.Module]:
    return (m for m in model.modules() if is_installed(m))


@contextmanager
def peft_roles_active(model: nn.Module, batch: RoleBatch, base_roles: Sequence[str] = ()):
    """Inside the block every installed layer routes ``batch`` (roles concatenated along the
    batch dimension, sample-major rows): a role named like one of the layer's adapters uses it,
    a role in ``base_roles`` (the teacher, H3's disable_adapters role) the base alone; any other
    role name is an error. Restored on exit."""
    if not isinstance(batch, RoleBatch):
        raise ValueError("peft roles: a RoleBatch is required")
    mods = list(_installed(model))
    if not mods:
        raise ValueError("peft roles: no installed PEFT LoRA layer (call install_peft_multi_lora first)")
    base_roles = tuple(base_roles)
    for m in mods:
        for role, _ in batch.parts:
            if role not in base_roles and role not in m.lora_A:
                raise ValueError(f"peft roles: role {role!r} is neither an adapter of every layer nor a base role")
    prev = [m.__dict__.get("peft_roles") for m in mods]
    for m in mods:
        m.__dict__["peft_roles"] = (batch, base_roles)
    try:
        yield model
    finally:
        for m, p in zip(mods, prev):
            if p is None:
                m.__dict__.pop("peft_roles", None)
            else:
                m.__dict__["peft_roles"] = p
