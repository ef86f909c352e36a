"""LiveWan's critic LoRA on the HIP path (the LiveWan call site of the LoRA linear).

The LiveWan critic shares the frozen teacher weights through a minimal LoRA module
(reference/livewan_wan21/wanstreamer/lora.py:8-27):

    base (nn.Linear, weight and bias frozen), rank, scale = (alpha or rank) / rank,
    a [rank, in] ~ N(0, (1/rank)^2), b [out, rank] zeros, enabled (bool)

    forward: y = base(x); if not enabled: y
             else y + linear(linear(x.to(a.dtype), a), b).to(y.dtype) * scale

``inject_lora`` (:34-56) wraps the targets of every block (``self_attn.q/k/v/o``,
``ffn.0``, ``ffn.2``) with fp32 ``a`` / ``b`` over the bf16 critic
(runtime/livewan_crossscale_worker.py:1587,1594), and ``lora_enabled(model, on)`` (:65-74)
switches the adapters off for the teacher's conditional / unconditional pass and on for the
critic's (livewan_crossscale_worker.py:2614-2645). ``lora_state_dict`` keeps the ``.a`` / ``.b``
keys (:77-79).

This module gives the same interface over the multi-LoRA op:

* ``LiveWanLoRALinear(base, rank=32, alpha=None)``: the same attributes, initialisation and
  state-dict keys; its forward runs the multi-LoRA op with one adapter (``enabled``) or none
  (disabled: the base alone through the same GEMM, and ``a`` / ``b`` stay out of the graph, as
  in the reference). ``inject_lora``, ``set_lora``, ``lora_enabled``, ``lora_state_dict`` mirror
  the reference's functions and act on every module of this layout.
* ``install_livewan_multi_lora(model)``: modules of the reference's own class (recognised by
  their attribute layout) keep their class, Parameters and ``enabled`` flag; only their forward
  is replaced, so the reference's ``lora_enabled`` and ``lora_state_dict`` keep working on them.
* ``roles.fuse_roles({'teacher': critic, 'critic': critic}, base_roles=('teacher',))`` batches
  the teacher pass (base only) and the critic pass into one call per linear; a role whose
  modules are disabled at call time is base-only too.

Arithmetic (the same rules as the other modules of this package): fp32 ``a`` / ``b`` over a
bf16 base outside autocast are used at fp32-class precision (hi + lo bf16 parts) and the LoRA
term is added to the base product in the fp32 accumulators before one rounding to bf16; the
reference rounds the update to bf16, multiplies by the scale in bf16 and adds in bf16 (three
roundings), so these outputs are closer to the exact result. Under bf16 autocast the adapters
are rounded to bf16, as autocast rounds F.linear's operands.
"""
from __future__ import annotations

import types
from contextlib import contextmanager
from typing import Sequence

import torch
from torch import nn

from .function import multi_lora_linear
from .low_rank import transposed_base
from .routing import BASE_ONLY, SegmentRouting

TARGETS = ('self_attn.q', 'self_attn.k', 'self_attn.v', 'self_attn.o', 'ffn.0', 'ffn.2')


def is_livewan_lora_linear(m: nn.Module) -> bool:
    """A module of LiveWan's LoRA layout: ``base`` nn.Linear, Parameters ``a`` [r, in] and
    ``b`` [out, r], an ``enabled`` flag and a ``scale``."""
    base = getattr(m, 'base', None)
    a, b = getattr(m, 'a', None), getattr(m, 'b', None)
    return (isinstance(base, nn.Linear) and isinstance(a, nn.Parameter) and isinstance(b, nn.Parameter)
            and isinstance(getattr(m, 'enabled', None), bool) and hasattr(m, 'scale')
            and a.dim() == 2 and b.dim() == 2 and a.shape[1] == base.in_features
            and b.shape == (base.out_features, a.shape[0]))


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0


def livewan_forward(self: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """The forward of a LiveWan-layout module on the multi-LoRA op."""
    group = self.__dict__.get('shared_input')
    if group is not None and self.enabled:  # stacked with the other linears that read this input
        return group(self, x)
    return _single(self, x)


def _single(self: nn.Module, x: torch.Tensor, routing: SegmentRouting | None = None) -> torch.Tensor:
    base = self.base
    wt = transposed_base(base.weight, x, getattr(self, 'transposed_base_for_dx', True))
    if not self.enabled:  # the base alone; a and b take no part (no gradient, as in the reference)
        return multi_lora_linear(x, base.weight, base.bias, [], [], [], SegmentRouting.single(_rows(x), BASE_ONLY),
                                 weight_t=wt)
    return multi_lora_linear(x, base.weight, base.bias, [self.a], [self.b], [float(self.scale)],
                             routing or SegmentRouting.single(_rows(x), 0), weight_t=wt)


class LiveWanLoRALinear(nn.Module):
    """LiveWan's LoRALinear (wanstreamer/lora.py:8-27) on the multi-LoRA op: same attributes
    (``base``, ``rank``, ``scale``, ``a``, ``b``, ``enabled``), initialisation and keys."""

    def __init__(self, base: nn.Linear, rank: int = 32, alpha=None):
        super().__init__()
        self.base = base
        self.base.weight.requires_grad_(False)
        if self.base.bias is not None:
            self.base.bias.requires_grad_(False)
        self.rank = rank
        self.scale = (alpha or rank) / rank
        self.a = nn.Parameter(torch.zeros(rank, base.in_features))
        self.b = nn.Parameter(torch.zeros(base.out_features, rank))
        nn.init.normal_(self.a, std=1.0 / rank)
        self.enabled = True

    forward = livewan_forward
    _single = _single


def _target(block: nn.Module, name: str) -> tuple[nn.Module, str, nn.Module]:
    parent, _, leaf = name.rpartition('.')
    mod = block.get_submodule(parent) if parent else block
    lin = mod[int(leaf)] if leaf.isdigit() else getattr(mod, leaf)
    return mod, leaf, lin


def inject_lora(model: nn.Module, rank: int = 32, alpha=None, targets: Sequence[str] = TARGETS):
    """Freeze ``model`` and wrap ``targets`` of every ``model.blocks`` entry with
    LiveWanLoRALinear (fp32 ``a`` / ``b`` on the base's device), skipping targets already
    wrapped; returns (trainable parameters, modules wrapped, trainable element count), as
    wanstreamer/lora.py:34-56 does."""
    for p in model.parameters():
        p.requires_grad_(False)
    n = 0
    for blk in model.blocks:
        for name in targets:
            mod, leaf, lin = _target(blk, name)
            if is_livewan_lora_linear(lin):
                continue
            wrapped = LiveWanLoRALinear(lin, rank, alpha).to(lin.weight.device)
            wrapped.a.data = wrapped.a.data.float()
            wrapped.b.data = wrapped.b.data.float()
            if leaf.isdigit():
                mod[int(leaf)] = wrapped
            else:
                setattr(mod, leaf, wrapped)
            n += 1
    params = [p for p in model.parameters() if p.requires_grad]
    return params, n, sum(p.numel() for p in params)


def _modules(model: nn.Module) -> list[nn.Module]:
    return [m for m in model.modules() if is_livewan_lora_linear(m)]


def set_lora(model: nn.Module, on: bool) -> None:
    """``enabled = on`` on every LiveWan-layout module of ``model`` (wanstreamer/lora.py:59-62)."""
    for m in _modules(model):
        m.enabled = on


@contextmanager
def lora_enabled(model: nn.Module, on: bool):
    """Inside the block every LiveWan-layout module of ``model`` has ``enabled = on``; each
    module's own flag is restored on exit (wanstreamer/lora.py:65-74)."""
    mods = _modules(model)
    prev = [m.enabled for m in mods]
    for m in mods:
        m.enabled = on
    try:
        yield
    finally:
        for m, p in zip(mods, prev):
            m.enabled = p


def lora_state_dict(model: nn.Module) -> dict:
    """The ``.a`` / ``.b`` entries of the state dict (wanstreamer/lora.py:77-79)."""
    return {k: v for k, v in model.state_dict().items() if k.endswith('.a') or k.endswith('.b')}


def install_livewan_multi_lora(model: nn.Module) -> list[str]:
    """Route every LiveWan-layout module of ``model`` (the reference's own class included)
    through the multi-LoRA op; returns their names. Class, Parameters, ``enabled`` and keys are
    kept. ValueError if there is none (nothing would run on the HIP path)."""
    found = [(name, m) for name, m in model.named_modules() if is_livewan_lora_linear(m)]
    if not found:
        raise ValueError('no LiveWan LoRA modules (base / a / b / enabled / scale) in the model')
    for _, m in found:
        if isinstance(m, LiveWanLoRALinear) or '_livewan_original_forward' in m.__dict__:
            continue
        m.__dict__['_livewan_original_forward'] = m.__dict__.get('forward')
        m.forward = types.MethodType(livewan_forward, m)
        m._single = types.MethodType(_single, m)
    return [name for name, _ in found]


def uninstall_livewan_multi_lora(model: nn.Module) -> None:
    """Give every installed module its own forward back."""
    for m in model.modules():
        if '_livewan_original_forward' in m.__dict__:
            orig = m.__dict__.pop('_livewan_original_forward')
            m.__dict__.pop('_single', None)
            if orig is None:
                del m.forward
            else:
                m.forward = orig
