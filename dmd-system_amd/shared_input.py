"""Linears that read one input, run as one stacked call (q/k/v; cross-attention k/v).

A DiT block feeds the same tensor to several LoRA linears: self-attention q, k, v take
the normed hidden states, cross-attention k, v take the text context
(reference/livewan_wan21/wan/modules/model.py:123-126). The reference notices this only
to reuse one fp32 cast of that tensor across the PEFT modules, keyed by tensor
identity and in-place version (runtime/wan13b_lora_cast.py:265-300). Here the linears
themselves are stacked: ``fuse_shared_inputs(model, [["q", "k", "v"], ["cross.k",
"cross.v"]])`` links each group's modules to one ``SharedInputGroup``. When the first
member is called with a tensor, the group runs every member on it in one
``SharedInputMultiLoRAFunction`` call (one shrink read of X for the stacked A, one
reduction over X for their dA, their dX summed in the dX GEMM's epilogue) and hands each
member its output; the other members, called with the same unmodified tensor (same
object, same in-place version, same routing and grad mode), get theirs without another
launch.

The modules keep their parameters, names and state-dict keys; the stacked call reads
the members' own adapter Parameters, so gradients reach each member's ``lora_a`` /
``lora_b``, and a stacked bf16 copy of their frozen bases (and its transpose for dX), made
once per set of bases and remade when one of them changes. An output that nobody consumes is still
computed (and kept until the group's next call); a group is for linears that are all
called on the tensor.
"""
from __future__ import annotations

from typing import Sequence

import torch
from torch import nn

from . import _lib
from .function import shared_input_multi_lora
from .low_rank import MultiLoRALinear, TrainableLowRankLinear
from .routing import SegmentRouting


def _require(value, message):
    if not value:
        raise ValueError('shared input: ' + message)


def _adapters(m: nn.Module) -> tuple[list, list, list]:
    if isinstance(m, TrainableLowRankLinear):
        return [m.lora_a], [m.lora_b], [m.scale]
    return list(m.lora_a), list(m.lora_b), list(m.scales)


class SharedInputGroup:
    """Members (MultiLoRALinear, or TrainableLowRankLinear) that read one input; see the module doc."""

    def __init__(self, members: Sequence[nn.Module], names: Sequence[str] = ()):
        members = list(members)
        _require(len(members) >= 2, 'a group needs at least two linears')
        kinds = {type(m) for m in members}
        _require(kinds <= {MultiLoRALinear, TrainableLowRankLinear} and len(kinds) == 1,
                 'members must all be MultiLoRALinear or all TrainableLowRankLinear')
        _require(all(getattr(m, 'base_wq', None) is None for m in members), 'e4m3 bases are not stacked')
        bases = [m.base for m in members]
        K = bases[0].in_features
        _require(all(b.in_features == K for b in bases), 'members must have one in_features')
        ads = [_adapters(m) for m in members]
        n = len(ads[0][0])
        _require(all(len(a[0]) == n for a in ads), 'members must have the same number of adapters')
        ranks = {int(a.shape[0]) for ad in ads for a in ad[0]}
        _require(len(ranks) == 1 and next(iter(ranks)) % 16 == 0,
                 f'one LoRA rank, a multiple of 16, for every member and adapter (got {sorted(ranks)})')
        _require(len(members) * next(iter(ranks)) <= _lib.MAX_RANK,
                 f'{len(members)} members of rank {next(iter(ranks))} exceed the stacked rank limit {_lib.MAX_RANK}')
        for i in range(n):
            _require(len({ad[2][i] for ad in ads}) == 1, f'adapter {i} has different scales across members')
        if kinds == {MultiLoRALinear}:
            _require(all(m.role_ids == members[0].role_ids for m in members), 'members route different roles')
        self.members = members
        self.names = tuple(names)
        self.K, self.n, self.rank = K, n, next(iter(ranks))
        self.launches = 0      # stacked calls run (for tests and accounting)
        self._out = None       # (input, key, outputs, members not yet served)

    def _routing(self, member: nn.Module, x: torch.Tensor, routing: SegmentRouting | None) -> SegmentRouting:
        rows = x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0
        if isinstance(member, TrainableLowRankLinear):
            return SegmentRouting.single(rows, 0)
        if routing is not None:
            return routing
        if member.active_roles is None:
            raise ValueError('multi-LoRA linear: no routing given and no role batch active')
        return member.active_roles.routing(rows, member.role_ids)

    def _stackable(self, x: torch.Tensor) -> bool:
        """The stacked call is the bf16 path with bf16-rounded adapters: under bf16 autocast, or
        bf16 input with bf16 adapters. float32 inputs, and fp32 adapter masters outside autocast
        (fp32-class LoRA), run per member."""
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            return True
        if x.dtype != torch.bfloat16:
            return False
        return all(t.dtype == torch.bfloat16 for m in self.members for ad in _adapters(m)[:2] for t in ad)

    def __call__(self, member: nn.Module, x: torch.Tensor, routing: SegmentRouting | None = None) -> torch.Tensor:
        if x.is_inference() or not self._stackable(x):  # one call per linear
            return member._single(x, routing)
        idx = next(i for i, m in enumerate(self.members) if m is member)
        routing = self._routing(member, x, routing)
        key = (x._version, routing, torch.is_grad_enabled(), torch.is_autocast_enabled("cuda"))
        if self._out is not None and self._out[0] is x and self._out[1] == key and idx in self._out[3]:
            _, _, outs, pending = self._out
            pending.discard(idx)
            if not pending:
                self._out = None
            return outs[idx]
        ads = [_adapters(m) for m in self.members]
        outs = shared_input_multi_lora(x, [m.base.weight for m in self.members], [m.base.bias for m in self.members],
                                       [ad[0] for ad in ads], [ad[1] for ad in ads], ads[0][2], routing,
                                       all(getattr(m, 'transposed_base_for_dx', True) for m in self.members))
        self.launches += 1
        pending = set(range(len(self.members))) - {idx}
        self._out = (x, key, outs, pending) if pending else None
        return outs[idx]

    def release(self) -> None:
        """Drop the cached outputs."""
        self._out = None


def fuse_shared_inputs(model: nn.Module, groups: Sequence[Sequence[str]]) -> list[SharedInputGroup]:
    """Link each group of named LoRA linears of ``model`` (e.g. ``[["q", "k", "v"]]``) into a
    SharedInputGroup. Fails closed (ValueError) when a name is missing, already grouped, not a
    LoRA linear, or the group cannot be stacked (different in_features, ranks, scales or roles)."""
    out = []
    seen = set()
    for names in groups:
        names = list(names)
        mods = []
        for name in names:
            _require(name not in seen, f'{name!r} is in two groups')
            seen.add(name)
            try:
                mod = model.get_submodule(name)
            except AttributeError as exc:
                raise ValueError('shared input: missing linear ' + name) from exc
            _require(isinstance(mod, (MultiLoRALinear, TrainableLowRankLinear)), f'{name!r} is not a LoRA linear')
            _require(mod.__dict__.get('shared_input') is None, f'{name!r} is already in a shared-input group')
            mods.append(mod)
        group = SharedInputGroup(mods, names)
        for m in mods:
            m.shared_input = group
        out.append(group)
    return out


def release_shared_inputs(model: nn.Module) -> None:
    """Undo fuse_shared_inputs on every module of ``model``."""
    for m in model.modules():
        g = m.__dict__.get('shared_input')
        if g is not None:
            g.release()
            m.shared_input = None
