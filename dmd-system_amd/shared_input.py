"""Linears that read one input, run as one stacked call (q/k/v; cross-attention k/v).

A DiT block feeds the same tensor to several LoRA linears: self-attention q, k, v take
the normed hidden states, cross-attention k, v take the text context
(reference/livewan_wan21/wan/modules/model.py:123-126). The reference notices this only
to reuse one fp32 cast of that tensor across the PEFT modules, keyed by tensor
identity and in-place version (runtime/wan13b_lora_cast.py:265-300). Here the linears
themselves are stacked: ``fuse_shared_inputs(model, [["q", "k", "v"], ["cross.k",
"cross.v"]])`` links each group's modules to one ``SharedInputGroup``. When the first
member is called with a tensor, the group runs every member on it in one stacked call
(shrinks of X by the stacked A, 256 rank columns per call; one GEMM over the stacked bases;
their dX summed in one dX GEMM; the dA of every 256-column slice from one reduction over X)
and hands each member its output; the other members, called with the same unmodified tensor
(same object, same in-place version, same routing and grad mode), get theirs without another
launch.

Members are the LoRA linears of every call site this package serves: MultiLoRALinear (roles
as segments), the single-adapter wrappers (TrainableLowRankLinear, the native LoRALinear,
LiveWan's layout, its own class or the reference's after install_livewan_multi_lora) and PEFT
LoRA layers after install_peft_multi_lora (their active adapter, or the active role batch).
The stacked call computes what the members' own calls compute (bf16 adapters, or fp32
masters at fp32-class precision over a bf16 base), each member with its own adapters (PEFT
members may be on different active adapters of one rank and scaling); a call whose members
would not stack (a disabled LiveWan member, disabled PEFT adapters, different routings or
scales, float32 inputs) runs each member on its own.

The modules keep their parameters, names and state-dict keys; the stacked call reads
the members' own adapter Parameters, so gradients reach each member's adapters, and a
stacked bf16 copy of their frozen bases (and its transpose for dX), made once per set of
bases and remade when one of them changes. An output that nobody consumes is still computed
(and kept until the group's next call); a group is for linears that are all called on the
tensor.
"""
from __future__ import annotations

from typing import Sequence

import torch
from torch import nn

from . import _lib, peft_site
from .function import shared_input_multi_lora
from .livewan import LiveWanLoRALinear, livewan_forward
from .low_rank import LoRALinear, MultiLoRALinear, TrainableLowRankLinear, lora_pair
from .routing import BASE_ONLY, SegmentRouting


def _require(value, message):
    if not value:
        raise ValueError('shared input: ' + message)


def _rows(x: torch.Tensor) -> int:
    return x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0


def _family(m: nn.Module) -> str | None:
    """'multi' (MultiLoRALinear), 'peft' (an installed PEFT layer), 'pair' (a single-adapter
    wrapper whose forward consults its group), or None."""
    if isinstance(m, MultiLoRALinear):
        return 'multi'
    if peft_site.is_peft_lora_linear(m):
        return 'peft' if peft_site.is_installed(m) else None
    if lora_pair(m) is None:
        return None
    if isinstance(m, (TrainableLowRankLinear, LoRALinear, LiveWanLoRALinear)):
        return 'pair'
    return 'pair' if getattr(m.__dict__.get('forward'), '__func__', None) is livewan_forward else None


def _base(m: nn.Module) -> nn.Linear:
    return m.base_layer if peft_site.is_peft_lora_linear(m) else m.base


def _static_adapters(m: nn.Module, family: str) -> dict:
    """{adapter key: (rank, scale)}: list positions for 'multi' / 'pair', names for 'peft'."""
    if family == 'multi':
        return {i: (int(a.shape[0]), float(s)) for i, (a, s) in enumerate(zip(m.lora_a, m.scales))}
    if family == 'pair':
        a, _, s = lora_pair(m)
        return {0: (int(a.shape[0]), s)}
    return {n: (int(m.lora_A[n].weight.shape[0]), float(m.scaling[n])) for n in m.lora_A}


def _plan(m: nn.Module, family: str, x: torch.Tensor, routing: SegmentRouting | None):
    """(lora_as, lora_bs, scales, routing) of member m's own call on x."""
    rows = _rows(x)
    if family == 'multi':
        return list(m.lora_a), list(m.lora_b), list(m.scales), routing or m.role_routing(rows)
    if family == 'peft':
        names, r = peft_site.peft_plan(m, x)
        return ([m.lora_A[n].weight for n in names], [m.lora_B[n].weight for n in names],
                [float(m.scaling[n]) for n in names], r)
    if not getattr(m, 'enabled', True):  # a disabled LiveWan module: the base alone
        return [], [], [], SegmentRouting.single(rows, BASE_ONLY)
    a, b, s = lora_pair(m)
    return [a], [b], [s], SegmentRouting.single(rows, 0)


def _single(m: nn.Module, family: str, x: torch.Tensor, routing: SegmentRouting | None) -> torch.Tensor:
    """Member m's own call."""
    if family == 'peft':
        return peft_site._peft_single(m, x)
    return m._single(x, routing)


class SharedInputGroup:
    """Members (LoRA linears of one family, see the module doc) that read one input."""

    def __init__(self, members: Sequence[nn.Module], names: Sequence[str] = ()):
        members = list(members)
        _require(len(members) >= 2, 'a group needs at least two linears')
        families = [_family(m) for m in members]
        _require(None not in families, 'members must be LoRA linears on the multi-LoRA op')
        _require(len(set(families)) == 1, 'members must be all MultiLoRALinear, all single-adapter LoRA linears '
                 'or all PEFT layers')
        family = families[0]
        _require(all(getattr(m, 'base_wq', None) is None for m in members), 'e4m3 bases are not stacked')
        bases = [_base(m) for m in members]
        K = bases[0].in_features
        _require(all(b.in_features == K for b in bases), 'members must have one in_features')
        ads = [_static_adapters(m, family) for m in members]
        _require(all(len(a) == len(ads[0]) for a in ads), 'members must have the same number of adapters')
        _require(all(a.keys() == ads[0].keys() for a in ads), 'members must have the same adapters')
        ranks = {r for a in ads for r, _ in a.values()}
        _require(len(ranks) == 1 and next(iter(ranks)) % 16 == 0,
                 f'one LoRA rank, a multiple of 16, for every member and adapter (got {sorted(ranks)})')
        rank = next(iter(ranks))
        _require(rank <= _lib.MAX_RANK, f'rank {rank} is above the kernels\' {_lib.MAX_RANK}')
        for key in ads[0]:
            _require(len({a[key][1] for a in ads}) == 1, f'adapter {key} has different scales across members')
        if family == 'multi':
            _require(all(m.role_ids == members[0].role_ids for m in members), 'members route different roles')
        self.members = members
        self.names = tuple(names)
        self.family = family
        self.K, self.n, self.rank = K, len(ads[0]), rank
        self.launches = 0      # stacked calls run (for tests and accounting)
        self._out = None       # (input, key, outputs, members not yet served)

    def _stackable(self, x: torch.Tensor) -> bool:
        """The stacked call is the bf16 path: under bf16 autocast, or bf16 input over bf16 bases
        (bf16 adapters, or fp32 masters at fp32-class precision). float32 inputs run per member."""
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
            return True
        return x.dtype == torch.bfloat16 and all(_base(m).weight.dtype == torch.bfloat16 for m in self.members)

    def __call__(self, member: nn.Module, x: torch.Tensor, routing: SegmentRouting | None = None) -> torch.Tensor:
        if x.is_inference() or not self._stackable(x):  # one call per linear
            return _single(member, self.family, x, routing)
        idx = next(i for i, m in enumerate(self.members) if m is member)
        own = _plan(member, self.family, x, routing)
        key = (x._version, own[3], torch.is_grad_enabled(), torch.is_autocast_enabled("cuda"))
        if self._out is not None and self._out[0] is x and self._out[1] == key and idx in self._out[3]:
            _, _, outs, pending = self._out
            pending.discard(idx)
            if not pending:
                self._out = None
            return outs[idx]
        plans = [own if i == idx else _plan(m, self.family, x, routing) for i, m in enumerate(self.members)]
        if not self._plans_stack(plans):
            self._out = None
            return _single(member, self.family, x, routing)
        outs = shared_input_multi_lora(x, [_base(m).weight for m in self.members],
                                       [_base(m).bias for m in self.members],
                                       [p[0] for p in plans], [p[1] for p in plans], plans[0][2], own[3],
                                       all(getattr(m, 'transposed_base_for_dx', True) for m in self.members))
        self.launches += 1
        pending = set(range(len(self.members))) - {idx}
        self._out = (x, key, outs, pending) if pending else None
        return outs[idx]

    @staticmethod
    def _plans_stack(plans) -> bool:
        """The members' calls share one routing, adapter count, scales and rank (a multiple of 16)."""
        As0, _, scales0, routing0 = plans[0]
        if not As0:
            return False
        R = int(As0[0].shape[0])
        return all(p[3] == routing0 and len(p[0]) == len(As0) and list(p[2]) == list(scales0)
                   and all(int(a.shape[0]) == R for a in p[0]) for p in plans) and R % 16 == 0

    def release(self) -> None:
        """Drop the cached outputs."""
        self._out = None


def fuse_shared_inputs(model: nn.Module, groups: Sequence[Sequence[str]]) -> list[SharedInputGroup]:
    """Link each group of named LoRA linears of ``model`` (e.g. ``[["q", "k", "v"]]``) into a
    SharedInputGroup. Fails closed (ValueError) when a name is missing, already grouped, not a
    LoRA linear on the multi-LoRA op (a PEFT layer or a reference-layout LiveWan module needs its
    install_* call first), or the group cannot be stacked (different in_features, adapters,
    ranks, scales or roles)."""
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
            if _family(mod) is None:
                hint = ''
                if peft_site.is_peft_lora_linear(mod):
                    hint = ' (a PEFT layer: call install_peft_multi_lora first)'
                elif lora_pair(mod) is not None:
                    hint = ' (call install_livewan_multi_lora first)'
                raise ValueError(f'shared input: {name!r} is not a LoRA linear on the multi-LoRA op{hint}')
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
