"""Multi-role call site: several roles' forwards as one pass over the shared frozen base.

The reference calls every role on its own batch: the teacher and the fake critic each
run a full denoise (training/dmd.py:324-345), and LiveWan batches the teacher's
conditional and unconditional passes (``torch.cat([z_t, z_t])``) under
``lora_enabled(teacher, False)`` and then runs the critic separately
(runtime/livewan_crossscale_worker.py:2614-2645). Roles can share one base because
frozen construction aliases their frozen Parameters by canonical name
(training/construction_sharing.py:35-48,58-102; ``x.base.weight`` of a LoRA wrapper is
``x.weight`` of the teacher) while adapters and buffers stay per role
(tests/test_training_construction.py:79-94).

Here those roles become one module tree and one call:

* ``fuse_roles({'teacher': t, 'fake': f, ...})`` checks the aliasing (every frozen
  Parameter one object across roles, buffers equal, no trainable Parameter outside a
  LoRA wrapper) and returns a module tree that shares every tensor with the roles, in
  which each LoRA target is a ``MultiLoRALinear`` over the roles' own ``lora_a`` /
  ``lora_b`` Parameters (so each role's optimizer keeps owning exactly its trainables).
  A role without an adapter at a target (the teacher) is base-only there.
* ``RoleBatch([('teacher', 2 * B), ('fake', B)])`` names the roles of the samples
  concatenated along the batch dimension (``cat`` / ``split``);
  ``with roles_active(fused, batch): fused(...)`` runs the model once, and every fused
  linear turns the batch into a SegmentRouting over its own rows, whatever its rows per
  sample are (video tokens for self-attention, text tokens for cross-attention k/v).

Row order contract: a fused linear's input is sample-major (leading dimension the
batch, or rows flattened batch-major), so sample i's rows are contiguous.
"""
from __future__ import annotations

import copy
from contextlib import contextmanager
from dataclasses import dataclass
from typing import Iterator, Mapping, Sequence

import torch
from torch import nn

from .low_rank import MultiLoRALinear, lora_pair
from .routing import BASE_ONLY, SegmentRouting


def _require(value, message):
    if not value:
        raise ValueError('multi-role call: ' + message)


@dataclass(frozen=True)
class RoleBatch:
    """Roles of a batch concatenated along dimension 0: ((role, samples), ...) in order."""
    parts: tuple[tuple[str, int], ...]

    def __init__(self, parts: Sequence[tuple[str, int]]):
        parts = tuple((str(name), int(n)) for name, n in parts)
        _require(len(parts) > 0, 'a role batch needs at least one role')
        _require(all(n >= 0 for _, n in parts), 'sample counts must be >= 0')
        object.__setattr__(self, 'parts', parts)

    @property
    def samples(self) -> int:
        return sum(n for _, n in self.parts)

    def cat(self, tensors: Sequence[torch.Tensor]) -> torch.Tensor:
        """Concatenate one tensor per part along dimension 0 (sizes checked)."""
        _require(len(tensors) == len(self.parts), f'{len(self.parts)} tensors required, got {len(tensors)}')
        for (name, n), t in zip(self.parts, tensors):
            _require(t.dim() >= 1 and t.shape[0] == n, f'role {name!r} has {n} samples, tensor has '
                     f'{t.shape[0] if t.dim() else 0}')
        return torch.cat(list(tensors), dim=0)

    def split(self, t: torch.Tensor) -> tuple[torch.Tensor, ...]:
        """Views of ``t`` [samples, ...] per part, in order."""
        _require(t.dim() >= 1 and t.shape[0] == self.samples, f'tensor has {t.shape[0] if t.dim() else 0} '
                 f'samples, batch has {self.samples}')
        return tuple(torch.split(t, [n for _, n in self.parts], dim=0))

    def routing(self, rows: int, role_ids: Mapping[str, int]) -> SegmentRouting:
        """Routing of ``rows`` sample-major rows: rows / samples per sample, each part's rows
        to its role's adapter id (roles absent from ``role_ids`` are base-only); empty parts
        are dropped and adjacent parts with the same id form one segment."""
        total = self.samples
        _require(total > 0 and rows % total == 0, f'{rows} rows do not split into {total} samples')
        per = rows // total
        lengths: list[int] = []
        ids: list[int] = []
        for name, n in self.parts:
            if n == 0:
                continue
            a = int(role_ids.get(name, BASE_ONLY))
            if ids and ids[-1] == a:
                lengths[-1] += n * per
            else:
                lengths.append(n * per)
                ids.append(a)
        return SegmentRouting.from_lengths(lengths, ids)


def _fused_linears(model: nn.Module) -> Iterator[MultiLoRALinear]:
    return (m for m in model.modules() if isinstance(m, MultiLoRALinear))


@contextmanager
def roles_active(model: nn.Module, batch: RoleBatch):
    """Route every fused linear of ``model`` by ``batch`` inside the block (restored after)."""
    _require(isinstance(batch, RoleBatch), 'a RoleBatch is required')
    mods = list(_fused_linears(model))
    _require(mods, 'the model has no fused multi-role linear (build it with fuse_roles)')
    known = set().union(*(m.role_ids for m in mods))
    for name, _ in batch.parts:
        _require(name in known or name in getattr(model, 'role_names', ()), f'unknown role {name!r}')
    prev = [m.active_roles for m in mods]
    for m in mods:
        m.active_roles = batch
    try:
        yield model
    finally:
        for m, p in zip(mods, prev):
            m.active_roles = p


def _canonical(name: str, wrappers: Sequence[str]) -> str:
    """Parameter name with a LoRA wrapper's ``.base.`` removed (construction_sharing.py:38-47)."""
    for w in wrappers:
        prefix = w + '.base.'
        if name.startswith(prefix):
            return w + '.' + name[len(prefix):]
    return name


def _is_wrapper(mod: nn.Module) -> bool:
    return not isinstance(mod, MultiLoRALinear) and lora_pair(mod) is not None


def fuse_roles(roles: Mapping[str, nn.Module], base_roles: Sequence[str] = ()) -> nn.Module:
    """One module tree running every role of ``roles`` (name -> role model) in one pass.

    LoRA wrappers are TrainableLowRankLinear modules, native-model LoRALinear modules or
    modules of LiveWan's LoRA layout (``a`` / ``b`` / ``enabled``, wanstreamer/lora.py:8-27).
    Roles named in ``base_roles`` use the frozen base alone at every target even where their
    model holds wrappers: LiveWan's teacher pass is the critic model under
    ``lora_enabled(model, False)`` (runtime/livewan_crossscale_worker.py:2614-2632), so
    ``fuse_roles({'teacher': critic, 'critic': critic}, base_roles=('teacher',))`` runs both
    passes in one call per linear. One model object may serve several roles only if all but
    one of them are base roles.

    Fail-closed checks (``ValueError('multi-role call: …')``): the roles have the same
    module structure up to LoRA wrappers; every frozen Parameter is the same object in
    every role (the shared construction aliases them); every trainable Parameter is a
    wrapper's adapter; buffers are equal in dtype, shape and value.
    The result shares all of these tensors; it holds no copy of any of them.
    """
    _require(isinstance(roles, Mapping) and len(roles) > 0, 'a mapping of role name -> module is required')
    names = list(roles)
    models = [roles[n] for n in names]
    _require(all(isinstance(m, nn.Module) for m in models), 'roles must be nn.Module trees')
    base_roles = tuple(base_roles)
    _require(all(r in names for r in base_roles), f'base roles {base_roles} must name roles of the mapping')
    adapter_models = [m for n, m in zip(names, models) if n not in base_roles]
    _require(len({id(m) for m in adapter_models}) == len(adapter_models),
             'one model object serves two adapter roles (make all but one of them base roles)')

    wrappers = [sorted((k for k, mod in m.named_modules() if _is_wrapper(mod)), key=len, reverse=True)
                for m in models]
    targets = sorted(set().union(*wrappers))

    # module structure: same names and types, a wrapper where another role has its plain Linear
    ref_mods = None
    for name, m, wr in zip(names, models, wrappers):
        inner = {k + '.base' for k in wr}
        mods = {}
        for k, mod in m.named_modules():
            if k in inner:
                continue
            mods[k] = nn.Linear if _is_wrapper(mod) else type(mod)
        if ref_mods is None:
            ref_mods = mods
        _require(mods == ref_mods, f'role {name!r} has a different module structure')
    for t in targets:
        _require(ref_mods.get(t) is nn.Linear, f'LoRA target {t!r} is not an nn.Linear in every role')

    # parameters: frozen ones aliased by canonical name, trainable ones only LoRA
    frozen_ref: dict[str, nn.Parameter] | None = None
    for name, m, wr in zip(names, models, wrappers):
        lora = {id(p) for k in wr for p in lora_pair(m.get_submodule(k))[:2]}
        frozen: dict[str, nn.Parameter] = {}
        for pname, p in m.named_parameters(remove_duplicate=False):
            if id(p) in lora:
                continue
            _require(not p.requires_grad, f'role {name!r} trains {pname!r}, which is not a LoRA adapter')
            frozen[_canonical(pname, wr)] = p
        if frozen_ref is None:
            frozen_ref = frozen
            continue
        _require(frozen.keys() == frozen_ref.keys(), f'role {name!r} has different frozen parameters')
        for k, p in frozen.items():
            _require(p is frozen_ref[k], f'frozen parameter {k!r} of role {name!r} is not shared with role '
                     f'{names[0]!r} (build the roles with the shared frozen construction)')

    # buffers: owned per role, equal in value
    ref_bufs = dict(models[0].named_buffers())
    for name, m in zip(names[1:], models[1:]):
        bufs = dict(m.named_buffers())
        _require(bufs.keys() == ref_bufs.keys(), f'role {name!r} has different buffers')
        for k, b in bufs.items():
            r = ref_bufs[k]
            _require(b.dtype == r.dtype and b.shape == r.shape and b.device == r.device and torch.equal(b, r),
                     f'buffer {k!r} of role {name!r} differs from role {names[0]!r}')

    # the fused tree: the first role's structure, every tensor shared, targets batched
    template = models[0]
    memo = {id(t): t for t in template.parameters()}
    memo.update({id(t): t for t in template.buffers()})
    fused = copy.deepcopy(template, memo)
    for t in targets:
        base_linear = None
        adapters: list[tuple[str, nn.Module]] = []
        for name, m in zip(names, models):
            mod = m.get_submodule(t)
            if _is_wrapper(mod):
                if name not in base_roles:
                    adapters.append((name, mod))
                base_linear = base_linear or mod.base
            elif base_linear is None:
                base_linear = mod
        fused.set_submodule(t, MultiLoRALinear.from_roles([w for _, w in adapters], base=base_linear,
                                                          role_names=[n for n, _ in adapters]))
    fused.role_names = tuple(names)
    return fused
