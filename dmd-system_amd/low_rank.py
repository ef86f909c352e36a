"""Drop-in LoRA modules over a shared frozen base, backed by the HIP kernels.

Mirrors the reference's native LoRA interface (training/low_rank.py):
``TrainableLowRankLinear(base, rank=, alpha=)`` with parameters ``base``,
``lora_a`` [r, in] (Kaiming-uniform, a=sqrt(5)), ``lora_b`` [out, r] (zeros),
``scale = alpha / rank``, and ``trainable_scope(native, config)`` with the
same schema and the same fail-closed ``ValueError`` messages. Checkpoint keys
are therefore unchanged (training/checkpoint.py:177 packs named parameters).

``MultiLoRALinear`` is the batched form: one frozen base, several adapters
(``lora_a.{i}``, ``lora_b.{i}``) and a SegmentRouting per call, so that the
generator and fake-critic roles (and base-only teacher rows) share one
launch of the base GEMM.
"""
from __future__ import annotations

import math
import weakref
from typing import Sequence

import torch
from torch import nn

from .function import multi_lora_linear, multi_lora_linear_fp8, multi_lora_linear_gated
from .kernels import quantize_rows_fp8
from .routing import SegmentRouting


def _require(value, message):
    if not value:
        raise ValueError('native trainable scope: ' + message)


# Transposed copies of frozen base weights, one per weight tensor: every module that aliases
# one base (shared construction, fused roles, TrainableLowRankLinear and MultiLoRALinear
# over the same Parameter) uses the same copy. Keyed by the weight's identity (tensors do
# not hash by value); an entry is dropped when its weight tensor is freed.
_BASE_T: dict[int, tuple] = {}


def _drop_base_t(key: int) -> None:
    _BASE_T.pop(key, None)


def transposed_base(w: torch.Tensor, x: torch.Tensor, enabled: bool = True) -> torch.Tensor | None:
    """The frozen base weight ``w`` transposed ([in, out] bf16, contiguous), for the NT form of
    the dX GEMM (3-5% faster than the NN form at the Wan shapes); made on the first forward that
    will need dX and remade when the weight changes (storage, in-place version, device). It
    costs in·out·2 bytes per distinct base weight, shared by every module over that weight; not
    a buffer, so no state-dict entry. None when no dX will be computed, on the float32 path (no
    bf16 GEMM), or when not ``enabled`` (then dX runs on the NN kernel and no copy is kept)."""
    if not (enabled and torch.is_grad_enabled() and x.requires_grad):
        return None
    autocast = torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16
    if not autocast and w.dtype != torch.bfloat16:
        return None
    key = (w.data_ptr(), w._version, w.device)
    entry = _BASE_T.get(id(w))
    if entry is None or entry[0]() is not w:
        entry = (weakref.ref(w), None, None)
        weakref.finalize(w, _drop_base_t, id(w))
    if entry[1] != key:
        with torch.no_grad():
            entry = (entry[0], key, w.detach().to(torch.bfloat16).t().contiguous())
    _BASE_T[id(w)] = entry
    return entry[2]


# Stacked copies of the frozen bases of linears that read one input (q / k / v), keyed by the
# identities of the member weights and biases: (weights stacked by rows [G·N, K] bf16, biases
# stacked [G·N] or None, and the stack transposed [K, G·N] when dX needs it). Entries are remade
# when a member tensor changes (storage or in-place version) or is replaced by another object,
# and dropped as soon as any member weight or bias is freed.
_STACKED: dict[tuple, tuple] = {}


def _drop_stacked(key: tuple) -> None:
    _STACKED.pop(key, None)


def stacked_bases(weights, biases, want_t: bool):
    """(w_cat, b_cat, w_cat_t or None) for the frozen bases of stacked linears. Costs the bases'
    bf16 size once more (twice with the transpose), per distinct set of bases."""
    members = [*weights, *(b for b in biases if b is not None)]
    ident = tuple(id(w) for w in weights) + tuple(id(b) if b is not None else 0 for b in biases)
    ver = tuple((w.data_ptr(), w._version) for w in weights) + tuple(
        (b.data_ptr(), b._version) if b is not None else (0, 0) for b in biases)
    entry = _STACKED.get(ident)
    if entry is None or len(entry[0]) != len(members) or any(r() is not t for r, t in zip(entry[0], members)):
        # a new set of tensors (an id can be reused by a later object: compare the objects themselves)
        entry = (tuple(weakref.ref(t) for t in members), None, None, None, None)
        for t in members:
            weakref.finalize(t, _drop_stacked, ident)
    refs, v, w_cat, b_cat, w_cat_t = entry
    if v != ver:
        with torch.no_grad():
            w_cat = torch.cat([w.detach().to(torch.bfloat16) for w in weights]).contiguous()
            b_cat = None
            if any(b is not None for b in biases):  # float32 holds bf16 and fp32 biases exactly
                b_cat = torch.cat([b.detach().float() if b is not None else
                                   torch.zeros(w.shape[0], device=w.device) for w, b in zip(weights, biases)])
        w_cat_t = None
    if want_t and w_cat_t is None:
        with torch.no_grad():
            w_cat_t = w_cat.t().contiguous()
    _STACKED[ident] = (refs, ver, w_cat, b_cat, w_cat_t)
    return w_cat, b_cat, w_cat_t


def _base_t(module: nn.Module, x: torch.Tensor) -> torch.Tensor | None:
    """transposed_base of ``module.base.weight``; ``module.transposed_base_for_dx = False`` turns
    the copy off for that module."""
    return transposed_base(module.base.weight, x, getattr(module, 'transposed_base_for_dx', True))


def _init_pair(rank: int, base: nn.Linear, dtype=None) -> tuple[nn.Parameter, nn.Parameter]:
    # low_rank.py:21-23: A Kaiming-uniform(a=sqrt(5)) i.e. U(±1/sqrt(in)), B zeros
    dt = dtype or base.weight.dtype
    a = nn.Parameter(torch.empty(rank, base.in_features, device=base.weight.device, dtype=dt))
    b = nn.Parameter(torch.zeros(base.out_features, rank, device=base.weight.device, dtype=dt))
    nn.init.kaiming_uniform_(a, a=5 ** .5)
    return a, b


def lora_pair(m: nn.Module):
    """(A [r, in], B [out, r], scale) of a single-adapter LoRA wrapper over ``m.base``: a
    TrainableLowRankLinear (``lora_a`` / ``lora_b``), a native LoRALinear or a module of LiveWan's
    layout (``a`` / ``b``); None for anything else."""
    base = getattr(m, 'base', None)
    if not isinstance(base, nn.Linear):
        return None
    for an, bn in (('lora_a', 'lora_b'), ('a', 'b')):
        a, b = getattr(m, an, None), getattr(m, bn, None)
        if (isinstance(a, nn.Parameter) and isinstance(b, nn.Parameter) and a.dim() == 2 and b.dim() == 2
                and a.shape[1] == base.in_features and b.shape == (base.out_features, a.shape[0])
                and isinstance(getattr(m, 'scale', None), (int, float))):
            return a, b, float(m.scale)
    return None


class TrainableLowRankLinear(nn.Module):
    """Frozen W*x + (alpha/rank)*B(A*x), with separately owned trainable A/B.

    Same constructor contract as training/low_rank.py:13-24; forward runs the
    HIP multi-LoRA path with one adapter over all rows.
    """

    def __init__(self, base, *, rank, alpha):
        super().__init__()
        _require(type(base) is nn.Linear and type(rank) is int and 0 < rank <= min(base.in_features, base.out_features)
                 and type(alpha) in (int, float) and math.isfinite(alpha) and alpha > 0,
                 'invalid native Linear LoRA scope/rank/alpha')
        self.base = base.requires_grad_(False)
        self.lora_a, self.lora_b = _init_pair(rank, base)
        self.scale = float(alpha) / rank

    def forward(self, value):
        group = self.__dict__.get('shared_input')
        if group is not None:  # stacked with the other linears that read this input
            return group(self, value)
        return self._single(value)

    def _single(self, value, routing=None):
        rows = value.numel() // value.shape[-1] if value.dim() else 0
        return multi_lora_linear(value, self.base.weight, self.base.bias, [self.lora_a], [self.lora_b],
                                 [self.scale], SegmentRouting.single(rows, 0), weight_t=_base_t(self, value))

    def gated_residual(self, value, residual, gate):
        """``residual + self(value) * gate`` of a DiT block (model.py:305-313), fused into the
        GEMM epilogue (bf16 or float32 residual stream, output in its dtype; frozen fp32 gate)."""
        rows = value.numel() // value.shape[-1] if value.dim() else 0
        return multi_lora_linear_gated(value, self.base.weight, self.base.bias, [self.lora_a], [self.lora_b],
                                       [self.scale], SegmentRouting.single(rows, 0), residual, gate,
                                       weight_t=_base_t(self, value))


def trainable_scope(native, config):
    """Install TrainableLowRankLinear on the named nn.Linear targets (training/low_rank.py:31-50)."""
    _require(isinstance(config, dict) and config.get('mode') in ('full', 'lora'), 'explicit full or lora trainable scope required')
    if config['mode'] == 'full':
        _require(set(config) == {'mode'}, 'full mode accepts no ignored LoRA settings')
        native.requires_grad_(True)
        return
    _require(set(config) == {'mode', 'rank', 'alpha', 'targets'} and isinstance(config['targets'], list)
             and config['targets'] and all(isinstance(name, str) and name for name in config['targets'])
             and len(config['targets']) == len(set(config['targets'])), 'exact nonempty native Linear LoRA targets required')
    targets = {}
    for name in config['targets']:
        try:
            targets[name] = native.get_submodule(name)
        except AttributeError as exc:
            raise ValueError('missing actual native LoRA target: ' + name) from exc
        _require(type(targets[name]) is nn.Linear, 'LoRA target is not an actual native Linear: ' + name)
    native.requires_grad_(False)
    for name, module in targets.items():
        native.set_submodule(name, TrainableLowRankLinear(module, rank=config['rank'], alpha=config['alpha']))


class LoRALinear(nn.Module):
    """The reference's parameterised native LoRA (native/models.py:33-51), on the HIP path.

    Frozen ``base`` (bf16 in the native models, models.py:150-156) and fp32 masters ``a``
    [r, in] (Kaiming-uniform, a=sqrt(5)) and ``b`` [out, r] (zeros), ``scale = alpha /
    rank``. The reference computes update = F.linear(F.linear(x.float(), a), b) in fp32 and
    returns (base(x).float() + update·scale).to(base dtype); here the shrinks use the masters
    at fp32-class precision (hi + lo bf16 parts) and the base GEMM adds the update in its fp32
    accumulators before one rounding to the base dtype. A float32 base runs the float32 path.
    ``use_fused`` / ``fused_calls`` keep the reference's switch and counter for its no-grad
    fused epilogue (wan13b_lora_epilogue.py:55-92); the epilogue is always fused here.
    """

    def __init__(self, base: nn.Linear, task) -> None:
        super().__init__()
        self.base = base.requires_grad_(False)
        self.scale = float(task.lora_alpha / task.lora_rank)
        dev = base.weight.device
        self.a = nn.Parameter(torch.empty(task.lora_rank, base.in_features, dtype=torch.float32, device=dev))
        self.b = nn.Parameter(torch.zeros(base.out_features, task.lora_rank, dtype=torch.float32, device=dev))
        nn.init.kaiming_uniform_(self.a, a=5 ** 0.5)
        self.use_fused = False
        self.fused_calls = 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.use_fused and not torch.is_grad_enabled():
            self.fused_calls += 1
        group = self.__dict__.get('shared_input')
        if group is not None:  # stacked with the other linears that read this input
            return group(self, x)
        return self._single(x)

    def _single(self, x: torch.Tensor, routing=None) -> torch.Tensor:
        rows = x.numel() // x.shape[-1] if x.dim() else 0
        return multi_lora_linear(x, self.base.weight, self.base.bias, [self.a], [self.b], [self.scale],
                                 SegmentRouting.single(rows, 0), weight_t=_base_t(self, x))


def install_lora(model: nn.Module, task) -> list[str]:
    """Replace the nn.Linear modules named (or suffixed ``.<key>``) by ``task.target_modules``
    with LoRALinear (native/models.py:54-64): same matching, the same ValueError messages for
    no match or an unmatched key; returns the replaced names."""
    model.requires_grad_(False)
    found = [(name, mod) for name, mod in model.named_modules() if isinstance(mod, nn.Linear)
             and any(name == key or name.endswith("." + key) for key in task.target_modules)]
    if not found:
        raise ValueError("no matching LoRA targets in native model; cannot silently train zero parameters")
    for key in task.target_modules:
        if not any(n == key or n.endswith("." + key) for n, _ in found):
            raise ValueError(f"unmatched LoRA target: {key}")
    for name, mod in found:
        parent, _, leaf = name.rpartition(".")
        setattr(model.get_submodule(parent) if parent else model, leaf, LoRALinear(mod, task))
    return [n for n, _ in found]


def _routing_from_arrays(seg_offsets, adapter_ids) -> SegmentRouting:
    """SegmentRouting from segment offsets [S+1] and adapter ids [S] (integer sequences or CPU
    tensors: the routing is host data, read when the kernels are launched)."""
    def ints(v, name):
        if isinstance(v, torch.Tensor):
            if v.is_cuda or v.is_floating_point() or v.dim() != 1:
                raise ValueError(f'multi-LoRA linear: {name} must be a 1-D integer CPU tensor or a sequence')
            v = v.tolist()
        if v is None:
            raise ValueError(f'multi-LoRA linear: {name} is required with adapter_ids')
        return [int(e) for e in v]
    return SegmentRouting(tuple(ints(seg_offsets, 'seg_offsets')), tuple(ints(adapter_ids, 'adapter_ids')))


class MultiLoRALinear(nn.Module):
    """One frozen base nn.Linear shared by several adapters, routed by segment.

    ``forward(x, routing)``: x [..., in]; routing a SegmentRouting over the
    flattened rows (adapter id -1 = base only, the teacher role), or, with no
    routing, the RoleBatch that ``roles.roles_active`` set on the module.
    """

    def __init__(self, base: nn.Linear, *, ranks: Sequence[int], alphas: Sequence[float], dtype=None):
        super().__init__()
        _require(type(base) is nn.Linear, 'multi-LoRA base must be an actual native Linear')
        _require(len(ranks) == len(alphas) and len(ranks) > 0, 'one alpha per adapter rank required')
        for r, al in zip(ranks, alphas):
            _require(type(r) is int and 0 < r <= min(base.in_features, base.out_features)
                     and type(al) in (int, float) and math.isfinite(al) and al > 0,
                     'invalid native Linear LoRA scope/rank/alpha')
        self.base = base.requires_grad_(False)
        pairs = [_init_pair(r, base, dtype) for r in ranks]
        self.lora_a = nn.ParameterList([a for a, _ in pairs])
        self.lora_b = nn.ParameterList([b for _, b in pairs])
        self.scales = [float(al) / r for r, al in zip(ranks, alphas)]
        self.role_ids: dict[str, int] = {}  # role name -> adapter id (multi-role call sites)
        self.active_roles = None             # RoleBatch routing calls without an explicit routing

    @classmethod
    def from_roles(cls, roles: Sequence[nn.Module], *, base: nn.Linear | None = None,
                   role_names: Sequence[str] | None = None) -> "MultiLoRALinear":
        """Batch per-role LoRA wrappers that alias one frozen base.

        A wrapper is a TrainableLowRankLinear (``lora_a`` / ``lora_b``), a native-model
        LoRALinear (``a`` / ``b`` fp32 masters) or a module of LiveWan's LoRA layout (``a`` /
        ``b`` and an ``enabled`` flag, wanstreamer/lora.py:8-27). The adapters are the roles'
        own Parameters (not copies), so each role's optimizer keeps owning exactly its
        trainables (open_workload/dmd.py:266-275); the base must be the same Parameter object
        in every role, as construction_sharing.place_frozen_role arranges
        (construction_sharing.py:105-118). ``base`` (default: the first role's) may be a
        base-only role's own nn.Linear over the same Parameters; ``role_names`` names the roles
        in order, adapter i being role_names[i] (used by a RoleBatch routing); with no roles the
        module is the base alone (every role base-only). A wrapper with
        an ``enabled`` flag that is False when a RoleBatch routes a call leaves its role's rows
        base-only (LiveWan's ``lora_enabled(model, False)``).
        """
        _require(len(roles) > 0 or base is not None, 'at least one role module (or the base) required')
        pairs = [lora_pair(m) for m in roles]
        _require(all(p is not None for p in pairs),
                 'roles must be LoRA wrappers (TrainableLowRankLinear, LoRALinear or LiveWan LoRA)')
        base = roles[0].base if base is None else base
        _require(type(base) is nn.Linear, 'multi-LoRA base must be an actual native Linear')
        for m in roles:
            _require(m.base.weight is base.weight and m.base.bias is base.bias,
                     'roles must alias one frozen base (shared construction)')
        names = list(role_names) if role_names is not None else []
        _require(role_names is None or (len(names) == len(roles) and len(set(names)) == len(names)),
                 'one distinct role name per adapter required')
        obj = cls.__new__(cls)
        nn.Module.__init__(obj)
        obj.base = base
        obj.lora_a = nn.ParameterList([a for a, _, _ in pairs])
        obj.lora_b = nn.ParameterList([b for _, b, _ in pairs])
        obj.scales = [s for _, _, s in pairs]
        obj.role_ids = {n: i for i, n in enumerate(names)}
        obj.active_roles = None
        # the source wrappers (not submodules: no second state-dict entry), for their enabled flags
        obj.__dict__['_role_wrappers'] = list(roles)
        return obj

    @property
    def num_adapters(self) -> int:
        return len(self.scales)

    def quantize_base_fp8(self, dx_bf16: bool | None = None) -> "MultiLoRALinear":
        """Store the frozen base weight as e4m3 with one fp32 scale per output
        channel (buffers ``base_wq`` [out, in], ``base_wscale`` [out]); forward and dX
        then run on the e4m3 MFMA. The bf16/fp32 ``base.weight`` is left in place for
        its other users (shared construction aliases it). The e4m3 copy follows the
        weight: if ``base.weight`` changes (in place, or by a state-dict load) it is
        quantised again on the next call; ``base_wq`` transposed (for the e4m3 dX) is
        remade whenever ``base_wq`` changes. ``dx_bf16=True`` runs dX on the bf16 MFMA
        against the dequantised base instead (dY not quantised; +16-17% per fwd+bwd step at config 5)."""
        if dx_bf16 is not None:
            self.__dict__['_fp8_dx_bf16'] = bool(dx_bf16)
        w = self.base.weight.detach().to(torch.bfloat16).contiguous()
        wq, ws = quantize_rows_fp8(w)
        if getattr(self, "base_wq", None) is None:
            self.register_buffer("base_wq", wq, persistent=True)
            self.register_buffer("base_wscale", ws, persistent=True)
        else:
            with torch.no_grad():
                self.base_wq.copy_(wq)
                self.base_wscale.copy_(ws)
        self.__dict__['_wq_source'] = self._weight_key()
        return self

    def _weight_key(self):
        w = self.base.weight
        return (w.data_ptr(), w._version, w.device)

    def _fp8_base(self):
        """(base_wq, base_wscale, base_wq transposed), requantised / re-transposed when stale."""
        if self.__dict__.get('_wq_source') != self._weight_key():
            self.quantize_base_fp8()
        wq = self.base_wq
        key = (wq.data_ptr(), wq._version, wq.device)
        cache = self.__dict__.get('_wq_t_cache')
        if cache is None or cache[0] != key:
            with torch.no_grad():
                cache = (key, wq.t().contiguous())
            self.__dict__['_wq_t_cache'] = cache
        return wq, self.base_wscale, cache[1]

    def forward(self, x: torch.Tensor, routing=None, adapter_ids=None) -> torch.Tensor:
        """x [..., in] -> [..., out]. ``routing``: a SegmentRouting, or the segment offsets
        [S+1] with ``adapter_ids`` [S] given too (sequences or CPU integer tensors; -1 = base
        only). Without either, the active RoleBatch (set by ``roles.roles_active``) routes x's
        sample-major rows."""
        if adapter_ids is not None:
            routing = _routing_from_arrays(routing, adapter_ids)
        elif routing is not None and not isinstance(routing, SegmentRouting):
            raise ValueError('multi-LoRA linear: routing is a SegmentRouting, or seg_offsets with adapter_ids')
        group = self.__dict__.get('shared_input')
        if group is not None:  # stacked with the other linears that read this input
            return group(self, x, routing)
        return self._single(x, routing)

    def role_routing(self, rows: int) -> SegmentRouting:
        """The active RoleBatch's routing of ``rows`` sample-major rows: each role to its
        adapter, roles without one (or whose source wrapper is disabled) to the base alone."""
        if self.active_roles is None:
            raise ValueError('multi-LoRA linear: no routing given and no role batch active')
        role_ids = self.role_ids
        wrappers = self.__dict__.get('_role_wrappers')
        if wrappers is not None:
            role_ids = {n: i for n, i in role_ids.items() if getattr(wrappers[i], 'enabled', True)}
        return self.active_roles.routing(rows, role_ids)

    def _routing(self, x: torch.Tensor, routing: SegmentRouting | None) -> SegmentRouting:
        if routing is None:
            rows = x.numel() // x.shape[-1] if x.dim() and x.shape[-1] else 0
            routing = self.role_routing(rows)
        return routing

    def gated_residual(self, x: torch.Tensor, residual: torch.Tensor, gate: torch.Tensor,
                       routing: SegmentRouting | None = None) -> torch.Tensor:
        """``residual + self(x, routing) * gate`` of a DiT block (model.py:305-313), fused into
        the GEMM epilogue (bf16 or float32 residual stream, output in its dtype; frozen fp32 gate)."""
        if getattr(self, "base_wq", None) is not None:
            raise RuntimeError("gated residual: the e4m3 base is not fused; call the linear and add")
        return multi_lora_linear_gated(x, self.base.weight, self.base.bias, list(self.lora_a), list(self.lora_b),
                                       self.scales, self._routing(x, routing), residual, gate,
                                       weight_t=_base_t(self, x))

    def _single(self, x: torch.Tensor, routing: SegmentRouting | None = None) -> torch.Tensor:
        routing = self._routing(x, routing)
        if getattr(self, "base_wq", None) is not None:
            wq, ws, wq_t = self._fp8_base()
            return multi_lora_linear_fp8(x, wq, ws, self.base.bias, list(self.lora_a), list(self.lora_b),
                                         self.scales, routing, wq_t=wq_t,
                                         dx_bf16=self.__dict__.get('_fp8_dx_bf16', False))
        return multi_lora_linear(x, self.base.weight, self.base.bias, list(self.lora_a), list(self.lora_b),
                                 self.scales, routing, weight_t=_base_t(self, x))
