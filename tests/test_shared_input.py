"""Host-side logic of shared-input stacking on CPU: which linears can be grouped, the
fail-closed checks, and that grouping leaves parameters and state-dict keys alone.
No kernel runs."""
import pytest
import torch
from torch import nn

from toy_dit import make_roles

GROUPS = [["q", "k", "v"], ["cross.k", "cross.v"]]


def _fused(pkg, **kw):
    teacher, fake, gen = make_roles(pkg, hidden=256, ffn=512, heads=4, rank=16, **kw)
    return teacher, fake, gen, pkg.fuse_roles({"teacher": teacher, "fake": fake, "gen": gen})


def test_groups_link_members_and_keep_state_dict(pkg):
    _, fake, _, fused = _fused(pkg)
    keys = list(fused.state_dict())
    groups = pkg.fuse_shared_inputs(fused, GROUPS)
    assert [g.names for g in groups] == [("q", "k", "v"), ("cross.k", "cross.v")]
    assert all(fused.get_submodule(n).shared_input is groups[0] for n in GROUPS[0])
    assert fused.cross.v.shared_input is groups[1] and fused.o.__dict__.get("shared_input") is None
    assert (groups[0].K, groups[0].n, groups[0].rank) == (256, 2, 16)
    assert list(fused.state_dict()) == keys
    assert groups[0].members[1].lora_a[0] is fake.k.lora_a
    pkg.release_shared_inputs(fused)
    assert all(fused.get_submodule(n).shared_input is None for g in GROUPS for n in g)
    # a single role's own modules group the same way
    g = pkg.fuse_shared_inputs(fake, [["q", "k", "v"]])[0]
    assert g.n == 1 and isinstance(g.members[0], pkg.TrainableLowRankLinear)


def test_groups_fail_closed(pkg):
    teacher, fake, gen, fused = _fused(pkg)
    with pytest.raises(ValueError, match="shared input: missing linear nope"):
        pkg.fuse_shared_inputs(fused, [["q", "nope"]])
    with pytest.raises(ValueError, match="'norm1' is not a LoRA linear"):
        pkg.fuse_shared_inputs(fused, [["q", "norm1"]])
    with pytest.raises(ValueError, match="'k' is in two groups"):
        pkg.fuse_shared_inputs(fused, [["q", "k"], ["k", "v"]])
    pkg.release_shared_inputs(fused)
    with pytest.raises(ValueError, match="one in_features"):
        pkg.fuse_shared_inputs(fused, [["q", "ffn.2"]])
    with pytest.raises(ValueError, match="at least two"):
        pkg.fuse_shared_inputs(fused, [["q"]])
    pkg.fuse_shared_inputs(fused, [["q", "k"]])
    with pytest.raises(ValueError, match="already in a shared-input group"):
        pkg.fuse_shared_inputs(fused, [["k", "v"]])
    # rank 8 is not a whole 16-rank fragment tile
    _, f8, _ = make_roles(pkg, hidden=256, ffn=512, heads=4, rank=8)
    with pytest.raises(ValueError, match="multiple of 16"):
        pkg.fuse_shared_inputs(f8, [["q", "k"]])
    # linears of different out_features that read one input stack too (q with ffn.0)
    _, small, _ = make_roles(pkg, hidden=32, ffn=64, heads=2, rank=16)
    assert pkg.fuse_shared_inputs(small, [["q", "ffn.0"]])[0].K == 32
    # members that route different roles cannot share one routing
    _, _, _, partial = _fused(pkg, fake_targets=["q", "k", "v"], gen_targets=["q", "k"])
    with pytest.raises(ValueError, match="members must have the same number of adapters|route different roles"):
        pkg.fuse_shared_inputs(partial, [["q", "v"]])


def test_scales_must_agree(pkg):
    base = nn.Linear(256, 256)
    a = pkg.MultiLoRALinear(base, ranks=[16], alphas=[16])
    b = pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[16], alphas=[32])
    holder = nn.Module()
    holder.a, holder.b = a, b
    with pytest.raises(ValueError, match="different scales"):
        pkg.fuse_shared_inputs(holder, [["a", "b"]])
    # biases may differ: one member with, one without
    holder.b = pkg.MultiLoRALinear(nn.Linear(256, 512, bias=False), ranks=[16], alphas=[16])
    assert len(pkg.fuse_shared_inputs(holder, [["a", "b"]])) == 1


def test_wan_ranks_stack(pkg):
    """G members of rank r share h of G·r columns: the shrinks and reductions take 256 of them
    per call, the GEMMs all of them, so q/k/v at the reference's ranks 128 and 256 stack."""
    for rank in (128, 256):
        holder = nn.Module()
        for name in ("q", "k", "v"):
            setattr(holder, name, pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[rank], alphas=[rank]))
        assert pkg.fuse_shared_inputs(holder, [["q", "k", "v"]])[0].rank == rank
    from dmd_system_amd.function import _stack_slices
    assert _stack_slices(3, 128) == [(0, 2), (2, 3)]
    assert _stack_slices(3, 256) == [(0, 1), (1, 2), (2, 3)]
    assert _stack_slices(3, 64) == [(0, 3)]
    assert _stack_slices(8, 32) == [(0, 8)]


def test_every_call_site_layout_groups(pkg):
    """PEFT layers (after install_peft_multi_lora), the native LoRALinear and LiveWan's layout
    group; an uninstalled PEFT layer or reference-layout module, or a mixture of families, fails
    closed with the reason."""
    from types import SimpleNamespace

    from livewan_layout import RefLayoutLoRA
    from peft_layout import PeftLoraLinear
    holder = nn.Module()
    for name in ("q", "k", "v"):
        setattr(holder, name, PeftLoraLinear(nn.Linear(256, 256), {"default": (128, 128)}))
    with pytest.raises(ValueError, match="install_peft_multi_lora first"):
        pkg.fuse_shared_inputs(holder, [["q", "k", "v"]])
    pkg.install_peft_multi_lora(holder)
    g = pkg.fuse_shared_inputs(holder, [["q", "k", "v"]])[0]
    assert g.family == "peft" and g.rank == 128 and g.n == 1
    pkg.release_shared_inputs(holder)
    # PEFT layers whose adapters differ by name or scaling do not stack
    holder.v = PeftLoraLinear(nn.Linear(256, 256), {"other": (128, 128)})
    pkg.install_peft_multi_lora(holder)
    with pytest.raises(ValueError, match="same adapters"):
        pkg.fuse_shared_inputs(holder, [["q", "v"]])
    holder.v = PeftLoraLinear(nn.Linear(256, 256), {"default": (128, 64)})
    pkg.install_peft_multi_lora(holder)
    with pytest.raises(ValueError, match="different scales"):
        pkg.fuse_shared_inputs(holder, [["q", "v"]])

    task = SimpleNamespace(lora_rank=256, lora_alpha=256)
    native = nn.Module()
    for name in ("q", "k", "v"):
        setattr(native, name, pkg.LoRALinear(nn.Linear(256, 256), task))
    assert pkg.fuse_shared_inputs(native, [["q", "k", "v"]])[0].family == "pair"

    lw = nn.Module()
    for name in ("q", "k"):
        setattr(lw, name, RefLayoutLoRA(nn.Linear(256, 256), rank=32))
    with pytest.raises(ValueError, match="install_livewan_multi_lora first"):
        pkg.fuse_shared_inputs(lw, [["q", "k"]])
    pkg.install_livewan_multi_lora(lw)
    assert pkg.fuse_shared_inputs(lw, [["q", "k"]])[0].family == "pair"

    mixed = nn.Module()
    mixed.q = pkg.LoRALinear(nn.Linear(256, 256), task)
    mixed.k = pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[256], alphas=[256])
    with pytest.raises(ValueError, match="all MultiLoRALinear"):
        pkg.fuse_shared_inputs(mixed, [["q", "k"]])


def test_stacked_bases_follow_replaced_biases_and_free_with_any_member(pkg):
    """The stacked-base cache compares member weights AND biases by identity: a bias replaced by
    a new Parameter (which may reuse the freed one's id and storage, at in-place version 0) is
    stacked again; freeing any member drops the entry."""
    import gc
    from dmd_system_amd import low_rank as L
    ws = [torch.nn.Parameter(torch.randn(16, 8), requires_grad=False) for _ in range(3)]
    bs = [torch.nn.Parameter(torch.randn(16), requires_grad=False) for _ in range(3)]
    _, b_cat, _ = L.stacked_bases(ws, bs, want_t=False)
    assert torch.equal(b_cat, torch.cat([b.float() for b in bs]))
    bs[1] = torch.nn.Parameter(torch.full((16,), 5.0), requires_grad=False)
    _, b_cat2, _ = L.stacked_bases(ws, bs, want_t=False)
    assert torch.equal(b_cat2[16:32], torch.full((16,), 5.0))
    keys_before = set(L._STACKED)
    del bs[2]
    gc.collect()
    assert not (set(L._STACKED) & keys_before), "freeing one member bias must drop the cached stack"


def test_more_fuse_time_refusals(pkg):
    """An e4m3 base, a PEFT adapter above the kernels' rank limit, and ranks that are not one
    multiple of 16 are refused when the group is made."""
    from peft_layout import PeftLoraLinear
    holder = nn.Module()
    holder.q = pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[16], alphas=[16])
    holder.k = pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[16], alphas=[16])
    holder.k.base_wq = torch.zeros(1)  # stands in for a quantised base
    with pytest.raises(ValueError, match="e4m3 bases are not stacked"):
        pkg.fuse_shared_inputs(holder, [["q", "k"]])
    peft = nn.Module()
    for name in ("q", "k"):
        setattr(peft, name, PeftLoraLinear(nn.Linear(512, 512), {"default": (320, 320)}))
    pkg.install_peft_multi_lora(peft)
    with pytest.raises(ValueError, match="above the kernels' 256"):
        pkg.fuse_shared_inputs(peft, [["q", "k"]])
    mixed = nn.Module()
    mixed.q = pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[16], alphas=[16])
    mixed.k = pkg.MultiLoRALinear(nn.Linear(256, 256), ranks=[32], alphas=[32])
    with pytest.raises(ValueError, match="one LoRA rank"):
        pkg.fuse_shared_inputs(mixed, [["q", "k"]])


def test_call_time_plans_that_do_not_stack(pkg):
    """At call time the members stack only with one routing, adapter count, scales and rank (a
    multiple of 16); otherwise each runs its own call. Checked on the plans alone (no kernel)."""
    from dmd_system_amd.shared_input import SharedInputGroup
    R = pkg.SegmentRouting
    a16, b16 = torch.zeros(16, 8), torch.zeros(8, 16)
    a32 = torch.zeros(32, 8)
    one = R.single(10, 0)
    ok = [([a16], [b16], [1.0], one), ([a16], [b16], [1.0], R.single(10, 0))]
    assert SharedInputGroup._plans_stack(ok)
    assert not SharedInputGroup._plans_stack([ok[0], ([a16], [b16], [2.0], one)])           # scales
    assert not SharedInputGroup._plans_stack([ok[0], ([a16], [b16], [1.0], R.single(10, -1))])  # routing
    assert not SharedInputGroup._plans_stack([ok[0], ([a32], [b16], [1.0], one)])           # rank
    assert not SharedInputGroup._plans_stack([ok[0], ([], [], [], one)])                    # a disabled member
    assert not SharedInputGroup._plans_stack([([], [], [], one), ([], [], [], one)])        # no adapter at all
    a8 = torch.zeros(8, 8)
    assert not SharedInputGroup._plans_stack([([a8], [b16], [1.0], one), ([a8], [b16], [1.0], one)])  # rank 8
