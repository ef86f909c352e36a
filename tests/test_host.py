"""Host-side logic of the package on CPU: routing, the drop-in trainable scope,
parameter naming, workload definitions, and the no-CPU-path contract."""
import pytest
import torch
from torch import nn


# ---------------------------------------------------------------- routing

def test_routing_from_lengths_and_rows(pkg):
    r = pkg.SegmentRouting.from_lengths([3, 0, 2], [1, 0, -1])
    assert r.seg_offsets == (0, 3, 3, 5)
    assert r.num_rows == 5 and r.num_segments == 3
    assert r.row_adapter() == [1, 1, 1, -1, -1]
    r.validate_for(5, 2)
    with pytest.raises(ValueError):
        r.validate_for(6, 2)
    with pytest.raises(ValueError):
        r.validate_for(5, 1)


@pytest.mark.parametrize("off,ids", [((1, 3), (0,)), ((0, 3, 2), (0, 0)), ((0, 3), (0, 1)), ((0, 3), (-2,))])
def test_routing_rejects_malformed(pkg, off, ids):
    with pytest.raises(ValueError):
        pkg.SegmentRouting(off, ids)


def test_routing_groups_cover_rows_exactly(pkg):
    lengths = [(i * 7) % 5 for i in range(300)]
    ids = [(i % 3) - 1 for i in range(300)]
    r = pkg.SegmentRouting.from_lengths(lengths, ids)
    rows = []
    nseg = 0
    for r0, r1, off, gids in r.groups(128):
        assert len(gids) <= 128 and off[0] == 0 and off[-1] == r1 - r0
        sub = pkg.SegmentRouting(off, gids)
        rows.extend(sub.row_adapter())
        nseg += len(gids)
    assert nseg == 300 and rows == r.row_adapter()


from hypothesis import given, settings, strategies as st  # noqa: E402


@settings(max_examples=300, deadline=None)
@given(segs=st.lists(st.tuples(st.integers(0, 20), st.integers(-1, 5)), min_size=1, max_size=700),
       per_call=st.integers(1, 200))
def test_routing_groups_property(pkg, segs, per_call):
    """Any routing split into calls of at most `per_call` segments: the calls tile the rows in order,
    each with local offsets from 0, and give every row its adapter."""
    r = pkg.SegmentRouting.from_lengths([n for n, _ in segs], [a for _, a in segs])
    rows, nseg, end = [], 0, 0
    for r0, r1, off, gids in r.groups(per_call):
        assert r0 == end and 1 <= len(gids) <= per_call and off[0] == 0 and off[-1] == r1 - r0
        rows.extend(pkg.SegmentRouting(off, gids).row_adapter())
        nseg, end = nseg + len(gids), r1
    assert nseg == len(segs) and end == r.num_rows and rows == r.row_adapter()


# ---------------------------------------------------------------- drop-in trainable scope

class Native(nn.Module):
    """The reference's construction fixture (tests/test_training_construction.py:24-36)."""

    def __init__(self):
        super().__init__()
        self.hidden = nn.Linear(4, 4)
        self.proj_out = nn.Linear(4, 4)
        with torch.no_grad():
            for p in self.parameters():
                p.fill_(0.25)


def test_trainable_scope_installs_same_parameter_names(pkg):
    native = Native()
    pkg.trainable_scope(native, {'mode': 'lora', 'rank': 2, 'alpha': 2., 'targets': ['proj_out']})
    mod = native.proj_out
    assert isinstance(mod, pkg.TrainableLowRankLinear)
    names = dict(native.named_parameters())
    assert set(names) == {'hidden.weight', 'hidden.bias', 'proj_out.base.weight', 'proj_out.base.bias',
                          'proj_out.lora_a', 'proj_out.lora_b'}
    trainable = {n for n, p in names.items() if p.requires_grad}
    assert trainable == {'proj_out.lora_a', 'proj_out.lora_b'}
    assert mod.scale == 1.0
    assert mod.lora_a.shape == (2, 4) and mod.lora_b.shape == (4, 2)
    assert not mod.lora_b.any()
    assert mod.lora_a.abs().max() <= 1 / 4 ** .5 + 1e-7  # kaiming_uniform(a=sqrt 5) bound 1/sqrt(in)


@pytest.mark.parametrize("config,msg", [
    ({'mode': 'lora'}, 'exact nonempty native Linear LoRA targets required'),
    ({'mode': 'full', 'rank': 2}, 'full mode accepts no ignored LoRA settings'),
    ({'mode': 'lora', 'rank': 2, 'alpha': 2., 'targets': ['nope']}, 'missing actual native LoRA target: nope'),
    ({'mode': 'lora', 'rank': 2, 'alpha': 2., 'targets': ['proj_out', 'proj_out']},
     'exact nonempty native Linear LoRA targets required'),
    ({'mode': 'lora', 'rank': 0, 'alpha': 2., 'targets': ['proj_out']}, 'invalid native Linear LoRA scope/rank/alpha'),
    ({'mode': 'lora', 'rank': 2, 'alpha': -1., 'targets': ['proj_out']}, 'invalid native Linear LoRA scope/rank/alpha'),
    ({'mode': 'other'}, 'explicit full or lora trainable scope required'),
])
def test_trainable_scope_fails_closed_like_the_reference(pkg, config, msg):
    with pytest.raises(ValueError, match='native trainable scope: ' + msg if 'missing' not in msg else msg):
        pkg.trainable_scope(Native(), config)


def test_full_mode_makes_everything_trainable(pkg):
    native = Native()
    pkg.trainable_scope(native, {'mode': 'full'})
    assert all(p.requires_grad for p in native.parameters())


def test_multi_lora_parameter_names_and_from_roles(pkg):
    base = nn.Linear(16, 8)
    m = pkg.MultiLoRALinear(base, ranks=[8, 4], alphas=[8, 8])
    assert set(dict(m.named_parameters())) == {'base.weight', 'base.bias', 'lora_a.0', 'lora_a.1',
                                               'lora_b.0', 'lora_b.1'}
    assert m.scales == [1.0, 2.0]
    roles = [pkg.TrainableLowRankLinear(base, rank=4, alpha=4) for _ in range(2)]
    mm = pkg.MultiLoRALinear.from_roles(roles)
    assert mm.lora_a[0] is roles[0].lora_a and mm.lora_b[1] is roles[1].lora_b
    other = pkg.TrainableLowRankLinear(nn.Linear(16, 8), rank=4, alpha=4)
    with pytest.raises(ValueError):
        pkg.MultiLoRALinear.from_roles([roles[0], other])


def test_no_cpu_path(pkg):
    base = nn.Linear(16, 8).to(torch.bfloat16)
    m = pkg.MultiLoRALinear(base, ranks=[8], alphas=[8])
    x = torch.randn(4, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm device only"):
        m(x, pkg.SegmentRouting.single(4))
    with pytest.raises(RuntimeError, match="ROCm device only"):
        m.float()(x.float(), pkg.SegmentRouting.single(4))  # the float32 path is a device path too
    with pytest.raises(RuntimeError, match="bfloat16 or float32"):
        m(x.half(), pkg.SegmentRouting.single(4))
    mixed = pkg.MultiLoRALinear(nn.Linear(16, 8), ranks=[8], alphas=[8], dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="adapters must be float32"):
        mixed(x.float(), pkg.SegmentRouting.single(4))


def test_forward_takes_segment_arrays(pkg):
    """forward(x, seg_offsets, adapter_ids): the routing as plain arrays (sequences or 1-D
    integer CPU tensors) is the same SegmentRouting; malformed arrays fail closed before any
    device work."""
    from dmd_system_amd.low_rank import _routing_from_arrays
    want = pkg.SegmentRouting.from_lengths((3, 1), (0, -1))
    assert _routing_from_arrays([0, 3, 4], [0, -1]) == want
    assert _routing_from_arrays(torch.tensor([0, 3, 4]), torch.tensor([0, -1], dtype=torch.int32)) == want
    m = pkg.MultiLoRALinear(nn.Linear(16, 8).to(torch.bfloat16), ranks=[8], alphas=[8])
    x = torch.randn(4, 16, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="1-D integer CPU tensor"):
        m(x, torch.tensor([0.0, 4.0]), [0])
    with pytest.raises(ValueError, match="seg_offsets is required"):
        m(x, None, [0])
    with pytest.raises(ValueError, match="SegmentRouting, or seg_offsets with adapter_ids"):
        m(x, [0, 4])
    with pytest.raises(RuntimeError, match="ROCm device only"):  # well-formed: reaches the device check
        m(x, [0, 4], [0])


def test_native_lora_install_contract(pkg):
    """install_lora / LoRALinear keep native/models.py:33-64: fp32 masters `a` (Kaiming-uniform) and
    `b` (zeros) over a frozen base, scale alpha / rank, suffix matching, fail-closed messages."""
    from types import SimpleNamespace
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(8, 16), nn.GELU(), nn.Sequential(nn.Linear(16, 8)))
    model.to(torch.bfloat16)
    task = SimpleNamespace(lora_rank=4, lora_alpha=8.0, target_modules=["0", "2.0"])
    names = pkg.install_lora(model, task)
    assert names == ["0", "2.0"]
    for m in (model[0], model[2][0]):
        assert isinstance(m, pkg.LoRALinear) and m.scale == 2.0
        assert m.a.dtype == torch.float32 and m.b.dtype == torch.float32 and not m.b.any()
        assert m.a.shape == (4, m.base.in_features) and m.b.shape == (m.base.out_features, 4)
        assert m.a.abs().max() <= 1 / m.base.in_features ** 0.5 + 1e-6
        assert not m.base.weight.requires_grad and m.base.weight.dtype == torch.bfloat16
    assert {n for n, p in model.named_parameters() if p.requires_grad} == {"0.a", "0.b", "2.0.a", "2.0.b"}
    with pytest.raises(ValueError, match="no matching LoRA targets"):
        pkg.install_lora(nn.Sequential(nn.Linear(2, 2)), SimpleNamespace(lora_rank=1, lora_alpha=1., target_modules=["q"]))
    with pytest.raises(ValueError, match="unmatched LoRA target: q"):
        pkg.install_lora(nn.Sequential(nn.Linear(2, 2)), SimpleNamespace(lora_rank=1, lora_alpha=1.,
                                                                         target_modules=["0", "q"]))


# ---------------------------------------------------------------- workloads

def test_workload_flops_match_baseline_table(pkg):
    from dmd_system_amd import workloads as W
    cfg = W.CONFIGS["wan13b"]
    total = sum(cfg.flops_fwd_bwd(K, N) for _, K, N in cfg.linears())
    assert abs(total / 1e12 - 10.524) < 0.001  # 10.524 TFLOP per 6-linear block (the headline metric's figure)
    lora = total - sum(4 * cfg.tokens * K * N for _, K, N in cfg.linears())
    assert abs(lora / 1e12 - 0.837) < 0.001
    for c in W.CONFIGS.values():
        assert sum(c.seg_lengths) == c.tokens and len(c.seg_lengths) == len(c.seg_adapters)
        assert all(-1 <= a < len(c.ranks) for a in c.seg_adapters)
    assert sorted(set(W.CONFIGS["flux"].ranks)) <= [16, 32, 64, 128]
    assert min(W.CONFIGS["wan22_5b"].seg_lengths) >= 256


def test_make_linear_is_seeded(pkg):
    from dmd_system_amd import workloads as W
    cfg = W.CONFIGS["tiny"]
    a = W.make_linear(cfg, 256, 256, torch.device("cpu"), seed=3)
    b = W.make_linear(cfg, 256, 256, torch.device("cpu"), seed=3)
    for u, v in zip(a, b):
        if isinstance(u, list):
            assert all(torch.equal(p, q) for p, q in zip(u, v))
        else:
            assert torch.equal(u, v)
