"""The benchmark/parity configurations of the multi-LoRA linear, with seeded inputs.

Shapes follow the DiT blocks that run the LoRA linear in the reference:
every block applies q, k, v, o (hidden -> hidden) and ffn.0 / ffn.2
(hidden -> ffn -> hidden) (reference/livewan_wan21/wan/modules/model.py:123-126,271-273;
wanstreamer/lora.py:30-31). Tokens of the roles that share the frozen base
are concatenated into segments, one adapter per role.

Input distributions: X ~ N(0,1), W ~ N(0, 1/in), bias ~ N(0, 1/in),
lora_a ~ U(±1/sqrt(in)) (Kaiming-uniform with a=sqrt(5), low_rank.py:23),
lora_b ~ N(0, 0.02) (nonzero so the adapter term is exercised), dY ~ N(0,1).
"""
from __future__ import annotations

import math
import random
from dataclasses import dataclass, field

import torch

from .routing import SegmentRouting

BLOCK_LINEARS = ("q", "k", "v", "o", "ffn.0", "ffn.2")


@dataclass(frozen=True)
class LoraConfig:
    name: str
    tokens: int
    hidden: int
    ffn: int
    ranks: tuple[int, ...]          # per adapter
    seg_lengths: tuple[int, ...]    # per segment
    seg_adapters: tuple[int, ...]   # adapter id per segment
    scale: float
    dtype: str = "bf16"
    seed: int = 0
    notes: str = ""
    base_fp8: bool = False
    extra: dict = field(default_factory=dict)

    @property
    def routing(self) -> SegmentRouting:
        return SegmentRouting.from_lengths(self.seg_lengths, self.seg_adapters)

    def linears(self) -> list[tuple[str, int, int]]:
        """(name, in_features, out_features) of the six block linears."""
        h, f = self.hidden, self.ffn
        return [("q", h, h), ("k", h, h), ("v", h, h), ("o", h, h), ("ffn.0", h, f), ("ffn.2", f, h)]

    def flops_fwd_bwd(self, K: int, N: int) -> int:
        """4·M·K·N + Σ_seg 6·M_s·r_s·(K+N): base fwd + dX, and the LoRA shrink/expand/grads."""
        lora = sum(6 * m * self.ranks[a] * (K + N) for m, a in zip(self.seg_lengths, self.seg_adapters) if a >= 0)
        return 4 * self.tokens * K * N + lora

    def flops_fwd(self, K: int, N: int) -> int:
        lora = sum(2 * m * self.ranks[a] * (K + N) for m, a in zip(self.seg_lengths, self.seg_adapters) if a >= 0)
        return 2 * self.tokens * K * N + lora


def _partition(total: int, parts: int, seed: int, minimum: int = 256) -> tuple[int, ...]:
    """Seeded random positive partition of `total` into `parts` lengths (each >= minimum)."""
    rng = random.Random(seed)
    cuts = sorted(rng.sample(range(1, (total - parts * minimum) + 1), parts - 1)) if parts > 1 else []
    edges = [0, *cuts, total - parts * minimum]
    return tuple(b - a + minimum for a, b in zip(edges, edges[1:]))


def _cfg4_ranks(seed: int) -> tuple[int, ...]:
    rng = random.Random(seed)
    return tuple(rng.choice((16, 32, 64, 128)) for _ in range(16))


CONFIGS: dict[str, LoraConfig] = {
    "tiny": LoraConfig(
        name="tiny", tokens=512, hidden=256, ffn=256, ranks=(8, 8), seg_lengths=(256, 256), seg_adapters=(0, 1),
        scale=1.0, dtype="fp32", seed=1,
        notes="reference CPU-runnable case: X [2x256 tokens, 256], W [256,256], 2 adapters rank 8, 2 equal segments"),
    "wan13b": LoraConfig(
        name="wan13b", tokens=65520, hidden=1536, ffn=8960, ranks=(64, 64), seg_lengths=(32760, 32760),
        seg_adapters=(0, 1), scale=1.0, seed=2,
        notes="Wan-1.3B DiT linears, 32760 tokens (21x30x52) per role, generator + fake critic rank 64"),
    "wan22_5b": LoraConfig(
        name="wan22_5b", tokens=27280, hidden=3072, ffn=14336, ranks=(128, 128, 128),
        seg_lengths=_partition(27280, 3, 3), seg_adapters=(0, 1, 2), scale=2.0, seed=3,
        notes="Wan2.2-TI2V-5B, 27280 tokens (31x22x40), 3 adapters rank 128, seeded random segment lengths"),
    "flux": LoraConfig(
        name="flux", tokens=16 * 4608, hidden=3072, ffn=12288, ranks=_cfg4_ranks(4),
        seg_lengths=(4608,) * 16, seg_adapters=tuple(range(16)), scale=1.0, seed=4,
        notes="FLUX-style MMDiT: 16 samples x (4096 image + 512 text) tokens, one adapter per sample, "
              "ranks drawn from {16,32,64,128}"),
    "wan13b_fp8": LoraConfig(
        name="wan13b_fp8", tokens=65520, hidden=1536, ffn=8960, ranks=(64, 64, 64, 64),
        seg_lengths=_partition(65520, 4, 5), seg_adapters=(0, 1, 2, 3), scale=1.0, seed=5, base_fp8=True,
        notes="config wan13b with the frozen base stored fp8 e4m3 + per-output-channel scale, 4 adapters"),
    "wan13b_roles": LoraConfig(
        name="wan13b_roles", tokens=98280, hidden=1536, ffn=8960, ranks=(64,), seg_lengths=(65520, 32760),
        seg_adapters=(-1, 0), scale=1.0, seed=6,
        notes="multi-role call site at the Wan-1.3B shape: teacher conditional + unconditional passes "
              "(base only, 2 x 32760 tokens) and the fake critic (rank 64, 32760 tokens) in one call"),
}


def make_linear(cfg: LoraConfig, K: int, N: int, device, seed: int, dtype=torch.bfloat16, bias: bool = True):
    """Seeded (x, w, b, As, Bs, dy) for one linear of `cfg` on `device`."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    M = cfg.tokens

    def randn(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    def uniform(*shape, bound):
        return ((torch.rand(*shape, generator=gen, device=device, dtype=torch.float32) * 2 - 1) * bound).to(dtype)

    x = randn(M, K)
    w = randn(N, K, std=1 / math.sqrt(K))
    b = randn(N, std=1 / math.sqrt(K)) if bias else None
    As = [uniform(r, K, bound=1 / math.sqrt(K)) for r in cfg.ranks]
    Bs = [randn(N, r, std=0.02) for r in cfg.ranks]
    dy = randn(M, N)
    return x, w, b, As, Bs, dy
