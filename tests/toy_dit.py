"""A small Wan-style DiT block and the shared-base role construction, for the multi-role tests.

The block has the LoRA target linears of the reference's DiT blocks (self-attention
q, k, v, o; cross-attention over a text context; ffn.0 / ffn.2 around a tanh-GELU,
reference/livewan_wan21/wan/modules/model.py:123-126,271-273), LayerNorms and a
per-role buffer, so that rows per sample differ between linears (video tokens for
self-attention, text tokens for the cross-attention k/v).

``make_roles`` builds teacher / fake / generator the way the shared frozen construction
leaves them (training/construction_sharing.py:58-118): every frozen Parameter one
object across roles, buffers copied per role, adapters per role via ``trainable_scope``.
"""
from __future__ import annotations

import copy

import torch
from torch import nn

TARGETS = ["q", "k", "v", "o", "cross.q", "cross.k", "cross.v", "cross.o", "ffn.0", "ffn.2"]


def _attention(q, k, v, heads):
    """Per-sample multi-head attention in fp32 (q [B, L, h], k/v [B, Lk, h])."""
    B, L, h = q.shape
    d = h // heads
    qh = q.float().reshape(B, L, heads, d).transpose(1, 2).contiguous()
    kh = k.float().reshape(B, k.shape[1], heads, d).transpose(1, 2).contiguous()
    vh = v.float().reshape(B, v.shape[1], heads, d).transpose(1, 2).contiguous()
    s = torch.matmul(qh, kh.transpose(-1, -2).contiguous()) / d ** 0.5
    o = torch.matmul(torch.softmax(s, dim=-1), vh)
    return o.transpose(1, 2).reshape(B, L, h).to(q.dtype)


class CrossAttention(nn.Module):
    def __init__(self, hidden):
        super().__init__()
        self.q, self.k, self.v, self.o = (nn.Linear(hidden, hidden) for _ in range(4))


class ToyDiTBlock(nn.Module):
    def __init__(self, hidden: int, ffn: int, heads: int):
        super().__init__()
        self.heads = heads
        self.norm1 = nn.LayerNorm(hidden)
        self.q, self.k, self.v, self.o = (nn.Linear(hidden, hidden) for _ in range(4))
        self.norm2 = nn.LayerNorm(hidden)
        self.cross = CrossAttention(hidden)
        self.norm3 = nn.LayerNorm(hidden)
        self.ffn = nn.Sequential(nn.Linear(hidden, ffn), nn.GELU(approximate="tanh"), nn.Linear(ffn, hidden))
        self.register_buffer("shift", torch.linspace(-0.1, 0.1, hidden))

    def forward(self, x, context):
        y = self.norm1(x) + self.shift.to(x.dtype)
        x = x + self.o(_attention(self.q(y), self.k(y), self.v(y), self.heads))
        y = self.norm2(x)
        x = x + self.cross.o(_attention(self.cross.q(y), self.cross.k(context), self.cross.v(context), self.heads))
        return x + self.ffn(self.norm3(x))


def make_roles(pkg, hidden=256, ffn=512, heads=4, rank=16, device="cpu", dtype=torch.float32, seed=0,
               fake_targets=None, gen_targets=None):
    """(teacher, fake, generator): one frozen base by alias, per-role buffers and adapters.

    lora_b is drawn N(0, 0.02) instead of the reference's zeros so the adapters act."""
    g = torch.Generator().manual_seed(seed)
    teacher = ToyDiTBlock(hidden, ffn, heads)
    with torch.no_grad():
        for p in teacher.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * (0.02 if p.dim() == 1 else p.shape[-1] ** -0.5))
    teacher = teacher.to(device=device, dtype=dtype).requires_grad_(False)

    def aliased(model):
        return copy.deepcopy(model, {id(p): p for p in model.parameters()})

    fake, gen = aliased(teacher), aliased(teacher)
    torch.manual_seed(seed + 1)
    for role, targets in ((fake, fake_targets or TARGETS), (gen, gen_targets or TARGETS)):
        pkg.trainable_scope(role, {"mode": "lora", "rank": rank, "alpha": rank, "targets": list(targets)})
        with torch.no_grad():
            for m in role.modules():
                if isinstance(m, pkg.TrainableLowRankLinear):
                    m.lora_b.copy_(torch.randn(m.lora_b.shape, generator=g) * 0.02)
    return teacher, fake, gen


def inputs(batch: int, tokens: int, ctx_tokens: int, hidden: int, device, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, tokens, hidden, generator=g).to(device=device, dtype=dtype)
    c = torch.randn(batch, ctx_tokens, hidden, generator=g).to(device=device, dtype=dtype)
    return x, c


def rel_l2(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


__all__ = ["TARGETS", "ToyDiTBlock", "make_roles", "inputs", "rel_l2"]
