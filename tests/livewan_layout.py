"""A module with the attribute layout of LiveWan's critic LoRA (reference/livewan_wan21/wanstreamer/
lora.py:8-27) and its eager forward in the reference's operator order, plus a small Wan-style
model whose ``blocks`` carry the reference's LoRA targets (``self_attn.q/k/v/o``, ``ffn.0``,
``ffn.2``; reference/livewan_wan21/wan/modules/model.py:123-126,271-273). The reference module
is not imported; this stands in for it in tests.

    y = base(x); disabled: y;  else y + linear(linear(x.to(a.dtype), a), b).to(y.dtype) * scale
"""
import torch
import torch.nn.functional as F
from torch import nn


class RefLayoutLoRA(nn.Module):
    def __init__(self, base: nn.Linear, rank: int = 32, alpha=None):
        super().__init__()
        self.base = base
        base.weight.requires_grad_(False)
        if base.bias is not None:
            base.bias.requires_grad_(False)
        self.rank = rank
        self.scale = (alpha or rank) / rank
        self.a = nn.Parameter(torch.zeros(rank, base.in_features, device=base.weight.device))
        self.b = nn.Parameter(torch.zeros(base.out_features, rank, device=base.weight.device))
        nn.init.normal_(self.a, std=1.0 / rank)
        self.enabled = True

    def forward(self, x):
        y = self.base(x)
        if not self.enabled:
            return y
        update = F.linear(F.linear(x.to(self.a.dtype), self.a), self.b)
        return y + update.to(y.dtype) * self.scale


class SelfAttention(nn.Module):
    def __init__(self, hidden):
        super().__init__()
        self.q, self.k, self.v, self.o = (nn.Linear(hidden, hidden) for _ in range(4))


class WanLikeBlock(nn.Module):
    def __init__(self, hidden: int, ffn: int, heads: int):
        super().__init__()
        self.heads = heads
        self.norm1 = nn.LayerNorm(hidden, elementwise_affine=False)
        self.self_attn = SelfAttention(hidden)
        self.norm2 = nn.LayerNorm(hidden, elementwise_affine=False)
        self.ffn = nn.Sequential(nn.Linear(hidden, ffn), nn.GELU(approximate="tanh"), nn.Linear(ffn, hidden))

    def forward(self, x):
        B, L, h = x.shape
        d = h // self.heads
        y = self.norm1(x.float()).to(x.dtype)
        a = self.self_attn

        def heads(t):
            return t.float().reshape(B, L, self.heads, d).transpose(1, 2).contiguous()

        q, k, v = heads(a.q(y)), heads(a.k(y)), heads(a.v(y))
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / d ** 0.5
        o = torch.matmul(torch.softmax(s, dim=-1), v).transpose(1, 2).reshape(B, L, h).to(x.dtype)
        x = x + a.o(o)
        return x + self.ffn(self.norm2(x.float()).to(x.dtype))


class WanLike(nn.Module):
    def __init__(self, hidden=256, ffn=512, heads=4, layers=2, seed=0):
        super().__init__()
        self.blocks = nn.ModuleList([WanLikeBlock(hidden, ffn, heads) for _ in range(layers)])
        g = torch.Generator().manual_seed(seed)
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=g) * (0.02 if p.dim() == 1 else p.shape[-1] ** -0.5))

    def forward(self, x):
        for blk in self.blocks:
            x = blk(x)
        return x


TARGETS = ('self_attn.q', 'self_attn.k', 'self_attn.v', 'self_attn.o', 'ffn.0', 'ffn.2')


def wrap_reference_layout(model: nn.Module, rank: int = 32, alpha=None, seed: int = 1, b_std: float = 0.02):
    """Freeze ``model`` and wrap every block's targets with RefLayoutLoRA (fp32 a / b); b drawn
    N(0, b_std) instead of zeros so the adapters act."""
    model.requires_grad_(False)
    g = torch.Generator().manual_seed(seed)
    for blk in model.blocks:
        for name in TARGETS:
            parent, _, leaf = name.rpartition('.')
            mod = blk.get_submodule(parent)
            lin = mod[int(leaf)] if leaf.isdigit() else getattr(mod, leaf)
            w = RefLayoutLoRA(lin, rank, alpha)
            with torch.no_grad():
                w.b.copy_(torch.randn(w.b.shape, generator=g) * b_std)
            if leaf.isdigit():
                mod[int(leaf)] = w
            else:
                setattr(mod, leaf, w)
    return model
