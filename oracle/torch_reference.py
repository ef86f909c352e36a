"""The reference's per-adapter LoRA linear as plain torch CPU ops — TEST INFRASTRUCTURE ONLY.

Used as the timed CPU baseline of bench.py (kind "port") and as a second,
independent evaluation in tests (torch.autograd supplies the backward, so it
pins the numpy oracle's hand-written gradients).

Restates training/low_rank.py:26-28 — ``base(value) + scale * F.linear(F.linear(value, lora_a), lora_b)`` —
once per segment, i.e. once per role module call (training/dmd.py:301-353);
base-only segments (adapter id -1) are the teacher / ``lora_enabled(model, False)``
path (reference/livewan_wan21/wanstreamer/lora.py:65-74).
"""
from __future__ import annotations

from typing import Sequence

import torch
import torch.nn.functional as F


def per_adapter_forward(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, As: Sequence[torch.Tensor],
                        Bs: Sequence[torch.Tensor], scales: Sequence[float], seg_offsets: Sequence[int],
                        adapter_ids: Sequence[int]) -> torch.Tensor:
    outs = []
    for s, a in enumerate(adapter_ids):
        lo, hi = int(seg_offsets[s]), int(seg_offsets[s + 1])
        xs = x[lo:hi]
        base = F.linear(xs, w, b)
        if a < 0:
            outs.append(base)
        else:
            outs.append(base + scales[a] * F.linear(F.linear(xs, As[a]), Bs[a]))
    return torch.cat(outs, 0)


def per_adapter_step(x, w, b, As, Bs, scales, seg_offsets, adapter_ids, dy):
    """One fwd+bwd of the per-adapter path; returns (y, dx, dAs, dBs)."""
    x = x.detach().requires_grad_(True)
    As = [a.detach().requires_grad_(True) for a in As]
    Bs = [bb.detach().requires_grad_(True) for bb in Bs]
    y = per_adapter_forward(x, w, b, As, Bs, scales, seg_offsets, adapter_ids)
    y.backward(dy)
    return y.detach(), x.grad, [a.grad for a in As], [bb.grad for bb in Bs]
