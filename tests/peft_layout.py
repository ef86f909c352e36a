"""A module with the attribute layout of PEFT's LoRA Linear layer (peft.tuners.lora.layer.Linear,
peft 0.15-0.18) and its eager forward in the operator order the reference replays at
runtime/wan13b_lora_cast.py:204-229. peft is not installed here; this stands in for it in tests.

    result = base_layer(x); x = x.to(lora_A.weight.dtype)
    result = result + lora_B(lora_A(dropout(x))) * scaling; result.to(result dtype)

with PEFT's mixed-batch rule (adapter_names per sample, '__base__' for none) and
disable_adapters (base only).
"""
import math

import torch
from torch import nn


class PeftLoraLinear(nn.Module):
    def __init__(self, base: nn.Linear, adapters, dtype=torch.float32):
        """adapters: {name: (rank, alpha)} in order; the first is active."""
        super().__init__()
        self.base_layer = base
        self.lora_A = nn.ModuleDict()
        self.lora_B = nn.ModuleDict()
        self.lora_dropout = nn.ModuleDict()
        self.scaling = {}
        self.lora_variant = {}
        self.use_dora = {}
        self.merged_adapters = []
        self._disable_adapters = False
        for name, (r, alpha) in adapters.items():
            self.lora_A[name] = nn.Linear(base.in_features, r, bias=False, dtype=dtype, device=base.weight.device)
            self.lora_B[name] = nn.Linear(r, base.out_features, bias=False, dtype=dtype, device=base.weight.device)
            nn.init.kaiming_uniform_(self.lora_A[name].weight, a=math.sqrt(5))
            nn.init.zeros_(self.lora_B[name].weight)
            self.lora_dropout[name] = nn.Identity()
            self.scaling[name] = alpha / r
        self._active_adapter = [next(iter(adapters))]
        base.requires_grad_(False)

    @property
    def active_adapters(self):
        return list(self._active_adapter)

    @property
    def merged(self):
        return bool(self.merged_adapters)

    @property
    def disable_adapters(self):
        return self._disable_adapters

    def set_adapter(self, name):
        self._active_adapter = [name] if isinstance(name, str) else list(name)

    def enable_adapters(self, enabled: bool):
        self._disable_adapters = not enabled

    def forward(self, x, *args, adapter_names=None, **kwargs):
        if self.disable_adapters:
            return self.base_layer(x)
        result = self.base_layer(x)
        dtype = result.dtype
        if adapter_names is not None:
            out = result.clone()
            per = x.reshape(-1, x.shape[-1]).shape[0] // x.shape[0]
            flat = out.reshape(-1, out.shape[-1])
            xf = x.reshape(-1, x.shape[-1])
            for i, name in enumerate(adapter_names):
                if name == "__base__":
                    continue
                xs = xf[i * per:(i + 1) * per].to(self.lora_A[name].weight.dtype)
                upd = self.lora_B[name](self.lora_A[name](self.lora_dropout[name](xs))) * self.scaling[name]
                flat[i * per:(i + 1) * per] = (flat[i * per:(i + 1) * per] + upd).to(dtype)
            return out
        for name in self.active_adapters:
            xa = x.to(self.lora_A[name].weight.dtype)
            result = result + self.lora_B[name](self.lora_A[name](self.lora_dropout[name](xa))) * self.scaling[name]
        return result.to(dtype)


def peft_model(dims, adapters, dtype=torch.float32, base_dtype=torch.bfloat16, seed=0):
    """A small stack of PEFT-layout linears (GELU between) with the given adapters."""
    torch.manual_seed(seed)
    layers = []
    for i, (k, n) in enumerate(dims):
        base = nn.Linear(k, n).to(base_dtype)
        layers.append(PeftLoraLinear(base, adapters, dtype=dtype))
        if i + 1 < len(dims):
            layers.append(nn.GELU())
    return nn.Sequential(*layers)
