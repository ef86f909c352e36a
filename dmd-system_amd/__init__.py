"""MI355X-native batched multi-LoRA linear (gfx950 HIP kernels behind a C ABI).

Public API:
    SegmentRouting, BASE_ONLY            row-segment -> adapter routing
    MultiLoRAFunction, multi_lora_linear autograd op
    MultiLoRAFP8Function, multi_lora_linear_fp8   the same with an e4m3 frozen base
    TrainableLowRankLinear, trainable_scope, MultiLoRALinear   drop-in modules
    RoleBatch, fuse_roles, roles_active  several roles' forwards in one pass over the shared base
    kernels                              torch front end of each C-ABI entry point
    load_library()                       load libmlora.so (raises if missing)

The directory name is not a Python identifier; importers load it as
``dmd_system_amd`` by path (see ``load_package`` in the repository's
``__graft_entry__.py``).
"""
from . import _lib, kernels
from .function import MultiLoRAFP8Function, MultiLoRAFunction, multi_lora_linear, multi_lora_linear_fp8
from .low_rank import MultiLoRALinear, TrainableLowRankLinear, trainable_scope
from .roles import RoleBatch, fuse_roles, roles_active
from .routing import BASE_ONLY, SegmentRouting


def load_library():
    return _lib.load()


__all__ = [
    "BASE_ONLY", "SegmentRouting", "MultiLoRAFunction", "multi_lora_linear", "MultiLoRAFP8Function",
    "multi_lora_linear_fp8", "MultiLoRALinear",
    "TrainableLowRankLinear", "trainable_scope", "RoleBatch", "fuse_roles", "roles_active", "kernels",
    "load_library",
]
