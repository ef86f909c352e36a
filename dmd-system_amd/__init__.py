"""MI355X-native batched multi-LoRA linear (gfx950 HIP kernels behind a C ABI).

Public API:
    SegmentRouting, BASE_ONLY            row-segment -> adapter routing
    MultiLoRAFunction, multi_lora_linear autograd op
    MultiLoRAFP8Function, multi_lora_linear_fp8   the same with an e4m3 frozen base
    MultiLoRAGatedResidualFunction, multi_lora_linear_gated   with the block's gated residual fused
    TrainableLowRankLinear, trainable_scope, MultiLoRALinear   drop-in modules
    LoRALinear, install_lora             the native models' fp32-master LoRA (native/models.py)
    MultiLoRAF32Function                 the float32 path (precision='fp32')
    RoleBatch, fuse_roles, roles_active  several roles' forwards in one pass over the shared base
    fuse_shared_inputs, SharedInputGroup, SharedInputMultiLoRAFunction   linears reading one input, stacked
    export_adapters, import_adapters, save_adapters, load_adapters   PEFT / DiffSynth adapter state
    install_peft_multi_lora, peft_roles_active   PEFT LoRA layers (W1 / H3) on the multi-LoRA op
    livewan, LiveWanLoRALinear, install_livewan_multi_lora   LiveWan's critic LoRA (wanstreamer/lora.py)
    restore_identity()                   kernel / source identity for the run's model metadata
    kernels                              torch front end of each C-ABI entry point
    fused_modulated_norm_epilogue, fused_modulated_norm_materialization,
    fused_bf16_layernorm_modulation, fused_layernorm_modulation   the block's modulated LayerNorm
    fused_bf16_layernorm_modulation_hidden_backward, fused_reduced_component_gradient,
    fused_tensor4d_component_gradient      its fused backward
    ModulatedLayerNormFunction, modulated_layer_norm   the same as one autograd op
    load_library()                       load libmlora.so (raises if missing)

The directory name is not a Python identifier; importers load it as
``dmd_system_amd`` by path (see ``load_package`` in the repository's
``__graft_entry__.py``).
"""
from . import _lib, kernels
from .adapters import export_adapters, import_adapters, load_adapters, save_adapters
from .function import (MultiLoRAF32Function, MultiLoRAFP8Function, MultiLoRAFunction,
                       MultiLoRAGatedResidualFunction, SharedInputMultiLoRAFunction, StackedLinearsFunction,
                       multi_lora_linear,
                       multi_lora_linear_fp8, multi_lora_linear_gated, shared_input_multi_lora)
from .low_rank import LoRALinear, MultiLoRALinear, TrainableLowRankLinear, install_lora, trainable_scope
from .roles import RoleBatch, fuse_roles, roles_active
from .routing import BASE_ONLY, SegmentRouting
from .shared_input import SharedInputGroup, fuse_shared_inputs, release_shared_inputs
from .peft_site import install_peft_multi_lora, peft_roles_active, uninstall_peft_multi_lora
from . import livewan
from .livewan import LiveWanLoRALinear, install_livewan_multi_lora, uninstall_livewan_multi_lora
from ._lib import restore_identity
from .modulated_norm import (ModulatedLayerNormFunction, fused_bf16_layernorm_modulation,
                             fused_bf16_layernorm_modulation_hidden_backward, fused_layernorm_modulation,
                             fused_layernorm_modulation_hidden_backward, fused_modulated_norm_epilogue,
                             fused_modulated_norm_materialization, fused_reduced_component_gradient,
                             fused_tensor4d_component_gradient, modulated_layer_norm)


def load_library():
    return _lib.load()


__all__ = [
    "BASE_ONLY", "SegmentRouting", "MultiLoRAFunction", "multi_lora_linear", "MultiLoRAFP8Function",
    "MultiLoRAF32Function", "LoRALinear", "install_lora",
    "multi_lora_linear_fp8", "MultiLoRAGatedResidualFunction", "multi_lora_linear_gated", "MultiLoRALinear",
    "TrainableLowRankLinear", "trainable_scope", "RoleBatch", "fuse_roles", "roles_active",
    "SharedInputMultiLoRAFunction", "StackedLinearsFunction", "shared_input_multi_lora", "SharedInputGroup", "fuse_shared_inputs",
    "release_shared_inputs", "export_adapters", "import_adapters", "save_adapters", "load_adapters", "kernels",
    "load_library", "install_peft_multi_lora", "uninstall_peft_multi_lora", "peft_roles_active",
    "livewan", "LiveWanLoRALinear", "install_livewan_multi_lora", "uninstall_livewan_multi_lora",
    "restore_identity",
    "fused_modulated_norm_epilogue", "fused_modulated_norm_materialization", "fused_bf16_layernorm_modulation",
    "fused_layernorm_modulation", "fused_bf16_layernorm_modulation_hidden_backward",
    "fused_layernorm_modulation_hidden_backward", "fused_reduced_component_gradient",
    "fused_tensor4d_component_gradient", "ModulatedLayerNormFunction", "modulated_layer_norm",
]
