"""ctypes binding of the C ABI in ``include/mlora.h`` (``libmlora.so``).

The library is built in-tree by ``build.py``. Loading it never falls back to
anything else: a missing or stale library is an error for every caller. A library
is stale when its ABI version differs, or when the sources next to it (csrc/ and
include/) hash to another value than the one it was built with.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libmlora.so"

ABI_VERSION = 9
MAX_SEGMENTS = 128
MAX_ADAPTERS = 32
MAX_RANK = 256
MAX_STACKED = 8
MAX_GEMM_RANK = MAX_RANK * MAX_STACKED  # the GEMM entry points: the stacked LoRA term of up to 8 linears

F32, BF16, FP8_E4M3 = 0, 1, 2

OK = 0
ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_LAUNCH, ERR_LIMIT, ERR_DEVICE = -1, -2, -3, -4, -5, -6
NOALLOC_SCRATCH_BYTES = 64 << 20

# Every entry point declared in include/mlora.h with its ctypes signature.
_vp, _i64, _i32, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int
_pvp = ctypes.POINTER(ctypes.c_void_p)
_pi32 = ctypes.POINTER(ctypes.c_int32)
_pi64 = ctypes.POINTER(ctypes.c_int64)
_pf32 = ctypes.POINTER(ctypes.c_float)

SIGNATURES = {
    "mlora_abi_version": (_int, []),
    "mlora_status_string": (ctypes.c_char_p, [_int]),
    "mlora_source_hash": (ctypes.c_char_p, []),
    "mlora_shrink": (_int, [_vp, _i64, _i64, _i64, _pvp, _pvp, _int, _pi32, _pf32, _i32,
                            _pi64, _pi32, _i32, _vp, _i64, _vp, _i32, _vp, _vp]),
    "mlora_frag_bytes": (_i64, [_i64, _i32, _pi64, _pi32, _i32]),
    "mlora_gemm_fwd": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _int, _vp, _i64,
                              _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _int, _vp]),
    "mlora_gemm_fwd_stacked": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _int, _vp, _i64, _i64,
                                      _pvp, _pi32, _i32, _pi64, _pi32, _i32, _pvp, _i64, _vp]),
    "mlora_gemm_dx_stacked": (_int, [_pvp, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                     _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _vp]),
    "mlora_gemm_fwd_gated": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _int, _vp, _i64,
                                    _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _vp, _i64, _i64,
                                    _vp, _i64, _int, _vp]),
    "mlora_gate_scale_rows": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _int, _vp]),
    "mlora_modulated_norm": (_int, [_vp, _int, _i64, _i64, _int, ctypes.c_float, _vp, _vp, _int, _vp, _int, _vp, _int,
                                    _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _vp]),
    "mlora_modulated_norm_backward": (_int, [_vp, _int, _i64, _i64, _vp, _int, _i64, _i64, _vp, _int,
                                             _vp, _int, _i64, _i64, _vp, _int, _i64, _i64, _vp, _vp, ctypes.c_float,
                                             _i64, _i64, _i64, _vp]),
    "mlora_modulated_norm_component_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "mlora_modulated_norm_component_grad": (_int, [_vp, _int, _i64, _i64, _vp, _int, _i64, _i64, _vp, _vp,
                                                   _vp, _int, _i64, _i64, _i64, _int, _int, _int, _vp, _i64,
                                                   _i64, _i64, _i64, _vp]),
    "mlora_gemm_dx": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                             _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _int, _vp]),
    "mlora_seg_outer": (_int, [_vp, _i64, _i64, _i64, _vp, _i32, _pvp, _int, _int, _pi32, _i32,
                               _pi64, _pi32, _i32, _vp, _i64, _vp]),
    "mlora_seg_outer_workspace_bytes": (_i64, [_i64, _i64, _pi32, _i32, _pi64, _pi32, _i32]),
    "mlora_seg_outer_noalloc": (_int, [_vp, _i64, _i64, _i64, _vp, _i32, _pvp, _int, _int, _pi32, _i32,
                                       _pi64, _pi32, _i32, _vp]),
    "mlora_quantize_rows_fp8": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _vp]),
    "mlora_dequant_rows_fp8": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "mlora_div_rows_bf16": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "mlora_div_rows_bf16_batch": (_int, [_pvp, _pi64, _vp, _i64, _pi64, _pvp, _pi64, _i32, _vp]),
    "mlora_gemm_fwd_fp8": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _i64, _vp, _int, _vp, _i64,
                                  _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _int, _vp]),
    "mlora_f32_shrink": (_int, [_vp, _i64, _i64, _i64, _pvp, _int, _pi32, _pf32, _i32,
                                _pi64, _pi32, _i32, _vp, _i64, _i64, _vp]),
    "mlora_f32_gemm_fwd": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64,
                                  _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _vp]),
    "mlora_f32_gemm_dx": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64,
                                 _pvp, _pi32, _i32, _pi64, _pi32, _i32, _vp, _i64, _vp]),
    "mlora_f32_seg_outer": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _pvp, _int, _pi32, _i32,
                                   _pi64, _pi32, _i32, _vp]),
}

_LIB = None


class MloraError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, name: str, status: int, message: str):
        super().__init__(f"{name} failed with status {status}: {message}")
        self.status = status


def load():
    """Load ``libmlora.so`` once and bind every declared symbol."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python dmd-system_amd/build.py` "
                           "(or __graft_entry__.build()) before using the HIP path")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    version = lib.mlora_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"libmlora ABI version {version} != expected {ABI_VERSION}; rebuild the library")
    built = lib.mlora_source_hash().decode()
    expected = expected_source_hash()
    if expected is not None and built != expected:
        raise RuntimeError(f"{LIB_PATH} was built from other sources (hash {built[:16]}…, the sources here hash "
                           f"to {expected[:16]}…): rebuild it with `python dmd-system_amd/build.py`")
    _LIB = lib
    return lib


def expected_source_hash() -> str | None:
    """Hash of the HIP sources beside the library (None when they are not shipped with it)."""
    from . import build
    if not any(build.CSRC.glob("*.hip")):
        return None
    return build.source_hash()


def check(name: str, status: int) -> None:
    if status != OK:
        msg = load().mlora_status_string(status).decode()
        raise MloraError(name, status, msg)


def ptr_array(values) -> ctypes.Array:
    return (ctypes.c_void_p * max(1, len(values)))(*[v or None for v in values])


def i32_array(values) -> ctypes.Array:
    return (ctypes.c_int32 * max(1, len(values)))(*values)


def i64_array(values) -> ctypes.Array:
    return (ctypes.c_int64 * max(1, len(values)))(*values)


def f32_array(values) -> ctypes.Array:
    return (ctypes.c_float * max(1, len(values)))(*values)


def python_source_hash() -> str:
    """SHA-256 over this package's Python modules (name and bytes of each, in name order)."""
    import hashlib
    h = hashlib.sha256()
    for f in sorted(LIB_PATH.parent.glob("*.py")):
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
        h.update(b"\0")
    return h.hexdigest()


def restore_identity() -> dict:
    """The entries a model factory adds to ``ModelComponents.metadata`` so that the reference's
    restore identity follows this op's arithmetic. session.construct stores the metadata as
    ``model_metadata`` in the run identity (training/session.py:164-169), and a resume is refused
    when the identity differs. The reference's source-derived semantics
    (training/semantics.py:466-474) binds Python it reaches through static imports; the HIP
    sources and the library are not Python, and a by-path import of this package is not static,
    so they enter here: the C ABI version, the hash of the sources the loaded libmlora.so was
    built from (csrc/ and include/, the value it returns from mlora_source_hash), the hash of the
    package's Python modules, and the GPU architecture the kernels are compiled for."""
    lib = load()
    return {"mi355x_multi_lora": {
        "abi_version": int(lib.mlora_abi_version()),
        "kernel_source_sha256": lib.mlora_source_hash().decode(),
        "python_source_sha256": python_source_hash(),
        "arch": "gfx950",
    }}
