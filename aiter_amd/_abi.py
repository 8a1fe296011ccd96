"""ctypes binding of libaiter_amd.so (declared in include/aiter_amd.h).

Mirrors the reference's ctypes path (aiter/jit/core.py:1105-1363): plain
device pointers and int64 scalars go in, the stream is the last argument,
a non-zero return raises RuntimeError carrying aiter_amd_get_last_error().
There is no fallback: a missing or unloadable library raises immediately.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

_LIB_PATH = Path(__file__).resolve().parent / "libaiter_amd.so"
_lock = threading.Lock()
_lib = None

ABI_VERSION = 3   # AITER_AMD_ABI_VERSION of include/aiter_amd.h

c_i32p = ctypes.c_void_p
c_vp = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_int = ctypes.c_int

# name -> (restype, argtypes); the order follows include/aiter_amd.h
_SIGNATURES = {
    "aiter_amd_abi_version": (c_int, []),
    "aiter_amd_get_last_error": (ctypes.c_char_p, []),
    "aiter_amd_clear_last_error": (None, []),
    "aiter_amd_moe_sorting_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64]),
    "aiter_amd_default_block_m": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "aiter_amd_layer_timing_begin": (c_int, [c_i64]),
    "aiter_amd_layer_timing_end": (c_i64, [c_vp, c_i64]),
    "aiter_amd_topk_softmax": (
        c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_int, c_vp]),
    "aiter_amd_topk_softmax_shared": (
        c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_int,
                c_vp]),
    "aiter_amd_topk_sigmoid": (
        c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp]),
    "aiter_amd_grouped_topk": (
        c_int,
        [c_vp, c_int, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_int, c_int, ctypes.c_float, c_vp,
         c_i64, c_vp, c_i64, c_vp]),
    "aiter_amd_moe_sorting_fwd": (
        c_int,
        [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp, c_i64, c_i64,
         c_i64, c_vp, c_vp, c_i64, c_vp, c_i64, c_vp],
    ),
    "aiter_amd_dynamic_per_group_quant_fp8": (
        c_int, [c_vp, c_int, c_i64, c_i64, c_i64, c_vp, c_vp, c_int, c_vp, c_i64, c_vp]),
    "aiter_amd_moe_stage1_fp8_blockscale": (
        c_int,
        [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "aiter_amd_moe_stage2_fp8_blockscale": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "aiter_amd_moe_stage1_a8w4": (
        c_int,
        [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "aiter_amd_moe_stage2_a8w4": (
        c_int,
        [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "aiter_amd_moe_stage1_rows": (
        c_int,
        [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "aiter_amd_act_and_mul": (c_int, [c_vp, c_int, c_vp, c_int, c_i64, c_i64, c_i64, c_vp]),
    "aiter_amd_fused_moe_sorted_workspace_bytes": (
        c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "aiter_amd_fused_moe_sorted_fp8_blockscale": (
        c_int,
        [c_vp, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_vp,
         c_int, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "aiter_amd_moe_acc_to_out": (c_int, [c_vp, c_vp, c_int, c_vp, c_i64, c_i64, c_vp]),
    "aiter_amd_fused_moe_workspace_bytes": (c_i64, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64]),
    "aiter_amd_fused_moe_workspace_a2_offsets": (
        c_int, [c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "aiter_amd_fused_moe_fp8_blockscale": (
        c_int,
        [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "aiter_amd_fused_moe_fp8_blockscale_noalloc": (
        c_int,
        [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp],
    ),
    "aiter_amd_fused_moe_a8w4": (
        c_int,
        [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "aiter_amd_fused_moe_1stage_fp8_blockscale": (
        c_int,
        [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
    "aiter_amd_fused_moe_1stage_a8w4": (
        c_int,
        [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_i64, c_i64,
         c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp],
    ),
}

EXPORTED = tuple(_SIGNATURES)


def lib_path() -> Path:
    return Path(os.environ.get("AITER_AMD_LIB", _LIB_PATH))


def load() -> ctypes.CDLL:
    """Load the library once; raises if it is missing or has the wrong ABI."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = lib_path()
        if not path.exists():
            raise RuntimeError(
                f"aiter_amd: {path} is missing; build it with `python -m aiter_amd.build`")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.aiter_amd_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"aiter_amd: ABI version {ver} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    """Call a status-returning entry point; raise RuntimeError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.aiter_amd_get_last_error().decode(errors="replace")
        lib.aiter_amd_clear_last_error()
        raise RuntimeError(f"{name} failed: {msg}")


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))
