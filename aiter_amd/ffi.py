"""The reference-shaped ctypes boundary of libaiter_amd.so (include/aiter_ctypes.h).

`ctypes_op` binds a typed Python stub to the library function of the same
name the way the reference's `compile_ops(..., ffi_type="ctypes")` does
(aiter/jit/core.py:1105-1363), from the stub's type hints:

    Tensor / Optional[Tensor] -> aiter_tensor_t* (NULL for None)
    int / Optional[int]       -> int64_t (-1 for None)
    bool -> int,  float -> float,  str / Optional[str] -> const char*
    (appended)                -> hipStream_t: torch's current stream

A call clears the library's last error, calls, and raises RuntimeError with
`aiter_get_last_error()` when the status is non-zero or an error was left.
The stubs below carry the reference's names and signatures
(aiter/ops/moe_sorting.py:11-25, aiter/ops/quant.py:472-481,
aiter/ops/moe_op.py:15-42, 172-213, 295-340, aiter/ops/activation.py:10-19,
aiter/ops/topk.py:15-38), so
a maintainer's own `compile_ops` stubs bind the same symbols unchanged.
"""
from __future__ import annotations

import ctypes
import functools
import inspect
import struct
import threading
import typing
from typing import Optional

import torch
from torch import Tensor

from . import _abi
from .enums import AITER_DTYPE, ActivationType, QuantType


class aiter_tensor_t(ctypes.Structure):
    """csrc/include/aiter_tensor.h:8-37: the layout is the contract (160 bytes)."""

    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("numel_", ctypes.c_size_t),
        ("ndim", ctypes.c_int),
        ("shape", ctypes.c_int64 * 8),
        ("strides", ctypes.c_int64 * 8),
        ("dtype_", ctypes.c_int),
        ("device_id", ctypes.c_int),
    ]


assert ctypes.sizeof(aiter_tensor_t) == 160


_DIMS = ctypes.c_int64 * 8


def to_aiter_tensor(t: Tensor) -> aiter_tensor_t:
    """Describe a torch tensor (device memory, at most 8 dims) without copying."""
    nd = t.dim()
    if nd > 8:
        raise ValueError(f"aiter_tensor_t holds at most 8 dims, got {nd}")
    code = AITER_DTYPE.get(t.dtype)
    if code is None:
        raise ValueError(f"dtype {t.dtype} has no AiterDtype code")
    dev = t.device
    if dev.type == "cuda":
        device_id = dev.index if dev.index is not None else torch.cuda.current_device()
    else:
        device_id = -1
    return aiter_tensor_t(t.data_ptr(), t.numel(), nd, _DIMS(*t.shape), _DIMS(*t.stride()), code,
                          device_id)


# The binder writes the descriptors of a call into a per-thread buffer with
# one struct.pack_into each (the aiter_tensor_t layout above: ptr, numel,
# ndim + 4 pad bytes, shape[8], strides[8], dtype, device_id) and passes
# their addresses. Building a ctypes Structure per tensor and binding the
# arguments through inspect.Signature took most of a call's host time:
# ck_moe_stage2 (ten tensors) against a no-op library, best of 15 x 1000
# calls on an x86 host, 48-50 -> 22-28 us.
_DESC = struct.Struct("<QQi4x8q8qii")
assert _DESC.size == ctypes.sizeof(aiter_tensor_t)
_ZERO8 = (0,) * 8


def _pack_desc(buf, off: int, t: Tensor, device_id: int) -> None:
    shape = t.shape
    nd = len(shape)
    if nd > 8:
        raise ValueError(f"aiter_tensor_t holds at most 8 dims, got {nd}")
    code = AITER_DTYPE.get(t.dtype)
    if code is None:
        raise ValueError(f"dtype {t.dtype} has no AiterDtype code")
    _DESC.pack_into(buf, off, t.data_ptr(), t.numel(), nd, *shape, *_ZERO8[nd:], *t.stride(),
                    *_ZERO8[nd:], code, device_id)


# torch's current raw stream of a device index (one C call); the public
# accessor builds a Stream object first
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_of(device_id: int):
    """torch's current stream on GPU device_id, None for host tensors (-1)."""
    if device_id < 0:
        return None
    if _RAW_STREAM is not None:
        return _RAW_STREAM(device_id)
    return torch.cuda.current_stream(device_id).cuda_stream


def _kind(hint):
    origin, args = typing.get_origin(hint), typing.get_args(hint)
    optional = origin is typing.Union and type(None) in args
    base = next((a for a in args if a is not type(None)), hint) if optional else hint
    return base, optional


def ctypes_op(func):
    """Bind `func`'s signature to the library symbol of its name."""
    hints = typing.get_type_hints(func)
    sig = inspect.signature(func)
    names = list(sig.parameters)
    kinds = [_kind(hints[n]) for n in names]
    argtypes = []
    for base, _ in kinds:
        if base is Tensor:
            argtypes.append(ctypes.POINTER(aiter_tensor_t))
        elif base is bool:
            argtypes.append(ctypes.c_int)
        elif base is int:
            argtypes.append(ctypes.c_int64)
        elif base is float:
            argtypes.append(ctypes.c_float)
        elif base is str:
            argtypes.append(ctypes.c_char_p)
        else:
            raise TypeError(f"{func.__name__}: no C type for parameter hint {base!r}")
    argtypes.append(ctypes.c_void_p)   # hipStream_t

    @functools.lru_cache(maxsize=1)
    def symbol():
        lib = _abi.load()
        fn = getattr(lib, func.__name__)
        fn.restype = ctypes.c_int
        fn.argtypes = argtypes
        lib.aiter_get_last_error.restype = ctypes.c_char_p
        lib.aiter_get_last_error.argtypes = []
        lib.aiter_clear_last_error.restype = None
        lib.aiter_clear_last_error.argtypes = []
        # a handle of its own that takes the descriptors' addresses (the same
        # C signature: a pointer is a pointer)
        fast = lib[func.__name__]
        fast.restype = ctypes.c_int
        fast.argtypes = [ctypes.c_void_p if a is ctypes.POINTER(aiter_tensor_t) else a
                         for a in argtypes]
        return lib, fast

    # per parameter: (name, is tensor, optional, converter of a non-tensor
    # value); positional calls without keywords skip Signature.bind
    def conv(base):
        if base is bool:
            return lambda v: 1 if v else 0
        if base is int:
            return lambda v: -1 if v is None else int(v)
        if base is float:
            return float
        return lambda v: None if v is None else str(v).encode()

    params = [(n, base is Tensor, optional, None if base is Tensor else conv(base))
              for n, (base, optional) in zip(names, kinds)]
    empty = inspect.Parameter.empty
    defaults = [sig.parameters[n].default for n in names]
    n_desc = sum(1 for p in params if p[1])
    local = threading.local()

    def descriptors():
        # this thread's buffer for the call's descriptors and its address
        b = getattr(local, "b", None)
        if b is None:
            raw = bytearray(_DESC.size * max(n_desc, 1))
            cbuf = (ctypes.c_char * len(raw)).from_buffer(raw)
            b = local.b = (raw, cbuf, ctypes.addressof(cbuf))
        return b

    @functools.wraps(func)
    def call(*args, **kwargs):
        lib, fn = symbol()
        if kwargs or len(args) > len(names):
            bound = sig.bind(*args, **kwargs)
            bound.apply_defaults()
            values = [bound.arguments[n] for n in names]
        else:
            values = list(args) + defaults[len(args):]
            for n, v in zip(names[len(args):], values[len(args):]):
                if v is empty:
                    raise TypeError(f"{func.__name__}() missing required argument: '{n}'")
        raw, _, base = descriptors()
        cargs, device, off = [], None, 0    # device: the first tensor's (-1: host)
        for (name, tensor, optional, cv), v in zip(params, values):
            if not tensor:
                cargs.append(cv(v))
            elif v is None:
                if not optional:
                    raise TypeError(f"{func.__name__}: '{name}' is required")
                cargs.append(None)
            elif not isinstance(v, Tensor):
                raise TypeError(f"{func.__name__}: '{name}' expects a tensor")
            else:
                dev = v.get_device()
                if device is None:
                    device = dev
                _pack_desc(raw, off, v, dev)
                cargs.append(base + off)
                off += _DESC.size
        lib.aiter_clear_last_error()
        rc = fn(*cargs, None if device is None else _stream_of(device))
        err = lib.aiter_get_last_error()
        if rc != 0 or err:
            lib.aiter_clear_last_error()
            raise RuntimeError(f"{func.__name__} failed: "
                               f"{err.decode(errors='replace') if err else f'status {rc}'}")

    call.argtypes = argtypes
    return call


# ------------------------------------------------------------- the entries ---
@ctypes_op
def moe_sorting_fwd(
    topk_ids: Tensor,
    topk_weights: Tensor,
    sorted_token_ids: Tensor,
    sorted_weights: Tensor,
    sorted_expert_ids: Tensor,
    num_valid_ids: Tensor,
    moe_buf: Tensor,
    num_experts: int,
    unit_size: int,
    local_expert_mask: Optional[Tensor] = None,
    num_local_tokens: Optional[Tensor] = None,
    dispatch_policy: int = 0,
) -> None: ...


@ctypes_op
def dynamic_per_token_scaled_quant(
    out: Tensor,
    input: Tensor,
    scales: Tensor,
    scale_ub: Optional[Tensor] = None,
    shuffle_scale: bool = False,
    num_rows: Optional[Tensor] = None,
    num_rows_factor: int = 1,
) -> None: ...


@ctypes_op
def moe_stage1_g1u1(
    input: Tensor,
    w1: Tensor,
    w2: Tensor,
    sorted_token_ids: Tensor,
    sorted_expert_ids: Tensor,
    num_valid_ids: Tensor,
    out: Tensor,
    inter_dim: int,
    kernelName: Optional[str],
    block_m: int,
    ksplit: int = 0,
    activation: Optional[int] = ActivationType.Silu.value,
    quant_type: Optional[int] = QuantType.No.value,
    a1_scale: Optional[Tensor] = None,
    w1_scale: Optional[Tensor] = None,
    sorted_weights: Optional[Tensor] = None,
) -> None: ...


@ctypes_op
def ck_moe_stage2(
    inter_states: Tensor,
    w1: Tensor,
    w2: Tensor,
    sorted_token_ids: Tensor,
    sorted_expert_ids: Tensor,
    num_valid_ids: Tensor,
    out: Tensor,
    topk: int,
    kernelName: Optional[str] = None,
    w2_scale: Optional[Tensor] = None,
    a2_scale: Optional[Tensor] = None,
    block_m: Optional[int] = 32,
    sorted_weights: Optional[Tensor] = None,
    quant_type: int = 0,
    activation: int = 0,
    splitk: int = 1,
    use_non_temporal_load: bool = False,
    dst_type: Optional[str] = None,
    is_shuffled: bool = True,
) -> None: ...


@ctypes_op
def ck_moe_stage1(
    hidden_states: Tensor,
    w1: Tensor,
    w2: Tensor,
    sorted_token_ids: Tensor,
    sorted_expert_ids: Tensor,
    num_valid_ids: Tensor,
    out: Tensor,
    topk: int,
    kernelName: Optional[str] = None,
    w1_scale: Optional[Tensor] = None,
    a1_scale: Optional[Tensor] = None,
    block_m: Optional[int] = 32,
    sorted_weights: Optional[Tensor] = None,
    quant_type: int = 0,
    activation: int = 0,
    splitk: Optional[int] = 1,
    use_non_temporal_load: bool = False,
    dst_type: Optional[str] = None,
    is_shuffled: bool = True,
) -> None: ...


@ctypes_op
def silu_and_mul(out: Tensor, input: Tensor) -> None: ...


@ctypes_op
def gelu_and_mul(out: Tensor, input: Tensor) -> None: ...


@ctypes_op
def fmoe_fp8_blockscale_g1u1(
    out: Tensor,
    input: Tensor,
    gate: Tensor,
    down: Tensor,
    sorted_token_ids: Tensor,
    sorted_weights: Tensor,
    sorted_expert_ids: Tensor,
    num_valid_ids: Tensor,
    topk: int,
    input_scale: Tensor,
    fc1_scale: Tensor,
    fc2_scale: Tensor,
    kernelName: Optional[str] = "",
    fc_scale_blkn: int = 128,
    fc_scale_blkk: int = 128,
    fc2_smooth_scale: Optional[Tensor] = None,
    activation: Optional[int] = ActivationType.Silu.value,
    block_size_M: int = 32,
) -> None: ...


@ctypes_op
def topk_softmax(
    topk_weights: Tensor,
    topk_indices: Tensor,
    token_expert_indices: Optional[Tensor],
    gating_output: Tensor,
    need_renorm: bool,
    num_shared_experts: int = 0,
    shared_expert_scoring_func: str = "",
) -> None: ...


@ctypes_op
def topk_sigmoid(topk_weights: Tensor, topk_indices: Tensor, gating_output: Tensor) -> None: ...


@ctypes_op
def grouped_topk(
    gating_output: Tensor,
    topk_weights: Tensor,
    topk_ids: Tensor,
    num_expert_group: int,
    topk_group: int,
    need_renorm: bool,
    is_softmax: bool = True,
    routed_scaling_factor: float = 1.0,
) -> None: ...


@ctypes_op
def biased_grouped_topk(
    gating_output: Tensor,
    correction_bias: Tensor,
    topk_weights: Tensor,
    topk_ids: Tensor,
    num_expert_group: int,
    topk_grp: int,
    need_renorm: bool,
    routed_scaling_factor: float = 1.0,
) -> None: ...


ENTRIES = ("moe_sorting_fwd", "dynamic_per_token_scaled_quant", "moe_stage1_g1u1",
           "ck_moe_stage1", "ck_moe_stage2", "silu_and_mul", "gelu_and_mul",
           "fmoe_fp8_blockscale_g1u1", "topk_softmax", "topk_sigmoid", "grouped_topk",
           "biased_grouped_topk")
