"""The reference-shaped ctypes boundary (include/aiter_ctypes.h) without a GPU.

The reference's binder, compile_ops(..., ffi_type="ctypes")
(aiter/jit/core.py:1105-1363), looks every function up by name, turns each
torch tensor into an aiter_tensor_t passed by reference (1277-1361), probes
aiter_ctypes_abi_version / aiter_get_last_error / aiter_clear_last_error
(1165-1169), clears the error, calls, and raises with the error text when one
is left. These tests do exactly that against libaiter_amd.so: descriptors
built from CPU tensors make each entry fail in its host-side checks, before
any device work, and the message comes back through the reference-named
getter.
"""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from aiter_amd import _abi, ffi
from aiter_amd.enums import AITER_DTYPE

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def lib():
    lib = _abi.load()
    lib.aiter_ctypes_abi_version.restype = ctypes.c_int
    lib.aiter_get_last_error.restype = ctypes.c_char_p
    lib.aiter_clear_last_error.restype = None
    return lib


def _declared():
    """name -> number of parameters, from include/aiter_ctypes.h."""
    text = (ROOT / "include" / "aiter_ctypes.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:int|const char\*|void)\s+(\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_error_bridge_has_the_reference_names(lib):
    assert lib.aiter_ctypes_abi_version() == 2          # status-return mode
    lib.aiter_clear_last_error()
    assert lib.aiter_get_last_error() is None           # no error reads as NULL
    # the plain entries' errors land in the same thread-local string
    assert _abi.load().aiter_amd_fused_moe_fp8_blockscale(
        16, 3, 16, 16, 16, 16, 16, 16, None, None, 16, 3, 4, 4096, 2000, 8, 8, 2, 0, 0, 0, 1,
        16, 10, None) == -1
    assert b"inter_dim" in lib.aiter_get_last_error()
    lib.aiter_clear_last_error()
    assert lib.aiter_get_last_error() is None


def test_header_entries_are_exported_and_bound_alike(lib):
    decl = _declared()
    assert set(ffi.ENTRIES) <= set(decl)
    for name in decl:
        assert hasattr(lib, name), name
    # each stub binds the header's parameters: its own plus the stream
    for name in ffi.ENTRIES:
        assert len(getattr(ffi, name).argtypes) == decl[name], name


def test_descriptor_layout():
    assert ctypes.sizeof(ffi.aiter_tensor_t) == 160
    t = torch.zeros(3, 5, dtype=torch.bfloat16)[:, 1:4]
    d = ffi.to_aiter_tensor(t)
    assert (d.ptr, d.numel_, d.ndim) == (t.data_ptr(), 9, 2)
    assert list(d.shape[:2]) == [3, 3] and list(d.strides[:2]) == [5, 1]
    assert d.dtype_ == 3 and d.device_id == -1


def test_packed_descriptor_matches_the_structure():
    """The binder packs descriptors with struct; each must be the bytes of
    the ctypes aiter_tensor_t of the same tensor (views, 8 dims, empty, 0-d)."""
    cases = [torch.zeros(3, 5, dtype=torch.bfloat16)[:, 1:4],
             torch.zeros(2, 1, 3, 1, 2, 1, 2, 3, dtype=torch.int32).transpose(0, 7),
             torch.zeros(0, 4, dtype=torch.float32), torch.tensor(1.5), torch.zeros(7, dtype=torch.uint8)]
    for t in cases:
        buf = bytearray(ctypes.sizeof(ffi.aiter_tensor_t))
        ffi._pack_desc(buf, 0, t, t.get_device())
        assert bytes(buf) == bytes(ffi.to_aiter_tensor(t)), t.shape
    with pytest.raises(ValueError, match="at most 8 dims"):
        ffi._pack_desc(bytearray(160), 0, torch.zeros([1] * 9), -1)


def _call_like_the_reference(lib, name, *args):
    """What aiter/jit/core.py's caller does: clear, call with tensors by
    reference and ints as int64, then read the error."""
    fn = getattr(lib, name)
    refs, cargs = [], []
    for a in args:
        if isinstance(a, torch.Tensor):
            d = ffi.to_aiter_tensor(a)
            refs.append(d)
            cargs.append(ctypes.byref(d))
        elif a is None:
            cargs.append(ctypes.POINTER(ffi.aiter_tensor_t)())
        elif isinstance(a, bool):
            cargs.append(ctypes.c_int(int(a)))
        elif isinstance(a, int):
            cargs.append(ctypes.c_int64(a))
        elif isinstance(a, str):
            cargs.append(ctypes.c_char_p(a.encode()))
        else:
            raise TypeError(a)
    cargs.append(ctypes.c_void_p(None))
    fn.restype = ctypes.c_int
    lib.aiter_clear_last_error()
    rc = fn(*cargs)
    err = lib.aiter_get_last_error()
    lib.aiter_clear_last_error()
    return rc, (err or b"").decode()


def test_entries_reject_bad_descriptors_before_device_work(lib):
    M, k, E, bm = 300, 8, 256, 32
    cap = M * k + E * bm - k
    ids = torch.zeros(M, k, dtype=torch.int32)
    w = torch.zeros(M, k)
    sid = torch.zeros(cap, dtype=torch.int32)
    sw = torch.zeros(cap)
    se = torch.zeros((cap + bm - 1) // bm, dtype=torch.int32)
    nv = torch.zeros(2, dtype=torch.int32)
    buf = torch.zeros(M, 512, dtype=torch.bfloat16)
    rc, err = _call_like_the_reference(lib, "moe_sorting_fwd", ids.float(), w, sid, sw, se, nv,
                                       buf, E, bm, None, None, 0)
    assert rc == -1 and "topk_ids must be i32, got fp32" in err
    rc, err = _call_like_the_reference(lib, "moe_sorting_fwd", ids, w[:, :4].contiguous(), sid, sw, se, nv,
                                       buf, E, bm, None, None, 0)
    assert rc == -1 and "topk_weights must be [300, 8]" in err
    rc, err = _call_like_the_reference(lib, "moe_sorting_fwd", ids, w, sid, sw, se, nv[:1],
                                       buf, E, bm, None, None, 0)
    assert rc == -1 and "num_valid_ids holds 1 elements, 2 needed" in err
    rc, err = _call_like_the_reference(lib, "moe_sorting_fwd", ids, w, sid, sw, se, nv,
                                       buf[:, :4], E, bm, None, None, 0)
    assert rc == -1 and "must be contiguous" in err
    # a non-contiguous view is refused, not read with the wrong strides
    T, H, I = 16, 512, 256
    a1 = torch.zeros(T, H, dtype=torch.float8_e4m3fn)
    w1 = torch.zeros(E, 2 * I, H, dtype=torch.float8_e4m3fn)
    s1 = torch.ones(E, 2 * I // 128, H // 128)
    a1s = torch.ones(H // 128, T)
    out = torch.zeros(T + 1, k, I, dtype=torch.float8_e4m3fn)
    se16 = torch.zeros(100, dtype=torch.int32)
    args = [a1, w1, w1, sid, se16, nv, out, I, "", 16, 0, 0, 4, a1s, s1, None]
    rc, err = _call_like_the_reference(lib, "moe_stage1_g1u1", *args[:12], 2, *args[13:])
    assert rc == -1 and "only QuantType.per_1x128" in err
    rc, err = _call_like_the_reference(lib, "moe_stage1_g1u1", *args[:10], 1, *args[11:])
    assert rc == -1 and "ksplit must be 0" in err
    rc, err = _call_like_the_reference(lib, "moe_stage1_g1u1", *args[:6],
                                       torch.zeros(T, k, I, dtype=torch.float8_e4m3fn),
                                       *args[7:])
    assert rc == -1 and "out must be [17, 8, 256]" in err
    rc, err = _call_like_the_reference(lib, "moe_stage1_g1u1", *args[:14],
                                       torch.ones(E, 2 * I // 128, 1), None)
    assert rc == -1 and "w1_scale must be" in err
    # stage 2 into a bf16 moe_buf of the wrong width
    a2 = torch.zeros(T, k, I, dtype=torch.float8_e4m3fn)
    w2 = torch.zeros(E, H, I, dtype=torch.float8_e4m3fn)
    s2 = torch.ones(E, H // 128, I // 128)
    a2s = torch.ones(T, k, I // 128)
    rc, err = _call_like_the_reference(lib, "ck_moe_stage2", a2, w2, w2, sid, se16, nv,
                                       torch.zeros(T, H + 2, dtype=torch.bfloat16), k, "", s2,
                                       a2s, 16, None, 4, 0, 1, False, "", True)
    assert rc == -1 and "out must be [16, 512]" in err
    rc, err = _call_like_the_reference(lib, "ck_moe_stage2", a2, w2, w2, sid, se16, nv,
                                       torch.zeros(T, H, dtype=torch.bfloat16), k, "", s2,
                                       a2s, 16, None, 3, 0, 1, False, "", True)
    assert rc == -1 and "fp8 w2 needs QuantType.per_1x128" in err
    rc, err = _call_like_the_reference(lib, "dynamic_per_token_scaled_quant",
                                       torch.zeros(4, 256, dtype=torch.float8_e4m3fn),
                                       torch.zeros(4, 256, dtype=torch.bfloat16),
                                       torch.zeros(8), None, False, None, 1)
    assert rc == -1 and "viewed as [groups, 128]" in err
    # shared experts: the reference's only scoring function is sigmoid, and
    # num_shared_experts > 0 with no function is an error
    rc, err = _call_like_the_reference(lib, "topk_softmax", torch.zeros(4, 3),
                                       torch.zeros(4, 2, dtype=torch.int32), None,
                                       torch.zeros(4, 9), True, 1, "")
    assert rc == -1 and "needs shared_expert_scoring_func 'sigmoid'" in err
    rc, err = _call_like_the_reference(lib, "topk_softmax", torch.zeros(4, 3),
                                       torch.zeros(4, 2, dtype=torch.int32), None,
                                       torch.zeros(4, 9), True, 1, "softmax")
    assert rc == -1 and "Only 'sigmoid' scoring function" in err


def test_python_binder_raises_with_the_library_message():
    with pytest.raises(RuntimeError, match="moe_sorting_fwd failed: .*topk_ids must be i32"):
        ffi.moe_sorting_fwd(torch.zeros(4, 2), torch.zeros(4, 2), torch.zeros(8, dtype=torch.int32),
                            torch.zeros(8), torch.zeros(8, dtype=torch.int32),
                            torch.zeros(2, dtype=torch.int32),
                            torch.zeros(4, 128, dtype=torch.bfloat16), 4, 4)
    assert AITER_DTYPE[torch.uint8] == 11


def test_reference_sequence_entries_reject_bad_descriptors(lib):
    """ck_moe_stage1, silu_and_mul / gelu_and_mul and fmoe_fp8_blockscale_g1u1
    check their descriptors the way the other entries do (before any device
    work or workspace allocation)."""
    T, H, I, E, k, bm = 16, 512, 256, 8, 2, 16
    cap = T * k + E * bm - k
    sid = torch.zeros(cap, dtype=torch.int32)
    sw = torch.zeros(cap)
    se = torch.zeros((cap + bm - 1) // bm, dtype=torch.int32)
    nv = torch.zeros(2, dtype=torch.int32)
    a1 = torch.zeros(T, H, dtype=torch.float8_e4m3fn)
    a1s = torch.ones(T, H // 128)
    w1 = torch.zeros(E, 2 * I, H, dtype=torch.float8_e4m3fn)
    w2 = torch.zeros(E, H, I, dtype=torch.float8_e4m3fn)
    s1 = torch.ones(E, 2 * I // 128, H // 128)
    s2 = torch.ones(E, H // 128, I // 128)
    a2 = torch.zeros(T, k, I, dtype=torch.bfloat16)
    base = [a1, w1, w2, sid, se, nv, a2, k, "", s1, a1s, bm, None, 4, 0, 0, False, "", True]

    def stage1(**over):
        args = list(base)
        names = ["hidden_states", "w1", "w2", "sid", "se", "nv", "out", "topk", "kernelName",
                 "w1_scale", "a1_scale", "block_m", "sorted_weights", "quant_type",
                 "activation", "splitk", "nt", "dst_type", "is_shuffled"]
        for key, v in over.items():
            args[names.index(key)] = v
        return _call_like_the_reference(lib, "ck_moe_stage1", *args)

    rc, err = stage1(quant_type=3)
    assert rc == -1 and "fp8 w1 needs QuantType.per_1x128" in err
    rc, err = stage1(out=torch.zeros(T, k, I))
    assert rc == -1 and "out must be bf16 or fp16" in err
    rc, err = stage1(splitk=2)          # split K writes fp32 gate|up rows
    assert rc == -1 and "out must be fp32" in err
    rc, err = stage1(splitk=2, out=torch.zeros(T * k, I))
    assert rc == -1 and "with splitk > 1, out must be fp32" in err
    rc, err = stage1(splitk=3, out=torch.zeros(T * k, 2 * I))
    assert rc == -1 and "ksplit must divide model_dim / 128" in err
    rc, err = stage1(block_m=48)
    assert rc == -1 and "block_m must be 16, 32, 64 or 128" in err
    rc, err = stage1(activation=2)
    assert rc == -1 and "ActivationType.Silu (0) and Gelu (1)" in err
    rc, err = stage1(w1_scale=torch.ones(E, 2 * I // 128, 1))
    assert rc == -1 and "w1_scale must be [8, 4, 4]" in err

    rc, err = _call_like_the_reference(lib, "silu_and_mul", torch.zeros(4, 10),
                                       torch.zeros(4, 21))
    assert rc == -1 and "twice out's" in err
    rc, err = _call_like_the_reference(lib, "gelu_and_mul", torch.zeros(4, 10, dtype=torch.int32),
                                       torch.zeros(4, 20))
    assert rc == -1 and "out must be fp32 or bf16 or fp16" in err
    rc, err = _call_like_the_reference(lib, "silu_and_mul", torch.zeros(4, 10),
                                       torch.zeros(8, 20)[::2])
    assert rc == -1 and "input must be contiguous" in err

    out = torch.zeros(T, H, dtype=torch.bfloat16)
    fm = [out, a1, w1, w2, sid, sw, se, nv, k, a1s.t().contiguous(), s1, s2, "", 128, 128, None,
          0, bm]
    rc, err = _call_like_the_reference(lib, "fmoe_fp8_blockscale_g1u1", *fm[:13], 64, *fm[14:])
    assert rc == -1 and "only 128x128 weight scale blocks" in err
    rc, err = _call_like_the_reference(lib, "fmoe_fp8_blockscale_g1u1", *fm[:15], s2, *fm[16:])
    assert rc == -1 and "fc2_smooth_scale is not supported" in err
    rc, err = _call_like_the_reference(lib, "fmoe_fp8_blockscale_g1u1", *fm[:3],
                                       torch.zeros(E, H, I + 128, dtype=torch.float8_e4m3fn),
                                       *fm[4:])
    assert rc == -1 and "down must be [8, 512, 256]" in err
    rc, err = _call_like_the_reference(lib, "fmoe_fp8_blockscale_g1u1",
                                       torch.zeros(T, H), *fm[1:])
    assert rc == -1 and "out must be bf16 or fp16" in err
    rc, err = _call_like_the_reference(lib, "fmoe_fp8_blockscale_g1u1", *fm[:6], se[:2], *fm[7:])
    assert rc == -1 and "sorted_expert_ids holds fewer blocks" in err
    rc, err = _call_like_the_reference(lib, "fmoe_fp8_blockscale_g1u1", *fm[:16], 2, bm)
    assert rc == -1 and "Silu (0) and Gelu (1)" in err
