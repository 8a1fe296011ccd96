"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/aiter_amd.h declares, reports its ABI version, and rejects invalid
arguments (before any device work) with -1 and a readable last error --
the reference's ctypes error bridge (csrc/include/aiter_ctypes_error.h:
60-147).  Also host-side logic of the Python layer.
"""
import ctypes
import importlib
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import aiter_amd as A
from aiter_amd import _abi
from oracle import moe_ref as R

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "aiter_amd.h").read_text()
    return sorted(set(re.findall(r"\b(aiter_amd_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _abi.load()


def test_header_and_binding_agree():
    assert _declared_symbols() == sorted(_abi.EXPORTED)
    text = (ROOT / "include" / "aiter_amd.h").read_text()
    assert int(re.search(r"#define AITER_AMD_ABI_VERSION (\d+)", text).group(1)) == _abi.ABI_VERSION


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_symbols():
        assert hasattr(lib, name), name


def test_abi_version(lib):
    assert lib.aiter_amd_abi_version() == _abi.ABI_VERSION == 3


def _expect_error(name, *args, match):
    with pytest.raises(RuntimeError, match=match):
        _abi.call(name, *args)


def test_sorting_validation_errors(lib):
    # topk out of range, block_size out of range, capacity too small, NULL
    _expect_error("aiter_amd_moe_sorting_fwd", 1, 1, 4, 0, 1, 1, 1, 1, 100, 10, None, 0, 8, 32,
                  None, None, 0, None, 0, None, match="topk must be")
    _expect_error("aiter_amd_moe_sorting_fwd", 1, 1, 4, 2, 1, 1, 1, 1, 100, 10, None, 0, 8, 0,
                  None, None, 0, None, 0, None, match="block_size")
    _expect_error("aiter_amd_moe_sorting_fwd", 1, 1, 4, 2, 1, 1, 1, 1, 10, 10, None, 0, 8, 32,
                  None, None, 0, None, 0, None, match="capacity")
    _expect_error("aiter_amd_moe_sorting_fwd", None, 1, 4, 2, 1, 1, 1, 1, 1000, 100, None, 0, 8,
                  32, None, None, 0, None, 0, None, match="NULL")
    _expect_error("aiter_amd_moe_sorting_fwd", 16, 16, 4, 2, 16, 16, 16, 16, 1000, 100, 16, 24,
                  8, 32, None, None, 0, None, 0, None, match="multiple of 16")
    # large token counts need a workspace
    need = lib.aiter_amd_moe_sorting_workspace_bytes(100000, 8, 256)
    assert need > 0 and lib.aiter_amd_moe_sorting_workspace_bytes(8, 8, 256) == 0
    _expect_error("aiter_amd_moe_sorting_fwd", 16, 16, 100000, 8, 16, 16, 16, 16, 10**7, 10**6,
                  None, 0, 256, 32, None, None, 0, None, 0, None, match="workspace")


def test_quant_validation_errors():
    _expect_error("aiter_amd_dynamic_per_group_quant_fp8", 16, 3, 4, 256, 64, 16, 16, 0, None, 1,
                  None, match="group_size 128")
    _expect_error("aiter_amd_dynamic_per_group_quant_fp8", 16, 4, 4, 256, 128, 16, 16, 0, None, 1,
                  None, match="bf16 or fp16")
    _expect_error("aiter_amd_dynamic_per_group_quant_fp8", 16, 3, 4, 200, 128, 16, 16, 0, None, 1,
                  None, match="multiple of 128")
    _expect_error("aiter_amd_dynamic_per_group_quant_fp8", 8, 3, 4, 256, 128, 16, 16, 0, None, 1,
                  None, match="aligned")


def test_stage_validation_errors():
    # a1, a1_scale, transposed, w1, w1_scale, sorted_ids, sorted_weights (NULL: no
    # doweight_stage1), sorted_expert_ids, num_valid_ids, a2, a2_scale
    args = [16, 16, 0, 16, 16, 16, None, 16, 16, 16, 16]
    _expect_error("aiter_amd_moe_stage1_fp8_blockscale", *args, 4, 4096, 2000, 8, 2, 32, 10, 0, 1,
                  None, match="inter_dim must be")
    _expect_error("aiter_amd_moe_stage1_fp8_blockscale", *args, 4, 4096, 2048, 8, 2, 256, 10, 0,
                  1, None, match="block_m must be 16, 32, 64 or 128")
    _expect_error("aiter_amd_moe_stage1_fp8_blockscale", *args, 4, 4224, 1152, 8, 2, 128, 10, 0,
                  1, None, match="block_m 128 needs")
    _expect_error("aiter_amd_moe_stage1_fp8_blockscale", *args, 4, 4096, 2048, 8, 2, 32, 10, 2, 1,
                  None, match=r"Silu \(0\) and Gelu \(1\)")
    _expect_error("aiter_amd_moe_stage2_fp8_blockscale", 16, 16, 16, 16, 16, 16, 16, 16, 16, 4,
                  4, 4096, 2048, 8, 40, 32, 10, 1, None, match="topk must be")
    _expect_error("aiter_amd_moe_stage2_fp8_blockscale", 16, 16, 16, 16, 16, 16, 16, 16, 16, 0,
                  4, 4096, 2048, 8, 2, 32, 10, 1, None, match="fp32, bf16 or fp16")
    _expect_error("aiter_amd_moe_acc_to_out", 16, 16, 4, 16, 4, 64, None, match="bf16 or fp16")


def test_fused_validation_errors(lib):
    base = [16, 3, 16, 16, 16, 16, 16, 16, None, None, 16, 3]
    # ... tokens, model_dim, inter_dim, E, global E, topk, block_m, activation,
    # doweight_stage1, w_shuffled, workspace, workspace_bytes, stream
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *base, 4, 4096, 2048, 8, 8, 2, 0, 0, 0, 1,
                  16, 10, None, match="workspace of")
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *base, 4, 4096, 2048, 8, 8, 2, 0, 2, 0, 1,
                  16, 10, None, match="Gelu")
    masked = [16, 3, 16, 16, 16, 16, 16, 16, 16, None, 16, 3]    # expert_mask given
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *masked, 4, 4096, 2048, 8, 4, 2, 0, 0, 0,
                  1, 16, 10**9, None, match="global_experts")
    # an expert-parallel share may hold fewer experts than topk (4 local of 33
    # with top-8): validation passes and stops only at the too-small workspace
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *masked, 4, 4096, 2048, 4, 33, 8, 0, 0, 0,
                  1, 16, 10, None, match="workspace of")
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *masked, 4, 4096, 2048, 4, 6, 8, 0, 0, 0,
                  1, 16, 10, None, match="topk must not exceed")
    # the one-launch entries take 16/32-row blocks and model_dim % 256 == 0 only
    for name in ("aiter_amd_fused_moe_1stage_fp8_blockscale", "aiter_amd_fused_moe_1stage_a8w4"):
        _expect_error(name, *base, 4, 4096, 2048, 8, 8, 2, 64, 0, 0, 1, 16, 10**9, None,
                      match="one-launch layer needs block_m 16 or 32")
        _expect_error(name, *base, 4, 384, 256, 8, 8, 2, 16, 0, 0, 1, 16, 10**9, None,
                      match="one-launch layer needs")
    ws = lib.aiter_amd_fused_moe_workspace_bytes(8192, 4096, 2048, 256, 256, 8, 64)
    # sorted ids/weights + a1 + a2 + f32 accumulator dominate
    assert ws > 8192 * 4096 * (1 + 4) + 8192 * 8 * 2048
    assert lib.aiter_amd_fused_moe_workspace_bytes(64, 4096, 2048, 32, 16, 8, 0) == -1


def test_cached_workspace_size_follows_the_ksplit_override(lib, monkeypatch):
    """The host path caches the layer's workspace size per shape; the
    stage-1 K-split override (AITER_AMD_ST_KSPLIT1) sizes the split's partial
    sums, so a new value must give the new size, not the cached one."""
    F = importlib.import_module("aiter_amd.fused_moe")   # the module, not the function
    shape = (5, 2048, 512, 8, 8, 4, 16)
    monkeypatch.setenv("AITER_AMD_ST_KSPLIT1", "1")
    one = F._layer_workspace_bytes(*shape)
    monkeypatch.setenv("AITER_AMD_ST_KSPLIT1", "4")
    four = F._layer_workspace_bytes(*shape)
    assert four > one
    assert four == lib.aiter_amd_fused_moe_workspace_bytes(*shape)
    monkeypatch.setenv("AITER_AMD_ST_KSPLIT1", "1")
    assert F._layer_workspace_bytes(*shape) == one


def test_workspace_a2_offsets_lie_inside_the_workspace():
    """The a2 section the one-call layer exposes: 256-byte aligned, the
    fp8 rows [T*k, I] before their f32 scales [T*k, I/128], both inside the
    workspace the size query reports, at every block size and for an EP
    share; invalid sizes are rejected."""
    import ctypes
    for T, H, I, E, G, k in ((8192, 4096, 2048, 256, 256, 8), (4096, 4096, 2048, 32, 256, 8),
                             (1, 1024, 512, 8, 8, 2), (0, 4096, 2048, 256, 256, 8)):
        for bm in (0, 16, 32, 64, 128):
            off = (ctypes.c_int64 * 2)()
            _abi.call("aiter_amd_fused_moe_workspace_a2_offsets", T, H, I, E, G, k, bm,
                      ctypes.addressof(off))
            ws = _abi.query("aiter_amd_fused_moe_workspace_bytes", T, H, I, E, G, k, bm)
            a2, a2s = off[0], off[1]
            assert a2 % 256 == 0 and a2s % 256 == 0
            assert a2 + T * k * I <= a2s
            assert a2s + T * k * (I // 128) * 4 <= ws
    off = (ctypes.c_int64 * 2)()
    _expect_error("aiter_amd_fused_moe_workspace_a2_offsets", 64, 4096, 2048, 32, 16, 8, 0,
                  ctypes.addressof(off), match="invalid layer dimensions")
    _expect_error("aiter_amd_fused_moe_workspace_a2_offsets", 64, 4096, 2048, 32, 32, 8, 0,
                  None, match="offsets is NULL")


def test_workspace_query_resolves_block_m_like_the_layer(lib):
    """block_m = 0 resolves the same way in the workspace query and the
    one-call entries, from the routed rows per expert over all the router's
    experts: an EP share (32 of 256 experts) at T=64, top-8 averages 2 rows
    per expert and picks 16, where the 32 local experts alone would suggest
    16 rows and 32. The workspace the query reports is accepted by the
    entry: the call gets past the size check to the pointer checks."""
    T, H, I, E, G, k = 64, 4096, 2048, 32, 256, 8
    assert lib.aiter_amd_default_block_m(T, k, E, 0, H, I) == 32
    assert lib.aiter_amd_default_block_m(T, k, E, G, H, I) == 16
    ws = lib.aiter_amd_fused_moe_workspace_bytes(T, H, I, E, G, k, 0)
    assert ws == lib.aiter_amd_fused_moe_workspace_bytes(T, H, I, E, G, k, 16)
    assert ws < lib.aiter_amd_fused_moe_workspace_bytes(T, H, I, E, G, k, 32)
    masked = [16, 3, 16, 16, 16, 16, 16, 16, 16, None, 16, 3]
    # one byte short is rejected, the reported size passes the size check and
    # stops at the (misaligned) workspace pointer
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *masked, T, H, I, E, G, k, 0, 0, 0, 1,
                  16, ws - 1, None, match="workspace of")
    _expect_error("aiter_amd_fused_moe_fp8_blockscale", *masked, T, H, I, E, G, k, 0, 0, 0, 1,
                  8, ws, None, match="workspace is not 16-byte aligned")


def test_block_m_128_needs_32bit_operands(lib, monkeypatch):
    # the 128-row kernels use 32-bit buffer offsets: T*topk*inter >= 2^32 bytes
    # (T = 262144 at topk 8, inter 2048) must not pick or accept them
    assert lib.aiter_amd_default_block_m(262143, 8, 256, 0, 4096, 2048) == 128
    assert lib.aiter_amd_default_block_m(262144, 8, 256, 0, 4096, 2048) == 64
    args = [16, 16, 0, 16, 16, 16, None, 16, 16, 16, 16]
    _expect_error("aiter_amd_moe_stage1_fp8_blockscale", *args, 262144, 4096, 2048, 256, 8, 128,
                  10, 0, 1, None, match="32-bit offsets")
    import importlib

    F = importlib.import_module("aiter_amd.fused_moe")   # the module, not the function
    monkeypatch.setattr(F, "_cu_num", lambda dev: 256)    # the MI355X's CU count, no GPU here
    assert F.select_block_m(8192, 8, 256, 4096, 2048, False, torch.device("cpu")) == 128
    assert F.select_block_m(262144, 8, 256, 4096, 2048, False, torch.device("cpu")) == 64


def test_default_block_m(lib):
    assert lib.aiter_amd_default_block_m(1, 8, 256, 0, 4096, 2048) == 16
    assert lib.aiter_amd_default_block_m(32, 8, 256, 0, 4096, 2048) == 16
    assert lib.aiter_amd_default_block_m(512, 8, 256, 0, 4096, 2048) == 32
    assert lib.aiter_amd_default_block_m(1024, 8, 256, 0, 4096, 2048) == 64
    # 128-row tiles once experts average >= 64 rows and stage 1 is >= 16
    # rounds of 64-row workgroups (pairs * inter_dim >= 2^26)
    assert lib.aiter_amd_default_block_m(2048, 8, 256, 0, 4096, 2048) == 64
    assert lib.aiter_amd_default_block_m(4096, 8, 256, 256, 4096, 2048) == 128
    assert lib.aiter_amd_default_block_m(8192, 8, 256, 0, 4096, 2048) == 128
    # an EP share (32 of 256 experts) holds an eighth of the pairs
    assert lib.aiter_amd_default_block_m(8192, 8, 32, 256, 4096, 2048) == 64
    assert lib.aiter_amd_default_block_m(65536, 8, 32, 256, 4096, 2048) == 128
    # 128-row tiles need model_dim % 256 == 0 and dims <= 8192
    assert lib.aiter_amd_default_block_m(8192, 8, 256, 0, 4224, 2048) == 64
    assert lib.aiter_amd_default_block_m(8192, 8, 256, 0, 0, 0) == 64


def test_python_layer_rejects_unsupported_modes():
    from aiter_amd import ActivationType, QuantType, fused_moe

    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    w1 = torch.zeros(2, 256, 256, dtype=torch.float8_e4m3fn)
    w2 = torch.zeros(2, 256, 128, dtype=torch.float8_e4m3fn)
    ids = torch.zeros(4, 1, dtype=torch.int32)
    tw = torch.ones(4, 1)
    s1 = torch.ones(2, 2, 2)
    s2 = torch.ones(2, 2, 1)
    with pytest.raises(NotImplementedError, match="quant_type"):
        fused_moe(x, w1, w2, tw, ids, quant_type=QuantType.No)
    with pytest.raises(NotImplementedError, match="activation"):
        fused_moe(x, w1, w2, tw, ids, quant_type=QuantType.per_128x128,
                  activation=ActivationType.Swiglu, w1_scale=s1, w2_scale=s2)
    with pytest.raises(NotImplementedError, match="bias"):
        fused_moe(x, w1, w2, tw, ids, quant_type=QuantType.per_128x128, bias1=torch.zeros(2, 256),
                  w1_scale=s1, w2_scale=s2)
    with pytest.raises(ValueError, match="w1_scale"):
        fused_moe(x, w1, w2, tw, ids, quant_type=QuantType.per_128x128)


def test_python_layer_validates_tensors_before_the_c_abi():
    """Every tensor fused_moe hands to the raw-pointer C ABI is checked first
    (dtype, shape, device): a wrong one raises ValueError on the host instead
    of a kernel reading out of bounds. CPU tensors pass every check up to
    the device one, so each case below fails at its own check."""
    from aiter_amd import QuantType, fused_moe

    M, H, I, E, k = 4, 256, 128, 2, 2
    x = torch.zeros(M, H, dtype=torch.bfloat16)
    w1 = torch.zeros(E, 2 * I, H, dtype=torch.float8_e4m3fn)
    w2 = torch.zeros(E, H, I, dtype=torch.float8_e4m3fn)
    ids = torch.zeros(M, k, dtype=torch.int32)
    tw = torch.ones(M, k)
    s1 = torch.ones(E, 2 * I // 128, H // 128)
    s2 = torch.ones(E, H // 128, I // 128)
    qt = QuantType.per_128x128
    run = lambda **kw: fused_moe(**{**dict(hidden_states=x, w1=w1, w2=w2, topk_weight=tw,
                                           topk_ids=ids, quant_type=qt, w1_scale=s1,
                                           w2_scale=s2), **kw})
    with pytest.raises(ValueError, match="runs on the GPU"):
        run()
    with pytest.raises(ValueError, match="static a2_scale"):
        run(a2_scale=torch.ones(M, k, I // 128))
    with pytest.raises(ValueError, match="hidden_states must be"):
        run(hidden_states=torch.zeros(M, H + 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="hidden_states must be"):
        run(hidden_states=torch.zeros(M + 1, H, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="topk_weight must be"):
        run(topk_weight=torch.ones(M, k + 1))
    with pytest.raises(ValueError, match="w1_scale must be the 128x128"):
        run(w1_scale=torch.ones(E, 2 * I // 128, 1))
    with pytest.raises(ValueError, match="w2_scale must be the 128x128"):
        run(w2_scale=torch.ones(E, H // 128, 2))
    x8 = torch.zeros(M, H, dtype=torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="a1_scale must be provided"):
        run(hidden_states=x8)
    with pytest.raises(ValueError, match="a1_scale must be the f32 1x128"):
        run(hidden_states=x8, a1_scale=torch.ones(M, 1))
    with pytest.raises(ValueError, match="expert_mask must be"):
        run(expert_mask=torch.ones(1, dtype=torch.int32))
    with pytest.raises(ValueError, match="num_local_tokens"):
        run(num_local_tokens=torch.ones(1, dtype=torch.int64))
    with pytest.raises(ValueError, match="multiples of 128"):
        run(w1=torch.zeros(E, 2 * 64, H, dtype=torch.float8_e4m3fn),
            w2=torch.zeros(E, H, 64, dtype=torch.float8_e4m3fn))


def test_fused_moe_is_a_registered_custom_op():
    """fused_moe_ is torch.ops.aiter_amd.fused_moe_ with fused_moe_fake as its
    fake (the reference's registration, aiter/fused_moe.py:172-205): under
    FakeTensorMode the op produces the [M, model_dim] output's shape and
    dtype without running anything."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from aiter_amd import QuantType

    op = torch.ops.aiter_amd.fused_moe_.default
    names = [a.name for a in op._schema.arguments]
    assert names[:5] == ["hidden_states", "w1", "w2", "topk_weight", "topk_ids"]
    assert names[-2:] == ["bias1", "bias2"]
    with FakeTensorMode():
        x = torch.empty(6, 256, dtype=torch.float16, device="cuda")
        w1 = torch.empty(2, 256, 256, dtype=torch.float8_e4m3fn, device="cuda")
        w2 = torch.empty(2, 256, 128, dtype=torch.float8_e4m3fn, device="cuda")
        ids = torch.empty(6, 2, dtype=torch.int32, device="cuda")
        tw = torch.empty(6, 2, device="cuda")
        out = torch.ops.aiter_amd.fused_moe_(x, w1, w2, tw, ids, None, 0,
                                             int(QuantType.per_128x128))
        assert out.shape == (6, 256) and out.dtype == torch.float16


def test_enum_values_match_reference():
    from aiter_amd import ActivationType, QuantType

    # csrc/include/aiter_enum.h:7-26
    assert [ActivationType.No, ActivationType.Silu, ActivationType.Gelu,
            ActivationType.Swiglu] == [-1, 0, 1, 2]
    assert QuantType.per_1x128 == 4 and QuantType.per_128x128 == 5 and QuantType.per_1x32 == 3


def test_shuffle_roundtrip_and_layout():
    import numpy as np

    from aiter_amd import shuffle_weight, unshuffle_weight
    from oracle import moe_ref as R

    w = torch.randint(0, 255, (3, 64, 256), dtype=torch.uint8)
    sh = shuffle_weight(w)
    assert sh.is_shuffled
    assert np.array_equal(sh.numpy(), R.shuffle_16x16(w.numpy()))
    assert torch.equal(unshuffle_weight(sh), w)


def test_weight_quant_matches_oracle():
    import numpy as np

    from aiter_amd import quant_weight_per_128x128
    from oracle import moe_ref as R

    w = torch.randn(2, 256, 384) * 0.02
    q, s = quant_weight_per_128x128(w)
    qo, so = R.quant_weight_128x128(w.numpy())
    assert np.array_equal(q.view(torch.uint8).numpy(), qo)
    assert np.array_equal(s.numpy(), so)


def test_torch_mxfp4_quant_matches_oracle():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(3, 64, 256, generator=g) * 0.02
    w[0, 0, :32] = 0.0
    w[1, 2, 64:96] *= 1e4
    w[2, 5, 7] = -0.0
    p, s = A.per_1x32_f4_quant(w)
    assert p.dtype == A.dtypes.fp4x2 and s.dtype == A.dtypes.fp8_e8m0
    rp, rs = R.quant_weight_mxfp4(w.numpy())
    np.testing.assert_array_equal(p.view(torch.uint8).numpy(), rp)
    np.testing.assert_array_equal(s.view(torch.uint8).numpy(), rs)
    e = torch.arange(1, 255, dtype=torch.uint8)
    np.testing.assert_array_equal(A.e8m0_to_f32(e).numpy(), R.e8m0_to_f32(e.numpy()))


def test_a8w4_validation_errors():
    args = [16, 16, 0, 16]
    tail = [16, None, 16, 16, 16, 16, 4, 4096, 2048, 8, 2, 32, 10, 0, 1, None]
    _expect_error("aiter_amd_moe_stage1_a8w4", *args, None, *tail, match="w1_scale is NULL")
    _expect_error("aiter_amd_moe_stage1_a8w4", *args, 18, *tail, match="4-byte aligned")
    _expect_error("aiter_amd_moe_stage2_a8w4", 16, 16, 16, None, 16, 16, 16, 16, 16, 4, 4,
                  4096, 2048, 8, 2, 32, 10, 1, None, match="w2_scale is NULL")
    base = [16, 3, 16, 16, 16, None, 16, 16, None, None, 16, 3]
    _expect_error("aiter_amd_fused_moe_a8w4", *base, 4, 4096, 2048, 8, 8, 2, 0, 0, 0, 1, 16, 10,
                  None, match="w2_scale is NULL")


def test_python_layer_a8w4_checks():
    from aiter_amd import QuantType, fused_moe, fused_moe_a8w4

    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    ids = torch.zeros(4, 1, dtype=torch.int32)
    tw = torch.ones(4, 1)
    w1 = torch.zeros(2, 256, 128, dtype=torch.uint8)    # [E, 2I, H/2]
    w2 = torch.zeros(2, 256, 64, dtype=torch.uint8)     # [E, H, I/2]
    s1 = torch.zeros(2, 256, 8, dtype=torch.uint8)
    s2 = torch.zeros(2, 256, 4, dtype=torch.uint8)
    assert A.get_inter_dim(w1.shape, w2.shape) == (2, 256, 128)
    # the drop-in's per_1x32 is A4W4 in the reference (fp4 activations): refused,
    # the A8W4 layer has its own entry
    with pytest.raises(NotImplementedError, match="A4W4"):
        fused_moe(x, w1, w2, tw, ids, quant_type=QuantType.per_1x32, w1_scale=s1, w2_scale=s2)
    with pytest.raises(ValueError, match="e8m0 scales must be"):
        fused_moe_a8w4(x, w1, w2, tw, ids, w1_scale=s1[..., :4], w2_scale=s2)
    with pytest.raises(ValueError, match="per_1x32 needs packed fp4x2"):
        fused_moe_a8w4(x, w1.view(torch.float8_e4m3fn), w2.view(torch.float8_e4m3fn), tw, ids,
                       w1_scale=s1, w2_scale=s2)
    with pytest.raises(ValueError, match="e8m0"):
        fused_moe_a8w4(x, w1, w2, tw, ids, w1_scale=s1.float(), w2_scale=s2)
    with pytest.raises(ValueError, match="runs on the GPU"):   # checks all pass up to the device
        fused_moe_a8w4(x, w1, w2, tw, ids, w1_scale=s1, w2_scale=s2)


def test_routing_validation_errors(lib):
    # topk_softmax: topk > 32, E > 1024, strides < topk, bad dtype, NULL
    _expect_error("aiter_amd_topk_softmax", 16, 4, 8, 256, 33, 16, 33, 16, 33, None, 1, None,
                  match="topk")
    _expect_error("aiter_amd_topk_softmax", 16, 4, 8, 2048, 8, 16, 8, 16, 8, None, 1, None,
                  match="num_experts <= 1024")
    _expect_error("aiter_amd_topk_softmax", 16, 4, 8, 256, 8, 16, 4, 16, 8, None, 1, None,
                  match="strides")
    _expect_error("aiter_amd_topk_softmax", 16, 0, 8, 256, 8, 16, 8, 16, 8, None, 1, None,
                  match="dtype")
    _expect_error("aiter_amd_topk_sigmoid", None, 4, 8, 256, 8, 16, 8, 16, 8, None,
                  match="NULL")
    # grouped: groups must divide E, topk_group <= groups, topk <= kept experts,
    # biased needs sigmoid scores
    _expect_error("aiter_amd_grouped_topk", 16, 4, None, 8, 256, 8, 7, 4, 1, 1, 1.0, 16, 8, 16,
                  8, None, match="divide")
    _expect_error("aiter_amd_grouped_topk", 16, 4, None, 8, 256, 8, 8, 9, 1, 1, 1.0, 16, 8, 16,
                  8, None, match="topk_group")
    _expect_error("aiter_amd_grouped_topk", 16, 4, None, 8, 256, 9, 32, 1, 1, 1, 1.0, 16, 9, 16,
                  9, None, match="kept groups")
    _expect_error("aiter_amd_grouped_topk", 16, 4, 16, 8, 256, 8, 8, 4, 1, 1, 1.0, 16, 8, 16, 8,
                  None, match="sigmoid")
    # zero tokens is a no-op
    _abi.call("aiter_amd_topk_softmax", None, 4, 0, 256, 8, None, 8, None, 8, None, 1, None)


def test_e8m0_shuffle_layout_and_loader():
    """e8m0_shuffle is the reference's index permutation (pinned by the
    oracle's index formula); fused_moe's loader turns it back into the
    kernels' row-major [E, N, K/32] and caches the result on the tensor."""
    from aiter_amd.fused_moe import e8m0_rowmajor
    rng = np.random.default_rng(5)
    for m, n in [(300, 13), (512, 64), (1024, 128)]:
        x = rng.integers(0, 255, (m, n)).astype(np.uint8)
        ref, filled = R.e8m0_shuffle_ref(x)
        got = A.e8m0_shuffle(torch.from_numpy(x)).numpy()
        assert got.shape == ref.shape and np.array_equal(got[filled], ref[filled])
        assert np.array_equal(A.e8m0_unshuffle(torch.from_numpy(got), m, n).numpy(), x)
    # per_1x32_f4_quant(shuffle=True) == e8m0_shuffle of the 2-D scales
    w = torch.randn(4, 64, 256) * 0.05
    p, s3 = A.per_1x32_f4_quant(w)
    p2, s2 = A.per_1x32_f4_quant(w, shuffle=True)
    assert torch.equal(p.view(torch.uint8), p2.view(torch.uint8))
    assert torch.equal(s2.view(torch.uint8), A.e8m0_shuffle(s3.view(torch.uint8).reshape(-1, 8)))
    rm = e8m0_rowmajor(s2, 4, 64, 8)
    assert torch.equal(rm.view(torch.uint8), s3.view(torch.uint8))
    assert e8m0_rowmajor(s2, 4, 64, 8) is rm               # cached
    s2.view(torch.uint8)[0, 0] ^= 1                        # an in-place update converts again
    assert e8m0_rowmajor(s2, 4, 64, 8) is not rm
    assert e8m0_rowmajor(s3, 4, 64, 8) is s3                # 3-D scales pass through
    with pytest.raises(ValueError, match="e8m0_shuffle scales must be"):
        e8m0_rowmajor(torch.zeros(100, 8, dtype=torch.uint8), 4, 64, 8)


@pytest.mark.parametrize("nlane", [16, 32])
@pytest.mark.parametrize("gate_up", [True, False])
def test_a16w4_layouts_convert_to_row_major(nlane, gate_up):
    """The reference's a16w4 weight and scale layouts (its Swiglu fp4 kernels'
    inputs): the view/permute implementation matches the oracle's explicit
    index formula, the unshuffle functions invert it, and an A8W4 checkpoint
    packed that way comes back as the row-major weights and [E, N, K/32]
    scales fused_moe reads."""
    rng = np.random.default_rng(nlane + gate_up)
    E, N, K = 3, 128, 512
    w = rng.integers(0, 256, (E, N, K // 2)).astype(np.uint8)
    s = rng.integers(100, 140, (E * N, K // 32)).astype(np.uint8)
    wt, st = torch.from_numpy(w), torch.from_numpy(s)
    ws = A.shuffle_weight_a16w4(wt, nlane, gate_up)
    ss = A.shuffle_scale_a16w4(st, E, gate_up)
    assert np.array_equal(ws.numpy(), R.a16w4_weight_ref(w, nlane, gate_up))
    assert np.array_equal(ss.numpy(), R.a16w4_scale_ref(s, E, gate_up))
    assert not np.array_equal(ws.numpy(), w) and not np.array_equal(ss.numpy(), s)
    assert torch.equal(A.unshuffle_weight_a16w4(ws, nlane, gate_up), wt)
    assert torch.equal(A.unshuffle_scale_a16w4(ss, E, gate_up), st)
    # typed tensors keep their dtype
    wf = wt.view(torch.float8_e4m3fn)
    assert A.shuffle_weight_a16w4(wf, nlane, gate_up).dtype == torch.float8_e4m3fn
    with pytest.raises(ValueError, match="does not tile"):
        A.shuffle_weight_a16w4(wt[:, :, :100], nlane, gate_up)
    with pytest.raises(ValueError, match="N % 32"):
        A.shuffle_scale_a16w4(st[: E * 16], E, gate_up)


def test_tuned_dispatch_table():
    """The committed block_m table (aiter_amd/tune.py) answers for the MiMo
    shapes it was swept on and buckets token counts like get_padded_M."""
    from aiter_amd import tune as T
    assert [T.padded_tokens(m) for m in (1, 3, 32, 33, 40000)] == [1, 4, 32, 64, 32768]
    bm = {t: T.tuned_block_m(256, t, 4096, 2048, 256, 8, "per_1x128", "fp8")
          for t in (1, 32, 8192)}
    assert all(b in (16, 32, 64, 128) for b in bm.values()), bm
    assert T.tuned_block_m(256, 20, 4096, 2048, 256, 8, "per_1x128", "fp8") == \
        T.tuned_block_m(256, 32, 4096, 2048, 256, 8, "per_1x128", "fp8")
    assert T.tuned_block_m(256, 32, 4096, 2048, 256, 8, "per_1x32", "fp4x2") in (16, 32, 64, 128)
    assert T.tuned_block_m(304, 32, 4096, 2048, 256, 8, "per_1x128", "fp8") is None
    assert T.tuned_block_m(256, 32, 1024, 512, 8, 2, "per_1x128", "fp8") is None


def test_no_alloc_rejects_layers_over_the_buffer():
    """The size check comes before any device work: placeholder pointers are
    never dereferenced."""
    from aiter_amd import workloads as W
    from aiter_amd.enums import AITER_DTYPE

    cfg = W.mimo_prefill(2048)
    need = _abi.query("aiter_amd_fused_moe_workspace_bytes", cfg.tokens, cfg.model_dim,
                      cfg.inter_dim, cfg.experts, cfg.experts, cfg.topk, 128)
    assert need > 32 << 20
    lib = _abi.load()
    p = 256
    rc = lib.aiter_amd_fused_moe_fp8_blockscale_noalloc(
        p, AITER_DTYPE[torch.bfloat16], p, p, p, p, p, p, None, None, p,
        AITER_DTYPE[torch.bfloat16], cfg.tokens, cfg.model_dim, cfg.inter_dim, cfg.experts,
        cfg.experts, cfg.topk, 128, 0, 0, 1, ctypes.c_void_p(0))
    assert rc == -1
    msg = lib.aiter_amd_get_last_error().decode()
    lib.aiter_amd_clear_last_error()
    assert "bytes of workspace" in msg, msg


def test_tuned_table_run_1stage(tmp_path, monkeypatch):
    """The tuned table's run_1stage column picks the one-launch layer per shape
    (the reference's cfg["run_1stage"], aiter/fused_moe.py:903-911);
    AITER_AMD_FUSED overrides it; rows without the column, shapes without a
    row, block sizes the one-launch kernel does not run and block sizes other
    than the row's keep two launches."""
    import importlib

    from aiter_amd import tune

    F = importlib.import_module("aiter_amd.fused_moe")   # the module, not the function

    table = tmp_path / "t.csv"
    table.write_text(
        "cu_num,token,model_dim,inter_dim,expert,topk,act_type,q_type,q_dtype_w,block_m,"
        "run_1stage,us\n"
        "256,2,4096,2048,256,8,Silu,per_1x128,fp8,16,1,76.0\n"
        "256,4,4096,2048,256,8,Silu,per_1x128,fp8,16,0,133.0\n")
    monkeypatch.setenv("AITER_AMD_TUNED_FMOE", str(table))
    monkeypatch.delenv("AITER_AMD_FUSED", raising=False)
    monkeypatch.setattr(F, "_cu_num", lambda dev: 256)
    tune.clear_cache()
    try:
        args = (4096, 2048, False, 16, torch.device("cpu"))
        assert F.select_run_1stage(2, 8, 256, *args)
        assert not F.select_run_1stage(4, 8, 256, *args)
        assert not F.select_run_1stage(8, 8, 256, *args)                 # no row
        assert not F.select_run_1stage(2, 8, 256, 4096, 2048, False, 64, torch.device("cpu"))
        # the row's run_1stage was measured at its own block_m (16): a caller's
        # block_size_M of 32 keeps two launches
        assert not F.select_run_1stage(2, 8, 256, 4096, 2048, False, 32, torch.device("cpu"))
        assert tune.tuned_block_m(256, 2, 4096, 2048, 256, 8, "per_1x128", "fp8") == 16
        monkeypatch.setenv("AITER_AMD_FUSED", "0")
        assert not F.select_run_1stage(2, 8, 256, *args)
        monkeypatch.setenv("AITER_AMD_FUSED", "1")
        assert F.select_run_1stage(8, 8, 256, *args)
    finally:
        tune.clear_cache()
