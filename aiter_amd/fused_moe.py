"""Drop-in `fused_moe` / `moe_sorting` for the FP8 block-scale MoE path.

Keeps the reference's Python surface (aiter/fused_moe.py:70-169 fused_moe
and moe_sorting, 172-364 fused_moe_fake / fused_moe_) and runs the gfx950
HIP kernels of libaiter_amd.so through the C ABI:

  sorting (+ clearing the f32 accumulator) -> 1x128 fp8 quant of the
  activations -> stage-1 gather-GEMM with fused SiLU*up and fp8 requant ->
  stage-2 down-GEMM with top-k weighted accumulate -> f32 -> bf16/fp16.

Supported: quant_type per_128x128 / per_1x128 with fp8 e4m3fn weights and
fp32 block scales (or per_1x32 with MXFP4 weights), activation Silu or Gelu, g1u1
(w1 holds gate and up), bf16/fp16 activations (or fp8 activations with
a1_scale), expert_mask (EP share), num_local_tokens, doweight_stage1.
Anything else raises NotImplementedError; there is no fallback path.
"""
from __future__ import annotations

import functools
import os
from typing import Optional

import torch

from . import _abi, ffi
from .enums import AITER_DTYPE, ActivationType, QuantType, dtypes, quant_remap
from .quant import e8m0_unshuffle, per_group_quant_hip
from .topk import fused_topk  # noqa: F401  (aiter.fused_moe.fused_topk)
from .tune import tuned_block_m, tuned_config

BLOCK_SIZE_M = 32


# torch's current stream as a raw hipStream_t without building a Stream
# object (a few microseconds of host time per layer call at decode sizes)
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(dev: torch.device) -> int:
    if _RAW_STREAM is not None and dev.index is not None:
        return _RAW_STREAM(dev.index)
    return torch.cuda.current_stream(dev).cuda_stream


def _layer_workspace_bytes(M: int, model_dim: int, inter_dim: int, E: int, global_E: int,
                           topk: int, block_m: int) -> int:
    # AITER_AMD_ST_KSPLIT1 (the stage-1 K-split override) sizes the split's
    # partial sums and AITER_AMD_SORT_CT (the sorting chunk override) the
    # sorting's chunk counts, so their values are part of the cached query's key
    return _workspace_query(M, model_dim, inter_dim, E, global_E, topk, block_m,
                            os.environ.get("AITER_AMD_ST_KSPLIT1"),
                            os.environ.get("AITER_AMD_SORT_CT"))


@functools.lru_cache(maxsize=1024)
def _workspace_query(M, model_dim, inter_dim, E, global_E, topk, block_m, ksplit_env, ct_env):
    return _abi.query("aiter_amd_fused_moe_workspace_bytes", M, model_dim, inter_dim, E,
                      global_E, topk, block_m)


@functools.lru_cache(maxsize=16)
def _cu_num(dev: torch.device) -> int:
    return torch.cuda.get_device_properties(dev).multi_processor_count


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def sorted_capacity(tokens: int, topk: int, num_experts: int, block_size: int) -> int:
    """max_num_tokens_padded of the reference (aiter/fused_moe.py:41)."""
    return int(tokens * topk + num_experts * block_size - topk)


def moe_sorting(
    topk_ids: torch.Tensor,
    topk_weights: torch.Tensor,
    num_experts: int,
    model_dim: int,
    moebuf_dtype: torch.dtype,
    block_size: int = BLOCK_SIZE_M,
    expert_mask: Optional[torch.Tensor] = None,
    num_local_tokens: Optional[torch.Tensor] = None,
    dispatch_policy: int = 0,
):
    """Returns (sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids,
    moe_buf) exactly like aiter.fused_moe.moe_sorting (fused_moe.py:27-103);
    moe_buf [M, model_dim] is zeroed for the local token rows."""
    device = topk_ids.device
    M, topk = topk_ids.shape
    if topk_ids.dtype != torch.int32 or topk_weights.dtype != torch.float32:
        raise ValueError("topk_ids must be int32 and topk_weights float32")
    topk_ids = topk_ids.contiguous()
    topk_weights = topk_weights.contiguous()
    cap = sorted_capacity(M, topk, num_experts, block_size)
    nblocks = (cap + block_size - 1) // block_size
    sorted_ids = torch.empty(cap, dtype=dtypes.i32, device=device)
    sorted_weights = torch.empty(cap, dtype=dtypes.fp32, device=device)
    sorted_expert_ids = torch.empty(nblocks, dtype=dtypes.i32, device=device)
    num_valid_ids = torch.empty(2, dtype=dtypes.i32, device=device)
    moe_buf = torch.empty((M, model_dim), dtype=moebuf_dtype, device=device)
    if expert_mask is not None:
        expert_mask = expert_mask.to(torch.int32).contiguous()
        if expert_mask.numel() != num_experts:
            raise ValueError("expert_mask must have num_experts entries")
    row_bytes = model_dim * moe_buf.element_size()
    ws_bytes = _abi.query("aiter_amd_moe_sorting_workspace_bytes", M, topk, num_experts)
    if row_bytes % 16 == 0 and ws_bytes <= M * row_bytes:
        # the reference-shaped entry (include/aiter_ctypes.h); with more than one
        # chunk of tokens it keeps its counts in moe_buf and clears them after
        ffi.moe_sorting_fwd(topk_ids, topk_weights, sorted_ids, sorted_weights,
                            sorted_expert_ids, num_valid_ids, moe_buf, num_experts,
                            int(block_size), expert_mask, num_local_tokens, int(dispatch_policy))
    else:
        # a moe_buf too small for the chunk counts (thousands of experts, narrow
        # rows), or rows the 16-byte clearing stores cannot cover: the counts go
        # to a workspace of their own, and moe_buf is cleared by the sorting
        # launch or, for such rows, here
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
        clear = row_bytes % 16 == 0
        _abi.call(
            "aiter_amd_moe_sorting_fwd",
            topk_ids.data_ptr(), topk_weights.data_ptr(), M, topk, sorted_ids.data_ptr(),
            sorted_weights.data_ptr(), sorted_expert_ids.data_ptr(), num_valid_ids.data_ptr(),
            cap, nblocks, moe_buf.data_ptr() if clear else None, row_bytes, num_experts,
            int(block_size), _ptr(expert_mask), _ptr(num_local_tokens), int(dispatch_policy),
            _ptr(ws), ws_bytes, _stream(device))
        if not clear:
            moe_buf.zero_()
    return sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf


@functools.lru_cache(maxsize=2048)
def get_inter_dim(w1_shape, w2_shape):
    """(E, model_dim, inter_dim) from the weight shapes (fused_moe.py:108-115);
    packed fp4 weights hold two K values per byte, which the model_dim /
    w1.shape[-1] factor undoes."""
    E, _, model_dim = w1_shape
    E, model_dim, inter_dim = w2_shape
    inter_dim *= model_dim // w1_shape[-1]
    return E, model_dim, inter_dim


def default_block_m(tokens: int, topk: int, num_experts: int, model_dim: int = 0,
                    inter_dim: int = 0, global_experts: int = 0) -> int:
    """M-block for a layer; model_dim/inter_dim 0 rule out 128-row tiles.
    global_experts: the expert_mask size of an expert-parallel share (0: num_experts)."""
    return _abi.query("aiter_amd_default_block_m", tokens, topk, num_experts, global_experts,
                      model_dim, inter_dim)


def fused_moe(
    hidden_states,
    w1,  # [E, inter_dim*2, dim] fp8 (optionally shuffled (16,16))
    w2,  # [E, dim, inter_dim] fp8
    topk_weight,
    topk_ids,
    expert_mask: Optional[torch.Tensor] = None,
    activation=ActivationType.Silu,
    quant_type=QuantType.No,
    doweight_stage1=False,
    w1_scale: Optional[torch.Tensor] = None,  # [E, 2*inter_dim/128, dim/128]
    w2_scale: Optional[torch.Tensor] = None,  # [E, dim/128, inter_dim/128]
    a1_scale: Optional[torch.Tensor] = None,
    a2_scale: Optional[torch.Tensor] = None,
    block_size_M=None,
    num_local_tokens: Optional[torch.Tensor] = None,
    moe_sorting_dispatch_policy=0,
    dtype=None,
    hidden_pad=0,
    intermediate_pad=0,
    bias1=None,
    bias2=None,
    splitk=0,
):
    """Same signature and result as aiter.fused_moe.fused_moe (fused_moe.py:118-169);
    runs the registered custom op torch.ops.aiter_amd.fused_moe_ as the reference
    runs torch.ops.aiter.fused_moe_ (fused_moe.py:172-205)."""
    return torch.ops.aiter_amd.fused_moe_(
        hidden_states, w1, w2, topk_weight, topk_ids, expert_mask, int(activation),
        int(quant_type), bool(doweight_stage1), w1_scale, w2_scale, a1_scale, a2_scale,
        int(block_size_M) if block_size_M else -1, num_local_tokens,
        int(moe_sorting_dispatch_policy), dtype, int(hidden_pad), int(intermediate_pad), bias1,
        bias2)


def fused_moe_a8w4(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,  # [E, inter_dim*2, dim/2] packed e2m1 (fp4x2 or uint8)
    w2: torch.Tensor,  # [E, dim, inter_dim/2]
    topk_weight: torch.Tensor,
    topk_ids: torch.Tensor,
    expert_mask: Optional[torch.Tensor] = None,
    activation=ActivationType.Silu,
    doweight_stage1: bool = False,
    w1_scale: Optional[torch.Tensor] = None,  # e8m0 [E, 2*inter_dim, dim/32] or e8m0_shuffle
    w2_scale: Optional[torch.Tensor] = None,  # e8m0 [E, dim, inter_dim/32] or e8m0_shuffle
    a1_scale: Optional[torch.Tensor] = None,
    block_size_M=None,
    num_local_tokens: Optional[torch.Tensor] = None,
    dtype=None,
):
    """The A8W4 layer: fp8 e4m3 activations with 1x128 fp32 scales (quantised here
    from bf16/fp16 hidden_states, or given as fp8 with a1_scale) x MXFP4 weights
    (e2m1 with e8m0 1x32 scales, as per_1x32_f4_quant makes them).

    This is an explicit entry of its own: in the reference, fused_moe with
    quant_type=per_1x32 and Silu/Gelu quantises the activations to fp4 (A4W4,
    aiter/fused_moe.py:267-274), which is not provided here, so fused_moe raises
    for it instead of silently computing this layer."""
    return _fused_moe_impl(
        hidden_states, w1, w2, topk_weight, topk_ids, expert_mask, int(activation),
        int(QuantType.per_1x32), bool(doweight_stage1), w1_scale, w2_scale, a1_scale, None,
        int(block_size_M) if block_size_M else -1, num_local_tokens, 0, dtype, 0, 0, None, None,
        a8w4=True)


def fused_moe_fake(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                   topk_weight: torch.Tensor, topk_ids: torch.Tensor,
                   expert_mask: Optional[torch.Tensor] = None, activation: int = 0,
                   quant_type: int = 0, doweight_stage1: bool = False,
                   w1_scale: Optional[torch.Tensor] = None,
                   w2_scale: Optional[torch.Tensor] = None,
                   a1_scale: Optional[torch.Tensor] = None,
                   a2_scale: Optional[torch.Tensor] = None, block_size_M: int = -1,
                   num_local_tokens: Optional[torch.Tensor] = None,
                   moe_sorting_dispatch_policy: int = 0, dtype: Optional[torch.dtype] = None,
                   hidden_pad: int = 0, intermediate_pad: int = 0,
                   bias1: Optional[torch.Tensor] = None,
                   bias2: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Shape-only twin for tracing (fused_moe.py:172-202)."""
    M, _ = topk_ids.shape
    out_dtype = _out_dtype(hidden_states, dtype)
    return torch.empty((M, w2.shape[1]), dtype=out_dtype, device=topk_ids.device)


def _out_dtype(hidden_states, dtype):
    if dtype is not None:
        return dtype
    return hidden_states.dtype if hidden_states.dtype in (dtypes.bf16, dtypes.fp16) else dtypes.bf16


_FP4_DTYPES = (torch.uint8, dtypes.fp4x2)
_E8M0_DTYPES = (torch.uint8, dtypes.fp8_e8m0)


def select_block_m(tokens: int, topk: int, num_experts: int, model_dim: int, inter_dim: int,
                   a8w4: bool, device: torch.device, global_experts: int = 0) -> int:
    """fused_moe's block_m when the caller gives none: the tuned table
    (aiter_amd/tune.py, the get_2stage_cfgs lookup of aiter/fused_moe.py:719-1100),
    else the heuristic default_block_m (global_experts: the expert_mask size of
    an expert-parallel share)."""
    tuned = tuned_block_m(_cu_num(device), tokens, model_dim, inter_dim, num_experts, topk,
                          "per_1x32" if a8w4 else "per_1x128", "fp4x2" if a8w4 else "fp8")
    bm = tuned or default_block_m(tokens, topk, num_experts, model_dim, inter_dim, global_experts)
    # the 128-row kernels address their activation operand with 32-bit offsets
    if bm == 128 and max(tokens * model_dim, tokens * topk * inter_dim) >= 1 << 32:
        bm = 64
    return bm


def select_run_1stage(tokens: int, topk: int, num_experts: int, model_dim: int,
                      inter_dim: int, a8w4: bool, block_m: int, device: torch.device) -> bool:
    """Whether fused_moe runs the one-launch layer (both GEMMs in one kernel,
    the role of the reference's fused_moe_1stage): AITER_AMD_FUSED=0/1 when
    set, else the tuned table's run_1stage for this shape (the reference's
    cfg["run_1stage"], aiter/fused_moe.py:903-911). The one-launch kernel
    runs 16/32-row M-blocks with model_dim a multiple of 256 up to 8192.
    The table's run_1stage was measured at the row's own block_m, so it is
    honoured only when the layer runs at that block_m (a caller's
    block_size_M may differ)."""
    if block_m not in (16, 32) or model_dim % 256 or model_dim > 8192:
        return False
    env = os.environ.get("AITER_AMD_FUSED")
    if env is not None:
        return int(env) != 0
    cfg = tuned_config(_cu_num(device), tokens, model_dim, inter_dim, num_experts, topk,
                       "per_1x32" if a8w4 else "per_1x128", "fp4x2" if a8w4 else "fp8")
    return bool(cfg and cfg[1] and cfg[0] == block_m)


def e8m0_rowmajor(scale: torch.Tensor, E: int, N: int, KS: int) -> torch.Tensor:
    """The kernels' MXFP4 scale layout, row-major e8m0 bytes [E, N, KS], from
    either form a caller may hold:
    * [E, N, KS] (per_1x32_f4_quant of [E, N, K]) is used as it is;
    * a 2-D [ceil(E*N/256)*256, ceil(KS/8)*8] array is the reference's
      e8m0_shuffle layout, the form its fused kernels take
      (op_tests/test_moe_2stage.py:166-184, aiter/utility/fp4_utils.py:72-92).
      It is un-shuffled once and the result cached on the tensor, keyed by
      the tensor's version counter (an in-place update converts again)."""
    if scale.dim() == 3:
        if tuple(scale.shape) != (E, N, KS):
            raise ValueError(f"e8m0 scales must be {(E, N, KS)}, got {tuple(scale.shape)}")
        return scale
    if scale.dim() != 2:
        raise ValueError(f"e8m0 scales must be 3-D [E, N, K/32] or the 2-D e8m0_shuffle layout, "
                         f"got {tuple(scale.shape)}")
    shp = ((E * N + 255) // 256 * 256, (KS + 7) // 8 * 8)
    if tuple(scale.shape) != shp:
        raise ValueError(f"e8m0_shuffle scales must be {shp}, got {tuple(scale.shape)}")
    cached = getattr(scale, "_aiter_amd_rowmajor", None)
    if cached is not None and cached[0] == scale._version:
        return cached[1]
    rm = e8m0_unshuffle(scale.view(torch.uint8), E * N, KS).view(E, N, KS)
    scale._aiter_amd_rowmajor = (scale._version, rm)
    return rm


def _shape_str(t):
    return "None" if t is None else str(tuple(t.shape))


def _check_supported(hidden_states, w1, w2, topk_weight, topk_ids, expert_mask, activation,
                     quant_type, w1_scale, w2_scale, a1_scale, a2_scale, num_local_tokens,
                     hidden_pad, intermediate_pad, bias1, bias2, out_dtype, a8w4):
    """Everything fused_moe_ checks before a tensor reaches the C ABI, which
    takes raw pointers: unsupported modes raise NotImplementedError, tensors
    of the wrong dtype, shape or device raise ValueError."""
    if quant_type == QuantType.per_1x32 and not a8w4:
        raise NotImplementedError(
            "quant_type per_1x32 with Silu/Gelu: the reference quantises the activations to "
            "fp4 (A4W4, aiter/fused_moe.py:267-274), which is not implemented; for fp8 "
            "activations x MXFP4 weights call aiter_amd.fused_moe_a8w4")
    if quant_type not in (QuantType.per_1x128, QuantType.per_1x32):
        raise NotImplementedError(
            f"quant_type {quant_type!r}: only per_128x128 / per_1x128 fp8 blockscale "
            "(and fused_moe_a8w4) are implemented")
    if activation not in (ActivationType.Silu, ActivationType.Gelu):
        raise NotImplementedError(f"activation {activation!r}: only Silu and Gelu are implemented")
    if hidden_pad or intermediate_pad or bias1 is not None or bias2 is not None:
        raise NotImplementedError("hidden_pad / intermediate_pad / bias are not implemented")
    if a2_scale is not None:
        # the reference's per_1x128 requant raises for a static scale
        # (per_group_quant_hip, aiter/ops/quant.py:272-276)
        raise ValueError("unsupported: static a2_scale (the stage-1 output is quantised "
                         "dynamically, 1x128)")
    if w1_scale is None or w2_scale is None:
        raise ValueError("w1_scale and w2_scale are required")
    if topk_ids.dim() != 2:
        raise ValueError(f"topk_ids must be [M, topk], got {_shape_str(topk_ids)}")
    M, topk = topk_ids.shape
    E, model_dim, inter_dim = get_inter_dim(tuple(w1.shape), tuple(w2.shape))
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"topk_ids must be int32, got {topk_ids.dtype}")
    if tuple(topk_weight.shape) != (M, topk) or not topk_weight.is_floating_point():
        raise ValueError(f"topk_weight must be a float [M, topk] = {(M, topk)} tensor, got "
                         f"{topk_weight.dtype} {_shape_str(topk_weight)}")
    if hidden_states.dim() != 2 or tuple(hidden_states.shape) != (M, model_dim):
        raise ValueError(f"hidden_states must be [M, model_dim] = {(M, model_dim)}, got "
                         f"{_shape_str(hidden_states)}")
    if a8w4:
        if w1.dtype not in _FP4_DTYPES or w2.dtype not in _FP4_DTYPES:
            raise ValueError(f"per_1x32 needs packed fp4x2 (or uint8) w1/w2, got "
                             f"{w1.dtype}/{w2.dtype}")
        if w1_scale.dtype not in _E8M0_DTYPES or w2_scale.dtype not in _E8M0_DTYPES:
            raise ValueError("per_1x32 w1_scale / w2_scale must be e8m0 (or uint8)")
        if tuple(w1.shape) != (E, 2 * inter_dim, model_dim // 2):
            raise ValueError(f"w1 must be [E, 2*inter_dim, model_dim/2], got {_shape_str(w1)}")
    else:
        if w1.dtype != dtypes.fp8 or w2.dtype != dtypes.fp8:
            raise ValueError(f"w1/w2 must be {dtypes.fp8}, got {w1.dtype}/{w2.dtype}")
        if w1_scale.dtype != dtypes.fp32 or w2_scale.dtype != dtypes.fp32:
            raise ValueError("w1_scale / w2_scale must be float32")
        if model_dim % 128 or inter_dim % 128:
            raise ValueError(f"model_dim {model_dim} and inter_dim {inter_dim} must be "
                             "multiples of 128")
        for name, t, want in (("w1_scale", w1_scale, (E, 2 * inter_dim // 128, model_dim // 128)),
                              ("w2_scale", w2_scale, (E, model_dim // 128, inter_dim // 128))):
            if tuple(t.shape) != want:
                raise ValueError(f"{name} must be the 128x128 block scales {want}, got "
                                 f"{_shape_str(t)}")
    if out_dtype not in (dtypes.bf16, dtypes.fp16):
        raise ValueError(f"Fused_moe unsupported out dtype: {out_dtype}")
    if hidden_states.dtype not in (dtypes.bf16, dtypes.fp16, dtypes.fp8):
        raise ValueError(f"unsupported hidden_states dtype {hidden_states.dtype}")
    if hidden_states.dtype == dtypes.fp8:
        if a1_scale is None:
            raise ValueError("a1_scale must be provided for fp8 hidden_states")
        if a1_scale.dtype != dtypes.fp32 or tuple(a1_scale.shape) != (M, model_dim // 128):
            raise ValueError(f"a1_scale must be the f32 1x128 scales {(M, model_dim // 128)}, "
                             f"got {a1_scale.dtype} {_shape_str(a1_scale)}")
    if expert_mask is not None and (expert_mask.dim() != 1 or expert_mask.numel() < E):
        raise ValueError(f"expert_mask must be [global_experts >= {E}], got "
                         f"{_shape_str(expert_mask)}")
    if num_local_tokens is not None and (num_local_tokens.numel() < 1 or
                                         num_local_tokens.dtype != torch.int32):
        raise ValueError("num_local_tokens must be an int32 tensor of one element")


def _check_devices(hidden_states, w1, w2, topk_weight, topk_ids, w1_scale, w2_scale, a1_scale,
                   expert_mask, num_local_tokens):
    """The C ABI takes device pointers: every tensor must live on topk_ids' GPU."""
    dev = topk_ids.device
    if dev.type != "cuda":
        raise ValueError(f"fused_moe runs on the GPU: topk_ids is on {dev}")
    named = (("hidden_states", hidden_states), ("w1", w1), ("w2", w2),
             ("topk_weight", topk_weight), ("w1_scale", w1_scale), ("w2_scale", w2_scale),
             ("a1_scale", a1_scale), ("expert_mask", expert_mask),
             ("num_local_tokens", num_local_tokens))
    for name, t in named:
        if t is not None and t.device != dev:
            raise ValueError(f"{name} is on {t.device}, topk_ids on {dev}")


def fused_moe_(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
               topk_weight: torch.Tensor, topk_ids: torch.Tensor,
               expert_mask: Optional[torch.Tensor] = None,
               activation: int = ActivationType.Silu.value,
               quant_type: int = QuantType.No.value, doweight_stage1: bool = False,
               w1_scale: Optional[torch.Tensor] = None, w2_scale: Optional[torch.Tensor] = None,
               a1_scale: Optional[torch.Tensor] = None, a2_scale: Optional[torch.Tensor] = None,
               block_size_M: int = -1, num_local_tokens: Optional[torch.Tensor] = None,
               moe_sorting_dispatch_policy: int = 0, dtype: Optional[torch.dtype] = None,
               hidden_pad: int = 0, intermediate_pad: int = 0,
               bias1: Optional[torch.Tensor] = None,
               bias2: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Body of the drop-in (fused_moe.py:205-364) for the fp8 blockscale path;
    registered as the custom op torch.ops.aiter_amd.fused_moe_ (with
    fused_moe_fake) like the reference's torch_compile_guard registration
    (aiter/jit/utils/torch_guard.py:192-349)."""
    return _fused_moe_impl(hidden_states, w1, w2, topk_weight, topk_ids, expert_mask,
                           activation, quant_type, doweight_stage1, w1_scale, w2_scale, a1_scale,
                           a2_scale, block_size_M, num_local_tokens, moe_sorting_dispatch_policy,
                           dtype, hidden_pad, intermediate_pad, bias1, bias2, a8w4=False)


def _fused_moe_impl(hidden_states, w1, w2, topk_weight, topk_ids, expert_mask, activation,
                    quant_type, doweight_stage1, w1_scale, w2_scale, a1_scale, a2_scale,
                    block_size_M, num_local_tokens, moe_sorting_dispatch_policy, dtype,
                    hidden_pad, intermediate_pad, bias1, bias2, a8w4):
    activation = ActivationType(activation)
    quant_type = quant_remap.get(QuantType(quant_type), QuantType(quant_type))
    M, topk = topk_ids.shape
    E, model_dim, inter_dim = get_inter_dim(tuple(w1.shape), tuple(w2.shape))
    if w1.shape[1] != 2 * inter_dim:
        raise NotImplementedError(f"only g1u1 weights are supported: {w1.shape=} {w2.shape=}")
    out_dtype = _out_dtype(hidden_states, dtype)
    _check_supported(hidden_states, w1, w2, topk_weight, topk_ids, expert_mask, activation,
                     quant_type, w1_scale, w2_scale, a1_scale, a2_scale, num_local_tokens,
                     hidden_pad, intermediate_pad, bias1, bias2, out_dtype, a8w4)
    if a8w4:
        w1_scale = e8m0_rowmajor(w1_scale, E, 2 * inter_dim, model_dim // 32)
        w2_scale = e8m0_rowmajor(w2_scale, E, model_dim, inter_dim // 32)
    _check_devices(hidden_states, w1, w2, topk_weight, topk_ids, w1_scale, w2_scale, a1_scale,
                   expert_mask, num_local_tokens)
    shuffled = bool(getattr(w1, "is_shuffled", False))
    if bool(getattr(w2, "is_shuffled", False)) != shuffled:
        raise ValueError("w1 and w2 must both be shuffled or both be plain")
    global_E = expert_mask.numel() if expert_mask is not None else E
    if block_size_M not in (None, -1):
        block_m = int(block_size_M)
    else:
        block_m = select_block_m(M, topk, E, model_dim, inter_dim, a8w4, topk_ids.device,
                                 global_E)
    device = topk_ids.device
    topk_ids = topk_ids.to(torch.int32).contiguous()
    topk_weight = topk_weight.to(torch.float32).contiguous()
    w1c, w2c = w1.contiguous(), w2.contiguous()
    w1s, w2s = w1_scale.contiguous(), w2_scale.contiguous()
    if a8w4:   # byte views; the kernels read packed e2m1 and e8m0 bytes
        w1c, w2c = w1c.view(torch.uint8), w2c.view(torch.uint8)
        w1s, w2s = w1s.view(torch.uint8), w2s.view(torch.uint8)
    mask = expert_mask.to(torch.int32).contiguous() if expert_mask is not None else None
    out = torch.empty((M, model_dim), dtype=out_dtype, device=device)
    if M == 0:
        return out
    stream = _stream(device)

    if hidden_states.dtype != dtypes.fp8:
        # one C-ABI call runs the whole layer
        x = hidden_states.contiguous()
        ws_bytes = _layer_workspace_bytes(M, model_dim, inter_dim, E, global_E, topk, block_m)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
        one = select_run_1stage(M, topk, E, model_dim, inter_dim, a8w4, block_m, device)
        _abi.call(
            ("aiter_amd_fused_moe_1stage_a8w4" if one else "aiter_amd_fused_moe_a8w4") if a8w4
            else ("aiter_amd_fused_moe_1stage_fp8_blockscale" if one
                  else "aiter_amd_fused_moe_fp8_blockscale"),
            x.data_ptr(), AITER_DTYPE[x.dtype], w1c.data_ptr(), w1s.data_ptr(), w2c.data_ptr(),
            w2s.data_ptr(), topk_weight.data_ptr(), topk_ids.data_ptr(), _ptr(mask),
            _ptr(num_local_tokens), out.data_ptr(), AITER_DTYPE[out_dtype], M, model_dim,
            inter_dim, E, global_E, topk, block_m, int(activation), int(bool(doweight_stage1)),
            int(shuffled), ws.data_ptr(), ws_bytes, stream)
        return out

    # fp8 activations with caller-provided 1x128 scales: skip the quant step
    sorted_ids, sorted_w, sorted_eids, num_valid, acc = moe_sorting(
        topk_ids, topk_weight, global_E, model_dim, dtypes.fp32, block_m, mask,
        num_local_tokens, moe_sorting_dispatch_policy)
    st1 = moe_stage1_a8w4 if a8w4 else moe_stage1_fp8_blockscale
    st2 = moe_stage2_a8w4 if a8w4 else moe_stage2_fp8_blockscale
    # doweight_stage1: the routing weights go to stage 1, stage 2 sums unweighted
    # (aiter/fused_moe.py:1253, 1330)
    a2, a2s = st1(hidden_states.contiguous(), a1_scale.contiguous(), w1c, w1s, sorted_ids,
                  sorted_eids, num_valid, topk, block_m, shuffled,
                  sorted_weights=sorted_w if doweight_stage1 else None, activation=activation)
    st2(a2, a2s, w2c, w2s, sorted_ids, None if doweight_stage1 else sorted_w, sorted_eids,
        num_valid, acc, block_m, shuffled)
    _abi.call("aiter_amd_moe_acc_to_out", acc.data_ptr(), out.data_ptr(), AITER_DTYPE[out_dtype],
              num_valid.data_ptr(), M, model_dim, stream)
    return out


def _register_custom_op():
    """torch.ops.aiter_amd.fused_moe_ with its fake, for the CUDA (HIP) and CPU
    dispatch keys as the reference registers torch.ops.aiter.fused_moe_ (the CPU
    kernel only validates and raises: the layer needs the GPU)."""
    if hasattr(torch.ops.aiter_amd, "fused_moe_"):
        return
    lib = torch.library.Library("aiter_amd", "FRAGMENT")
    schema = torch.library.infer_schema(fused_moe_, mutates_args=())
    lib.define("fused_moe_" + schema)
    lib.impl("fused_moe_", fused_moe_, "CUDA")
    lib.impl("fused_moe_", fused_moe_, "CPU")
    torch.library.register_fake("aiter_amd::fused_moe_", fused_moe_fake, lib=lib)
    _register_custom_op.lib = lib


_register_custom_op()


def _stage1(entry, a1, a1_scale, w1, w1_scale, sorted_ids, sorted_expert_ids, num_valid_ids,
            topk, block_m, shuffled, a1_scale_transposed, sorted_weights, activation):
    T, H = a1.shape
    E, N1, _ = w1.shape
    inter = N1 // 2
    a2 = torch.empty((T, topk, inter), dtype=dtypes.fp8, device=a1.device)
    a2s = torch.empty((T, topk, inter // 128), dtype=dtypes.fp32, device=a1.device)
    _abi.call(
        entry,
        a1.data_ptr(), a1_scale.data_ptr(), int(bool(a1_scale_transposed)), w1.data_ptr(),
        w1_scale.data_ptr(), sorted_ids.data_ptr(), _ptr(sorted_weights),
        sorted_expert_ids.data_ptr(), num_valid_ids.data_ptr(), a2.data_ptr(), a2s.data_ptr(),
        T, H, inter, E, topk,
        int(block_m), sorted_expert_ids.numel(), int(ActivationType(activation)),
        int(bool(shuffled)),
        _stream(a1.device))
    return a2, a2s


def moe_stage1_fp8_blockscale(a1, a1_scale, w1, w1_scale, sorted_ids, sorted_expert_ids,
                              num_valid_ids, topk, block_m, shuffled, a1_scale_transposed=False,
                              sorted_weights=None, activation=ActivationType.Silu):
    """Stage 1 (gate+up GEMM, SiLU*up, fp8 1x128 requant).

    Returns (a2 fp8 [T, topk, I], a2_scale f32 [T, topk, I/128]) -- the pair
    the reference builds from ck_moe_stage1 + quant (fused_moe.py:1297-1314).
    sorted_weights (doweight_stage1): each pair's routing weight scales its
    gate and up rows before the activation (fused_moe.py:1568-1571).
    activation: Silu or Gelu (torch's exact erf form) on gate.
    """
    return _stage1("aiter_amd_moe_stage1_fp8_blockscale", a1, a1_scale, w1, w1_scale,
                   sorted_ids, sorted_expert_ids, num_valid_ids, topk, block_m, shuffled,
                   a1_scale_transposed, sorted_weights, activation)


def moe_stage1_a8w4(a1, a1_scale, w1, w1_scale, sorted_ids, sorted_expert_ids, num_valid_ids,
                    topk, block_m, shuffled, a1_scale_transposed=False, sorted_weights=None,
                    activation=ActivationType.Silu):
    """A8W4 stage 1: fp8 1x128 activations x MXFP4 w1 (packed uint8 [E, 2I, H/2],
    e8m0 [E, 2I, H/32] or its 2-D e8m0_shuffle layout); same outputs as
    moe_stage1_fp8_blockscale."""
    E, N1 = w1.shape[0], w1.shape[1]
    w1_scale = e8m0_rowmajor(w1_scale, E, N1, a1.shape[1] // 32)
    return _stage1("aiter_amd_moe_stage1_a8w4", a1, a1_scale, w1.view(torch.uint8),
                   w1_scale.view(torch.uint8), sorted_ids, sorted_expert_ids, num_valid_ids,
                   topk, block_m, shuffled, a1_scale_transposed, sorted_weights, activation)


def _stage2(a2, a2_scale, w2, w2_scale, sorted_ids, sorted_weights, sorted_expert_ids,
            num_valid_ids, out_acc, block_m, shuffled, quant_type):
    T, topk, inter = a2.shape
    E, H, _ = w2.shape
    if out_acc.dtype not in (dtypes.fp32, dtypes.bf16, dtypes.fp16):
        raise ValueError(f"out_acc must be float32, bfloat16 or float16, got {out_acc.dtype}")
    # the reference-shaped entry (include/aiter_ctypes.h); its w1 is unused
    ffi.ck_moe_stage2(a2, w2, w2, sorted_ids, sorted_expert_ids, num_valid_ids, out_acc, topk,
                      None, w2_scale, a2_scale, int(block_m), sorted_weights, int(quant_type),
                      0, 1, False, None, bool(shuffled))


def moe_stage2_fp8_blockscale(a2, a2_scale, w2, w2_scale, sorted_ids, sorted_weights,
                              sorted_expert_ids, num_valid_ids, out_acc, block_m, shuffled):
    """Stage 2: out_acc[t] += w * (a2 . w2^T) with block-scale dequant, accumulated
    atomically into out_acc: fp32 (one rounding at the end, by the caller), or bf16 /
    fp16 -- the reference's moe_buf, zeroed by moe_sorting, rounded after every add as
    ck_moe_stage2 does (gemm_moe_ck2stages.cu:118-181, aiter/fused_moe.py:1316-1332).
    sorted_weights None: w = 1 (doweight_stage1 applied the weights in stage 1)."""
    _stage2(a2, a2_scale, w2, w2_scale, sorted_ids, sorted_weights, sorted_expert_ids,
            num_valid_ids, out_acc, block_m, shuffled, QuantType.per_1x128)


def moe_stage2_a8w4(a2, a2_scale, w2, w2_scale, sorted_ids, sorted_weights, sorted_expert_ids,
                    num_valid_ids, out_acc, block_m, shuffled):
    """A8W4 stage 2: MXFP4 w2 (packed uint8 [E, H, I/2], e8m0 [E, H, I/32] or its
    2-D e8m0_shuffle layout)."""
    w2_scale = e8m0_rowmajor(w2_scale, w2.shape[0], w2.shape[1], a2.shape[-1] // 32)
    _stage2(a2, a2_scale, w2.view(torch.uint8), w2_scale.view(torch.uint8), sorted_ids,
            sorted_weights, sorted_expert_ids, num_valid_ids, out_acc, block_m, shuffled,
            QuantType.per_1x32)


__all__ = [
    "BLOCK_SIZE_M", "fused_moe", "fused_moe_", "fused_moe_a8w4", "fused_moe_fake", "moe_sorting",
    "e8m0_rowmajor",
    "select_block_m",
    "moe_stage1_fp8_blockscale", "moe_stage2_fp8_blockscale", "moe_stage1_a8w4",
    "moe_stage2_a8w4", "per_group_quant_hip",
    "get_inter_dim", "default_block_m", "sorted_capacity",
]
