"""The reference's untuned FP8-blockscale `fused_moe_` call sequence on
gfx950, restated over the reference-shaped ctypes stubs of aiter_amd.ffi.

Test infrastructure: it drives libaiter_amd.so the way aiter/fused_moe.py
would once its compile_ops stubs bind this library, so the GPU tests can
check the reference's own sequence end to end. Each step cites the lines
it follows:

* metadata (`get_2stage_cfgs`, fused_moe.py:856-893, 1035-1076): the
  shape key is the padded token count (`get_padded_M`, 606-612); for
  per_1x128 with Silu / Gelu, bf16 out, fp8 weights and no doweight the
  1-stage table holds `fmoe_fp8_blockscale_g1u1` (568-594) and
  `run_1stage = token > 32 and inter_dim % 128 == 0`; otherwise the 2-stage
  path takes block_m 16 (64 above 32 tokens) and `get_ksplit` (540-563);
* sorting (`moe_sorting`, 27-103) at that block size;
* 1-stage (`fused_moe_1stage`, 367-511): 1x128 quant with transposed
  scales, then `fmoe_fp8_blockscale_g1u1` into moe_buf;
* 2-stage (`fused_moe_2stages`, 1103-1334): 1x128 quant (row-major
  scales), `ck_moe_stage1` (1669-1725: bf16 a2, or fp32 gate|up rows plus
  `silu_and_mul` / `gelu_and_mul` when ksplit > 1), the a2 requant with
  `num_rows_factor=topk` (1306-1314), `ck_moe_stage2` into moe_buf
  (1316-1332).
"""
from __future__ import annotations

from typing import Optional

import torch

from aiter_amd import ffi
from aiter_amd.enums import ActivationType, QuantType

BLOCK_SIZE_M = 32          # fused_moe.py:22
CU_NUM = 256               # MI355X


def next_pow2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def get_padded_M(M: int) -> int:
    return next_pow2(M) if M < 32768 else 32768


def get_ksplit(token, topk, expert, inter_dim, model_dim, cu_num=CU_NUM) -> int:
    if token * topk > expert:
        return 0
    tg_num = ((inter_dim + 127) // 128) * token * topk
    if tg_num >= cu_num:
        return 0
    split_max = (cu_num + tg_num - 1) // tg_num
    for i in reversed(range(2, split_max + 1)):
        if model_dim % i == 0 and (model_dim // i) % 256 == 0:
            return i
    return 0


def untuned_metadata(M, topk, E, model_dim, inter_dim, activation=ActivationType.Silu,
                     doweight_stage1=False):
    """(run_1stage, block_m, ksplit) of get_2stage_cfgs with no tuned row."""
    token = get_padded_M(M)
    in_1stage_table = (activation in (ActivationType.Silu, ActivationType.Gelu)
                       and not doweight_stage1)
    run_1stage = in_1stage_table and token > 32 and inter_dim % 128 == 0
    if run_1stage:
        return True, BLOCK_SIZE_M, 0
    block_m = 64 if token > 32 else 16
    return False, block_m, get_ksplit(token, topk, E, inter_dim, model_dim)


def moe_sorting(topk_ids, topk_weights, num_experts, model_dim, dtype, block_size,
                expert_mask=None, num_local_tokens=None):
    M, topk = topk_ids.shape
    dev = topk_ids.device
    cap = int(topk_ids.numel() + num_experts * block_size - topk)
    sorted_ids = torch.empty(cap, dtype=torch.int32, device=dev)
    sorted_weights = torch.empty(cap, dtype=torch.float32, device=dev)
    sorted_expert_ids = torch.empty((cap + block_size - 1) // block_size, dtype=torch.int32,
                                    device=dev)
    num_valid_ids = torch.empty(2, dtype=torch.int32, device=dev)
    moe_buf = torch.empty((M, model_dim), dtype=dtype, device=dev)
    ffi.moe_sorting_fwd(topk_ids, topk_weights, sorted_ids, sorted_weights, sorted_expert_ids,
                        num_valid_ids, moe_buf, num_experts, int(block_size), expert_mask,
                        num_local_tokens, 0)
    return sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf


def per_group_quant_hip(x, transpose_scale=False, num_rows=None, num_rows_factor=1):
    """aiter/ops/quant.py:260-292 with group_size 128 and fp8 output."""
    scale = torch.empty((*x.shape[:-1], x.shape[-1] // 128), dtype=torch.float32,
                        device=x.device)
    y = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    ffi.dynamic_per_token_scaled_quant(y, x.view(-1, 128), scale, None, transpose_scale,
                                       num_rows, num_rows_factor)
    return y, scale


def ck_moe_stage1(hidden_states, w1, w2, sorted_token_ids, sorted_expert_ids, num_valid_ids,
                  out, topk, block_m, a1_scale, w1_scale, sorted_weights=None,
                  activation=ActivationType.Silu, splitk=0, is_shuffled=True):
    """fused_moe.py:1669-1725 (quant_type per_1x128)."""
    token_num = hidden_states.shape[0]
    is_splitk = splitk > 1
    if is_splitk:
        sorted_size = min(token_num * topk * block_m, sorted_token_ids.shape[0])
        tmp_out = torch.empty((sorted_size, w1.shape[1]), dtype=torch.float32,
                              device=out.device)
    else:
        tmp_out = out
    ffi.ck_moe_stage1(hidden_states, w1, w2, sorted_token_ids, sorted_expert_ids,
                      num_valid_ids, tmp_out, topk, "", w1_scale, a1_scale, block_m,
                      sorted_weights, int(QuantType.per_1x128), int(activation),
                      splitk if is_splitk else 0, False, None, is_shuffled)
    if is_splitk:
        valid_out = tmp_out[: token_num * topk, :]
        if activation == ActivationType.Silu:
            ffi.silu_and_mul(out, valid_out)
        else:
            ffi.gelu_and_mul(out, valid_out)
    return out


def fused_moe(hidden_states, w1, w2, topk_weight, topk_ids, w1_scale, w2_scale,
              expert_mask=None, activation=ActivationType.Silu, num_local_tokens=None,
              force_path: Optional[str] = None, trace: Optional[list] = None):
    """fused_moe_ (fused_moe.py:205-364) for quant_type per_128x128 /
    per_1x128 with pre-shuffled fp8 weights. force_path "1stage" / "2stage"
    stands in for a tuned row that picks the other path; trace collects the
    steps taken."""
    M, topk = topk_ids.shape
    E, model_dim, inter_dim = w1.shape[0], w2.shape[1], w2.shape[2]
    global_E = expert_mask.numel() if expert_mask is not None else E
    dtype = hidden_states.dtype
    run_1stage, block_m, ksplit = untuned_metadata(M, topk, E, model_dim, inter_dim, activation)
    if force_path is not None:
        run_1stage = force_path == "1stage"
        if run_1stage:
            block_m, ksplit = BLOCK_SIZE_M, 0
    trace = trace if trace is not None else []
    trace.append(("metadata", run_1stage, block_m, ksplit))
    sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf = moe_sorting(
        topk_ids, topk_weight, global_E, model_dim, dtype, block_m, expert_mask,
        num_local_tokens)
    if run_1stage:
        # fused_moe_1stage (fused_moe.py:430-507)
        a1, a1_scale = per_group_quant_hip(hidden_states, transpose_scale=True,
                                           num_rows=num_local_tokens)
        ffi.fmoe_fp8_blockscale_g1u1(moe_buf, a1, w1, w2, sorted_ids, sorted_weights,
                                     sorted_expert_ids, num_valid_ids, topk, a1_scale, w1_scale,
                                     w2_scale, "", 128, 128, None, int(activation), block_m)
        trace.append(("fmoe_fp8_blockscale_g1u1",))
        return moe_buf
    # fused_moe_2stages (fused_moe.py:1223-1334) with ck_moe_stage1
    a1, a1_scale = per_group_quant_hip(hidden_states, num_rows=num_local_tokens)
    a2 = torch.empty((M, topk, inter_dim), dtype=dtype, device=hidden_states.device)
    ck_moe_stage1(a1, w1, w2, sorted_ids, sorted_expert_ids, num_valid_ids, a2, topk, block_m,
                  a1_scale, w1_scale, None, activation, ksplit)
    trace.append(("ck_moe_stage1", ksplit))
    a2q, a2_scale = per_group_quant_hip(a2, num_rows=num_local_tokens, num_rows_factor=topk)
    a2q = a2q.view(M, topk, inter_dim)
    ffi.ck_moe_stage2(a2q, w1, w2, sorted_ids, sorted_expert_ids, num_valid_ids, moe_buf, topk,
                      "", w2_scale, a2_scale, block_m, sorted_weights,
                      int(QuantType.per_1x128), int(activation), 1, False, None, True)
    trace.append(("ck_moe_stage2",))
    return moe_buf
