"""MoE routing: router logits -> top-k experts and their weights per token,
the step before ``moe_sorting``.

Mirrors aiter's routing surface, with the same argument names, in-place
outputs and return values:

* ``topk_softmax(topk_weights, topk_indices, token_expert_indices,
  gating_output, need_renorm, num_shared_experts=0,
  shared_expert_scoring_func="")`` -- aiter/ops/moe_op.py:15-36;
* ``topk_sigmoid(topk_weights, topk_indices, gating_output)`` --
  aiter/ops/moe_op.py:39-42;
* ``grouped_topk(gating_output, topk_weights, topk_ids, num_expert_group,
  topk_group, need_renorm, is_softmax=True, routed_scaling_factor=1.0)`` --
  aiter/ops/topk.py:28-38;
* ``biased_grouped_topk(gating_output, correction_bias, topk_weights,
  topk_ids, num_expert_group, topk_group, need_renorm,
  routed_scaling_factor=1.0)`` -- aiter/ops/topk.py:90-125;
* ``fused_topk(hidden_states, gating_output, topk, renormalize)`` --
  aiter/fused_moe.py:1853-1923.

Every op runs the HIP kernel of moe_route.hip through the C ABI; there is no
torch fallback. Output rows may be strided (row stride >= topk, unit column
stride), as the reference kernels allow.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import ffi
from .enums import dtypes


def _check(gating_output: torch.Tensor, topk_weights: torch.Tensor, topk_ids: torch.Tensor):
    if gating_output.dim() != 2 or not gating_output.is_contiguous():
        raise ValueError("gating_output must be a contiguous [tokens, num_experts] tensor")
    if gating_output.dtype not in (dtypes.fp32, dtypes.bf16, dtypes.fp16):
        raise ValueError(f"gating_output dtype {gating_output.dtype} is not fp32/bf16/fp16")
    M = gating_output.shape[0]
    outs = ((topk_weights, "topk_weights", dtypes.fp32), (topk_ids, "topk_ids", dtypes.i32))
    for t, name, dt in outs:
        if t.dtype != dt:
            raise ValueError(f"{name} must be {dt}, got {t.dtype}")
        if t.dim() != 2 or t.shape[0] != M or t.shape[1] != topk_weights.shape[1]:
            raise ValueError(f"{name} must be [tokens, topk], got {tuple(t.shape)}")
        if t.shape[1] > 0 and t.stride(1) != 1:
            raise ValueError(f"{name} needs a unit column stride")
        if t.device != gating_output.device:
            raise ValueError(f"{name} is on {t.device}, gating_output on {gating_output.device}")
    return M, gating_output.shape[1], topk_weights.shape[1]


def topk_softmax(topk_weights: torch.Tensor, topk_indices: torch.Tensor,
                 token_expert_indices: Optional[torch.Tensor], gating_output: torch.Tensor,
                 need_renorm: bool, num_shared_experts: int = 0,
                 shared_expert_scoring_func: str = "") -> None:
    """Experts ranked by logit (ties: lower index first); weight
    exp(x - rowmax) divided by the sum over the topk (need_renorm) or over
    the whole row; token_expert_indices[t, j] = j * tokens + t
    (csrc/kernels/topk_softmax_kernels.cu:380-500).

    With num_shared_experts = S > 0 and shared_expert_scoring_func
    "sigmoid" (the only one the reference supports), gating_output is
    [tokens, E + S]: the first E columns are routed as above and
    topk_weights [tokens, topk + S] receives sigmoid(gating_output[:, E + j])
    in column topk + j (topk_softmax_kernels.cu:326-353, 760-810)."""
    S = int(num_shared_experts)
    if S == 0:
        M, E, k = _check(gating_output, topk_weights, topk_indices)
    else:
        if shared_expert_scoring_func != "sigmoid":
            raise ValueError("Only 'sigmoid' scoring function is supported for shared experts, "
                             f"got: {shared_expert_scoring_func!r}")
        if topk_weights.dim() != 2 or topk_weights.shape[1] != topk_indices.shape[-1] + S:
            raise ValueError("topk_weights must be [tokens, topk + num_shared_experts]")
        M, _, k = _check(gating_output, topk_weights[:, :topk_indices.shape[-1]], topk_indices)
    if token_expert_indices is not None:
        if (token_expert_indices.dtype != dtypes.i32 or not token_expert_indices.is_contiguous()
                or tuple(token_expert_indices.shape) != (M, k)):
            raise ValueError("token_expert_indices must be a contiguous [tokens, topk] i32 tensor")
    ffi.topk_softmax(topk_weights, topk_indices, token_expert_indices, gating_output,
                     bool(need_renorm), S, shared_expert_scoring_func)


def topk_sigmoid(topk_weights: torch.Tensor, topk_indices: torch.Tensor,
                 gating_output: torch.Tensor) -> None:
    """Experts ranked by logit; weight sigmoid(logit)
    (op_tests/test_moe_topk_sigmoid.py:28-32)."""
    M, E, k = _check(gating_output, topk_weights, topk_indices)
    ffi.topk_sigmoid(topk_weights, topk_indices, gating_output)


def _grouped(gating_output, bias, topk_weights, topk_ids, num_expert_group, topk_group,
             need_renorm, is_softmax, routed_scaling_factor):
    M, E, k = _check(gating_output, topk_weights, topk_ids)
    if bias is not None:
        if bias.dtype != dtypes.fp32 or bias.numel() != E or not bias.is_contiguous():
            raise ValueError("correction_bias must be a contiguous f32 [num_experts] tensor")
        ffi.biased_grouped_topk(gating_output, bias.view(E), topk_weights, topk_ids,
                                int(num_expert_group), int(topk_group), bool(need_renorm),
                                float(routed_scaling_factor))
    else:
        ffi.grouped_topk(gating_output, topk_weights, topk_ids, int(num_expert_group),
                         int(topk_group), bool(need_renorm), bool(is_softmax),
                         float(routed_scaling_factor))


def grouped_topk(gating_output: torch.Tensor, topk_weights: torch.Tensor,
                 topk_ids: torch.Tensor, num_expert_group: int, topk_group: int,
                 need_renorm: bool, is_softmax: bool = True,
                 routed_scaling_factor: float = 1.0) -> None:
    """Softmax (or sigmoid) scores; a group's score is its best expert score;
    the topk_group best groups are kept and their experts ranked by score
    (aiter/ops/topk.py:163-197); weight = score * routed_scaling_factor
    (/ the topk sum when need_renorm)."""
    _grouped(gating_output, None, topk_weights, topk_ids, num_expert_group, topk_group,
             need_renorm, is_softmax, routed_scaling_factor)


def biased_grouped_topk(gating_output: torch.Tensor, correction_bias: torch.Tensor,
                        topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                        num_expert_group: int, topk_group: int, need_renorm: bool,
                        routed_scaling_factor: float = 1.0) -> None:
    """Sigmoid scores; choice = score + correction_bias; a group's score is
    the sum of its two best choices; experts of the topk_group best groups
    ranked by choice; weight = the unbiased score * routed_scaling_factor
    (/ the topk sum when need_renorm) (aiter/ops/topk.py:90-160). Experts of
    groups that are not kept are never chosen."""
    _grouped(gating_output, correction_bias, topk_weights, topk_ids, num_expert_group,
             topk_group, need_renorm, False, routed_scaling_factor)


biased_grouped_topk_hip = biased_grouped_topk


def fused_topk(hidden_states: torch.Tensor, gating_output: torch.Tensor, topk: int,
               renormalize: bool, topk_ids: Optional[torch.Tensor] = None,
               topk_weights: Optional[torch.Tensor] = None
               ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax top-k routing of fused_moe's inputs (aiter/fused_moe.py:1853-1923):
    returns (topk_weights f32 [M, topk], topk_ids i32 [M, topk])."""
    if hidden_states.shape[0] != gating_output.shape[0]:
        raise ValueError("Number of tokens mismatch")
    M = gating_output.shape[0]
    dev = gating_output.device
    if topk_weights is None:
        topk_weights = torch.empty(M, topk, dtype=dtypes.fp32, device=dev)
    if topk_ids is None:
        topk_ids = torch.empty(M, topk, dtype=dtypes.i32, device=dev)
    topk_softmax(topk_weights, topk_ids, None, gating_output, renormalize)
    return topk_weights, topk_ids
