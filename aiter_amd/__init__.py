"""aiter_amd: MI355X (gfx950) blockscale fused-MoE, a drop-in for
aiter.fused_moe's FP8 block-scale path, plus an A8W4 layer (fp8 activations x
MXFP4 weights) behind its own entry, fused_moe_a8w4.

    from aiter_amd import fused_moe, QuantType, ActivationType
    out = fused_moe(x, w1, w2, topk_weight, topk_ids,
                    quant_type=QuantType.per_128x128, w1_scale=s1, w2_scale=s2)

The compute runs in libaiter_amd.so (HIP kernels behind a C ABI, see
include/aiter_amd.h and, in the reference's ctypes shape, include/aiter_ctypes.h);
build it with ``python -m aiter_amd.build``.
"""
from .enums import ActivationType, QuantType, dtypes, quant_remap
from .fused_moe import (
    BLOCK_SIZE_M,
    default_block_m,
    fused_moe,
    fused_moe_,
    fused_moe_a8w4,
    fused_moe_fake,
    get_inter_dim,
    moe_sorting,
    moe_stage1_a8w4,
    moe_stage1_fp8_blockscale,
    moe_stage2_a8w4,
    moe_stage2_fp8_blockscale,
    select_block_m,
    sorted_capacity,
)
from .quant import (
    dynamic_per_token_scaled_quant,
    e8m0_shuffle,
    e8m0_to_f32,
    e8m0_unshuffle,
    f32_to_e8m0,
    per_1x32_f4_quant,
    per_group_quant_hip,
    quant_weight_per_128x128,
)
from .shuffle import (shuffle_scale_a16w4, shuffle_weight, shuffle_weight_a16w4,
                      unshuffle_scale_a16w4, unshuffle_weight, unshuffle_weight_a16w4)
from .topk import (
    biased_grouped_topk,
    biased_grouped_topk_hip,
    fused_topk,
    grouped_topk,
    topk_sigmoid,
    topk_softmax,
)

__all__ = [
    "ActivationType", "QuantType", "dtypes", "quant_remap", "BLOCK_SIZE_M", "default_block_m",
    "fused_moe", "fused_moe_", "fused_moe_a8w4", "fused_moe_fake", "get_inter_dim", "moe_sorting",
    "moe_stage1_fp8_blockscale", "moe_stage2_fp8_blockscale", "moe_stage1_a8w4",
    "moe_stage2_a8w4", "select_block_m", "sorted_capacity", "dynamic_per_token_scaled_quant", "per_group_quant_hip",
    "quant_weight_per_128x128", "per_1x32_f4_quant", "f32_to_e8m0", "e8m0_to_f32", "e8m0_shuffle",
    "e8m0_unshuffle",
    "shuffle_weight", "unshuffle_weight", "shuffle_weight_a16w4", "unshuffle_weight_a16w4",
    "shuffle_scale_a16w4", "unshuffle_scale_a16w4", "topk_softmax", "topk_sigmoid", "grouped_topk",
    "biased_grouped_topk", "biased_grouped_topk_hip", "fused_topk",
]
