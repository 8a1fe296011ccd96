"""Enums and dtype aliases of the MoE interface.

Integer values are those of the reference (csrc/include/aiter_enum.h:7-26),
so callers that pass `.value` ints (fused_moe_ schema) keep working.
fp8 is OCP e4m3fn on gfx950 (aiter/utility/dtypes.py:10-33).
"""
from enum import IntEnum

import torch


class ActivationType(IntEnum):
    No = -1
    Silu = 0
    Gelu = 1
    Swiglu = 2


class QuantType(IntEnum):
    No = 0
    per_Tensor = 1
    per_Token = 2
    per_1x32 = 3
    per_1x128 = 4
    per_128x128 = 5
    per_256x128 = 6
    per_1024x128 = 7


# per_128x128 weights are consumed with 1x128 activation groups
# (aiter/fused_moe.py:597 quant_remap).
quant_remap = {QuantType.per_128x128: QuantType.per_1x128}


class dtypes:
    fp8 = torch.float8_e4m3fn
    fp8_e8m0 = getattr(torch, "float8_e8m0fnu", torch.uint8)
    fp4x2 = getattr(torch, "float4_e2m1fn_x2", torch.uint8)
    fp16 = torch.float16
    bf16 = torch.bfloat16
    fp32 = torch.float32
    i32 = torch.int32
    u8 = torch.uint8


# AiterDtype codes (csrc/include/aiter_enum.h:27-43) used on the C ABI
AITER_DTYPE = {
    torch.float8_e4m3fn: 0,
    torch.float16: 2,
    torch.bfloat16: 3,
    torch.float32: 4,
    torch.int32: 8,
    torch.uint8: 11,
}
if dtypes.fp8_e8m0 is not torch.uint8:
    AITER_DTYPE[dtypes.fp8_e8m0] = 1
if dtypes.fp4x2 is not torch.uint8:
    AITER_DTYPE[dtypes.fp4x2] = 6
