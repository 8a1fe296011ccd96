"""1x128 FP8 activation quantisation (HIP) and host-side weight preparation.

`per_group_quant_hip` / `dynamic_per_token_scaled_quant` keep the reference
signatures (aiter/ops/quant.py:260-292, csrc/kernels/quant_kernels.cu:710-757)
and run the gfx950 kernel through the C ABI.

`quant_weight_per_128x128` is the weight-preparation step callers run once
at load time (the reference test does the same, op_tests/test_moe_2stage.py:
82-111, with pertoken_quant semantics aiter/ops/quant.py:42-72): it is
ordinary torch code on whatever device the weights live on, not part of
the per-token hot path.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from .enums import dtypes


def dynamic_per_token_scaled_quant(
    out: torch.Tensor,
    input: torch.Tensor,
    scales: torch.Tensor,
    scale_ub: Optional[torch.Tensor] = None,
    shuffle_scale: bool = False,
    num_rows: Optional[torch.Tensor] = None,
    num_rows_factor: int = 1,
) -> None:
    """Quantise `input` viewed as [rows, 128] groups into fp8 `out` (in place).

    `input` has shape [..., 128] (the reference passes x.view(-1, 128)); `out`
    has the original [rows, cols] shape and fixes `cols`. Runs the
    reference-shaped entry of the same name (include/aiter_ctypes.h).
    """
    if scale_ub is not None:
        raise NotImplementedError("scale_ub is not supported for 1x128 group quant")
    from . import ffi

    ffi.dynamic_per_token_scaled_quant(out, input, scales, None, shuffle_scale, num_rows,
                                       num_rows_factor)


def per_group_quant_hip(
    x: torch.Tensor,
    scale: Optional[torch.Tensor] = None,
    quant_dtype: torch.dtype = dtypes.fp8,
    group_size: int = 128,
    transpose_scale: bool = False,
    num_rows: Optional[torch.Tensor] = None,
    num_rows_factor: int = 1,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Dynamic 1 x group_size FP8 quant; returns (y, scale) like the reference."""
    if scale is not None:
        raise ValueError("unsupported: static per token quant")
    if quant_dtype != dtypes.fp8:
        raise NotImplementedError(f"quant_dtype {quant_dtype} is not supported (fp8 only)")
    if group_size != 128:
        raise NotImplementedError(f"group_size {group_size} is not supported (128 only)")
    shape = x.shape
    scale = torch.empty((*shape[:-1], shape[-1] // group_size), dtype=dtypes.fp32,
                        device=x.device)
    y = torch.empty(shape, dtype=quant_dtype, device=x.device)
    dynamic_per_token_scaled_quant(y, x.contiguous().view(-1, group_size), scale,
                                   shuffle_scale=transpose_scale, num_rows=num_rows,
                                   num_rows_factor=num_rows_factor)
    return y, scale


def quant_weight_per_128x128(w: torch.Tensor, quant_dtype: torch.dtype = dtypes.fp8):
    """[E, N, K] float weights -> (fp8 [E, N, K], fp32 scales [E, N/128, K/128]).

    scale = amax(block)/448 (a zero block gets scale 1), q = fp8(w/scale)
    (pertoken_quant over each 128x128 block, aiter/ops/quant.py:42-72).
    """
    E, N, K = w.shape
    if N % 128 or K % 128:
        raise ValueError("weight dims must be multiples of 128")
    blk = w.float().view(E, N // 128, 128, K // 128, 128).permute(0, 1, 3, 2, 4)
    amax = blk.abs().amax(dim=(-1, -2), keepdim=True)
    scale = amax / torch.finfo(quant_dtype).max
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)
    q = (blk / scale).to(quant_dtype)
    q = q.permute(0, 1, 3, 2, 4).contiguous().view(E, N, K)
    return q, scale.view(E, N // 128, K // 128).contiguous()


# ------------------------------------------------------------------ MXFP4 ---
# Weight preparation for the A8W4 path (run once at load time, like
# quant_weight_per_128x128).  OCP MX FP4: e2m1 values, two per byte with the
# even element in the low nibble, one e8m0 scale per 32 consecutive K.


def f32_to_e8m0(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> e8m0 byte as aiter/utility/fp4_utils.py:49-58: the biased
    exponent, plus one when mantissa bit 22 is set and a lower bit is set or
    the value is normal (1.5*2^e and above round to 2^(e+1))."""
    u = x.float().contiguous().view(torch.int32)
    exp = (u >> 23) & 0xFF
    up = ((u & 0x400000) != 0) & (((u & 0x200000) != 0) | ((u & 0x1FFFFF) != 0) | (exp > 0))
    e = (exp + up.to(torch.int32)) & 0xFF
    e = torch.where(exp == 0xFF, torch.full_like(e, 0xFF), e)
    return e.to(torch.uint8)


def e8m0_to_f32(e: torch.Tensor) -> torch.Tensor:
    """e8m0 byte -> 2^(e-127) (aiter/utility/fp4_utils.py:61-69; 0 -> 2^-127)."""
    ei = e.view(torch.uint8).to(torch.int32)
    bits = ei << 23
    bits = torch.where(ei == 0, torch.full_like(bits, 0x00400000), bits)
    bits = torch.where(ei == 0xFF, torch.full_like(bits, 0x7F800001), bits)
    return bits.view(torch.float32)


def f32_to_e2m1(y: torch.Tensor) -> torch.Tensor:
    """fp32 -> e2m1 code (uint8 0..15): round to nearest even, |y| >= 6
    saturates, sign kept -- the saturating conversion of
    aiter/utility/fp4_utils.py:120-235.  Below 1.0 the value is rounded on
    the 0.5 grid by adding 2^22 in fp32; above, the exponent is rebased
    (bias 127 -> 1) and the 22 dropped mantissa bits are rounded half-even."""
    u = y.float().contiguous().view(torch.int32)
    sign = (u >> 31) & 1
    a = (u & 0x7FFFFFFF).view(torch.float32)
    denorm = (a + 2.0 ** 22).view(torch.int32) - (149 << 23)
    ua = a.view(torch.int32)
    normal = (ua + ((1 - 127) << 23) + ((1 << 21) - 1) + ((ua >> 22) & 1)) >> 22
    code = torch.where(a >= 6.0, torch.full_like(ua, 7), torch.where(a < 1.0, denorm, normal))
    return ((code & 7) | (sign << 3)).to(torch.uint8)


def per_1x32_f4_quant(x: torch.Tensor, scale=None, quant_dtype=dtypes.fp4x2,
                      shuffle: bool = False):
    """MXFP4 quant of [..., K] (aiter/ops/quant.py:75-105): per 32-element
    block, scale = e8m0(amax / 4), values e2m1(x / 2^(scale-127)).
    Returns (packed [..., K/2] as fp4x2, scales [..., K/32] as e8m0); with
    shuffle, the scales are the reference's 2-D e8m0_shuffle layout."""
    if scale is not None:
        raise ValueError("unsupported: static MXFP4 scale")
    if quant_dtype != dtypes.fp4x2:
        raise NotImplementedError(f"quant_dtype {quant_dtype} is not supported (fp4x2 only)")
    shape = x.shape
    K = shape[-1]
    if K % 32:
        raise ValueError(f"last dim {K} must be a multiple of 32")
    b = x.float().reshape(-1, K // 32, 32)
    e = f32_to_e8m0(b.abs().amax(dim=-1) / 4.0)
    codes = f32_to_e2m1(b / e8m0_to_f32(e).unsqueeze(-1)).reshape(*shape)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).contiguous()
    if shuffle:   # the reference's 2-D scale, then e8m0_shuffle (aiter/ops/quant.py:101-105)
        return packed.view(dtypes.fp4x2), e8m0_shuffle(e.reshape(-1, K // 32)).view(dtypes.fp8_e8m0)
    return packed.view(dtypes.fp4x2), e.reshape(*shape[:-1], K // 32).view(dtypes.fp8_e8m0)


def e8m0_shuffle(scale: torch.Tensor) -> torch.Tensor:
    """The reference's MXFP4 scale layout for its fused kernels
    (aiter/utility/fp4_utils.py:72-92): a 2-D [m, n] byte array, padded to
    [ceil(m/256)*256, ceil(n/8)*8], viewed as (m/32, 2, 16, n/8, 2, 4) and
    permuted to (0, 3, 5, 2, 4, 1). fp32 scales pass through."""
    if scale is None or scale.dtype == torch.float32:
        return scale
    if scale.dim() != 2:
        raise ValueError("scale must be a 2D tensor")
    m, n = scale.shape
    sm, sn = (m + 255) // 256 * 256, (n + 7) // 8 * 8
    pad = torch.empty((sm, sn), dtype=scale.dtype, device=scale.device)
    pad[:m, :n] = scale
    return (pad.view(sm // 32, 2, 16, sn // 8, 2, 4).permute(0, 3, 5, 2, 4, 1)
            .contiguous().view(sm, sn))


def e8m0_unshuffle(scale: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """Inverse of e8m0_shuffle: the row-major [rows, cols] scales."""
    sm, sn = scale.shape
    if sm % 256 or sn % 8 or rows > sm or cols > sn:
        raise ValueError(f"[{sm}, {sn}] is not an e8m0_shuffle layout of [{rows}, {cols}]")
    return (scale.view(sm // 32, sn // 8, 4, 16, 2, 2).permute(0, 5, 3, 1, 4, 2)
            .contiguous().view(sm, sn)[:rows, :cols].contiguous())
