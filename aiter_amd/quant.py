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

from . import _abi
from .enums import AITER_DTYPE, dtypes


def _stream_ptr(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


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
    has the original [rows, cols] shape and fixes `cols`.
    """
    if scale_ub is not None:
        raise NotImplementedError("scale_ub is not supported for 1x128 group quant")
    if not (input.is_contiguous() and out.is_contiguous() and scales.is_contiguous()):
        raise ValueError("input, out and scales must be contiguous")
    if out.dtype != dtypes.fp8:
        raise ValueError(f"out must be {dtypes.fp8}, got {out.dtype}")
    group = input.shape[-1]
    cols = out.shape[-1]
    rows = out.numel() // cols
    if input.numel() != out.numel():
        raise ValueError("input and out sizes differ")
    _abi.call(
        "aiter_amd_dynamic_per_group_quant_fp8",
        input.data_ptr(), AITER_DTYPE[input.dtype], rows, cols, group, out.data_ptr(),
        scales.data_ptr(), int(bool(shuffle_scale)), _ptr(num_rows), int(num_rows_factor),
        _stream_ptr(input))


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
