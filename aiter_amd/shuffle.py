"""Weight pre-shuffle: the reference's (16, 16) layout for 8-bit weights.

Same contract as aiter/ops/shuffle.py:7-27 (shuffle_weight): an [.., N, K]
byte tensor is viewed as [-1, N/16, 16, K/32, 2, 16] and permuted to
[-1, N/16, K/32, 2, 16, 16], i.e. for every 16-row group and every 32-byte
K chunk, the 16 rows' first 16 bytes then the 16 rows' next 16 bytes.  The
result carries `is_shuffled = True`, which fused_moe reads.  The GEMM
kernels copy each 16-row x 128-K block of this layout verbatim into LDS.
"""
from __future__ import annotations

import torch


def shuffle_weight(x: torch.Tensor, layout=(16, 16), use_int4: bool = False) -> torch.Tensor:
    if use_int4:
        raise NotImplementedError("int4 weights are not supported")
    if tuple(layout) != (16, 16):
        raise NotImplementedError(f"layout {layout} is not supported, only (16, 16)")
    x_type = x.dtype
    xb = x.view(torch.uint8) if x.element_size() == 1 else x
    if xb.element_size() != 1:
        raise NotImplementedError("only 8-bit (fp8 / packed fp4) weights are supported")
    n, k = xb.shape[-2], xb.shape[-1]
    if n % 16 or k % 32:
        raise ValueError(f"weight shape {tuple(xb.shape)} must have N % 16 == 0, K % 32 == 0")
    y = xb.reshape(-1, n // 16, 16, k // 32, 2, 16).permute(0, 1, 3, 4, 2, 5).contiguous()
    y = y.view(*x.shape[:-2], n, k).view(x_type)
    y.is_shuffled = True
    return y


def unshuffle_weight(x: torch.Tensor) -> torch.Tensor:
    """Inverse of shuffle_weight (for checks and checkpoint export)."""
    x_type = x.dtype
    xb = x.view(torch.uint8)
    n, k = xb.shape[-2], xb.shape[-1]
    y = xb.reshape(-1, n // 16, k // 32, 2, 16, 16).permute(0, 1, 4, 2, 3, 5).contiguous()
    return y.view(*x.shape[:-2], n, k).view(x_type)
