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


# ---- the reference's layouts for its Swiglu fp4 kernels (a16w4) ---------
# aiter/ops/shuffle.py:51-113 (shuffle_weight_a16w4 / shuffle_scale_a16w4);
# op_tests/test_moe_2stage.py:167-175 packs per_1x32 fp4x2 weights this way
# for bf16 and fp8 activations. The GEMMs here read row-major or (16, 16)
# weights and row-major or e8m0_shuffle'd scales, so checkpoints packed this
# way are converted once at load time with the unshuffle_* functions below.
#
# Weight byte (e, n, k) of an [E, N, K/2] fp4x2 tensor, with KLane = 64 /
# NLane, KPack = 16, n = half * N/2 + n0 * NLane + nl (gate_up; half = 0
# gate, 1 up) or n0 * NLane + nl, and k = (k0 * KLane + kl) * KPack + kp,
# lands at [n0][half][k0][kl][nl][kp] of its expert (no half index without
# gate_up).
# Scale byte (e, n, k) of the 2-D [E * N, K/32] e8m0 array, with
# n = np * N/2 + n1 * 16 + nl (gate_up) or n1 * 32 + np * 16 + nl, and
# k = (k1 * 2 + kk) * 4 + kl, lands at [n1][k1][kl][nl][kk][np] of its expert.
def _a16w4_weight_dims(shape, NLane: int, gate_up: bool):
    if len(shape) != 3:
        raise ValueError(f"a16w4 weights are [E, N, K/2], got {tuple(shape)}")
    E, N, Kp = shape
    KLane, KPack = 64 // NLane, 16
    h = N // 2 if gate_up else N
    if NLane <= 0 or 64 % NLane or h % NLane or Kp % (KLane * KPack) or (gate_up and N % 2):
        raise ValueError(f"a16w4 weight shape {tuple(shape)} does not tile by NLane={NLane}")
    N0, K0 = h // NLane, Kp // (KLane * KPack)
    if gate_up:
        return (E, 2, N0, NLane, K0, KLane, KPack), (0, 2, 1, 4, 5, 3, 6)
    return (E, N0, NLane, K0, KLane, KPack), (0, 1, 3, 4, 2, 5)


def _inverse(perm):
    inv = [0] * len(perm)
    for i, p in enumerate(perm):
        inv[p] = i
    return tuple(inv)


def _bytes(x: torch.Tensor) -> torch.Tensor:
    return x.view(torch.uint8) if x.element_size() == 1 else x


def shuffle_weight_a16w4(src: torch.Tensor, NLane: int, gate_up: bool) -> torch.Tensor:
    """Row-major [E, N, K/2] fp4x2 -> the reference's a16w4 weight layout."""
    dims, perm = _a16w4_weight_dims(src.shape, NLane, gate_up)
    y = _bytes(src).reshape(dims).permute(perm).contiguous()
    return y.view(src.shape).view(src.dtype)


def unshuffle_weight_a16w4(src: torch.Tensor, NLane: int, gate_up: bool) -> torch.Tensor:
    """The reference's a16w4 weight layout -> row-major [E, N, K/2]."""
    dims, perm = _a16w4_weight_dims(src.shape, NLane, gate_up)
    packed = tuple(dims[p] for p in perm)
    y = _bytes(src).reshape(packed).permute(_inverse(perm)).contiguous()
    return y.view(src.shape).view(src.dtype)


def _a16w4_scale_dims(shape, experts_cnt: int, gate_up: bool):
    if len(shape) != 2 or experts_cnt <= 0 or shape[0] % experts_cnt:
        raise ValueError(f"a16w4 scales are [E * N, K/32], got {tuple(shape)}")
    n, k = shape[0] // experts_cnt, shape[1]
    if n % 32 or k % 8:
        raise ValueError(f"a16w4 scale shape {tuple(shape)}: N % 32 and K/32 % 8 must be 0")
    N1, K1 = n // 32, k // 8
    if gate_up:
        return (experts_cnt, 2, N1, 16, K1, 2, 4), (0, 2, 4, 6, 3, 5, 1)
    return (experts_cnt, N1, 2, 16, K1, 2, 4), (0, 1, 4, 6, 3, 5, 2)


def shuffle_scale_a16w4(src: torch.Tensor, experts_cnt: int, gate_up: bool) -> torch.Tensor:
    """Row-major [E * N, K/32] e8m0 -> the reference's a16w4 scale layout."""
    dims, perm = _a16w4_scale_dims(src.shape, experts_cnt, gate_up)
    y = _bytes(src).reshape(dims).permute(perm).contiguous()
    return y.view(src.shape).view(src.dtype)


def unshuffle_scale_a16w4(src: torch.Tensor, experts_cnt: int, gate_up: bool) -> torch.Tensor:
    """The reference's a16w4 scale layout -> row-major [E * N, K/32] (view it
    as [E, N, K/32] for fused_moe)."""
    dims, perm = _a16w4_scale_dims(src.shape, experts_cnt, gate_up)
    packed = tuple(dims[p] for p in perm)
    y = _bytes(src).reshape(packed).permute(_inverse(perm)).contiguous()
    return y.view(src.shape).view(src.dtype)
