"""PyTorch-CPU restatement of the reference's torch MoE path -- TEST
INFRASTRUCTURE ONLY (the CPU baseline and its checks).

Only tests/ and bench.py's cpu_baseline leg import this module; the
aiter_amd package never calls it.

fused_moe_torch follows the op sequence of the reference's own torch
oracle for the FP8 blockscale layer (aiter/fused_moe.py:1483-1666,
torch_moe_stage1 / torch_moe_stage2 with quant_type per_1x128, as
op_tests/test_moe_2stage.py:187-231 chains them), in torch on whatever
device its tensors live on (the CPU for the baseline):
  1. the fp8 weights dequantised with their 128x128 fp32 scales;
  2. the activations quantised 1x128 with pertoken_quant semantics
     (aiter/ops/quant.py:42-72: scale = amax / 448, codes = the fp8 cast of
     x / scale) and dequantised;
  3. per expert: stage-1 fp32 matmul, silu(gate) * up (or gelu), bf16,
     1x128 requant and dequant, stage-2 fp32 matmul;
  4. the routing weights, the sum over the top-k slots, bf16.
tests/test_oracle.py pins it against oracle.moe_ref.fused_moe_ref with
act_quant='torch' (the same semantics in numpy).
"""
from __future__ import annotations

import torch

FP8_MAX = 448.0


def pertoken_quant_1x128(x: torch.Tensor):
    """(codes fp8 [rows, K], scales f32 [rows, K/128]): aiter/ops/quant.py:42-72
    with group size 128 and fp8 e4m3fn output."""
    rows, K = x.shape
    g = x.float().view(rows, K // 128, 128)
    amax = g.abs().amax(dim=-1, keepdim=True)
    scale = amax / FP8_MAX
    scale = torch.where(scale == 0, torch.ones_like(scale), scale)   # an all-zero group
    q = (g / scale).to(torch.float8_e4m3fn)
    return q.view(rows, K), scale.view(rows, K // 128)


def dequant_1x128(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    rows, K = q.shape
    return (q.float().view(rows, K // 128, 128) * scale.view(rows, K // 128, 1)).view(rows, K)


def dequant_weight_128x128(wq: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    """[E, N, K] fp8 codes with [E, N/128, K/128] scales -> fp32 [E, N, K]."""
    E, N, K = wq.shape
    return (wq.float().view(E, N // 128, 128, K // 128, 128) *
            ws.view(E, N // 128, 1, K // 128, 1)).view(E, N, K)


def fused_moe_torch(x: torch.Tensor, w1q: torch.Tensor, w1s: torch.Tensor, w2q: torch.Tensor,
                    w2s: torch.Tensor, topk_ids: torch.Tensor, topk_w: torch.Tensor,
                    activation: str = "silu") -> torch.Tensor:
    """The layer: x bf16 [T, H]; w1q fp8 [E, 2I, H] + w1s [E, 2I/128, H/128];
    w2q fp8 [E, H, I] + w2s [E, H/128, I/128]; topk_ids [T, k], topk_w
    [T, k]. Returns bf16 [T, H]."""
    T, H = x.shape
    k = topk_ids.shape[1]
    w1 = dequant_weight_128x128(w1q, w1s)
    w2 = dequant_weight_128x128(w2q, w2s)
    inter = w2.shape[2]
    a1q, a1s = pertoken_quant_1x128(x)
    a1 = dequant_1x128(a1q, a1s)
    act = torch.nn.functional.gelu if activation == "gelu" else torch.nn.functional.silu
    h = torch.zeros(T, k, inter)
    for e in torch.unique(topk_ids).tolist():
        tok, slot = torch.nonzero(topk_ids == e, as_tuple=True)
        y = a1[tok] @ w1[e].T
        h[tok, slot] = (act(y[:, :inter]) * y[:, inter:]).to(torch.bfloat16).float()
    a2q, a2s = pertoken_quant_1x128(h.view(T * k, inter))
    a2 = dequant_1x128(a2q, a2s).view(T, k, inter)
    out = torch.zeros(T, k, H)
    for e in torch.unique(topk_ids).tolist():
        tok, slot = torch.nonzero(topk_ids == e, as_tuple=True)
        out[tok, slot] = a2[tok, slot] @ w2[e].T
    return (out * topk_w.float()[..., None]).sum(dim=1).to(torch.bfloat16)
