"""Synthetic MoE-layer workloads (the configurations the benchmarks and the
parity tests run), generated with seeded torch RNGs.

Routing follows the reference's helpers: softmax over N(0,1) logits, top-k,
renormalise (fused_topk, aiter/fused_moe.py:1853-1923, as the tuner seeds
it, csrc/ck_gemm_moe_2stages_codegen/gemm_moe_tune.py:560-592); sigmoid
scores + top-k + renormalise for the expert-parallel share
(aiter/ops/topk.py:116-157); a Zipf(s) popularity prior added to the logits
(log p_e, p_e ~ rank^-s over a seeded expert permutation) for skewed
prefill.  Weights are N(0, 0.02), quantised to fp8 e4m3fn with 128x128
block scales (or, for A8W4, to MXFP4 with e8m0 1x32 scales) and,
optionally, pre-shuffled to the (16,16) layout.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from .quant import per_1x32_f4_quant, quant_weight_per_128x128
from .shuffle import shuffle_weight


@dataclass
class MoEConfig:
    name: str
    tokens: int
    model_dim: int
    inter_dim: int
    experts: int
    topk: int
    routing: str = "softmax"        # softmax | zipf | sigmoid
    zipf_s: float = 1.1
    local_experts: Optional[int] = None  # EP share: experts held by this GPU
    seed: int = 0
    weights: str = "fp8"            # fp8 (128x128 blockscale) | mxfp4 (A8W4)
    extra: dict = field(default_factory=dict)


# BASELINE.json configs (one GPU)
CONFIG_A = MoEConfig("cpu_ref_A", 64, 1024, 512, 8, 2, seed=0)
MIMO = dict(model_dim=4096, inter_dim=2048, experts=256, topk=8)


def mimo_decode(tokens: int, seed: int = 1) -> MoEConfig:
    return MoEConfig(f"mimo_decode_T{tokens}", tokens, routing="softmax", seed=seed, **MIMO)


def mimo_prefill(tokens: int, seed: int = 5) -> MoEConfig:
    return MoEConfig(f"mimo_prefill_T{tokens}", tokens, routing="zipf", seed=seed, **MIMO)


def mimo_a8w4(tokens: int, seed: Optional[int] = None) -> MoEConfig:
    """A8W4 layer: uniform routing, seeds 6 / 7 / 8 for T = 32 / 1024 / 8192."""
    if seed is None:
        seed = {32: 6, 1024: 7, 8192: 8}.get(tokens, 6)
    return MoEConfig(f"mimo_a8w4_T{tokens}", tokens, routing="softmax", seed=seed,
                     weights="mxfp4", **MIMO)


def mimo_ep_share(tokens: int = 4096, seed: int = 9) -> MoEConfig:
    return MoEConfig(f"mimo_ep32_T{tokens}", tokens, routing="sigmoid", local_experts=32,
                     seed=seed, **MIMO)


def route(logits: torch.Tensor, topk: int, scoring: str = "softmax", renorm: bool = True):
    """(topk_weights f32 [T, k], topk_ids i32 [T, k]) from router logits."""
    logits = logits.float()
    scores = torch.softmax(logits, dim=-1) if scoring == "softmax" else torch.sigmoid(logits)
    w, ids = torch.topk(scores, topk, dim=-1)
    if renorm:
        w = w / w.sum(dim=-1, keepdim=True)
    return w.to(torch.float32).contiguous(), ids.to(torch.int32).contiguous()


def make_routing(cfg: MoEConfig, device="cpu"):
    g = torch.Generator(device="cpu").manual_seed(cfg.seed * 7919 + 17)
    logits = torch.randn(cfg.tokens, cfg.experts, generator=g)
    if cfg.routing == "zipf":
        perm = torch.randperm(cfg.experts, generator=g)
        ranks = torch.empty(cfg.experts)
        ranks[perm] = torch.arange(1, cfg.experts + 1, dtype=torch.float32)
        logits = logits + torch.log(ranks.pow(-cfg.zipf_s) / ranks.pow(-cfg.zipf_s).sum())
    scoring = "sigmoid" if cfg.routing == "sigmoid" else "softmax"
    w, ids = route(logits, cfg.topk, scoring)
    return w.to(device), ids.to(device)


def make_hidden(cfg: MoEConfig, device="cpu", dtype=torch.bfloat16):
    g = torch.Generator(device="cpu").manual_seed(cfg.seed * 7919 + 29)
    return torch.randn(cfg.tokens, cfg.model_dim, generator=g).to(dtype).to(device)


def make_expert_mask(cfg: MoEConfig, device="cpu"):
    """Contiguous block of local experts (expert-parallel rank 0's share)."""
    if cfg.local_experts is None:
        return None
    m = torch.zeros(cfg.experts, dtype=torch.int32)
    m[: cfg.local_experts] = 1
    return m.to(device)


def make_weights(cfg: MoEConfig, device="cpu", shuffle: bool = True, chunk: int = 8):
    """Quantised weights for the experts held locally.

    fp8 (cfg.weights == "fp8"): dict(w1, w1_scale, w2, w2_scale) with w1
    [E, 2I, H], w2 [E, H, I] fp8 and fp32 128x128 scales.  mxfp4: w1
    [E, 2I, H/2], w2 [E, H, I/2] packed e2m1 (uint8) and e8m0 scales (uint8)
    [E, 2I, H/32], [E, H, I/32].  Weights are optionally shuffled (carrying
    is_shuffled).  Generated `chunk` experts at a time on `device` with a
    per-chunk seeded generator, so large layers never hold their fp32
    weights at once; the fp32 draws are the same for both formats.
    """
    E = cfg.local_experts or cfg.experts
    H, I = cfg.model_dim, cfg.inter_dim
    dev = torch.device(device)
    if cfg.weights == "mxfp4":
        w1 = torch.empty(E, 2 * I, H // 2, dtype=torch.uint8, device=dev)
        w2 = torch.empty(E, H, I // 2, dtype=torch.uint8, device=dev)
        s1 = torch.empty(E, 2 * I, H // 32, dtype=torch.uint8, device=dev)
        s2 = torch.empty(E, H, I // 32, dtype=torch.uint8, device=dev)
        for c0 in range(0, E, chunk):
            c1 = min(E, c0 + chunk)
            g = torch.Generator(device=dev).manual_seed(cfg.seed * 104729 + c0)
            f1 = torch.randn(c1 - c0, 2 * I, H, generator=g, device=dev) * 0.02
            q1, sc1 = per_1x32_f4_quant(f1)
            del f1
            f2 = torch.randn(c1 - c0, H, I, generator=g, device=dev) * 0.02
            q2, sc2 = per_1x32_f4_quant(f2)
            del f2
            w1[c0:c1], s1[c0:c1] = q1.view(torch.uint8), sc1.view(torch.uint8)
            w2[c0:c1], s2[c0:c1] = q2.view(torch.uint8), sc2.view(torch.uint8)
        if shuffle:
            w1 = shuffle_weight(w1)
            w2 = shuffle_weight(w2)
        return {"w1": w1, "w1_scale": s1, "w2": w2, "w2_scale": s2}
    w1 = torch.empty(E, 2 * I, H, dtype=torch.float8_e4m3fn, device=dev)
    w2 = torch.empty(E, H, I, dtype=torch.float8_e4m3fn, device=dev)
    s1 = torch.empty(E, 2 * I // 128, H // 128, dtype=torch.float32, device=dev)
    s2 = torch.empty(E, H // 128, I // 128, dtype=torch.float32, device=dev)
    for c0 in range(0, E, chunk):
        c1 = min(E, c0 + chunk)
        g = torch.Generator(device=dev).manual_seed(cfg.seed * 104729 + c0)
        f1 = torch.randn(c1 - c0, 2 * I, H, generator=g, device=dev) * 0.02
        q1, sc1 = quant_weight_per_128x128(f1)
        del f1
        f2 = torch.randn(c1 - c0, H, I, generator=g, device=dev) * 0.02
        q2, sc2 = quant_weight_per_128x128(f2)
        del f2
        w1[c0:c1], s1[c0:c1], w2[c0:c1], s2[c0:c1] = q1, sc1, q2, sc2
    if shuffle:
        w1 = shuffle_weight(w1)
        w2 = shuffle_weight(w2)
    return {"w1": w1, "w1_scale": s1, "w2": w2, "w2_scale": s2}


def layer_flops(cfg: MoEConfig, pairs: Optional[int] = None) -> float:
    """Algorithmic FLOPs: 2 * pairs * (2I*H + H*I) (gemm_moe_tune.py:1399-1468)."""
    p = cfg.tokens * cfg.topk if pairs is None else pairs
    return 2.0 * p * (2 * cfg.inter_dim * cfg.model_dim + cfg.model_dim * cfg.inter_dim)


def expert_bytes_fp8(cfg: MoEConfig) -> int:
    """fp8 weights + fp32 block scales of one expert."""
    H, I = cfg.model_dim, cfg.inter_dim
    return 2 * I * H + H * I + 4 * ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128))


def expert_bytes_a8w4(cfg: MoEConfig) -> int:
    """Packed e2m1 weights + e8m0 1x32 scales of one expert."""
    H, I = cfg.model_dim, cfg.inter_dim
    return (2 * I * H + H * I) // 2 + (2 * I * H + H * I) // 32


def expert_bytes(cfg: MoEConfig) -> int:
    return expert_bytes_a8w4(cfg) if cfg.weights == "mxfp4" else expert_bytes_fp8(cfg)


def layer_bytes(cfg: MoEConfig, distinct_experts: int, tokens: Optional[int] = None) -> float:
    """Algorithmic HBM bytes: touched experts' weights + x (bf16) + out (bf16)
    + routing ids/weights (4 B each per slot)."""
    T = cfg.tokens if tokens is None else tokens
    return float(distinct_experts * expert_bytes(cfg) +
                 T * (cfg.model_dim * 2 + cfg.model_dim * 2 + 8 * cfg.topk))


def run_layer(weights: str, hidden_states, w1, w2, topk_weight, topk_ids, **kw):
    """One MoE layer of the given weight format: fused_moe with the FP8
    128x128 blockscale quant type, or, for "mxfp4", fused_moe_a8w4 (fp8
    activations x MXFP4 weights); keyword arguments go through unchanged."""
    from .enums import QuantType
    from .fused_moe import fused_moe, fused_moe_a8w4

    if weights == "mxfp4":
        return fused_moe_a8w4(hidden_states, w1, w2, topk_weight, topk_ids, **kw)
    return fused_moe(hidden_states, w1, w2, topk_weight, topk_ids,
                     quant_type=QuantType.per_128x128, **kw)
