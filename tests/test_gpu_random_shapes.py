"""Seeded random layer shapes against the CPU oracle (through the C ABI).

Each case draws a token count, expert count, top-k, model and intermediate
dims (multiples of 128; model_dim 384 and 640 send stage 2 to the general
kernels, inter_dim 640 gives an odd K-step count), a block size (or the
default), shuffled or row-major weights, FP8 blockscale or MXFP4 weights,
softmax or sigmoid routing, and sometimes an expert mask, then checks the
layer against the oracle at the reference tests' bar (max-rel <= 2e-2,
RMS-rel <= 4e-3, op_tests/triton_tests/moe/test_moe_gemm_a8w4.py:104-160).
With few routed pairs one fp8 requant tie -- a SiLU*up value that the GPU
and the oracle, summing stage 1 in different orders, round to neighbouring
e4m3 codes -- can move a dominant output element by a few per cent. A case
that misses the end-to-end bar must then pass the per-stage check of the
full-size tests (tests/_fullshape.stagewise_vs_oracle): at most 0.5% of
stage 1's codes differ from the oracle's, each by at most one top-binade
step, and the output meets the strict bar against the oracle's stage 2 on
the kernel's own a2."""
import os
import random

import numpy as np
import pytest
import torch

import aiter_amd as A
from aiter_amd import workloads as W
from oracle import moe_ref as R

import _fullshape

pytestmark = pytest.mark.gpu


def _case(seed):
    rnd = random.Random(seed)
    E = rnd.choice([4, 8, 16, 33])
    k = rnd.randint(1, min(8, E))
    H = rnd.choice([256, 384, 512, 640, 1024])
    I = rnd.choice([512, 640, 768, 1024])
    T = rnd.choice([1, 3, 17, 64, 129, 300])
    bm = rnd.choice([None, 16, 32, 64, 128])
    if bm == 128 and H % 256:
        bm = 64
    weights = rnd.choice(["fp8", "mxfp4"])
    shuffle = rnd.random() < 0.7
    routing = rnd.choice(["softmax", "sigmoid"])
    local = rnd.choice([None, None, max(1, E // 2)])
    return dict(T=T, E=E, k=k, H=H, I=I, bm=bm, weights=weights, shuffle=shuffle,
                routing=routing, local=local)


def _seeds(base, n=16):
    """n seeds from base; AITER_AMD_RANDOM_CASES sets n for a longer sweep."""
    env = os.environ.get("AITER_AMD_RANDOM_CASES")
    return list(range(base, base + (int(env) if env else n)))


CASES = _seeds(1000)


@pytest.mark.parametrize("seed", CASES)
def test_random_layer_vs_oracle(cuda_device, seed):
    c = _case(seed)
    print(f"[random shape {seed}] {c}", flush=True)
    cfg = W.MoEConfig(f"rand{seed}", c["T"], c["H"], c["I"], c["E"], c["k"],
                      routing=c["routing"], local_experts=c["local"], seed=seed,
                      weights=c["weights"])
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    x = W.make_hidden(cfg)
    tw, ids = W.make_routing(cfg)
    mask = W.make_expert_mask(cfg)
    mx4 = c["weights"] == "mxfp4"
    w1n = wts["w1"].view(torch.uint8).numpy()
    w2n = wts["w2"].view(torch.uint8).numpy()
    ref = R.fused_moe_ref(x.float().numpy(), w1n, wts["w1_scale"].numpy(), w2n,
                          wts["w2_scale"].numpy(), ids.numpy(), tw.numpy(),
                          None if mask is None else mask.numpy(),
                          **({"weight_format": "mxfp4"} if mx4 else {}))
    w1, w2 = wts["w1"], wts["w2"]
    if c["shuffle"]:
        w1, w2 = A.shuffle_weight(w1), A.shuffle_weight(w2)
    w1, w2 = w1.to(cuda_device), w2.to(cuda_device)
    if c["shuffle"]:
        w1.is_shuffled = True
        w2.is_shuffled = True
    dev = dict(x=x.to(cuda_device), w1=w1, w2=w2, s1=wts["w1_scale"].to(cuda_device),
               s2=wts["w2_scale"].to(cuda_device), tw=tw.to(cuda_device), ids=ids.to(cuda_device),
               mask=None if mask is None else mask.to(cuda_device))
    out = W.run_layer(c["weights"], dev["x"], w1, w2, dev["tw"], dev["ids"],
                      expert_mask=dev["mask"], w1_scale=dev["s1"], w2_scale=dev["s2"],
                      block_size_M=c["bm"])
    got = out.float().cpu().numpy()
    mx, rms = R.normalized_errors(ref["out"], got)
    print(f"[random shape {seed}] max-rel {mx:.3e} rms-rel {rms:.3e}", flush=True)
    assert np.isfinite(got).all()
    if not (mx <= R.MAXTOL and rms <= R.RMSTOL):
        bm = c["bm"] or A.select_block_m(c["T"], c["k"], cfg.local_experts or c["E"], c["H"],
                                         c["I"], c["weights"] == "mxfp4", cuda_device)
        # the per-stage bar; the end-to-end RMS is left out only for layers of
        # under 32 routed pairs, where one flipped code dominates it
        pairs = int((ref["ids_local"] >= 0).sum())
        _fullshape.stagewise_vs_oracle(cfg, dev, ref, got, bm, A.ActivationType.Silu,
                                       log=lambda m: print(m, flush=True),
                                       e2e_rms=pairs >= 32)
    if mask is not None:
        none_local = (ref["ids_local"] < 0).all(axis=1)
        assert np.count_nonzero(got[none_local]) == 0


def _variant(seed):
    rnd = random.Random(seed)
    c = _case(seed)
    c["E"] = rnd.choice([8, 16, 33, 64])
    c["k"] = rnd.randint(1, min(16, c["E"]))
    c["T"] = rnd.choice([2, 40, 257, 600])
    c["local"] = rnd.choice([None, max(1, c["E"] // 4)])
    c["doweight"] = rnd.random() < 0.4
    c["gelu"] = rnd.random() < 0.4
    c["fp16"] = rnd.random() < 0.3
    c["num_local"] = rnd.choice([None, None, max(1, (3 * c["T"]) // 4)])
    return c


VARIANTS = _seeds(2000)


@pytest.mark.parametrize("seed", VARIANTS)
def test_random_layer_variants_vs_oracle(cuda_device, seed):
    """As above with doweight_stage1, Gelu, fp16 in/out, num_local_tokens
    (outputs past the local rows are not compared), topk up to 16, up to 64
    experts and token counts of several sorting chunks."""
    c = _variant(seed)
    print(f"[random variant {seed}] {c}", flush=True)
    cfg = W.MoEConfig(f"randv{seed}", c["T"], c["H"], c["I"], c["E"], c["k"],
                      routing=c["routing"], local_experts=c["local"], seed=seed,
                      weights=c["weights"])
    act = "gelu" if c["gelu"] else "silu"
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    x = W.make_hidden(cfg)
    tw, ids = W.make_routing(cfg)
    mask = W.make_expert_mask(cfg)
    mx4 = c["weights"] == "mxfp4"
    ref = R.fused_moe_ref(x.float().numpy(), wts["w1"].view(torch.uint8).numpy(),
                          wts["w1_scale"].numpy(), wts["w2"].view(torch.uint8).numpy(),
                          wts["w2_scale"].numpy(), ids.numpy(), tw.numpy(),
                          None if mask is None else mask.numpy(),
                          doweight_stage1=c["doweight"], activation=act,
                          num_local_tokens=c["num_local"],
                          **({"weight_format": "mxfp4"} if mx4 else {}))
    w1, w2 = wts["w1"], wts["w2"]
    if c["shuffle"]:
        w1, w2 = A.shuffle_weight(w1), A.shuffle_weight(w2)
    w1, w2 = w1.to(cuda_device), w2.to(cuda_device)
    if c["shuffle"]:
        w1.is_shuffled = True
        w2.is_shuffled = True
    xd = x.to(cuda_device)
    if c["fp16"]:
        xd = xd.to(torch.float16)        # N(0,1) bf16 values are exact in fp16
    dev = dict(x=xd, w1=w1, w2=w2, s1=wts["w1_scale"].to(cuda_device),
               s2=wts["w2_scale"].to(cuda_device), tw=tw.to(cuda_device), ids=ids.to(cuda_device),
               mask=None if mask is None else mask.to(cuda_device))
    nl = None
    if c["num_local"] is not None:
        nl = torch.tensor([c["num_local"]], dtype=torch.int32, device=cuda_device)
    out = W.run_layer(c["weights"], dev["x"], w1, w2, dev["tw"], dev["ids"],
                      expert_mask=dev["mask"], w1_scale=dev["s1"], w2_scale=dev["s2"],
                      block_size_M=c["bm"], doweight_stage1=c["doweight"],
                      activation=A.ActivationType.Gelu if c["gelu"] else A.ActivationType.Silu,
                      num_local_tokens=nl)
    assert out.dtype == (torch.float16 if c["fp16"] else torch.bfloat16)
    rows = c["num_local"] if c["num_local"] is not None else c["T"]
    got = out.float().cpu().numpy()
    assert np.isfinite(got[:rows]).all()
    mx, rms = R.normalized_errors(ref["out"][:rows], got[:rows])
    print(f"[random variant {seed}] max-rel {mx:.3e} rms-rel {rms:.3e}", flush=True)
    if not (mx <= R.MAXTOL and rms <= R.RMSTOL):
        got[rows:] = 0
        ref["ids_local"][rows:] = -1
        bm = c["bm"] or A.select_block_m(c["T"], c["k"], cfg.local_experts or c["E"], c["H"],
                                         c["I"], mx4, cuda_device)
        pairs = int((ref["ids_local"] >= 0).sum())
        _fullshape.stagewise_vs_oracle(
            cfg, dev, ref, got, bm,
            A.ActivationType.Gelu if c["gelu"] else A.ActivationType.Silu,
            doweight=c["doweight"], log=lambda m: print(m, flush=True), e2e_rms=pairs >= 32)
