"""Pins the torch checker of the full-size GPU tests (tests/_fullshape.py:
TorchChain, torch_layer_ref) against the numpy oracle, on the CPU.

Both state the same layer (torch_moe_stage1/2 semantics,
aiter/fused_moe.py:1483-1666) in fp32 with different summation orders, so:
* the 1x128 activation quant is bit-equal;
* stage 1's requantised fp8 codes are equal except where a bf16 rounding tie
  of act(gate)*up falls the other way (at most 0.5%, never more than one
  e4m3 step);
* stage 2 fed the oracle's own a2 agrees to fp32 ordering (normalised
  max-rel <= 4e-3, one bf16 ulp, and RMS-rel <= 1e-3);
* the whole chain meets RMS-rel <= 1e-3 against the oracle's output.
A chain with gate and up swapped fails the stage-1 bar, so the checker
would see that mistake in a kernel.
"""
import numpy as np
import pytest
import torch

from aiter_amd import workloads as W
from oracle import moe_ref as R

import _fullshape as F


def _signed_step(c):
    c = c.astype(np.int32)
    return np.where(c & 0x80, -(c & 0x7F), c & 0x7F)


@pytest.mark.parametrize("cfg", [
    W.CONFIG_A,
    W.MoEConfig("pin_k8", 48, 512, 256, 16, 8, seed=61),
    W.MoEConfig("pin_mx", 40, 512, 256, 8, 2, seed=62, weights="mxfp4"),
])
def test_torch_chain_matches_the_oracle(cfg):
    mx4 = cfg.weights == "mxfp4"
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    x = W.make_hidden(cfg)
    tw, ids = W.make_routing(cfg)
    w1, s1, w2, s2 = wts["w1"], wts["w1_scale"], wts["w2"], wts["w2_scale"]
    as_np = (lambda t: t.numpy()) if mx4 else (lambda t: t.view(torch.uint8).numpy())
    ref = R.fused_moe_ref(x.float().numpy(), as_np(w1), s1.numpy(), as_np(w2), s2.numpy(),
                          ids.numpy(), tw.numpy(), weight_format="mxfp4" if mx4 else
                          "fp8_128x128")
    deq = F.deq_mxfp4 if mx4 else F.deq_fp8_128x128
    chain = F.TorchChain(w1, s1, w2, s2, ids, tw, deq)
    T, k, I = cfg.tokens, cfg.topk, cfg.inter_dim

    a1q, a1s = F.q1x128(x)
    assert np.array_equal(a1q.view(torch.uint8).numpy(), ref["a1q"])
    assert np.array_equal(a1s.numpy().view(np.int32), ref["a1s"].view(np.int32))

    q, sc = chain.stage1(F.deq1x128(a1q, a1s))
    codes = q.view(torch.uint8).numpy().reshape(T, k, I)
    differ = (codes != ref["a2q"]).mean()
    assert differ <= 0.005, differ
    assert np.abs(_signed_step(codes) - _signed_step(ref["a2q"])).max() <= 1

    a2_oracle = torch.from_numpy(R.dequant_1x128(ref["a2q"].reshape(T * k, I),
                                                 ref["a2s"].reshape(T * k, -1)))
    out2 = chain.stage2(a2_oracle).to(torch.bfloat16).float().numpy()
    mx, rms = R.normalized_errors(ref["out"], out2)
    assert mx <= 4e-3 and rms <= 1e-3, (mx, rms)

    out = F.torch_layer_ref(x, w1, s1, w2, s2, ids, tw, deq).numpy()
    mx, rms = R.normalized_errors(ref["out"], out)
    assert rms <= 1e-3, (mx, rms)


def test_a_swapped_gate_and_up_fails_the_stage1_bar():
    cfg = W.CONFIG_A
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    x = W.make_hidden(cfg)
    tw, ids = W.make_routing(cfg)
    ref = R.fused_moe_ref(x.float().numpy(), wts["w1"].view(torch.uint8).numpy(),
                          wts["w1_scale"].numpy(), wts["w2"].view(torch.uint8).numpy(),
                          wts["w2_scale"].numpy(), ids.numpy(), tw.numpy())
    I = cfg.inter_dim
    # the planted mistake: gate and up rows (and their scale blocks) exchanged
    w1 = torch.cat([wts["w1"][:, I:], wts["w1"][:, :I]], dim=1)
    s1 = torch.cat([wts["w1_scale"][:, I // 128:], wts["w1_scale"][:, :I // 128]], dim=1)
    chain = F.TorchChain(w1, s1, wts["w2"], wts["w2_scale"], ids, tw)
    a1q, a1s = F.q1x128(x)
    q, _ = chain.stage1(F.deq1x128(a1q, a1s))
    differ = (q.view(torch.uint8).numpy().reshape(ref["a2q"].shape) != ref["a2q"]).mean()
    assert differ > 0.5
