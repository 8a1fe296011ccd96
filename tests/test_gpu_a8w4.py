"""GPU parity of the A8W4 path (fp8 1x128 activations x MXFP4 weights,
quant_type per_1x32) against the CPU oracle, through the C ABI.

Same bar as the FP8 blockscale path: the oracle is the reference's
torch_moe_stage1/2 with the per_1x32 weight dequant
(aiter/fused_moe.py:1539-1553, 1635-1649) and 1x128 activation quant;
outputs agree within max-rel <= 2e-2, RMS-rel <= 4e-3
(op_tests/triton_tests/moe/test_moe_gemm_a8w4.py:104-160).
"""
import dataclasses

import numpy as np
import pytest
import torch

import aiter_amd as A
from aiter_amd import workloads as W
from oracle import moe_ref as R

import _fullshape

pytestmark = pytest.mark.gpu

MAXTOL, RMSTOL = R.MAXTOL, R.RMSTOL


def _np(t):
    return t.detach().cpu().numpy()


def _a8w4(cfg):
    return dataclasses.replace(cfg, weights="mxfp4")


def _make_layer(cfg, device, shuffle, doweight=False, activation="silu"):
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    x = W.make_hidden(cfg)
    tw, ids = W.make_routing(cfg)
    mask = W.make_expert_mask(cfg)
    ref = R.fused_moe_ref(x.float().numpy(), wts["w1"].numpy(), wts["w1_scale"].numpy(),
                          wts["w2"].numpy(), wts["w2_scale"].numpy(), ids.numpy(), tw.numpy(),
                          None if mask is None else mask.numpy(), weight_format="mxfp4",
                          doweight_stage1=doweight, activation=activation)
    w1, w2 = wts["w1"], wts["w2"]
    if shuffle:
        w1, w2 = A.shuffle_weight(w1), A.shuffle_weight(w2)
    dev = dict(x=x.to(device), w1=w1.to(device), w2=w2.to(device),
               s1=wts["w1_scale"].to(device), s2=wts["w2_scale"].to(device), tw=tw.to(device),
               ids=ids.to(device), mask=None if mask is None else mask.to(device))
    if shuffle:
        dev["w1"].is_shuffled = True
        dev["w2"].is_shuffled = True
    return dev, ref


def _run(dev, **kw):
    return A.fused_moe_a8w4(dev["x"], dev["w1"], dev["w2"], dev["tw"], dev["ids"],
                            expert_mask=dev["mask"], w1_scale=dev["s1"], w2_scale=dev["s2"], **kw)


def _check(ref_out, got, tag):
    mx, rms = R.normalized_errors(ref_out, got)
    print(f"[{tag}] max-rel {mx:.3e} rms-rel {rms:.3e}", flush=True)
    assert mx <= MAXTOL and rms <= RMSTOL, (mx, rms)


@pytest.mark.parametrize("shuffle", [True, False])
@pytest.mark.parametrize("bm", [16, 32, 64, 128])
def test_a8w4_config_a(cuda_device, shuffle, bm):
    cfg = _a8w4(W.CONFIG_A)
    dev, ref = _make_layer(cfg, cuda_device, shuffle)
    out = _run(dev, block_size_M=bm)
    assert out.dtype == torch.bfloat16 and out.shape == (cfg.tokens, cfg.model_dim)
    _check(ref["out"], _np(out.float()), f"A8W4 A shuffle={shuffle} bm={bm}")


@pytest.mark.parametrize("bm", [16, 64, 128])
@pytest.mark.parametrize("T", [32, 512])
def test_a8w4_doweight_stage1(cuda_device, bm, T):
    """doweight_stage1 on the A8W4 layer: the stream (bm 16) and, at bm
    64/128, the direct-to-LDS (T=32, 8 routed rows per expert) or prefill
    (T=512, 128) stage-1 kernels; stage 2 unweighted."""
    cfg = dataclasses.replace(_a8w4(W.CONFIG_A), tokens=T)
    dev, ref = _make_layer(cfg, cuda_device, True, doweight=True)
    out = _run(dev, block_size_M=bm, doweight_stage1=True)
    _check(ref["out"], _np(out.float()), f"A8W4 doweight_stage1 T={T} bm={bm}")


@pytest.mark.parametrize("bm", [16, 128])
@pytest.mark.parametrize("T", [32, 64, 512])
def test_a8w4_gelu(cuda_device, bm, T):
    """ActivationType.Gelu on the A8W4 stage-1 kernels (stream at bm 16; at
    bm 128 direct-to-LDS at T=32, prefill at T=64 and 512). At T=64 one a2
    value sits on an fp8 requant tie whose one-step flip moves a small output
    3% (normalised) from the oracle's, so the check is split at the stage
    boundary."""
    cfg = dataclasses.replace(_a8w4(W.CONFIG_A), tokens=T)
    dev, ref = _make_layer(cfg, cuda_device, True, activation="gelu")
    out = _run(dev, block_size_M=bm, activation=A.ActivationType.Gelu)
    _fullshape.stagewise_vs_oracle(cfg, dev, ref, _np(out.float()), bm, A.ActivationType.Gelu)


def test_a8w4_torch_dtypes_match_byte_views(cuda_device):
    """fp4x2 / e8m0 tensors and their uint8 views give the same bits."""
    cfg = _a8w4(W.CONFIG_A)
    dev, _ = _make_layer(cfg, cuda_device, True)
    out_u8 = _run(dev)
    typed = dict(dev)
    typed["w1"] = dev["w1"].view(A.dtypes.fp4x2)
    typed["w2"] = dev["w2"].view(A.dtypes.fp4x2)
    typed["w1"].is_shuffled = typed["w2"].is_shuffled = True
    typed["s1"] = dev["s1"].view(A.dtypes.fp8_e8m0)
    typed["s2"] = dev["s2"].view(A.dtypes.fp8_e8m0)
    out_typed = _run(typed)
    # same kernels, same inputs: equal up to the f32 atomic order of stage 2
    mx, rms = R.normalized_errors(_np(out_u8.float()), _np(out_typed.float()))
    assert mx <= 1e-2 and rms <= 1e-3


@pytest.mark.parametrize("bm", [64, 128])
@pytest.mark.parametrize("T", [512, 96, 48])
def test_a8w4_prefill_shape(cuda_device, bm, T):
    """Large M-blocks with K > 1 pipeline depth. The experts average 128
    routed rows at T=512 (both stages on the prefill kernels, the tile's
    e8m0 bytes in LDS), 24 at T=96 (stage 1 prefill, stage 2 direct-to-LDS
    at 64 rows) and 12 at T=48 (both direct-to-LDS at 64 rows); stage 2 at
    128 rows is always the prefill kernel."""
    cfg = W.MoEConfig("a8w4_prefill", T, 1024, 512, 8, 2, seed=11, weights="mxfp4")
    dev, ref = _make_layer(cfg, cuda_device, True)
    _check(ref["out"], _np(_run(dev, block_size_M=bm).float()), f"A8W4 T={T} bm={bm}")


def test_a8w4_fp8_input_path(cuda_device):
    cfg = _a8w4(W.CONFIG_A)
    dev, ref = _make_layer(cfg, cuda_device, True)
    a1, a1s = A.per_group_quant_hip(dev["x"])
    out = A.fused_moe_a8w4(a1, dev["w1"], dev["w2"], dev["tw"], dev["ids"],
                           w1_scale=dev["s1"], w2_scale=dev["s2"], a1_scale=a1s,
                           dtype=torch.bfloat16)
    _check(ref["out"], _np(out.float()), "A8W4 fp8 input")


def test_a8w4_ep_share_small(cuda_device):
    cfg = W.MoEConfig("a8w4_ep", 96, 512, 512, 16, 4, routing="sigmoid", local_experts=4,
                      seed=3, weights="mxfp4")
    dev, ref = _make_layer(cfg, cuda_device, False)
    out = _run(dev)
    _check(ref["out"], _np(out.float()), "A8W4 EP small")
    none_local = (ref["ids_local"] < 0).all(axis=1)
    assert none_local.any()
    assert torch.count_nonzero(out[torch.from_numpy(none_local).to(cuda_device)]).item() == 0


# ------------------------------------------- full MiMo shape (decode) ---

def _torch_ref_gpu(x, w1, s1, w2, s2, ids, tw, inter):
    """Plain torch fp32 reference on the GPU with the LUT dequant of the MXFP4
    weights (tests/_fullshape.TorchChain)."""
    return _fullshape.torch_layer_ref(x, w1, s1, w2, s2, ids, tw, _fullshape.deq_mxfp4)


def test_a8w4_mimo_decode_T32(cuda_device):
    cfg = W.mimo_a8w4(32)
    wts = W.make_weights(cfg, device=cuda_device, shuffle=False)
    x = W.make_hidden(cfg, device=cuda_device)
    tw, ids = W.make_routing(cfg, device=cuda_device)
    ref = _torch_ref_gpu(x, wts["w1"], wts["w1_scale"], wts["w2"], wts["w2_scale"], ids, tw,
                         cfg.inter_dim)
    w1s, w2s = A.shuffle_weight(wts["w1"]), A.shuffle_weight(wts["w2"])
    out = A.fused_moe_a8w4(x, w1s, w2s, tw, ids, w1_scale=wts["w1_scale"],
                           w2_scale=wts["w2_scale"])
    _check(_np(ref), _np(out.float()), "A8W4 MiMo T=32")


@pytest.mark.parametrize("bm", [16, 32, 64])
def test_a8w4_odd_model_dim(cuda_device, bm):
    cfg = W.MoEConfig("a8w4_odd_h", 48, 384, 256, 6, 2, seed=8, weights="mxfp4")
    dev, ref = _make_layer(cfg, cuda_device, False)
    _check(ref["out"], _np(_run(dev, block_size_M=bm).float()), f"A8W4 H=384 bm={bm}")


def test_a8w4_num_local_tokens(cuda_device):
    cfg = W.MoEConfig("a8w4_local", 80, 512, 512, 8, 2, seed=4, weights="mxfp4")
    dev, _ = _make_layer(cfg, cuda_device, True)
    loc = torch.tensor([50], dtype=torch.int32, device=cuda_device)
    out = _run(dev, num_local_tokens=loc)
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    ref = R.fused_moe_ref(dev["x"].float().cpu().numpy(), wts["w1"].numpy(),
                          wts["w1_scale"].numpy(), wts["w2"].numpy(), wts["w2_scale"].numpy(),
                          _np(dev["ids"]), _np(dev["tw"]), num_local_tokens=50,
                          weight_format="mxfp4")
    _check(ref["out"][:50], _np(out.float())[:50], "A8W4 num_local_tokens")


@pytest.mark.parametrize("bm", [64, 128])
def test_a8w4_prefill_large_k_grouped_e8m0(cuda_device, bm):
    """model_dim 8192 (K/32 = 256 e8m0 bytes per weight row, more than the
    LDS rows hold) with 32 routed rows per expert: stage 1 runs on the
    prefill kernel with the e8m0 bytes loaded a group of K steps at a time,
    64 K steps long; checked against the oracle."""
    cfg = W.MoEConfig("a8w4_bigk", 64, 8192, 256, 8, 4, seed=17, weights="mxfp4")
    dev, ref = _make_layer(cfg, cuda_device, True)
    _check(ref["out"], _np(_run(dev, block_size_M=bm).float()), f"A8W4 H=8192 bm={bm}")


@pytest.mark.parametrize("bm", [64, 128])
def test_a8w4_e8m0_lds_bit_exact(cuda_device, monkeypatch, bm):
    """On the prefill kernels the tile's e8m0 bytes are staged in LDS once per
    tile (AITER_AMD_PF_E8LDS = 0 loads them a group of K steps at a time
    instead); both feed the same byte to every MFMA, so the layer outputs are
    bitwise equal. 150 routed rows per expert put both stages on the prefill
    kernels."""
    cfg = W.MoEConfig("e8lds", 600, 2048, 1024, 16, 4, seed=31, weights="mxfp4")
    wts = W.make_weights(cfg, device=cuda_device, shuffle=True)
    x = W.make_hidden(cfg, device=cuda_device)
    tw, ids = W.make_routing(cfg, device=cuda_device)

    def layer(e8):
        monkeypatch.setenv("AITER_AMD_PF_E8LDS", str(e8))
        out = W.run_layer("mxfp4", x, wts["w1"], wts["w2"], tw, ids, w1_scale=wts["w1_scale"],
                          w2_scale=wts["w2_scale"], block_size_M=bm)
        torch.cuda.synchronize()
        return out

    out0, out1 = layer(0), layer(1)
    assert torch.count_nonzero(out1).item() > 0
    assert torch.equal(out0, out1), (out0.float() - out1.float()).abs().max().item()


@pytest.mark.parametrize("T,block_ms", [(256, (64,)), (1024, (64, 128)), (2048, (64,)),
                                        (8192, (128,))])
def test_a8w4_mimo_stagewise(cuda_device, T, block_ms):
    """Full MiMo dims for the A8W4 mid-size and prefill configs, checked per
    stage. At 64-row blocks stage 1 runs on the prefill kernel from 16 routed
    rows per expert on average (T=512) and stage 2 from 48 (T=2048); T=256
    runs both on the direct-to-LDS kernels; 128-row blocks run stage 2 on the
    prefill kernel."""
    _fullshape.stagewise_check(W.mimo_a8w4(T), cuda_device, block_ms)


@pytest.mark.parametrize("bm", [16, 64, 128])
def test_a8w4_reference_scale_layout(cuda_device, bm):
    """The reference hands its fused kernels e8m0_shuffle'd 2-D scales
    (op_tests/test_moe_2stage.py:166-184): the same layer as row-major
    [E, N, K/32] scales, and the same stage-wise results."""
    cfg = _a8w4(W.CONFIG_A)
    dev, ref = _make_layer(cfg, cuda_device, True)
    out_rm = _run(dev, block_size_M=bm)
    s1 = A.e8m0_shuffle(dev["s1"].view(torch.uint8).reshape(-1, dev["s1"].shape[-1]))
    s2 = A.e8m0_shuffle(dev["s2"].view(torch.uint8).reshape(-1, dev["s2"].shape[-1]))
    sh = dict(dev, s1=s1.view(A.dtypes.fp8_e8m0), s2=s2.view(A.dtypes.fp8_e8m0))
    out_sh = _run(sh, block_size_M=bm)
    # the same kernel inputs: equal up to fp32 atomic order (one bf16 rounding)
    mx, _ = R.normalized_errors(_np(out_rm.float()), _np(out_sh.float()))
    assert mx <= 1e-2, mx
    _check(ref["out"], _np(out_sh.float()), f"A8W4 e8m0_shuffle scales bm={bm}")


@pytest.mark.parametrize("bm,split", [(16, 2), (16, 4), (32, 8)])
def test_a8w4_stream_stage1_split_k(cuda_device, monkeypatch, bm, split):
    """The A8W4 decode stage 1 with its K range split over several
    workgroups per tile (AITER_AMD_ST_KSPLIT1 forces the count): the e8m0
    scale groups start at the split's first K step. Same bar as the unsplit
    layer on two calls in a row, through both the two-launch and the
    one-launch layer."""
    cfg = _a8w4(W.MoEConfig("ksplit4", 5, 2048, 512, 8, 4, seed=42))
    dev, ref = _make_layer(cfg, cuda_device, True)
    monkeypatch.setenv("AITER_AMD_ST_KSPLIT1", str(split))
    for fused in (0, 1):
        monkeypatch.setenv("AITER_AMD_FUSED", str(fused))
        for call in range(2):
            out = _run(dev, block_size_M=bm)
            _check(ref["out"], _np(out.float()),
                   f"A8W4 split-K {split} bm={bm} fused={fused} call {call}")


@pytest.mark.parametrize("bm", [16, 32])
def test_a8w4_fused_layer_one_launch(cuda_device, monkeypatch, bm):
    """The one-launch layer on MXFP4 weights (AITER_AMD_FUSED=1): the slice's
    fp8 rows from LDS against the fp4 K block of w2 on the scaled MFMA, with
    the e8m0 bytes of that block. Config A against the mxfp4 oracle."""
    monkeypatch.setenv("AITER_AMD_FUSED", "1")
    cfg = _a8w4(W.CONFIG_A)
    for shuffle in (True, False):
        dev, ref = _make_layer(cfg, cuda_device, shuffle)
        _check(ref["out"], _np(_run(dev, block_size_M=bm).float()),
               f"A8W4 one-launch shuffle={shuffle} bm={bm}")
