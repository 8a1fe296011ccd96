"""GPU parity of the routing kernels (moe_route.hip) against the CPU oracle
(oracle/route_ref.py), through the C ABI.

Bar: ids and token_expert_indices bit-exact (the ranking of topk_softmax and
topk_sigmoid compares the logits themselves); weights within rtol 2e-6. The
grouped modes rank by scores the GPU computes with its own exp, so a row may
differ from the oracle only where the oracle's keys tie to within 1e-6; every
such row must still be a valid top-k under the oracle's keys. The reference
tests compare ids after sorting and weights with checkAllclose
(op_tests/test_moeTopkSoftmax.py:102-125, 257-310).
"""
import numpy as np
import pytest
import torch

import aiter_amd as A
from oracle import route_ref as RR

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _logits(M, E, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, E, generator=g) * 2
    return x.to(dtype).to(dev)


def _strided(M, k, dtype, dev, pad):
    buf = torch.full((M, k + pad), -7, dtype=dtype, device=dev)
    return buf[:, :k], buf


@pytest.mark.parametrize("E,k", [(8, 2), (60, 6), (128, 8), (256, 8), (384, 8), (1024, 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_softmax_parity(cuda_device, E, k, dtype, renorm):
    M = 1000 if E <= 256 else 300
    x = _logits(M, E, dtype, E * 3 + k, cuda_device)
    w, wbuf = _strided(M, k, torch.float32, cuda_device, 10)   # row stride k+10, as the reference test
    ids, ibuf = _strided(M, k, torch.int32, cuda_device, 10)
    tei = torch.empty(M, k, dtype=torch.int32, device=cuda_device)
    A.topk_softmax(w, ids, tei, x, renorm)
    rw, rids, rtei = RR.topk_softmax_ref(_np(x.float()), k, renorm)
    assert np.array_equal(_np(ids), rids)
    assert np.array_equal(_np(tei), rtei)
    np.testing.assert_allclose(_np(w), rw, rtol=2e-6, atol=1e-9)
    # the padding columns of the strided outputs are untouched
    assert (_np(wbuf[:, k:]) == -7).all() and (_np(ibuf[:, k:]) == -7).all()


@pytest.mark.parametrize("E,S,k", [(256, 1, 8), (256, 2, 8), (128, 8, 6), (60, 4, 4),
                                   (512, 1, 8)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_softmax_shared_experts(cuda_device, E, S, k, dtype, renorm):
    """topk_softmax's shared-expert fusion against the oracle: routed ids and
    token_expert_indices bit-exact, weights (routed and shared sigmoid)
    within rtol 2e-6, through the Python op and the reference-shaped ctypes
    entry; the shared logits are raised so they would win if they were
    ranked; the padding columns of strided outputs stay untouched."""
    M = 700
    x = _logits(M, E + S, dtype, E * 5 + S, cuda_device)
    x[:, E:] += 8.0
    wbuf = torch.full((M, k + S + 3), -7.0, device=cuda_device)
    w = wbuf[:, :k + S]
    ids, ibuf = _strided(M, k, torch.int32, cuda_device, 5)
    tei = torch.empty(M, k, dtype=torch.int32, device=cuda_device)
    A.topk_softmax(w, ids, tei, x, renorm, S, "sigmoid")
    rw, rids, rtei = RR.topk_softmax_shared_ref(_np(x.float()), k, renorm, S)
    assert np.array_equal(_np(ids), rids)
    assert np.array_equal(_np(tei), rtei)
    np.testing.assert_allclose(_np(w), rw, rtol=2e-6, atol=1e-9)
    assert (_np(wbuf[:, k + S:]) == -7).all() and (_np(ibuf[:, k:]) == -7).all()
    from aiter_amd import ffi
    w2 = torch.empty(M, k + S, device=cuda_device)
    ids2 = torch.empty(M, k, dtype=torch.int32, device=cuda_device)
    ffi.topk_softmax(w2, ids2, None, x, renorm, S, "sigmoid")
    assert torch.equal(ids2, ids) and torch.equal(w2, w)


def test_topk_softmax_ties_and_fused_topk(cuda_device):
    M, E, k = 64, 256, 8
    x = torch.zeros(M, E, device=cuda_device)
    x[1::2, 100:] = 1.0                       # equal maxima: the lowest ids win
    w, ids = A.fused_topk(torch.empty(M, 16, device=cuda_device), x, k, True)
    assert (_np(ids[0::2]) == np.arange(k)).all()
    assert (_np(ids[1::2]) == np.arange(100, 100 + k)).all()
    np.testing.assert_allclose(_np(w), 1.0 / k, rtol=1e-6)
    with pytest.raises(ValueError, match="Number of tokens"):
        A.fused_topk(torch.empty(M + 1, 16, device=cuda_device), x, k, True)


@pytest.mark.parametrize("E,k", [(64, 1), (128, 4), (256, 8)])
def test_topk_sigmoid_parity(cuda_device, E, k):
    x = _logits(500, E, torch.bfloat16, E + k, cuda_device)
    w = torch.empty(500, k, dtype=torch.float32, device=cuda_device)
    ids = torch.empty(500, k, dtype=torch.int32, device=cuda_device)
    A.topk_sigmoid(w, ids, x)
    rw, rids = RR.topk_sigmoid_ref(_np(x.float()), k)
    assert np.array_equal(_np(ids), rids)
    np.testing.assert_allclose(_np(w), rw, rtol=2e-6)


def _check_grouped(x, w, ids, k, n_group, topk_group, renorm, softmax, scaling, bias):
    rw, rids = RR.grouped_topk_ref(x, k, n_group, topk_group, renorm, softmax, scaling, bias)
    gids, gw = _np(ids), _np(w)
    same = (gids == rids).all(axis=1)
    assert same.mean() >= 0.999, same.mean()
    np.testing.assert_allclose(gw[same], rw[same], rtol=2e-6)
    # rows that differ: the GPU's choice is a valid top-k of the oracle's keys
    s = RR.route_scores(x, softmax if bias is None else False)
    c = s if bias is None else s + bias[None, :]
    for r in np.nonzero(~same)[0]:
        chosen = set(gids[r].tolist())
        assert len(chosen) == k
        lo = min(c[r, list(chosen)])
        rest = [c[r, e] for e in rids[r] if e not in chosen]
        assert all(v <= lo + 1e-6 for v in rest), (r, gids[r], rids[r])


@pytest.mark.parametrize("M", [37, 2000])   # whole-wave rows under 1024 tokens, 16-lane above
@pytest.mark.parametrize("E,n_group,topk_group,k", [(256, 8, 4, 8), (64, 4, 2, 4), (96, 3, 1, 5)])
@pytest.mark.parametrize("softmax,renorm,scaling", [(True, True, 1.0), (False, False, 2.5),
                                                    (False, True, 1.5)])
def test_grouped_topk_parity(cuda_device, M, E, n_group, topk_group, k, softmax, renorm,
                             scaling):
    x = _logits(M, E, torch.float32, E + n_group, cuda_device)
    w = torch.empty(M, k, dtype=torch.float32, device=cuda_device)
    ids = torch.empty(M, k, dtype=torch.int32, device=cuda_device)
    A.grouped_topk(x, w, ids, n_group, topk_group, renorm, softmax, scaling)
    _check_grouped(_np(x), w, ids, k, n_group, topk_group, renorm, softmax, scaling, None)


@pytest.mark.parametrize("M", [37, 2000])
@pytest.mark.parametrize("E,n_group,topk_group,k", [(256, 8, 4, 8), (64, 4, 2, 6)])
@pytest.mark.parametrize("renorm,scaling", [(True, 2.5), (False, 1.0)])
def test_biased_grouped_topk_parity(cuda_device, M, E, n_group, topk_group, k, renorm, scaling):
    """The DeepSeek-V3 router shape (256 experts, 8 groups, 4 kept, top-8)."""
    x = _logits(M, E, torch.bfloat16, E * 7 + k, cuda_device)
    g = torch.Generator().manual_seed(E)
    bias = (torch.randn(E, generator=g) * 0.3).to(cuda_device)
    w = torch.empty(M, k, dtype=torch.float32, device=cuda_device)
    ids = torch.empty(M, k, dtype=torch.int32, device=cuda_device)
    A.biased_grouped_topk(x, bias, w, ids, n_group, topk_group, renorm, scaling)
    _check_grouped(_np(x.float()), w, ids, k, n_group, topk_group, renorm, False, scaling,
                   _np(bias))


def test_routing_feeds_the_layer(cuda_device):
    """Router logits -> fused_topk -> fused_moe at config A: the same output as
    routing computed by the oracle (bit-identical ids and weights)."""
    from aiter_amd import workloads as W
    cfg = W.CONFIG_A
    wts = W.make_weights(cfg, device=cuda_device, shuffle=True)
    x = W.make_hidden(cfg, device=cuda_device)
    logits = _logits(cfg.tokens, cfg.experts, torch.float32, 5, cuda_device)
    tw, ids = A.fused_topk(x, logits, cfg.topk, True)
    rw, rids, _ = RR.topk_softmax_ref(_np(logits), cfg.topk, True)
    assert np.array_equal(_np(ids), rids)
    out = A.fused_moe(x, wts["w1"], wts["w2"], tw, ids, quant_type=A.QuantType.per_128x128,
                      w1_scale=wts["w1_scale"], w2_scale=wts["w2_scale"])
    out2 = A.fused_moe(x, wts["w1"], wts["w2"], torch.from_numpy(rw).to(cuda_device),
                       torch.from_numpy(rids).to(cuda_device), quant_type=A.QuantType.per_128x128,
                       w1_scale=wts["w1_scale"], w2_scale=wts["w2_scale"])
    d = (out.float() - out2.float()).abs().max().item()
    assert d <= 2e-2 * out2.float().abs().max().item(), d
