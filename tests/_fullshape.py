"""Full-size parity checks split at the stage boundary (GPU, torch fp32).

At MiMo's dimensions a stage-1 accumulation in another fp32 order moves a
few SiLU*up values across a bf16 rounding boundary, and their fp8 1x128
requant then differs by one e4m3 ulp (32/448 of the group amax at the top
binade). The product of two Gaussians behind SiLU*up is heavy-tailed, so
one such flip on a dominant element shifts an output by a few per cent:
the end-to-end max-rel bar of the small cases is then a statement about
torch's accumulation order, not about the kernel. These checks pin each
stage to what it can be held to instead:

* stage 1 against torch's stage 1 (same fp8 activations): every 1x128
  scale within one bf16 ulp of amax/448, every dequantised a2 element
  within one top-binade e4m3 ulp of its group, and at most 0.5% of the fp8
  codes different (measured 0.03-0.2%);
* stage 2 on the kernel's own a2 against torch's fp32 product: the strict
  normalised bar (max-rel <= 2e-2, RMS-rel <= 4e-3,
  op_tests/triton_tests/moe/test_moe_gemm_a8w4.py:104-160), both for the
  stage-2 entry and for the one-call layer fused_moe times (its per-pair
  bf16 rows and slot sum on the prefill kernels), whose a2 is read back
  from the workspace;
* end to end against torch's chain: the reference's own bar for this
  layer, allclose(rtol=atol=0.05) on at least 95% of the outputs
  (op_tests/test_moe_blockscale.py:288 via aiter/test_common.py:399-430),
  plus RMS-rel <= 4e-3.
"""
import ctypes

import numpy as np
import torch

import aiter_amd as A
from aiter_amd import _abi
from aiter_amd import workloads as W
from aiter_amd.enums import AITER_DTYPE
from oracle import moe_ref as R

E4M3_TOP_ULP = 32.0 / 448.0
BF16_ULP = 2.0 ** -7


def deq_fp8_128x128(wq, sc):
    N, K = wq.shape
    return (wq.float().view(N // 128, 128, K // 128, 128) *
            sc.view(N // 128, 1, K // 128, 1)).view(N, K)


def deq_mxfp4(wp, sc):
    """[N, K/2] packed e2m1 + [N, K/32] e8m0 -> fp32 [N, K]."""
    lut = torch.tensor(R.FP4_LUT, device=wp.device)
    N = wp.shape[0]
    v = torch.stack([lut[(wp & 15).long()], lut[(wp >> 4).long()]], dim=-1).view(N, -1)
    s = torch.exp2(sc.float() - 127.0)
    return (v.view(N, -1, 32) * s[..., None]).view(N, -1)


def q1x128(v):
    """Kernel-semantics fp8 1x128 quant: (codes, scales) of a [rows, K] tensor."""
    g = v.float().view(v.shape[0], -1, 128)
    amax = g.abs().amax(-1, keepdim=True).clamp_min(1e-10)
    sc = amax * np.float32(1 / 448)
    q = (g * (1.0 / sc)).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(v.shape[0], -1), sc.view(v.shape[0], -1)


def deq1x128(q, sc):
    rows = q.shape[0]
    return (q.float().view(rows, -1, 128) * sc.view(rows, -1, 1)).view(rows, -1)


class TorchChain:
    """The 2-stage layer in plain torch fp32 on any device: per touched expert,
    stage 1 from dequantised activations, act(gate)*up rounded to bf16, the
    kernel-semantics 1x128 fp8 requant, and stage 2's routing-weighted sum
    (the semantics of torch_moe_stage1/2, aiter/fused_moe.py:1483-1666). It is
    the checker of the full-size GPU tests, where the numpy oracle is too
    slow; tests/test_fullshape_ref.py pins it against the oracle on the CPU.
    Experts >= `local` hold no weights here (an expert-parallel share)."""

    def __init__(self, w1, s1, w2, s2, ids, tw, deq=deq_fp8_128x128, local=None):
        self.w1, self.s1, self.w2, self.s2, self.tw, self.deq = w1, s1, w2, s2, tw, deq
        self.T, self.k = ids.shape
        self.H = w2.shape[1]
        self.I = s2.shape[2] * (32 if deq is deq_mxfp4 else 128)
        local = w1.shape[0] if local is None else local
        self.experts = [e for e in torch.unique(ids).tolist() if 0 <= e < local]
        self.routes = {e: torch.nonzero(ids == e, as_tuple=True) for e in self.experts}
        self.local_rows = torch.nonzero(((ids >= 0) & (ids < local)).view(-1)).squeeze(1)

    def stage1(self, a1d):
        """(codes, scales) [T*k, I] of the requantised act(gate)*up from the
        dequantised activations a1d [T, H]; rows of pairs with no local
        expert are zero."""
        T, k, I = self.T, self.k, self.I
        y = torch.zeros(T, k, 2 * I, device=a1d.device)
        for e in self.experts:
            tok, slot = self.routes[e]
            y[tok, slot] = a1d[tok] @ self.deq(self.w1[e], self.s1[e]).T
        h = (torch.nn.functional.silu(y[..., :I]) * y[..., I:]).to(torch.bfloat16)
        del y
        return q1x128(h.view(T * k, I))

    def stage2(self, a2d):
        """fp32 [T, H]: sum over slots of tw * (a2 row . w2^T) from the
        dequantised a2d [T*k, I]."""
        out = torch.zeros(self.T, self.H, device=a2d.device)
        for e in self.experts:
            tok, slot = self.routes[e]
            rows = tok * self.k + slot
            out.index_add_(0, tok, (a2d[rows] @ self.deq(self.w2[e], self.s2[e]).T) *
                           self.tw[tok, slot][:, None])
        return out


def torch_layer_ref(x, w1, s1, w2, s2, ids, tw, deq=deq_fp8_128x128):
    """The layer from bf16 x through TorchChain, rounded to bf16 (as fp32)."""
    c = TorchChain(w1, s1, w2, s2, ids, tw, deq)
    a1q, a1s = q1x128(x)
    q, sc = c.stage1(deq1x128(a1q, a1s))
    return c.stage2(deq1x128(q, sc)).to(torch.bfloat16).float()


def run_layer_keep_a2(cfg, x, w1s, w2s, s1, s2, tw, ids, mask, bm):
    """The one-call two-launch layer as fused_moe / fused_moe_a8w4 call it
    (the same C-ABI entry and arguments, Silu, routing weights in stage 2,
    shuffled weights) at block_m bm, on a workspace owned here, so the
    layer's own stage-1 output can be read back afterwards:
    (out bf16 [T, H], a2 fp8 [T*k, I], a2 scales f32 [T*k, I/128])."""
    mx4 = cfg.weights == "mxfp4"
    T, k = ids.shape
    H, I = x.shape[1], cfg.inter_dim
    E = w1s.shape[0]
    G = mask.numel() if mask is not None else E
    ws_bytes = _abi.query("aiter_amd_fused_moe_workspace_bytes", T, H, I, E, G, k, bm)
    # zeroed, so the rows of pairs routed elsewhere dequantise to zeros
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=x.device)
    off = (ctypes.c_int64 * 2)()
    _abi.call("aiter_amd_fused_moe_workspace_a2_offsets", T, H, I, E, G, k, bm,
              ctypes.addressof(off))
    out = torch.empty(T, H, dtype=torch.bfloat16, device=x.device)
    ids32, tw32 = ids.to(torch.int32).contiguous(), tw.float().contiguous()
    m32 = mask.to(torch.int32).contiguous() if mask is not None else None
    if mx4:
        w1s, w2s, s1, s2 = (t.view(torch.uint8) for t in (w1s, w2s, s1, s2))
    _abi.call("aiter_amd_fused_moe_a8w4" if mx4 else "aiter_amd_fused_moe_fp8_blockscale",
              x.data_ptr(), AITER_DTYPE[x.dtype], w1s.data_ptr(), s1.data_ptr(), w2s.data_ptr(),
              s2.data_ptr(), tw32.data_ptr(), ids32.data_ptr(),
              None if m32 is None else m32.data_ptr(), None, out.data_ptr(),
              AITER_DTYPE[torch.bfloat16], T, H, I, E, G, k, bm, 0, 0, 1, ws.data_ptr(), ws_bytes,
              torch.cuda.current_stream(x.device).cuda_stream)
    a2 = ws[off[0]:off[0] + T * k * I].view(torch.float8_e4m3fn).view(T * k, I)
    a2s = ws[off[1]:off[1] + T * k * (I // 128) * 4].view(torch.float32).view(T * k, I // 128)
    return out, a2, a2s


def stagewise_check(cfg, device, block_ms, log=print):
    mx4 = cfg.weights == "mxfp4"
    deq = deq_mxfp4 if mx4 else deq_fp8_128x128
    stage1 = A.moe_stage1_a8w4 if mx4 else A.moe_stage1_fp8_blockscale
    stage2 = A.moe_stage2_a8w4 if mx4 else A.moe_stage2_fp8_blockscale
    T, H, I, E, k = cfg.tokens, cfg.model_dim, cfg.inter_dim, cfg.experts, cfg.topk

    wts = W.make_weights(cfg, device=device, shuffle=False)
    x = W.make_hidden(cfg, device=device)
    tw, ids = W.make_routing(cfg, device=device)
    w1, s1, w2, s2 = wts["w1"], wts["w1_scale"], wts["w2"], wts["w2_scale"]
    w1s, w2s = A.shuffle_weight(w1), A.shuffle_weight(w2)
    # an expert-parallel share holds global experts 0 .. local-1 (their
    # local ids are the same); the other pairs contribute nothing and their
    # a2 rows are never written, so the stage-1 checks skip them
    mask = W.make_expert_mask(cfg, device=device)
    chain = TorchChain(w1, s1, w2, s2, ids, tw, deq, cfg.local_experts)
    rows_l = chain.local_rows

    # the fp8 activation quant is bit-exact with the oracle (its own tests);
    # both stage-1 paths start from the kernel's a1
    a1, a1s = A.per_group_quant_hip(x)
    q_ref, sc_ref = chain.stage1(deq1x128(a1, a1s))
    a2_ref = deq1x128(q_ref, sc_ref)
    stage2_torch = chain.stage2
    chain_ref = stage2_torch(a2_ref)
    for bm in block_ms:
        tag = f"{cfg.name} bm={bm}"
        sid, sw, se, nv, _ = A.moe_sorting(ids, tw, E, H, torch.bfloat16, bm, mask)
        a2, a2s = stage1(a1, a1s, w1s, s1, sid, se, nv, k, bm, True)
        a2s = a2s.view(T * k, -1)
        a2 = a2.view(T * k, I)
        a2d = deq1x128(a2, a2s)
        n_l = rows_l.numel()
        srel = ((a2s[rows_l] - sc_ref[rows_l]).abs() / sc_ref[rows_l]).max().item()
        err = ((a2d[rows_l] - a2_ref[rows_l]).abs().view(n_l, -1, 128) /
               (sc_ref[rows_l].view(n_l, -1, 1) * 448)).max().item()
        codes = (a2.view(torch.uint8)[rows_l] !=
                 q_ref.view(torch.uint8)[rows_l]).float().mean().item()
        log(f"[{tag}] stage 1: scale rel {srel:.2e}, element err/amax {err:.4f}, "
            f"codes differing {codes:.3%}")
        assert srel <= BF16_ULP * (1 + 1e-6), srel
        assert err <= E4M3_TOP_ULP * (1 + 2 * BF16_ULP), err
        assert codes <= 0.005, codes

        acc = torch.zeros(T, H, dtype=torch.float32, device=device)
        stage2(a2.view(T, k, I), a2s.view(T, k, -1), w2s, s2, sid, sw, se, nv, acc, bm, True)
        mx, rms = R.normalized_errors(stage2_torch(a2d).cpu().numpy(), acc.cpu().numpy())
        log(f"[{tag}] stage 2 on the kernel's a2: max-rel {mx:.2e} rms-rel {rms:.2e}")
        assert mx <= R.MAXTOL and rms <= R.RMSTOL, (mx, rms)

        # the timed layer's stage 2 (per-pair bf16 rows and the slot sum on the
        # prefill kernels, fp32 atomics on the others) on its own a2: the strict bar
        lay, la2, la2s = run_layer_keep_a2(cfg, x, w1s, w2s, s1, s2, tw, ids, mask, bm)
        lay_codes = (la2.view(torch.uint8)[rows_l] !=
                     q_ref.view(torch.uint8)[rows_l]).float().mean().item()
        assert lay_codes <= 0.005, lay_codes
        mx, rms = R.normalized_errors(stage2_torch(deq1x128(la2, la2s)).cpu().numpy(),
                                      lay.float().cpu().numpy())
        log(f"[{tag}] one-call layer on its own a2: max-rel {mx:.2e} rms-rel {rms:.2e} "
            f"(its a2 codes differing from torch's {lay_codes:.3%})")
        assert mx <= R.MAXTOL and rms <= R.RMSTOL, (mx, rms)

        out = W.run_layer(cfg.weights, x, w1s, w2s, tw, ids, expert_mask=mask, w1_scale=s1,
                          w2_scale=s2, block_size_M=bm).float()
        ref = chain_ref.to(torch.bfloat16).float()
        far = (~torch.isclose(out, ref, rtol=0.05, atol=0.05)).float().mean().item()
        mx, rms = R.normalized_errors(ref.cpu().numpy(), out.cpu().numpy())
        log(f"[{tag}] end to end: outside allclose(0.05) {far:.4%}, "
            f"max-rel {mx:.2e} rms-rel {rms:.2e}")
        assert far <= 0.05 and rms <= R.RMSTOL, (far, rms)


def stagewise_vs_oracle(cfg, dev, ref, out, bm, activation, doweight=False, log=print,
                        e2e_rms=True):
    """The same split for a small layer, against the CPU oracle: stage 1's
    fp8 codes against the oracle's a2 (each group scale within one bf16 ulp,
    at most 0.5% of the codes different in the groups whose scales agree,
    each element within one top-binade e4m3 step of its group), the layer's output against the oracle's stage 2 applied to
    the kernel's own a2 (the strict normalised bar), and RMS-rel against the
    whole oracle chain. For layers whose smallest outputs sit next to a
    one-step requant flip (GELU(gate)·up makes such ties common), where the
    end-to-end max-rel bar would test the fp8 tie, not the kernel.
    dev / ref: the device tensors and the oracle's fused_moe_ref dict;
    doweight: the layer ran with doweight_stage1; e2e_rms=False drops the
    last check (RMS-rel against the whole oracle chain) for layers of a few
    routed pairs, where one flipped code on a dominant element moves the RMS
    of the whole output."""
    mx4 = cfg.weights == "mxfp4"
    stage1 = A.moe_stage1_a8w4 if mx4 else A.moe_stage1_fp8_blockscale
    T, I, k = cfg.tokens, cfg.inter_dim, cfg.topk
    a1, a1s = A.per_group_quant_hip(dev["x"])
    sid, sw, se, nv, _ = A.moe_sorting(dev["ids"], dev["tw"], cfg.experts, cfg.model_dim,
                                        torch.float32, bm, dev["mask"])
    a2, a2s = stage1(a1, a1s, dev["w1"], dev["s1"], sid, se, nv, k, bm,
                     bool(getattr(dev["w1"], "is_shuffled", False)),
                     sorted_weights=sw if doweight else None, activation=activation)
    loc = ref["ids_local"] >= 0
    codes = a2.view(torch.uint8).cpu().numpy()
    # rows of unrouted pairs hold whatever the buffers held (masked out below)
    with np.errstate(over="ignore", invalid="ignore"):
        a2d = R.dequant_1x128(codes.reshape(T * k, I),
                              a2s.cpu().numpy().reshape(T * k, -1)).reshape(T, k, I)
    ref_d = R.dequant_1x128(ref["a2q"].reshape(T * k, I),
                            ref["a2s"].reshape(T * k, -1)).reshape(T, k, I)
    # each element within one top-binade e4m3 step of its group (32/448 of the
    # group amax, i.e. 32 x the oracle's scale), as in stagewise_check
    sc = np.repeat(ref["a2s"], 128, axis=-1)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):   # unrouted pairs
        err = (np.abs(a2d - ref_d) / (sc * 448))[loc]
    # a group whose largest element sits on a bf16 rounding tie gets a scale
    # one bf16 ulp away, which moves every code of the group: the scales are
    # held to that ulp, and the codes are compared in the groups whose scales
    # agree (with one token such a group alone is 1/8 of a pair's codes)
    gs = a2s.cpu().numpy().reshape(T, k, -1)
    srel = np.abs(gs[loc] - ref["a2s"][loc]) / ref["a2s"][loc]   # routed pairs only
    same = np.repeat(gs == ref["a2s"], 128, axis=-1)
    differ = (codes != ref["a2q"])[same & loc[..., None]].mean()
    log(f"[{cfg.name} bm={bm}] stage 1 codes differing {differ:.3%} (groups with equal scales; "
        f"{int((srel > 0).sum())} of {srel.size} scales one bf16 ulp off), element err/amax "
        f"{err.max():.4f}")
    assert srel.max() <= BF16_ULP * (1 + 1e-6), srel.max()
    assert differ <= 0.005 and err.max() <= E4M3_TOP_ULP * (1 + 2 * BF16_ULP), (differ, err.max())
    a2d[~loc] = 0
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    w2 = wts["w2"].numpy() if mx4 else wts["w2"].view(torch.uint8).numpy()
    deq = R.dequant_weight_mxfp4 if mx4 else R.dequant_weight_128x128
    own = R.moe_stage2_ref(a2d, deq(w2, wts["w2_scale"].numpy()), ref["ids_local"],
                           None if doweight else dev["tw"].float().cpu().numpy())
    mx, rms = R.normalized_errors(own, out)
    log(f"[{cfg.name} bm={bm}] on the kernel's a2: max-rel {mx:.2e} rms-rel {rms:.2e}")
    assert mx <= R.MAXTOL and rms <= R.RMSTOL, (mx, rms)
    if e2e_rms:
        assert R.normalized_errors(ref["out"], out)[1] <= R.RMSTOL
