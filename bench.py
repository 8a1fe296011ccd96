"""Benchmark of the MI355X blockscale fused-MoE layer (one GPU).

Default workload (BASELINE.json metric, first leg): the MiMo-style prefill
layer, E=256, top-8, hidden 4096, inter 2048, T=8192 tokens with
Zipf(1.1)-skewed routing, fp8 e4m3fn 128x128 weight scales, 1x128 activation
scales, bf16 in/out.  A step is one aiter_amd.fused_moe call (sorting,
activation quant, stage 1, stage 2, output conversion) on inputs resident
in HBM.  The decode leg (T=32, uniform softmax routing) is reported under
"decode"; the other single-GPU configurations -- A8W4 (fp8 activations x
MXFP4 weights) at T=32/1024/2048/8192 and the expert-parallel share (32 of 256
experts, T=4096), the router, and two references for the roofline
fractions (the library's plain dense FP8 GEMM at the stage-1 shape, torch's
streaming read and copy) -- under "legs".  Prints
one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload prefill8192|decode32|...]
                  [--legs a8w4_32,a8w4_1024,a8w4_8192,ep4096|none]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP8_FLOPS = 5.0e15   # MI355X dense fp8 MFMA
PEAK_HBM_BPS = 8.0e12     # MI355X HBM3E


def _workload(name):
    import re

    if not re.fullmatch(r"(prefill|decode|a8w4_|ep)[1-9][0-9]*", name):
        raise argparse.ArgumentTypeError(f"unknown workload {name!r}")
    return name


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="prefill8192", type=_workload,
                   help="prefill<T> | decode<T> | a8w4_<T> | ep<T> (e.g. prefill8192, "
                        "decode32, a8w4_1024, ep4096)")
    p.add_argument("--legs",
                   default="decode1,decode8,decode128,prefill2048,a8w4_32,a8w4_1024,a8w4_2048,"
                           "a8w4_8192,"
                           "ep4096,route_32,route_8192,one_launch_1,one_launch_4,one_launch_32,"
                           "dense_fp8_ceiling,hbm_ceiling",
                   help="comma-separated extra workloads reported under 'legs' ('none': "
                        "skip); route_<T> times the router top-k kernels at T tokens; "
                        "one_launch_<T> the one-launch layer against the two-launch one; "
                        "dense_fp8_ceiling times the library's plain FP8 GEMM and "
                        "hbm_ceiling torch's streaming read and copy")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--block-m", type=int, default=0, help="override the M-block (0 = default)")
    p.add_argument("--kernel-only", choices=["stage1", "stage2", "layer"], default=None,
                   help="profiling mode: run a 256 MiB device copy (counter calibration) "
                        "then only this kernel --steps times ('layer': the one-call layer "
                        "the bench times, every kernel of it)")
    return p.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_cfg(name):
    from aiter_amd import workloads as W

    if name.startswith("prefill"):
        return W.mimo_prefill(int(name[len("prefill"):]))
    if name.startswith("decode"):
        return W.mimo_decode(int(name[len("decode"):]))
    if name.startswith("a8w4_"):
        return W.mimo_a8w4(int(name[len("a8w4_"):]))
    return W.mimo_ep_share(int(name[len("ep"):]))


class Layer:
    """Inputs of one MoE layer resident on the GPU."""

    def __init__(self, cfg, dev, block_m=0):
        import torch

        from aiter_amd import workloads as W

        self.cfg = cfg
        self.block_m = block_m
        self.dev = dev
        self.w = W.make_weights(cfg, device=dev, shuffle=True)
        self.x = W.make_hidden(cfg, device=dev)
        self.tw, self.ids = W.make_routing(cfg, device=dev)
        self.mask = W.make_expert_mask(cfg, device=dev)
        ids = self.ids
        if self.mask is not None:
            local = self.mask.bool()[ids.long()]
            self.pairs = int(local.sum().item())
            self.distinct = int(torch.unique(ids[local]).numel())
        else:
            self.pairs = ids.numel()
            self.distinct = int(torch.unique(ids).numel())
        torch.cuda.synchronize()

    @property
    def a8w4(self):
        return self.cfg.weights == "mxfp4"

    def run(self):
        from aiter_amd import workloads as W

        return W.run_layer(self.cfg.weights, self.x, self.w["w1"], self.w["w2"], self.tw,
                           self.ids, expert_mask=self.mask, w1_scale=self.w["w1_scale"],
                           w2_scale=self.w["w2_scale"], block_size_M=self.block_m or None)

    def stages(self):
        """(stage-1 fn, stage-2 fn) of this layer's weight format."""
        import aiter_amd as A

        if self.a8w4:
            return A.moe_stage1_a8w4, A.moe_stage2_a8w4
        return A.moe_stage1_fp8_blockscale, A.moe_stage2_fp8_blockscale

    def block_m_used(self):
        import aiter_amd as A

        cfg = self.cfg
        return self.block_m or A.select_block_m(
            cfg.tokens, cfg.topk, cfg.local_experts or cfg.experts, cfg.model_dim,
            cfg.inter_dim, self.a8w4, self.dev, cfg.experts if cfg.local_experts else 0)


def time_steps(fn, steps, warmup):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return s.elapsed_time(e) / steps, wall


def time_steady(fn, args, min_ms=50.0, warm_ms=20.0):
    """(ms per step, steps timed) for a workload reported beside the headline:
    at least max(--steps, 20) steps and at least min_ms of device time, after
    at least warm_ms of warm-up. A timed region of about a millisecond
    measures the GPU leaving its idle clocks rather than the kernels
    (measured on MI355X, the decode T=1 layer: 47-55 us over 20 steps after
    3 warm-up steps, 45.4 us over 200 after 20)."""
    import math

    wait = _SETTLE_AFTER - time.monotonic()
    if wait > 0:
        time.sleep(wait)
    est, _ = time_steps(fn, 5, max(args.warmup, 1))
    est = max(est, 1e-3)
    steps = max(args.steps, 20, math.ceil(min_ms / est))
    warm = max(args.warmup, math.ceil(warm_ms / est))
    ms, _ = time_steps(fn, steps, warm)
    return ms, steps


STEP_NAMES = ("sorting", "act_quant", "stage1", "stage2", "finish")


def layer_step_times(layer, steps):
    """Device time of each step of the one-call layer, averaged over `steps`
    calls: the library records HIP events on the layer's stream (torch's
    current stream) around its launches -- sorting (with the activation quant
    when it rides in that launch), the separate activation quant, stage 1,
    stage 2 and the finishing pass (aiter_amd_layer_timing_begin / _end).
    Returns ({step: seconds}, ms per instrumented call)."""
    import ctypes

    import torch

    from aiter_amd import _abi

    torch.cuda.synchronize()
    _abi.call("aiter_amd_layer_timing_begin", steps)
    try:
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(steps):
            layer.run()
        e.record()
    finally:
        buf = (ctypes.c_float * (steps * len(STEP_NAMES)))()
        n = _abi.query("aiter_amd_layer_timing_end", ctypes.addressof(buf), steps)
    torch.cuda.synchronize()
    if n < 1:
        raise RuntimeError("the layer timing hooks recorded no call")
    per = [sum(buf[c * len(STEP_NAMES) + k] for c in range(n)) / n
           for k in range(len(STEP_NAMES))]
    return {k: v * 1e-3 for k, v in zip(STEP_NAMES, per)}, s.elapsed_time(e) / steps


def kernel_only(layer, which, steps):
    """Profiling mode for rocprofv3 counter runs: a plain 256 MiB copy
    (known bytes, for scaling FETCH_SIZE / WRITE_SIZE) and then one stage
    kernel alone, or the whole one-call layer (each of its kernels is a
    dispatch of its own in the counter output)."""
    import torch

    import aiter_amd as A

    src = torch.empty(256 << 20, dtype=torch.uint8, device=layer.dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    if which == "layer":
        for _ in range(steps):
            layer.run()
        torch.cuda.synchronize()
        log(f"kernel-only layer: {steps} layers done")
        return
    cfg = layer.cfg
    bm = layer.block_m_used()
    st1, st2 = layer.stages()
    sid, sw, se, nv, acc, a1, a1s = stage_inputs(layer)
    a2, a2s = st1(a1, a1s, layer.w["w1"], layer.w["w1_scale"], sid, se, nv, cfg.topk, bm, True)
    torch.cuda.synchronize()
    for _ in range(steps):
        if which == "stage1":
            st1(a1, a1s, layer.w["w1"], layer.w["w1_scale"], sid, se, nv, cfg.topk, bm, True)
        else:
            st2(a2, a2s, layer.w["w2"], layer.w["w2_scale"], sid, sw, se, nv, acc, bm, True)
    torch.cuda.synchronize()
    log(f"kernel-only {which}: {steps} launches done")


def stage_inputs(layer):
    """The layer's sorted metadata (at its block_m, expert-parallel ids under
    its mask), fp32 accumulator and quantised activations, for running one
    stage kernel alone: (sorted_ids, sorted_weights, sorted_expert_ids,
    num_valid_ids, acc, a1, a1_scale)."""
    import torch

    import aiter_amd as A

    cfg = layer.cfg
    sid, sw, se, nv, acc = A.moe_sorting(layer.ids, layer.tw, cfg.experts, cfg.model_dim,
                                         torch.float32, layer.block_m_used(), layer.mask)
    a1, a1s = A.per_group_quant_hip(layer.x)
    return sid, sw, se, nv, acc, a1, a1s


_SETTLE_AFTER = 0.0


def graph_seconds(fn, reps, replays):
    """Device seconds per call of fn: reps calls captured back to back in a
    HIP graph, the graph replayed `replays` times between two events."""
    import torch

    global _SETTLE_AFTER
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    ms, _ = time_steps(graph.replay, replays, 0)
    del graph
    torch.cuda.synchronize()
    _SETTLE_AFTER = time.monotonic() + 3.0       # see stage1_b2b_seconds
    return ms * 1e-3 / reps


def stage1_b2b_seconds(layer, reps, warmup, replays=3, min_replay_ms=4.0):
    """Device time of one stage-1 launch: launches on the layer's own inputs
    captured back to back in a HIP graph, replayed between two events. The
    launches queue behind one another with no host work in between, so no
    per-launch dispatch latency is counted. A replay itself adds a fixed
    15-21 us to the event interval (measured on MI355X against rocprofv3's
    dispatch timestamps, from a 30 us to a 1.5 ms kernel), so the graph holds
    at least `reps` launches and at least min_replay_ms of them, which keeps
    that cost under 0.5% of a launch. Before the timed replays the graph is
    replayed for at least 20 ms, so the time does not depend on how busy the
    GPU was before. Returns (seconds per launch, stage-1 launches issued
    here, launches per timed replay)."""
    import math

    import torch

    cfg = layer.cfg
    st1, _ = layer.stages()
    sid, sw, se, nv, acc, a1, a1s = stage_inputs(layer)
    bm = layer.block_m_used()
    fn = lambda: st1(a1, a1s, layer.w["w1"], layer.w["w1_scale"], sid, se, nv, cfg.topk, bm,
                     True)

    def capture(n):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(n):
                fn()
        return graph

    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    graph = capture(reps)
    graph.replay()
    torch.cuda.synchronize()
    one, _ = time_steps(graph.replay, 1, 0)
    launches = max(warmup, 1) + 2 * reps
    n = max(reps, math.ceil(min_replay_ms * reps / max(one, 1e-3)))
    if n > reps:
        del graph
        graph = capture(n)
    warm = max(1, math.ceil(20.0 * reps / (max(one, 1e-3) * n)))
    for _ in range(warm):
        graph.replay()
    ms, _ = time_steps(graph.replay, replays, 0)
    launches += n * (warm + replays)
    del graph
    torch.cuda.synchronize()
    # short launches issued in the next few seconds run slower (measured on
    # MI355X: the decode T=1 layer timed right after this function ran on
    # decode T=32 took 48.9 us, 3 s later 45.0 us, with or without the graph
    # destroyed): the next timing waits that long
    global _SETTLE_AFTER
    _SETTLE_AFTER = time.monotonic() + 3.0
    return ms * 1e-3 / n, launches, n


def stage1_roofline(layer, flops, byts, workload, reps, warmup):
    """The roofline object of the stage-1 kernel: algorithmic work over its
    back-to-back launch time, the committed traffic summary of this
    workload, and the launch time itself (kernel_us)."""
    sec, launches, per_replay = stage1_b2b_seconds(layer, reps, warmup)
    return dict(roofline(flops, byts, sec), traffic=measured_traffic(workload),
                alg_bytes=round(byts), kernel_us=round(sec * 1e6, 1), launches=launches,
                launches_per_replay=per_replay)


def stage1_work(layer):
    """Algorithmic FLOPs and HBM bytes of one stage-1 launch: P routed pairs x
    2I x H MACs; bytes = the D touched experts' w1 (+ scales), x in fp8 + its
    scales, a2 out in fp8 + scales, and the sorted ids."""
    cfg = layer.cfg
    H, I, P, D, T = cfg.model_dim, cfg.inter_dim, layer.pairs, layer.distinct, cfg.tokens
    flops = 2.0 * P * (2 * I) * H
    if layer.a8w4:
        w_bytes = D * (2 * I * H // 2 + 2 * I * H // 32)
    else:
        w_bytes = D * (2 * I * H + 4 * (2 * I // 128) * (H // 128))
    act_bytes = T * H + T * (H // 128) * 4 + P * I + P * (I // 128) * 4 + P * 4
    return flops, float(w_bytes + act_bytes)


def measured_traffic(workload, kernel="stage1"):
    """HBM bytes per launch of a stage kernel from the committed rocprofv3
    FETCH_SIZE + WRITE_SIZE summary (profiles/traffic_<workload>_<stage>.md,
    each counter scaled by what it reads for a 256 MiB copy), or None."""
    import re

    path = os.path.join(ROOT, "profiles", f"traffic_{workload}_{kernel}.md")
    try:
        m = re.search(r"^traffic_bytes_per_launch: (\d+)$", open(path).read(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def roofline(flops, bytes_, seconds):
    t_mfma = flops / PEAK_FP8_FLOPS
    t_hbm = bytes_ / PEAK_HBM_BPS
    if t_hbm >= t_mfma:
        ach = bytes_ / seconds / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_BPS / 1e9,
                "unit": "GB/s", "frac": round(ach / (PEAK_HBM_BPS / 1e9), 4), "traffic": None,
                "mfma_frac": round(flops / seconds / PEAK_FP8_FLOPS, 4)}
    ach = flops / seconds / 1e12
    return {"bound": "mfma", "achieved": round(ach, 1), "peak": PEAK_FP8_FLOPS / 1e12,
            "unit": "TFLOP/s", "frac": round(ach / (PEAK_FP8_FLOPS / 1e12), 4), "traffic": None,
            "hbm_frac": round(bytes_ / seconds / PEAK_HBM_BPS, 4)}


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _blas_threads():
    """Threads the numpy BLAS actually runs with (threadpoolctl), else 1."""
    try:
        from threadpoolctl import threadpool_info

        n = [p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"]
        return int(max(n)) if n else 1
    except Exception:  # pragma: no cover
        return 1


def cpu_baseline_config_a(warmup=2, runs=10):
    """The reference's CPU torch MoE path at BASELINE.json's CPU configuration
    (config A: E=8, top-2, hidden 1024, inter 512, T=64, the seeded inputs of
    the GPU tests), restated in PyTorch (oracle/torch_ref.py, the op sequence
    of aiter/fused_moe.py:1483-1666 with pertoken_quant activations) and run
    on this host's CPU with torch's thread count: the whole layer -- weight
    dequant, activation quant, both GEMM stages, the requant and the weighted
    sum -- 2 warm-ups, then the median of 10 wall-clock runs. The numpy
    oracle's time on the same layer is reported beside it."""
    import statistics

    import torch

    from aiter_amd import workloads as W
    from oracle import moe_ref as R
    from oracle import torch_ref as TR

    cfg = W.CONFIG_A
    wts = W.make_weights(cfg, device="cpu", shuffle=False)
    xb = W.make_hidden(cfg)
    tw, ids = W.make_routing(cfg)

    def median_time(fn):
        for _ in range(warmup):
            fn()
        times = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times)

    t = median_time(lambda: TR.fused_moe_torch(xb, wts["w1"], wts["w1_scale"], wts["w2"],
                                               wts["w2_scale"], ids, tw))
    args = (xb.float().numpy(), wts["w1"].view(torch.uint8).numpy(), wts["w1_scale"].numpy(),
            wts["w2"].view(torch.uint8).numpy(), wts["w2_scale"].numpy(), ids.numpy(),
            tw.numpy())
    t_np = median_time(lambda: R.fused_moe_ref(*args, act_quant="torch"))
    flops = 2.0 * cfg.tokens * cfg.topk * 3 * cfg.inter_dim * cfg.model_dim
    threads = torch.get_num_threads()
    return {
        "value": round(cfg.tokens / t, 1), "unit": "tokens/s", "cores": threads,
        "kind": "port", "measured": True,
        "sample": (f"config A full layer (T={cfg.tokens}, E={cfg.experts}, top-{cfg.topk}, "
                   f"hidden {cfg.model_dim}, inter {cfg.inter_dim}) through the PyTorch-CPU "
                   f"restatement of the reference's torch MoE path ({threads} threads): "
                   f"{warmup} warm-ups, median of {runs} runs"),
        "latency_ms": round(t * 1e3, 3), "gflops": round(flops / t / 1e9, 2),
        "numpy_oracle": {"value": round(cfg.tokens / t_np, 1), "unit": "tokens/s",
                         "latency_ms": round(t_np * 1e3, 3), "blas_threads": _blas_threads()},
        "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(), "torch_threads": threads,
    }


def cpu_extrapolated_mimo(layer, budget_s=8.0):
    """A bounded sample of the headline workload itself, extrapolated (second,
    labelled figure): the PyTorch-CPU restatement on a seeded sample of the
    touched experts, each for all of its routed pairs (dequant of its
    weights, stage-1 GEMM, act(gate)*up, requant, stage-2 GEMM); full layer
    time = quant + D * (mean dequant time per expert) + P * (mean GEMM time
    per pair)."""
    import numpy as np
    import torch

    from aiter_amd.shuffle import unshuffle_weight
    from oracle import torch_ref as TR

    if layer.a8w4:
        return {"measured": False, "note": "the CPU restatement covers the FP8 layer only"}
    cfg = layer.cfg
    ids = layer.ids.cpu()
    tw = layer.tw.cpu()
    x = layer.x.cpu()
    if layer.mask is not None:
        m = layer.mask.cpu().bool()
        ids = torch.where(m[ids.long()], torch.cumsum(m.int(), 0)[ids.long()] - 1, -1)
    experts = torch.unique(ids[ids >= 0]).numpy()
    rng = np.random.default_rng(0)
    rng.shuffle(experts)
    I = cfg.inter_dim
    t_deq = t_gemm = 0.0
    n_exp = n_pairs = 0
    t_start = time.perf_counter()
    a1q, a1s = TR.pertoken_quant_1x128(x)
    a1 = TR.dequant_1x128(a1q, a1s)
    t_quant = time.perf_counter() - t_start
    for e in experts.tolist():
        w1q = unshuffle_weight(layer.w["w1"][e:e + 1]).cpu()
        w2q = unshuffle_weight(layer.w["w2"][e:e + 1]).cpu()
        s1 = layer.w["w1_scale"][e:e + 1].cpu()
        s2 = layer.w["w2_scale"][e:e + 1].cpu()
        t0 = time.perf_counter()
        w1 = TR.dequant_weight_128x128(w1q, s1)[0]
        w2 = TR.dequant_weight_128x128(w2q, s2)[0]
        t1 = time.perf_counter()
        tok, slot = torch.nonzero(ids == e, as_tuple=True)
        y = a1[tok] @ w1.T
        h = (torch.nn.functional.silu(y[:, :I]) * y[:, I:]).to(torch.bfloat16).float()
        hq, hs = TR.pertoken_quant_1x128(h)
        (TR.dequant_1x128(hq, hs) @ w2.T) * tw[tok, slot][:, None]
        t2 = time.perf_counter()
        t_deq += t1 - t0
        t_gemm += t2 - t1
        n_exp += 1
        n_pairs += tok.numel()
        if time.perf_counter() - t_start > budget_s and n_exp >= 2:
            break
    whole = n_exp == len(experts)
    full = (t_quant + t_deq + t_gemm if whole else
            t_quant + len(experts) * (t_deq / n_exp) + layer.pairs * (t_gemm / max(n_pairs, 1)))
    how = ("the whole layer ran (no extrapolation)" if whole else
           "extrapolated as quant + D*dequant/expert + P*gemm/pair")
    return {"value": round(cfg.tokens / full, 2), "unit": "tokens/s", "measured": whole,
            "cores": torch.get_num_threads(),
            "sample": (f"PyTorch-CPU restatement on {n_exp} of {len(experts)} touched experts "
                       f"({n_pairs} of {layer.pairs} routed pairs) of the T={cfg.tokens} layer; "
                       f"{how}: {full:.2f} s")}


def route_leg(name, args, dev):
    """The router step before the layer (moe_route.hip) at T tokens: MiMo's
    softmax top-8 of 256 experts (bf16 logits) and the DeepSeek-V3-shaped
    biased grouped top-8 (8 groups, 4 kept). HBM-bound: algorithmic bytes =
    T*E*2 read + T*k*8 written."""
    import torch

    import aiter_amd as A

    T = int(name.split("_")[1])
    E, k = 256, 8
    g = torch.Generator().manual_seed(T)
    x = (torch.randn(T, E, generator=g) * 2).to(torch.bfloat16).to(dev)
    bias = (torch.randn(E, generator=g) * 0.3).to(dev)
    w = torch.empty(T, k, dtype=torch.float32, device=dev)
    ids = torch.empty(T, k, dtype=torch.int32, device=dev)
    byts = T * E * 2 + T * k * 8
    out = {"workload": name, "tokens": T, "experts": E, "topk": k, "alg_bytes": byts}
    for tag, fn in (("softmax_topk", lambda: A.topk_softmax(w, ids, None, x, True)),
                    ("biased_grouped_topk",
                     lambda: A.biased_grouped_topk(x, bias, w, ids, 8, 4, True, 2.5))):
        # the router kernel alone: a call's host side (~15 us of Python and
        # ctypes) is longer than the kernel, so eager calls would time the
        # host; 100 calls back to back in a HIP graph time the kernel
        time_steady(fn, args)                       # warm the clocks
        ms = graph_seconds(fn, 100, 5) * 1e3
        sec = ms * 1e-3
        out[tag] = {"us": round(ms * 1e3, 2), "hbm_gbps": round(byts / sec / 1e9, 1),
                    "hbm_peak_frac": round(byts / sec / PEAK_HBM_BPS, 4)}
    return out


def dense_ceiling_leg(name, args, dev):
    """Context for the stage-1 MFMA fraction, not part of the layer: the
    vendor library's plain dense FP8 GEMM (torch._scaled_mm, hipBLASLt) at
    the stage-1 shape of all T=8192 pairs as one matrix (M = 65536 rows,
    N = 2I = 4096, K = H = 4096) and at one expert's share (M = 512). It has
    no block scales, no gather and no fused epilogue, so it bounds what an
    FP8 MFMA GEMM of this size reaches on the card."""
    import torch

    f8 = torch.float8_e4m3fn
    out = {"workload": name, "library": "torch._scaled_mm (hipBLASLt)"}
    for M, N, K in ((65536, 4096, 4096), (512, 4096, 4096)):
        a = torch.randn(M, K, device=dev).to(f8)
        b = torch.randn(N, K, device=dev).to(f8).t()
        for scales in ("tensor", "rowwise"):
            if scales == "tensor":
                sa = torch.tensor(1.0, device=dev)
                sb = torch.tensor(1.0, device=dev)
            else:
                sa = torch.rand(M, 1, device=dev) + 0.5
                sb = torch.rand(1, N, device=dev) + 0.5
            fn = lambda: torch._scaled_mm(a, b, scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16)
            ms, _ = time_steady(fn, args)
            tf = 2.0 * M * N * K / (ms * 1e-3)
            out[f"M{M}_{scales}"] = {"us": round(ms * 1e3, 1), "tflops": round(tf / 1e12, 1),
                                     "fp8_peak_frac": round(tf / PEAK_FP8_FLOPS, 4)}
        del a, b
    return out


def hbm_ceiling_leg(name, args, dev):
    """Context for the decode HBM fraction, not part of the layer: torch's
    own streaming kernels on 4 GiB resident in HBM -- a read-only reduction
    (sum over int64) and a device copy (read + write bytes)."""
    import torch

    n = 4 << 30
    x = torch.empty(n, dtype=torch.uint8, device=dev).random_()
    y = torch.empty_like(x)
    out = {"workload": name, "bytes": n}
    for tag, fn, byts in (("sum_read", lambda: torch.sum(x.view(torch.int64)), n),
                          ("copy", lambda: y.copy_(x), 2 * n)):
        ms, _ = time_steady(fn, args)
        bw = byts / (ms * 1e-3)
        out[tag] = {"us": round(ms * 1e3, 1), "tbps": round(bw / 1e12, 3),
                    "hbm_peak_frac": round(bw / PEAK_HBM_BPS, 4)}
    del x, y
    return out


def one_launch_leg(name, args, dev):
    """The one-launch layer (both GEMMs in one kernel, the role of the
    reference's fused_moe_1stage) against the two-launch layer on the same
    MiMo FP8 decode inputs at T tokens: layer times with AITER_AMD_FUSED=1 and
    =0, and the tuned table's choice."""
    import importlib
    import os

    from aiter_amd import workloads as W

    fm = importlib.import_module("aiter_amd.fused_moe")   # the module, not the function
    T = int(name[len("one_launch_"):])
    cfg = W.mimo_decode(T)
    log(f"leg {name}")
    lay = Layer(cfg, dev)
    bm = lay.block_m_used()
    out = {"workload": name, "tokens": T, "block_m": bm,
           "table_picks_one_launch": bool(fm.select_run_1stage(
               T, cfg.topk, cfg.experts, cfg.model_dim, cfg.inter_dim, False, bm, dev))}
    old = os.environ.get("AITER_AMD_FUSED")
    try:
        for tag, v in (("one_launch", "1"), ("two_launch", "0")):
            os.environ["AITER_AMD_FUSED"] = v
            ms, _ = time_steady(lay.run, args)
            out[f"{tag}_ms"] = round(ms, 4)
    finally:
        if old is None:
            os.environ.pop("AITER_AMD_FUSED", None)
        else:
            os.environ["AITER_AMD_FUSED"] = old
    out["one_launch_speedup"] = round(out["two_launch_ms"] / out["one_launch_ms"], 3)
    del lay
    return out


def leg(name, args, dev):
    """One extra workload: layer time, throughput, roofline fractions and
    per-stage kernel times."""
    if name.startswith("route_"):
        return route_leg(name, args, dev)
    if name.startswith("one_launch_"):
        return one_launch_leg(name, args, dev)
    if name == "dense_fp8_ceiling":
        return dense_ceiling_leg(name, args, dev)
    if name == "hbm_ceiling":
        return hbm_ceiling_leg(name, args, dev)
    from aiter_amd import workloads as W

    cfg = make_cfg(name)
    log(f"leg {cfg.name}")
    lay = Layer(cfg, dev)
    ms, steps = time_steady(lay.run, args)
    sec = ms * 1e-3
    flops = 2.0 * lay.pairs * 3 * cfg.inter_dim * cfg.model_dim
    byts = W.layer_bytes(cfg, lay.distinct)
    kt, _ = layer_step_times(lay, steps)
    f1, b1 = stage1_work(lay)
    out = {"workload": cfg.name, "weights": cfg.weights, "tokens": cfg.tokens,
           "ms_per_step": round(ms, 4), "steps_timed": steps,
           "tokens_per_s": round(cfg.tokens / sec, 1),
           "tflops": round(flops / sec / 1e12, 2),
           "fp8_peak_frac": round(flops / sec / PEAK_FP8_FLOPS, 4),
           "hbm_gbps": round(byts / sec / 1e9, 1),
           "hbm_peak_frac": round(byts / sec / PEAK_HBM_BPS, 4),
           "routed_pairs": lay.pairs, "distinct_experts": lay.distinct,
           "block_m": lay.block_m_used(),
           "kernels_us": {k: round(v * 1e6, 1) for k, v in kt.items()},
           "stage1_roofline": stage1_roofline(lay, f1, b1, name, max(args.steps, 20),
                                              args.warmup)}
    # the leg's tensors go back to torch's cache, not to the driver: the next
    # workload reuses those blocks. Returning several GiB to the driver slows
    # the GPU for a few seconds (measured on MI355X, decode T=1 layer: 45.0 us,
    # 48.8 us right after an empty_cache of 6 GiB, 45.3 us 5 s later), and
    # the next workload's timing would fall inside that window.
    del lay
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus N>1 is not "
                                   "supported (across GPUs the layer would shard by expert: "
                                   "each GPU runs its experts' share under an expert_mask)"}))
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    cfg = make_cfg(args.workload)
    log(f"building {cfg.name} inputs")
    layer = Layer(cfg, dev, args.block_m)
    if args.kernel_only:
        kernel_only(layer, args.kernel_only, args.steps)
        return
    log(f"timing {args.steps} steps after {args.warmup} warmup")
    ms, wall = time_steps(layer.run, args.steps, args.warmup)
    log(f"layer {ms:.3f} ms/step; timing its kernels")
    layer_s = ms * 1e-3
    flops_layer = 2.0 * layer.pairs * 3 * cfg.inter_dim * cfg.model_dim
    from aiter_amd import workloads as W

    bytes_layer = W.layer_bytes(cfg, layer.distinct)
    # the same one-call layer again, with the library's launch-timing events
    kt, ms_hooked = layer_step_times(layer, args.steps)
    f1, b1 = stage1_work(layer)
    fmt = "A8W4 (fp8 x MXFP4)" if layer.a8w4 else "FP8 blockscale"
    line = {
        "metric": "MoE-layer tokens/s (MiMo-style %s layer, T=%d)" % (fmt, cfg.tokens),
        "value": round(cfg.tokens / layer_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8",
        "data": ("synthetic (seeded N(0,0.02) weights -> %s, N(0,1) bf16 activations)"
                 % ("MXFP4 e2m1 + e8m0 1x32" if layer.a8w4 else "fp8 128x128")),
        "config": {"workload": cfg.name, "tokens": cfg.tokens, "model_dim": cfg.model_dim,
                   "inter_dim": cfg.inter_dim, "experts": cfg.experts, "topk": cfg.topk,
                   "routing": cfg.routing, "local_experts": cfg.local_experts,
                   "block_m": layer.block_m_used(), "distinct_experts": layer.distinct},
        "layer": {"tflops": round(flops_layer / layer_s / 1e12, 2),
                  "fp8_peak_frac": round(flops_layer / layer_s / PEAK_FP8_FLOPS, 4),
                  "hbm_gbps": round(bytes_layer / layer_s / 1e9, 1),
                  "hbm_peak_frac": round(bytes_layer / layer_s / PEAK_HBM_BPS, 4),
                  "alg_flops": flops_layer, "alg_bytes": bytes_layer,
                  "wall_s_timed_region": round(wall, 4)},
        # device time of each launch of the one-call layer (HIP events around
        # its launches on the layer's stream, averaged over `steps` calls)
        "kernels_us": dict({k: round(v * 1e6, 1) for k, v in kt.items()},
                           sum=round(sum(kt.values()) * 1e6, 1),
                           layer_with_events=round(ms_hooked * 1e3, 1)),
        "roofline": dict(stage1_roofline(layer, f1, b1, args.workload, args.steps,
                                         args.warmup), kernel="stage-1 gather-GEMM"),
    }
    legs = [] if args.legs in ("", "none") else [x for x in args.legs.split(",") if x]
    if not args.no_cpu_baseline:
        log("cpu baseline: the PyTorch-CPU restatement at config A, then this workload")
        line["cpu_baseline"] = cpu_baseline_config_a()
        line["cpu_baseline"]["extrapolated_" + cfg.name] = cpu_extrapolated_mimo(layer)
    if not args.no_decode and not args.workload.startswith("decode"):
        dcfg = make_cfg("decode32")
        del layer                      # kept in torch's cache (see leg())
        log(f"decode leg {dcfg.name}")
        dl = Layer(dcfg, dev)
        dms, dsteps = time_steady(dl.run, args)
        db = W.layer_bytes(dcfg, dl.distinct)
        dkt, _ = layer_step_times(dl, dsteps)
        df1, db1 = stage1_work(dl)
        line["decode"] = {"workload": dcfg.name, "ms_per_step": round(dms, 4),
                          "steps_timed": dsteps,
                          "tokens_per_s": round(dcfg.tokens / (dms * 1e-3), 1),
                          "hbm_gbps": round(db / (dms * 1e-3) / 1e9, 1),
                          "hbm_peak_frac": round(db / (dms * 1e-3) / PEAK_HBM_BPS, 4),
                          "distinct_experts": dl.distinct, "block_m": dl.block_m_used(),
                          "kernels_us": {k: round(v * 1e6, 1) for k, v in dkt.items()},
                          "stage1_roofline": stage1_roofline(dl, df1, db1, "decode32",
                                                             max(args.steps, 20), args.warmup)}
        del dl
    if legs:
        if "layer" in locals():
            del layer
        line["legs"] = {}
        for name in legs:
            try:
                line["legs"][name] = leg(name, args, dev)
            except Exception as exc:  # keep the headline line even if a leg fails
                line["legs"][name] = {"error": f"{type(exc).__name__}: {exc}"}
                log(f"leg {name} failed: {exc}")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
