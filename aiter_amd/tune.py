"""Shape-keyed tuned dispatch for fused_moe: the block_m table and its tuner.

Plays the part of aiter's get_2stage_cfgs + tuned_fmoe.csv
(aiter/fused_moe.py:719-1100, aiter/configs/tuned_fmoe.csv) for this path:
one row per (cu_num, padded token count, model_dim, inter_dim, expert, topk,
act_type, q_type, q_dtype_w) holding the block_m that measured fastest, the
layer time of every candidate, and run_1stage: 1 when the one-launch layer
(both GEMMs in one kernel, block_m 16 or 32) beat every two-launch candidate,
as the reference's tuned_fmoe.csv records it. Token counts are bucketed as the
reference does (next power of two below 32768, get_padded_M,
aiter/fused_moe.py:600-612). Shapes without a row use the heuristic
default_block_m.

Tuning runs the whole layer on the GPU for every block_m the dims allow and
writes the table:

    python -m aiter_amd.tune --tokens 1,2,4,8,16,32,64,128,256,512,1024,2048,4096,8192 \\
        --weights fp8,mxfp4 --out aiter_amd/configs/tuned_fmoe.csv
"""
from __future__ import annotations

import argparse
import csv
import functools
import os
import sys
from pathlib import Path

TABLE = Path(__file__).resolve().parent / "configs" / "tuned_fmoe.csv"
COLUMNS = ["cu_num", "token", "model_dim", "inter_dim", "expert", "topk", "act_type", "q_type",
           "q_dtype_w", "block_m", "run_1stage", "us", "us_bm16", "us_bm32", "us_bm64",
           "us_bm128", "us_1stage_bm16", "us_1stage_bm32"]
_KEY = COLUMNS[:9]
CANDIDATES = (16, 32, 64, 128)


def next_pow2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def padded_tokens(m: int) -> int:
    """aiter's get_padded_M: the power of two at or above m, 32768 beyond."""
    return next_pow2(m) if m < 32768 else 32768


@functools.lru_cache(maxsize=8)
def _load(path: str):
    """{key: (block_m, run_1stage)}; rows without run_1stage run two launches."""
    if not os.path.exists(path):
        return {}
    with open(path, newline="") as f:
        return {tuple(r[c] for c in _KEY): (int(r["block_m"]), int(r.get("run_1stage") or 0))
                for r in csv.DictReader(f)}


def _key(cu_num, token, model_dim, inter_dim, expert, topk, q_type, q_dtype_w):
    return (str(cu_num), str(padded_tokens(token)), str(model_dim), str(inter_dim), str(expert),
            str(topk), "Silu", q_type, q_dtype_w)


def tuned_block_m(cu_num: int, token: int, model_dim: int, inter_dim: int, expert: int,
                  topk: int, q_type: str, q_dtype_w: str):
    """The tuned block_m for this shape, or None when the table has no row
    (AITER_AMD_TUNED_FMOE overrides the table's path)."""
    cfg = tuned_config(cu_num, token, model_dim, inter_dim, expert, topk, q_type, q_dtype_w)
    return cfg[0] if cfg else None


def tuned_config(cu_num: int, token: int, model_dim: int, inter_dim: int, expert: int,
                 topk: int, q_type: str, q_dtype_w: str):
    """(block_m, run_1stage) for this shape, or None when the table has no row."""
    return _config(os.environ.get("AITER_AMD_TUNED_FMOE", str(TABLE)), cu_num,
                   padded_tokens(token), model_dim, inter_dim, expert, topk, q_type, q_dtype_w)


def clear_cache() -> None:
    """Forget the loaded tables and their lookups (after a table file changed)."""
    _load.cache_clear()
    _config.cache_clear()


@functools.lru_cache(maxsize=4096)
def _config(path, cu_num, token, model_dim, inter_dim, expert, topk, q_type, q_dtype_w):
    # one lookup per shape and table: fused_moe asks twice per call
    return _load(path).get(_key(cu_num, token, model_dim, inter_dim, expert, topk, q_type,
                                q_dtype_w))


def _candidates(model_dim: int, inter_dim: int):
    out = []
    for bm in CANDIDATES:
        if bm == 128 and (model_dim % 256 or model_dim > 8192 or inter_dim > 8192):
            continue
        out.append(bm)
    return out


def tune(tokens, weights, model_dim, inter_dim, experts, topk, steps, warmup, log=print):
    """Time the layer at every block_m for each (weights, token count); returns rows."""
    import torch

    from aiter_amd import workloads as W

    dev = torch.device("cuda:0")
    cu_num = torch.cuda.get_device_properties(dev).multi_processor_count
    rows = []
    for wfmt in weights:
        base = W.MoEConfig("tune", 1, model_dim, inter_dim, experts, topk, seed=11, weights=wfmt)
        wts = W.make_weights(base, device=dev, shuffle=True)
        for T in tokens:
            cfg = W.MoEConfig("tune", T, model_dim, inter_dim, experts, topk, seed=T,
                              weights=wfmt)
            x = W.make_hidden(cfg, device=dev)
            tw, ids = W.make_routing(cfg, device=dev)
            times = {}
            # (block_m, one launch): every two-launch block_m, and the
            # one-launch layer at the block sizes it runs on
            cands = [(bm, False) for bm in _candidates(model_dim, inter_dim)]
            if model_dim % 256 == 0 and model_dim <= 8192:
                cands += [(16, True), (32, True)]
            for bm, one in cands:
                # AITER_AMD_FUSED picks the one- or two-launch layer over the table
                os.environ["AITER_AMD_FUSED"] = "1" if one else "0"

                def run():
                    W.run_layer(wfmt, x, wts["w1"], wts["w2"], tw, ids,
                                w1_scale=wts["w1_scale"], w2_scale=wts["w2_scale"],
                                block_size_M=bm)
                times[(bm, one)] = _time_layer(run, steps, warmup)
            os.environ.pop("AITER_AMD_FUSED", None)
            best = min(times, key=times.get)
            qt = "per_1x32" if wfmt == "mxfp4" else "per_1x128"
            row = dict(zip(_KEY, _key(cu_num, T, model_dim, inter_dim, experts, topk, qt,
                                      "fp4x2" if wfmt == "mxfp4" else "fp8")))
            nan = float("nan")
            row.update(block_m=best[0], run_1stage=int(best[1]), us=round(times[best], 2),
                       **{f"us_bm{bm}": round(times.get((bm, False), nan), 2)
                          for bm in CANDIDATES},
                       **{f"us_1stage_bm{bm}": round(times.get((bm, True), nan), 2)
                          for bm in (16, 32)})
            rows.append(row)
            log(f"[tune] {wfmt} T={T}: block_m {best[0]}{' one launch' if best[1] else ''} "
                f"({times[best]:.1f} us); "
                + ", ".join(f"{b}{'/1' if o else ''}: {t:.1f}" for (b, o), t in times.items()))
    return rows


def _time_layer(run, steps, warmup, warm_ms=20.0, min_ms=50.0):
    """us per call over at least `steps` calls and min_ms of device time,
    after at least `warmup` calls and warm_ms of them: a window of a few short
    calls times the GPU leaving its idle clocks (measured on MI355X, the MiMo
    T=1 layer: 47-55 us over 20 calls after 3 warm-up calls, 45.4 us over 200
    after 20)."""
    import math

    import torch

    def timed(n):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(n):
            run()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e)

    per = timed(max(warmup, 1)) / max(warmup, 1)             # ms per call, first estimate
    timed(max(warmup, math.ceil(warm_ms / max(per, 1e-3))))
    n = max(steps, math.ceil(min_ms / max(per, 1e-3)))
    return timed(n) / n * 1e3


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--tokens", default="1,2,4,8,16,32,64,128,256,512,1024,2048,4096,8192")
    p.add_argument("--weights", default="fp8,mxfp4")
    p.add_argument("--model-dim", type=int, default=4096)
    p.add_argument("--inter-dim", type=int, default=2048)
    p.add_argument("--experts", type=int, default=256)
    p.add_argument("--topk", type=int, default=8)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--out", default=str(TABLE))
    a = p.parse_args(argv)
    tokens = sorted({padded_tokens(int(t)) for t in a.tokens.split(",")})
    rows = tune(tokens, a.weights.split(","), a.model_dim, a.inter_dim, a.experts, a.topk,
                a.steps, a.warmup, log=lambda m: print(m, file=sys.stderr, flush=True))
    # keep the table's rows for other shapes / devices, replace the tuned ones
    old = []
    if os.path.exists(a.out):
        with open(a.out, newline="") as f:
            old = [r for r in csv.DictReader(f)]
    new_keys = {tuple(str(r[c]) for c in _KEY) for r in rows}
    keep = [r for r in old if tuple(r[c] for c in _KEY) not in new_keys]
    Path(a.out).parent.mkdir(parents=True, exist_ok=True)
    with open(a.out, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COLUMNS)
        w.writeheader()
        order = lambda r: (str(r["cu_num"]), str(r["q_dtype_w"]), str(r["q_type"]),
                           str(r["act_type"]), int(r["model_dim"]), int(r["inter_dim"]),
                           int(r["expert"]), int(r["topk"]), int(r["token"]))
        for r in sorted(keep + rows, key=order):
            w.writerow({c: r.get(c, "") for c in COLUMNS})
    clear_cache()
    print(f"wrote {len(keep) + len(rows)} rows to {a.out}", file=sys.stderr)


if __name__ == "__main__":
    main()
