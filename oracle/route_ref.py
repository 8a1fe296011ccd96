"""CPU oracle for MoE routing (router logits -> top-k) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker; the aiter_amd package never
calls it.

numpy restatements of the reference's routing semantics, fp32 arithmetic as
the kernels do it:
* topk_softmax_ref -- csrc/kernels/topk_softmax_kernels.cu:380-500 (the
  fused kernel: rank by logit, ties to the lower index; weight
  exp(x - rowmax) times 1/(sum of the k chosen) when renormalising, else
  times 1/(that sum + the sum over the other experts));
  token_expert_indices = rank * tokens + row (same file, 436-451);
* topk_softmax_shared_ref -- the shared-expert fusion of topk_softmax
  (same file, 326-353, 760-810);
* topk_sigmoid_ref -- op_tests/test_moe_topk_sigmoid.py:28-32;
* grouped_topk_ref -- aiter/ops/topk.py:163-197 (grouped, max per group)
  and 127-160 (biased: group score = sum of the two best choices), with the
  HIP kernels' routed_scaling_factor (csrc/kernels/topk_softmax_kernels_group.cu:
  596-603) and their restriction of the final ranking to the kept groups.
How each is pinned is listed in tests/test_oracle.py.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


def _rank(keys: np.ndarray, k: int) -> np.ndarray:
    """Per row, the indices of the k largest keys, largest first, ties to the
    lower index (a stable sort of the negated keys)."""
    return np.argsort(-keys, axis=1, kind="stable")[:, :k]


def topk_softmax_ref(logits: np.ndarray, k: int, renorm: bool):
    x = np.asarray(logits, dtype=F32)
    M, E = x.shape
    ids = _rank(x, k)
    m = x.max(axis=1, keepdims=True)
    numer = np.exp(np.take_along_axis(x, ids, 1) - m).astype(F32)
    tot = np.zeros((M, 1), dtype=F32)
    for t in range(k):                       # the kernel sums in rank order
        tot = (tot + numer[:, t:t + 1]).astype(F32)
    if not renorm:
        rest = np.exp(x - m).astype(F32)
        np.put_along_axis(rest, ids, F32(0), 1)
        tot = (tot + rest.sum(axis=1, keepdims=True, dtype=F32)).astype(F32)
    scale = np.where(tot != 0, F32(1) / np.where(tot != 0, tot, F32(1)), F32(1)).astype(F32)
    w = (numer * scale).astype(F32)
    tei = (np.arange(k, dtype=np.int64)[None, :] * M + np.arange(M)[:, None]).astype(np.int32)
    return w, ids.astype(np.int32), tei


def topk_softmax_shared_ref(logits: np.ndarray, k: int, renorm: bool, num_shared: int):
    """topk_softmax with its shared-expert fusion (topk_softmax_kernels.cu:
    326-353, 760-810): the first E = columns - num_shared logits are routed
    by topk_softmax_ref; the weights gain num_shared columns
    sigmoid(logit) of the last num_shared logits, 1 / (1 + exp(-x)) in fp32."""
    x = np.asarray(logits, dtype=F32)
    E = x.shape[1] - num_shared
    w, ids, tei = topk_softmax_ref(x[:, :E], k, renorm)
    sh = (F32(1) / (F32(1) + np.exp(-x[:, E:]).astype(F32))).astype(F32)
    return np.concatenate([w, sh], axis=1), ids, tei


def topk_sigmoid_ref(logits: np.ndarray, k: int):
    x = np.asarray(logits, dtype=F32)
    ids = _rank(x, k)
    v = np.take_along_axis(x, ids, 1)
    w = (F32(1) / (F32(1) + np.exp(-v).astype(F32))).astype(F32)
    return w, ids.astype(np.int32)


def route_scores(logits: np.ndarray, softmax: bool) -> np.ndarray:
    x = np.asarray(logits, dtype=F32)
    if softmax:
        e = np.exp(x - x.max(axis=1, keepdims=True)).astype(F32)
        return (e / e.sum(axis=1, keepdims=True, dtype=F32)).astype(F32)
    return (F32(1) / (F32(1) + np.exp(-x).astype(F32))).astype(F32)


def grouped_topk_ref(logits: np.ndarray, k: int, n_group: int, topk_group: int, renorm: bool,
                     softmax: bool = True, scaling: float = 1.0, bias: np.ndarray = None):
    """bias None: grouped_topk; bias [E]: biased_grouped_topk (sigmoid scores)."""
    s = route_scores(logits, softmax if bias is None else False)
    M, E = s.shape
    G = E // n_group
    choice = s if bias is None else (s + np.asarray(bias, dtype=F32)[None, :]).astype(F32)
    grp = choice.reshape(M, n_group, G)
    if bias is None:
        gscore = grp.max(axis=2)
    else:
        top2 = -np.sort(-grp, axis=2)[:, :, :2]
        gscore = (top2[:, :, 0] + top2[:, :, 1]).astype(F32)
    gsel = _rank(gscore, topk_group)
    keep = np.zeros((M, n_group), dtype=bool)
    np.put_along_axis(keep, gsel, True, 1)
    masked = np.where(np.repeat(keep, G, axis=1), choice, -np.inf).astype(F32)
    ids = _rank(masked, k)
    w = np.take_along_axis(s, ids, 1).astype(F32)
    if renorm:
        tot = np.zeros((M, 1), dtype=F32)
        for t in range(k):
            tot = (tot + w[:, t:t + 1]).astype(F32)
        w = (w * (F32(scaling) / tot)).astype(F32)
    else:
        w = (w * F32(scaling)).astype(F32)
    return w, ids.astype(np.int32)
