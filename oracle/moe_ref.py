"""CPU oracle for the blockscale fused-MoE path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline);
the aiter_amd package never calls it.

Each function restates the reference algorithm in numpy (no torch, no GPU)
and cites the reference file:line it follows.  How each is pinned (golden
vectors, closed forms, invariants, independent second implementations) is
listed in tests/test_oracle.py; every function below has such a check.
"""
from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------- fp8 ---
# OCP FP8 E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no inf,
# 0x7F / 0xFF are NaN, max finite 448.  torch.float8_e4m3fn is this format
# (aiter/utility/dtypes.py:10-33: fp8 == e4m3fn on gfx950).


def _e4m3fn_value(code: int) -> float:
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


FP8_LUT = np.array([_e4m3fn_value(c) for c in range(256)], dtype=np.float32)
_POS_CODES = np.arange(0x7F, dtype=np.int64)          # 0x00..0x7E: 0 .. 448
_POS_VALUES = FP8_LUT[:0x7F].astype(np.float64)       # ascending
FP8_MAX = 448.0


def fp8_decode(codes: np.ndarray) -> np.ndarray:
    return FP8_LUT[np.asarray(codes, dtype=np.uint8)]


def fp8_encode_rne_sat(x: np.ndarray) -> np.ndarray:
    """fp32 -> e4m3fn code, round to nearest (ties to even code), values
    beyond +-448 saturate, the sign is kept (negative values that round to
    zero give 0x80, as torch's float8_e4m3fn cast does).  The reference
    kernel clamps to +-448 and then converts RNE
    (csrc/include/aiter_opus_plus.h:33-49)."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    a = np.minimum(np.abs(x), FP8_MAX)
    hi = np.searchsorted(_POS_VALUES, a, side="left")      # first value >= a
    hi = np.clip(hi, 0, len(_POS_VALUES) - 1)
    lo = np.clip(hi - 1, 0, len(_POS_VALUES) - 1)
    d_hi = _POS_VALUES[hi] - a
    d_lo = a - _POS_VALUES[lo]
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & ((_POS_CODES[hi] & 1) == 0))
    code = np.where(pick_hi, _POS_CODES[hi], _POS_CODES[lo])
    code = np.where(a == _POS_VALUES[hi], _POS_CODES[hi], code)
    sign = np.signbit(x).astype(np.int64) << 7          # -0 and tiny negatives -> 0x80
    return (code | sign).astype(np.uint8)


# ---------------------------------------------------------------- bf16 ---
def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 -> fp32, round to nearest even (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------- 1x128 act quant ---
_INV_FP8_MAX = np.float32(1.0 / 448.0)


def quant_1x128_kernel(x: np.ndarray):
    """Dynamic per-token-group fp8 quant with the HIP kernel's arithmetic
    (csrc/kernels/quant_kernels.cu:70-126):
      amax = max(1e-10, max|x|); scale = amax * fp32(1/448);
      q = e4m3fn(clamp(x * fp32(1/scale))).
    x: [rows, cols] float32 (bf16 values); returns (codes u8 [rows, cols],
    scale f32 [rows, cols/128])."""
    x = np.asarray(x, dtype=np.float32)
    rows, cols = x.shape
    g = x.reshape(rows, cols // 128, 128)
    amax = np.maximum(np.abs(g).max(axis=-1), np.float32(1e-10)).astype(np.float32)
    scale = (amax * _INV_FP8_MAX).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    y = (g * inv[..., None]).astype(np.float32)
    return fp8_encode_rne_sat(y).reshape(rows, cols), scale


def pertoken_quant_torch_semantics(x: np.ndarray):
    """pertoken_quant over 1x128 groups as the reference's torch oracle does
    it (aiter/ops/quant.py:42-72 via per_block_quant_wrapper 157-172):
    scale = amax/448 (0 -> 1), q = e4m3fn(x / scale)."""
    x = np.asarray(x, dtype=np.float32)
    rows, cols = x.shape
    g = x.reshape(rows, cols // 128, 128)
    amax = np.abs(g).max(axis=-1).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    y = (g / scale[..., None]).astype(np.float32)
    return fp8_encode_rne_sat(y).reshape(rows, cols), scale


def dequant_1x128(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    rows, cols = codes.shape
    return (fp8_decode(codes).reshape(rows, cols // 128, 128) *
            scale[..., None]).reshape(rows, cols).astype(np.float32)


# ------------------------------------------------- 128x128 weight quant ---
def quant_weight_128x128(w: np.ndarray):
    """[E, N, K] -> (codes u8 [E, N, K], scale f32 [E, N/128, K/128]);
    pertoken_quant per 128x128 block (op_tests/test_moe_2stage.py:82-111)."""
    w = np.asarray(w, dtype=np.float32)
    E, N, K = w.shape
    b = w.reshape(E, N // 128, 128, K // 128, 128)
    amax = np.abs(b).max(axis=(2, 4)).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    scale = np.where(scale == 0, np.float32(1.0), scale).astype(np.float32)
    q = fp8_encode_rne_sat((b / scale[:, :, None, :, None]).astype(np.float32))
    return q.reshape(E, N, K), scale


def dequant_weight_128x128(codes: np.ndarray, scale: np.ndarray) -> np.ndarray:
    E, N, K = codes.shape
    v = fp8_decode(codes).reshape(E, N // 128, 128, K // 128, 128)
    return (v * scale[:, :, None, :, None]).reshape(E, N, K).astype(np.float32)


def shuffle_16x16(w: np.ndarray) -> np.ndarray:
    """(16,16) pre-shuffle of an [E, N, K] byte array (aiter/ops/shuffle.py:7-27)."""
    E, N, K = w.shape
    return np.ascontiguousarray(
        w.reshape(E, N // 16, 16, K // 32, 2, 16).transpose(0, 1, 3, 4, 2, 5)).reshape(E, N, K)


# --------------------------------------------------------------- mxfp4 ---
# OCP MX FP4: e2m1 elements (1 sign, 2 exponent bits with bias 1, 1 mantissa
# bit; values 0, 0.5, 1, 1.5, 2, 3, 4, 6), two per byte with the even element
# in the low nibble (aiter/utility/fp4_utils.py:19-46 unpack, 100-105 pack),
# and one e8m0 scale 2^(e-127) per 32 consecutive K elements.
FP4_LUT = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)
FP4_MAX = 6.0


def fp4_encode_rne_sat(x: np.ndarray) -> np.ndarray:
    """fp32 -> e2m1 code (uint8 0..15), round to nearest even, magnitudes
    >= 6 saturate to 6, sign kept.  Bit-level statement of the reference's
    _f32_to_floatx_unpacked with ebits=2, mbits=1
    (aiter/utility/fp4_utils.py:120-235): values below the smallest normal
    (1.0) are rounded on the 0.5 grid by adding 2^22 in fp32; normal values
    get their exponent rebased and the dropped 22 mantissa bits rounded
    half-to-even."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.int64)
    sign = (u >> 31) & 1
    a = (u & 0x7FFFFFFF).astype(np.uint32).view(np.float32)
    # denormal branch: a + 2^22 rounds a to a multiple of 0.5 (fp32 ulp there)
    denorm = ((a + np.float32(2.0 ** 22)).view(np.uint32).astype(np.int64)
              - (149 << 23))
    # normal branch: rebase exponent (127 -> 1), round the 22 dropped bits RNE
    ua = a.view(np.uint32).astype(np.int64)
    odd = (ua >> 22) & 1
    normal = (ua + ((1 - 127) << 23) + ((1 << 21) - 1) + odd) >> 22
    code = np.where(a >= np.float32(FP4_MAX), 7,
                    np.where(a < np.float32(1.0), denorm, normal))
    return ((code & 7) | (sign << 3)).astype(np.uint8)


def fp4_pack(codes: np.ndarray) -> np.ndarray:
    """[..., K] e2m1 codes -> [..., K/2] bytes, even element in the low nibble."""
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def fp4_unpack(packed: np.ndarray) -> np.ndarray:
    b = np.asarray(packed, dtype=np.uint8)
    out = np.empty(b.shape[:-1] + (b.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = b & 0xF
    out[..., 1::2] = b >> 4
    return out


def mxfp4_decode(packed: np.ndarray) -> np.ndarray:
    return FP4_LUT[fp4_unpack(packed)]


def f32_to_e8m0(x: np.ndarray) -> np.ndarray:
    """fp32 -> e8m0 exponent byte (aiter/utility/fp4_utils.py:49-58): the
    biased exponent of x, plus one when mantissa bit 22 is set and either a
    lower mantissa bit is set or x is normal (so 1.5*2^e and above go to
    2^(e+1)); NaN/inf exponents stay 0xFF."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.int64)
    exp = (u >> 23) & 0xFF
    up = ((u & 0x400000) != 0) & (((u & 0x200000) != 0) | ((u & 0x1FFFFF) != 0) | (exp > 0))
    out = (exp + up.astype(np.int64)) & 0xFF
    return np.where(exp == 0xFF, 0xFF, out).astype(np.uint8)


def e8m0_to_f32(e: np.ndarray) -> np.ndarray:
    """e8m0 byte -> 2^(e-127) (aiter/utility/fp4_utils.py:61-69): 0 is
    2^-127 (fp32 subnormal 0x00400000), 0xFF is NaN."""
    e = np.asarray(e, dtype=np.uint8).astype(np.uint32)
    bits = e << 23
    bits = np.where(e == 0, np.uint32(0x00400000), bits)
    bits = np.where(e == 0xFF, np.uint32(0x7F800001), bits)
    return bits.astype(np.uint32).view(np.float32)


def quant_weight_mxfp4(w: np.ndarray):
    """per_1x32_f4_quant (aiter/ops/quant.py:75-105) of [..., K]:
    per 32-element block, scale = e8m0(amax / 4) (4 = 2^floor(log2 6)),
    codes = e2m1(x / 2^(scale-127)).  Returns (packed u8 [..., K/2],
    scale u8 [..., K/32])."""
    w = np.asarray(w, dtype=np.float32)
    lead, K = w.shape[:-1], w.shape[-1]
    b = w.reshape(-1, K // 32, 32)
    amax = np.abs(b).max(axis=-1).astype(np.float32)
    e = f32_to_e8m0((amax / np.float32(4.0)).astype(np.float32))
    y = (b / e8m0_to_f32(e)[..., None]).astype(np.float32)
    codes = fp4_encode_rne_sat(y).reshape(*lead, K)
    return fp4_pack(codes), e.reshape(*lead, K // 32)


def dequant_weight_mxfp4(packed: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """[..., K/2] packed e2m1 + [..., K/32] e8m0 -> fp32 [..., K]
    (torch_moe_stage1's per_1x32 weight branch, aiter/fused_moe.py:1504-1553)."""
    v = mxfp4_decode(packed)
    K = v.shape[-1]
    s = e8m0_to_f32(scale)
    return (v.reshape(*v.shape[:-1], K // 32, 32) * s[..., None]).reshape(v.shape).astype(
        np.float32)


# ------------------------------------------------------------- sorting ---
def moe_sorting_ref(topk_ids: np.ndarray, topk_w: np.ndarray, num_experts: int,
                    block_size: int, expert_mask=None, num_local_tokens=None):
    """Closed form of the sorting kernel output.

    Follows moe_sorting_native (op_tests/test_moe_sorting.py:15-70) with the
    kernel's conventions: padding id = (topk << 24) | tokens where tokens is
    the local token count (csrc/include/moe_sorting_opus.h:1038-1058,
    2584-2591), experts without tokens are skipped (187), masked experts get
    no segment and later experts take local ids (831-957).
    Returns (sorted_ids, sorted_weights, sorted_expert_ids, num_valid) holding
    only the defined prefix: num_valid[0] entries / num_valid[0]/bm blocks.
    """
    topk_ids = np.asarray(topk_ids, dtype=np.int64)
    topk_w = np.asarray(topk_w, dtype=np.float32)
    M, topk = topk_ids.shape
    tokens = M if num_local_tokens is None else int(num_local_tokens)
    ids = topk_ids[:tokens]
    pad_id = np.int32((topk << 24) | tokens)
    out_ids, out_w, out_e = [], [], []
    local = 0
    for e in range(num_experts):
        if expert_mask is not None and int(expert_mask[e]) == 0:
            continue
        tok, slot = np.nonzero(ids == e)            # row-major: token asc, slot asc
        n = tok.size
        if n:
            nblk = (n + block_size - 1) // block_size
            seg = np.full(nblk * block_size, pad_id, dtype=np.int32)
            seg[:n] = ((slot << 24) | tok).astype(np.int32)
            segw = np.zeros(nblk * block_size, dtype=np.float32)
            segw[:n] = topk_w[tok, slot]
            out_ids.append(seg)
            out_w.append(segw)
            out_e.append(np.full(nblk, local if expert_mask is not None else e, np.int32))
        local += int(expert_mask[e]) if expert_mask is not None else 1
    cat = lambda xs, dt: np.concatenate(xs).astype(dt) if xs else np.zeros(0, dt)
    sid, sw, se = cat(out_ids, np.int32), cat(out_w, np.float32), cat(out_e, np.int32)
    return sid, sw, se, np.array([sid.size, tokens], dtype=np.int32)


def moe_sorting_argsort(topk_ids, topk_w, num_experts, block_size, expert_mask=None,
                        num_local_tokens=None):
    """Independent second statement of the same contract via one stable
    argsort over expert ids (no per-expert loop); used to pin
    moe_sorting_ref."""
    topk_ids = np.asarray(topk_ids, dtype=np.int64)
    M, topk = topk_ids.shape
    tokens = M if num_local_tokens is None else int(num_local_tokens)
    flat = topk_ids[:tokens].reshape(-1)
    enabled = np.ones(num_experts, bool) if expert_mask is None else np.asarray(expert_mask) != 0
    local_ids = (np.arange(num_experts) if expert_mask is None else
                 np.cumsum(np.asarray(expert_mask, np.int64)) - np.asarray(expert_mask, np.int64))
    valid = (flat >= 0) & (flat < num_experts)
    valid[valid] &= enabled[flat[valid]]
    idx = np.nonzero(valid)[0]
    order = idx[np.argsort(flat[idx], kind="stable")]
    experts = flat[order]
    counts = np.bincount(experts, minlength=num_experts)
    padded = (counts + block_size - 1) // block_size * block_size
    starts = np.concatenate([[0], np.cumsum(padded)[:-1]])
    total = int(padded.sum())
    sid = np.full(total, np.int32((topk << 24) | tokens), dtype=np.int32)
    sw = np.zeros(total, dtype=np.float32)
    first = np.concatenate([[0], np.cumsum(counts)[:-1]])
    rank = np.arange(order.size) - first[experts]
    pos = starts[experts] + rank
    sid[pos] = ((order % topk) << 24 | (order // topk)).astype(np.int32)
    sw[pos] = np.asarray(topk_w, np.float32).reshape(-1)[order]
    se = np.repeat(local_ids.astype(np.int32), padded // block_size)
    return sid, sw, se, np.array([total, tokens], dtype=np.int32)


# --------------------------------------------------------- stage oracles ---
def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def local_expert_ids(topk_ids: np.ndarray, expert_mask=None) -> np.ndarray:
    """Global -> local expert ids, -1 for experts not on this GPU
    (aiter/fused_moe.py:1431-1434)."""
    if expert_mask is None:
        return np.asarray(topk_ids, dtype=np.int64)
    m = np.asarray(expert_mask, dtype=np.int64)
    lut = np.cumsum(m) - 1
    lut[m == 0] = -1
    return lut[np.asarray(topk_ids, dtype=np.int64)]


def gelu(x: np.ndarray) -> np.ndarray:
    """torch.nn.functional.gelu, approximate='none' (aiter/ops/quant.py:398-404):
    x/2 * (1 + erf(x/sqrt(2))), in fp64 then fp32."""
    from scipy.special import erf
    x = np.asarray(x, dtype=np.float64)
    return (0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))).astype(np.float32)


def moe_stage1_ref(a1: np.ndarray, w1: np.ndarray, topk_ids_local: np.ndarray,
                   topk_w: np.ndarray = None, activation: str = "silu") -> np.ndarray:
    """torch_moe_stage1 with per_1x128 (aiter/fused_moe.py:1483-1585), given
    already-dequantised fp32 a1 [T, H] and w1 [E, 2I, H]:
    out[t, j] = silu(g) * u with [g, u] = a1[t] @ w1[e_tj]^T, fp32, then bf16.
    topk_w given (doweight): [g, u] are first scaled by w[t, j]
    (fused_moe.py:1568-1571).  Rows whose expert is not local stay 0.
    Returns fp32 holding bf16 values [T, topk, I]."""
    T, _ = a1.shape
    topk = topk_ids_local.shape[1]
    E, N1, _ = w1.shape
    inter = N1 // 2
    out = np.zeros((T, topk, N1), dtype=np.float32)
    for e in range(E):
        mask = topk_ids_local == e
        if mask.any():
            tok, slot = np.nonzero(mask)
            out[tok, slot] = a1[tok] @ w1[e].T
            if topk_w is not None:
                out[tok, slot] *= np.asarray(topk_w, np.float32)[tok, slot][:, None]
    act = gelu if activation == "gelu" else silu
    h = act(out[..., :inter]) * out[..., inter:]
    return bf16_round(h)


def moe_stage2_ref(a2: np.ndarray, w2: np.ndarray, topk_ids_local: np.ndarray,
                   topk_w: np.ndarray) -> np.ndarray:
    """torch_moe_stage2 with per_1x128 (aiter/fused_moe.py:1588-1666), given
    dequantised fp32 a2 [T, topk, I] and w2 [E, H, I]: sum over slots of
    w[t, j] * a2[t, j] @ w2[e]^T in fp32, then bf16 (topk_w None: w = 1, the
    doweight=False branch, 1664-1666).  Returns fp32 [T, H]."""
    T, topk, _ = a2.shape
    E, H, _ = w2.shape
    out = np.zeros((T, topk, H), dtype=np.float32)
    for e in range(E):
        mask = topk_ids_local == e
        if mask.any():
            tok, slot = np.nonzero(mask)
            out[tok, slot] = a2[tok, slot] @ w2[e].T
    if topk_w is not None:
        out = out * np.asarray(topk_w, np.float32)[..., None]
    return bf16_round(out.sum(axis=1, dtype=np.float32))


def fused_moe_ref(x_bf16: np.ndarray, w1q, w1s, w2q, w2s, topk_ids, topk_w,
                  expert_mask=None, num_local_tokens=None, act_quant="kernel",
                  weight_format="fp8_128x128", doweight_stage1=False, activation="silu"):
    """The whole 2-stage FP8 blockscale layer as the reference's fused_moe
    computes it (aiter/fused_moe.py:1103-1334 with the oracles of
    op_tests/test_moe_2stage.py:187-231): 1x128 quant of x, stage 1 with
    fp32 dequant, bf16, 1x128 requant, stage 2, bf16.
    act_quant='kernel' uses the HIP kernel's quant arithmetic (what
    fused_moe runs), 'torch' the test's pertoken_quant.
    weight_format='mxfp4' is the A8W4 layer: the same 1x128 fp8 activations
    with packed e2m1 weights [E, N, K/2] and e8m0 scales [E, N, K/32]
    dequantised as in torch_moe_stage1/2's per_1x32 weight branch
    (aiter/fused_moe.py:1539-1553, 1635-1649).
    doweight_stage1: the routing weights go to stage 1 and stage 2 sums
    unweighted (fused_moe.py:1253, 1330). activation 'silu' or 'gelu'.
    Returns dict with out [T, H] (fp32 of bf16 values) and intermediates."""
    deq = dequant_weight_mxfp4 if weight_format == "mxfp4" else dequant_weight_128x128
    q = quant_1x128_kernel if act_quant == "kernel" else pertoken_quant_torch_semantics
    x = np.asarray(x_bf16, dtype=np.float32)
    T, H = x.shape
    tokens = T if num_local_tokens is None else int(num_local_tokens)
    ids_local = local_expert_ids(topk_ids, expert_mask)
    ids_local = np.where(np.arange(T)[:, None] < tokens, ids_local, -1)
    a1q, a1s = q(x)
    a1 = dequant_1x128(a1q, a1s)
    w1 = deq(w1q, w1s)
    h = moe_stage1_ref(a1, w1, ids_local, topk_w if doweight_stage1 else None, activation)
    topk = h.shape[1]
    inter = h.shape[2]
    a2q, a2s = q(h.reshape(T * topk, inter))
    a2 = dequant_1x128(a2q, a2s).reshape(T, topk, inter)
    w2 = deq(w2q, w2s)
    out = moe_stage2_ref(a2, w2, ids_local, None if doweight_stage1 else topk_w)
    return {"out": out, "a1q": a1q, "a1s": a1s, "h": h, "a2q": a2q.reshape(T, topk, inter),
            "a2s": a2s.reshape(T, topk, inter // 128), "ids_local": ids_local}


# ------------------------------------------------------------ tolerance ---
def normalized_errors(ref: np.ndarray, got: np.ndarray):
    """(max, rms) of the normalised relative error used by the reference's
    MoE tests (op_tests/triton_tests/moe/test_moe_gemm_a8w4.py:104-160):
    both tensors are scaled by 1/max|ref|, then
    err = |ref - got| / max(rms(ref), |ref|)."""
    ref = np.asarray(ref, dtype=np.float64)
    got = np.asarray(got, dtype=np.float64)
    if ref.size == 0:
        return 0.0, 0.0
    eps = 1.0e-30
    mult = 1.0 / (np.abs(ref).max() + eps)
    refn, gotn = ref * mult, got * mult
    ref_rms = np.sqrt(np.square(refn).mean()) + eps
    rel = np.abs(refn - gotn) / np.maximum(ref_rms, np.abs(refn))
    return float(rel.max()), float(np.sqrt(np.square(rel).mean()))


MAXTOL = 2e-2
RMSTOL = 4e-3


# ------------------------------------------------------- e8m0 shuffle ---
def e8m0_shuffle_ref(scale: np.ndarray) -> np.ndarray:
    """e8m0_shuffle (aiter/utility/fp4_utils.py:72-92) as an index formula:
    the byte of row m = 32a + 16b + c, column n = 8d + 4e + f of the padded
    [sm, sn] array lands at ((((a*(sn/8) + d)*4 + f)*16 + c)*2 + e)*2 + b."""
    m, n = scale.shape
    sm, sn = (m + 255) // 256 * 256, (n + 7) // 8 * 8
    out = np.zeros(sm * sn, dtype=scale.dtype)
    filled = np.zeros(sm * sn, dtype=bool)
    for r in range(m):
        a, b, c = r >> 5, (r >> 4) & 1, r & 15
        for col in range(n):
            d, e, f = col >> 3, (col >> 2) & 1, col & 3
            off = ((((a * (sn // 8) + d) * 4 + f) * 16 + c) * 2 + e) * 2 + b
            out[off] = scale[r, col]
            filled[off] = True
    return out.reshape(sm, sn), filled.reshape(sm, sn)


# ------------------------------------------------------ a16w4 layouts ---
def a16w4_weight_ref(w: np.ndarray, nlane: int, gate_up: bool) -> np.ndarray:
    """shuffle_weight_a16w4 (aiter/ops/shuffle.py:51-81) as an index formula:
    byte (e, n, k) with KLane = 64 / nlane, KPack = 16, n = half*N/2 +
    n0*nlane + nl (gate_up) or n0*nlane + nl, k = (k0*KLane + kl)*16 + kp
    lands at ((((n0*H + half)*K0 + k0)*KLane + kl)*nlane + nl)*16 + kp of its
    expert, H = 2 with gate_up, else 1 (half = 0)."""
    E, N, Kp = w.shape
    klane = 64 // nlane
    h = N // 2 if gate_up else N
    H = 2 if gate_up else 1
    K0 = Kp // (klane * 16)
    out = np.empty_like(w).reshape(E, -1)
    for n in range(N):
        half, r = (n // h, n % h)
        n0, nl = r // nlane, r % nlane
        for k in range(Kp):
            k0, rem = k // (klane * 16), k % (klane * 16)
            kl, kp = rem // 16, rem % 16
            off = ((((n0 * H + half) * K0 + k0) * klane + kl) * nlane + nl) * 16 + kp
            out[:, off] = w[:, n, k]
    return out.reshape(w.shape)


def a16w4_scale_ref(s: np.ndarray, experts: int, gate_up: bool) -> np.ndarray:
    """shuffle_scale_a16w4 (aiter/ops/shuffle.py:84-113) as an index formula:
    byte (e, n, k) of the [E*N, K/32] array, n = np*N/2 + n1*16 + nl
    (gate_up) or n1*32 + np*16 + nl, k = (k1*2 + kk)*4 + kl, lands at
    ((((n1*K1 + k1)*4 + kl)*16 + nl)*2 + kk)*2 + np of its expert."""
    n_all, k_ = s.shape
    N = n_all // experts
    K1 = k_ // 8
    src = s.reshape(experts, N, k_)
    out = np.empty((experts, N * k_), dtype=s.dtype)
    for n in range(N):
        if gate_up:
            np_, r = n // (N // 2), n % (N // 2)
            n1, nl = r // 16, r % 16
        else:
            n1, r = n // 32, n % 32
            np_, nl = r // 16, r % 16
        for k in range(k_):
            k1, r2 = k // 8, k % 8
            kk, kl = r2 // 4, r2 % 4
            off = ((((n1 * K1 + k1) * 4 + kl) * 16 + nl) * 2 + kk) * 2 + np_
            out[:, off] = src[:, n, k]
    return out.reshape(n_all, k_)
