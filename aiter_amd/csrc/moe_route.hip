// MoE routing for gfx950: per token row, top-k experts and their weights
// from the router's logits (the step before sorting).
//
// Modes (reference interface in parentheses):
//   * softmax top-k (topk_softmax, csrc/kernels/topk_softmax_kernels.cu:
//     380-500; fused_topk, aiter/fused_moe.py:1853-1923): experts ranked by
//     logit; weight exp(x - rowmax), divided by the sum over the k chosen
//     (renormalise) or over the whole row (plain softmax); optionally with
//     shared experts after the routed ones in each gating row, whose sigmoid
//     scores follow the k weights (topk_softmax_kernels.cu:326-353, 760-810);
//   * sigmoid top-k (topk_sigmoid, op_tests/test_moe_topk_sigmoid.py:28-32):
//     ranked by logit, weight sigmoid(x);
//   * grouped top-k (grouped_topk, aiter/ops/topk.py:163-197): softmax or
//     sigmoid scores; groups ranked by their best score; experts of the
//     topk_group best groups ranked by score;
//   * biased grouped top-k (biased_grouped_topk, aiter/ops/topk.py:116-160):
//     sigmoid scores; choice = score + correction bias; groups ranked by the
//     sum of their two best choices; experts of the chosen groups ranked by
//     choice; the weight is the unbiased score.
// Grouped modes multiply the weights by routed_scaling_factor (after the
// renormalisation when it is on). Ties go to the lower expert / group
// index. Weights come out in rank order.
//
// LPR lanes per token row (16 for E <= 256, four rows per wave; else the
// whole wave): lane l of a row holds experts l*V .. l*V+V-1 in registers
// (E <= LPR*V <= 1024); each rank is one arg-max over the row's lanes.
#include "common.h"

namespace aiter_amd {

namespace route {

constexpr int kWaves = 4;         // waves per workgroup
constexpr int kMaxK = 32;
constexpr int kMaxGroups = 32;

enum Mode : int { SOFTMAX = 0, SIGMOID = 1, GROUPED = 2, BIASED = 3 };

struct Args {
    const void* gating;
    int dtype;
    int64_t M;
    int E;
    int k;
    int mode;
    int need_renorm;
    int softmax_scores;           // grouped: softmax (1) or sigmoid (0) scores
    int n_group;
    int topk_group;
    float scaling;
    const float* bias;
    float* w;
    int64_t ws;                   // row strides (elements) of the outputs
    int32_t* ids;
    int64_t is;
    int32_t* tei;                 // optional token_expert_indices [M, k]
    int64_t gs;                   // gating row stride (elements, >= E + ns)
    int ns;                       // shared experts: gating columns E .. E+ns-1
};

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t i) {
    if (dtype == DT_FP32) return reinterpret_cast<const float*>(p)[i];
    const uint16_t b = reinterpret_cast<const uint16_t*>(p)[i];
    if (dtype == DT_BF16) return bf16_bits_to_f32(b);
    return (float)__builtin_bit_cast(_Float16, b);
}

// Reductions over the LPR lanes of one row: LPR = 64 uses cross-lane
// shuffles; LPR = 16 (four rows per wave) uses DPP row rotations, which stay
// in the VALU (no LDS round trip per step).
template <int LPR>
__device__ __forceinline__ float lane_xchg(float v, int step) {
    if constexpr (LPR == 64) {
        return __shfl_xor(v, step, 64);
    } else {
        int r;
        const int b = __builtin_bit_cast(int, v);
        switch (step) {   // row_ror:step within each 16-lane row
            case 8: r = __builtin_amdgcn_update_dpp(b, b, 0x128, 0xF, 0xF, false); break;
            case 4: r = __builtin_amdgcn_update_dpp(b, b, 0x124, 0xF, 0xF, false); break;
            case 2: r = __builtin_amdgcn_update_dpp(b, b, 0x122, 0xF, 0xF, false); break;
            default: r = __builtin_amdgcn_update_dpp(b, b, 0x121, 0xF, 0xF, false); break;
        }
        return __builtin_bit_cast(float, r);
    }
}

template <int LPR>
__device__ __forceinline__ int lane_xchg_i(int v, int step) {
    return __builtin_bit_cast(int, lane_xchg<LPR>(__builtin_bit_cast(float, v), step));
}

template <int LPR>
__device__ __forceinline__ float row_max(float v) {
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) v = __builtin_fmaxf(v, lane_xchg<LPR>(v, o));
    return v;
}

template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) v += lane_xchg<LPR>(v, o);
    return v;
}

// (value, index) arg-max over the row's lanes: larger value, then lower index
template <int LPR>
__device__ __forceinline__ void row_argmax(float& v, int& i) {
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) {
        const float ov = lane_xchg<LPR>(v, o);
        const int oi = lane_xchg_i<LPR>(i, o);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
}

// top-2 of the row's (a1 >= a2) pairs
template <int LPR>
__device__ __forceinline__ void row_top2(float& a1, float& a2) {
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) {
        const float b1 = lane_xchg<LPR>(a1, o);
        const float b2 = lane_xchg<LPR>(a2, o);
        const float hi = __builtin_fmaxf(a1, b1);
        const float lo = __builtin_fminf(a1, b1);
        a2 = __builtin_fmaxf(lo, __builtin_fmaxf(a2, b2));
        a1 = hi;
    }
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

template <int V, int LPR>
__global__ __launch_bounds__(64 * kWaves) void moe_route_kernel(Args g) {
    constexpr int RPW = 64 / LPR;                     // rows per wave
    const int lane = threadIdx.x & (LPR - 1);         // lane within the row
    const int64_t row = ((int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6)) * RPW +
                        ((threadIdx.x & 63) / LPR);
    // rows past M still run (their loads are clamped, their stores skipped)
    // so every lane of a wave takes part in the row reductions
    const bool live = row < g.M;
    const int64_t lrow = live ? row : g.M - 1;
    const int E = g.E, k = g.k;
    const float NEG = -__builtin_inff();

    float x[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        const int e = lane * V + j;
        x[j] = e < E ? load_logit(g.gating, g.dtype, lrow * g.gs + e) : NEG;
    }

    // score s (what the weight is taken from) and ranking key per expert
    float s[V], key[V];
    float m = NEG;
    if (g.mode == SOFTMAX || (g.mode == GROUPED && g.softmax_scores)) {
        float lm = NEG;
#pragma unroll
        for (int j = 0; j < V; ++j) lm = __builtin_fmaxf(lm, x[j]);
        m = row_max<LPR>(lm);
    }
    if (g.mode == SOFTMAX || g.mode == SIGMOID) {
#pragma unroll
        for (int j = 0; j < V; ++j) key[j] = x[j];
    } else {
        if (g.softmax_scores && g.mode == GROUPED) {
            float ls = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                s[j] = lane * V + j < E ? expf(x[j] - m) : 0.0f;
                ls += s[j];
            }
            const float sum = row_sum<LPR>(ls);
#pragma unroll
            for (int j = 0; j < V; ++j) s[j] /= sum;
        } else {
#pragma unroll
            for (int j = 0; j < V; ++j) s[j] = lane * V + j < E ? sigmoid_f32(x[j]) : 0.0f;
        }
        // choice values, then the group scores
        float c[V];
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int e = lane * V + j;
            c[j] = e < E ? (g.mode == BIASED ? s[j] + g.bias[e] : s[j]) : NEG;
        }
        const int G = E / g.n_group;
        int ge[V];                    // group of each held expert (n_group: none)
#pragma unroll
        for (int j = 0; j < V; ++j) ge[j] = lane * V + j < E ? (lane * V + j) / G : g.n_group;
        float gsc[kMaxGroups];
#pragma unroll
        for (int gi = 0; gi < kMaxGroups; ++gi) {
            if (gi >= g.n_group) break;
            float a1 = NEG, a2 = NEG;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                if (ge[j] == gi) {
                    if (c[j] > a1) {
                        a2 = a1;
                        a1 = c[j];
                    } else if (c[j] > a2) {
                        a2 = c[j];
                    }
                }
            }
            if (g.mode == BIASED) {
                row_top2<LPR>(a1, a2);
                gsc[gi] = a1 + a2;
            } else {
                gsc[gi] = row_max<LPR>(a1);
            }
        }
        // the topk_group best groups (lane-uniform)
        uint32_t chosen = 0;
        for (int t = 0; t < g.topk_group; ++t) {
            int best = -1;
            float bv = NEG;
#pragma unroll
            for (int gi = 0; gi < kMaxGroups; ++gi) {
                if (gi >= g.n_group) break;
                if (!((chosen >> gi) & 1u) && (best < 0 || gsc[gi] > bv)) {
                    best = gi;
                    bv = gsc[gi];
                }
            }
            chosen |= 1u << best;
        }
#pragma unroll
        for (int j = 0; j < V; ++j) {
            key[j] = ge[j] < g.n_group && ((chosen >> ge[j]) & 1u) ? c[j] : NEG;
        }
    }

    // ---- k ranks: wave arg-max, the owner retires the winner ----
    float sel_v[kMaxK];
    int sel_i[kMaxK];
    float sum_sel = 0.0f;
#pragma unroll
    for (int t = 0; t < kMaxK; ++t) {
        if (t >= k) break;
        float v = NEG;
        int i = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (key[j] > v) {          // ascending index: the lower one wins a tie
                v = key[j];
                i = lane * V + j;
            }
        row_argmax<LPR>(v, i);
        float w;
        if (g.mode == SOFTMAX) {
            w = expf(v - m);
        } else if (g.mode == SIGMOID) {
            w = sigmoid_f32(v);
        } else {
            // the unbiased score of expert i, from its owner
            float own = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j)
                if (lane * V + j == i) own = s[j];
            w = __shfl(own, (threadIdx.x & 63 & ~(LPR - 1)) + i / V, 64);
        }
#pragma unroll
        for (int j = 0; j < V; ++j)
            if (lane * V + j == i) key[j] = NEG, x[j] = NEG;
        sel_v[t] = w;
        sel_i[t] = i;
        sum_sel += w;
    }

    float scale = 1.0f;
    if (g.mode == SOFTMAX) {
        if (g.need_renorm) {
            if (sum_sel != 0.0f) scale = 1.0f / sum_sel;
        } else {
            float rest = 0.0f;
#pragma unroll
            for (int j = 0; j < V; ++j)
                if (lane * V + j < E && x[j] != NEG) rest += expf(x[j] - m);
            const float Z = sum_sel + row_sum<LPR>(rest);
            if (Z != 0.0f) scale = 1.0f / Z;
        }
    } else if (g.mode != SIGMOID) {
        scale = g.need_renorm ? g.scaling / sum_sel : g.scaling;
    }
#pragma unroll
    for (int t = 0; t < kMaxK; ++t) {
        if (t >= k) break;
        if (lane == t && live) {
            g.w[row * g.ws + t] = sel_v[t] * scale;
            g.ids[row * g.is + t] = sel_i[t];
            if (g.tei) g.tei[row * k + t] = (int32_t)((int64_t)t * g.M + row);
        }
    }
    // shared experts (topk_softmax's fusion, topk_softmax_kernels.cu:326-353):
    // weight column k + j is sigmoid of gating column E + j, outside the
    // ranking and the renormalisation
    for (int j = lane; j < g.ns; j += LPR)
        if (live)
            g.w[row * g.ws + k + j] =
                sigmoid_f32(load_logit(g.gating, g.dtype, row * g.gs + E + j));
}

}  // namespace route

bool route_supported(int64_t E, int64_t k) {
    return E >= 1 && E <= 1024 && k >= 1 && k <= route::kMaxK && k <= E;
}

void launch_moe_route(const void* gating, int dtype, int64_t M, int64_t E, int64_t k, int mode,
                      int need_renorm, int softmax_scores, int64_t n_group, int64_t topk_group,
                      float scaling, const float* bias, float* w, int64_t ws, int32_t* ids,
                      int64_t is, int32_t* tei, hipStream_t stream, int64_t gating_stride,
                      int64_t num_shared) {
    route::Args g{};
    g.gs = gating_stride > 0 ? gating_stride : E;
    g.ns = (int)num_shared;
    g.gating = gating;
    g.dtype = dtype;
    g.M = M;
    g.E = (int)E;
    g.k = (int)k;
    g.mode = mode;
    g.need_renorm = need_renorm;
    g.softmax_scores = softmax_scores;
    g.n_group = (int)n_group;
    g.topk_group = (int)topk_group;
    g.scaling = scaling;
    g.bias = bias;
    g.w = w;
    g.ws = ws;
    g.ids = ids;
    g.is = is;
    g.tei = tei;
    // E <= 256: 16 lanes per row (four rows per wave); wider rows, and the
    // grouped modes under 1024 tokens (a per-group pass over each lane's
    // experts, latency-bound when there are few rows): the whole wave per
    // row. Measured on MI355X, E = 256: softmax top-8 12 vs 21 us at
    // T=8192; biased grouped 15 vs 25 us at T=32, 30 vs 38 us at T=8192.
    const dim3 block(64 * route::kWaves);
    const dim3 g16((unsigned)ceil_div(M, 4 * route::kWaves));
    const dim3 g64((unsigned)ceil_div(M, route::kWaves));
    if (mode >= route::GROUPED && M < 1024) {
        if (E <= 64)
            hipLaunchKernelGGL((route::moe_route_kernel<1, 64>), g64, block, 0, stream, g);
        else if (E <= 128)
            hipLaunchKernelGGL((route::moe_route_kernel<2, 64>), g64, block, 0, stream, g);
        else if (E <= 256)
            hipLaunchKernelGGL((route::moe_route_kernel<4, 64>), g64, block, 0, stream, g);
        else if (E <= 512)
            hipLaunchKernelGGL((route::moe_route_kernel<8, 64>), g64, block, 0, stream, g);
        else
            hipLaunchKernelGGL((route::moe_route_kernel<16, 64>), g64, block, 0, stream, g);
    } else if (E <= 16)
        hipLaunchKernelGGL((route::moe_route_kernel<1, 16>), g16, block, 0, stream, g);
    else if (E <= 64)
        hipLaunchKernelGGL((route::moe_route_kernel<4, 16>), g16, block, 0, stream, g);
    else if (E <= 128)
        hipLaunchKernelGGL((route::moe_route_kernel<8, 16>), g16, block, 0, stream, g);
    else if (E <= 256)
        hipLaunchKernelGGL((route::moe_route_kernel<16, 16>), g16, block, 0, stream, g);
    else if (E <= 512)
        hipLaunchKernelGGL((route::moe_route_kernel<8, 64>), g64, block, 0, stream, g);
    else
        hipLaunchKernelGGL((route::moe_route_kernel<16, 64>), g64, block, 0, stream, g);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
