// FP8 block-scale MoE gather-GEMMs for gfx950 (MI355X).
//
// Stage 1 (reference: ck_moe_stage1 gemm_moe_ck2stages.cu:46-116 and the
// torch oracle torch_moe_stage1, aiter/fused_moe.py:1483-1585):
//   for each sorted row r of M-block b (expert e = sorted_expert_ids[b],
//   token t, slot s from sorted_ids[r]):
//     y[n]  = sum_kb  (a_q[t, kb] . w1_q[e, n, kb]) * a_s[t, kb] * w1_s[e, n/128, kb]
//     h[i]  = bf16( silu(y[i]) * y[I + i] )                (i < I)
//     a2[t, s, :], a2_s[t, s, :] = 1x128 fp8 quant of h    (fused requant;
//     the reference runs it as a separate kernel, fused_moe.py:1306-1314)
// Stage 2 (reference: ck_moe_stage2 gemm_moe_ck2stages.cu:118-181, oracle
// torch_moe_stage2 fused_moe.py:1588-1666):
//     acc[t, n] += sorted_w[r] * sum_kb (a2_q[t,s,kb] . w2_q[e,n,kb]) *
//                  a2_s[t,s,kb] * w2_s[e, n/128, kb]
//   into an fp32 accumulator (zeroed by the sorting launch), converted to
//   bf16 afterwards; padding rows (token >= tokens) are skipped.
//
// Kernel shape (both stages): 256 threads = 4 wave64s, one M-block of BM
// sorted rows x 128 output columns per workgroup, K stepped in 128-wide
// scale blocks.  Each 128-K step is exactly one v_mfma_f32_16x16x128_f8f6f4
// per 16x16 output tile; its fp32 result is multiplied by the row's
// combined scale a_s * w_s and added into the fp32 accumulator, so the
// block-scale dequant costs one FMA per output per K block and nothing in
// the MFMA loop.  Stage 1 loads 256 weight rows (128 gate + the matching 128
// up rows) so SiLU(gate)*up and the 1x128 requant of the 128 outputs finish
// inside the workgroup.
//
// Weight layouts: the reference's pre-shuffled (16,16) layout
// (aiter/ops/shuffle.py:7-27: [E, N/16, K/32, 2, 16 rows, 16 bytes]) is
// copied verbatim into LDS, 2 KB per 16-row group per K block, and an MFMA
// B fragment is two conflict-free 16-byte LDS reads.  Plain row-major
// [E, N, K] weights are rearranged into the same LDS layout while staging.
//
// A8W4 (W4 = true): the weights are MXFP4 -- packed e2m1 [E, N, K/2] bytes
// (shuffled on the byte view the same way, or row-major) with e8m0 scales
// [E, N, K/32] (the layout torch_moe_stage1/2 read in their per_1x32
// branch, aiter/fused_moe.py:1539-1553, 1635-1649).  A 16-row group's K
// block is 1 KB and lane l's B fragment is its 16 bytes at l*16 (MX block
// l/16 of row l%16); the lane's e8m0 byte goes into the scaled MFMA, so the
// dequant FMA only applies the activation scale.  The A fragment takes K
// bytes 16q..16q+15 and 64+16q..64+16q+15 (q = lane/16), the K pairing of
// the fp8 x fp4 MFMA (see mfma16x16x128_fp8_fp4).
#include "common.h"

namespace aiter_amd {

constexpr int kGemmThreads = 256;
constexpr int kBK = 128;           // K per step == scale block
constexpr int kAStride = kBK + 16; // LDS row stride of the A tile (bytes)

struct GemmArgs {
    const uint8_t* a;           // activation rows, fp8 [a_rows, K]
    const float* a_scale;       // per (row, kb): a_scale[row*sa_row + kb*sa_kb]
    int64_t sa_row;
    int64_t sa_kb;
    const uint8_t* w;           // [E, N, K] fp8 (shuffled or row-major)
    const float* w_scale;       // [E, N/128, K/128] (fp8 weights)
    const uint8_t* w_scale8;    // [E, N, K/32] e8m0 (MXFP4 weights)
    const int32_t* sorted_ids;
    const float* sorted_w;
    int act;                   // stage 1: activation of gate (kActSilu / kActGelu)
    const int32_t* sorted_eids;
    const int32_t* num_valid;
    uint8_t* a2;                // stage 1 out: fp8 [T*topk, I]
    float* a2_scale;            // stage 1 out: [T*topk, I/128]
    void* acc;                  // stage 2 out [T, N]: fp32, bf16 or fp16 (acc_dtype)
    int acc_dtype;
    int K;
    int N;                      // weight rows per expert (2I or H)
    int inter;                  // I (stage 1)
    int topk;
    int E;
    int64_t a_rows;
};

template <int BM, int STAGE, bool SHUFFLED, bool W4>
__global__ __launch_bounds__(kGemmThreads) void moe_gemm_fp8bs_kernel(GemmArgs g) {
    constexpr int NGRP = STAGE == 1 ? 16 : 8;           // 16-row weight groups per tile
    constexpr int NCT = STAGE == 1 ? 4 : 2;             // 16-col MFMA tiles per wave
    constexpr int NRT = BM / 16;                        // 16-row MFMA tiles
    constexpr int GB = W4 ? 1024 : 2048;                // bytes per 16-row group per K block
    constexpr int A_PIECES = (BM * 8 + kGemmThreads - 1) / kGemmThreads;
    constexpr int B_PIECES = NGRP * (GB / 16) / kGemmThreads; // 16-byte pieces per thread
    static_assert(BM % 16 == 0 && BM <= 64, "BM must be 16, 32 or 64");

    __shared__ __attribute__((aligned(16))) uint8_t s_a[BM * kAStride];
    __shared__ __attribute__((aligned(16))) uint8_t s_b[NGRP * GB];
    __shared__ float s_sa[BM];
    __shared__ int64_t s_arow[BM];   // activation row (or -1)
    __shared__ int64_t s_orow[BM];   // output row (or -1)
    __shared__ float s_w[BM];
    __shared__ float s_amax[4][BM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int lr = lane & 15;
    const int lq = lane >> 4;

    const int mb = blockIdx.y;
    const int n0 = blockIdx.x * 128;                    // output column base
    const int nvalid = g.num_valid[0];
    if (mb * BM >= nvalid) return;
    const int tokens = g.num_valid[1];
    const int e = g.sorted_eids[mb];
    if (e < 0 || e >= g.E) return;

    for (int r = tid; r < BM; r += kGemmThreads) {
        const uint32_t id = (uint32_t)g.sorted_ids[mb * BM + r];
        const int t = (int)(id & 0xFFFFFFu);
        const int s = (int)(id >> 24);
        const bool valid = t < tokens && s < g.topk;
        const int64_t pair = (int64_t)t * g.topk + s;
        int64_t arow = -1, orow = -1;
        if (valid) {
            arow = STAGE == 1 ? (int64_t)t : pair;
            orow = STAGE == 1 ? pair : (int64_t)t;
            if (arow >= g.a_rows) arow = orow = -1;
        }
        s_arow[r] = arow;
        s_orow[r] = orow;
        // routing weight of the pair (1 when none is passed: stage 2 without
        // weights, or stage 1 without doweight); stage 1 applies it only when given
        s_w[r] = valid ? (g.sorted_w ? g.sorted_w[mb * BM + r] : 1.0f) : 0.0f;
    }
    __syncthreads();

    const int K = g.K;
    const int KB = K / kBK;
    const int KBY = W4 ? K / 2 : K;                     // weight bytes per row
    const uint8_t* we = g.w + (int64_t)e * g.N * KBY;
    const float* wse = W4 ? nullptr : g.w_scale + (int64_t)e * (g.N / 128) * KB;

    // Per-thread staging descriptors (fixed across K blocks).
    const uint8_t* a_src[A_PIECES];
    int a_dst[A_PIECES];
#pragma unroll
    for (int i = 0; i < A_PIECES; ++i) {
        const int q = tid + i * kGemmThreads;
        const int row = q >> 3, part = q & 7;
        a_dst[i] = -1;
        a_src[i] = nullptr;
        if (row < BM) {
            a_dst[i] = row * kAStride + part * 16;
            const int64_t arow = s_arow[row];
            if (arow >= 0) a_src[i] = g.a + arow * K + part * 16;
        }
    }
    int64_t b_src[B_PIECES];
    int b_dst[B_PIECES];
#pragma unroll
    for (int i = 0; i < B_PIECES; ++i) {
        const int q = tid + i * kGemmThreads;
        if (W4) {
            // group grp's K block: 16 rows x 64 B; LDS holds it lane-linear
            // (MX block j of row r at j*256 + r*16), which is also the shuffled
            // byte layout of the block
            const int grp = q >> 6, within = q & 63;
            const int r = within & 15, j = within >> 4;
            int row0;
            if (STAGE == 1)
                row0 = grp < 8 ? n0 + 16 * grp : g.inter + n0 + 16 * (grp - 8);
            else
                row0 = n0 + 16 * grp;
            b_src[i] = SHUFFLED ? (int64_t)row0 * KBY + within * 16
                                : (int64_t)(row0 + r) * KBY + j * 16;
            b_dst[i] = q * 16;
        } else if (SHUFFLED) {
            const int grp = q >> 7, within = q & 127;
            int row0;
            if (STAGE == 1)
                row0 = grp < 8 ? n0 + 16 * grp : g.inter + n0 + 16 * (grp - 8);
            else
                row0 = n0 + 16 * grp;
            b_src[i] = (int64_t)row0 * K + within * 16;
            b_dst[i] = q * 16;
        } else {
            const int r = q >> 3, j = q & 7;
            int row;
            if (STAGE == 1)
                row = r < 128 ? n0 + r : g.inter + n0 + (r - 128);
            else
                row = n0 + r;
            b_src[i] = (int64_t)row * K + j * 16;
            b_dst[i] = (r >> 4) * 2048 + (j >> 1) * 512 + (j & 1) * 256 + (r & 15) * 16;
        }
    }
    const int64_t sa_self = tid < BM ? s_arow[tid] : -1;

    // column tile ct of this wave -> 16-row weight group
    auto group_of = [&](int ct) {
        if (STAGE == 1) return ct < 2 ? 2 * wv + ct : 8 + 2 * wv + (ct - 2);
        return 2 * wv + ct;
    };
    // A8W4: lane's e8m0 scale row (the weight row of its column) per column tile
    const uint8_t* bs_row[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        bs_row[ct] = nullptr;
        if (W4) {
            const int grp = group_of(ct);
            const int row = STAGE == 1 ? (grp < 8 ? n0 + 16 * grp : g.inter + n0 + 16 * (grp - 8))
                                       : n0 + 16 * grp;
            bs_row[ct] = g.w_scale8 + ((int64_t)e * g.N + row + lr) * (K / 32);
        }
    }

    v4i ra[A_PIECES];
    v4i rb[B_PIECES];
    uint32_t rbs[NCT];
    float rsa = 0.0f;
    auto load_kb = [&](int kb) {
#pragma unroll
        for (int i = 0; i < A_PIECES; ++i) {
            v4i z = {0, 0, 0, 0};
            ra[i] = a_src[i] ? *reinterpret_cast<const v4i*>(a_src[i] + kb * kBK) : z;
        }
#pragma unroll
        for (int i = 0; i < B_PIECES; ++i) {
            const int64_t off = W4 ? b_src[i] + (int64_t)kb * (SHUFFLED ? 1024 : 64)
                                   : (SHUFFLED ? b_src[i] + (int64_t)kb * 2048 : b_src[i] + kb * kBK);
            rb[i] = *reinterpret_cast<const v4i*>(we + off);
        }
        if (W4) {
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct)
                rbs[ct] = *reinterpret_cast<const uint32_t*>(bs_row[ct] + kb * 4);
        }
        rsa = sa_self >= 0 ? g.a_scale[sa_self * g.sa_row + kb * g.sa_kb] : 0.0f;
    };

    v4f acc[NRT][NCT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};

    // weight-scale block rows of this tile
    const int nb0 = STAGE == 1 ? n0 / 128 : n0 / 128;
    const int nb1 = STAGE == 1 ? (g.inter + n0) / 128 : 0;

    load_kb(0);
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int i = 0; i < A_PIECES; ++i)
            if (a_dst[i] >= 0) *reinterpret_cast<v4i*>(s_a + a_dst[i]) = ra[i];
#pragma unroll
        for (int i = 0; i < B_PIECES; ++i) *reinterpret_cast<v4i*>(s_b + b_dst[i]) = rb[i];
        if (tid < BM) s_sa[tid] = rsa;
        int bsc[NCT];                   // this step's e8m0 byte per column tile (A8W4)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) bsc[ct] = W4 ? (int)(rbs[ct] >> (8 * lq)) : 0;
        __syncthreads();
        if (kb + 1 < KB) load_kb(kb + 1);

        const float sw0 = W4 ? 1.0f : wse[nb0 * KB + kb];
        const float sw1 = !W4 && STAGE == 1 ? wse[nb1 * KB + kb] : 1.0f;

        v8i bfrag[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            const int grp = group_of(ct);
            if (W4) {
                const v4i lo = *reinterpret_cast<const v4i*>(s_b + grp * 1024 + lane * 16);
                bfrag[ct] = v8i{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
            } else {
                const uint8_t* p = s_b + grp * 2048 + lq * 512 + lr * 16;
                const v4i lo = *reinterpret_cast<const v4i*>(p);
                const v4i hi = *reinterpret_cast<const v4i*>(p + 256);
                bfrag[ct] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
        }
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const uint8_t* p = s_a + (rt * 16 + lr) * kAStride;
            const v4i lo = *reinterpret_cast<const v4i*>(p + (W4 ? lq * 16 : lq * 32));
            const v4i hi = *reinterpret_cast<const v4i*>(p + (W4 ? 64 + lq * 16 : lq * 32 + 16));
            const v8i afrag = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            float sa[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) sa[v] = s_sa[rt * 16 + 4 * lq + v];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                const v4f blk = W4 ? mfma16x16x128_fp8_fp4(afrag, bfrag[ct], bsc[ct])
                                   : mfma16x16x128_fp8(afrag, bfrag[ct]);
                const float sw = (STAGE == 1 && ct >= 2) ? sw1 : sw0;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[rt][ct][v] += W4 ? blk[v] * sa[v] : blk[v] * (sa[v] * sw);
            }
        }
        __syncthreads();
    }

    if (STAGE == 2) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = rt * 16 + 4 * lq + v;
                const int64_t t = s_orow[row];
                if (t < 0) continue;
                const float wgt = s_w[row];
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    const int col = n0 + 32 * wv + 16 * ct + lr;
                    acc_add(g.acc, g.acc_dtype, t * g.N + col, acc[rt][ct][v] * wgt);
                }
            }
        return;
    }

    // ---- stage 1 epilogue: silu(gate)*up -> bf16 -> 1x128 fp8 requant ----
    float h[NRT][2][4];
    // act(gate) * up; the activation is chosen once per workgroup
    auto act_up = [&](auto act) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    // doweight_stage1: the pair's weight scales gate and up before the
                    // activation (aiter/fused_moe.py:1568-1571)
                    const float wg = g.sorted_w ? s_w[rt * 16 + 4 * lq + v] : 1.0f;
                    h[rt][j][v] = bf16_round(act(acc[rt][j][v] * wg) * (acc[rt][2 + j][v] * wg));
                }
    };
    if (g.act == kActGelu)
        act_up([](float x) { return gelu_f32(x); });
    else
        act_up([](float x) { return silu_f32(x); });
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float m = __builtin_fmaxf(__builtin_fabsf(h[rt][0][v]), __builtin_fabsf(h[rt][1][v]));
            m = warp_max_16(m);
            if (lr == 0) s_amax[wv][rt * 16 + 4 * lq + v] = m;
        }
    __syncthreads();
    uint8_t* s_q = s_a;  // reuse the A tile as the [BM][128] fp8 staging tile
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = rt * 16 + 4 * lq + v;
            float amax = __builtin_fmaxf(__builtin_fmaxf(s_amax[0][row], s_amax[1][row]),
                                         __builtin_fmaxf(s_amax[2][row], s_amax[3][row]));
            amax = __builtin_fmaxf(amax, 1e-10f);
            const float inv = 1.0f / (amax * kInvFp8Max);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t b = f32x2_to_fp8x2(h[rt][j][v] * inv, 0.0f) & 0xFFu;
                s_q[row * kAStride + 32 * wv + 16 * j + lr] = (uint8_t)b;
            }
        }
    __syncthreads();
    const int I = g.inter;
    for (int q = tid; q < BM * 8; q += kGemmThreads) {
        const int row = q >> 3, part = q & 7;
        const int64_t orow = s_orow[row];
        if (orow < 0) continue;
        *reinterpret_cast<v4i*>(g.a2 + orow * I + n0 + part * 16) =
            *reinterpret_cast<const v4i*>(s_q + row * kAStride + part * 16);
        if (part == 0) {
            float amax = __builtin_fmaxf(__builtin_fmaxf(s_amax[0][row], s_amax[1][row]),
                                         __builtin_fmaxf(s_amax[2][row], s_amax[3][row]));
            amax = __builtin_fmaxf(amax, 1e-10f);
            g.a2_scale[orow * (I / 128) + n0 / 128] = amax * kInvFp8Max;
        }
    }
}

template <int STAGE, bool SHUFFLED, bool W4>
static void launch_gemm_bm(int bm, dim3 grid, GemmArgs& g, hipStream_t stream) {
    switch (bm) {
        case 16:
            hipLaunchKernelGGL((moe_gemm_fp8bs_kernel<16, STAGE, SHUFFLED, W4>), grid,
                               dim3(kGemmThreads), 0, stream, g);
            break;
        case 32:
            hipLaunchKernelGGL((moe_gemm_fp8bs_kernel<32, STAGE, SHUFFLED, W4>), grid,
                               dim3(kGemmThreads), 0, stream, g);
            break;
        case 64:
            hipLaunchKernelGGL((moe_gemm_fp8bs_kernel<64, STAGE, SHUFFLED, W4>), grid,
                               dim3(kGemmThreads), 0, stream, g);
            break;
        default:
            AMD_CHECK(false, "block_m must be 16, 32 or 64, got " + std::to_string(bm));
    }
}

template <int STAGE>
static void launch_gemm(int bm, dim3 grid, GemmArgs& g, int shuffled, bool w4,
                        hipStream_t stream) {
    if (w4) {
        if (shuffled)
            launch_gemm_bm<STAGE, true, true>(bm, grid, g, stream);
        else
            launch_gemm_bm<STAGE, false, true>(bm, grid, g, stream);
    } else {
        if (shuffled)
            launch_gemm_bm<STAGE, true, false>(bm, grid, g, stream);
        else
            launch_gemm_bm<STAGE, false, false>(bm, grid, g, stream);
    }
}

void launch_moe_stage1_fp8bs(const uint8_t* a, const float* a_scale, int64_t sa_row,
                             int64_t sa_kb, const uint8_t* w1, const float* w1_scale,
                             const uint8_t* w1_scale_e8m0,
                             const int32_t* sorted_ids, const int32_t* sorted_eids,
                             const int32_t* num_valid, uint8_t* a2, float* a2_scale,
                             int64_t a_rows, int64_t K, int64_t inter, int64_t E, int64_t topk,
                             int64_t block_m, int64_t max_m_blocks, int shuffled,
                             hipStream_t stream, const float* sorted_w, int act) {
    GemmArgs g{};
    g.sorted_w = sorted_w;                 // doweight_stage1 (or NULL)
    g.act = act;
    g.a = a;
    g.a_scale = a_scale;
    g.sa_row = sa_row;
    g.sa_kb = sa_kb;
    g.w = w1;
    g.w_scale = w1_scale;
    g.w_scale8 = w1_scale_e8m0;
    g.sorted_ids = sorted_ids;
    g.sorted_eids = sorted_eids;
    g.num_valid = num_valid;
    g.a2 = a2;
    g.a2_scale = a2_scale;
    g.acc = nullptr;
    g.K = (int)K;
    g.N = (int)(2 * inter);
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    if (max_m_blocks == 0) return;
    dim3 grid((unsigned)(inter / 128), (unsigned)max_m_blocks);
    launch_gemm<1>((int)block_m, grid, g, shuffled, w1_scale_e8m0 != nullptr, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

void launch_moe_stage2_fp8bs(const uint8_t* a2, const float* a2_scale, const uint8_t* w2,
                             const float* w2_scale, const uint8_t* w2_scale_e8m0,
                             const int32_t* sorted_ids,
                             const float* sorted_w, const int32_t* sorted_eids,
                             const int32_t* num_valid, void* acc, int acc_dtype, int64_t a_rows, int64_t inter,
                             int64_t hidden, int64_t E, int64_t topk, int64_t block_m,
                             int64_t max_m_blocks, int shuffled, hipStream_t stream) {
    GemmArgs g{};
    g.a = a2;
    g.a_scale = a2_scale;
    g.sa_row = inter / 128;
    g.sa_kb = 1;
    g.w = w2;
    g.w_scale = w2_scale;
    g.w_scale8 = w2_scale_e8m0;
    g.sorted_ids = sorted_ids;
    g.sorted_w = sorted_w;
    g.sorted_eids = sorted_eids;
    g.num_valid = num_valid;
    g.a2 = nullptr;
    g.a2_scale = nullptr;
    g.acc = acc;
    g.acc_dtype = acc_dtype;
    g.K = (int)inter;
    g.N = (int)hidden;
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    if (max_m_blocks == 0) return;
    dim3 grid((unsigned)(hidden / 128), (unsigned)max_m_blocks);
    launch_gemm<2>((int)block_m, grid, g, shuffled, w2_scale_e8m0 != nullptr, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
