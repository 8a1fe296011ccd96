// Decode-shaped MoE gather-GEMMs for gfx950: the weights stream from HBM
// straight into MFMA operand registers, D K-steps in flight per wave.
//
// Same contract as moe_gemm_fp8bs.hip (stage 1: gate+up GEMM, SiLU*up, bf16
// rounding, fused 1x128 fp8 requant; stage 2: down GEMM, routing weight,
// fp32 atomic accumulate; FP8 128x128 blockscale or MXFP4 weights), for
// M-blocks of 16 or 32 sorted rows -- the token counts where a layer is a
// pass over the touched experts' weights and the MFMA work is small.
//
// Why registers and not LDS: at decode sizes the kernel is bound by how many
// weight bytes each CU keeps in flight.  LDS (160 KB per CU) caps a staged
// pipeline near 128 KB; the register file holds far more.  Every lane loads
// exactly its own MFMA fragments: in the (16,16)-shuffled layout a 16-row
// group's K block is [K/32][2][16 rows][16 B], so lane (q = lane/16,
// r = lane%16) takes the 16-byte pieces at q*512 + r*16 and +256 (fp8; for
// packed fp4 the block is 1 KB and lane l's piece sits at l*16); row-major
// weights give the same fragments as contiguous pieces of row r.  Nothing is
// shared between waves, so there is no barrier in the K loop.
//
// Workgroup: 256 threads = 4 waves; one M-block (BM rows) x 256 weight rows
// (stage 1: 128 gate rows + the matching 128 up rows = 128 outputs; stage 2:
// 256 outputs).  Wave w owns 4 16-row weight groups (stage 1: gate rows
// 32w..32w+31 and the same up rows), so each K step is BM/16 * 4 MFMAs.
// The K loop is unrolled by D with D operand buffers: step k computes from
// buffer k % D and then refills it with step k + D, so D steps of loads are
// always outstanding and the compiler's wait counts target the oldest.
// Weight loads are non-temporal: each weight byte is used by one workgroup
// once, so it should not displace the activations and scales in the caches.
#include <algorithm>
#include <cstdlib>

#include "common.h"
#include "quant_dev.h"

namespace aiter_amd {

namespace stream {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kNCT = 4;      // 16-row weight groups (MFMA column tiles) per wave
constexpr int kMaxKB = 64;   // K <= 8192
constexpr int kMaxSplit = 8; // stage-1 K ranges per tile

struct Args {
    const uint8_t* a;          // activation rows, fp8 [a_rows, K]
    const float* a_scale;      // a_scale[row*sa_row + kb*sa_kb]
    int64_t sa_row;
    int64_t sa_kb;
    const uint8_t* w;          // fp8 [E, N, K] or packed e2m1 [E, N, K/2]
    const float* w_scale;      // [E, N/128, K/128] (fp8 weights)
    const uint8_t* w_scale8;   // [E, N, K/32] e8m0 (MXFP4 weights)
    const int32_t* sorted_ids;
    const float* sorted_w;
    int act;                   // stage 1: activation of gate (kActSilu / kActGelu)
    const int32_t* sorted_eids;
    const int32_t* num_valid;
    uint8_t* a2;
    float* a2_scale;
    void* acc;                 // stage 2 out [T, N]: fp32, bf16 or fp16 (acc_dtype)
    int acc_dtype;
    int K;
    int N;                     // weight rows per expert
    int inter;
    int topk;
    int E;
    int64_t a_rows;
    int ntw;                   // stage 2: 256-column groups per workgroup, one K loop
    // stage 1 split-K: ksplit workgroups per tile, each over KB / ksplit K
    // steps, leave fp32 partial sums in kpart; the last to arrive (counted in
    // kcnt[tile], zero on entry and left zero) adds them in split order and
    // runs the epilogue.  kmb: the M-blocks kpart and kcnt cover.
    int ksplit;
    v4f* kpart;
    int32_t* kcnt;
    int kmb;
    // fused layer (STAGE 3): after stage 1 of its 128-wide slice of the
    // intermediate dim, a workgroup multiplies the slice's requantised rows
    // (kept in LDS) by the matching 128-wide K block of w2 [E, H, inter] for
    // all H outputs and adds w2_route * row into acc2 [tokens, H] (fp32
    // atomics); the per-pair a2 never leaves the workgroup
    const uint8_t* w2;
    const float* w2_scale;     // [E, H/128, inter/128]
    const uint8_t* w2_scale8;  // [E, H, inter/32] e8m0 (MXFP4)
    const float* w2_route;     // sorted routing weights for stage 2 (NULL: 1)
    float* acc2;
    int H;
    // stage 1 / fused: start each workgroup's K walk (and the fused down
    // GEMM's column walk) at a staggered offset
    int krot;
    // stage 1 output form (kOutA2 / kOutAct / kOutGateUp); the last two write
    // rows t * topk + slot of out (kOutAct in out_dtype; kOutGateUp fp32,
    // added atomically into rows the caller zeroed when ksplit > 1)
    int out_mode;
    void* out;
    int out_dtype;
    // sorted_eids holds one expert per BM << eid_shift sorted rows: a caller's
    // 64- or 128-row M-blocks are walked as 32-row ones
    int eid_shift;
    // direct M-blocks, for a layer too small to be worth a sorting launch:
    // with dir_ids set, M-block p holds routing pair p = token * topk + slot
    // of dir_tokens tokens in its first row (the rest is padding), its expert
    // is dir_ids[p] and its routing weight sorted_w[p] (sorted_w is then the
    // caller's [tokens, topk] weights); sorted_ids, sorted_eids and num_valid
    // are not read
    const int32_t* dir_ids;
    int dir_tokens;
    // stage 1 with direct M-blocks: the activations bf16 / fp16 [tokens, K],
    // quantised 1x128 to fp8 by each workgroup into LDS with the quant
    // kernel's arithmetic (a and a_scale are not read)
    const uint16_t* xq;
    int xq_bf16;
};

// One K step of one wave's operands.
template <int NRT, bool W4>
struct Step {
    v4i a[NRT][2];
    v4i b[kNCT][W4 ? 1 : 2];
};

// STAGE 1: gate+up GEMM -> SiLU*up -> a2 (fp8 + 1x128 scales); STAGE 2:
// down GEMM accumulated into acc; STAGE 3: both for one 128-wide slice of
// the intermediate dim per workgroup (the fused layer).
template <int BM, int STAGE, bool SHUFFLED, bool W4, int D, bool XQ = false>
__global__ __launch_bounds__(kThreads) void moe_gemm_stream_kernel(Args g) {
    constexpr int NRT = BM / 16;
    constexpr bool G1 = STAGE != 2;                      // runs the gate+up GEMM
    constexpr bool FUSED = STAGE == 3;
    static_assert(BM == 16 || BM == 32, "stream tiles are 16 or 32 rows");
    __shared__ __attribute__((aligned(16))) float s_sa[kMaxKB * BM];   // [kb][row]
    // weight-scale blocks [block][kb]: stage 1 gate / up (row stride kMaxKB),
    // stage 2 the 2 * ntw 128-column blocks (row stride KB)
    __shared__ float s_sw[2 * kMaxKB];
    __shared__ float s_w2s[FUSED ? kMaxKB : 1];          // fused: w2 scales of the slice's K block
    __shared__ int32_t s_arow[BM];
    __shared__ int64_t s_orow[BM];
    __shared__ float s_w[BM];
    __shared__ float s_amax[kWaves][BM];
    __shared__ int32_t s_tok[FUSED ? BM : 1];            // fused: token of the row (or -1)
    __shared__ float s_rs[FUSED ? BM : 1];               // fused: a2 scale x routing weight
    __shared__ __attribute__((aligned(16))) uint8_t s_q[G1 ? BM * 144 : 16];
    __shared__ int s_last;
    // XQ: the routed row's fp8 codes [K] and 1x128 scales [K / 128]
    __shared__ __attribute__((aligned(16))) uint8_t s_xq[XQ ? kMaxKB * 128 : 16];
    __shared__ float s_xs[XQ ? kMaxKB : 1];
    static_assert(!XQ || (BM == 16 && STAGE == 1), "in-kernel quant: direct 16-row stage 1");

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int lr = lane & 15;
    const int lq = lane >> 4;

    const int mb = blockIdx.y;
    const bool direct = g.dir_ids != nullptr;
    const int nvalid = direct ? g.dir_tokens * g.topk * BM : g.num_valid[0];
    if (mb * BM >= nvalid) return;
    const int tokens = direct ? g.dir_tokens : g.num_valid[1];
    const int e = direct ? g.dir_ids[mb] : g.sorted_eids[mb >> g.eid_shift];
    if (e < 0 || e >= g.E) return;
    // stage 2 may walk ntw consecutive 256-column groups in one K loop (steps
    // s = jt * KB + kb); stage 1 always has one tile, whose K range the S
    // workgroups blockIdx.x = tile * S + ks split
    const int ntw = STAGE == 2 ? g.ntw : 1;
    const int S = G1 ? g.ksplit : 1;
    const int nt = (int)blockIdx.x / S;
    const int ks = (int)blockIdx.x - nt * S;
    if (S > 1 && mb >= g.kmb) return;    // never: a routed M-block holds >= 1 of the tokens*topk pairs
    const int n0 = nt * (G1 ? 128 : 256 * ntw);

    for (int r = tid; r < BM; r += kThreads) {
        // a direct M-block's first row is pair mb, the rest padding
        const uint32_t id =
            !direct ? (uint32_t)g.sorted_ids[mb * BM + r]
            : r == 0 ? ((uint32_t)(mb % g.topk) << 24) | (uint32_t)(mb / g.topk)
                     : ((uint32_t)g.topk << 24) | (uint32_t)tokens;
        const int t = (int)(id & 0xFFFFFFu);
        const int s = (int)(id >> 24);
        const bool valid = t < tokens && s < g.topk;
        const int64_t pair = (int64_t)t * g.topk + s;
        int64_t arow = -1, orow = -1;
        if (valid) {
            arow = G1 ? (int64_t)t : pair;
            orow = G1 ? pair : (int64_t)t;
            if (arow >= g.a_rows) arow = orow = -1;
        }
        s_arow[r] = (int32_t)arow;
        s_orow[r] = orow;
        if constexpr (FUSED) {
            s_tok[r] = orow >= 0 ? t : -1;
            s_rs[r] = orow >= 0 && g.w2_route ? g.w2_route[mb * BM + r] : 1.0f;
        }
        // routing weight of the pair (1 when none is passed: stage 2 without
        // weights, or stage 1 without doweight); stage 1 applies it only when given
        s_w[r] = valid ? (g.sorted_w ? g.sorted_w[direct ? mb : mb * BM + r] : 1.0f) : 0.0f;
    }
    __syncthreads();
    if constexpr (XQ) {
        // the block's routed row (row 0) quantised 1x128: 16 lanes per group,
        // 8 elements each, as the quant kernel does
        const int t = s_arow[0];
        const uint16_t* xr = g.xq + (int64_t)(t < 0 ? 0 : t) * g.K;
        for (int c = tid; c < g.K / 8; c += kThreads) {
            float v[8] = {};
            if (t >= 0) {
                if (g.xq_bf16)
                    load8_f32<true>(xr + c * 8, v);
                else
                    load8_f32<false>(xr + c * 8, v);
            }
            uint2 q;
            const float sc = quant8(v, t >= 0, &q);
            *reinterpret_cast<uint2*>(&s_xq[c * 8]) = q;
            if ((c & 15) == 0) s_xs[c >> 4] = sc;
        }
        __syncthreads();
    }

    const int K = g.K;
    const int KB = K / 128;
    const int KBY = W4 ? K / 2 : K;
    // this workgroup's K steps [kbeg, kend): all of them unless split
    const int KBS = KB / S;
    const int kbeg = ks * KBS;
    const int kend = kbeg + KBS;
    // activation scales of the block's rows, [kb][row]; weight-scale blocks
    // of the tile (stage 1: gate / up; stage 2: the two 128-column halves)
    for (int i = tid; i < BM * KBS; i += kThreads) {
        const int r = i % BM, kb = kbeg + i / BM;
        const int arow = s_arow[r];
        s_sa[kb * BM + r] = arow < 0 ? 0.0f
                            : XQ   ? s_xs[kb]
                                   : g.a_scale[arow * g.sa_row + kb * g.sa_kb];
    }
    if (!W4) {
        // stage 1: blocks gate, up; stage 2: the 2 * ntw 128-column blocks
        const float* wse = g.w_scale + (int64_t)e * (g.N / 128) * KB;
        const int nb0 = n0 / 128;
        const int nb1 = G1 ? (g.inter + n0) / 128 : n0 / 128 + 1;
        for (int i = tid; i < 2 * ntw * KB; i += kThreads) {
            const int blk = i / KB;
            s_sw[blk * (G1 ? kMaxKB : KB) + i % KB] =
                wse[(G1 ? (blk == 0 ? nb0 : nb1) : nb0 + blk) * KB + (i % KB)];
        }
        if constexpr (FUSED) {
            // w2_scale[e, nb, n0 / 128] for the H / 128 output blocks nb
            const int KB2 = g.inter / 128;
            for (int nb = tid; nb < g.H / 128; nb += kThreads)
                s_w2s[nb] = g.w2_scale[((int64_t)e * (g.H / 128) + nb) * KB2 + n0 / 128];
        }
    }
    __syncthreads();

    // ---- per-lane operand sources (K step 0) ----
    const uint8_t* we = g.w + (int64_t)e * g.N * KBY;
    const uint8_t* bsrc[kNCT];
    const uint8_t* bssrc[kNCT];
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) {
        int row0;
        if (G1)
            row0 = ct < 2 ? n0 + 32 * wv + 16 * ct : g.inter + n0 + 32 * wv + 16 * (ct - 2);
        else
            row0 = n0 + 64 * wv + 16 * ct;
        if (W4)
            bsrc[ct] = SHUFFLED ? we + (int64_t)row0 * KBY + lane * 16
                                : we + (int64_t)(row0 + lr) * KBY + lq * 16;
        else
            bsrc[ct] = SHUFFLED ? we + (int64_t)row0 * K + lq * 512 + lr * 16
                                : we + (int64_t)(row0 + lr) * K + lq * 32;
        // A8W4: the e8m0 bytes of the lane's weight row (all four lane quarters)
        bssrc[ct] = W4 ? g.w_scale8 + ((int64_t)e * g.N + row0 + lr) * (K / 32) : nullptr;
    }
    constexpr int BSTEP = W4 ? (SHUFFLED ? 1024 : 64) : (SHUFFLED ? 2048 : 128);
    constexpr int BHI = SHUFFLED ? 256 : 16;       // fp8: offset of the fragment's second half
    constexpr int AHI = W4 ? 64 : 16;              // second half of the A fragment
    const uint8_t* asrc[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
        int arow = s_arow[rt * 16 + lr];
        if (arow < 0) arow = 0;                    // pad rows: any valid row, result unused
        asrc[rt] = g.a + (int64_t)arow * K + (W4 ? lq * 16 : lq * 32);
    }

    // operands of K block kb of column group jt
    auto load = [&](Step<NRT, W4>& s, int kb, int jt) {
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
            const uint8_t* p = bsrc[ct] + (int64_t)kb * BSTEP + (int64_t)jt * 256 * KBY;
            s.b[ct][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
            if (!W4)
                s.b[ct][W4 ? 0 : 1] =
                    __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p + BHI));
        }
        // XQ: A comes from LDS when the step is computed (no registers held)
        if constexpr (!XQ) {
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                const uint8_t* p = asrc[rt] + kb * 128;
                s.a[rt][0] = *reinterpret_cast<const v4i*>(p);
                s.a[rt][1] = *reinterpret_cast<const v4i*>(p + AHI);
            }
        }
    };

    v4f acc[NRT][kNCT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};

    // A8W4 scales of a group of D steps in one load: k-groups 4*kb .. 4*(kb+D)-1
    // of the row (the row and kb*4 are multiples of 4*D bytes, as D divides
    // K/128); step d's byte for this lane is byte lq of dword d
    auto load_sg = [&](int (&dst)[kNCT][D], int kb, int jt) {
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
            const uint8_t* p = bssrc[ct] + kb * 4 + (int64_t)jt * 256 * (K / 32);
            if constexpr (D == 8) {
                const v4i v = *reinterpret_cast<const v4i*>(p);
                const v4i u = *reinterpret_cast<const v4i*>(p + 16);
                dst[ct][0] = v[0], dst[ct][1] = v[1], dst[ct][2] = v[2], dst[ct][3] = v[3];
                dst[ct][4] = u[0], dst[ct][5] = u[1], dst[ct][6] = u[2], dst[ct][7] = u[3];
            } else if constexpr (D == 4) {
                const v4i v = *reinterpret_cast<const v4i*>(p);
                dst[ct][0] = v[0], dst[ct][1] = v[1], dst[ct][2] = v[2], dst[ct][3] = v[3];
            } else if constexpr (D == 2) {
                const v2i v = *reinterpret_cast<const v2i*>(p);
                dst[ct][0] = v[0], dst[ct][1] = v[1];
            } else {
                dst[ct][0] = *reinterpret_cast<const int*>(p);
            }
        }
    };

    auto compute = [&](const Step<NRT, W4>& s, int kb, int jt, const int (&sg)[kNCT][D], int d) {
        // stage 1: tiles 0,1 gate (scale block 0), 2,3 up (block 1); stage 2:
        // the wave's 64 columns lie in 128-column block wv/2 of group jt
        const float sw0 = W4 ? 1.0f : G1 ? s_sw[kb] : s_sw[(2 * jt + (wv >> 1)) * KB + kb];
        const float sw1 =
            W4 ? 1.0f : G1 ? s_sw[kMaxKB + kb] : s_sw[(2 * jt + (wv >> 1)) * KB + kb];
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const v4f sa = *reinterpret_cast<const v4f*>(&s_sa[kb * BM + rt * 16 + 4 * lq]);
            v4i a0 = s.a[rt][0], a1 = s.a[rt][1];
            if constexpr (XQ) {
                // every row of the tile reads the routed row (row 0); the
                // padding rows' results are not stored
                const int o = kb * 128 + (W4 ? lq * 16 : lq * 32);
                a0 = *reinterpret_cast<const v4i*>(&s_xq[o]);
                a1 = *reinterpret_cast<const v4i*>(&s_xq[o + AHI]);
            }
            const v8i af = v8i{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
#pragma unroll
            for (int ct = 0; ct < kNCT; ++ct) {
                v4f blk;
                if (W4) {
                    const v8i bf = v8i{s.b[ct][0][0], s.b[ct][0][1], s.b[ct][0][2],
                                       s.b[ct][0][3], 0, 0, 0, 0};
                    blk = mfma16x16x128_fp8_fp4(af, bf, sg[ct][d] >> (8 * lq));
                } else {
                    const v8i bf = v8i{s.b[ct][0][0], s.b[ct][0][1], s.b[ct][0][2],
                                       s.b[ct][0][3], s.b[ct][W4 ? 0 : 1][0],
                                       s.b[ct][W4 ? 0 : 1][1], s.b[ct][W4 ? 0 : 1][2],
                                       s.b[ct][W4 ? 0 : 1][3]};
                    blk = mfma16x16x128_fp8(af, bf);
                }
                const float sw = ct < 2 ? sw0 : sw1;
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[rt][ct][v] += W4 ? blk[v] * sa[v] : blk[v] * (sa[v] * sw);
            }
        }
    };

    // ---- stage 2 epilogue of column group jt: weighted fp32 atomics ----
    auto epilogue2 = [&](int jt) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = rt * 16 + 4 * lq + v;
                const int64_t t = s_orow[row];
                if (t < 0) continue;
                const float wgt = s_w[row];
                const int64_t dst = t * g.N + n0 + jt * 256 + 64 * wv + lr;
#pragma unroll
                for (int ct = 0; ct < kNCT; ++ct)
                    acc_add(g.acc, g.acc_dtype, dst + 16 * ct, acc[rt][ct][v] * wgt);
            }
    };

    // stage 1: K step k of the walk is K block km(k), the walk rotated by a
    // per-workgroup multiple of D so that concurrent workgroups stream
    // different offsets of their weight rows
    const int krot = G1 && g.krot ? D * (int)((blockIdx.x * 5u + blockIdx.y * 3u) % (KBS / D)) : 0;
    auto km = [&](int k) {
        int r = k - kbeg + krot;
        if (r >= KBS) r -= KBS;
        return kbeg + r;
    };
    Step<NRT, W4> buf[D];
    int sgc[kNCT][D], sgn[kNCT][D];            // A8W4 scales: current / next group
    if (W4) load_sg(sgc, G1 ? km(kbeg) : kbeg, 0);
#pragma unroll
    for (int d = 0; d < D; ++d) load(buf[d], G1 ? km(kbeg + d) : kbeg + d, 0);
    auto next_scales = [&]() {
        if (W4) {
#pragma unroll
            for (int ct = 0; ct < kNCT; ++ct)
#pragma unroll
                for (int d = 0; d < D; ++d) sgc[ct][d] = sgn[ct][d];
        }
    };
    if constexpr (G1) {
        // ---- K loop over [kbeg, kend): D steps in flight ----
        for (int kb0 = kbeg; kb0 < kend - D; kb0 += D) {
            if (W4) load_sg(sgn, km(kb0 + D), 0);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(buf[d], km(kb0 + d), 0, sgc, d);
                load(buf[d], km(kb0 + d + D), 0);
            }
            next_scales();
        }
#pragma unroll
        for (int d = 0; d < D; ++d) compute(buf[d], km(kend - D + d), 0, sgc, d);
        if constexpr (!FUSED) {
            if (g.out_mode == kOutGateUp) {
                // ---- fp32 gate | up rows before the activation; a K range of
                // a split tile adds its partial sums (the rows start at zero) ----
                float* out = reinterpret_cast<float*>(g.out);
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int row = rt * 16 + 4 * lq + v;
                        const int64_t orow = s_orow[row];
                        if (orow < 0) continue;
                        // doweight_stage1 scales gate and up (linear in the partials)
                        const float wg = g.sorted_w ? s_w[row] : 1.0f;
                        float* dst = out + orow * 2 * g.inter + n0 + 32 * wv + lr;
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            const float gate = acc[rt][j][v] * wg;
                            const float up = acc[rt][2 + j][v] * wg;
                            if (S > 1) {
                                unsafeAtomicAdd(dst + 16 * j, gate);
                                unsafeAtomicAdd(dst + g.inter + 16 * j, up);
                            } else {
                                dst[16 * j] = gate;
                                dst[g.inter + 16 * j] = up;
                            }
                        }
                    }
                return;
            }
        }
        if (S > 1) {
            // ---- split-K: publish this K range's partial sums; the last
            // workgroup of the tile to arrive adds all S in split order (the
            // same sum whichever arrives last) and finishes the tile. The
            // partials are stored and loaded with the sc1 cache policy, which
            // makes each access coherent across the XCDs' L2s by itself (the
            // gfx94x/gfx950 form of an agent-scope atomic store / load), and
            // the stores are waited for before the arrival count: an
            // agent-scope release fence would instead write back the XCD's
            // whole L2 in every workgroup.
            constexpr int NP = NRT * kNCT;                 // v4f per thread
            constexpr int kSc1 = 16;                       // buffer cache policy: sc1
            const int64_t tile = (int64_t)mb * (gridDim.x / S) + nt;
            const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
                g.kpart + tile * S * NP * kThreads, (short)0, S * NP * kThreads * 16, 0x00020000);
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int ct = 0; ct < kNCT; ++ct)
                    __builtin_amdgcn_raw_buffer_store_b128(
                        __builtin_bit_cast(v4i, acc[rt][ct]), rp,
                        ((ks * NP + rt * kNCT + ct) * kThreads + tid) * 16, 0, kSc1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0) s_last = atomicAdd(&g.kcnt[tile], 1) == S - 1;
            __syncthreads();
            if (!s_last) return;
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int ct = 0; ct < kNCT; ++ct) {
                    const int j = rt * kNCT + ct;
                    auto part = [&](int q) {
                        return __builtin_bit_cast(
                            v4f, __builtin_amdgcn_raw_buffer_load_b128(
                                     rp, ((q * NP + j) * kThreads + tid) * 16, 0, kSc1));
                    };
                    v4f sum = ks == 0 ? acc[rt][ct] : part(0);
                    for (int q = 1; q < S; ++q) sum += q == ks ? acc[rt][ct] : part(q);
                    acc[rt][ct] = sum;
                }
            if (tid == 0)                                  // zero again for the next call
                __hip_atomic_store(&g.kcnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else {
        // ---- K loop over ntw * KB steps: D steps in flight; a group's last
        // steps are followed by its epilogue while the next group's first D
        // steps load (D divides KB) ----
        const int KBT = KB * ntw;
        int kbl = 0, jt = 0;                   // K block and column group of step kb0
        for (int kb0 = 0; kb0 < KBT - D; kb0 += D) {
            // K block and group of step kb0 + D
            int kbn = kbl + D, jn = jt;
            if (kbn == KB) {
                kbn = 0;
                ++jn;
            }
            if (W4) load_sg(sgn, kbn, jn);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(buf[d], kbl + d, jt, sgc, d);
                load(buf[d], kbn + d, jn);
            }
            next_scales();
            if (jn != jt) {
                epilogue2(jt);
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < kNCT; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};
            }
            kbl = kbn;
            jt = jn;
        }
#pragma unroll
        for (int d = 0; d < D; ++d) compute(buf[d], kbl + d, jt, sgc, d);
        epilogue2(jt);
        return;
    }

    // ---- fused: the down GEMM's weight sources; its first D2 column groups
    // are loaded before the stage-1 epilogue, which they do not depend on ----
    const int H = g.H;
    const int NG = FUSED ? H / 256 : 0;
    // groups of w2 fragments in flight (fp8 fragments take twice the registers)
    constexpr int D2 = W4 || D < 2 ? D : 2;
    const int I2 = g.inter;
    const int kb2 = n0 / 128;
    const int64_t KY2 = W4 ? I2 / 2 : I2;
    const uint8_t* w2e = g.w2 + (int64_t)e * H * KY2;
    const uint8_t* b2src[kNCT];
    const uint8_t* b2ssrc[kNCT];
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) {
        const int row0 = 64 * wv + 16 * ct;
        if (W4)
            b2src[ct] = SHUFFLED ? w2e + row0 * KY2 + lane * 16 + kb2 * 1024
                                 : w2e + (row0 + lr) * KY2 + lq * 16 + kb2 * 64;
        else
            b2src[ct] = SHUFFLED ? w2e + (int64_t)row0 * I2 + lq * 512 + lr * 16 + kb2 * 2048
                                 : w2e + (int64_t)(row0 + lr) * I2 + lq * 32 + kb2 * 128;
        b2ssrc[ct] = W4 ? g.w2_scale8 + ((int64_t)e * H + row0 + lr) * (I2 / 32) + kb2 * 4
                        : nullptr;
    }
    struct B2 {
        v4i b[kNCT][W4 ? 1 : 2];
        int sc[kNCT];
    };
    auto load2 = [&](B2& q, int gi) {
#pragma unroll
        for (int ct = 0; ct < kNCT; ++ct) {
            const uint8_t* p = b2src[ct] + (int64_t)gi * 256 * KY2;
            q.b[ct][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
            if (!W4)
                q.b[ct][W4 ? 0 : 1] =
                    __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p + BHI));
            q.sc[ct] = W4 ? *reinterpret_cast<const int*>(b2ssrc[ct] + (int64_t)gi * 256 * (I2 / 32))
                          : 0;
        }
    };
    // column group of walk position p (rotated like stage 1's K walk)
    const int grot =
        FUSED && g.krot ? (int)((blockIdx.x * 5u + blockIdx.y * 3u) % (unsigned)NG) : 0;
    auto gm = [&](int p) { return p + grot < NG ? p + grot : p + grot - NG; };
    B2 bq[D2];
#pragma unroll
    for (int d = 0; d < D2; ++d)
        if (d < NG) load2(bq[d], gm(d));

    // ---- stage 1 epilogue: silu(gate)*up -> bf16 -> 1x128 fp8 requant ----
    // wave wv holds output columns 32*wv + 16*j + lr (j = 0, 1) of the tile's 128
    if constexpr (!FUSED) {
        if (g.out_mode == kOutAct) {
            // ---- act(gate) * up rows, rounded once to the output dtype ----
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = rt * 16 + 4 * lq + v;
                    const int64_t orow = s_orow[row];
                    if (orow < 0) continue;
                    const float wg = g.sorted_w ? s_w[row] : 1.0f;
                    const int64_t base = orow * g.inter + n0 + 32 * wv + lr;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const float x = acc[rt][j][v] * wg;
                        const float y = (g.act == kActGelu ? gelu_f32(x) : silu_f32(x)) *
                                        (acc[rt][2 + j][v] * wg);
                        const int64_t i = base + 16 * j;
                        if (g.out_dtype == DT_FP32)
                            reinterpret_cast<float*>(g.out)[i] = y;
                        else
                            reinterpret_cast<uint16_t*>(g.out)[i] =
                                g.out_dtype == DT_BF16 ? f32_to_bf16_bits(y) : f32_to_fp16_bits(y);
                    }
                }
            return;
        }
    }
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
    auto row_amax = [&](int row) {
        const float m = __builtin_fmaxf(__builtin_fmaxf(s_amax[0][row], s_amax[1][row]),
                                        __builtin_fmaxf(s_amax[2][row], s_amax[3][row]));
        return __builtin_fmaxf(m, 1e-10f);
    };
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = rt * 16 + 4 * lq + v;
            const float inv = 1.0f / (row_amax(row) * kInvFp8Max);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t b = f32x2_to_fp8x2(h[rt][j][v] * inv, 0.0f) & 0xFFu;
                s_q[row * 144 + 32 * wv + 16 * j + lr] = (uint8_t)b;
            }
        }
    __syncthreads();
    const int I = g.inter;
    if constexpr (!FUSED) {
        for (int q = tid; q < BM * 8; q += kThreads) {
            const int row = q >> 3, part = q & 7;
            const int64_t orow = s_orow[row];
            if (orow < 0) continue;
            *reinterpret_cast<v4i*>(g.a2 + orow * I + n0 + part * 16) =
                *reinterpret_cast<const v4i*>(s_q + row * 144 + part * 16);
            if (part == 0) g.a2_scale[orow * (I / 128) + n0 / 128] = row_amax(row) * kInvFp8Max;
        }
    } else {
        // ---- fused: the slice's requantised rows (s_q, row scale
        // amax / 448) times w2's K block n0 / 128, for all H outputs in
        // 256-column groups (wave wv: columns 64 wv .. 64 wv + 63 of each),
        // D groups of weight fragments in flight; each routed row adds
        // route_w * a2_scale * w2_scale * (a2 . w2) into acc2[token] ----
        float rs[NRT][4];
        float* dst[NRT][4];              // the row's accumulator at this wave's first column
        v8i af[NRT];
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = rt * 16 + 4 * lq + v;
                const int t = s_tok[row];
                rs[rt][v] = t >= 0 ? row_amax(row) * kInvFp8Max * s_rs[row] : 0.0f;
                dst[rt][v] = t >= 0 ? g.acc2 + (int64_t)t * H + 64 * wv + lr : nullptr;
            }
            // fp8 x fp8 pairs K 32q..32q+31; fp8 x fp4 takes K 16q..16q+15 and
            // 64+16q..64+16q+15 in the A lane
            const uint8_t* p = s_q + (rt * 16 + lr) * 144 + (W4 ? lq * 16 : lq * 32);
            const v4i lo = *reinterpret_cast<const v4i*>(p);
            const v4i hi = *reinterpret_cast<const v4i*>(p + (W4 ? 64 : 16));
            af[rt] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        for (int gi0 = 0; gi0 < NG; gi0 += D2) {
#pragma unroll
            for (int d = 0; d < D2; ++d) {
                if (gi0 + d >= NG) break;
                const int gi = gm(gi0 + d);
                const float w2s = W4 ? 1.0f : s_w2s[2 * gi + (wv >> 1)];
#pragma unroll
                for (int ct = 0; ct < kNCT; ++ct) {
#pragma unroll
                    for (int rt = 0; rt < NRT; ++rt) {
                        v4f blk;
                        if (W4) {
                            const v8i bf = v8i{bq[d].b[ct][0][0], bq[d].b[ct][0][1],
                                               bq[d].b[ct][0][2], bq[d].b[ct][0][3], 0, 0, 0, 0};
                            blk = mfma16x16x128_fp8_fp4(af[rt], bf, bq[d].sc[ct] >> (8 * lq));
                        } else {
                            const v8i bf = v8i{bq[d].b[ct][0][0], bq[d].b[ct][0][1],
                                               bq[d].b[ct][0][2], bq[d].b[ct][0][3],
                                               bq[d].b[ct][W4 ? 0 : 1][0], bq[d].b[ct][W4 ? 0 : 1][1],
                                               bq[d].b[ct][W4 ? 0 : 1][2], bq[d].b[ct][W4 ? 0 : 1][3]};
                            blk = mfma16x16x128_fp8(af[rt], bf);
                        }
#pragma unroll
                        for (int v = 0; v < 4; ++v)
                            if (dst[rt][v])
                                unsafeAtomicAdd(dst[rt][v] + gi * 256 + 16 * ct,
                                                blk[v] * (rs[rt][v] * w2s));
                    }
                }
                if (gi0 + d + D2 < NG) load2(bq[d], gm(gi0 + d + D2));
            }
        }
    }
}

// K steps in flight: as many as divide the K-step count, up to the depth
// the registers of the tile allow.
template <int BM>
constexpr int max_depth() { return BM == 16 ? 4 : 2; }

// KB: the K steps of one workgroup (split-K: KB / ksplit).
template <int BM, int STAGE, bool SHUFFLED, bool W4, bool XQ = false>
static void launch_depth(int KB, dim3 grid, const Args& a, hipStream_t s) {
    constexpr int DM = max_depth<BM>();
    // One-token MXFP4 stage 1 (XQ: A from LDS, so a step holds only weight
    // fragments, 16 bytes per lane and column tile) keeps 8 steps in flight.
    // Measured on MI355X at MiMo T=1, alternating: A8W4 layer 30.6-30.8 ->
    // 30.0-30.1 us; FP8 at 8 steps (256 VGPRs + 60 AGPRs, one workgroup per
    // CU) was slower, 43.4-43.5 -> 43.9-44.0 us, so FP8 keeps 4.
    if constexpr (XQ && W4) {
        if (KB % 8 == 0) {
            hipLaunchKernelGGL((moe_gemm_stream_kernel<BM, STAGE, SHUFFLED, W4, 8, XQ>), grid,
                               dim3(kThreads), 0, s, a);
            return;
        }
    }
    if (DM >= 4 && KB % 4 == 0)
        hipLaunchKernelGGL((moe_gemm_stream_kernel<BM, STAGE, SHUFFLED, W4, DM >= 4 ? 4 : 2, XQ>),
                           grid, dim3(kThreads), 0, s, a);
    else if (KB % 2 == 0)
        hipLaunchKernelGGL((moe_gemm_stream_kernel<BM, STAGE, SHUFFLED, W4, 2, XQ>), grid,
                           dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((moe_gemm_stream_kernel<BM, STAGE, SHUFFLED, W4, 1, XQ>), grid,
                           dim3(kThreads), 0, s, a);
}

template <int STAGE, bool SHUFFLED, bool W4>
static void launch_bm(int bm, int KB, dim3 grid, const Args& a, hipStream_t s) {
    if constexpr (STAGE == 1) {
        if (a.xq) {
            AMD_CHECK(bm == 16 && a.dir_ids && a.ksplit == 1,
                      "in-kernel activation quant needs direct 16-row M-blocks, one K range");
            launch_depth<16, STAGE, SHUFFLED, W4, true>(KB, grid, a, s);
            return;
        }
    }
    if (bm == 16)
        launch_depth<16, STAGE, SHUFFLED, W4>(KB, grid, a, s);
    else if (bm == 32)
        launch_depth<32, STAGE, SHUFFLED, W4>(KB, grid, a, s);
    else
        AMD_CHECK(false, "streaming GEMM block_m must be 16 or 32");
}

template <int STAGE>
static void launch(int bm, int KB, dim3 grid, const Args& a, int shuffled, hipStream_t s) {
    const bool w4 = a.w_scale8 != nullptr;
    if (w4) {
        if (shuffled)
            launch_bm<STAGE, true, true>(bm, KB, grid, a, s);
        else
            launch_bm<STAGE, false, true>(bm, KB, grid, a, s);
    } else {
        if (shuffled)
            launch_bm<STAGE, true, false>(bm, KB, grid, a, s);
        else
            launch_bm<STAGE, false, false>(bm, KB, grid, a, s);
    }
}

// Stage 2's 256-column groups per workgroup. A stage-2 workgroup streams
// 256 x K weight bytes per group (MiMo dims: 512 KB fp8, 256 KB fp4, against
// a stage-1 workgroup's 1 MB / 512 KB), so its setup and epilogue weigh more;
// walking groups in one K loop, up to ~1 MB of weights per workgroup, evens
// that out while the grid stays large enough to keep every CU streaming.
// Measured on MI355X (stage 2, MiMo dims): fp8 T=32 231 -> 213 us at two
// groups, T=128 378 -> 351 us; fp4 T=32 128 -> 124 us at four; T=1 15 ->
// 24 us at two (64 workgroups), hence the grid floor. est_blocks: the
// expected M-blocks (at decode sizes one per touched expert).
// fp8 weights follow a table of the single-walk grid's rounds r1 (est_blocks
// x groups / 512 workgroup slots), measured on MI355X at MiMo dims (stage 2,
// us at one / two / four groups): T=8 (r1 = 2) 81.7 / 78.2 / 81.5, T=16
// (r1 = 4) 151 / 148 / 139, T=32 (r1 = 8) 237 / 217 / 222, T=128 (r1 = 32)
// 377 / 352 / 343 -- a walk that leaves one full round wins, and larger
// grids prefer two groups up to ~24 rounds, four beyond.
// AITER_AMD_ST_NTW2 forces a count (tests use it).
static int pick_ntw2(int64_t groups, int64_t KB, int64_t KBY, int64_t est_blocks) {
    if (const char* env = getenv("AITER_AMD_ST_NTW2")) {
        const int c = atoi(env);
        if (c >= 1 && groups % c == 0 && c * KB <= kMaxKB) return c;
    }
    if (KBY == KB * 128) {   // fp8 weights
        const int64_t w1 = est_blocks * groups;     // workgroups of the single walk
        int c = w1 >= 24 * 512 ? 4 : w1 >= 6 * 512 ? 2 : w1 >= 3 * 512 ? 4 : w1 >= 768 ? 2 : 1;
        while (c > 1 && (groups % c != 0 || c * KB > kMaxKB)) c /= 2;
        return c;
    }
    constexpr int64_t kMinWgs = 1024;             // 256 CUs x 2 workgroups x 2 rounds
    constexpr int64_t kTargetBytes = 1 << 20;     // weight bytes per workgroup
    for (int64_t c = std::max<int64_t>(1, kTargetBytes / (256 * KBY)); c > 1; c /= 2) {
        if (groups % c == 0 && c * KB <= kMaxKB && est_blocks * groups / c >= kMinWgs)
            return (int)c;
    }
    return 1;
}

// Stage-1 split-K: K ranges per column tile. Measured on MI355X at MiMo
// dims (stage 1, HIP-event times): a layer that routes to few experts has
// few tiles, and two K ranges per tile help there -- one expert (16 tiles,
// an expert-parallel share at T=2) 18.7 -> 15.9 us, six experts (96 tiles)
// 29.0 -> 26.1 us -- while at 128 tiles (T=1, eight experts) the split
// costs 30.4 -> 33.5 us, and four or eight ranges are slower everywhere
// (each range then streams too few bytes to amortise the setup chain). So
// the K range is halved when fewer than 128 tiles are expected.
// AITER_AMD_ST_KSPLIT1 forces a count (tests use it; a power of two up to
// 8 that divides the K steps into whole rounds of D).
static int pick_ksplit1(int64_t bm, int64_t KB, int64_t n_tiles, int64_t est_blocks) {
    const int64_t D = (bm == 16 && KB % 4 == 0) ? 4 : (KB % 2 == 0 ? 2 : 1);
    auto fits = [&](int64_t c) { return KB % c == 0 && (KB / c) % D == 0; };
    if (const char* env = getenv("AITER_AMD_ST_KSPLIT1")) {
        const int c = atoi(env);
        if (c >= 1 && c <= kMaxSplit && (c & (c - 1)) == 0 && fits(c)) return c;
    }
    constexpr int64_t kSplitBelow = 128;          // expected tiles
    return est_blocks * n_tiles < kSplitBelow && fits(2) ? 2 : 1;
}

// Staggered K walks: measured on MI355X at MiMo dims, T=32 FP8 0.6515 ->
// 0.6386 ms and A8W4 0.3744 -> 0.3680 ms, T=1 and T=8 unchanged (every
// workgroup then reads a different 2 KB of its 64 KB weight-row groups at a
// time). AITER_AMD_ST_ROT=0 turns it off.
static int k_rotation() {
    const char* env = getenv("AITER_AMD_ST_ROT");
    return !env || atoi(env) != 0;
}

// ---- one token: stage 2 with the token's routed slots summed in a workgroup ----
// With one token every routed pair adds into the same output row, so a
// workgroup can own 32 output columns and run the down GEMM of all the
// token's pairs for them: wave w takes slots w, w + 4, ... Each slot's K
// blocks fold into a per-slot fp32 sum (a2 scale x w2 scale per 128-K block,
// as in the streaming kernel), which is weighted and added to the wave's
// row; the four waves' rows meet in LDS and are added in wave order, rounded
// once and stored (plus the addend when one is given). No atomics, no
// accumulator and no finishing pass, and the summation order is fixed.
// Measured on MI355X at MiMo T=1 against the streaming stage 2 with its fp32
// atomics and finishing pass: FP8 45.0 -> 43.6 us; MXFP4 29.9-30.0 -> 29.5
// us with each lane loading its rows' e8m0 bytes of the D steps in flight at
// once (4 D bytes, as the streaming kernel does), where a load per step had
// made it slower (33.7 us).
struct TokArgs {
    const uint8_t* a2;          // fp8 [topk, I]: the token's pairs
    const float* a2_scale;      // [topk, I / 128]
    const uint8_t* w2;          // fp8 [E, H, I] or packed e2m1 [E, H, I / 2]
    const float* w2_scale;      // [E, H / 128, I / 128] (fp8 weights)
    const uint8_t* w2_scale8;   // [E, H, I / 32] e8m0 (MXFP4 weights)
    const int32_t* ids;         // [topk] experts of the token's slots
    const float* route_w;       // [topk] routing weights, or NULL (weights applied in stage 1)
    void* out;                  // [H] bf16 / fp16
    int out_dtype;
    const void* addend;         // [H] added before the rounding, or NULL (may alias out)
    int topk;
    int H;
    int I;
    int E;
};

template <bool W4>
struct TokStep {
    v4i a[2];
    v4i b[2][W4 ? 1 : 2];
    float sc;                   // a2 scale (x w2 scale for fp8 weights)
};

template <bool SHUFFLED, bool W4, int D>
__global__ __launch_bounds__(kThreads) void moe_token_stage2_kernel(TokArgs g) {
    __shared__ float s_row[kWaves][32];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int lr = lane & 15;
    const int lq = lane >> 4;
    const int c0 = blockIdx.x * 32;
    const int I = g.I;
    const int KB = I / 128;
    const int KBY = W4 ? I / 2 : I;
    constexpr int BSTEP = W4 ? (SHUFFLED ? 1024 : 64) : (SHUFFLED ? 2048 : 128);
    constexpr int BHI = SHUFFLED ? 256 : 16;
    constexpr int AHI = W4 ? 64 : 16;
    const int nsl = wv < g.topk ? (g.topk - wv + kWaves - 1) / kWaves : 0;
    const int nsteps = nsl * KB;          // a multiple of D (D divides KB)

    // step q: slot wv + 4 (q / KB), K block q % KB; eraw is that slot's expert
    // id, fetched a slot ahead so that no weight load waits on it
    auto load = [&](TokStep<W4>& st, int q, int eraw) __attribute__((always_inline)) {
        const int sl = wv + kWaves * (q / KB);
        const int kb = q - (q / KB) * KB;
        const bool ok = eraw >= 0 && eraw < g.E;
        const int e = ok ? eraw : 0;
        const uint8_t* ap = g.a2 + (int64_t)sl * I + kb * 128 + (W4 ? lq * 16 : lq * 32);
        const v4i a0 = *reinterpret_cast<const v4i*>(ap);
        const v4i a1 = *reinterpret_cast<const v4i*>(ap + AHI);
        // a slot routed outside [0, E) contributes nothing: zero operands
        st.a[0] = ok ? a0 : v4i{0, 0, 0, 0};
        st.a[1] = ok ? a1 : v4i{0, 0, 0, 0};
        const uint8_t* we = g.w2 + (int64_t)e * g.H * KBY;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const int row0 = c0 + 16 * ct;
            const uint8_t* bp;
            if (W4)
                bp = SHUFFLED ? we + (int64_t)row0 * KBY + lane * 16
                              : we + (int64_t)(row0 + lr) * KBY + lq * 16;
            else
                bp = SHUFFLED ? we + (int64_t)row0 * I + lq * 512 + lr * 16
                              : we + (int64_t)(row0 + lr) * I + lq * 32;
            bp += (int64_t)kb * BSTEP;
            st.b[ct][0] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bp));
            if (!W4)
                st.b[ct][W4 ? 0 : 1] =
                    __builtin_nontemporal_load(reinterpret_cast<const v4i*>(bp + BHI));
        }
        const float sa = g.a2_scale[(int64_t)sl * KB + kb];
        st.sc = W4 ? sa : sa * g.w2_scale[((int64_t)e * (g.H / 128) + c0 / 128) * KB + kb];
    };
    // MXFP4: the e8m0 dwords of the D steps from q (one slot, kb a multiple
    // of D) of the lane's two weight rows; step d's byte for this lane is
    // byte lq of dword d
    auto load_e8 = [&](int (&dst)[2][D], int q, int eraw) __attribute__((always_inline)) {
        if constexpr (W4) {
            const int kb = q - (q / KB) * KB;
            const int e = eraw >= 0 && eraw < g.E ? eraw : 0;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                const uint8_t* p =
                    g.w2_scale8 + ((int64_t)e * g.H + c0 + 16 * ct + lr) * (I / 32) + kb * 4;
#pragma unroll
                for (int h = 0; h < (D + 3) / 4; ++h) {
                    if constexpr (D >= 4) {
                        const v4i v = *reinterpret_cast<const v4i*>(p + 16 * h);
#pragma unroll
                        for (int i = 0; i < 4; ++i) dst[ct][4 * h + i] = v[i];
                    } else if constexpr (D == 2) {
                        const v2i v = *reinterpret_cast<const v2i*>(p);
                        dst[ct][0] = v[0], dst[ct][1] = v[1];
                    } else {
                        dst[ct][0] = *reinterpret_cast<const int*>(p);
                    }
                }
            }
        }
    };
    v4f pacc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    v4f row[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    int e8c[2][D], e8n[2][D];               // MXFP4: the steps computed / loaded
    auto compute = [&](const TokStep<W4>& st, int d) __attribute__((always_inline)) {
        const v8i af = v8i{st.a[0][0], st.a[0][1], st.a[0][2], st.a[0][3],
                           st.a[1][0], st.a[1][1], st.a[1][2], st.a[1][3]};
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            v4f blk;
            if constexpr (W4) {
                const v8i bf = v8i{st.b[ct][0][0], st.b[ct][0][1], st.b[ct][0][2],
                                   st.b[ct][0][3], 0, 0, 0, 0};
                blk = mfma16x16x128_fp8_fp4(af, bf, e8c[ct][d] >> (8 * lq));
            } else {
                const v8i bf = v8i{st.b[ct][0][0], st.b[ct][0][1], st.b[ct][0][2],
                                   st.b[ct][0][3], st.b[ct][W4 ? 0 : 1][0],
                                   st.b[ct][W4 ? 0 : 1][1], st.b[ct][W4 ? 0 : 1][2],
                                   st.b[ct][W4 ? 0 : 1][3]};
                blk = mfma16x16x128_fp8(af, bf);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) pacc[ct][v] += blk[v] * st.sc;
        }
    };
    // a slot's K blocks are done: weight its sum into the row
    auto fold_slot = [&](float rw) __attribute__((always_inline)) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
            for (int v = 0; v < 4; ++v) row[ct][v] += pacc[ct][v] * rw;
            pacc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto slot_id = [&](int j) { return j < nsl ? g.ids[wv + kWaves * j] : 0; };
    auto slot_w = [&](int j) { return g.route_w ? g.route_w[wv + kWaves * j] : 1.0f; };
    TokStep<W4> buf[D];
    if (nsteps > 0) {
        // D divides KB, so a group of D steps lies in one slot and slots
        // change only between groups
        int jl = 0;                         // slot of the steps being loaded
        int el = slot_id(0), en = slot_id(1);
        float rw = slot_w(0);               // weight of the slot being computed
        load_e8(e8c, 0, el);
#pragma unroll
        for (int d = 0; d < D; ++d) load(buf[d], d, el);
        int q0 = 0;
        for (; q0 < nsteps - D; q0 += D) {
            const bool slot_end = (q0 + D) % KB == 0;
            if (slot_end) {                 // this group's loads start slot jl + 1
                ++jl;
                el = en;
                en = slot_id(jl + 1);
            }
            load_e8(e8n, q0 + D, el);
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute(buf[d], d);
                load(buf[d], q0 + D + d, el);
            }
            if constexpr (W4) {
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int d = 0; d < D; ++d) e8c[ct][d] = e8n[ct][d];
            }
            if (slot_end) {
                fold_slot(rw);
                rw = slot_w(jl);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) compute(buf[d], d);
        fold_slot(rw);
    }
    // output row 0 sits in lanes lq == 0, element 0: column lr of each tile
    if (lq == 0) {
        s_row[wv][lr] = row[0][0];
        s_row[wv][16 + lr] = row[1][0];
    }
    __syncthreads();
    if (tid < 32) {
        float v = s_row[0][tid];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v += s_row[w][tid];
        uint16_t* o = reinterpret_cast<uint16_t*>(g.out) + c0 + tid;
        const uint16_t* ad = reinterpret_cast<const uint16_t*>(g.addend);
        if (g.out_dtype == DT_BF16) {
            if (ad) v += bf16_bits_to_f32(ad[c0 + tid]);
            *o = f32_to_bf16_bits(v);
        } else {
            if (ad) v += fp16_bits_to_f32(ad[c0 + tid]);
            *o = f32_to_fp16_bits(v);
        }
    }
}

// D K steps in flight per wave (D divides the K steps): 8 where it can, as
// many weight bytes in flight as the streaming stage 2 (measured on MI355X
// at MiMo T=1: the layer 43.6 us at 8, 44.8 us at 4).
template <bool SHUFFLED, bool W4>
static void launch_token_stage2(int KB, int grid, const TokArgs& a, hipStream_t s) {
    if (KB % 8 == 0)
        hipLaunchKernelGGL((moe_token_stage2_kernel<SHUFFLED, W4, 8>), dim3(grid), dim3(kThreads),
                           0, s, a);
    else if (KB % 4 == 0)
        hipLaunchKernelGGL((moe_token_stage2_kernel<SHUFFLED, W4, 4>), dim3(grid), dim3(kThreads),
                           0, s, a);
    else if (KB % 2 == 0)
        hipLaunchKernelGGL((moe_token_stage2_kernel<SHUFFLED, W4, 2>), dim3(grid), dim3(kThreads),
                           0, s, a);
    else
        hipLaunchKernelGGL((moe_token_stage2_kernel<SHUFFLED, W4, 1>), dim3(grid), dim3(kThreads),
                           0, s, a);
}

}  // namespace stream

bool stream_supported(int64_t block_m, int64_t K);

int stream_stage1_ksplit(int64_t block_m, int64_t K, int64_t inter, int64_t est_blocks) {
    if (!stream_supported(block_m, K)) return 1;
    return stream::pick_ksplit1(block_m, K / 128, inter / 128, est_blocks);
}

// Partial sums of split-K stage 1: per tile and split, 256 threads x
// (block_m / 16) x 4 v4f.
int64_t stream_ksplit_part_bytes(int64_t block_m, int64_t mblocks, int64_t inter, int64_t ksplit) {
    if (ksplit <= 1) return 0;
    return mblocks * (inter / 128) * ksplit * stream::kThreads * (block_m / 16) * stream::kNCT * 16;
}

// Stage 2 of a one-token layer straight into its bf16 / fp16 output row (see
// moe_token_stage2_kernel): a2 [topk, inter] fp8 with its 1x128 scales, w2
// fp8 with 128x128 scales or MXFP4 with e8m0 bytes (w2_scale_e8m0 given), the
// token's expert ids and routing weights (NULL: applied in stage 1), out and
// an optional addend [hidden]. hidden a multiple of 32, inter of 128.
void launch_moe_token_stage2(const uint8_t* a2, const float* a2_scale, const uint8_t* w2,
                             const float* w2_scale, const uint8_t* w2_scale_e8m0,
                             const int32_t* ids, const float* route_w, void* out, int out_dtype,
                             const void* addend, int64_t topk, int64_t hidden, int64_t inter,
                             int64_t E, int shuffled, hipStream_t stream) {
    AMD_CHECK(hidden % 32 == 0 && hidden > 0, "model_dim must be a multiple of 32");
    AMD_CHECK(inter % 128 == 0 && inter > 0 && inter / 128 <= stream::kMaxKB,
              "inter_dim must be a multiple of 128 up to 8192");
    AMD_CHECK(topk >= 1 && topk <= 32, "topk must be in [1, 32]");
    AMD_CHECK(out_dtype == DT_BF16 || out_dtype == DT_FP16, "out dtype must be bf16 or fp16");
    AMD_CHECK(w2_scale_e8m0 ? true : w2_scale != nullptr, "w2 scales are NULL");
    stream::TokArgs g{};
    g.a2 = a2;
    g.a2_scale = a2_scale;
    g.w2 = w2;
    g.w2_scale = w2_scale;
    g.w2_scale8 = w2_scale_e8m0;
    g.ids = ids;
    g.route_w = route_w;
    g.out = out;
    g.out_dtype = out_dtype;
    g.addend = addend;
    g.topk = (int)topk;
    g.H = (int)hidden;
    g.I = (int)inter;
    g.E = (int)E;
    const int KB = (int)(inter / 128), grid = (int)(hidden / 32);
    const bool w4 = w2_scale_e8m0 != nullptr;
    if (w4)
        shuffled ? stream::launch_token_stage2<true, true>(KB, grid, g, stream)
                 : stream::launch_token_stage2<false, true>(KB, grid, g, stream);
    else
        shuffled ? stream::launch_token_stage2<true, false>(KB, grid, g, stream)
                 : stream::launch_token_stage2<false, false>(KB, grid, g, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

// 16/32-row M-blocks, K a multiple of 128 up to 8192; stage 2 also needs
// 256-column output tiles (model_dim % 256 == 0).
bool stream_supported(int64_t block_m, int64_t K) {
    return (block_m == 16 || block_m == 32) && K > 0 && K % 128 == 0 &&
           K / 128 <= stream::kMaxKB;
}

void launch_moe_stage1_stream(const uint8_t* a, const float* a_scale, int64_t sa_row,
                              int64_t sa_kb, const uint8_t* w1, const float* w1_scale,
                              const uint8_t* w1_scale_e8m0, const int32_t* sorted_ids,
                              const int32_t* sorted_eids, const int32_t* num_valid, uint8_t* a2,
                              float* a2_scale, int64_t a_rows, int64_t K, int64_t inter,
                              int64_t E, int64_t topk, int64_t block_m, int64_t max_m_blocks,
                              int shuffled, hipStream_t stream, const float* sorted_w, int act,
                              int ksplit, void* kpart, int32_t* kcnt, int64_t kmb,
                              StreamDirect direct) {
    stream::Args g{};
    g.ksplit = ksplit > 1 ? ksplit : 1;
    AMD_CHECK(!direct.ids || (block_m == 16 && g.ksplit == 1 && max_m_blocks == direct.tokens * topk),
              "direct M-blocks need block_m 16, one K range and one M-block per pair");
    AMD_CHECK(!direct.xq || direct.xq_dtype == DT_BF16 || direct.xq_dtype == DT_FP16,
              "activations to quantise must be bf16 or fp16");
    g.dir_ids = direct.ids;
    g.dir_tokens = direct.tokens;
    g.xq = reinterpret_cast<const uint16_t*>(direct.xq);
    g.xq_bf16 = direct.xq_dtype == DT_BF16;
    AMD_CHECK(g.ksplit == 1 || (kpart && kcnt && kmb > 0 && (K / 128) % g.ksplit == 0),
              "split-K needs partial and counter buffers and K steps divisible by the split");
    g.kpart = reinterpret_cast<v4f*>(kpart);
    g.kcnt = kcnt;
    g.kmb = (int)std::min<int64_t>(kmb, max_m_blocks);
    g.krot = stream::k_rotation();
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
    g.K = (int)K;
    g.N = (int)(2 * inter);
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    if (max_m_blocks == 0) return;
    // split-K: only the M-blocks the partial buffers cover can hold routed rows
    const int64_t mblocks = g.ksplit > 1 ? g.kmb : max_m_blocks;
    const dim3 grid((unsigned)(inter / 128 * g.ksplit), (unsigned)mblocks);
    stream::launch<1>((int)block_m, (int)(K / 128 / g.ksplit), grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

// Stage 1 writing rows t * topk + slot of `out` instead of the fp8 a2:
// act(gate) * up [pairs, inter] in out_dtype (kOutAct) or fp32 gate | up
// [pairs, 2 * inter] (kOutGateUp). M-blocks of block_m 16, 32, 64 or 128
// sorted rows (64 and 128 are walked as 32-row blocks of the same expert).
// ksplit > 1 (kOutGateUp only): the K range of a tile is split ksplit ways,
// each adding its partial sums into out, whose rows must be zero on entry.
void launch_moe_stage1_stream_rows(const uint8_t* a, const float* a_scale, int64_t sa_row,
                                   int64_t sa_kb, const uint8_t* w1, const float* w1_scale,
                                   const uint8_t* w1_scale_e8m0, const int32_t* sorted_ids,
                                   const int32_t* sorted_eids, const int32_t* num_valid,
                                   void* out, int out_mode, int out_dtype, int64_t a_rows,
                                   int64_t K, int64_t inter, int64_t E, int64_t topk,
                                   int64_t block_m, int64_t max_m_blocks, int shuffled,
                                   hipStream_t stream, const float* sorted_w, int act,
                                   int ksplit) {
    AMD_CHECK(out_mode == kOutAct || out_mode == kOutGateUp, "unknown stage-1 output form");
    AMD_CHECK(block_m == 16 || block_m == 32 || block_m == 64 || block_m == 128,
              "block_m must be 16, 32, 64 or 128");
    AMD_CHECK(K > 0 && K % 128 == 0 && K / 128 <= stream::kMaxKB,
              "model_dim must be a multiple of 128 up to 8192");
    const int KB = (int)(K / 128);
    const int S = ksplit > 1 ? ksplit : 1;
    AMD_CHECK(S == 1 || (out_mode == kOutGateUp && KB % S == 0),
              "split-K needs the fp32 gate|up output and K / 128 divisible by the split");
    const int bmk = block_m <= 32 ? (int)block_m : 32;
    const int shift = block_m == 128 ? 2 : block_m == 64 ? 1 : 0;
    stream::Args g{};
    g.ksplit = S;
    g.kmb = (int)(max_m_blocks << shift);
    g.krot = stream::k_rotation();
    g.sorted_w = sorted_w;
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
    g.out_mode = out_mode;
    g.out = out;
    g.out_dtype = out_dtype;
    g.eid_shift = shift;
    g.K = (int)K;
    g.N = (int)(2 * inter);
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    if (max_m_blocks == 0) return;
    const dim3 grid((unsigned)(inter / 128 * S), (unsigned)(max_m_blocks << shift));
    stream::launch<1>(bmk, KB / S, grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

void launch_moe_stage2_stream(const uint8_t* a2, const float* a2_scale, const uint8_t* w2,
                              const float* w2_scale, const uint8_t* w2_scale_e8m0,
                              const int32_t* sorted_ids, const float* sorted_w,
                              const int32_t* sorted_eids, const int32_t* num_valid, void* acc, int acc_dtype,
                              int64_t a_rows, int64_t inter, int64_t hidden, int64_t E,
                              int64_t topk, int64_t block_m, int64_t max_m_blocks, int shuffled,
                              hipStream_t stream) {
    stream::Args g{};
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
    g.acc = acc;
    g.acc_dtype = acc_dtype;
    g.K = (int)inter;
    g.N = (int)hidden;
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    if (max_m_blocks == 0) return;
    g.ntw = stream::pick_ntw2(hidden / 256, inter / 128, w2_scale_e8m0 ? inter / 2 : inter,
                              std::min<int64_t>(a_rows, E));
    const dim3 grid((unsigned)(hidden / 256 / g.ntw), (unsigned)max_m_blocks);
    stream::launch<2>((int)block_m, (int)(inter / 128), grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

// The fused layer on the stream kernel: 16/32-row M-blocks, model_dim a
// multiple of 256 up to 8192.
bool stream_fused_supported(int64_t block_m, int64_t hidden, int64_t inter) {
    return stream_supported(block_m, hidden) && hidden % 256 == 0 && inter % 128 == 0;
}

// One launch for both GEMMs of a decode-sized layer (see Args::w2): grid =
// 128-wide intermediate slices (x ksplit) x M-blocks. acc2 [tokens, hidden]
// fp32 must be zero on entry (the sorting launch clears it); sw1: routing
// weights applied before the activation (doweight_stage1) or NULL; sw2: the
// routing weights of the down GEMM or NULL.
void launch_moe_fused_stream(const uint8_t* a, const float* a_scale, int64_t sa_row,
                             int64_t sa_kb, const uint8_t* w1, const float* w1_scale,
                             const uint8_t* w1_scale_e8m0, const uint8_t* w2,
                             const float* w2_scale, const uint8_t* w2_scale_e8m0,
                             const int32_t* sorted_ids, const float* sw1, const float* sw2,
                             const int32_t* sorted_eids, const int32_t* num_valid, float* acc2,
                             int64_t a_rows, int64_t hidden, int64_t inter, int64_t E,
                             int64_t topk, int64_t block_m, int64_t max_m_blocks, int shuffled,
                             hipStream_t stream, int act, int ksplit, void* kpart, int32_t* kcnt,
                             int64_t kmb) {
    AMD_CHECK(stream_fused_supported(block_m, hidden, inter),
              "the fused layer needs block_m 16 or 32 and model_dim a multiple of 256 up to 8192");
    AMD_CHECK((w1_scale_e8m0 != nullptr) == (w2_scale_e8m0 != nullptr),
              "w1 and w2 must both be fp8 or both MXFP4");
    stream::Args g{};
    g.ksplit = ksplit > 1 ? ksplit : 1;
    AMD_CHECK(g.ksplit == 1 || (kpart && kcnt && kmb > 0 && (hidden / 128) % g.ksplit == 0),
              "split-K needs partial and counter buffers and K steps divisible by the split");
    g.kpart = reinterpret_cast<v4f*>(kpart);
    g.kcnt = kcnt;
    g.kmb = (int)std::min<int64_t>(kmb, max_m_blocks);
    g.krot = stream::k_rotation();
    g.sorted_w = sw1;
    g.w2_route = sw2;
    g.act = act;
    g.a = a;
    g.a_scale = a_scale;
    g.sa_row = sa_row;
    g.sa_kb = sa_kb;
    g.w = w1;
    g.w_scale = w1_scale;
    g.w_scale8 = w1_scale_e8m0;
    g.w2 = w2;
    g.w2_scale = w2_scale;
    g.w2_scale8 = w2_scale_e8m0;
    g.acc2 = acc2;
    g.H = (int)hidden;
    g.sorted_ids = sorted_ids;
    g.sorted_eids = sorted_eids;
    g.num_valid = num_valid;
    g.K = (int)hidden;
    g.N = (int)(2 * inter);
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    if (max_m_blocks == 0) return;
    const int64_t mblocks = g.ksplit > 1 ? g.kmb : max_m_blocks;
    const dim3 grid((unsigned)(inter / 128 * g.ksplit), (unsigned)mblocks);
    stream::launch<3>((int)block_m, (int)(hidden / 128 / g.ksplit), grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
