// Prefill-shaped MoE gather-GEMMs for gfx950 (64/128-row M-blocks): weight
// fragments stream straight into registers, activations through LDS.
//
// Same contract as moe_gemm_fp8bs.hip (stage 1: gate+up GEMM, SiLU*up, bf16
// rounding, fused 1x128 fp8 requant; stage 2: down GEMM, routing weight,
// fp32 atomic accumulate; FP8 128x128 blockscale or MXFP4 weights).
//
// What bounds this shape on MI355X, measured: LDS reads run at ~128 B/clk
// per CU, so a 2x4-wave tile that reads both operands from LDS spends as
// long reading LDS as the MFMAs take; and VALU issue barely overlaps MFMA --
// 16x16x128 fp8 MFMAs with the 4 fp32 FMAs per MFMA that the per-128-K
// block scales need reach ~65% of peak with two waves per SIMD.  So:
//   * B (weights) never touches LDS: every lane loads its own MFMA
//     fragments from global memory (the (16,16) layout puts them in 16-byte
//     pieces), D K-steps ahead in registers.  The two M-waves that share a
//     weight group issue the same addresses back to back, so the second
//     read hits the CU's L1.
//   * A (token rows, gathered) is loaded to registers one step ahead and
//     written to one of two LDS stages, fragment-major with a per-row swap
//     of the 16-byte halves ((r>>2 ^ r>>3) & 1) so 16-byte reads are
//     conflict-free; one barrier per K step.
//   * The products a_scale[row, kb] * w_scale[block, kb] of the whole K
//     range are computed once per workgroup into LDS, so the K loop's VALU
//     work is the 4 FMAs per MFMA and little else.
// Workgroup: 512 threads = 2 (M) x 4 (N) waves, two per SIMD; tile BM rows
// x 256 weight rows (stage 1: 128 gate rows + the matching 128 up rows = 128
// outputs; stage 2: 256 outputs); each wave (BM/2) x 64.  Tile order is
// XCD-aware: workgroup L runs on XCD L % 8, and each XCD owns n_tiles/8
// column tiles of every M-block so an expert's weight slice stays in its L2.
#include "common.h"

namespace aiter_amd {

namespace pf {

constexpr int kThreads = 512;
constexpr int kWaves = 8;
constexpr int kMaxKB = 64;     // K <= 8192

struct Args {
    const uint8_t* a;
    const float* a_scale;
    int64_t sa_row;            // a_scale element strides (row, K block)
    int64_t sa_kb;
    const uint8_t* w;
    const float* w_scale;      // [E, N/128, K/128] (fp8 weights)
    const uint8_t* w_scale8;   // [E, N, K/32] e8m0 (MXFP4 weights)
    const int32_t* sorted_ids;
    const float* sorted_w;
    const int32_t* sorted_eids;
    const int32_t* num_valid;
    uint8_t* a2;
    float* a2_scale;
    float* acc;
    int K;
    int N;                     // weight rows per expert
    int inter;
    int topk;
    int E;
    int64_t a_rows;
    int n_tiles;
    int m_blocks;
};

__device__ __forceinline__ int frag_swap(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

// Raw buffer resource over [base, base + bytes): loads take a 32-bit lane
// offset plus a wave-uniform K-step offset, and read 0 past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// Waves along M in the 8-wave workgroup (template WM): 2 -> 2 x 4 waves of
// (BM/2) x 64 (the two M-waves of a SIMD load the same weight fragments, the
// second from L1); 1 -> each wave owns all BM rows and 32 weight rows (no
// weight fragment is loaded twice, every wave reads all A rows from LDS).
// Measured on MI355X: 2 x 4 for stage 1 (K = 4096), 1 x 8 for stage 2.

// One K step of a wave's B operand (NCT 16-row weight groups).
template <bool W4, int NCT>
struct BStep {
    v4i b[NCT][W4 ? 1 : 2];
    int bs[NCT];
};

template <int BM, int STAGE, bool SHUFFLED, bool W4, int D, int kWM>
__global__ __launch_bounds__(kThreads, 1) void moe_gemm_prefill_kernel(Args g) {
    constexpr int WN = kWaves / kWM;                     // waves along N
    constexpr int NCT = 16 / WN;                         // 16-row weight groups per wave
    constexpr int NRT = BM / 16 / kWM;                   // 16-row MFMA tiles per wave
    constexpr int A_BYTES = BM * 128;
    constexpr int A_PT = A_BYTES / 16 / kThreads;        // 16-byte A pieces per thread
    constexpr int NH = W4 ? 1 : 2;                       // scale products per (row, kb)
    static_assert(BM == 64 || BM == 128, "prefill tiles are 64 or 128 rows");
    static_assert(A_PT >= 1, "one A piece per thread at least");
    __shared__ __attribute__((aligned(1024))) uint8_t s_a[2][A_BYTES];
    __shared__ __attribute__((aligned(16))) float s_sc[kMaxKB * NH * BM];   // [kb][h][row]
    __shared__ int32_t s_arow[BM];
    __shared__ int64_t s_orow[BM];
    __shared__ float s_w[BM];
    __shared__ float s_amax[WN][BM];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int wm = wv / WN;
    const int wn = wv % WN;
    const int lr = lane & 15;
    const int lq = lane >> 4;

    // ---- XCD-aware tile order ----
    const int L = blockIdx.x;
    int nt, mb;
    if ((g.n_tiles & 7) == 0) {
        const int per = g.n_tiles >> 3;
        const int idx = L >> 3;
        nt = (L & 7) * per + idx % per;
        mb = idx / per;
    } else {
        nt = L % g.n_tiles;
        mb = L / g.n_tiles;
    }
    if (mb >= g.m_blocks) return;
    const int nvalid = g.num_valid[0];
    if (mb * BM >= nvalid) return;
    const int tokens = g.num_valid[1];
    const int e = g.sorted_eids[mb];
    if (e < 0 || e >= g.E) return;
    const int n0 = STAGE == 1 ? nt * 128 : nt * 256;

    for (int r = tid; r < BM; r += kThreads) {
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
        s_arow[r] = (int32_t)arow;
        s_orow[r] = orow;
        s_w[r] = STAGE == 2 && valid ? g.sorted_w[mb * BM + r] : 0.0f;
    }
    __syncthreads();

    const int K = g.K;
    const int KB = K / 128;
    const int KBY = W4 ? K / 2 : K;

    // ---- scale products of the whole K range: [kb][h][row] ----
    // fp8: h = 0 / 1 are stage 1's gate / up blocks or stage 2's two
    // 128-column blocks; A8W4: the activation scale only (the weight scale
    // goes into the MFMA)
    {
        const float* wse = W4 ? nullptr : g.w_scale + (int64_t)e * (g.N / 128) * KB;
        const int nb0 = n0 / 128;
        const int nb1 = STAGE == 1 ? (g.inter + n0) / 128 : n0 / 128 + 1;
        for (int i = tid; i < KB * NH * BM; i += kThreads) {
            const int r = i % BM;
            const int h = (i / BM) % NH;
            const int kb = i / (NH * BM);
            const int arow = s_arow[r];
            float v = arow >= 0 ? g.a_scale[arow * g.sa_row + kb * g.sa_kb] : 0.0f;
            if (!W4) v *= wse[(h == 0 ? nb0 : nb1) * KB + kb];
            s_sc[i] = v;
        }
    }

    // ---- A staging: piece p = tid + j*512 -> 1 KB chunk c = p/64 (rows
    // 32*(c % (BM/32)) .. +31 of K quarter kq = c / (BM/32)), position l = p%64
    // (row 32*.. + l/2, half l&1 of its 32-byte slot, swapped per row) ----
    const __amdgpu_buffer_rsrc_t ra = rsrc(g.a, g.a_rows * K);
    uint32_t a_off[A_PT];
    int a_dst[A_PT];
#pragma unroll
    for (int j = 0; j < A_PT; ++j) {
        const int p = tid + j * kThreads;
        const int c = p >> 6, l = p & 63;
        const int kq = c / (BM / 32);
        const int row = (c % (BM / 32)) * 32 + (l >> 1);
        const int h = (l & 1) ^ frag_swap(row);
        int arow = s_arow[row];
        if (arow < 0) arow = 0;                          // pad rows: any valid row, result unused
        a_off[j] = (uint32_t)arow * (uint32_t)K + (uint32_t)(W4 ? kq * 16 + h * 64 : kq * 32 + h * 16);
        a_dst[j] = c * 1024 + l * 16;
    }

    // ---- B sources of this wave's four 16-row weight groups ----
    const int KS = K / 32;                               // e8m0 bytes per weight row
    const __amdgpu_buffer_rsrc_t rb = rsrc(g.w + (int64_t)e * g.N * KBY, (int64_t)g.N * KBY);
    const __amdgpu_buffer_rsrc_t rbs =
        rsrc(W4 ? g.w_scale8 + (int64_t)e * g.N * KS : g.w, W4 ? (int64_t)g.N * KS : 0);
    uint32_t boff[NCT], bsoff[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        // stage 1: the wave's gate tiles (ct < NCT/2) and the matching up tiles
        int row0;
        if (STAGE == 1)
            row0 = ct < NCT / 2 ? n0 + 16 * (wn * (NCT / 2) + ct)
                                : g.inter + n0 + 16 * (wn * (NCT / 2) + ct - NCT / 2);
        else
            row0 = n0 + 16 * (wn * NCT + ct);
        if (W4)
            boff[ct] = SHUFFLED ? (uint32_t)(row0 * KBY + lane * 16)
                                : (uint32_t)((row0 + lr) * KBY + lq * 16);
        else
            boff[ct] = SHUFFLED ? (uint32_t)(row0 * K + lq * 512 + lr * 16)
                                : (uint32_t)((row0 + lr) * K + lq * 32);
        bsoff[ct] = (uint32_t)((row0 + lr) * KS + lq);
    }
    constexpr int BSTEP = W4 ? (SHUFFLED ? 1024 : 64) : (SHUFFLED ? 2048 : 128);
    constexpr int BHI = SHUFFLED ? 256 : 16;

    using BS = BStep<W4, NCT>;
    auto load_b = [&](BS& s, int kb) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            s.b[ct][0] = __builtin_amdgcn_raw_buffer_load_b128(rb, boff[ct], kb * BSTEP, 0);
            if (!W4)
                s.b[ct][W4 ? 0 : 1] =
                    __builtin_amdgcn_raw_buffer_load_b128(rb, boff[ct] + BHI, kb * BSTEP, 0);
            s.bs[ct] = W4 ? (int)__builtin_amdgcn_raw_buffer_load_b8(rbs, bsoff[ct], kb * 4, 0)
                          : 0;
        }
    };
    // A of step k is staged in areg[k & 1]: loaded two steps ahead, stored
    // to LDS stage k & 1 one step ahead
    v4i areg[2][A_PT];
    auto load_a = [&](int buf, int kb) {
#pragma unroll
        for (int j = 0; j < A_PT; ++j)
            areg[buf][j] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[j], kb * 128, 0);
    };
    auto store_a = [&](int buf) {
#pragma unroll
        for (int j = 0; j < A_PT; ++j)
            *reinterpret_cast<v4i*>(&s_a[buf][a_dst[j]]) = areg[buf][j];
    };

    v4f acc[NRT][NCT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};
    const int row_base = wm * (BM / kWM);
    const int h0 = frag_swap(lr);

    // One K step: NRT x 4 MFMAs, row tile by row tile (the B fragments stay
    // in registers for the whole step, so only two A fragments are live);
    // the MFMAs of row tile r+1 are issued into the other of two result sets
    // while the FMAs fold tile r.
    auto compute = [&](const BS& bsv, int kb, int stage) {
        const uint8_t* sa_src = &s_a[stage][0];
        auto afrag = [&](int rt) {
            const uint8_t* slot = sa_src + lq * (BM * 32) + (row_base + rt * 16 + lr) * 32;
            const v4i lo = *reinterpret_cast<const v4i*>(slot + h0 * 16);
            const v4i hi = *reinterpret_cast<const v4i*>(slot + (h0 ^ 1) * 16);
            return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        auto bfrag = [&](int ct) {
            if (W4)
                return v8i{bsv.b[ct][0][0], bsv.b[ct][0][1], bsv.b[ct][0][2], bsv.b[ct][0][3],
                           0, 0, 0, 0};
            return v8i{bsv.b[ct][0][0], bsv.b[ct][0][1], bsv.b[ct][0][2], bsv.b[ct][0][3],
                       bsv.b[ct][W4 ? 0 : 1][0], bsv.b[ct][W4 ? 0 : 1][1],
                       bsv.b[ct][W4 ? 0 : 1][2], bsv.b[ct][W4 ? 0 : 1][3]};
        };
        auto mfma = [&](const v8i& a, int ct) {
            return W4 ? mfma16x16x128_fp8_fp4(a, bfrag(ct), bsv.bs[ct])
                      : mfma16x16x128_fp8(a, bfrag(ct));
        };
        // scale half of column tile ct: stage 1 gate (tiles 0,1) / up (2,3);
        // stage 2 the wave's 128-column block
        const int hblk = (wn * NCT * 16) / 128;           // stage 2: the wave's 128-column block
        const int hsel0 = W4 ? 0 : (STAGE == 1 ? 0 : hblk);
        const int hsel1 = W4 ? 0 : (STAGE == 1 ? 1 : hblk);
        const float* sc_row = &s_sc[kb * NH * BM + row_base + 4 * lq];
        v4f blk[2][NCT];
        {
            const v8i a0 = afrag(0);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) blk[0][ct] = mfma(a0, ct);
        }
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const int cur = rt & 1;
            if (rt + 1 < NRT) {
                const v8i an = afrag(rt + 1);
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) blk[cur ^ 1][ct] = mfma(an, ct);
            }
            const v4f s0 = *reinterpret_cast<const v4f*>(sc_row + hsel0 * BM + rt * 16);
            const v4f s1 = *reinterpret_cast<const v4f*>(sc_row + hsel1 * BM + rt * 16);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[rt][ct][v] += blk[cur][ct][v] * (ct < NCT / 2 ? s0[v] : s1[v]);
#pragma unroll
            for (int i = 0; i < NCT; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
            }
        }
    };

    // ---- K loop: B D steps ahead in registers; A two steps ahead in
    // registers and double-buffered in LDS; one barrier per step ----
    BS bbuf[D];
#pragma unroll
    for (int d = 0; d < D; ++d) load_b(bbuf[d], d);
    load_a(0, 0);
    store_a(0);
    load_a(1, KB > 1 ? 1 : 0);
    load_a(0, KB > 2 ? 2 : KB - 1);
    __syncthreads();                      // stage 0 and the scale products
    for (int kb0 = 0; kb0 < KB; kb0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int k = kb0 + d;
            // Everything in the step is unconditional so the loop is one basic
            // block and the compiler's wait counts stay exact: past the end the
            // loads re-read the last step (L2 hits) and the store fills the
            // stage that step k does not read.
            store_a((k + 1) & 1);
            load_a((k + 1) & 1, k + 3 < KB ? k + 3 : KB - 1);
            // issue the A loads before the step's math (a full step to land)
            __builtin_amdgcn_sched_barrier(0);
            compute(bbuf[d], k, k & 1);
            load_b(bbuf[d], k + D < KB ? k + D : KB - 1);
            __syncthreads();
            // keep the scheduler from interleaving the unrolled steps (their
            // operand sets would all be live at once)
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    if (STAGE == 2) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = row_base + rt * 16 + 4 * lq + v;
                const int64_t t = s_orow[row];
                if (t < 0) continue;
                const float wgt = s_w[row];
                float* dst = g.acc + t * g.N + n0 + wn * NCT * 16 + lr;
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct)
                    unsafeAtomicAdd(dst + ct * 16, acc[rt][ct][v] * wgt);
            }
        return;
    }

    // ---- stage 1 epilogue: silu(gate)*up -> bf16 -> 1x128 fp8 requant ----
    // wave wn holds output columns wn*NH1*16 + j*16 + lr (j < NH1) of the tile's 128
    constexpr int NH1 = NCT / 2;
    float h[NRT][NH1][4];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int j = 0; j < NH1; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                h[rt][j][v] = bf16_round(silu_f32(acc[rt][j][v]) * acc[rt][NH1 + j][v]);
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < NH1; ++j) m = __builtin_fmaxf(m, __builtin_fabsf(h[rt][j][v]));
            m = warp_max_16(m);
            if (lr == 0) s_amax[wn][row_base + rt * 16 + 4 * lq + v] = m;
        }
    __syncthreads();
    auto row_amax = [&](int row) {
        float m = s_amax[0][row];
#pragma unroll
        for (int w = 1; w < WN; ++w) m = __builtin_fmaxf(m, s_amax[w][row]);
        return __builtin_fmaxf(m, 1e-10f);
    };
    uint8_t* s_q = &s_a[0][0];  // [BM][128] fp8 staging (the K loop is done)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = row_base + rt * 16 + 4 * lq + v;
            const float inv = 1.0f / (row_amax(row) * kInvFp8Max);
#pragma unroll
            for (int j = 0; j < NH1; ++j) {
                const uint32_t b = f32x2_to_fp8x2(h[rt][j][v] * inv, 0.0f) & 0xFFu;
                s_q[row * 128 + wn * NH1 * 16 + j * 16 + lr] = (uint8_t)b;
            }
        }
    __syncthreads();
    const int I = g.inter;
    for (int q = tid; q < BM * 8; q += kThreads) {
        const int row = q >> 3, part = q & 7;
        const int64_t orow = s_orow[row];
        if (orow < 0) continue;
        *reinterpret_cast<v4i*>(g.a2 + orow * I + n0 + part * 16) =
            *reinterpret_cast<const v4i*>(s_q + row * 128 + part * 16);
        if (part == 0) g.a2_scale[orow * (I / 128) + n0 / 128] = row_amax(row) * kInvFp8Max;
    }
}

template <int BM, int STAGE, bool SHUFFLED, bool W4>
static void launch_depth(int KB, int grid, const Args& a, hipStream_t s) {
    constexpr int WM = STAGE == 1 ? 2 : 1;
    constexpr int DM = STAGE == 1 ? 2 : 4;      // the 1 x 8 tile has registers for 4 steps
    if (DM >= 4 && KB % 4 == 0)
        hipLaunchKernelGGL((moe_gemm_prefill_kernel<BM, STAGE, SHUFFLED, W4, DM >= 4 ? 4 : 2, WM>),
                           dim3(grid), dim3(kThreads), 0, s, a);
    else if (KB % 2 == 0)
        hipLaunchKernelGGL((moe_gemm_prefill_kernel<BM, STAGE, SHUFFLED, W4, 2, WM>), dim3(grid),
                           dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((moe_gemm_prefill_kernel<BM, STAGE, SHUFFLED, W4, 1, WM>), dim3(grid),
                           dim3(kThreads), 0, s, a);
}

template <int STAGE, bool SHUFFLED, bool W4>
static void launch_bm(int bm, int KB, int grid, const Args& a, hipStream_t s) {
    if (bm == 64)
        launch_depth<64, STAGE, SHUFFLED, W4>(KB, grid, a, s);
    else if (bm == 128)
        launch_depth<128, STAGE, SHUFFLED, W4>(KB, grid, a, s);
    else
        AMD_CHECK(false, "prefill GEMM block_m must be 64 or 128");
}

template <int STAGE>
static void launch(int bm, int KB, int grid, const Args& a, int shuffled, hipStream_t s) {
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

}  // namespace pf

bool prefill_supported(int64_t block_m, int64_t K) {
    return (block_m == 64 || block_m == 128) && K > 0 && K % 128 == 0 &&
           K / 128 <= pf::kMaxKB;
}

void launch_moe_stage1_prefill(const uint8_t* a, const float* a_scale, int64_t sa_row,
                               int64_t sa_kb, const uint8_t* w1, const float* w1_scale,
                               const uint8_t* w1_scale_e8m0, const int32_t* sorted_ids,
                               const int32_t* sorted_eids, const int32_t* num_valid,
                               uint8_t* a2, float* a2_scale, int64_t a_rows, int64_t K,
                               int64_t inter, int64_t E, int64_t topk, int64_t block_m,
                               int64_t max_m_blocks, int shuffled, hipStream_t stream) {
    pf::Args g{};
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
    g.n_tiles = (int)(inter / 128);
    g.m_blocks = (int)max_m_blocks;
    const int64_t grid = (int64_t)g.n_tiles * max_m_blocks;
    if (grid == 0) return;
    pf::launch<1>((int)block_m, (int)(K / 128), (int)grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

void launch_moe_stage2_prefill(const uint8_t* a2, const float* a2_scale, const uint8_t* w2,
                               const float* w2_scale, const uint8_t* w2_scale_e8m0,
                               const int32_t* sorted_ids, const float* sorted_w,
                               const int32_t* sorted_eids, const int32_t* num_valid, float* acc,
                               int64_t a_rows, int64_t inter, int64_t hidden, int64_t E,
                               int64_t topk, int64_t block_m, int64_t max_m_blocks, int shuffled,
                               hipStream_t stream) {
    pf::Args g{};
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
    g.K = (int)inter;
    g.N = (int)hidden;
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    g.n_tiles = (int)(hidden / 256);
    g.m_blocks = (int)max_m_blocks;
    const int64_t grid = (int64_t)g.n_tiles * max_m_blocks;
    if (grid == 0) return;
    pf::launch<2>((int)block_m, (int)(inter / 128), (int)grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
