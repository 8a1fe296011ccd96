// Prefill-shaped MoE gather-GEMMs for gfx950 (64/128-row M-blocks): weight
// fragments stream straight into registers, activations through LDS.
//
// Same contract as moe_gemm_fp8bs.hip (stage 1: gate+up GEMM, SiLU*up, bf16
// rounding, fused 1x128 fp8 requant; stage 2: down GEMM, routing weight,
// fp32 atomic accumulate; FP8 128x128 blockscale or MXFP4 weights).
//
// What bounds this shape on MI355X, measured: LDS reads run at ~128 B/clk
// per CU, so a tile that reads both operands from LDS spends as long reading
// LDS as the MFMAs take; and VALU issue barely overlaps MFMA -- 16x16x128
// fp8 MFMAs with the 4 fp32 FMAs per MFMA that the per-128-K block scales
// need reach ~65% of peak with two waves per SIMD.  So:
//   * B (weights) never touches LDS: every lane loads its own MFMA
//     fragments from global memory (the (16,16) layout puts them in 16-byte
//     pieces), D K-steps ahead in registers.
//   * A (token rows, gathered) is loaded to registers two steps ahead and
//     written to one of two LDS stages one step ahead, fragment-major with a
//     per-row swap of the 16-byte halves ((r>>2 ^ r>>3) & 1) so 16-byte
//     reads are conflict-free; one barrier per K step.
//   * The products a_scale[row, kb] * w_scale[block, kb] of the whole K
//     range are computed once per workgroup into LDS, so the K loop's VALU
//     work is the 4 FMAs per MFMA and little else; each wave folds row tile
//     r while the MFMAs of row tile r+1 run.
// Workgroup: 256 threads = 4 waves along N, two workgroups per CU (one wave
// of each per SIMD), so one workgroup's prologue and epilogue run under the
// other's K loop.  Stage 1: 64 rows (half a 128-row sorted block) x 256
// weight rows (128 gate + the matching 128 up rows = one 1x128 quant group
// per row); stage 2: 64 rows x 256 output columns (or, forced, block_m rows x
// 128 columns).  MXFP4 weights (A8W4) run the same tiles with half the weight
// bytes per K step and the tile's e8m0 scale bytes staged in LDS.  A tile
// whose rows are all padding exits at once, and padding rows of the others
// read zeros.  Tile order is XCD-aware: workgroup L
// runs on XCD L % 8; the XCDs form msplit groups along M (a contiguous range
// of the valid M-tiles each) x 8/msplit along N (each XCD owns that many
// column tiles of its range), so an expert's weight slice stays in one L2
// and each M-tile's A rows are gathered by 8/msplit XCDs.  A workgroup may walk
// ntw consecutive column tiles of its M-block in one pipelined K loop (setup
// paid once; the next tile's first loads are in flight during a tile's
// epilogue).
#include <cstdlib>

#include "common.h"

namespace aiter_amd {

namespace pf {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
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
    int act;                   // stage 1: activation of gate (kActSilu / kActGelu)
    const int32_t* sorted_eids;
    const int32_t* num_valid;
    uint8_t* a2;
    float* a2_scale;
    void* acc;                 // stage 2 out [T, N]: fp32, bf16 or fp16 (acc_dtype)
    int acc_dtype;
    uint16_t* part;            // stage 2: bf16 rows [pairs, N] instead of acc (or NULL)
    int K;
    int N;                     // weight rows per expert
    int inter;
    int topk;
    int E;
    int64_t a_rows;
    int n_tiles;
    int m_tiles;               // sorted M-blocks x workgroups per M-block
    int block_m;               // rows per sorted M-block (BM or 2 BM)
    int ntw;                   // column tiles per workgroup, walked in one pipelined K loop
    int msplit;                // XCD groups along M (1, 2, 4 or 8; see the tile order)
    int mrot;                  // stagger the M walk of the XCDs in a group
    int pad_skip;              // run tiles of few routed rows on a body without their padding MFMAs
    int e8_lds;                // A8W4: the tile's e8m0 bytes in LDS where they fit
};

// Slot of a row's 16-byte A piece in LDS: piece p of row r sits at slot
// p ^ a_swz(r). Any 16 consecutive rows then put one piece in 16 distinct
// (bank-half, slot) pairs, and any 8 in 8 distinct slots, so the fragment
// reads of a row tile and the row stores are conflict-free.
__device__ __forceinline__ int a_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Slot order of a row's eight 16-byte A pieces before the swizzle: identity
// for fp8 x fp8, whose lane q reads pieces 2q and 2q + 1; for fp8 x fp4,
// whose lane q reads pieces q and q + 4, piece p goes to slot 2p (p < 4) or
// 2(p - 4) + 1, so both read the same slots. Reading pieces q and q + 4 in
// place conflicted in LDS: measured on MI355X, A8W4 stage 1 at T=8192 had
// 9.2e7 bank-conflict cycles (FP8: 1.7e6); with this order 2.0e7, and stage
// 1 took 1194-1202 instead of 1213-1215 us.
template <bool W4>
__device__ __forceinline__ int a_slot(int p) {
    return W4 ? (p < 4 ? 2 * p : 2 * (p - 4) + 1) : p;
}

// Raw buffer resource over [base, base + bytes): loads take a 32-bit lane
// offset plus a wave-uniform K-step offset, and read 0 past the end.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// a_scale[row, kb] * w_scale[block h, kb] for row r, steps c = q, q + RP, ...
// (RP = threads per row) into s_sc[c][h][row]. Step c is K block c % KB of
// the workgroup's column tile c / KB, whose weight-scale blocks follow the
// first tile's TSM blocks (TSM * KB floats) on, TSM = the 128-column blocks
// of a stage-2 tile (1 in stage 1, whose gate and up blocks each advance by
// one), so w0 / w1 are indexed by (c - c % KB) * TSM + c % KB; NJ covers the
// KBT steps of all tiles. The loads (clamped addresses, no
// branches) and the products are separate calls so the caller can issue
// other loads in between.
template <int N>
struct IntC {
    static constexpr int value = N;
};

template <bool W4, int NJ>
struct ScaleRegs {
    float av[NJ];
    float b0[W4 ? 1 : NJ];
    float b1[W4 ? 1 : NJ];
};

template <int BM, int NH, bool W4, int NJ, int TSM = 1>
__device__ __forceinline__ void scale_load(ScaleRegs<W4, NJ>& sr, const float* sa, int64_t sa_kb,
                                           const float* w0, const float* w1, int KB, int KBT,
                                           int q) {
    constexpr int RP = kThreads / BM;
    // c % KB by a float reciprocal: c < 64 and KB <= 64, so the quotient of
    // (c + 1/2) / KB is at least 1/128 from an integer and rounds exactly
    const float rkb = 1.0f / (float)KB;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = q + j * RP;
        const int cc = c < KBT ? c : KBT - 1;
        const int kc = cc - KB * (int)(((float)cc + 0.5f) * rkb);
        sr.av[j] = sa[(int64_t)kc * sa_kb];
        if (!W4) {
            // column tile cc / KB's blocks are TSM blocks on from the previous tile's
            const int wi = (cc - kc) * TSM + kc;
            sr.b0[j] = w0[wi];
            if (NH == 2) sr.b1[j] = w1[wi];
        }
    }
}

template <int BM, int NH, bool W4, int NJ>
__device__ __forceinline__ void scale_store(const ScaleRegs<W4, NJ>& sr, float* s_sc, int KBT,
                                            int r, int q, bool valid) {
    constexpr int RP = kThreads / BM;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = q + j * RP;
        if (c < KBT) {
            const float v = valid ? sr.av[j] : 0.0f;
            s_sc[(c * NH) * BM + r] = W4 ? v : v * sr.b0[j];
            if (!W4 && NH == 2) s_sc[(c * NH + 1) * BM + r] = v * sr.b1[j];
        }
    }
}

// Waves along M (template kWM): 1 -> every wave owns all BM rows; 2 -> 2 x 2
// waves of BM/2 rows (the two M-waves load the same weight fragments).

// A8W4 with the tile's e8m0 bytes in LDS: the largest K/32 the LDS rows hold
// (two workgroups per CU still fit), and the row pitch, 16-byte aligned for
// the prologue's 16-byte stores. The per-step reads keep some bank conflicts
// at this pitch (2.0e7 cycles in stage 1 at T=8192, measured on MI355X); a
// 136-byte pitch removed them but ran 0.8% slower. In stage 2 the same pitch
// (with 8-byte stores) cut them 1.2e7 -> 2.3e6 and left its time unchanged.
template <int STAGE, int BM>
constexpr int e8_max_ks() { return STAGE == 2 && BM == 128 ? 64 : 128; }
template <int STAGE, int BM>
constexpr int e8_pitch() { return e8_max_ks<STAGE, BM>() + 16; }

// One K step of a wave's B operand (NCT 16-row weight groups).
template <bool W4, int NCT>
struct BStep {
    v4i b[NCT][W4 ? 1 : 2];
};

template <int BM, int STAGE, bool SHUFFLED, bool W4, int D, int kWM, int NW2 = 128,
          bool E8L = false>
__global__ __launch_bounds__(kThreads, 2) void moe_gemm_prefill_kernel(Args g) {
    constexpr int WN = kWaves / kWM;                     // waves along N
    // 16-row weight groups per wave: stage 1 256 weight rows (128 gate + the
    // matching 128 up rows) per workgroup, stage 2 NW2 (128 or 256)
    constexpr int NCT = STAGE == 1 ? 16 / WN : (NW2 / 16) / WN;
    constexpr int NW = 16 * NCT * WN;                    // weight rows per workgroup
    constexpr int NRT = BM / 16 / kWM;                   // 16-row MFMA tiles per wave
    // FP8 stage 1 computes the transposed tile (weights as the MFMA's A
    // operand): a lane then holds one token row and four consecutive output
    // columns, so its activation scale is one value per row tile and its
    // fp8 outputs pack into one dword
    constexpr bool TR = STAGE == 1;
    constexpr int A_BYTES = BM * 128;
    constexpr int A_PT = A_BYTES / 16 / kThreads;        // 16-byte A pieces per thread
    // scale products per (row, kb): stage 1 gate / up blocks; stage 2 the
    // workgroup's 128-column weight-scale blocks
    constexpr int NH = W4 ? 1 : (STAGE == 1 ? 2 : NW / 128);
    // weight rows one column tile advances: stage 1 128 gate (and 128 up)
    // rows, stage 2 the tile's NW output columns
    constexpr int TROWS = STAGE == 1 ? 128 : NW;
    constexpr int QP = 144;     // stage-1 fp8 staging row pitch: 16-byte aligned, conflict-free
    static_assert(BM == 64 || BM == 128, "prefill tiles are 64 or 128 rows");
    static_assert(A_PT >= 1, "one A piece per thread at least");
    __shared__ __attribute__((aligned(1024))) uint8_t s_a[2][A_BYTES];
    // [step][h][row]; the 256-column stage-2 tile also stages its bf16 output
    // rows here at a pitch of NW + 8 elements (SC_PW), rows that one write
    // instruction covers (4 apart) then start 16 banks apart
    constexpr int SC_PW = NW + 8;
    constexpr int SC_BASE = kMaxKB * NH * BM;
    constexpr int SC_RPP = (SC_BASE * 4 / (NW * 2)) >= BM ? BM : SC_BASE * 4 / (NW * 2);
    constexpr int SC_FLOATS = STAGE == 2 && NW2 > 128 && SC_RPP * SC_PW / 2 > SC_BASE
                                  ? SC_RPP * SC_PW / 2 : SC_BASE;
    __shared__ __attribute__((aligned(16))) float s_sc[SC_FLOATS];
    __shared__ __attribute__((aligned(16))) uint8_t s_q[STAGE == 1 ? BM * QP : 16];
    __shared__ int32_t s_arow[BM];
    __shared__ int64_t s_orow[BM];
    __shared__ float s_w[BM];
    __shared__ float s_amax[WN][BM];
    // A8W4 (E8L): the e8m0 bytes of the tile's NW weight rows over the whole K
    // range, loaded once per tile; row r at r * E8P
    constexpr int E8P = e8_pitch<STAGE, BM>();
    __shared__ __attribute__((aligned(16))) uint8_t s_e8[E8L ? NW * E8P : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int wm = wv / WN;
    const int wn = wv % WN;
    const int lr = lane & 15;
    const int lq = lane >> 4;

    // ---- XCD-aware tile order: the grid's columns are groups of ntw
    // column tiles ----
    const int L = blockIdx.x;
    const int ntw = g.ntw;
    const int ng = g.n_tiles / ntw;
    const int nvalid = g.num_valid[0];
    int nt, mt;
    if (!xcd_tile(L, ng, (g.m_tiles + g.msplit - 1) / g.msplit, (nvalid + BM - 1) / BM, g.msplit,
                  g.mrot, nt, mt))
        return;
    if (mt >= g.m_tiles) return;
    const int subs = g.block_m / BM;                     // workgroups per sorted M-block
    const int mb = mt / subs;
    const int srow0 = mb * g.block_m + (mt % subs) * BM; // first sorted row of the tile
    if (srow0 >= nvalid) return;
    const int tokens = g.num_valid[1];
    const int e = g.sorted_eids[mb];
    if (e < 0 || e >= g.E) return;
    const int n0 = nt * ntw * TROWS;                     // first column of the first tile

    int any_valid = 0;
    for (int r = tid; r < BM; r += kThreads) {
        const uint32_t id = (uint32_t)g.sorted_ids[srow0 + r];
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
        // routing weight of the pair (1 when none is passed: stage 2 without
        // weights, or stage 1 without doweight); stage 1 applies it only when given
        s_w[r] = valid ? (g.sorted_w ? g.sorted_w[srow0 + r] : 1.0f) : 0.0f;
        any_valid |= (int)valid;
    }
    // a tile whose rows are all padding (the end of an expert's last
    // M-block) has nothing to compute
    if (__syncthreads_or(any_valid) == 0) return;

    const int row_base = wm * (BM / kWM);
    // row tiles of this wave that hold a routed row (sorting pads each
    // expert's last block at its end): the MFMAs and FMAs of the others
    // are skipped, their accumulators stay 0 and their rows are not stored
    int nact = 0;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
        if (__builtin_amdgcn_ballot_w64(s_arow[row_base + rt * 16 + lr] >= 0) != 0) nact = rt + 1;
    nact = __builtin_amdgcn_readfirstlane(nact);

    // The rest of the tile, for waves with NA active row tiles. Each NA is a
    // whole copy from here on, so the copies share no live registers (a
    // second K-loop copy after a shared prologue spilled).
    auto body = [&](auto na) __attribute__((always_inline)) {
    const int K = g.K;
    const int KB = K / 128;
    const int KBY = W4 ? K / 2 : K;

    // ---- A staging: a K step of the tile's rows is [row][128 B] in LDS with
    // the 16-byte pieces of row r at slots p ^ a_swz(r). Piece q = tid + j*256
    // of the step is piece q % 8 of row q / 8, so each load instruction reads
    // 8 whole 128-byte rows (8 cache lines, every byte used) and each group
    // of 8 lanes stores one row's 8 distinct slots ----
    const __amdgpu_buffer_rsrc_t ra = rsrc(g.a, g.a_rows * K);
    uint32_t a_off[A_PT];
    int a_dst[A_PT];
#pragma unroll
    for (int j = 0; j < A_PT; ++j) {
        const int q = tid + j * kThreads;
        const int row = q >> 3, pc = q & 7;
        const int arow = s_arow[row];
        // pad rows read past the buffer's end, which returns zeros without a
        // memory access. Their results are unused, and zero operands switch
        // less in the MFMAs: measured on MI355X against re-reading row 0, the
        // T=8192 layer 2.644 -> 2.624 ms, T=2048 1.030 -> 1.015 ms, EP share
        // T=4096 0.307 -> 0.303 ms (the clock is power-bound under these GEMMs)
        a_off[j] = arow >= 0 ? (uint32_t)arow * (uint32_t)K + (uint32_t)(pc * 16) : 0xFFFFF000u;
        a_dst[j] = row * 128 + ((a_slot<W4>(pc) ^ a_swz(row)) << 4);
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
        bsoff[ct] = (uint32_t)((row0 + lr) * KS);
    }
    // E8L: the lane's e8m0 byte of step kb is byte lq of the dword at
    // s_e8[e8o[ct] + 4 kb] (the four lanes of a row read one address); the
    // tile's weight row r is stage 1's gate row n0 + r (r < 128) or up row
    // inter + n0 + r - 128, stage 2's row n0 + r
    int e8o[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
        const int lrow = STAGE == 1 ? (ct < NCT / 2 ? 16 * (wn * (NCT / 2) + ct)
                                                    : 128 + 16 * (wn * (NCT / 2) + ct - NCT / 2))
                                    : 16 * (wn * NCT + ct);
        e8o[ct] = (lrow + lr) * E8P;
    }
    constexpr int kE8Pieces = E8L ? NW * e8_max_ks<STAGE, BM>() / 16 / kThreads : 1;
    v4i e8r[kE8Pieces];
    const int e8_ppr = KS / 16;                          // 16-byte pieces per weight row
    auto e8_load = [&]() __attribute__((always_inline)) {
        if constexpr (E8L) {
#pragma unroll
            for (int j = 0; j < kE8Pieces; ++j) {
                const int q = tid + j * kThreads;
                const int r = q / e8_ppr, c = q - (q / e8_ppr) * e8_ppr;
                const int grow = STAGE == 1 ? (r < 128 ? n0 + r : g.inter + n0 + r - 128) : n0 + r;
                if (r < NW)
                    e8r[j] = __builtin_amdgcn_raw_buffer_load_b128(rbs, (uint32_t)(grow * KS + c * 16),
                                                                   0, 0);
            }
        }
    };
    auto e8_store = [&]() __attribute__((always_inline)) {
        if constexpr (E8L) {
#pragma unroll
            for (int j = 0; j < kE8Pieces; ++j) {
                const int q = tid + j * kThreads;
                const int r = q / e8_ppr, c = q - (q / e8_ppr) * e8_ppr;
                if (r < NW) *reinterpret_cast<v4i*>(&s_e8[r * E8P + c * 16]) = e8r[j];
            }
        }
    };
    constexpr int BSTEP = W4 ? (SHUFFLED ? 1024 : 64) : (SHUFFLED ? 2048 : 128);
    constexpr int BHI = SHUFFLED ? 256 : 16;

    using BS = BStep<W4, NCT>;
    // B of K block kb of column tile jt (wave-uniform offsets)
    auto load_b = [&](BS& s, int kb, int jt) __attribute__((always_inline)) {
        const int so = __builtin_amdgcn_readfirstlane(kb * BSTEP + jt * (TROWS * KBY));
        const int sso = __builtin_amdgcn_readfirstlane(kb * 4 + jt * (TROWS * KS));
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
            s.b[ct][0] = __builtin_amdgcn_raw_buffer_load_b128(rb, boff[ct], so, 0);
            if (!W4)
                s.b[ct][W4 ? 0 : 1] =
                    __builtin_amdgcn_raw_buffer_load_b128(rb, boff[ct] + BHI, so, 0);
        }
    };
    // A8W4: the e8m0 bytes of the D K steps kb .. kb + D - 1 of each of the
    // lane's weight rows in one load per D steps (4 D bytes per row, D
    // divides KB): dword d holds step kb + d's byte for lane group q in byte
    // q. A byte load per step and row group made the MXFP4 stage 1 wait on
    // its scale loads (each touches 16 rows' cache lines): measured on MI355X
    // at T=8192 with no scale loads at all, 1806 -> 1189 us.
    int sg_cur[NCT][D], sg_nxt[NCT][D];
    auto load_sg = [&](int (&dst)[NCT][D], int kb, int jt) __attribute__((always_inline)) {
        if constexpr (W4 && !E8L) {
            const int sso = __builtin_amdgcn_readfirstlane(kb * 4 + jt * (TROWS * KS));
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                if constexpr (D == 4) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b128(rbs, bsoff[ct], sso, 0);
#pragma unroll
                    for (int d = 0; d < 4; ++d) dst[ct][d] = (int)v[d];
                } else if constexpr (D == 2) {
                    const auto v = __builtin_amdgcn_raw_buffer_load_b64(rbs, bsoff[ct], sso, 0);
                    dst[ct][0] = (int)v[0];
                    dst[ct][1] = (int)v[1];
                } else {
                    dst[ct][0] = (int)__builtin_amdgcn_raw_buffer_load_b32(rbs, bsoff[ct], sso, 0);
                }
            }
        }
    };
    // A of step k is staged in areg[k & 1]: loaded two steps ahead, stored
    // to LDS stage k & 1 one step ahead
    v4i areg[2][A_PT];
    auto load_a = [&](int buf, int kb) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < A_PT; ++j)
            areg[buf][j] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_off[j], kb * 128, 0);
    };
    auto store_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < A_PT; ++j)
            *reinterpret_cast<v4i*>(&s_a[buf][a_dst[j]]) = areg[buf][j];
    };

    v4f acc[NRT][NCT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};
    // One K step: nact x NCT MFMAs, row tile by row tile (the B fragments
    // stay in registers for the whole step). Region r of the step issues the
    // MFMAs of row tile r+1 into one of two result sets, prefetches the next
    // A fragment and scale products from LDS, and folds row tile r's results
    // (issued one region earlier) into the accumulators. The regions are
    // fenced so the scheduler cannot pair an FMA with the MFMA that feeds it
    // (which serialises a wave on MFMA latency).
    auto compute = [&](const BS& bsv, int st, int stage, auto na, int d)
                       __attribute__((always_inline)) {
        constexpr int NA = decltype(na)::value;
        // A8W4: this step's e8m0 byte of the lane's weight row in byte 0
        int bsc[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
            bsc[ct] = !W4 ? 0
                      : E8L ? (int)(*reinterpret_cast<const uint32_t*>(&s_e8[e8o[ct] + 4 * st]) >>
                                    (8 * lq))
                            : sg_cur[ct][d] >> (8 * lq);
        const uint8_t* sa_src = &s_a[stage][0];
        // the lane's 32 K bytes of row tile rt: fp8 x fp8 pieces 2 lq, 2 lq + 1
        // (K 32 lq ..); fp8 x fp4 pieces lq, lq + 4 (K 16 lq .. and 64 + 16 lq ..)
        auto afrag = [&](int rt) {
            const int row = row_base + rt * 16 + lr;
            const uint8_t* rp = sa_src + row * 128;
            // (stored at slots a_slot(p) ^ a_swz: 2 lq and 2 lq + 1 either way)
            const int p0 = a_slot<W4>(W4 ? lq : 2 * lq), p1 = a_slot<W4>(W4 ? lq + 4 : 2 * lq + 1);
            const v4i lo = *reinterpret_cast<const v4i*>(rp + ((p0 ^ a_swz(row)) << 4));
            const v4i hi = *reinterpret_cast<const v4i*>(rp + ((p1 ^ a_swz(row)) << 4));
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
            if constexpr (TR)
                return W4 ? mfma16x16x128_fp4_fp8(bfrag(ct), a, bsc[ct])
                          : mfma16x16x128_fp8(bfrag(ct), a);
            return W4 ? mfma16x16x128_fp8_fp4(a, bfrag(ct), bsc[ct])
                      : mfma16x16x128_fp8(a, bfrag(ct));
        };
        // scale half of column tile ct: stage 1 gate (ct < NCT/2) / up;
        // stage 2 the wave's 128-column block
        const int hblk = (wn * NCT * 16) / 128;
        const int hsel0 = W4 ? 0 : (STAGE == 1 ? 0 : hblk);
        const int hsel1 = W4 ? 0 : (STAGE == 1 ? 1 : hblk);
        const float* sc_row = &s_sc[st * NH * BM + row_base + (TR ? lr : 4 * lq)];
        auto scales = [&](int rt, v4f& s0, v4f& s1) {
            if constexpr (TR) {
                const float x0 = sc_row[hsel0 * BM + rt * 16];
                const float x1 = sc_row[hsel1 * BM + rt * 16];
                s0 = v4f{x0, x0, x0, x0};
                s1 = v4f{x1, x1, x1, x1};
                return;
            }
            s0 = *reinterpret_cast<const v4f*>(sc_row + hsel0 * BM + rt * 16);
            s1 = *reinterpret_cast<const v4f*>(sc_row + hsel1 * BM + rt * 16);
        };
        auto fold = [&](const v4f (&b)[NCT], int rt, const v4f& s0, const v4f& s1) {
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    acc[rt][ct][v] += b[ct][v] * (ct < NCT / 2 ? s0[v] : s1[v]);
        };
        v4f blk[2][NCT];
        v8i an;
        v4f s0, s1;
        if (NA > 0) {
            an = afrag(0);
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) blk[0][ct] = mfma(an, ct);
            if (NRT > 1) an = afrag(1);
            scales(0, s0, s1);
        }
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const int cur = rt & 1;
            __builtin_amdgcn_sched_barrier(0);
            if (rt + 1 < NA) {
                v4f n0, n1;
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) blk[cur ^ 1][ct] = mfma(an, ct);
                if (rt + 2 < NRT) an = afrag(rt + 2);
                scales(rt + 1, n0, n1);
                fold(blk[cur], rt, s0, s1);
#pragma unroll
                for (int i = 0; i < NCT; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
                }
                s0 = n0;
                s1 = n1;
            } else if (rt < NA) {
                fold(blk[cur], rt, s0, s1);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // ---- K loop over the workgroup's ntw column tiles (KBT steps): B D
    // steps ahead in registers; A two steps ahead in registers and
    // double-buffered in LDS; one barrier per step. Step s is K block s % KB
    // of column tile s / KB; A depends on the K block only, so the loads of
    // the next tile's first steps are in flight while a tile's epilogue runs
    const int KBT = KB * ntw;
    BS bbuf[D];
    // ---- preheader: the loads of the K loop's virtual steps -3 .. -1 in the
    // loop's own order (step j loads A(j+3), then B(j+D)), so the wait
    // counts at the loop head are the steady-state ones; the scale loads go
    // first (oldest) and their products are stored once they land ----
    // scale products of all steps, [step][h][row]: fp8 h = 0 / 1 are
    // stage 1's gate / up blocks or stage 2's two 128-column blocks; A8W4 the
    // activation scale only (the weight scale goes into the MFMA)
    const int sr_r = tid % BM, sr_q = tid / BM;
    const int sr_arow = s_arow[sr_r];
    const float* sr_a = g.a_scale + (int64_t)(sr_arow < 0 ? 0 : sr_arow) * g.sa_row;
    const float* sr_w = W4 ? g.a_scale : g.w_scale + (int64_t)e * (g.N / 128) * KB;
    const float* sr_w0 = sr_w + (n0 / 128) * KB;
    // second block (NH == 2 only): stage 1's up rows, stage 2's next 128 columns
    const float* sr_w1 = sr_w + (STAGE == 1 ? (g.inter + n0) / 128 : n0 / 128 + NH - 1) * KB;
    auto last = [&](int m) { return m < KB ? m : KB - 1; };
    auto preheader = [&](auto nj) __attribute__((always_inline)) {
        constexpr int NJ = decltype(nj)::value;
        ScaleRegs<W4, NJ> sr;
        scale_load<BM, NH, W4, NJ, STAGE == 1 ? 1 : NW / 128>(sr, sr_a, g.sa_kb, sr_w0, sr_w1, KB,
                                                             KBT, sr_q);
        e8_load();
        // the e8m0 group of steps 0 .. D-1 follows the load of B step 0, as
        // the loop's group loads follow its step-0 B load
#pragma unroll
        for (int m = 0; m < D - 3; ++m) {
            load_b(bbuf[m], last(m), 0);
            if (m == 0) load_sg(sg_cur, 0, 0);
        }
        load_a(0, 0);                                           // step -3
        if constexpr (D >= 3) {
            load_b(bbuf[D - 3], last(D - 3), 0);
            if (D == 3) load_sg(sg_cur, 0, 0);
        }
        load_a(1, last(1));                                     // step -2
        if constexpr (D >= 2) {
            load_b(bbuf[D - 2], last(D - 2), 0);
            if (D == 2) load_sg(sg_cur, 0, 0);
        }
        scale_store<BM, NH, W4, NJ>(sr, s_sc, KBT, sr_r, sr_q, sr_arow >= 0);
        e8_store();
        store_a(0);                                             // step -1
        load_a(0, last(2));
        load_b(bbuf[D - 1], last(D - 1), 0);
        if (D == 1) load_sg(sg_cur, 0, 0);
    };
    constexpr int RP = kThreads / BM;
    if (KBT <= 16)
        preheader(IntC<16 / RP>{});
    else if (KBT <= 32)
        preheader(IntC<32 / RP>{});
    else
        preheader(IntC<kMaxKB / RP>{});
    __syncthreads();                      // stage 0 and the scale products

    // ---- epilogue of column tile jt; stage stg of s_a holds no live A ----
    auto epilogue = [&](int jt, int stg) __attribute__((always_inline)) {
        if constexpr (STAGE == 2) {
            const int nc = n0 + jt * TROWS;
            if (g.part) {
                // the pair's weighted row, rounded once to bf16, staged in LDS
                // RPP rows at a time and stored as whole 16-byte pieces at
                // part[pair, nc ..]: the 256-column tile (which walks one column
                // tile) through the scale products' buffer, whose last reader
                // was the final K step (an FP8 tile's 64 rows in one pass; four
                // through an A stage took T=8192 924-928 us against 917-921), the
                // 128-column tile through the free A stage
                auto stage_rows = [&](uint16_t* s_p, auto rpp, auto pw) __attribute__((always_inline)) {
                    constexpr int RPP = decltype(rpp)::value;
                    constexpr int PW = decltype(pw)::value;   // staged row pitch (elements)
                    static_assert(RPP % 16 == 0 && BM % RPP == 0,
                                  "a pass of bf16 rows is whole row tiles");
#pragma unroll
                    for (int hf = 0; hf < BM / RPP; ++hf) {
#pragma unroll
                        for (int rt = 0; rt < NRT; ++rt) {
                            if ((row_base + rt * 16) / RPP != hf) continue;
#pragma unroll
                            for (int v = 0; v < 4; ++v) {
                                const int row = row_base + rt * 16 + 4 * lq + v;
                                const float wgt = s_w[row];
                                const int lrow = row - hf * RPP;
#pragma unroll
                                for (int ct = 0; ct < NCT; ++ct)
                                    s_p[lrow * PW + wn * NCT * 16 + ct * 16 + lr] =
                                        f32_to_bf16_bits(acc[rt][ct][v] * wgt);
                            }
                        }
                        __syncthreads();
                        for (int q = tid; q < RPP * (NW / 8); q += kThreads) {
                            const int lrow = q / (NW / 8), piece = q % (NW / 8);
                            const int64_t pair = s_arow[lrow + hf * RPP];
                            if (pair < 0) continue;
                            *reinterpret_cast<v4i*>(g.part + pair * g.N + nc + piece * 8) =
                                *reinterpret_cast<const v4i*>(s_p + lrow * PW + piece * 8);
                        }
                        __syncthreads();
                    }
                };
                constexpr int A_ROWS = A_BYTES / (NW * 2);
                if constexpr (NW2 > 128)
                    stage_rows(reinterpret_cast<uint16_t*>(s_sc), IntC<SC_RPP>{}, IntC<SC_PW>{});
                else
                    stage_rows(reinterpret_cast<uint16_t*>(&s_a[stg][0]),
                               IntC<(A_ROWS >= BM ? BM : A_ROWS)>{}, IntC<NW>{});
            } else {
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int row = row_base + rt * 16 + 4 * lq + v;
                        const int64_t t = s_orow[row];
                        if (t < 0) continue;
                        const float wgt = s_w[row];
                        const int64_t dst = t * g.N + nc + wn * NCT * 16 + lr;
#pragma unroll
                        for (int ct = 0; ct < NCT; ++ct)
                            acc_add(g.acc, g.acc_dtype, dst + ct * 16, acc[rt][ct][v] * wgt);
                    }
            }
            return;
        } else {
        // ---- stage 1: silu(gate)*up -> bf16 -> 1x128 fp8 requant ----
        // wave wn holds output columns wn*NH1*16 + j*16 + (TR ? 4*lq + v : lr)
        // (j < NH1) of the tile's 128, for rows row_base + rt*16 + (TR ? lr :
        // 4*lq + v)
        constexpr int NH1 = NCT / 2;
        const int nc = n0 + jt * TROWS;
        float h[NRT][NH1][4];
        // act(gate) * up; the activation is chosen once per workgroup
        auto act_up = [&](auto act) {
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int j = 0; j < NH1; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        // doweight_stage1: the pair's weight scales gate and up before
                        // the activation (aiter/fused_moe.py:1568-1571)
                        const float wg =
                            g.sorted_w ? s_w[row_base + rt * 16 + (TR ? lr : 4 * lq + v)] : 1.0f;
                        h[rt][j][v] = bf16_round(act(acc[rt][j][v] * wg) *
                                                 (acc[rt][NH1 + j][v] * wg));
                    }
        };
        if (g.act == kActGelu)
            act_up([](float x) { return gelu_f32(x); });
        else
            act_up([](float x) { return silu_f32(x); });
        if constexpr (TR) {
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                float m = 0.0f;
#pragma unroll
                for (int j = 0; j < NH1; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        m = __builtin_fmaxf(m, __builtin_fabsf(h[rt][j][v]));
                m = __builtin_fmaxf(m, __shfl_xor(m, 16, 64));
                m = __builtin_fmaxf(m, __shfl_xor(m, 32, 64));
                if (lq == 0) s_amax[wn][row_base + rt * 16 + lr] = m;
            }
        } else {
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float m = 0.0f;
#pragma unroll
                    for (int j = 0; j < NH1; ++j)
                        m = __builtin_fmaxf(m, __builtin_fabsf(h[rt][j][v]));
                    m = warp_max_16(m);
                    if (lr == 0) s_amax[wn][row_base + rt * 16 + 4 * lq + v] = m;
                }
        }
        __syncthreads();
        auto row_amax = [&](int row) {
            float m = s_amax[0][row];
#pragma unroll
            for (int w = 1; w < WN; ++w) m = __builtin_fmaxf(m, s_amax[w][row]);
            return __builtin_fmaxf(m, 1e-10f);
        };
        if constexpr (TR) {
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                const int row = row_base + rt * 16 + lr;
                const float inv = 1.0f / (row_amax(row) * kInvFp8Max);
#pragma unroll
                for (int j = 0; j < NH1; ++j)
                    *reinterpret_cast<uint32_t*>(&s_q[row * QP + wn * NH1 * 16 + j * 16 + 4 * lq]) =
                        f32x4_to_fp8x4(h[rt][j][0] * inv, h[rt][j][1] * inv, h[rt][j][2] * inv,
                                       h[rt][j][3] * inv);
            }
        } else {
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = row_base + rt * 16 + 4 * lq + v;
                    const float inv = 1.0f / (row_amax(row) * kInvFp8Max);
#pragma unroll
                    for (int j = 0; j < NH1; ++j) {
                        const uint32_t b = f32x2_to_fp8x2(h[rt][j][v] * inv, 0.0f) & 0xFFu;
                        s_q[row * QP + wn * NH1 * 16 + j * 16 + lr] = (uint8_t)b;
                    }
                }
        }
        __syncthreads();
        const int I = g.inter;
        for (int q = tid; q < BM * 8; q += kThreads) {
            const int row = q >> 3, part = q & 7;
            const int64_t orow = s_orow[row];
            if (orow < 0) continue;
            *reinterpret_cast<v4i*>(g.a2 + orow * I + nc + part * 16) =
                *reinterpret_cast<const v4i*>(s_q + row * QP + part * 16);
            if (part == 0) g.a2_scale[orow * (I / 128) + nc / 128] = row_amax(row) * kInvFp8Max;
        }
        // s_q and s_amax are next written by the following tile's epilogue,
        // after that tile's K steps and their barriers
        }
    };

    auto kloop = [&](auto na) __attribute__((always_inline)) {
        int kbl = 0, jt = 0;             // K block and column tile of step kb0
        for (int kb0 = 0; kb0 < KBT; kb0 += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                const int k = kb0 + d;
                // Every load and store in the step is unconditional: past the
                // end A loads wrap to the first K blocks and B loads re-read the
                // last step (L2 hits), and the store fills the stage that step k
                // does not read.
                // A of step k + 3: K block kbl + d + 3 <= KB + 2, wrapped (KB >= 1)
                int ka = kbl + d + 3;
                ka = ka >= KB ? ka - KB : ka;
                ka = ka >= KB ? ka - KB : ka;
                ka = ka >= KB ? ka - KB : ka;
                store_a((k + 1) & 1);
                load_a((k + 1) & 1, ka);
                // issue the A loads before the step's math (a full step to land)
                __builtin_amdgcn_sched_barrier(0);
                // FP8 stage 1: the step's MFMAs and scale FMAs issue at raised
                // wave priority, ahead of the co-resident workgroup's setup and
                // epilogue. Measured on MI355X at T=8192, alternating builds on one
                // box: 1516-1529 -> 1510-1516 us; on another 1533-1553 -> 1537-1540 us.
                // MXFP4 stage 2 ran 1.5% slower with it, the other kernels alike.
                if constexpr (STAGE == 1 && !W4) __builtin_amdgcn_s_setprio(1);
                compute(bbuf[d], k, k & 1, na, d);
                if constexpr (STAGE == 1 && !W4) {
                    __builtin_amdgcn_s_setprio(0);
                    __builtin_amdgcn_sched_barrier(0);
                }
                // B of step k + D: this column tile or the next (D divides KB)
                int kn = kbl + d + D, jn = jt;
                if (kn >= KB) {
                    kn -= KB;
                    ++jn;
                }
                if (jn >= ntw) {
                    kn = KB - 1;
                    jn = ntw - 1;
                }
                load_b(bbuf[d], kn, jn);
                // the next D steps' e8m0 group (past the end: the last group)
                if (d == 0) load_sg(sg_nxt, kn - (kn % D), jn);
                __syncthreads();
                // keep the scheduler from interleaving the unrolled steps (their
                // operand sets would all be live at once)
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (W4 && !E8L) {
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
                    for (int d = 0; d < D; ++d) sg_cur[ct][d] = sg_nxt[ct][d];
            }
            kbl += D;
            if (kbl == KB) {
                // the tile's last step read A stage (kb0 + D - 1) & 1, which the
                // next step refills only after the epilogue's last barrier
                epilogue(jt, (kb0 + D - 1) & 1);
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                    for (int ct = 0; ct < NCT; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};
                kbl = 0;
                ++jt;
            }
        }
    };
    kloop(na);
    };
    // A wave whose rows are all padding runs the body without math (it still
    // stages A and meets every barrier, as every copy does). With pad_skip, a
    // stage-2 (or MXFP4 stage-1) tile of at most NRT/4 (and, in 128-row tiles,
    // NRT/2) active row tiles runs a copy that skips the MFMAs of the rest. Each copy adds ~20 KB
    // of code (the instruction cache is shared by two CUs), so 64-row tiles
    // get one. Not in the FP8 128-row tile (FP8 takes the 64-row wide tile),
    // where the copies spill. Measured on MI355X at MiMo dims, same boxes,
    // stage 2: T=8192 926-938 -> 920-928 us, T=2048 331-333 -> 329-331 us,
    // A8W4 T=8192 (128-row tiles) 960-971 -> 931-934 us. Stage 1 (a copy
    // at NRT/4) was no faster: T=8192 1540-1559 -> 1530-1538 us but T=2048
    // 574-577 -> 580-584 us and the EP share 160-162 -> 162-165 us; its small
    // tiles are bound by their weight stream, not by their MFMAs. MXFP4 stage 1
    // (half the weight bytes) gains: T=8192 1264-1271 -> 1237-1238 us, T=2048
    // and 1024 level.
    constexpr bool kPadCopies = (STAGE == 2 || W4) && NRT >= 4 && !(BM == 128 && !W4);
    if (kWM > 1 && nact == 0)
        body(IntC<0>{});
    else if (kPadCopies && g.pad_skip && nact <= NRT / 4)
        body(IntC<kPadCopies ? NRT / 4 : NRT>{});
    else if (kPadCopies && NRT >= 8 && g.pad_skip && nact <= NRT / 2)
        body(IntC<kPadCopies && NRT >= 8 ? NRT / 2 : NRT>{});
    else
        body(IntC<NRT>{});
}

template <int BM, int STAGE, bool SHUFFLED, bool W4, int NW2, bool E8L>
static void launch_e8(int KB, int grid, const Args& a, hipStream_t s) {
    // 1 x 4 waves: stage 1 64 rows x 64 weight rows per wave, B two steps
    // ahead; stage 2 BM rows x NW2/4 columns, B four steps ahead at 32
    // columns (measured on MI355X against 2 x 2 waves for stage 2: 1230 vs
    // 1282 us at T=8192), two at 64
    constexpr int WM = 1;
    constexpr int DM = STAGE == 1 || NW2 > 128 ? 2 : 4;
    if (DM >= 4 && KB % 4 == 0)
        hipLaunchKernelGGL((moe_gemm_prefill_kernel<BM, STAGE, SHUFFLED, W4, DM >= 4 ? 4 : 2, WM,
                                                    NW2, E8L>),
                           dim3(grid), dim3(kThreads), 0, s, a);
    else if (KB % 2 == 0)
        hipLaunchKernelGGL((moe_gemm_prefill_kernel<BM, STAGE, SHUFFLED, W4, 2, WM, NW2, E8L>),
                           dim3(grid), dim3(kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((moe_gemm_prefill_kernel<BM, STAGE, SHUFFLED, W4, 1, WM, NW2, E8L>),
                           dim3(grid), dim3(kThreads), 0, s, a);
}

// A8W4: the tile's e8m0 bytes go into LDS once per tile when they fit (K/32
// a multiple of 16 up to e8_max_ks) and the workgroup walks one column tile;
// otherwise each wave loads them a group of D K steps at a time (each such
// load still touches 16 weight rows' cache lines). Measured on MI355X at MiMo
// dims, stage 1: T=8192 1491-1497 -> 1277-1281 us, T=4096 876 -> 747 us,
// T=2048 586 -> 499 us, T=1024 495 -> 452 us. AITER_AMD_PF_E8LDS = 0 forces
// the grouped loads.
template <int BM, int STAGE, bool SHUFFLED, bool W4, int NW2 = 128>
static void launch_depth(int KB, int grid, const Args& a, hipStream_t s) {
    if constexpr (W4) {
        const int ks = KB * 4;
        if (a.ntw == 1 && ks % 16 == 0 && ks <= e8_max_ks<STAGE, BM>() && a.e8_lds) {
            launch_e8<BM, STAGE, SHUFFLED, W4, NW2, true>(KB, grid, a, s);
            return;
        }
    }
    launch_e8<BM, STAGE, SHUFFLED, W4, NW2, false>(KB, grid, a, s);
}

// Rows per workgroup: stage 1 always 64 (a 128-row sorted block is two
// workgroups); stage 2 the sorted block size.
template <int STAGE>
constexpr int wg_rows(int block_m) { return STAGE == 1 ? 64 : block_m; }

template <int STAGE, bool SHUFFLED, bool W4>
static void launch_bm(int bm, int KB, int grid, const Args& a, hipStream_t s, bool wide) {
    AMD_CHECK(bm == 64 || bm == 128, "prefill GEMM block_m must be 64 or 128");
    if constexpr (STAGE == 1)
        launch_depth<64, STAGE, SHUFFLED, W4>(KB, grid, a, s);
    else if (wide)
        launch_depth<64, STAGE, SHUFFLED, W4, 256>(KB, grid, a, s);
    else if (bm == 64)
        launch_depth<64, STAGE, SHUFFLED, W4>(KB, grid, a, s);
    else
        launch_depth<128, STAGE, SHUFFLED, W4>(KB, grid, a, s);
}

template <int STAGE>
static void launch(int bm, int KB, int grid, const Args& a, int shuffled, hipStream_t s,
                   bool wide = false) {
    const bool w4 = a.w_scale8 != nullptr;
    if (w4) {
        if (shuffled)
            launch_bm<STAGE, true, true>(bm, KB, grid, a, s, wide);
        else
            launch_bm<STAGE, false, true>(bm, KB, grid, a, s, wide);
    } else {
        if (shuffled)
            launch_bm<STAGE, true, false>(bm, KB, grid, a, s, wide);
        else
            launch_bm<STAGE, false, false>(bm, KB, grid, a, s, wide);
    }
}

// Stage 2 as 64-row x 256-column workgroups (two per 128-row sorted block;
// each wave 64 rows x 64 columns, as stage 1) instead of block_m x 128: half
// the LDS reads per MFMA, and a 128-row block's empty second half exits at
// once. Measured on MI355X at MiMo dims, FP8: T=2048 (64-row blocks) 363-367
// -> 338 us, EP share T=4096 97-99 -> 90-91 us, T=8192 950 -> 943 us, T=4096
// neutral (571 us); MXFP4 (with the e8m0 bytes loaded a group of K steps at
// a time): T=8192 (128-row blocks) 820 -> 767 us. AITER_AMD_PF_WIDE2 = 0 / 1
// forces it.
static bool pick_wide2(int64_t hidden) {
    if (hidden % 256 != 0) return false;
    if (const char* env = getenv("AITER_AMD_PF_WIDE2")) return atoi(env) != 0;
    return true;
}

// Column tiles per workgroup. Walking two amortises a tile's setup chain
// (sorted ids, then A rows and scales) and lets the next tile's first loads
// land while the epilogue runs, but the tiles that share an M-block's A rows
// then run one after another instead of side by side on one XCD, so A is
// fetched into L2 once per tile. Measured on MI355X at T=8192 (MiMo dims):
// stage 1 1735 -> 1783 us at two tiles; stage 2 1237 -> 1192 us at two,
// 1223 us at four; T=2048 (64-row blocks) 441 -> 421 us at two; a grid of a
// few rounds loses more to the longer tail (EP share T=4096, 32 of 256
// experts: 116 -> 120 us). So stage 2 walks two tiles when the pairs
// expected on this GPU fill at least kMinRounds rounds of workgroups after
// halving, stage 1 none. AITER_AMD_PF_NTW1 / AITER_AMD_PF_NTW2 force a count
// (tests use them; any divisor of n_tiles with ntw * KB <= kMaxKB).
// XCD groups along M. Both stages split the 8 XCDs into 2 groups along M x
// 4 along N, and stage 1 also staggers the walk of the 4 XCDs of a group
// (each starts a quarter of the group's M-tiles further on), so the XCDs
// gather different A rows and stream different experts' weights at any one
// time. Measured on MI355X at MiMo dims against one group (every XCD walks
// every M-tile in the same order): stage 1 T=8192 1720 -> 1603 us, T=2048
// 597 -> 581 us, EP share T=4096 (32 of 256 experts) 174 -> 160 us; stage 2
// 935 -> 939, 365 -> 362, 102 -> 98 us (staggering stage 2 made T=8192
// 969 us). Four groups: stage 1 1664 / 612 / 164 us. HBM fetch rises with
// the groups (stage 1 T=8192 6.5 -> 6.8 GB at two): an expert's weight slice
// on one XCD is then 4 column tiles (4 MB, the size of its L2), not 2.
// AITER_AMD_PF_MSPLIT1 / _2 force 1, 2, 4 or 8 groups and
// AITER_AMD_PF_MROT1 / _2 the stagger (tests use them).
static int pick_msplit(int stage, int ng) {
    if (ng % 8 != 0) return 1;
    if (const char* env = getenv(stage == 1 ? "AITER_AMD_PF_MSPLIT1" : "AITER_AMD_PF_MSPLIT2")) {
        const int c = atoi(env);
        if (c == 1 || c == 2 || c == 4 || c == 8) return c;
    }
    return 2;
}

// Stage-2 tiles with few routed rows (the end of an expert's last block, and
// the many experts of a skewed routing that get a handful of rows) run a copy
// of the tile's body that skips the MFMAs and FMAs of their padding row
// tiles. AITER_AMD_PF_PADSKIP = 0 runs every tile on the full body (tests
// use it).
static int pick_pad_skip() {
    if (const char* env = getenv("AITER_AMD_PF_PADSKIP")) return atoi(env) != 0;
    return 1;
}

static int pick_e8_lds() {
    if (const char* env = getenv("AITER_AMD_PF_E8LDS")) return atoi(env) != 0;
    return 1;
}

static int pick_mrot(int stage) {
    if (const char* env = getenv(stage == 1 ? "AITER_AMD_PF_MROT1" : "AITER_AMD_PF_MROT2"))
        return atoi(env) != 0;
    return stage == 1;
}

static int pick_ntw(int stage, int n_tiles, int KB, int64_t pairs, int rows, bool wide = false) {
    // the 256-column stage-2 tiles walk one (their epilogue stages the output
    // rows in the scale products' buffer, which a next tile would still need):
    // at two, T=8192 935-942 vs 939-944 us, T=4096 569 vs 537-540 us, T=2048
    // 342 vs 336 us, EP share 99.7 vs 89.5-91.7 us (four: 1030 / 662 / 358 /
    // 148 us)
    if (stage == 2 && wide) return 1;
    if (const char* env = getenv(stage == 1 ? "AITER_AMD_PF_NTW1" : "AITER_AMD_PF_NTW2")) {
        const int c = atoi(env);
        if (c >= 1 && n_tiles % c == 0 && c * KB <= kMaxKB) return c;
    }
    constexpr int64_t kSlots = 512;   // 256 CUs x 2 workgroups
    constexpr int64_t kMinRounds = 8;
    const int64_t wgs = (pairs + rows - 1) / rows * n_tiles;
    if (stage == 2 && n_tiles % 2 == 0 && (n_tiles / 2) % 8 == 0 && 2 * KB <= kMaxKB &&
        wgs / 2 >= kMinRounds * kSlots)
        return 2;
    return 1;
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
                               int64_t max_m_blocks, int shuffled, hipStream_t stream, const float* sorted_w, int act) {
    pf::Args g{};
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
    g.n_tiles = (int)(inter / 128);
    g.block_m = (int)block_m;
    g.m_tiles = (int)(max_m_blocks * (block_m / pf::wg_rows<1>((int)block_m)));
    g.ntw = pf::pick_ntw(1, g.n_tiles, (int)(K / 128), a_rows * topk, 64);
    g.msplit = pf::pick_msplit(1, g.n_tiles / g.ntw);
    g.mrot = pf::pick_mrot(1);
    g.e8_lds = pf::pick_e8_lds();
    g.pad_skip = pf::pick_pad_skip();
    const int64_t grid = xcd_grid(g.n_tiles / g.ntw, g.m_tiles, g.msplit);
    if (grid == 0) return;
    pf::launch<1>((int)block_m, (int)(K / 128), (int)grid, g, shuffled, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

void launch_moe_stage2_prefill(const uint8_t* a2, const float* a2_scale, const uint8_t* w2,
                               const float* w2_scale, const uint8_t* w2_scale_e8m0,
                               const int32_t* sorted_ids, const float* sorted_w,
                               const int32_t* sorted_eids, const int32_t* num_valid, void* acc, int acc_dtype,
                               uint16_t* part, int64_t a_rows, int64_t inter, int64_t hidden,
                               int64_t E, int64_t topk, int64_t block_m, int64_t max_m_blocks,
                               int shuffled, hipStream_t stream, int64_t est_pairs) {
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
    g.acc_dtype = acc_dtype;
    g.part = part;
    g.K = (int)inter;
    g.N = (int)hidden;
    g.inter = (int)inter;
    g.topk = (int)topk;
    g.E = (int)E;
    g.a_rows = a_rows;
    const bool wide = pf::pick_wide2(hidden);
    const int rows = wide ? 64 : (int)block_m;
    g.n_tiles = (int)(hidden / (wide ? 256 : 128));
    g.block_m = (int)block_m;
    g.m_tiles = (int)(max_m_blocks * (block_m / rows));
    g.ntw = pf::pick_ntw(2, g.n_tiles, (int)(inter / 128), est_pairs, rows, wide);
    g.msplit = pf::pick_msplit(2, g.n_tiles / g.ntw);
    g.mrot = pf::pick_mrot(2);
    g.e8_lds = pf::pick_e8_lds();
    g.pad_skip = pf::pick_pad_skip();
    const int64_t grid = xcd_grid(g.n_tiles / g.ntw, g.m_tiles, g.msplit);
    if (grid == 0) return;
    pf::launch<2>((int)block_m, (int)(inter / 128), (int)grid, g, shuffled, stream, wide);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
