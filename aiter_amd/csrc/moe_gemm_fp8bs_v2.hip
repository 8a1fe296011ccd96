// Prefill-shaped FP8 block-scale MoE GEMMs for gfx950: large tiles,
// direct-to-LDS loads, a 3-stage K pipeline, XCD-aware tile order.
//
// Same contract as moe_gemm_fp8bs.hip (stage 1: gate+up GEMM, SiLU*up,
// bf16 rounding and 1x128 fp8 requant; stage 2: down GEMM, routing weight,
// f32 atomic accumulate), for M-blocks of 64 or 128 sorted rows. The library
// runs it for MXFP4 layers whose experts average few routed rows (its waves
// skip padding-only halves); the prefill kernels take FP8 and larger MXFP4
// layers.
//
// Workgroup: 512 threads = 2 (M) x 4 (N) wave64s, two waves per SIMD so the
// block-scale FMAs of one wave run beside the other wave's MFMAs; tile BM
// rows x 256 weight rows (stage 1: 128 gate + the matching 128 up rows =
// 128 outputs; stage 2: 256 outputs); each wave owns (BM/2) x 64 weight
// columns, i.e. 4 16-wide MFMA column tiles (stage 1: 2 gate + the 2
// matching up tiles), so a 128-K step costs the wave BM/32 * 4
// v_mfma_f32_16x16x128_f8f6f4 against (BM/2 + 64) * 128 bytes of LDS reads.
//
// K pipeline: every operand of a K step -- the A rows (gathered by token),
// the B tile and the A scales -- is fetched with buffer_load ... lds
// straight into one of NS LDS stage buffers, NS-1 steps ahead of the step
// being computed.  Each step begins with s_waitcnt vmcnt(<loads of the
// steps still in flight>) and a barrier, issues the loads of step k+NS-1
// into the buffer step k-1 used, then computes step k.
// LDS layouts are fragment-major: an MFMA operand fragment (one row or
// column, 32 consecutive K bytes of quarter kq) sits in one 32-byte slot
// and the 16 lanes of a quarter read one 512-byte span, as two 16-byte
// reads.  Within each slot the two 16-byte halves are swapped for rows
// with h0(r) = ((r >> 2) ^ (r >> 3)) & 1, so each 16-byte read of 8 or 16
// consecutive lanes covers distinct banks.
//   A tile: [row BM][128 B], the 16-byte pieces of row r XOR-swizzled by
//   a_swz(r), so each A DMA reads 8 whole rows;  B tile: 16 groups of 16 weight rows,
//   each [kq 4][row 16][32 B] (the (16,16) shuffled 2 KB block with the two
//   16-byte halves of a row brought together).  The DMA lane -> global
//   address map does the reordering.
// Tile order (xcd_tile): the grid is 1-D; workgroup L runs on XCD L % 8;
// the XCDs form two groups along M (half the valid M-blocks each) x 4
// along N, so the weight slice of an expert stays in one XCD's L2 across
// the expert's consecutive M-blocks and each block's A rows are gathered by
// 4 XCDs, not 8.
//
// A8W4 (W4 = true): MXFP4 weights (packed e2m1 [E, N, K/2], e8m0 scales
// [E, N, K/32]).  A 16-row group's K step is 1 KB, kept lane-linear in LDS
// (lane l's B fragment = MX block l/16 of row l%16 at l*16, conflict-free);
// the e8m0 dwords of the tile's 256 weight rows (4 MX blocks per K step)
// ride in the scale DMA next to the activation scales, and each lane's byte
// goes into the scaled MFMA.  The A slots then hold K bytes 16q..16q+15 and
// 64+16q..64+16q+15 (the fp8 x fp4 K pairing, see mfma16x16x128_fp8_fp4).
#include "common.h"

namespace aiter_amd {

namespace v2 {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kBK = 128;
constexpr int kBRows = 256;                  // weight rows per tile
constexpr int kStages = 3;

typedef __attribute__((address_space(3))) void* lds_void_t;

struct Args {
    const uint8_t* a;
    const float* a_scale;
    int64_t sa_row;      // a_scale element strides (row, K block)
    int64_t sa_kb;
    int64_t sa_bytes;    // extent of a_scale in bytes
    const uint8_t* w;
    const float* w_scale;        // [E, N/128, K/128] (fp8 weights)
    const uint8_t* w_scale8;     // [E, N, K/32] e8m0 (MXFP4 weights)
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
    int N;           // weight rows per expert
    int inter;
    int topk;
    int E;
    int64_t a_rows;
    int n_tiles;     // column tiles
    int m_blocks;    // M-tiles of BM rows
    int block_m;     // rows per sorted block (BM or 2 BM): the expert of tile m is
                     // sorted_eids[m * BM / block_m]
    int msplit;      // XCD groups along M (xcd_tile)
    int mrot;        // stagger the M walk of the XCDs in a group
};

// Buffer resource (base, byte size) for the LDS-DMA loads: word1 carries
// the high address bits with stride 0; word3 is the raw-buffer config of
// gfx9-class parts.
struct Rsrc {
    v4i w;
};

__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    Rsrc r;
    r.w = v4i{(int)(uint32_t)p, (int)(uint32_t)((p >> 32) & 0xFFFFu), (int)bytes, 0x00020000};
    return r;
}

// Which 16-byte half of row r's 32-byte fragment slot holds K bytes 0-15
// (the B tile).
__device__ __forceinline__ int frag_swap(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

// The A tile of a K step is [row][128 B] with piece p of row r at slot
// p ^ a_swz(r): 16 consecutive rows put one piece in 16 distinct
// (bank-half, slot) pairs, so fragment reads are conflict-free.
__device__ __forceinline__ int a_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)reinterpret_cast<uintptr_t>((lds_void_t)(void*)p);
}

// buffer_load_dword{x4} ... lds: each lane's 4 or 16 bytes at r + voff +
// soff go to LDS at lds + lane * {4,16}.  Issued from inline asm, so the
// compiler's wait-count pass does not see them (it would drain the whole
// prefetch before every LDS read); the kernel waits for them itself with
// an explicit s_waitcnt vmcnt(N) and issues no other vector loads in the
// pipeline.  m0 holds the LDS base, and both statements declare it
// clobbered, so the compiler keeps nothing of its own there across them.
__device__ __forceinline__ void dma16(const Rsrc& r, uint32_t voff, uint32_t soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(r.w), "s"(soff), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ void dma4(const Rsrc& r, uint32_t voff, uint32_t soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dword %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(r.w), "s"(soff), "s"(lds)
                 : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

template <int BM, bool W4>
struct Tile {
    static constexpr int NRT = BM / 32;                 // 16-row MFMA tiles per wave
    static constexpr int A_BYTES = BM * kBK;
    static constexpr int GB = W4 ? 1024 : 2048;         // bytes per 16-row group per K step
    static constexpr int B_BYTES = 16 * GB;             // 256 weight rows
    static constexpr int A_INSTR = BM * kBK / 1024 / kWaves;  // 1 KB DMA instructions per wave
    static constexpr int B_INSTR = B_BYTES / 1024 / kWaves;   // 4 (fp8) or 2 (fp4) per wave
    static constexpr int LOADS = A_INSTR + B_INSTR + 1; // DMA instructions per wave per step
    static constexpr int SA_WAVES = BM / 64;            // waves whose scale DMA carries a_scale
    static_assert(BM == 64 || BM == 128, "v2 tiles are 64 or 128 rows");
    static_assert(A_INSTR >= 1, "every wave issues at least one A chunk");
    static_assert(!W4 || SA_WAVES + 4 <= kWaves, "room for the 256 e8m0 rows");
};

template <int BM, int STAGE, bool SHUFFLED, bool W4>
__global__ __launch_bounds__(kThreads, 1) void moe_gemm_fp8bs_v2_kernel(Args g) {
    using T = Tile<BM, W4>;
    constexpr int NRT = T::NRT;
    constexpr int A_INSTR = T::A_INSTR;
    constexpr int B_INSTR = T::B_INSTR;
    constexpr int GB = T::GB;
    __shared__ __attribute__((aligned(1024))) uint8_t s_a[kStages][T::A_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t s_b[kStages][T::B_BYTES];
    // per stage: a_scale of row r at [r]; A8W4: e8m0 dword (4 MX blocks) of tile
    // weight row j at [BM + j]
    __shared__ __attribute__((aligned(16))) float s_sa[kStages][kThreads];
    __shared__ int32_t s_arow[BM];
    __shared__ int64_t s_orow[BM];
    __shared__ float s_w[BM];
    __shared__ float s_amax[4][BM];
    __shared__ float s_sw[2][64];    // weight scales of the tile's two 128-row blocks per K block

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = tid >> 6;
    const int wvu = __builtin_amdgcn_readfirstlane(wv);   // wave-uniform copy (scalar)
    const int wm = wv >> 2;     // 0..1: row half
    const int wn = wv & 3;      // 0..3: 64-column quarter of the weight tile
    const int lr = lane & 15;
    const int lq = lane >> 4;

    // ---- XCD-aware tile order ----
    const int L = blockIdx.x;
    const int nvalid = g.num_valid[0];
    int nt, mb;
    if (!xcd_tile(L, g.n_tiles, (g.m_blocks + g.msplit - 1) / g.msplit, (nvalid + BM - 1) / BM,
                  g.msplit, g.mrot, nt, mb))
        return;
    if (mb >= g.m_blocks) return;
    if (mb * BM >= nvalid) return;
    const int tokens = g.num_valid[1];
    const int e = g.sorted_eids[(mb * BM) / g.block_m];
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
        // routing weight of the pair (1 when none is passed: stage 2 without
        // weights, or stage 1 without doweight); stage 1 applies it only when given
        s_w[r] = valid ? (g.sorted_w ? g.sorted_w[mb * BM + r] : 1.0f) : 0.0f;
    }

    const int K = g.K;
    const int KB = K / kBK;
    const int KBY = W4 ? K / 2 : K;                      // weight bytes per row
    const uint8_t* we = g.w + (int64_t)e * g.N * KBY;

    // weight-scale block rows of the tile: stage 1 gate / up, stage 2 the two
    // 128-column halves
    if (!W4) {
        const float* wse = g.w_scale + (int64_t)e * (g.N / 128) * KB;
        const int nb0 = n0 / 128;
        const int nb1 = STAGE == 1 ? (g.inter + n0) / 128 : n0 / 128 + 1;
        for (int i = tid; i < 2 * KB; i += kThreads)
            s_sw[i / KB][i % KB] = wse[(i < KB ? nb0 : nb1) * KB + (i % KB)];
    }
    const int swsel0 = STAGE == 1 ? 0 : (wn >> 1);
    const int swsel1 = STAGE == 1 ? 1 : (wn >> 1);
    __syncthreads();
    // a tile with only padding rows (the empty half of a 128-row block) has
    // nothing to compute; sorting pads each expert's segment at its end, so
    // such a tile is one whose first row is padding
    if (s_orow[0] < 0) return;

    // ---- per-lane DMA sources (byte offsets; the K step goes in soffset) ----
    uint32_t a_off[A_INSTR];
#pragma unroll
    for (int i = 0; i < A_INSTR; ++i) {   // 1 KB chunk c: whole rows 8c .. 8c+7
        // lane l fills LDS slot l % 8 of row 8c + l / 8, i.e. fetches the piece
        // (l % 8) ^ a_swz(row): each DMA reads 8 whole 128-byte rows
        const int c = wvu * A_INSTR + i;
        const int row = c * 8 + (lane >> 3);
        const int pc = (lane & 7) ^ a_swz(row);
        const int arow = s_arow[row];
        // pad rows read past the buffer's end (zeros, no memory access;
        // results unused, and zero operands switch less in the MFMAs)
        a_off[i] = arow >= 0 ? (uint32_t)arow * (uint32_t)K + (uint32_t)(pc * 16) : 0xFFFFF000u;
    }
    uint32_t b_off[B_INSTR];
#pragma unroll
    for (int i = 0; i < B_INSTR; ++i) {   // 1 KB chunk: half of a 16-row group, slot kq*32+rr*2+h
        const int chunk = wvu * B_INSTR + i;   // 32 (fp8) or 16 (fp4) chunks of 1 KB
        if (W4) {                              // chunk = group; lane-linear MX blocks
            const int grp = chunk;
            const int row0 = STAGE == 1 ? (grp < 8 ? n0 + 16 * grp : g.inter + n0 + 16 * (grp - 8))
                                        : n0 + 16 * grp;
            b_off[i] = SHUFFLED ? (uint32_t)row0 * (uint32_t)KBY + (uint32_t)(lane * 16)
                                : (uint32_t)(row0 + (lane & 15)) * (uint32_t)KBY +
                                      (uint32_t)((lane >> 4) * 16);
            continue;
        }
        const int grp = chunk >> 1;
        const int slot = (chunk & 1) * 64 + lane;
        const int kq = slot >> 5, rr = (slot >> 1) & 15, h = (slot & 1) ^ frag_swap(rr);
        int row0;
        if (STAGE == 1)
            row0 = grp < 8 ? n0 + 16 * grp : g.inter + n0 + 16 * (grp - 8);
        else
            row0 = n0 + 16 * grp;
        if (SHUFFLED)   // (16,16) layout: [K/32][h][row 16][16 B] per 16-row group
            b_off[i] = (uint32_t)row0 * (uint32_t)K + (uint32_t)(kq * 512 + h * 256 + rr * 16);
        else
            b_off[i] = (uint32_t)(row0 + rr) * (uint32_t)K + (uint32_t)(kq * 32 + h * 16);
    }
    uint32_t sa_off;                      // lane's scale: row tid (rows >= BM re-read row 0)
    {
        int arow = tid < BM ? s_arow[tid] : 0;
        if (arow < 0) arow = 0;
        sa_off = (uint32_t)((int64_t)arow * g.sa_row * 4);
    }
    const Rsrc ra = make_rsrc(g.a, (uint32_t)(g.a_rows * K));
    const Rsrc rb = make_rsrc(we, (uint32_t)((int64_t)g.N * KBY));
    Rsrc rs = make_rsrc(g.a_scale, (uint32_t)g.sa_bytes);
    uint32_t sa_kb_bytes = (uint32_t)(g.sa_kb * 4);
    // A8W4: waves SA_WAVES..SA_WAVES+3 fetch the e8m0 dwords of tile rows
    // j = (wave - SA_WAVES) * 64 + lane instead of activation scales
    if (W4 && wvu >= T::SA_WAVES && wvu < T::SA_WAVES + 4) {
        const int j = (wvu - T::SA_WAVES) * 64 + lane;
        const int row = STAGE == 1 ? (j < 128 ? n0 + j : g.inter + n0 + (j - 128)) : n0 + j;
        const int KS = K / 32;                           // e8m0 bytes per weight row
        rs = make_rsrc(g.w_scale8 + (int64_t)e * g.N * KS, (uint32_t)(g.N * KS));
        sa_off = (uint32_t)(row * KS);
        sa_kb_bytes = 4;
    }

    auto issue = [&](int kb, int stage) {
        kb = kb < KB ? kb : KB - 1;       // past the end: repeat the last step (keeps counts uniform)
        const uint32_t aoff = (uint32_t)kb * kBK;
#pragma unroll
        for (int i = 0; i < A_INSTR; ++i)
            dma16(ra, a_off[i], aoff, lds_addr(&s_a[stage][(wvu * A_INSTR + i) * 1024]));
        const uint32_t boff = (uint32_t)kb * (SHUFFLED ? (uint32_t)GB : (uint32_t)GB / 16u);
#pragma unroll
        for (int i = 0; i < B_INSTR; ++i)
            dma16(rb, b_off[i], boff, lds_addr(&s_b[stage][(wvu * B_INSTR + i) * 1024]));
        dma4(rs, sa_off, (uint32_t)kb * sa_kb_bytes, lds_addr(&s_sa[stage][wvu * 64]));
    };

    v4f acc[NRT][4];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = v4f{0.f, 0.f, 0.f, 0.f};
    const int row_base = wm * (BM / 2);
    const int h0 = frag_swap(lr);
    // a wave whose BM/2 rows are all padding (sorting pads an expert's last
    // block at its end, so the second half of a block at most half full)
    // skips its MFMAs and FMAs: it still issues its share of every step's
    // loads and meets every barrier, its accumulators stay 0 and no row of
    // it is stored
    bool wave_rows = false;
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
        wave_rows |= __builtin_amdgcn_ballot_w64(s_arow[row_base + rt * 16 + lr] >= 0) != 0;

    // One K step of the wave's (BM/2) x 128 tile, software-pipelined across
    // column tiles: the NRT MFMAs of tile c+1 go into the other of two
    // temporary sets while the VALU folds tile c's results into the
    // accumulators (acc += blk * a_scale * w_scale), so the MFMA pipe never
    // waits for the block-scale FMAs.  The combined scales of the half
    // (gate / up, or the wave's stage-2 block) are recomputed per half.
    auto compute = [&](int kb, int stage) {
        const uint8_t* sa_src = &s_a[stage][0];
        const uint8_t* sb_src = &s_b[stage][0];
        // fragment = K bytes 0-15 from half h0, 16-31 from half h0^1 (h0 depends
        // only on lr: row_base and rt*16 are multiples of 16)
        auto frag = [&](const uint8_t* slot) {
            const v4i lo = *reinterpret_cast<const v4i*>(slot + h0 * 16);
            const v4i hi = *reinterpret_cast<const v4i*>(slot + (h0 ^ 1) * 16);
            return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        };
        // the lane's 32 K bytes of row tile rt: fp8 x fp8 pieces 2 lq, 2 lq + 1
        // (K 32 lq ..); fp8 x fp4 pieces lq, lq + 4 (K 16 lq .. and 64 + 16 lq ..)
        v8i afrag[NRT];
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
            const int row = row_base + rt * 16 + lr;
            const uint8_t* rp = sa_src + row * 128;
            const int p0 = W4 ? lq : 2 * lq, p1 = W4 ? lq + 4 : 2 * lq + 1;
            const v4i lo = *reinterpret_cast<const v4i*>(rp + ((p0 ^ a_swz(row)) << 4));
            const v4i hi = *reinterpret_cast<const v4i*>(rp + ((p1 ^ a_swz(row)) << 4));
            afrag[rt] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
        // column tile ct (0..3) -> 16-row weight group: stage 1 tiles 0,1 are gate
        // rows, 2,3 the matching up rows; stage 2 four consecutive groups
        auto group_of = [&](int ct) {
            if (STAGE == 1) return ct < 2 ? wn * 2 + ct : 8 + wn * 2 + (ct - 2);
            return wn * 4 + ct;
        };
        auto bfrag_at = [&](int ct) {
            const int grp = group_of(ct);
            if (W4) {
                const v4i lo = *reinterpret_cast<const v4i*>(sb_src + grp * 1024 + lane * 16);
                return v8i{lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
            }
            return frag(sb_src + grp * 2048 + lq * 512 + lr * 32);
        };
        // A8W4: the lane's e8m0 byte (MX block lq of its weight row) for tile ct
        const uint8_t* s_bs = reinterpret_cast<const uint8_t*>(&s_sa[stage][BM]);
        auto bscale_at = [&](int ct) {
            return W4 ? (int)s_bs[(group_of(ct) * 16 + lr) * 4 + lq] : 0;
        };
        auto mfma = [&](const v8i& a, const v8i& b, int bs) {
            return W4 ? mfma16x16x128_fp8_fp4(a, b, bs) : mfma16x16x128_fp8(a, b);
        };
        float sc[NRT][4];
        auto load_scales = [&](int half) {
            const float sw = W4 ? 1.0f : s_sw[half == 0 ? swsel0 : swsel1][kb];
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
                const v4f s4 = *reinterpret_cast<const v4f*>(&s_sa[stage][row_base + rt * 16 + 4 * lq]);
#pragma unroll
                for (int v = 0; v < 4; ++v) sc[rt][v] = W4 ? s4[v] : s4[v] * sw;
            }
        };
        v4f blk[2][NRT];
        v8i bfrag = bfrag_at(0);
        int bs = bscale_at(0);
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) blk[0][rt] = mfma(afrag[rt], bfrag, bs);
        load_scales(0);
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
            const int cur = ct & 1;
            if (ct + 1 < 4) {
                bfrag = bfrag_at(ct + 1);
                bs = bscale_at(ct + 1);
#pragma unroll
                for (int rt = 0; rt < NRT; ++rt)
                    blk[cur ^ 1][rt] = mfma(afrag[rt], bfrag, bs);
            }
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[rt][ct][v] += blk[cur][rt][v] * sc[rt][v];
            if (ct == 1 && STAGE == 1 && !W4) load_scales(1);
#pragma unroll
            for (int i = 0; i < NRT; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
            }
        }
    };

    // ---- pipeline: the prologue fills two stages; step k waits for its own
    // loads (the next step's may stay in flight), syncs, refills the stage
    // step k-1 used, computes.  One loop body with a rotating stage index
    // keeps the accumulators in fixed registers. ----
    issue(0, 0);
    issue(1, 1);
    int cs = 0;                           // stage buffer of step kb
    for (int kb = 0; kb < KB; ++kb) {
        wait_vm<T::LOADS>();
        __syncthreads();
        const int ls = cs == 0 ? kStages - 1 : cs - 1;   // buffer step kb-1 used
        issue(kb + kStages - 1, ls);
        if (wave_rows) compute(kb, cs);
        cs = cs == kStages - 1 ? 0 : cs + 1;
    }
    wait_vm<0>();
    __syncthreads();

    if (STAGE == 2) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = row_base + rt * 16 + 4 * lq + v;
                const int64_t t = s_orow[row];
                if (t < 0) continue;
                const float wgt = s_w[row];
                const int64_t dst = t * g.N + n0 + wn * 64 + lr;
#pragma unroll
                for (int ct = 0; ct < 4; ++ct)
                    acc_add(g.acc, g.acc_dtype, dst + ct * 16, acc[rt][ct][v] * wgt);
            }
        return;
    }

    // ---- stage 1 epilogue: silu(gate)*up -> bf16 -> 1x128 fp8 requant ----
    // wave wn holds output columns wn*32 + j*16 + lr (j = 0, 1) of the tile's 128
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
                    const float wg = g.sorted_w ? s_w[row_base + rt * 16 + 4 * lq + v] : 1.0f;
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
            if (lr == 0) s_amax[wn][row_base + rt * 16 + 4 * lq + v] = m;
        }
    __syncthreads();
    auto row_amax = [&](int row) {
        const float m = __builtin_fmaxf(__builtin_fmaxf(s_amax[0][row], s_amax[1][row]),
                                        __builtin_fmaxf(s_amax[2][row], s_amax[3][row]));
        return __builtin_fmaxf(m, 1e-10f);
    };
    uint8_t* s_q = &s_a[0][0];  // [BM][128] fp8 staging (the pipeline is drained)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int row = row_base + rt * 16 + 4 * lq + v;
            const float inv = 1.0f / (row_amax(row) * kInvFp8Max);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t b = f32x2_to_fp8x2(h[rt][j][v] * inv, 0.0f) & 0xFFu;
                s_q[row * kBK + wn * 32 + j * 16 + lr] = (uint8_t)b;
            }
        }
    __syncthreads();
    const int I = g.inter;
    for (int q = tid; q < BM * 8; q += kThreads) {
        const int row = q >> 3, part = q & 7;
        const int64_t orow = s_orow[row];
        if (orow < 0) continue;
        *reinterpret_cast<v4i*>(g.a2 + orow * I + n0 + part * 16) =
            *reinterpret_cast<const v4i*>(s_q + row * kBK + part * 16);
        if (part == 0) g.a2_scale[orow * (I / 128) + n0 / 128] = row_amax(row) * kInvFp8Max;
    }
}

template <int STAGE, bool SHUFFLED, bool W4>
static void launch_bm(int bm, int grid, Args& a, hipStream_t stream) {
    if (bm == 64)
        hipLaunchKernelGGL((moe_gemm_fp8bs_v2_kernel<64, STAGE, SHUFFLED, W4>), dim3(grid),
                           dim3(kThreads), 0, stream, a);
    else if (bm == 128)
        hipLaunchKernelGGL((moe_gemm_fp8bs_v2_kernel<128, STAGE, SHUFFLED, W4>), dim3(grid),
                           dim3(kThreads), 0, stream, a);
    else
        AMD_CHECK(false, "v2 GEMM block_m must be 64 or 128");
}

template <int STAGE>
static void launch(int bm, int grid, Args& a, int shuffled, bool w4, hipStream_t stream) {
    if (w4) {
        if (shuffled)
            launch_bm<STAGE, true, true>(bm, grid, a, stream);
        else
            launch_bm<STAGE, false, true>(bm, grid, a, stream);
    } else {
        if (shuffled)
            launch_bm<STAGE, true, false>(bm, grid, a, stream);
        else
            launch_bm<STAGE, false, false>(bm, grid, a, stream);
    }
}

static int64_t scale_bytes(int64_t rows, int64_t KB, int64_t sa_row, int64_t sa_kb) {
    return ((rows - 1) * sa_row + (KB - 1) * sa_kb + 1) * 4;
}

}  // namespace v2

namespace v2 {

// XCD groups along M and the staggered walk (xcd_tile): two groups for both
// stages, stage 1 staggered. Measured on MI355X at MiMo dims (A8W4) against
// one unstaggered group: T=8192 stage 1 1765 -> 1714 us, stage 2 unchanged
// (1144 us; staggered 1195); T=1024 stage 1 519 -> 502 us, stage 2 270 ->
// 258 us (staggered 296). AITER_AMD_V2_MSPLIT1 / _2 (1, 2, 4 or 8) and
// AITER_AMD_V2_MROT1 / _2 force them.
static int pick_msplit(int stage, int ng) {
    if (ng % 8 != 0) return 1;
    if (const char* env = getenv(stage == 1 ? "AITER_AMD_V2_MSPLIT1" : "AITER_AMD_V2_MSPLIT2")) {
        const int c = atoi(env);
        if (c == 1 || c == 2 || c == 4 || c == 8) return c;
    }
    return 2;
}

static int pick_mrot(int stage) {
    if (const char* env = getenv(stage == 1 ? "AITER_AMD_V2_MROT1" : "AITER_AMD_V2_MROT2"))
        return atoi(env) != 0;
    return stage == 1;
}

}  // namespace v2

bool v2_supported(int64_t block_m, int64_t K) {
    return (block_m == 64 || block_m == 128) && K > 0 && K % 128 == 0 && K / 128 <= 64;
}

void launch_moe_stage1_fp8bs_v2(const uint8_t* a, const float* a_scale, int64_t sa_row,
                                int64_t sa_kb, const uint8_t* w1, const float* w1_scale,
                                const uint8_t* w1_scale_e8m0, const int32_t* sorted_ids, const int32_t* sorted_eids,
                                const int32_t* num_valid, uint8_t* a2, float* a2_scale,
                                int64_t a_rows, int64_t K, int64_t inter, int64_t E, int64_t topk,
                                int64_t block_m, int64_t max_m_blocks, int shuffled,
                                hipStream_t stream, const float* sorted_w, int act) {
    v2::Args g{};
    g.sorted_w = sorted_w;                 // doweight_stage1 (or NULL)
    g.act = act;
    g.a = a;
    g.a_scale = a_scale;
    g.sa_row = sa_row;
    g.sa_kb = sa_kb;
    g.sa_bytes = v2::scale_bytes(a_rows, K / 128, sa_row, sa_kb);
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
    // MXFP4 stage 1 on 128-row sorted blocks runs 64-row tiles (two per
    // block; an empty second half exits at once), as fast as on 64-row
    // blocks, so the layer can take 128-row blocks for its stage 2 (the
    // prefill kernel's). AITER_AMD_V2_TILE1=128 keeps whole-block tiles.
    int tile = (w1_scale_e8m0 != nullptr && block_m == 128) ? 64 : (int)block_m;
    if (const char* env = getenv("AITER_AMD_V2_TILE1"))
        if (atoi(env) == 128 && block_m == 128) tile = 128;
    g.block_m = (int)block_m;
    g.m_blocks = (int)(max_m_blocks * (block_m / tile));
    AMD_CHECK(a_rows * K < (1ll << 32) && 2 * inter * K < (1ll << 32) &&
                  g.sa_bytes < (1ll << 32),
              "v2 GEMM needs 32-bit buffer offsets");
    g.msplit = v2::pick_msplit(1, g.n_tiles);
    g.mrot = v2::pick_mrot(1);
    const int64_t grid = xcd_grid(g.n_tiles, g.m_blocks, g.msplit);
    if (grid == 0) return;
    v2::launch<1>(tile, (int)grid, g, shuffled, w1_scale_e8m0 != nullptr, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

void launch_moe_stage2_fp8bs_v2(const uint8_t* a2, const float* a2_scale, const uint8_t* w2,
                                const float* w2_scale, const uint8_t* w2_scale_e8m0,
                                const int32_t* sorted_ids,
                                const float* sorted_w, const int32_t* sorted_eids,
                                const int32_t* num_valid, void* acc, int acc_dtype, int64_t a_rows,
                                int64_t inter, int64_t hidden, int64_t E, int64_t topk,
                                int64_t block_m, int64_t max_m_blocks, int shuffled,
                                hipStream_t stream) {
    v2::Args g{};
    g.a = a2;
    g.a_scale = a2_scale;
    g.sa_row = inter / 128;
    g.sa_kb = 1;
    g.sa_bytes = v2::scale_bytes(a_rows, inter / 128, g.sa_row, g.sa_kb);
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
    g.n_tiles = (int)(hidden / 256);
    g.m_blocks = (int)max_m_blocks;
    g.block_m = (int)block_m;
    AMD_CHECK(a_rows * inter < (1ll << 32) && hidden * inter < (1ll << 32) &&
                  g.sa_bytes < (1ll << 32),
              "v2 GEMM needs 32-bit buffer offsets");
    g.msplit = v2::pick_msplit(2, g.n_tiles);
    g.mrot = v2::pick_mrot(2);
    const int64_t grid = xcd_grid(g.n_tiles, max_m_blocks, g.msplit);
    if (grid == 0) return;
    v2::launch<2>((int)block_m, (int)grid, g, shuffled, w2_scale_e8m0 != nullptr, stream);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
