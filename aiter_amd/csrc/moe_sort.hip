// MoE token sorting: bucket every (token, slot) routing pair into per-expert
// segments padded to a multiple of the GEMM M-block (block_m).
//
// Output contract (bit-exact with the reference's sorting kernels,
// csrc/include/moe_sorting_opus.h:266-352 for the encoding and the worked
// example, 724-1059 one-shot, 2612-3130 multi-phase; closed form
// op_tests/test_moe_sorting.py:15-70):
//   * experts are laid out in ascending id order; an expert with no pair, or
//     one switched off by expert_mask, gets no segment;
//   * a segment holds the expert's pairs ordered by (token, slot) and is
//     padded to ceil(count/block_m)*block_m entries;
//   * sorted_ids[i] = (slot << 24) | token, sorted_weights[i] = w[token, slot];
//     padding entries are (topk << 24) | tokens with weight 0;
//   * sorted_expert_ids[b] = expert id of M-block b (the local id, i.e. the
//     exclusive prefix sum of expert_mask, when a mask is given);
//   * num_valid_ids = {total padded length, tokens};
//   * entries past num_valid_ids[0] are not written;
//   * ids outside [0, num_experts) are ignored;
//   * the optional zero buffer (the fp32 accumulator of the down GEMM) is
//     cleared for `tokens` rows, as the reference clears moe_buf.
//
// MI355X design (not the reference's LDS mesh + lane-group walk): tokens are
// cut into chunks of `ct` tokens.  Each chunk builds an LDS bitmap
// table[token][expert] of slot masks (a byte per cell for topk <= 8, a u32
// up to topk 32, so duplicates of an expert inside one token's top-k are all
// kept, in slot order); a thread per expert then counts the expert's pairs
// in each group of 8 rows (1 for u32 cells) into an LDS prefix, and a thread
// per pair writes the pair at its segment's start + the expert's pairs in
// earlier chunks + in earlier row groups + in earlier bits of its own group
// (no thread walks an expert's pairs one store after another).  Small batches
// (one chunk) run the whole sort in one block of one launch; the other
// blocks of that launch clear the accumulator.  Larger batches take two
// launches: per-chunk expert counts (plus the clearing), then one block per
// chunk that sums the counts of the chunks before it (and of all chunks,
// for the segment layout) and writes its pairs -- the prefix is recomputed
// by every block in parallel instead of by a serial scan launch.
#include <algorithm>
#include <cstdlib>

#include "common.h"
#include "quant_dev.h"

namespace aiter_amd {

constexpr int kSortThreads = 256;

struct SortParams {
    const int32_t* topk_ids;    // [rows, topk]
    const float* topk_w;        // [rows, topk]
    const int32_t* expert_mask; // [E] or null
    const int32_t* local_tokens;// [1] device scalar or null
    int32_t* sorted_ids;
    float* sorted_w;
    int32_t* sorted_eids;
    int32_t* num_valid;         // [2]
    int32_t* ws;                // per-chunk expert counts [num_chunks][E]
    void* zero_buf;             // cleared for `tokens` rows (may be null)
    int64_t zero_row_bytes;     // multiple of 16
    int64_t zero_skip16;        // leading 16-byte units of zero_buf left to the clear launch
                                // (they hold the chunk counts when ws lives in zero_buf)
    void* zero2;                // a second region cleared whole (may be null): the
    int64_t zero2_n16;          // stage-1 split-K arrival counters, in 16-byte units
    int rows;
    int topk;
    int E;
    int bm;
    int ct;
    int cell_bytes;             // 1 when topk <= 8 (u8 slot masks), else 4
    int num_chunks;
    int sort_blocks;            // blocks of the launch doing sorting work
    int zero_blocks;            // then blocks clearing zero_buf
    // optional 1x128 fp8 quant of the activations, run by q_blocks blocks
    // after the zero blocks of the one-shot or the counting launch, or after
    // the chunks of the scatter launch
    const uint16_t* qx;
    uint8_t* qq;
    float* qs;
    const int32_t* q_num_rows;
    int64_t q_rows;
    int q_cols;
    int q_bf16;
    int q_blocks;
    int q_first;               // the scatter launch's quant blocks start at block q_first of the quant
};

__host__ __device__ inline int table_words(int ct, int E, int cell_bytes) {
    return (ct * E * cell_bytes + 3) / 4;
}

__device__ __forceinline__ int sort_tokens(const SortParams& p) {
    int t = p.local_tokens ? p.local_tokens[0] : p.rows;
    return min(max(t, 0), p.rows);
}

// Clear the accumulator rows [0, tokens) and the whole second region with
// 16-byte stores; run by the blocks of a launch that are not sorting.
__device__ void zero_rows(const SortParams& p, int tokens, int block, int nblocks) {
    if (nblocks <= 0) return;
    const v4i z = {0, 0, 0, 0};
    const int64_t first = (int64_t)block * kSortThreads + threadIdx.x;
    const int64_t stride = (int64_t)nblocks * kSortThreads;
    if (p.zero_buf) {
        const int64_t n16 = (int64_t)tokens * p.zero_row_bytes / 16;
        v4i* dst = reinterpret_cast<v4i*>(p.zero_buf);
        for (int64_t i = p.zero_skip16 + first; i < n16; i += stride) dst[i] = z;
    }
    if (p.zero2) {
        v4i* dst = reinterpret_cast<v4i*>(p.zero2);
        for (int64_t i = first; i < p.zero2_n16; i += stride) dst[i] = z;
    }
}

// Clears the chunk counts once the scatter launch has read them, when they
// were kept at the start of the caller's moe_buf instead of a workspace.
__global__ __launch_bounds__(kSortThreads) void moe_sort_clear_kernel(v4i* dst, int64_t n16) {
    const v4i z = {0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * kSortThreads + threadIdx.x; i < n16;
         i += (int64_t)gridDim.x * kSortThreads)
        dst[i] = z;
}

// The chunk table holds a slot-mask cell per (token, expert): one byte when
// topk <= 8 and one u32 otherwise; byte cells are set with a u32 atomicOr
// on the aligned word that holds them.
__device__ __forceinline__ int chunk_rows(const SortParams& p, int c, int tokens) {
    return max(0, min(p.ct, tokens - c * p.ct));
}

// Fill table[rows][E] with slot bitmasks of chunk c (only the chunk's rows
// are cleared and used).  Each thread's ids and weights are loaded
// kPairBatch at a time before any of them is used, so one batch costs one
// memory round trip (the first batch is in flight while the table clears).
constexpr int kPairBatch = 4;

__device__ void build_table(const SortParams& p, uint32_t* table, int c, int tokens) {
    const int nrows = chunk_rows(p, c, tokens);
    const int nwords = (nrows * p.E * p.cell_bytes + 3) / 4;
    const int npairs = nrows * p.topk;
    const int64_t base = (int64_t)c * p.ct * p.topk;
    for (int i0 = 0; i0 < npairs; i0 += kPairBatch * kSortThreads) {
        int ev[kPairBatch];
#pragma unroll
        for (int u = 0; u < kPairBatch; ++u) {
            const int i = i0 + u * kSortThreads + (int)threadIdx.x;
            ev[u] = i < npairs ? p.topk_ids[base + i] : -1;
        }
        if (i0 == 0) {   // block-uniform: every thread takes the first batch
            for (int i = threadIdx.x; i < nwords; i += kSortThreads) table[i] = 0u;
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < kPairBatch; ++u) {
            const int i = i0 + u * kSortThreads + (int)threadIdx.x;
            if (i >= npairs) continue;
            const int e = ev[u];
            if (e >= 0 && e < p.E) {
                const int tl = i / p.topk;
                const int j = i - tl * p.topk;
                const int cell = tl * p.E + e;
                if (p.cell_bytes == 1)
                    atomicOr(&table[cell >> 2], (1u << j) << (8 * (cell & 3)));
                else
                    atomicOr(&table[cell], 1u << j);
            }
        }
    }
    __syncthreads();
}

__device__ __forceinline__ int wave_incl_scan(int v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        int n = __shfl_up(v, off, 64);
        if (lane >= off) v += n;
    }
    return v;
}

// Block-wide exclusive scan of one int per thread; returns the block total
// through *total.  `scratch` holds kSortThreads/64 ints of LDS.
__device__ int block_excl_scan(int v, int* scratch, int* total) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int incl = wave_incl_scan(v);
    if (lane == 63) scratch[wave] = incl;
    __syncthreads();
    int pre = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kSortThreads / 64; ++w) {
        int s = scratch[w];
        if (w < wave) pre += s;
        tot += s;
    }
    __syncthreads();
    *total = tot;
    return pre + incl - v;
}

// Given per-expert pair counts in s_total, lay out segments: s_start (padded
// start offset) and s_local (local expert id); write num_valid_ids when
// `write` (the padding and sorted_expert_ids are write_segments').
__device__ void finalize_segments(const SortParams& p, const int* s_total, const int* s_mask,
                                  int* s_start, int* s_local, int* scratch, int tokens,
                                  bool write) {
    const int E = p.E;
    const int bm = p.bm;
    const int ept = (E + kSortThreads - 1) / kSortThreads;
    const int base = threadIdx.x * ept;
    int psum = 0, msum = 0;
    for (int i = 0; i < ept; ++i) {
        int e = base + i;
        if (e < E) {
            int cnt = s_total[e];
            psum += s_mask[e] != 0 ? ((cnt + bm - 1) / bm) * bm : 0;
            msum += s_mask[e];
        }
    }
    int ptot, mtot;
    int ppre = block_excl_scan(psum, scratch, &ptot);
    int mpre = block_excl_scan(msum, scratch, &mtot);
    for (int i = 0; i < ept; ++i) {
        int e = base + i;
        if (e < E) {
            int cnt = s_total[e];
            s_start[e] = ppre;
            s_local[e] = mpre;
            ppre += s_mask[e] != 0 ? ((cnt + bm - 1) / bm) * bm : 0;
            mpre += s_mask[e];
        }
    }
    if (threadIdx.x == 0 && write) {
        p.num_valid[0] = ptot;
        p.num_valid[1] = tokens;
    }
    __syncthreads();
}

// Padding entries and sorted_expert_ids of the segment layout. One block
// (the one-shot kernel) gives each thread an expert. The nranks blocks of the
// multi-chunk scatter share the work instead: block `rank` takes every
// nranks-th expert, one wave per expert with its lanes writing consecutive
// entries, so a heavy expert's many M-block ids and padding entries are not
// one thread's serial loop on the launch's critical path.
__device__ void write_segments(const SortParams& p, const int* s_total, const int* s_mask,
                               const int* s_start, const int* s_local, int tokens, int rank,
                               int nranks) {
    const int bm = p.bm;
    const int32_t pad_id = (int32_t)(((uint32_t)(p.topk & 0xFF) << 24) | ((uint32_t)tokens & 0xFFFFFFu));
    const bool per_wave = nranks > 1;
    const int lane = per_wave ? (int)(threadIdx.x & 63) : 0;
    const int step = per_wave ? 64 : 1;
    const int e0 = per_wave ? rank + (int)(threadIdx.x >> 6) * nranks : (int)threadIdx.x;
    const int estep = per_wave ? nranks * (kSortThreads / 64) : kSortThreads;
    for (int e = e0; e < p.E; e += estep) {
        if (s_mask[e] == 0) continue;
        const int cnt = s_total[e];
        if (cnt == 0) continue;
        const int start = s_start[e];
        const int padded = ((cnt + bm - 1) / bm) * bm;
        const int eid = p.expert_mask ? s_local[e] : e;
        for (int b = start / bm + lane; b < (start + padded) / bm; b += step) p.sorted_eids[b] = eid;
        for (int i = start + cnt + lane; i < start + padded; i += step) {
            p.sorted_ids[i] = pad_id;
            p.sorted_w[i] = 0.0f;
        }
    }
}

// The slot masks of expert e in the 8 rows from tl0 (byte cells) as one
// 64-bit word: bit 8u + j is slot j of row tl0 + u, so ascending bits are
// ascending (token, slot). The prefix groups of the chunk table are these 8
// rows for byte cells and one row for u32 cells.
__device__ __forceinline__ uint64_t cells8(const SortParams& p, const uint8_t* cells, int tl0,
                                           int nrows, int e) {
    // the 8 rows' cells as two little-endian dwords (rows past nrows read 0)
    uint32_t lo = 0, hi = 0;
    const uint8_t* src = cells + tl0 * p.E + e;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if (tl0 + u < nrows) lo |= (uint32_t)src[u * p.E] << (8 * u);
        if (tl0 + 4 + u < nrows) hi |= (uint32_t)src[(4 + u) * p.E] << (8 * u);
    }
    return ((uint64_t)hi << 32) | lo;
}

// Per expert (a thread each), the pairs of the chunk's row groups before
// each group: s_pre[group][e]; the chunk's total goes to s_tot when given.
__device__ void chunk_prefix(const SortParams& p, const uint32_t* table, int nrows,
                             uint16_t* s_pre, int* s_tot) {
    const int E = p.E;
    const uint8_t* cells = reinterpret_cast<const uint8_t*>(table);
    for (int e = threadIdx.x; e < E; e += kSortThreads) {
        int run = 0;
        if (p.cell_bytes == 1) {
            for (int tl0 = 0, g = 0; tl0 < nrows; tl0 += 8, ++g) {
                s_pre[g * E + e] = (uint16_t)run;
                run += __popcll((unsigned long long)cells8(p, cells, tl0, nrows, e));
            }
        } else {
            for (int tl = 0; tl < nrows; ++tl) {
                s_pre[tl * E + e] = (uint16_t)run;
                run += __popc(table[tl * E + e]);
            }
        }
        if (s_tot) s_tot[e] = run;
    }
}

// Emit the pairs of chunk c, a thread per pair: the pair's place in its
// expert's segment is s_pos[e] (the segment start plus the pairs of earlier
// chunks) + the expert's pairs in earlier row groups of the chunk (s_pre) +
// those before it in its own group; experts switched off by the mask are
// skipped. Ids and routing weights are read again from global memory (the
// table's build just brought them into L2), coalesced.
__device__ void scatter_pairs(const SortParams& p, const uint32_t* table, int c, int tokens,
                              const int* s_pos, const int* s_mask, const uint16_t* s_pre) {
    const int E = p.E;
    const int t0 = c * p.ct;
    const int nrows = chunk_rows(p, c, tokens);
    const int npairs = nrows * p.topk;
    const int32_t* ids = p.topk_ids + (int64_t)t0 * p.topk;
    const float* wts = p.topk_w + (int64_t)t0 * p.topk;
    const uint8_t* cells = reinterpret_cast<const uint8_t*>(table);
    // i / topk by a float reciprocal: i < 2^13 and topk <= 32, so (i + 1/2) / topk
    // is at least 1/64 from an integer and the product rounds to the right side
    const float rtk = 1.0f / (float)p.topk;
    for (int i = threadIdx.x; i < npairs; i += kSortThreads) {
        const int e = ids[i];
        if (e < 0 || e >= E || s_mask[e] == 0) continue;
        const int tl = (int)(((float)i + 0.5f) * rtk);
        const int j = i - tl * p.topk;
        int rank;
        if (p.cell_bytes == 1) {
            const int tl0 = tl & ~7;
            const uint64_t mm = cells8(p, cells, tl0, nrows, e);
            rank = s_pre[(tl0 >> 3) * E + e] +
                   __popcll((unsigned long long)(mm & ((1ull << (8 * (tl - tl0) + j)) - 1ull)));
        } else {
            rank = s_pre[tl * E + e] + __popc(table[tl * E + e] & ((1u << j) - 1u));
        }
        const int pos = s_pos[e] + rank;
        p.sorted_ids[pos] = (int32_t)(((uint32_t)j << 24) | (uint32_t)(t0 + tl));
        p.sorted_w[pos] = wts[i];
    }
}

// LDS layout of the sorting kernels: table[ct*E] | s_total[E] | s_start[E] |
// s_local[E] | s_pos[E] | s_mask[E] | scratch[kSortThreads/64] |
// s_pre[prefix_groups(ct)*E] u16
struct SortLds {
    uint32_t* table;
    int* s_total;
    int* s_start;
    int* s_local;
    int* s_pos;
    int* s_mask;
    int* scratch;
    uint16_t* s_pre;
};

__host__ __device__ inline int prefix_groups(int ct, int cell_bytes) {
    const int g = cell_bytes == 1 ? 8 : 1;
    return (ct + g - 1) / g;
}

__device__ SortLds carve_lds(const SortParams& p, uint32_t* smem) {
    SortLds L;
    L.table = smem;
    L.s_total = reinterpret_cast<int*>(smem + table_words(p.ct, p.E, p.cell_bytes));
    L.s_start = L.s_total + p.E;
    L.s_local = L.s_start + p.E;
    L.s_pos = L.s_local + p.E;
    L.s_mask = L.s_pos + p.E;
    L.scratch = L.s_mask + p.E;
    L.s_pre = reinterpret_cast<uint16_t*>(L.scratch + kSortThreads / 64);
    return L;
}

__global__ __launch_bounds__(kSortThreads) void moe_sort_oneshot_kernel(SortParams p) {
    extern __shared__ uint32_t smem[];
    const int tokens = sort_tokens(p);
    if ((int)blockIdx.x >= p.sort_blocks) {
        const int b = (int)blockIdx.x - p.sort_blocks;
        if (b < p.zero_blocks)
            zero_rows(p, tokens, b, p.zero_blocks);
        else if (p.q_bf16)
            quant_groups_block<true>(p.qx, p.qq, p.qs, p.q_rows, p.q_cols, 0, p.q_num_rows, 1,
                                     b - p.zero_blocks);
        else
            quant_groups_block<false>(p.qx, p.qq, p.qs, p.q_rows, p.q_cols, 0, p.q_num_rows, 1,
                                      b - p.zero_blocks);
        return;
    }
    const SortLds L = carve_lds(p, smem);
    for (int e = threadIdx.x; e < p.E; e += kSortThreads)
        L.s_mask[e] = p.expert_mask ? p.expert_mask[e] : 1;   // published by the table's barriers
    build_table(p, L.table, 0, tokens);
    chunk_prefix(p, L.table, chunk_rows(p, 0, tokens), L.s_pre, L.s_total);
    __syncthreads();
    finalize_segments(p, L.s_total, L.s_mask, L.s_start, L.s_local, L.scratch, tokens, true);
    write_segments(p, L.s_total, L.s_mask, L.s_start, L.s_local, tokens, 0, 1);
    scatter_pairs(p, L.table, 0, tokens, L.s_start, L.s_mask, L.s_pre);
}

// Per-chunk expert counts by an LDS histogram of the chunk's ids (every
// (token, slot) pair with an id in range counts once, as in the table).
__global__ __launch_bounds__(kSortThreads) void moe_sort_count_kernel(SortParams p) {
    extern __shared__ uint32_t smem[];
    const int tokens = sort_tokens(p);
    if ((int)blockIdx.x >= p.sort_blocks) {
        const int b = (int)blockIdx.x - p.sort_blocks;
        if (b < p.zero_blocks)
            zero_rows(p, tokens, b, p.zero_blocks);
        else if (p.q_bf16)
            quant_groups_block<true>(p.qx, p.qq, p.qs, p.q_rows, p.q_cols, 0, p.q_num_rows, 1,
                                     b - p.zero_blocks);
        else
            quant_groups_block<false>(p.qx, p.qq, p.qs, p.q_rows, p.q_cols, 0, p.q_num_rows, 1,
                                      b - p.zero_blocks);
        return;
    }
    const int c = blockIdx.x;
    int* s_cnt = reinterpret_cast<int*>(smem);
    const int npairs = chunk_rows(p, c, tokens) * p.topk;
    const int64_t base = (int64_t)c * p.ct * p.topk;
    for (int i0 = 0; i0 < npairs || i0 == 0; i0 += kPairBatch * kSortThreads) {
        int ev[kPairBatch];
#pragma unroll
        for (int u = 0; u < kPairBatch; ++u) {
            const int i = i0 + u * kSortThreads + (int)threadIdx.x;
            ev[u] = i < npairs ? p.topk_ids[base + i] : -1;
        }
        if (i0 == 0) {
            for (int e = threadIdx.x; e < p.E; e += kSortThreads) s_cnt[e] = 0;
            __syncthreads();
        }
#pragma unroll
        for (int u = 0; u < kPairBatch; ++u)
            if (ev[u] >= 0 && ev[u] < p.E) atomicAdd(&s_cnt[ev[u]], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < p.E; e += kSortThreads) p.ws[(int64_t)c * p.E + e] = s_cnt[e];
}

// Block c: per expert, the pairs of chunks before c (its write offset inside
// the expert's segment) and of all chunks (the segment layout, which every
// block derives identically); block 0 also writes the padding, the
// sorted_expert_ids and num_valid_ids.  Then the chunk's pairs.
constexpr int kChunkBatch = 16;   // per-chunk counts loaded per round trip

__global__ __launch_bounds__(kSortThreads) void moe_sort_scatter_kernel(SortParams p) {
    extern __shared__ uint32_t smem[];
    if ((int)blockIdx.x >= p.num_chunks) {   // the activation quant, beside the chunks
        const int b = (int)blockIdx.x - p.num_chunks + p.q_first;
        if (p.q_bf16)
            quant_groups_block<true>(p.qx, p.qq, p.qs, p.q_rows, p.q_cols, 0, p.q_num_rows, 1, b);
        else
            quant_groups_block<false>(p.qx, p.qq, p.qs, p.q_rows, p.q_cols, 0, p.q_num_rows, 1, b);
        return;
    }
    const int tokens = sort_tokens(p);
    const int c = blockIdx.x;
    const SortLds L = carve_lds(p, smem);
    const int E = p.E;
    for (int e = threadIdx.x; e < E; e += kSortThreads) {
        L.s_mask[e] = p.expert_mask ? p.expert_mask[e] : 1;   // in flight with the counts
        int before = 0, total = 0;
        for (int k = 0; k < p.num_chunks; k += kChunkBatch) {
            int v[kChunkBatch];
#pragma unroll
            for (int u = 0; u < kChunkBatch; ++u)
                v[u] = k + u < p.num_chunks ? p.ws[(int64_t)(k + u) * E + e] : 0;
#pragma unroll
            for (int u = 0; u < kChunkBatch; ++u) {
                before += k + u < c ? v[u] : 0;
                total += v[u];
            }
        }
        L.s_total[e] = total;
        L.s_pos[e] = before;
    }
    __syncthreads();
    finalize_segments(p, L.s_total, L.s_mask, L.s_start, L.s_local, L.scratch, tokens, c == 0);
    write_segments(p, L.s_total, L.s_mask, L.s_start, L.s_local, tokens, c, p.num_chunks);
    for (int e = threadIdx.x; e < E; e += kSortThreads) L.s_pos[e] += L.s_start[e];
    if (c * p.ct >= tokens) return;
    build_table(p, L.table, c, tokens);   // its barriers also publish s_pos
    chunk_prefix(p, L.table, chunk_rows(p, c, tokens), L.s_pre, nullptr);
    __syncthreads();
    scatter_pairs(p, L.table, c, tokens, L.s_pos, L.s_mask, L.s_pre);
}

// Tokens per chunk: at most the largest power of two <= 256 whose slot-mask
// table fits in 48 KB of LDS (one chunk, the one-shot launch, when the batch
// fits). With the five per-expert arrays (80 KB at E = 4096) and the
// row-group prefix (at most 16 KB) a block's LDS stays under gfx950's 160 KB.
// With several chunks, smaller ones spread the per-chunk walks over more
// blocks: about 64 chunks (ct = rows / 64 rounded down to a power of two, at
// least 16), about 128 above 4096 rows. Measured on MI355X at MiMo dims (E =
// 256, top-8; sort launches' time in the layer): T=512 30.2 -> 17.7 us (ct
// 16), T=1024 29.2 -> 20.2 us (16), T=2048 28.6 -> 21.6 us (32), EP share
// T=4096 33.2 -> 29.3 us (64), T=8192 with the activation quant split 37.6
// us at ct 128, 35.1 at 64, 38.0 at 32. AITER_AMD_SORT_CT forces a power of
// two up to the table limit.
static int sort_chunk_tokens(int E, int topk, int64_t rows) {
    const int cell = topk <= 8 ? 1 : 4;
    int ct = 256;
    while (ct > 1 && (int64_t)ct * E * cell > 48 * 1024) ct >>= 1;
    if (rows > ct) {
        if (const char* env = getenv("AITER_AMD_SORT_CT")) {
            const int c = atoi(env);
            if (c >= 1 && c <= ct && (c & (c - 1)) == 0) return c;
        }
        // T=2048, 4096 and the EP share measured level or slower with twice
        // the chunks
        const int64_t per_chunk = rows > 4096 ? 128 : 64;
        int c = 16;
        while (c * 2 <= ct && (int64_t)c * 2 * per_chunk <= rows) c *= 2;
        ct = c < ct ? c : ct;
    }
    return ct;
}

int64_t sort_workspace_bytes(int64_t rows, int64_t topk, int64_t E) {
    int ct = sort_chunk_tokens((int)E, (int)topk, rows);
    int64_t chunks = ceil_div(rows > 0 ? rows : 1, ct);
    if (chunks <= 1) return 0;
    return chunks * E * 4;
}

// Returns true when the launch also ran the activation quant given by qx
// (rows x q_cols, bf16 or fp16, scales row-major, num_rows = local_tokens),
// in extra blocks of the one-shot, the counting or the scatter launch.
bool launch_moe_sort(const int32_t* topk_ids, const float* topk_w, const int32_t* expert_mask,
                     const int32_t* local_tokens, int32_t* sorted_ids, float* sorted_w,
                     int32_t* sorted_eids, int32_t* num_valid, void* zero_buf,
                     int64_t zero_row_bytes, int64_t rows, int64_t topk, int64_t E, int64_t bm,
                     void* ws, int64_t ws_bytes, hipStream_t stream, const void* qx,
                     int qx_dtype, uint8_t* qq, float* qs, int64_t q_cols, void* zero2,
                     int64_t zero2_bytes) {
    AMD_CHECK(zero2_bytes % 16 == 0, "second clear region must be a multiple of 16 bytes");
    SortParams p;
    p.topk_ids = topk_ids;
    p.topk_w = topk_w;
    p.expert_mask = expert_mask;
    p.local_tokens = local_tokens;
    p.sorted_ids = sorted_ids;
    p.sorted_w = sorted_w;
    p.sorted_eids = sorted_eids;
    p.num_valid = num_valid;
    p.zero_buf = zero_buf;
    p.zero_row_bytes = zero_row_bytes;
    p.zero_skip16 = 0;
    p.zero2 = zero2_bytes > 0 ? zero2 : nullptr;
    p.zero2_n16 = zero2_bytes / 16;
    p.rows = (int)rows;
    p.topk = (int)topk;
    p.E = (int)E;
    p.bm = (int)bm;
    p.ct = sort_chunk_tokens((int)E, (int)topk, rows);
    p.cell_bytes = topk <= 8 ? 1 : 4;
    p.num_chunks = (int)ceil_div(rows > 0 ? rows : 1, p.ct);
    p.ws = reinterpret_cast<int32_t*>(ws);
    p.qx = nullptr;
    p.qq = nullptr;
    p.qs = nullptr;
    p.q_num_rows = nullptr;
    p.q_rows = 0;
    p.q_cols = 0;
    p.q_bf16 = 0;
    p.q_blocks = 0;
    p.q_first = 0;

    // zero blocks: about one 16-byte store per thread per 4 iterations
    int zero_blocks = 0;
    if ((zero_buf || p.zero2) && rows > 0) {
        int64_t n16 = (zero_buf ? rows * zero_row_bytes / 16 : 0) + p.zero2_n16;
        zero_blocks = (int)std::min<int64_t>(ceil_div(n16, (int64_t)kSortThreads * 4), 2048);
        if (zero_blocks < 1) zero_blocks = 1;
    }
    const size_t table_lds = (size_t)table_words(p.ct, (int)E, p.cell_bytes) * 4;
    const size_t full_lds = table_lds + (size_t)(5 * E + kSortThreads / 64) * 4 +
                            (size_t)prefix_groups(p.ct, p.cell_bytes) * E * 2;
    p.zero_blocks = zero_blocks;
    // the activation quant rides in extra blocks of one of the sorting launches
    bool quant_done = false;
    if (qx && rows > 0 && q_cols >= 128) {
        const int64_t qb = ceil_div(rows * (q_cols / 128), kQuantThreads / 16);
        AMD_CHECK(qb < (1ll << 30), "too many rows to quantise");
        p.qx = reinterpret_cast<const uint16_t*>(qx);
        p.qq = qq;
        p.qs = qs;
        p.q_num_rows = local_tokens;
        p.q_rows = rows;
        p.q_cols = (int)q_cols;
        p.q_bf16 = qx_dtype == DT_BF16;
        p.q_blocks = (int)qb;
        quant_done = true;
    }
    if (p.num_chunks == 1) {
        p.sort_blocks = 1;
        hipLaunchKernelGGL(moe_sort_oneshot_kernel, dim3(1 + zero_blocks + p.q_blocks),
                           dim3(kSortThreads), full_lds, stream, p);
    } else {
        const int64_t need = sort_workspace_bytes(rows, topk, E);
        AMD_CHECK(ws != nullptr && ws_bytes >= need, "sorting workspace too small");
        // the counts may live at the start of zero_buf itself (moe_buf, for
        // callers that pass no workspace): the counting launch then leaves
        // those bytes alone and a third launch clears them after the scatter
        const bool ws_in_buf = ws == zero_buf;
        if (ws_in_buf) {
            AMD_CHECK(rows * zero_row_bytes >= need, "moe_buf too small to hold the sorting counts");
            p.zero_skip16 = ceil_div(need, 16);
        }
        p.sort_blocks = p.num_chunks;
        // Up to 4096 rows the activation quant rides in the scatter launch,
        // whose few sorting blocks leave most CUs free; larger quants are
        // split, half in the counting launch and half in the scatter launch,
        // so that neither the latency-bound scatter nor the counting launch
        // waits on all of it. Measured on MI355X at MiMo dims (sort launches'
        // time in the layer, HIP events): EP share T=4096 all in the counting
        // launch 28.7 -> 23.0 us in the scatter launch; T=8192 42.4 us all in
        // the counting launch, 45.0 all in the scatter launch, 37.0 split in
        // half (39.6 at three quarters, 40.1 at one quarter); T=2048 and the
        // EP share are best with all of it in the scatter launch.
        const int q_count = rows <= 4096 ? 0 : p.q_blocks / 2;   // quant blocks [0, q_count)
        p.q_first = q_count;
        hipLaunchKernelGGL(moe_sort_count_kernel,
                           dim3(p.num_chunks + zero_blocks + q_count),
                           dim3(kSortThreads), (size_t)E * 4, stream, p);
        hipLaunchKernelGGL(moe_sort_scatter_kernel,
                           dim3(p.num_chunks + (p.q_blocks - q_count)),
                           dim3(kSortThreads), full_lds, stream, p);
        if (ws_in_buf) {
            const int64_t nb = std::min<int64_t>(ceil_div(p.zero_skip16, kSortThreads), 1024);
            hipLaunchKernelGGL(moe_sort_clear_kernel, dim3(nb), dim3(kSortThreads), 0, stream,
                               reinterpret_cast<v4i*>(zero_buf), p.zero_skip16);
        }
    }
    AMD_HIP_CHECK(hipGetLastError());
    return quant_done;
}

// ------------------------------------------ sorted metadata -> routing ---
// The inverse of sorting for one layer's sorted metadata: topk_ids[t, j] =
// the expert of the M-block holding entry (j << 24) | t, topk_w[t, j] its
// weight, for the entries below num_valid[0] with t < num_valid[1]; pairs
// with no entry (routed to experts another GPU holds) get id -1, which
// sorting and the slot sum ignore. Two launches: fill, then scatter.
__global__ __launch_bounds__(256) void unsort_fill_kernel(int32_t* __restrict__ ids,
                                                          float* __restrict__ w, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * 256) {
        ids[i] = -1;
        w[i] = 0.0f;
    }
}

__global__ __launch_bounds__(256) void unsort_scatter_kernel(
    const int32_t* __restrict__ sorted_ids, const float* __restrict__ sorted_w,
    const int32_t* __restrict__ sorted_eids, const int32_t* __restrict__ num_valid,
    int64_t capacity, int block_m, int32_t* __restrict__ ids, float* __restrict__ w,
    int64_t tokens, int topk, int E) {
    int64_t n = (int64_t)num_valid[0];
    n = n < capacity ? n : capacity;
    int64_t nt = (int64_t)num_valid[1];
    nt = nt < tokens ? nt : tokens;
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < n;
         r += (int64_t)gridDim.x * 256) {
        const uint32_t id = (uint32_t)sorted_ids[r];
        const int64_t t = (int64_t)(id & 0xFFFFFFu);
        const int s = (int)(id >> 24);
        if (t >= nt || s >= topk) continue;                 // padding entry
        const int e = sorted_eids[r / block_m];
        if (e < 0 || e >= E) continue;
        ids[t * topk + s] = e;
        w[t * topk + s] = sorted_w[r];
    }
}

void launch_unsort(const int32_t* sorted_ids, const float* sorted_w, const int32_t* sorted_eids,
                   const int32_t* num_valid, int64_t sorted_capacity, int64_t block_m,
                   int32_t* topk_ids, float* topk_w, int64_t tokens, int64_t topk, int64_t E,
                   hipStream_t stream) {
    const int64_t n = tokens * topk;
    if (n == 0) return;
    hipLaunchKernelGGL(unsort_fill_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(n, 256), 4096)),
                       dim3(256), 0, stream, topk_ids, topk_w, n);
    if (sorted_capacity > 0)
        hipLaunchKernelGGL(unsort_scatter_kernel,
                           dim3((unsigned)std::min<int64_t>(ceil_div(sorted_capacity, 256), 4096)),
                           dim3(256), 0, stream, sorted_ids, sorted_w, sorted_eids, num_valid,
                           sorted_capacity, (int)block_m, topk_ids, topk_w, tokens, (int)topk,
                           (int)E);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
