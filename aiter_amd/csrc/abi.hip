// extern "C" boundary of libaiter_amd.so: argument validation, the
// thread-local error bridge, workspace layout of the fused entry point, and
// dispatch to the kernel launchers.  Declarations and the reference
// interface each entry point replaces are in include/aiter_amd.h.
#include "../../include/aiter_amd.h"
#include "../../include/aiter_ctypes.h"

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "common.h"

namespace aiter_amd {

static thread_local std::string g_last_error;

void set_last_error(const std::string& msg) { g_last_error = msg; }
void clear_last_error() { g_last_error.clear(); }

// launchers (moe_sort.hip, quant.hip, moe_gemm_fp8bs.hip)
int64_t sort_workspace_bytes(int64_t rows, int64_t topk, int64_t E);
// returns true when it also ran the activation quant given by the last five arguments
bool launch_moe_sort(const int32_t*, const float*, const int32_t*, const int32_t*, int32_t*,
                     float*, int32_t*, int32_t*, void*, int64_t, int64_t, int64_t, int64_t,
                     int64_t, void*, int64_t, hipStream_t, const void* qx = nullptr,
                     int qx_dtype = 0, uint8_t* qq = nullptr, float* qs = nullptr,
                     int64_t q_cols = 0, void* zero2 = nullptr, int64_t zero2_bytes = 0);
void launch_per_group_quant_fp8(const void*, int, void*, float*, int64_t, int64_t, int,
                                const int32_t*, int64_t, hipStream_t);
// addend (optional): a [rows, cols] tensor of the output dtype added before
// the rounding (it may be out itself)
void launch_acc_to_out(const float*, void*, int, const int32_t*, int64_t, int64_t, hipStream_t,
                       const void* addend = nullptr);
// out[r, c] = act(in[r, c]) * in[r, d + c], rows of in 2d wide (quant.hip)
void launch_act_and_mul(const void* in, int in_dtype, void* out, int out_dtype, int64_t rows,
                        int64_t d, int act, hipStream_t stream);
// zero `bytes` (a multiple of 16) at a 16-byte aligned p with a kernel (quant.hip)
void launch_zero(void* p, int64_t bytes, hipStream_t stream);
// moe_sort.hip: per-pair expert ids and weights [tokens, topk] recovered from
// a layer's sorted metadata (-1 / 0 where the pair was not routed here)
void launch_unsort(const int32_t* sorted_ids, const float* sorted_w, const int32_t* sorted_eids,
                   const int32_t* num_valid, int64_t sorted_capacity, int64_t block_m,
                   int32_t* topk_ids, float* topk_w, int64_t tokens, int64_t topk, int64_t E,
                   hipStream_t stream);
void launch_moe_stage1_stream_rows(const uint8_t*, const float*, int64_t, int64_t,
                                   const uint8_t*, const float*, const uint8_t*, const int32_t*,
                                   const int32_t*, const int32_t*, void*, int, int, int64_t,
                                   int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int,
                                   hipStream_t, const float*, int, int);
// The GEMM launchers take the weight scales either as fp32 128x128 blocks
// (FP8 weights) or, when the e8m0 pointer is non-null, as e8m0 bytes per
// 1x32 K block (MXFP4 weights, A8W4).
void launch_moe_stage1_fp8bs(const uint8_t*, const float*, int64_t, int64_t, const uint8_t*,
                             const float*, const uint8_t*, const int32_t*, const int32_t*,
                             const int32_t*, uint8_t*, float*, int64_t, int64_t, int64_t, int64_t,
                             int64_t, int64_t, int64_t, int, hipStream_t,
                             const float*, int);
void launch_moe_stage2_fp8bs(const uint8_t*, const float*, const uint8_t*, const float*,
                             const uint8_t*, const int32_t*, const float*, const int32_t*,
                             const int32_t*, void*, int, int64_t, int64_t, int64_t, int64_t, int64_t,
                             int64_t, int64_t, int, hipStream_t);
// moe_gemm_fp8bs_v2.hip (64/128-row M-blocks)
bool v2_supported(int64_t block_m, int64_t K);
void launch_moe_stage1_fp8bs_v2(const uint8_t*, const float*, int64_t, int64_t, const uint8_t*,
                                const float*, const uint8_t*, const int32_t*, const int32_t*,
                                const int32_t*, uint8_t*, float*, int64_t, int64_t, int64_t,
                                int64_t, int64_t, int64_t, int64_t, int, hipStream_t,
                             const float*, int);
void launch_moe_stage2_fp8bs_v2(const uint8_t*, const float*, const uint8_t*, const float*,
                                const uint8_t*, const int32_t*, const float*, const int32_t*,
                                const int32_t*, void*, int, int64_t, int64_t, int64_t, int64_t,
                                int64_t, int64_t, int64_t, int, hipStream_t);

// moe_gemm_stream.hip (16/32-row M-blocks, weights streamed into registers)
bool stream_supported(int64_t block_m, int64_t K);
void launch_moe_stage1_stream(const uint8_t*, const float*, int64_t, int64_t, const uint8_t*,
                              const float*, const uint8_t*, const int32_t*, const int32_t*,
                              const int32_t*, uint8_t*, float*, int64_t, int64_t, int64_t,
                              int64_t, int64_t, int64_t, int64_t, int, hipStream_t,
                              const float*, int, int ksplit = 1, void* kpart = nullptr,
                              int32_t* kcnt = nullptr, int64_t kmb = 0,
                              StreamDirect direct = StreamDirect{});
// the fused layer (both GEMMs in one launch) on the stream kernel
bool stream_fused_supported(int64_t block_m, int64_t hidden, int64_t inter);
void launch_moe_fused_stream(const uint8_t*, const float*, int64_t, int64_t, const uint8_t*,
                             const float*, const uint8_t*, const uint8_t*, const float*,
                             const uint8_t*, const int32_t*, const float*, const float*,
                             const int32_t*, const int32_t*, float*, int64_t, int64_t, int64_t,
                             int64_t, int64_t, int64_t, int64_t, int, hipStream_t, int, int, void*,
                             int32_t*, int64_t);
// stage-1 split-K of the stream kernel: K ranges per tile for a layer
// expected to route est_blocks M-blocks, and its partial-sum bytes
int stream_stage1_ksplit(int64_t block_m, int64_t K, int64_t inter, int64_t est_blocks);
int64_t stream_ksplit_part_bytes(int64_t block_m, int64_t mblocks, int64_t inter, int64_t ksplit);
void launch_moe_stage2_stream(const uint8_t*, const float*, const uint8_t*, const float*,
                              const uint8_t*, const int32_t*, const float*, const int32_t*,
                              const int32_t*, void*, int, int64_t, int64_t, int64_t, int64_t,
                              int64_t, int64_t, int64_t, int, hipStream_t);

// one token: stage 2 with the token's slots summed per workgroup, into out
void launch_moe_token_stage2(const uint8_t*, const float*, const uint8_t*, const float*,
                             const uint8_t*, const int32_t*, const float*, void*, int, const void*,
                             int64_t, int64_t, int64_t, int64_t, int, hipStream_t);

// quant.hip: per-pair bf16 rows -> output
void launch_slot_sum(const uint16_t* part, const int32_t* topk_ids, const int32_t* mask,
                     int64_t num_experts, const int32_t* num_valid, void* out, int out_dtype,
                     int64_t rows, int64_t topk, int64_t cols, hipStream_t stream,
                     const void* addend = nullptr);

// moe_route.hip (router top-k)
bool route_supported(int64_t E, int64_t k);
void launch_moe_route(const void* gating, int dtype, int64_t M, int64_t E, int64_t k, int mode,
                      int need_renorm, int softmax_scores, int64_t n_group, int64_t topk_group,
                      float scaling, const float* bias, float* w, int64_t ws, int32_t* ids,
                      int64_t is, int32_t* tei, hipStream_t stream, int64_t gating_stride = 0,
                      int64_t num_shared = 0);

// moe_gemm_prefill.hip (64/128-row M-blocks, weight fragments in registers)
bool prefill_supported(int64_t block_m, int64_t K);
void launch_moe_stage1_prefill(const uint8_t*, const float*, int64_t, int64_t, const uint8_t*,
                               const float*, const uint8_t*, const int32_t*, const int32_t*,
                               const int32_t*, uint8_t*, float*, int64_t, int64_t, int64_t,
                               int64_t, int64_t, int64_t, int64_t, int, hipStream_t,
                             const float*, int);
void launch_moe_stage2_prefill(const uint8_t*, const float*, const uint8_t*, const float*,
                               const uint8_t*, const int32_t*, const float*, const int32_t*,
                               const int32_t*, void*, int, uint16_t*, int64_t, int64_t, int64_t,
                               int64_t, int64_t, int64_t, int64_t, int, hipStream_t, int64_t);

// The 64/128-row kernels (prefill, v2) read their activation operand through
// 32-bit buffer offsets, so its a_rows * K bytes must stay below 4 GiB.
// Larger operands take the general kernel (64-bit addresses, block_m <= 64).
static bool a_fits32(int64_t a_rows, int64_t K) { return a_rows * K < (int64_t(1) << 32); }

// Weight scales of one layer: fp32 128x128 blocks (fp8 weights) or e8m0
// bytes per 1x32 K block (MXFP4 weights); exactly one is set.
struct WScale {
    const float* f32;
    const uint8_t* e8m0;
};

// Kernel choice per shape (measured on MI355X): 16/32-row M-blocks
// (decode-sized layers) take the register-streaming kernels; 64/128-row
// M-blocks take, for FP8 weights, the register-B prefill kernels and, for
// MXFP4 weights, the same kernels once the experts average enough routed rows
// (below that the direct-to-LDS kernels; stage 2 at 128 rows always takes the
// prefill kernel).  Stage 2 of all of them needs 256-column output tiles
// (model_dim % 256 == 0); other shapes take the general kernels of
// moe_gemm_fp8bs.hip.
// sw: sorted routing weights for doweight_stage1 (applied to gate and up
// before the activation), or NULL; act: kActSilu or kActGelu.
// MXFP4 weights take the prefill kernels (weights in registers, the tile's
// e8m0 bytes in LDS) once the experts average at least 16 routed rows for
// stage 1 and 48 for stage 2, and the direct-to-LDS MXFP4 kernels below
// (their waves skip padding-only 32-row halves, and their stage 2 adds into
// an fp32 accumulator instead of writing per-pair rows that a second pass
// sums). Measured on MI355X at MiMo dims, bm 64, prefill vs MXFP4 kernel:
// stage 1 T=512 (16 rows per expert) 443-449 vs 452-454 us, T=2048 499 vs
// 664 us; stage 2 with its finishing pass T=1024 (32 rows) 274 vs 266 us,
// T=2048 316 vs 379 us. AITER_AMD_W4_PF_ROWS1 / _2 override the thresholds
// (tests use them).
static bool w4_on_prefill(int64_t pairs, int64_t E, int stage) {
    int64_t rows = stage == 1 ? 16 : 48;
    if (const char* env = getenv(stage == 1 ? "AITER_AMD_W4_PF_ROWS1" : "AITER_AMD_W4_PF_ROWS2"))
        rows = atoll(env);
    return pairs >= rows * E;
}

static void stage1_dispatch(const uint8_t* a, const float* sa, int64_t sa_row, int64_t sa_kb,
                            const uint8_t* w1, WScale w1s, const int32_t* sid,
                            const int32_t* seid, const int32_t* nv, uint8_t* a2, float* a2s,
                            int64_t a_rows, int64_t K, int64_t I, int64_t E, int64_t topk,
                            int64_t bm, int64_t mblocks, int sh, hipStream_t s,
                            const float* sw, int act, int ksplit = 1, void* kpart = nullptr,
                            int32_t* kcnt = nullptr, int64_t kmb = 0, int64_t est_pairs = -1) {
    if (stream_supported(bm, K))
        launch_moe_stage1_stream(a, sa, sa_row, sa_kb, w1, w1s.f32, w1s.e8m0, sid, seid, nv, a2,
                                 a2s, a_rows, K, I, E, topk, bm, mblocks, sh, s, sw, act, ksplit,
                                 kpart, kcnt, kmb);
    else if (prefill_supported(bm, K) &&
             (!w1s.e8m0 || w4_on_prefill(est_pairs < 0 ? a_rows * topk : est_pairs, E, 1)) &&
             a_fits32(a_rows, K))
        launch_moe_stage1_prefill(a, sa, sa_row, sa_kb, w1, w1s.f32, w1s.e8m0, sid, seid, nv, a2,
                                  a2s, a_rows, K, I, E, topk, bm, mblocks, sh, s, sw, act);
    else if (v2_supported(bm, K) && a_fits32(a_rows, K))
        launch_moe_stage1_fp8bs_v2(a, sa, sa_row, sa_kb, w1, w1s.f32, w1s.e8m0, sid, seid, nv, a2,
                                   a2s, a_rows, K, I, E, topk, bm, mblocks, sh, s, sw, act);
    else
        launch_moe_stage1_fp8bs(a, sa, sa_row, sa_kb, w1, w1s.f32, w1s.e8m0, sid, seid, nv, a2,
                                a2s, a_rows, K, I, E, topk, bm, mblocks, sh, s, sw, act);
}

// Stage 2 runs on the prefill kernel for this shape (the only stage-2
// kernel that can also write per-pair bf16 rows instead of accumulating).
static bool stage2_on_prefill(int64_t bm, int64_t I, int64_t H, WScale w2s, int64_t a_rows,
                              int64_t E, int64_t est_pairs) {
    return !(stream_supported(bm, I) && H % 256 == 0) && prefill_supported(bm, I) &&
           a_fits32(a_rows, I) &&
           H % 256 == 0 &&
           (!w2s.e8m0 || bm == 128 || w4_on_prefill(est_pairs < 0 ? a_rows : est_pairs, E, 2));
}

// acc: [tokens, H] accumulated atomically, fp32 or (the reference's moe_buf)
// bf16 / fp16 by acc_dtype; part (prefill kernel only): bf16 [pairs, H] rows
// written once each, acc unused.
// est_pairs: the pairs expected on this GPU (the EP share's fraction of
// tokens * topk when the caller knows it), a launch-shape hint only.
static void stage2_dispatch(const uint8_t* a2, const float* a2s, const uint8_t* w2,
                            WScale w2s, const int32_t* sid, const float* sw,
                            const int32_t* seid, const int32_t* nv, void* acc, int acc_dtype,
                            int64_t a_rows, int64_t I, int64_t H, int64_t E, int64_t topk,
                            int64_t bm, int64_t mblocks, int sh, hipStream_t s,
                            uint16_t* part = nullptr, int64_t est_pairs = -1) {
    const bool on_prefill = stage2_on_prefill(bm, I, H, w2s, a_rows, E, est_pairs);
    AMD_CHECK(!part || on_prefill, "per-pair rows need the prefill kernel");
    if (stream_supported(bm, I) && H % 256 == 0)
        launch_moe_stage2_stream(a2, a2s, w2, w2s.f32, w2s.e8m0, sid, sw, seid, nv, acc,
                                 acc_dtype, a_rows, I, H, E, topk, bm, mblocks, sh, s);
    else if (on_prefill)
        launch_moe_stage2_prefill(a2, a2s, w2, w2s.f32, w2s.e8m0, sid, sw, seid, nv, acc,
                                  acc_dtype, part, a_rows, I, H, E, topk, bm, mblocks, sh, s,
                                  est_pairs < 0 ? a_rows : est_pairs);
    else if (v2_supported(bm, I) && H % 256 == 0 && a_fits32(a_rows, I))
        launch_moe_stage2_fp8bs_v2(a2, a2s, w2, w2s.f32, w2s.e8m0, sid, sw, seid, nv, acc,
                                   acc_dtype, a_rows, I, H, E, topk, bm, mblocks, sh, s);
    else
        launch_moe_stage2_fp8bs(a2, a2s, w2, w2s.f32, w2s.e8m0, sid, sw, seid, nv, acc,
                                acc_dtype, a_rows, I, H, E, topk, bm, mblocks, sh, s);
}

namespace {

constexpr int64_t kMaxTokens = (1ll << 24) - 1;  // token id field of sorted_ids
constexpr int64_t kMaxTopk = 32;                 // slot bitmask width in sorting
constexpr int64_t kMaxExperts = 4096;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

void check_ptr(const void* p, const char* name) {
    AMD_CHECK(p != nullptr, std::string(name) + " is NULL");
    AMD_CHECK(aligned16(p), std::string(name) + " is not 16-byte aligned");
}

int64_t sorted_capacity_for(int64_t tokens, int64_t topk, int64_t E, int64_t bm) {
    return tokens * topk + E * bm - topk;
}

void check_block_m_gemm(int64_t bm, int64_t model_dim, int64_t inter_dim, int64_t tokens,
                        int64_t topk) {
    AMD_CHECK(bm == 16 || bm == 32 || bm == 64 || bm == 128,
              "block_m must be 16, 32, 64 or 128 for the fp8 blockscale GEMMs, got " +
                  std::to_string(bm));
    if (bm == 128)
        AMD_CHECK(v2_supported(bm, model_dim) && v2_supported(bm, inter_dim) &&
                      model_dim % 256 == 0,
                  "block_m 128 needs model_dim a multiple of 256 and model_dim, inter_dim <= 8192");
    if (bm == 128)
        AMD_CHECK(a_fits32(tokens, model_dim) && a_fits32(tokens * topk, inter_dim),
                  "block_m 128 needs tokens*model_dim and tokens*topk*inter_dim below 2^32 "
                  "(the 128-row kernels use 32-bit offsets); use block_m 64 or less");
}

void check_dims(int64_t model_dim, int64_t inter_dim) {
    AMD_CHECK(model_dim > 0 && model_dim % 128 == 0,
              "model_dim must be a positive multiple of 128, got " + std::to_string(model_dim));
    AMD_CHECK(inter_dim > 0 && inter_dim % 128 == 0,
              "inter_dim must be a positive multiple of 128, got " + std::to_string(inter_dim));
}

// E: the range of the routed expert ids (the global expert count under an
// expert mask). An expert-parallel share may hold fewer experts than topk
// (e.g. 4 local experts with top-8 routing); the sorted-length bound
// tokens*topk + E*block - topk needs topk <= E of the id range only.
void check_topk_experts(int64_t tokens, int64_t topk, int64_t E) {
    AMD_CHECK(tokens >= 0 && tokens <= kMaxTokens,
              "tokens must be in [0, 2^24), got " + std::to_string(tokens));
    AMD_CHECK(topk >= 1 && topk <= kMaxTopk,
              "topk must be in [1, 32], got " + std::to_string(topk));
    AMD_CHECK(E >= 1 && E <= kMaxExperts,
              "num_experts must be in [1, 4096], got " + std::to_string(E));
    AMD_CHECK(topk <= E, "topk must not exceed the number of experts the ids range over");
}

// The stage GEMMs index experts by sorted_expert_ids (local ids under a
// mask) and do not bound topk by the expert count.
void check_stage_dims(int64_t tokens, int64_t topk, int64_t E) {
    AMD_CHECK(tokens >= 0 && tokens <= kMaxTokens,
              "tokens must be in [0, 2^24), got " + std::to_string(tokens));
    AMD_CHECK(topk >= 1 && topk <= kMaxTopk,
              "topk must be in [1, 32], got " + std::to_string(topk));
    AMD_CHECK(E >= 1 && E <= kMaxExperts,
              "num_experts must be in [1, 4096], got " + std::to_string(E));
}

struct FusedLayout {
    int64_t cap, blocks;
    int64_t off_sorted_ids, off_sorted_w, off_sorted_eids, off_num_valid, off_sort_ws;
    int64_t off_a1, off_a1_scale, off_a2, off_a2_scale, off_acc, total;
    int64_t sort_ws_bytes;
    // stage-1 split-K (decode): K ranges per tile, the M-blocks its buffers
    // cover, the arrival counters (cleared by the sorting launch) and partials
    int ksplit;
    int64_t kmb, off_kcnt, kcnt_bytes, off_kpart;
};

int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// E_local: the experts this GPU holds (E_sort: the ids' range, global under
// an expert mask).
FusedLayout fused_layout(int64_t T, int64_t H, int64_t I, int64_t E_sort, int64_t E_local,
                         int64_t k, int64_t bm) {
    FusedLayout L;
    L.cap = sorted_capacity_for(T, k, E_sort, bm);
    L.blocks = ceil_div(L.cap, bm);
    // every routed M-block holds at least one of the T*k pairs
    L.kmb = std::min(L.blocks, T * k);
    // M-blocks expected at decode sizes: one per touched local expert, at most
    // the pairs routed here (an expert-parallel share gets ~E_local / E_sort of them)
    const int64_t est_blocks = std::min(ceil_div(T * k * E_local, E_sort), E_local);
    L.ksplit = T > 0 ? stream_stage1_ksplit(bm, H, I, est_blocks) : 1;
    L.sort_ws_bytes = sort_workspace_bytes(T, k, E_sort);
    int64_t o = 0;
    L.off_sorted_ids = o;  o = align256(o + L.cap * 4);
    L.off_sorted_w = o;    o = align256(o + L.cap * 4);
    L.off_sorted_eids = o; o = align256(o + L.blocks * 4);
    L.off_num_valid = o;   o = align256(o + 8);
    L.off_sort_ws = o;     o = align256(o + L.sort_ws_bytes);
    L.off_a1 = o;          o = align256(o + T * H);
    L.off_a1_scale = o;    o = align256(o + T * (H / 128) * 4);
    L.off_a2 = o;          o = align256(o + T * k * I);
    L.off_a2_scale = o;    o = align256(o + T * k * (I / 128) * 4);
    // fp32 accumulator [T, H], or per-pair bf16 rows [T*k, H] when stage 2
    // runs on the prefill kernel: room for either
    L.off_acc = o;         o = align256(o + std::max(T * H * 4, T * k * H * 2));
    L.kcnt_bytes = L.ksplit > 1 ? align256(L.kmb * (I / 128) * 4) : 0;
    L.off_kcnt = o;        o += L.kcnt_bytes;
    L.off_kpart = o;       o = align256(o + stream_ksplit_part_bytes(bm, L.kmb, I, L.ksplit));
    L.total = o;
    return L;
}

// Whether the two-launch entries run both GEMMs in one launch anyway
// (AITER_AMD_FUSED=1, a test and measurement switch). By default they keep
// two launches: measured on MI355X at MiMo dims, the one-launch layer is
// 2-4% faster at T = 2..4 and 3-20% slower at T = 1, 8, 32 (FP8 and A8W4),
// so the caller chooses it per shape (the tuned table's run_1stage) through
// the _1stage entries.
bool use_fused_layer(int64_t tokens, int64_t topk, int64_t bm, int64_t H, int64_t I) {
    (void)tokens;
    (void)topk;
    if (!stream_fused_supported(bm, H, I)) return false;
    const char* env = getenv("AITER_AMD_FUSED");
    return env && atoi(env) != 0;
}

// E: the experts this GPU holds; G: the experts the router spreads the
// tokens over (an expert-parallel share's global count; E otherwise).
int64_t default_block_m(int64_t tokens, int64_t topk, int64_t E, int64_t G, int64_t model_dim,
                        int64_t inter_dim) {
    // measured on MI355X (MiMo shape, FP8 and A8W4): 16-row blocks while experts
    // average <= 8 rows, 32 up to ~20, then 64; 128-row tiles halve the weight
    // re-reads once experts average >= 64 rows, and pay once stage 1 is at least
    // 16 rounds of 64-row workgroups (pairs * inter_dim >= 2^26: T=4096 at
    // MiMo dims). A share of a few rounds loses more to its last partial round:
    // the 32-of-256 EP share ran 64-row blocks 3.6-5.5% faster at T=2048..8192,
    // and T=2048 of the full layer 1.5% faster.
    if (G <= 0) G = E;
    const int64_t avg = G > 0 ? tokens * topk / G : 0;
    if (avg <= 8) return 16;
    if (avg <= 20) return 32;
    const int64_t pairs = G > 0 ? tokens * topk * E / G : 0;
    if (avg >= 64 && pairs * inter_dim >= (int64_t(1) << 26) && v2_supported(128, model_dim) &&
        v2_supported(128, inter_dim) && model_dim % 256 == 0 && a_fits32(tokens, model_dim) &&
        a_fits32(tokens * topk, inter_dim))
        return 128;
    return 64;
}

// Workspace of a layer run from a caller's sorted metadata: the recovered
// per-pair ids and weights, then the one-call layer's sections (its own
// sorting at its own block size; G: the experts the router spread the
// tokens over, a block-size hint).
int64_t sorted_layer_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int64_t G, int64_t k) {
    const int64_t bm = default_block_m(T, k, E, std::max(G, E), H, I);
    return 2 * align256(T * k * 4) + fused_layout(T, H, I, E, E, k, bm).total;
}

void check_e8m0(const uint8_t* p, const char* name) {
    AMD_CHECK(p != nullptr, std::string(name) + " is NULL");
    AMD_CHECK((reinterpret_cast<uintptr_t>(p) & 3u) == 0,
              std::string(name) + " is not 4-byte aligned");
}

void stage1_entry(const void* a1, const float* a1_scale, int64_t a1_scale_transposed,
                  const void* w1, WScale w1s, const int32_t* sorted_ids,
                  const float* sorted_weights, const int32_t* sorted_expert_ids,
                  const int32_t* num_valid_ids, void* a2,
                  float* a2_scale, int64_t tokens, int64_t model_dim, int64_t inter_dim,
                  int64_t num_experts, int64_t topk, int64_t block_m, int64_t max_m_blocks,
                  int64_t activation, int64_t w_shuffled, void* stream) {
    check_dims(model_dim, inter_dim);
    check_stage_dims(tokens, topk, num_experts);
    check_block_m_gemm(block_m, model_dim, inter_dim, tokens, topk);
    AMD_CHECK(activation == kActSilu || activation == kActGelu,
              "only ActivationType.Silu (0) and Gelu (1) are supported, got " +
                  std::to_string(activation));
    AMD_CHECK(max_m_blocks >= 0, "max_m_blocks must be >= 0");
    if (tokens == 0 || max_m_blocks == 0) return;
    check_ptr(a1, "a1");
    check_ptr(w1, "w1");
    check_ptr(a2, "a2");
    AMD_CHECK(a1_scale && a2_scale && sorted_ids && sorted_expert_ids && num_valid_ids,
              "a required pointer is NULL");
    const int64_t KB = model_dim / 128;
    const int64_t sa_row = a1_scale_transposed ? 1 : KB;
    const int64_t sa_kb = a1_scale_transposed ? tokens : 1;
    stage1_dispatch((const uint8_t*)a1, a1_scale, sa_row, sa_kb, (const uint8_t*)w1, w1s,
                    sorted_ids, sorted_expert_ids, num_valid_ids, (uint8_t*)a2, a2_scale, tokens,
                    model_dim, inter_dim, num_experts, topk, block_m, max_m_blocks,
                    (int)(w_shuffled != 0), (hipStream_t)stream, sorted_weights, (int)activation);
}

void stage2_entry(const void* a2, const float* a2_scale, const void* w2, WScale w2s,
                  const int32_t* sorted_ids, const float* sorted_weights,
                  const int32_t* sorted_expert_ids, const int32_t* num_valid_ids, void* out_acc,
                  int out_dtype, int64_t tokens, int64_t model_dim, int64_t inter_dim,
                  int64_t num_experts, int64_t topk, int64_t block_m, int64_t max_m_blocks,
                  int64_t w_shuffled, void* stream) {
    check_dims(model_dim, inter_dim);
    AMD_CHECK(out_dtype == DT_FP32 || out_dtype == DT_BF16 || out_dtype == DT_FP16,
              "stage-2 output dtype must be fp32, bf16 or fp16");
    check_stage_dims(tokens, topk, num_experts);
    check_block_m_gemm(block_m, model_dim, inter_dim, tokens, topk);
    AMD_CHECK(max_m_blocks >= 0, "max_m_blocks must be >= 0");
    if (tokens == 0 || max_m_blocks == 0) return;
    check_ptr(a2, "a2");
    check_ptr(w2, "w2");
    check_ptr(out_acc, "out_acc");
    // sorted_weights NULL: unit weights (the routing weights went into stage 1)
    AMD_CHECK(a2_scale && sorted_ids && sorted_expert_ids && num_valid_ids,
              "a required pointer is NULL");
    stage2_dispatch((const uint8_t*)a2, a2_scale, (const uint8_t*)w2, w2s, sorted_ids,
                    sorted_weights, sorted_expert_ids, num_valid_ids, out_acc, out_dtype,
                    tokens * topk,
                    inter_dim, model_dim, num_experts, topk, block_m, max_m_blocks,
                    (int)(w_shuffled != 0), (hipStream_t)stream);
}

// ---- launch timing of the one-call layer (measurement hooks) ----
// While enabled, the one-call entries record a HIP event on their stream
// before the first launch and after each step -- sorting (with the fused
// activation quant), the separate activation quant, stage 1, stage 2, the
// finishing pass -- for up to `cap` calls; the elapsed times between
// consecutive events are the steps' device times.
constexpr int kTimedSteps = 5;

struct LaunchTiming {
    bool on = false;
    int64_t cap = 0, calls = 0;
    std::vector<hipEvent_t> ev;   // [cap][kTimedSteps + 1]
};

static thread_local LaunchTiming g_timing;

// Records event `step` (0 = before the first launch) of the current call.
static void timing_mark(int step, hipStream_t s) {
    LaunchTiming& t = g_timing;
    if (!t.on || t.calls >= t.cap) return;
    AMD_HIP_CHECK(hipEventRecord(t.ev[t.calls * (kTimedSteps + 1) + step], s));
    if (step == kTimedSteps) ++t.calls;
}

// Whether a layer runs on direct M-blocks (no sorting launch): one token
// (each routed pair then fills its own 16-row M-block, as sorting would lay
// it out), every expert local, stage 1 on the decode kernel with one K range
// per tile and stage 2 on the one-token kernel. AITER_AMD_DIRECT=0 sorts
// anyway (tests compare the two). Measured on MI355X at MiMo dims, T=1,
// alternating on one box: FP8 50.2-50.3 -> 44.8-45.1 us, A8W4 36.9-37.1 ->
// 30.8-30.9 us with the streaming stage 2 (43.2-43.6 and 29.5-29.8 us with
// the one-token stage 2). Two or more tokens can route two pairs to one
// expert, whose weights two direct M-blocks would then stream twice; at
// T=2..8 direct M-blocks measured level or slower, so they keep the sorting
// launch.
bool direct_layer(int64_t tokens, int64_t block_m, int64_t H, int64_t I,
                  const int32_t* expert_mask, const int32_t* num_local_tokens, const void* part,
                  bool one_launch, int ksplit) {
    if (const char* env = getenv("AITER_AMD_DIRECT"))
        if (atoi(env) == 0) return false;
    return tokens == 1 && block_m == 16 && !expert_mask && !num_local_tokens && !part &&
           !one_launch && ksplit == 1 && stream_supported(16, H) && stream_supported(16, I) &&
           H % 256 == 0;
}

// Activations already quantised by the caller (fp8 [tokens, model_dim] and
// their 1x128 scales at a1_scale[row * sa_row + kb * sa_kb]) instead of
// bf16 / fp16 hidden states.
struct PreQuant {
    const uint8_t* a1 = nullptr;
    const float* a1_scale = nullptr;
    int64_t sa_row = 0, sa_kb = 0;
};

// accumulate: the layer is added to out's previous contents (rounded once
// from fp32) instead of replacing them.
void fused_entry(const void* hidden_states, int hidden_dtype, const void* w1, WScale w1s,
                 const void* w2, WScale w2s, const float* topk_weights, const int32_t* topk_ids,
                 const int32_t* expert_mask, const int32_t* num_local_tokens, void* out,
                 int out_dtype, int64_t tokens, int64_t model_dim, int64_t inter_dim,
                 int64_t num_experts, int64_t global_experts, int64_t topk, int64_t block_m,
                 int64_t activation, int64_t doweight_stage1, int64_t w_shuffled,
                 void* workspace, int64_t workspace_bytes, void* stream, bool one_launch = false,
                 PreQuant pre = PreQuant{}, bool accumulate = false) {
    check_dims(model_dim, inter_dim);
    AMD_CHECK(activation == kActSilu || activation == kActGelu,
              "only ActivationType.Silu (0) and Gelu (1) are supported, got " +
                  std::to_string(activation));
    check_stage_dims(tokens, topk, num_experts);
    if (!pre.a1)
        AMD_CHECK(hidden_dtype == DT_BF16 || hidden_dtype == DT_FP16,
                  "hidden_states dtype must be bf16 or fp16");
    AMD_CHECK(out_dtype == DT_BF16 || out_dtype == DT_FP16, "out dtype must be bf16 or fp16");
    const int64_t E_sort = expert_mask ? global_experts : num_experts;
    AMD_CHECK(E_sort >= num_experts && E_sort <= kMaxExperts,
              "global_experts must be in [num_experts, 4096]");
    check_topk_experts(tokens, topk, E_sort);
    if (block_m <= 0)
        block_m = default_block_m(tokens, topk, num_experts, E_sort, model_dim, inter_dim);
    check_block_m_gemm(block_m, model_dim, inter_dim, tokens, topk);
    AMD_CHECK(!one_launch || stream_fused_supported(block_m, model_dim, inter_dim),
              "the one-launch layer needs block_m 16 or 32 and model_dim a multiple of 256 up "
              "to 8192");
    if (tokens == 0) return;
    if (pre.a1) {
        check_ptr(pre.a1, "a1");
        AMD_CHECK(pre.a1_scale != nullptr, "a1_scale is NULL");
    } else {
        check_ptr(hidden_states, "hidden_states");
    }
    check_ptr(w1, "w1");
    check_ptr(w2, "w2");
    check_ptr(out, "out");
    AMD_CHECK(topk_weights && topk_ids, "a required pointer is NULL");
    const FusedLayout L =
        fused_layout(tokens, model_dim, inter_dim, E_sort, num_experts, topk, block_m);
    AMD_CHECK(workspace_bytes >= L.total, "workspace of " + std::to_string(L.total) +
                                              " bytes required, got " +
                                              std::to_string(workspace_bytes));
    check_ptr(workspace, "workspace");
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    int32_t* sorted_ids = reinterpret_cast<int32_t*>(ws + L.off_sorted_ids);
    float* sorted_w = reinterpret_cast<float*>(ws + L.off_sorted_w);
    int32_t* sorted_eids = reinterpret_cast<int32_t*>(ws + L.off_sorted_eids);
    int32_t* num_valid = reinterpret_cast<int32_t*>(ws + L.off_num_valid);
    uint8_t* a1 = pre.a1 ? const_cast<uint8_t*>(pre.a1) : ws + L.off_a1;
    float* a1_scale =
        pre.a1 ? const_cast<float*>(pre.a1_scale) : reinterpret_cast<float*>(ws + L.off_a1_scale);
    const int64_t sa_row = pre.a1 ? pre.sa_row : model_dim / 128;
    const int64_t sa_kb = pre.a1 ? pre.sa_kb : 1;
    uint8_t* a2 = ws + L.off_a2;
    float* a2_scale = reinterpret_cast<float*>(ws + L.off_a2_scale);
    float* acc = reinterpret_cast<float*>(ws + L.off_acc);
    // stage 2 on the prefill kernel writes each pair's weighted row once (bf16)
    // and one pass sums a token's slots: no fp32 atomics, no accumulator to clear
    // pairs expected on this GPU (the expert-parallel share of tokens * topk)
    const int64_t local_pairs = tokens * topk * num_experts / E_sort;
    uint16_t* part = stage2_on_prefill(block_m, inter_dim, model_dim, w2s, tokens * topk,
                                       num_experts, local_pairs)
                         ? reinterpret_cast<uint16_t*>(ws + L.off_acc) : nullptr;
    hipStream_t s = (hipStream_t)stream;
    timing_mark(0, s);
    const int sh = (int)(w_shuffled != 0);
    // doweight_stage1: the routing weights scale stage 1's gate and up, stage 2 sums unweighted
    const bool dw = doweight_stage1 != 0;
    const void* addend = accumulate ? out : nullptr;
    if (direct_layer(tokens, block_m, model_dim, inter_dim, expert_mask, num_local_tokens, part,
                     one_launch || use_fused_layer(tokens, topk, block_m, model_dim, inter_dim),
                     L.ksplit)) {
        // one token: each routed pair is its own 16-row M-block, so stage 1
        // reads the routing directly and quantises the token itself (no
        // sorting launch), and stage 2 sums the token's slots per workgroup
        // straight into out (no atomics, no finishing pass)
        StreamDirect d1;
        d1.ids = topk_ids;
        d1.tokens = (int)tokens;
        d1.xq = pre.a1 ? nullptr : hidden_states;
        d1.xq_dtype = (int)hidden_dtype;
        timing_mark(1, s);
        timing_mark(2, s);
        launch_moe_stage1_stream(a1, a1_scale, sa_row, sa_kb, (const uint8_t*)w1, w1s.f32,
                                 w1s.e8m0, nullptr, nullptr, nullptr, a2, a2_scale, tokens,
                                 model_dim, inter_dim, num_experts, topk, block_m, tokens * topk,
                                 sh, s, dw ? topk_weights : nullptr, (int)activation, 1, nullptr,
                                 nullptr, 0, d1);
        timing_mark(3, s);
        launch_moe_token_stage2(a2, a2_scale, (const uint8_t*)w2, w2s.f32, w2s.e8m0, topk_ids,
                                dw ? nullptr : topk_weights, out, out_dtype, addend, topk,
                                model_dim, inter_dim, num_experts, sh, s);
        timing_mark(4, s);
        timing_mark(5, s);
        return;
    }
    // decode-sized batches: the sorting launch also quantises the activations
    const bool quantised = launch_moe_sort(
        topk_ids, topk_weights, expert_mask, num_local_tokens, sorted_ids, sorted_w, sorted_eids,
        num_valid, part ? nullptr : acc, model_dim * 4, tokens, topk, E_sort, block_m,
        ws + L.off_sort_ws, L.sort_ws_bytes, s, pre.a1 ? nullptr : hidden_states,
        (int)hidden_dtype, a1, a1_scale, model_dim, ws + L.off_kcnt, L.kcnt_bytes);
    timing_mark(1, s);
    if (!quantised && !pre.a1)
        launch_per_group_quant_fp8(hidden_states, hidden_dtype, a1, a1_scale, tokens, model_dim,
                                   0, num_local_tokens, 1, s);
    timing_mark(2, s);
    if (!part && (one_launch || use_fused_layer(tokens, topk, block_m, model_dim, inter_dim))) {
        // decode sizes: both GEMMs in one launch, a2 kept per workgroup in LDS
        launch_moe_fused_stream(a1, a1_scale, sa_row, sa_kb, (const uint8_t*)w1, w1s.f32,
                                w1s.e8m0, (const uint8_t*)w2, w2s.f32, w2s.e8m0, sorted_ids,
                                dw ? sorted_w : nullptr, dw ? nullptr : sorted_w, sorted_eids,
                                num_valid, acc, tokens, model_dim, inter_dim, num_experts, topk,
                                block_m, L.blocks, sh, s, (int)activation, L.ksplit,
                                ws + L.off_kpart, reinterpret_cast<int32_t*>(ws + L.off_kcnt),
                                L.kmb);
        timing_mark(3, s);
        timing_mark(4, s);
        launch_acc_to_out(acc, out, out_dtype, num_valid, tokens, model_dim, s, addend);
        timing_mark(5, s);
        return;
    }
    stage1_dispatch(a1, a1_scale, sa_row, sa_kb, (const uint8_t*)w1, w1s, sorted_ids,
                    sorted_eids, num_valid, a2, a2_scale, tokens, model_dim, inter_dim,
                    num_experts, topk, block_m, L.blocks, sh, s, dw ? sorted_w : nullptr,
                    (int)activation, L.ksplit, ws + L.off_kpart,
                    reinterpret_cast<int32_t*>(ws + L.off_kcnt), L.kmb, local_pairs);
    timing_mark(3, s);
    stage2_dispatch(a2, a2_scale, (const uint8_t*)w2, w2s, sorted_ids, dw ? nullptr : sorted_w,
                    sorted_eids,
                    num_valid, part ? nullptr : acc, DT_FP32, tokens * topk, inter_dim, model_dim,
                    num_experts, topk, block_m, L.blocks, sh, s, part, local_pairs);
    timing_mark(4, s);
    if (part)
        launch_slot_sum(part, topk_ids, expert_mask, E_sort, num_valid, out, out_dtype, tokens,
                        topk, model_dim, s, addend);
    else
        launch_acc_to_out(acc, out, out_dtype, num_valid, tokens, model_dim, s, addend);
    timing_mark(5, s);
}

// ---- the library's own device workspace for callers that cannot allocate ----
// One copy per GPU the library runs on, held until the process ends. In host
// code `scratch` names a host-side stand-in, not device memory: the device
// address of each GPU's copy comes from hipGetSymbolAddress with that GPU
// current, and only that address is ever handed to kernels.
constexpr int64_t kScratchBytes = AITER_AMD_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// Device address of the current GPU's scratch copy, looked up on the first
// call per device and cached.
void* device_scratch() {
    int dev = -1;
    AMD_HIP_CHECK(hipGetDevice(&dev));
    AMD_CHECK(dev >= 0 && dev < kMaxDevices, "device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        AMD_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        AMD_CHECK(p != nullptr, "hipGetSymbolAddress returned NULL for the scratch buffer");
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace aiter_amd

using namespace aiter_amd;

extern "C" {

int aiter_amd_abi_version(void) { return AITER_AMD_ABI_VERSION; }

const char* aiter_amd_get_last_error(void) { return g_last_error.c_str(); }

void aiter_amd_clear_last_error(void) { g_last_error.clear(); }

// the reference's names for the same error state (aiter_ctypes_error.h:60-72):
// version 2 is its status-return convention, and no error reads as NULL
int aiter_ctypes_abi_version(void) { return 2; }

const char* aiter_get_last_error(void) {
    return g_last_error.empty() ? nullptr : g_last_error.c_str();
}

void aiter_clear_last_error(void) { g_last_error.clear(); }

int64_t aiter_amd_moe_sorting_workspace_bytes(int64_t tokens, int64_t topk, int64_t num_experts) {
    if (tokens < 0 || topk < 1 || num_experts < 1) return 0;
    return sort_workspace_bytes(tokens, topk, num_experts);
}

int aiter_amd_layer_timing_begin(int64_t max_calls) {
    return safe_call([&] {
        AMD_CHECK(max_calls >= 1 && max_calls <= 100000, "max_calls must be in [1, 100000]");
        LaunchTiming& t = g_timing;
        AMD_CHECK(!t.on, "layer timing is already on (call aiter_amd_layer_timing_end first)");
        t.ev.assign(max_calls * (kTimedSteps + 1), nullptr);
        for (auto& e : t.ev) AMD_HIP_CHECK(hipEventCreate(&e));
        t.cap = max_calls;
        t.calls = 0;
        t.on = true;
    });
}

int64_t aiter_amd_layer_timing_end(float* step_ms, int64_t max_calls) {
    LaunchTiming& t = g_timing;
    int64_t n = -1;
    const int rc = safe_call([&] {
        AMD_CHECK(t.on, "layer timing is off");
        t.on = false;
        n = std::min(t.calls, max_calls);
        if (n > 0) AMD_HIP_CHECK(hipEventSynchronize(t.ev[(n - 1) * (kTimedSteps + 1) + kTimedSteps]));
        for (int64_t c = 0; c < n; ++c)
            for (int k = 0; k < kTimedSteps; ++k) {
                float ms = 0.f;
                AMD_HIP_CHECK(hipEventElapsedTime(&ms, t.ev[c * (kTimedSteps + 1) + k],
                                                  t.ev[c * (kTimedSteps + 1) + k + 1]));
                step_ms[c * kTimedSteps + k] = ms;
            }
    });
    for (auto& e : t.ev)
        if (e) (void)hipEventDestroy(e);
    t.ev.clear();
    t.on = false;
    return rc == 0 ? n : -1;
}

int64_t aiter_amd_default_block_m(int64_t tokens, int64_t topk, int64_t num_experts,
                                  int64_t global_experts, int64_t model_dim, int64_t inter_dim) {
    return default_block_m(tokens, topk, num_experts, global_experts, model_dim, inter_dim);
}

int aiter_amd_moe_sorting_fwd(const int32_t* topk_ids, const float* topk_weights, int64_t tokens,
                              int64_t topk, int32_t* sorted_ids, float* sorted_weights,
                              int32_t* sorted_expert_ids, int32_t* num_valid_ids,
                              int64_t sorted_capacity, int64_t blocks_capacity, void* moe_buf,
                              int64_t moe_buf_row_bytes, int64_t num_experts, int64_t block_size,
                              const int32_t* expert_mask, const int32_t* num_local_tokens,
                              int64_t dispatch_policy, void* workspace, int64_t workspace_bytes,
                              void* stream) {
    (void)dispatch_policy;
    return safe_call([&] {
        check_topk_experts(tokens, topk, num_experts);
        AMD_CHECK(block_size >= 1 && block_size <= 256,
                  "block_size must be in [1, 256], got " + std::to_string(block_size));
        AMD_CHECK(topk_ids && topk_weights && sorted_ids && sorted_weights && sorted_expert_ids &&
                      num_valid_ids,
                  "a required pointer is NULL");
        const int64_t cap = sorted_capacity_for(tokens, topk, num_experts, block_size);
        AMD_CHECK(sorted_capacity >= cap, "sorted_ids capacity " +
                                              std::to_string(sorted_capacity) + " < required " +
                                              std::to_string(cap));
        AMD_CHECK(blocks_capacity >= ceil_div(cap, block_size),
                  "sorted_expert_ids capacity too small");
        if (moe_buf) {
            AMD_CHECK(aligned16(moe_buf), "moe_buf is not 16-byte aligned");
            AMD_CHECK(moe_buf_row_bytes > 0 && moe_buf_row_bytes % 16 == 0,
                      "moe_buf row bytes must be a positive multiple of 16");
        }
        const int64_t need = sort_workspace_bytes(tokens, topk, num_experts);
        AMD_CHECK(need == 0 || (workspace && workspace_bytes >= need),
                  "sorting workspace of " + std::to_string(need) + " bytes required");
        launch_moe_sort(topk_ids, topk_weights, expert_mask, num_local_tokens, sorted_ids,
                        sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf,
                        moe_buf_row_bytes, tokens, topk, num_experts, block_size, workspace,
                        workspace_bytes, (hipStream_t)stream);
    });
}

int aiter_amd_dynamic_per_group_quant_fp8(const void* input, int input_dtype, int64_t rows,
                                          int64_t cols, int64_t group_size, void* out,
                                          float* scales, int transpose_scale,
                                          const int32_t* num_rows, int64_t num_rows_factor,
                                          void* stream) {
    return safe_call([&] {
        AMD_CHECK(group_size == 128, "only group_size 128 is supported, got " +
                                         std::to_string(group_size));
        AMD_CHECK(input_dtype == DT_BF16 || input_dtype == DT_FP16,
                  "input dtype must be bf16 or fp16");
        AMD_CHECK(rows >= 0 && cols > 0 && cols % 128 == 0,
                  "cols must be a positive multiple of 128");
        AMD_CHECK(num_rows_factor >= 1, "num_rows_factor must be >= 1");
        if (rows == 0) return;
        check_ptr(input, "input");
        check_ptr(out, "out");
        AMD_CHECK(scales != nullptr, "scales is NULL");
        launch_per_group_quant_fp8(input, input_dtype, out, scales, rows, cols, transpose_scale,
                                   num_rows, num_rows_factor, (hipStream_t)stream);
    });
}

int aiter_amd_moe_stage1_fp8_blockscale(const void* a1, const float* a1_scale,
                                        int64_t a1_scale_transposed, const void* w1,
                                        const float* w1_scale, const int32_t* sorted_ids,
                                        const float* sorted_weights,
                                        const int32_t* sorted_expert_ids,
                                        const int32_t* num_valid_ids, void* a2, float* a2_scale,
                                        int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                        int64_t num_experts, int64_t topk, int64_t block_m,
                                        int64_t max_m_blocks, int64_t activation,
                                        int64_t w_shuffled, void* stream) {
    return safe_call([&] {
        AMD_CHECK(w1_scale != nullptr, "w1_scale is NULL");
        stage1_entry(a1, a1_scale, a1_scale_transposed, w1, WScale{w1_scale, nullptr}, sorted_ids,
                     sorted_weights,
                     sorted_expert_ids, num_valid_ids, a2, a2_scale, tokens, model_dim, inter_dim,
                     num_experts, topk, block_m, max_m_blocks, activation, w_shuffled, stream);
    });
}

int aiter_amd_moe_stage1_a8w4(const void* a1, const float* a1_scale, int64_t a1_scale_transposed,
                              const void* w1, const uint8_t* w1_scale,
                              const int32_t* sorted_ids,
                                        const float* sorted_weights, const int32_t* sorted_expert_ids,
                              const int32_t* num_valid_ids, void* a2, float* a2_scale,
                              int64_t tokens, int64_t model_dim, int64_t inter_dim,
                              int64_t num_experts, int64_t topk, int64_t block_m,
                              int64_t max_m_blocks, int64_t activation, int64_t w_shuffled,
                              void* stream) {
    return safe_call([&] {
        check_e8m0(w1_scale, "w1_scale");
        stage1_entry(a1, a1_scale, a1_scale_transposed, w1, WScale{nullptr, w1_scale}, sorted_ids,
                     sorted_weights,
                     sorted_expert_ids, num_valid_ids, a2, a2_scale, tokens, model_dim, inter_dim,
                     num_experts, topk, block_m, max_m_blocks, activation, w_shuffled, stream);
    });
}

int aiter_amd_moe_stage2_fp8_blockscale(const void* a2, const float* a2_scale, const void* w2,
                                        const float* w2_scale, const int32_t* sorted_ids,
                                        const float* sorted_weights,
                                        const int32_t* sorted_expert_ids,
                                        const int32_t* num_valid_ids, void* out_acc, int out_dtype,
                                        int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                        int64_t num_experts, int64_t topk, int64_t block_m,
                                        int64_t max_m_blocks, int64_t w_shuffled, void* stream) {
    return safe_call([&] {
        AMD_CHECK(w2_scale != nullptr, "w2_scale is NULL");
        stage2_entry(a2, a2_scale, w2, WScale{w2_scale, nullptr}, sorted_ids, sorted_weights,
                     sorted_expert_ids, num_valid_ids, out_acc, out_dtype, tokens, model_dim,
                     inter_dim, num_experts, topk, block_m, max_m_blocks, w_shuffled, stream);
    });
}

int aiter_amd_moe_stage2_a8w4(const void* a2, const float* a2_scale, const void* w2,
                              const uint8_t* w2_scale, const int32_t* sorted_ids,
                              const float* sorted_weights, const int32_t* sorted_expert_ids,
                              const int32_t* num_valid_ids, void* out_acc, int out_dtype, int64_t tokens,
                              int64_t model_dim, int64_t inter_dim, int64_t num_experts,
                              int64_t topk, int64_t block_m, int64_t max_m_blocks,
                              int64_t w_shuffled, void* stream) {
    return safe_call([&] {
        check_e8m0(w2_scale, "w2_scale");
        stage2_entry(a2, a2_scale, w2, WScale{nullptr, w2_scale}, sorted_ids, sorted_weights,
                     sorted_expert_ids, num_valid_ids, out_acc, out_dtype, tokens, model_dim,
                     inter_dim, num_experts, topk, block_m, max_m_blocks, w_shuffled, stream);
    });
}

int aiter_amd_moe_acc_to_out(const float* acc, void* out, int out_dtype,
                             const int32_t* num_valid_ids, int64_t tokens, int64_t model_dim,
                             void* stream) {
    return safe_call([&] {
        AMD_CHECK(out_dtype == DT_BF16 || out_dtype == DT_FP16, "out dtype must be bf16 or fp16");
        AMD_CHECK(model_dim > 0 && model_dim % 8 == 0, "model_dim must be a multiple of 8");
        AMD_CHECK(tokens >= 0, "tokens must be >= 0");
        if (tokens == 0) return;
        check_ptr(acc, "acc");
        check_ptr(out, "out");
        launch_acc_to_out(acc, out, out_dtype, num_valid_ids, tokens, model_dim,
                          (hipStream_t)stream);
    });
}

int64_t aiter_amd_fused_moe_workspace_bytes(int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                            int64_t num_experts, int64_t global_experts,
                                            int64_t topk, int64_t block_m) {
    if (tokens < 0 || model_dim <= 0 || inter_dim <= 0 || num_experts < 1 || topk < 1 ||
        global_experts < num_experts)
        return -1;
    // the block size the one-call entries resolve
    if (block_m <= 0)
        block_m = default_block_m(tokens, topk, num_experts, global_experts, model_dim, inter_dim);
    return fused_layout(tokens, model_dim, inter_dim, global_experts, num_experts, topk, block_m)
        .total;
}

int aiter_amd_fused_moe_workspace_a2_offsets(int64_t tokens, int64_t model_dim,
                                             int64_t inter_dim, int64_t num_experts,
                                             int64_t global_experts, int64_t topk,
                                             int64_t block_m, int64_t* offsets) {
    return safe_call([&] {
        AMD_CHECK(offsets != nullptr, "offsets is NULL");
        AMD_CHECK(tokens >= 0 && model_dim > 0 && inter_dim > 0 && num_experts >= 1 &&
                      topk >= 1 && global_experts >= num_experts,
                  "invalid layer dimensions");
        if (block_m <= 0)
            block_m = default_block_m(tokens, topk, num_experts, global_experts, model_dim,
                                      inter_dim);
        const FusedLayout L =
            fused_layout(tokens, model_dim, inter_dim, global_experts, num_experts, topk, block_m);
        offsets[0] = L.off_a2;
        offsets[1] = L.off_a2_scale;
    });
}

int aiter_amd_fused_moe_fp8_blockscale(const void* hidden_states, int hidden_dtype,
                                       const void* w1, const float* w1_scale, const void* w2,
                                       const float* w2_scale, const float* topk_weights,
                                       const int32_t* topk_ids, const int32_t* expert_mask,
                                       const int32_t* num_local_tokens, void* out, int out_dtype,
                                       int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                       int64_t num_experts, int64_t global_experts, int64_t topk,
                                       int64_t block_m, int64_t activation,
                                       int64_t doweight_stage1, int64_t w_shuffled, void* workspace,
                                       int64_t workspace_bytes, void* stream) {
    return safe_call([&] {
        AMD_CHECK(w1_scale && w2_scale, "a required pointer is NULL");
        fused_entry(hidden_states, hidden_dtype, w1, WScale{w1_scale, nullptr}, w2,
                    WScale{w2_scale, nullptr}, topk_weights, topk_ids, expert_mask,
                    num_local_tokens, out, out_dtype, tokens, model_dim, inter_dim, num_experts,
                    global_experts, topk, block_m, activation, doweight_stage1, w_shuffled, workspace,
                    workspace_bytes, stream);
    });
}

int aiter_amd_fused_moe_fp8_blockscale_noalloc(
    const void* hidden_states, int hidden_dtype, const void* w1, const float* w1_scale,
    const void* w2, const float* w2_scale, const float* topk_weights, const int32_t* topk_ids,
    const int32_t* expert_mask, const int32_t* num_local_tokens, void* out, int out_dtype,
    int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t num_experts,
    int64_t global_experts, int64_t topk, int64_t block_m, int64_t activation,
    int64_t doweight_stage1, int64_t w_shuffled, void* stream) {
    return safe_call([&] {
        AMD_CHECK(w1_scale && w2_scale, "a required pointer is NULL");
        check_dims(model_dim, inter_dim);
        check_stage_dims(tokens, topk, num_experts);
        const int64_t E_sort = expert_mask ? global_experts : num_experts;
        AMD_CHECK(E_sort >= num_experts && E_sort <= kMaxExperts,
                  "global_experts must be in [num_experts, 4096]");
        check_topk_experts(tokens, topk, E_sort);
        const int64_t bm = block_m > 0 ? block_m
                                       : default_block_m(tokens, topk, num_experts, E_sort,
                                                         model_dim, inter_dim);
        check_block_m_gemm(bm, model_dim, inter_dim, tokens, topk);
        const int64_t need =
            fused_layout(tokens, model_dim, inter_dim, E_sort, num_experts, topk, bm).total;
        AMD_CHECK(need <= kScratchBytes,
                  "this layer needs " + std::to_string(need) + " bytes of workspace; the "
                  "no-alloc entry point holds " + std::to_string(kScratchBytes) +
                  " (AITER_AMD_SCRATCH_BYTES): pass a workspace to "
                  "aiter_amd_fused_moe_fp8_blockscale instead");
        if (tokens == 0) return;
        // the stream must belong to the current device, whose scratch copy is used
        if (stream) {
            hipDevice_t sdev;
            int cur = -1;
            AMD_HIP_CHECK(hipStreamGetDevice((hipStream_t)stream, &sdev));
            AMD_HIP_CHECK(hipGetDevice(&cur));
            AMD_CHECK((int)sdev == cur, "stream belongs to device " + std::to_string(sdev) +
                                            ", the current device is " + std::to_string(cur));
        }
        // every section the layer reads before writing (the f32 accumulator)
        // is cleared by the sorting launch on each call, so a previous call's
        // contents never leak into this one
        fused_entry(hidden_states, hidden_dtype, w1, WScale{w1_scale, nullptr}, w2,
                    WScale{w2_scale, nullptr}, topk_weights, topk_ids, expert_mask,
                    num_local_tokens, out, out_dtype, tokens, model_dim, inter_dim, num_experts,
                    global_experts, topk, bm, activation, doweight_stage1, w_shuffled,
                    device_scratch(), kScratchBytes, stream);
    });
}

int aiter_amd_fused_moe_a8w4(const void* hidden_states, int hidden_dtype, const void* w1,
                             const uint8_t* w1_scale, const void* w2, const uint8_t* w2_scale,
                             const float* topk_weights, const int32_t* topk_ids,
                             const int32_t* expert_mask, const int32_t* num_local_tokens,
                             void* out, int out_dtype, int64_t tokens, int64_t model_dim,
                             int64_t inter_dim, int64_t num_experts, int64_t global_experts,
                             int64_t topk, int64_t block_m, int64_t activation,
                             int64_t doweight_stage1, int64_t w_shuffled, void* workspace,
                             int64_t workspace_bytes, void* stream) {
    return safe_call([&] {
        check_e8m0(w1_scale, "w1_scale");
        check_e8m0(w2_scale, "w2_scale");
        fused_entry(hidden_states, hidden_dtype, w1, WScale{nullptr, w1_scale}, w2,
                    WScale{nullptr, w2_scale}, topk_weights, topk_ids, expert_mask,
                    num_local_tokens, out, out_dtype, tokens, model_dim, inter_dim, num_experts,
                    global_experts, topk, block_m, activation, doweight_stage1, w_shuffled, workspace,
                    workspace_bytes, stream);
    });
}

int aiter_amd_fused_moe_1stage_fp8_blockscale(
    const void* hidden_states, int hidden_dtype, const void* w1, const float* w1_scale,
    const void* w2, const float* w2_scale, const float* topk_weights, const int32_t* topk_ids,
    const int32_t* expert_mask, const int32_t* num_local_tokens, void* out, int out_dtype,
    int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t num_experts,
    int64_t global_experts, int64_t topk, int64_t block_m, int64_t activation,
    int64_t doweight_stage1, int64_t w_shuffled, void* workspace, int64_t workspace_bytes,
    void* stream) {
    return safe_call([&] {
        AMD_CHECK(w1_scale && w2_scale, "a required pointer is NULL");
        fused_entry(hidden_states, hidden_dtype, w1, WScale{w1_scale, nullptr}, w2,
                    WScale{w2_scale, nullptr}, topk_weights, topk_ids, expert_mask,
                    num_local_tokens, out, out_dtype, tokens, model_dim, inter_dim, num_experts,
                    global_experts, topk, block_m, activation, doweight_stage1, w_shuffled, workspace,
                    workspace_bytes, stream, true);
    });
}

int aiter_amd_fused_moe_1stage_a8w4(
    const void* hidden_states, int hidden_dtype, const void* w1, const uint8_t* w1_scale,
    const void* w2, const uint8_t* w2_scale, const float* topk_weights, const int32_t* topk_ids,
    const int32_t* expert_mask, const int32_t* num_local_tokens, void* out, int out_dtype,
    int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t num_experts,
    int64_t global_experts, int64_t topk, int64_t block_m, int64_t activation,
    int64_t doweight_stage1, int64_t w_shuffled, void* workspace, int64_t workspace_bytes,
    void* stream) {
    return safe_call([&] {
        check_e8m0(w1_scale, "w1_scale");
        check_e8m0(w2_scale, "w2_scale");
        fused_entry(hidden_states, hidden_dtype, w1, WScale{nullptr, w1_scale}, w2,
                    WScale{nullptr, w2_scale}, topk_weights, topk_ids, expert_mask,
                    num_local_tokens, out, out_dtype, tokens, model_dim, inter_dim, num_experts,
                    global_experts, topk, block_m, activation, doweight_stage1, w_shuffled, workspace,
                    workspace_bytes, stream, true);
    });
}

int aiter_amd_moe_stage1_rows(const void* a1, const float* a1_scale, int64_t a1_scale_transposed,
                              const void* w1, const float* w1_scale,
                              const uint8_t* w1_scale_e8m0, const int32_t* sorted_ids,
                              const float* sorted_weights, const int32_t* sorted_expert_ids,
                              const int32_t* num_valid_ids, void* out, int out_form,
                              int out_dtype, int64_t tokens, int64_t model_dim,
                              int64_t inter_dim, int64_t num_experts, int64_t topk,
                              int64_t block_m, int64_t max_m_blocks, int64_t activation,
                              int64_t ksplit, int64_t w_shuffled, void* stream) {
    return safe_call([&] {
        check_dims(model_dim, inter_dim);
        check_stage_dims(tokens, topk, num_experts);
        AMD_CHECK(out_form == kOutAct || out_form == kOutGateUp,
                  "out_form must be 1 (act(gate) * up rows) or 2 (fp32 gate | up rows)");
        AMD_CHECK(out_form == kOutGateUp ? out_dtype == DT_FP32
                                         : (out_dtype == DT_BF16 || out_dtype == DT_FP16 ||
                                            out_dtype == DT_FP32),
                  out_form == kOutGateUp ? "gate | up rows are fp32"
                                         : "act rows must be bf16, fp16 or fp32");
        AMD_CHECK(block_m == 16 || block_m == 32 || block_m == 64 || block_m == 128,
                  "block_m must be 16, 32, 64 or 128, got " + std::to_string(block_m));
        AMD_CHECK(model_dim <= 8192, "model_dim must be at most 8192");
        AMD_CHECK(activation == kActSilu || activation == kActGelu,
                  "only ActivationType.Silu (0) and Gelu (1) are supported, got " +
                      std::to_string(activation));
        AMD_CHECK((w1_scale != nullptr) != (w1_scale_e8m0 != nullptr),
                  "exactly one of w1_scale (fp8 weights) and w1_scale_e8m0 (MXFP4) is given");
        const int64_t KB = model_dim / 128;
        AMD_CHECK(ksplit >= 0 && ksplit <= KB && (ksplit <= 1 || KB % ksplit == 0),
                  "ksplit must divide model_dim / 128 = " + std::to_string(KB) + ", got " +
                      std::to_string(ksplit));
        AMD_CHECK(ksplit <= 1 || out_form == kOutGateUp,
                  "a K split (ksplit > 1) writes fp32 gate | up rows (out_form 2)");
        AMD_CHECK(max_m_blocks >= 0, "max_m_blocks must be >= 0");
        if (w1_scale_e8m0) check_e8m0(w1_scale_e8m0, "w1_scale");
        if (tokens == 0 || max_m_blocks == 0) return;
        check_ptr(a1, "a1");
        check_ptr(w1, "w1");
        check_ptr(out, "out");
        AMD_CHECK(a1_scale && sorted_ids && sorted_expert_ids && num_valid_ids,
                  "a required pointer is NULL");
        hipStream_t s = (hipStream_t)stream;
        // the K ranges of a split tile add into zeroed rows
        if (ksplit > 1) launch_zero(out, tokens * topk * 2 * inter_dim * 4, s);
        launch_moe_stage1_stream_rows(
            (const uint8_t*)a1, a1_scale, a1_scale_transposed ? 1 : model_dim / 128,
            a1_scale_transposed ? tokens : 1, (const uint8_t*)w1, w1_scale, w1_scale_e8m0,
            sorted_ids, sorted_expert_ids, num_valid_ids, out, out_form, out_dtype, tokens,
            model_dim, inter_dim, num_experts, topk, block_m, max_m_blocks,
            (int)(w_shuffled != 0), s, sorted_weights, (int)activation, (int)ksplit);
    });
}

int aiter_amd_act_and_mul(const void* input, int input_dtype, void* out, int out_dtype,
                          int64_t rows, int64_t d, int64_t activation, void* stream) {
    return safe_call([&] {
        AMD_CHECK(input_dtype == DT_FP32 || input_dtype == DT_BF16 || input_dtype == DT_FP16,
                  "input dtype must be fp32, bf16 or fp16");
        AMD_CHECK(out_dtype == DT_FP32 || out_dtype == DT_BF16 || out_dtype == DT_FP16,
                  "out dtype must be fp32, bf16 or fp16");
        AMD_CHECK(activation == kActSilu || activation == kActGelu,
                  "only ActivationType.Silu (0) and Gelu (1) are supported, got " +
                      std::to_string(activation));
        AMD_CHECK(rows >= 0 && d >= 0, "rows and d must be >= 0");
        AMD_CHECK(rows * d < (int64_t(1) << 40), "too many elements");
        AMD_CHECK(d < (int64_t(1) << 31), "d must be below 2^31");
        if (rows == 0 || d == 0) return;
        AMD_CHECK(input && out, "a required pointer is NULL");
        launch_act_and_mul(input, input_dtype, out, out_dtype, rows, d, (int)activation,
                           (hipStream_t)stream);
    });
}

int64_t aiter_amd_fused_moe_sorted_workspace_bytes(int64_t tokens, int64_t model_dim,
                                                   int64_t inter_dim, int64_t num_experts,
                                                   int64_t global_experts, int64_t topk) {
    if (tokens < 0 || model_dim <= 0 || inter_dim <= 0 || num_experts < 1 || topk < 1)
        return -1;
    return sorted_layer_bytes(tokens, model_dim, inter_dim, num_experts, global_experts, topk);
}

int aiter_amd_fused_moe_sorted_fp8_blockscale(
    const void* a1, const float* a1_scale, int64_t a1_scale_transposed, const void* w1,
    const float* w1_scale, const void* w2, const float* w2_scale, const int32_t* sorted_ids,
    const float* sorted_weights, const int32_t* sorted_expert_ids, const int32_t* num_valid_ids,
    int64_t sorted_capacity, int64_t sorted_block_m, void* out, int out_dtype, int64_t tokens,
    int64_t model_dim, int64_t inter_dim, int64_t num_experts, int64_t global_experts,
    int64_t topk, int64_t activation, int64_t w_shuffled, void* workspace,
    int64_t workspace_bytes, void* stream) {
    return safe_call([&] {
        AMD_CHECK(w1_scale && w2_scale, "a required pointer is NULL");
        check_dims(model_dim, inter_dim);
        check_stage_dims(tokens, topk, num_experts);
        AMD_CHECK(out_dtype == DT_BF16 || out_dtype == DT_FP16, "out dtype must be bf16 or fp16");
        AMD_CHECK(sorted_block_m >= 1 && sorted_block_m <= 256,
                  "sorted_block_m must be in [1, 256]");
        AMD_CHECK(sorted_capacity >= 0, "sorted_capacity must be >= 0");
        const int64_t need = sorted_layer_bytes(tokens, model_dim, inter_dim, num_experts,
                                                global_experts, topk);
        AMD_CHECK(workspace_bytes >= need, "workspace of " + std::to_string(need) +
                                               " bytes required, got " +
                                               std::to_string(workspace_bytes));
        if (tokens == 0) return;
        check_ptr(workspace, "workspace");
        AMD_CHECK(sorted_ids && sorted_weights && sorted_expert_ids && num_valid_ids,
                  "a required pointer is NULL");
        hipStream_t s = (hipStream_t)stream;
        uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
        int32_t* ids = reinterpret_cast<int32_t*>(ws);
        float* wts = reinterpret_cast<float*>(ws + align256(tokens * topk * 4));
        const int64_t off = 2 * align256(tokens * topk * 4);
        // the pairs routed to these experts, recovered from the caller's sorting
        launch_unsort(sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids,
                      sorted_capacity, sorted_block_m, ids, wts, tokens, topk, num_experts, s);
        const int64_t G = std::max(global_experts, num_experts);
        const int64_t bm =
            default_block_m(tokens, topk, num_experts, G, model_dim, inter_dim);
        PreQuant pre;
        pre.a1 = (const uint8_t*)a1;
        pre.a1_scale = a1_scale;
        pre.sa_row = a1_scale_transposed ? 1 : model_dim / 128;
        pre.sa_kb = a1_scale_transposed ? tokens : 1;
        // the caller's token count (num_valid_ids[1]) bounds the rows; the
        // layer is added to out, which the caller's sorting zeroed
        fused_entry(nullptr, DT_FP8, w1, WScale{w1_scale, nullptr}, w2, WScale{w2_scale, nullptr},
                    wts, ids, nullptr, num_valid_ids + 1, out, out_dtype, tokens, model_dim,
                    inter_dim, num_experts, num_experts, topk, bm, activation, 0, w_shuffled,
                    ws + off, workspace_bytes - off, stream, false, pre, true);
    });
}

static void check_route(const void* gating, int dtype, int64_t tokens, int64_t E, int64_t topk,
                        const float* w, int64_t ws, const int32_t* ids, int64_t is) {
    AMD_CHECK(dtype == DT_FP32 || dtype == DT_BF16 || dtype == DT_FP16,
              "gating dtype must be fp32, bf16 or fp16");
    AMD_CHECK(tokens >= 0, "tokens must be >= 0");
    AMD_CHECK(route_supported(E, topk), "need 1 <= topk <= min(num_experts, 32) and "
                                        "num_experts <= 1024, got topk " + std::to_string(topk) +
                                        ", num_experts " + std::to_string(E));
    AMD_CHECK(ws >= topk && is >= topk, "output row strides must be >= topk");
    if (tokens == 0) return;
    AMD_CHECK(gating && w && ids, "a required pointer is NULL");
}

int aiter_amd_topk_softmax(const void* gating, int gating_dtype, int64_t tokens,
                           int64_t num_experts, int64_t topk, float* topk_weights,
                           int64_t weights_stride, int32_t* topk_ids, int64_t ids_stride,
                           int32_t* token_expert_indices, int need_renorm, void* stream) {
    return safe_call([&] {
        check_route(gating, gating_dtype, tokens, num_experts, topk, topk_weights,
                    weights_stride, topk_ids, ids_stride);
        if (tokens == 0) return;
        launch_moe_route(gating, gating_dtype, tokens, num_experts, topk, 0, need_renorm != 0, 0,
                         1, 1, 1.0f, nullptr, topk_weights, weights_stride, topk_ids, ids_stride,
                         token_expert_indices, (hipStream_t)stream);
    });
}

int aiter_amd_topk_softmax_shared(const void* gating, int gating_dtype, int64_t tokens,
                                  int64_t num_experts, int64_t num_shared_experts,
                                  int64_t topk, float* topk_weights, int64_t weights_stride,
                                  int32_t* topk_ids, int64_t ids_stride,
                                  int32_t* token_expert_indices, int need_renorm,
                                  void* stream) {
    return safe_call([&] {
        AMD_CHECK(num_shared_experts >= 0 && num_shared_experts <= kMaxExperts,
                  "num_shared_experts must be in [0, " + std::to_string(kMaxExperts) + "]");
        check_route(gating, gating_dtype, tokens, num_experts, topk, topk_weights,
                    weights_stride, topk_ids, ids_stride);
        AMD_CHECK(weights_stride >= topk + num_shared_experts,
                  "topk_weights rows must hold topk + num_shared_experts weights");
        if (tokens == 0) return;
        launch_moe_route(gating, gating_dtype, tokens, num_experts, topk, 0, need_renorm != 0, 0,
                         1, 1, 1.0f, nullptr, topk_weights, weights_stride, topk_ids, ids_stride,
                         token_expert_indices, (hipStream_t)stream,
                         num_experts + num_shared_experts, num_shared_experts);
    });
}

int aiter_amd_topk_sigmoid(const void* gating, int gating_dtype, int64_t tokens,
                           int64_t num_experts, int64_t topk, float* topk_weights,
                           int64_t weights_stride, int32_t* topk_ids, int64_t ids_stride,
                           void* stream) {
    return safe_call([&] {
        check_route(gating, gating_dtype, tokens, num_experts, topk, topk_weights,
                    weights_stride, topk_ids, ids_stride);
        if (tokens == 0) return;
        launch_moe_route(gating, gating_dtype, tokens, num_experts, topk, 1, 0, 0, 1, 1, 1.0f,
                         nullptr, topk_weights, weights_stride, topk_ids, ids_stride, nullptr,
                         (hipStream_t)stream);
    });
}

int aiter_amd_grouped_topk(const void* gating, int gating_dtype, const float* correction_bias,
                           int64_t tokens, int64_t num_experts, int64_t topk,
                           int64_t num_expert_group, int64_t topk_group, int need_renorm,
                           int is_softmax, float routed_scaling_factor, float* topk_weights,
                           int64_t weights_stride, int32_t* topk_ids, int64_t ids_stride,
                           void* stream) {
    return safe_call([&] {
        check_route(gating, gating_dtype, tokens, num_experts, topk, topk_weights,
                    weights_stride, topk_ids, ids_stride);
        AMD_CHECK(num_expert_group >= 1 && num_expert_group <= 32 &&
                      num_experts % num_expert_group == 0,
                  "num_expert_group must divide num_experts and be <= 32");
        AMD_CHECK(topk_group >= 1 && topk_group <= num_expert_group,
                  "topk_group must be in [1, num_expert_group]");
        const int64_t per = num_experts / num_expert_group;
        AMD_CHECK(topk <= topk_group * per, "topk exceeds the experts of the kept groups");
        if (correction_bias) {
            AMD_CHECK(!is_softmax, "biased grouped top-k uses sigmoid scores");
            AMD_CHECK(per >= 2, "biased grouped top-k needs >= 2 experts per group");
        }
        if (tokens == 0) return;
        launch_moe_route(gating, gating_dtype, tokens, num_experts, topk,
                         correction_bias ? 3 : 2, need_renorm != 0, is_softmax != 0,
                         num_expert_group, topk_group, routed_scaling_factor, correction_bias,
                         topk_weights, weights_stride, topk_ids, ids_stride, nullptr,
                         (hipStream_t)stream);
    });
}

}  // extern "C"
