/*
 * aiter_amd — C ABI of the MI355X (gfx950) blockscale fused-MoE library.
 *
 * Conventions (mirroring the reference's ctypes bridge,
 * csrc/include/aiter_ctypes_error.h:60-147 and aiter/jit/core.py:1105-1363):
 *   - every compute entry point returns 0 on success, -1 on failure; the
 *     failure text is read with aiter_amd_get_last_error() (per thread);
 *   - every buffer is caller-owned device memory passed as a plain pointer;
 *     the library never allocates or frees device memory;
 *   - `stream` is a hipStream_t (torch's current stream in the Python layer)
 *     and is always the last argument; no entry point synchronises the host;
 *   - all argument validation happens before any device work, so invalid
 *     calls fail without touching the GPU;
 *   - dtype codes are AiterDtype values (csrc/include/aiter_enum.h:27-43):
 *     fp8 = 0, fp16 = 2, bf16 = 3, fp32 = 4.
 * fp8 means OCP e4m3fn (torch.float8_e4m3fn), the gfx950 fp8 format.
 */
#ifndef AITER_AMD_H
#define AITER_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Raised whenever an entry point's arguments change: 2 added sorted_weights
   to the stage-1 entries and activation / doweight_stage1 to the one-call
   entries; 3 the output dtype of the stage-2 entries and global_experts of
   the workspace query. */
#define AITER_AMD_ABI_VERSION 3

/* Replaces aiter_ctypes_abi_version (aiter_ctypes_error.h:120-147). */
int aiter_amd_abi_version(void);
/* Replaces aiter_get_last_error / aiter_clear_last_error
 * (aiter_ctypes_error.h:60-118, read by aiter/jit/core.py:1341-1355). */
const char* aiter_amd_get_last_error(void);
void aiter_amd_clear_last_error(void);

/* Bytes of device workspace aiter_amd_moe_sorting_fwd needs for `tokens`
 * rows of topk_ids (0 when the one-launch path is taken).  Plays the role
 * of moe_sorting_get_workspace_size (csrc/include/moe_sorting_opus.h:1351-1379). */
int64_t aiter_amd_moe_sorting_workspace_bytes(int64_t tokens, int64_t topk,
                                              int64_t num_experts);

/* Replaces moe_sorting_fwd (csrc/py_itfs_ck/moe_sorting_kernels.cu:10-70)
 * and moe_sorting_opus_fwd (csrc/py_itfs_cu/moe_sorting_opus_kernels.cu:31-92).
 *   topk_ids [tokens, topk] i32, topk_weights [tokens, topk] f32
 *   sorted_ids / sorted_weights: capacity >= tokens*topk + E*block_size - topk
 *   sorted_expert_ids: capacity >= ceil(that / block_size); num_valid_ids [2]
 *   moe_buf: optional, cleared for the first `tokens` (or *num_local_tokens)
 *   rows of moe_buf_row_bytes bytes (a multiple of 16)
 *   expert_mask [num_experts] i32 or NULL; num_local_tokens: device i32[1] or NULL
 *   dispatch_policy is accepted for interface parity and ignored (every
 *   policy yields the same output). */
int aiter_amd_moe_sorting_fwd(const int32_t* topk_ids, const float* topk_weights,
                              int64_t tokens, int64_t topk, int32_t* sorted_ids,
                              float* sorted_weights, int32_t* sorted_expert_ids,
                              int32_t* num_valid_ids, int64_t sorted_capacity,
                              int64_t blocks_capacity, void* moe_buf,
                              int64_t moe_buf_row_bytes, int64_t num_experts,
                              int64_t block_size, const int32_t* expert_mask,
                              const int32_t* num_local_tokens, int64_t dispatch_policy,
                              void* workspace, int64_t workspace_bytes, void* stream);

/* Replaces dynamic_per_token_scaled_quant for 1x128 groups
 * (csrc/kernels/quant_kernels.cu:710-757, kernel 16-133), as called by
 * per_group_quant_hip (aiter/ops/quant.py:260-292).
 *   input [rows, cols] bf16/fp16 -> out [rows, cols] fp8, scales f32
 *   [rows, cols/128] (or [cols/128, rows] when transpose_scale != 0).
 *   group_size must be 128; num_rows: device i32[1] or NULL. */
int aiter_amd_dynamic_per_group_quant_fp8(const void* input, int input_dtype, int64_t rows,
                                          int64_t cols, int64_t group_size, void* out,
                                          float* scales, int transpose_scale,
                                          const int32_t* num_rows, int64_t num_rows_factor,
                                          void* stream);

/* Replaces ck_moe_stage1 with per_1x128 fp8 (gemm_moe_ck2stages.cu:46-116)
 * plus the a2 requant (aiter/fused_moe.py:1306-1314); the fused fp8-out
 * form matches moe_stage1_g1u1 blockscale (asm_moe_2stage.cu:148-280).
 *   a1 [tokens, model_dim] fp8, a1_scale f32 [tokens, model_dim/128]
 *   (or [model_dim/128, tokens] when a1_scale_transposed != 0)
 *   w1 [E, 2*inter_dim, model_dim] fp8, w1_scale [E, 2*inter_dim/128, model_dim/128]
 *   a2 [tokens, topk, inter_dim] fp8, a2_scale [tokens, topk, inter_dim/128]
 *   activation: 0 Silu or 1 Gelu (torch's exact erf form), applied to gate
 *   (aiter/ops/quant.py:398-404); w_shuffled: 1 for the (16,16) layout.
 *   sorted_weights: NULL, or the sorted routing weights for doweight_stage1
 *   (they scale gate and up before the activation, aiter/fused_moe.py:
 *   1568-1571; fused_moe_2stages passes them to stage 1 and none to stage 2,
 *   fused_moe.py:1253, 1330).
 *   block_m in {16, 32, 64, 128}; max_m_blocks = capacity of sorted_expert_ids. */
int aiter_amd_moe_stage1_fp8_blockscale(const void* a1, const float* a1_scale,
                                        int64_t a1_scale_transposed, const void* w1,
                                        const float* w1_scale, const int32_t* sorted_ids,
                                        const float* sorted_weights,
                                        const int32_t* sorted_expert_ids,
                                        const int32_t* num_valid_ids, void* a2, float* a2_scale,
                                        int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                        int64_t num_experts, int64_t topk, int64_t block_m,
                                        int64_t max_m_blocks, int64_t activation,
                                        int64_t w_shuffled, void* stream);

/* Replaces ck_moe_stage2 with per_1x128 fp8 (gemm_moe_ck2stages.cu:118-181).
 *   a2 [tokens, topk, inter_dim] fp8 + a2_scale [tokens, topk, inter_dim/128]
 *   w2 [E, model_dim, inter_dim] fp8, w2_scale [E, model_dim/128, inter_dim/128]
 *   out_acc [tokens, model_dim] accumulates sorted_weight * row with atomics;
 *   it must be zeroed first, e.g. by aiter_amd_moe_sorting_fwd's moe_buf.
 *   out_dtype 4 (fp32) keeps the sum in fp32 (aiter_amd_moe_acc_to_out then
 *   rounds once); 3 (bf16) or 2 (fp16) accumulate into the reference's
 *   moe_buf itself, rounding after every add as its 16-bit atomics do.
 *   sorted_weights NULL: unit weights (doweight_stage1 applied them). */
int aiter_amd_moe_stage2_fp8_blockscale(const void* a2, const float* a2_scale, const void* w2,
                                        const float* w2_scale, const int32_t* sorted_ids,
                                        const float* sorted_weights,
                                        const int32_t* sorted_expert_ids,
                                        const int32_t* num_valid_ids, void* out_acc,
                                        int out_dtype,
                                        int64_t tokens, int64_t model_dim, int64_t inter_dim,
                                        int64_t num_experts, int64_t topk, int64_t block_m,
                                        int64_t max_m_blocks, int64_t w_shuffled, void* stream);

/* A8W4 stage 1: fp8 1x128 activations x MXFP4 weights.  Replaces the per_1x32
 * fp4x2-weight stage 1 (cktile_moe_stage1, aiter/ops/moe_op.py:343-464 ->
 * csrc/ck_tile_gemm_moe_2stages/moe_cktile2stages.cu:316-345), with the
 * activations quantised 1x128 as for aiter_amd_moe_stage1_fp8_blockscale
 * (the reference's fp8-activation A8W4 branch casts them with unit e8m0
 * scales, aiter/fused_moe.py:1167-1177).
 *   w1 [E, 2*inter_dim, model_dim/2] packed e2m1 (even K in the low nibble),
 *   row-major or (16,16)-shuffled on the byte view (w_shuffled);
 *   w1_scale [E, 2*inter_dim, model_dim/32] e8m0 bytes (4-byte aligned).
 *   Everything else as aiter_amd_moe_stage1_fp8_blockscale. */
int aiter_amd_moe_stage1_a8w4(const void* a1, const float* a1_scale, int64_t a1_scale_transposed,
                              const void* w1, const uint8_t* w1_scale,
                              const int32_t* sorted_ids, const float* sorted_weights,
                              const int32_t* sorted_expert_ids,
                              const int32_t* num_valid_ids, void* a2, float* a2_scale,
                              int64_t tokens, int64_t model_dim, int64_t inter_dim,
                              int64_t num_experts, int64_t topk, int64_t block_m,
                              int64_t max_m_blocks, int64_t activation, int64_t w_shuffled,
                              void* stream);

/* A8W4 stage 2: replaces the per_1x32 fp4x2-weight stage 2 (cktile_moe_stage2,
 * aiter/ops/moe_op.py:343-464 -> moe_cktile2stages.cu:444-475).
 *   w2 [E, model_dim, inter_dim/2] packed e2m1, w2_scale [E, model_dim, inter_dim/32]
 *   e8m0 bytes; everything else as aiter_amd_moe_stage2_fp8_blockscale. */
int aiter_amd_moe_stage2_a8w4(const void* a2, const float* a2_scale, const void* w2,
                              const uint8_t* w2_scale, const int32_t* sorted_ids,
                              const float* sorted_weights, const int32_t* sorted_expert_ids,
                              const int32_t* num_valid_ids, void* out_acc, int out_dtype,
                              int64_t tokens,
                              int64_t model_dim, int64_t inter_dim, int64_t num_experts,
                              int64_t topk, int64_t block_m, int64_t max_m_blocks,
                              int64_t w_shuffled, void* stream);

/* Replaces ck_moe_stage1 (aiter/ops/moe_op.py:295-316 ->
 * csrc/ck_gemm_moe_2stages_codegen/gemm_moe_ck2stages.cu:46-116) as the
 * reference's ck_moe_stage1 wrapper calls it (aiter/fused_moe.py:1669-1725):
 * stage 1 without the fused requant.
 *   a1 [tokens, model_dim] fp8 with 1x128 scales (row-major [tokens,
 *   model_dim/128], or [model_dim/128, tokens] when a1_scale_transposed);
 *   w1 fp8 [E, 2*inter_dim, model_dim] with w1_scale f32 [E, 2*inter_dim/128,
 *   model_dim/128], or MXFP4 as aiter_amd_moe_stage1_a8w4 with
 *   w1_scale_e8m0 [E, 2*inter_dim, model_dim/32] (exactly one scale given).
 *   out_form 1: out [tokens*topk, inter_dim] rows t*topk+slot of
 *   act(gate) * up in out_dtype (bf16, fp16 or fp32), rounded once;
 *   out_form 2: out [>= tokens*topk, 2*inter_dim] fp32 rows of gate | up
 *   before the activation (the reference's splitk > 1 output, which
 *   silu_and_mul / gelu_and_mul finish); ksplit > 1 (out_form 2 only, a
 *   divisor of model_dim/128) splits each tile's K range that many ways,
 *   whose partial sums are added into the rows, which the call zeroes first.
 *   Pairs not routed here leave their rows unwritten (out_form 1; out_form 2
 *   with ksplit > 1 leaves them zero).
 *   block_m in {16, 32, 64, 128}; sorted_weights, activation, w_shuffled,
 *   max_m_blocks as aiter_amd_moe_stage1_fp8_blockscale; model_dim <= 8192. */
int aiter_amd_moe_stage1_rows(const void* a1, const float* a1_scale, int64_t a1_scale_transposed,
                              const void* w1, const float* w1_scale,
                              const uint8_t* w1_scale_e8m0, const int32_t* sorted_ids,
                              const float* sorted_weights, const int32_t* sorted_expert_ids,
                              const int32_t* num_valid_ids, void* out, int out_form,
                              int out_dtype, int64_t tokens, int64_t model_dim,
                              int64_t inter_dim, int64_t num_experts, int64_t topk,
                              int64_t block_m, int64_t max_m_blocks, int64_t activation,
                              int64_t ksplit, int64_t w_shuffled, void* stream);

/* Replaces silu_and_mul / gelu_and_mul (aiter/ops/activation.py:10-19,
 * csrc/kernels/activation_kernels.cu:24-90, 337-354):
 * out[r, c] = act(input[r, c]) * input[r, d + c] for rows r < rows and
 * c < d, input rows 2*d wide (fp32, bf16 or fp16), out rows d wide (fp32,
 * bf16 or fp16), both contiguous; computed in fp32, rounded once.
 * activation 0 Silu, 1 Gelu (exact erf). */
int aiter_amd_act_and_mul(const void* input, int input_dtype, void* out, int out_dtype,
                          int64_t rows, int64_t d, int64_t activation, void* stream);

/* Bytes of workspace for aiter_amd_fused_moe_sorted_fp8_blockscale. */
int64_t aiter_amd_fused_moe_sorted_workspace_bytes(int64_t tokens, int64_t model_dim,
                                                   int64_t inter_dim, int64_t num_experts,
                                                   int64_t global_experts, int64_t topk);

/* The whole FP8 blockscale layer from a caller's sorted metadata and
 * quantised activations, added into out: the work of fmoe_fp8_blockscale_g1u1
 * (aiter/ops/moe_op.py:172-192, csrc/py_itfs_cu/asm_fmoe.cu:858-922) as
 * fused_moe_1stage calls it (aiter/fused_moe.py:367-511).
 *   a1 [tokens, model_dim] fp8, a1_scale as aiter_amd_moe_stage1_rows
 *   (fused_moe_1stage passes them transposed); w1/w1_scale/w2/w2_scale as
 *   the stage calls; sorted_ids / sorted_weights (sorted_capacity entries),
 *   sorted_expert_ids and num_valid_ids as moe_sorting made them at
 *   sorted_block_m, for num_experts experts (local ids under an expert mask);
 *   global_experts: the experts the router spread the tokens over (a
 *   block-size hint; num_experts when unknown).
 *   out [tokens, model_dim] bf16/fp16: the layer is added to it (once, in
 *   fp32, then rounded) for the first num_valid_ids[1] rows; the reference's
 *   moe_buf arrives zeroed by moe_sorting.
 *   The pairs are read back from the sorted entries and sorted again at the
 *   block size this library picks for the shape, so the layer runs on the
 *   same kernels as aiter_amd_fused_moe_fp8_blockscale (two GEMM launches),
 *   whatever block size the caller sorted at. */
int aiter_amd_fused_moe_sorted_fp8_blockscale(
    const void* a1, const float* a1_scale, int64_t a1_scale_transposed, const void* w1,
    const float* w1_scale, const void* w2, const float* w2_scale, const int32_t* sorted_ids,
    const float* sorted_weights, const int32_t* sorted_expert_ids, const int32_t* num_valid_ids,
    int64_t sorted_capacity, int64_t sorted_block_m, void* out, int out_dtype, int64_t tokens,
    int64_t model_dim, int64_t inter_dim, int64_t num_experts, int64_t global_experts,
    int64_t topk, int64_t activation, int64_t w_shuffled, void* workspace,
    int64_t workspace_bytes, void* stream);

/* Converts the stage-2 f32 accumulator into moe_buf (bf16 or fp16) for the
 * first num_valid_ids[1] rows.  The reference accumulates into moe_buf
 * directly (gemm_moe_ck2stages.cu:118-181); this is the finishing pass of the
 * f32-accumulating design. */
int aiter_amd_moe_acc_to_out(const float* acc, void* out, int out_dtype,
                             const int32_t* num_valid_ids, int64_t tokens, int64_t model_dim,
                             void* stream);

/* Bytes of workspace for aiter_amd_fused_moe_fp8_blockscale and
 * aiter_amd_fused_moe_a8w4, given the same num_experts (experts held in
 * w1/w2), global_experts (expert_mask entries; num_experts when there is no
 * mask) and block_m (0: the default the one-call entries pick, from the
 * token count and num_experts). */
int64_t aiter_amd_fused_moe_workspace_bytes(int64_t tokens, int64_t model_dim,
                                            int64_t inter_dim, int64_t num_experts,
                                            int64_t global_experts, int64_t topk,
                                            int64_t block_m);

/* No counterpart in the reference.  Where the two-launch one-call layer
 * (aiter_amd_fused_moe_fp8_blockscale / aiter_amd_fused_moe_a8w4, not the
 * _1stage entries) keeps its stage-1 output in the caller's workspace, for
 * callers that inspect the intermediate (parity tests, debugging): after a
 * call with these sizes, the fp8 a2 [tokens*topk, inter_dim] (row
 * t*topk + slot) starts offsets[0] bytes into the workspace and its f32
 * 1x128 scales [tokens*topk, inter_dim/128] offsets[1] bytes in.  Rows of
 * pairs not routed to a local expert hold no data.  Arguments as
 * aiter_amd_fused_moe_workspace_bytes. */
int aiter_amd_fused_moe_workspace_a2_offsets(int64_t tokens, int64_t model_dim,
                                             int64_t inter_dim, int64_t num_experts,
                                             int64_t global_experts, int64_t topk,
                                             int64_t block_m, int64_t* offsets);

/* The whole 2-stage FP8 blockscale MoE in one call; replaces the sequence
 * of fused_moe_ -> moe_sorting -> fused_moe_2stages (aiter/fused_moe.py:
 * 205-364, 27-103, 1103-1334) for quant_type per_1x128 / per_128x128.
 *   hidden_states [tokens, model_dim] bf16/fp16 (hidden_dtype)
 *   w1/w2/w1_scale/w2_scale as for the stage calls; topk_ids/topk_weights
 *   [tokens, topk]; expert_mask [global_experts] or NULL (then
 *   global_experts == num_experts); num_local_tokens device i32[1] or NULL.
 *   out [tokens, model_dim] in out_dtype (bf16/fp16).
 *   block_m = 0 picks the default for the token count; activation 0 Silu /
 *   1 Gelu; doweight_stage1 as fused_moe's (the routing weights scale gate
 *   and up before the activation, stage 2 sums unweighted). */
int aiter_amd_fused_moe_fp8_blockscale(const void* hidden_states, int hidden_dtype,
                                       const void* w1, const float* w1_scale, const void* w2,
                                       const float* w2_scale, const float* topk_weights,
                                       const int32_t* topk_ids, const int32_t* expert_mask,
                                       const int32_t* num_local_tokens, void* out,
                                       int out_dtype, int64_t tokens, int64_t model_dim,
                                       int64_t inter_dim, int64_t num_experts,
                                       int64_t global_experts, int64_t topk, int64_t block_m,
                                       int64_t activation, int64_t doweight_stage1,
                                       int64_t w_shuffled, void* workspace,
                                       int64_t workspace_bytes, void* stream);

/* Bytes of the library-owned device workspace behind
 * aiter_amd_fused_moe_fp8_blockscale_noalloc (one copy per GPU). */
#define AITER_AMD_SCRATCH_BYTES (32ll << 20)

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture that must not allocate, tight serving
 * loops, harnesses that forbid hipMalloc): aiter_amd_fused_moe_fp8_blockscale
 * with its workspace taken from a static device buffer of
 * AITER_AMD_SCRATCH_BYTES that the library holds per GPU until the process
 * ends.  It calls no hipMalloc / hipFree.  A layer whose workspace
 * (aiter_amd_fused_moe_workspace_bytes) exceeds the buffer is rejected with
 * an error; at MiMo dims (hidden 4096, inter 2048, 256 experts, top-8) that
 * is above ~370 tokens.  The stream must belong to the current device.
 * Every call on one GPU shares that GPU's buffer: calls that overlap on one
 * GPU (other streams, other threads) race and must be serialised by the
 * caller.  The buffer keeps the last call's contents; the call itself clears
 * what it reads before writing. */
int aiter_amd_fused_moe_fp8_blockscale_noalloc(
    const void* hidden_states, int hidden_dtype, const void* w1, const float* w1_scale,
    const void* w2, const float* w2_scale, const float* topk_weights, const int32_t* topk_ids,
    const int32_t* expert_mask, const int32_t* num_local_tokens, void* out, int out_dtype,
    int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t num_experts,
    int64_t global_experts, int64_t topk, int64_t block_m, int64_t activation,
    int64_t doweight_stage1, int64_t w_shuffled, void* stream);

/* The whole 2-stage A8W4 MoE in one call: fused_moe_ with quant_type per_1x32
 * and fp4x2 weights (aiter/fused_moe.py:255-275, 1103-1334), fp8 1x128
 * activations.  Arguments as aiter_amd_fused_moe_fp8_blockscale with the
 * weights and e8m0 scales of aiter_amd_moe_stage{1,2}_a8w4. */
int aiter_amd_fused_moe_a8w4(const void* hidden_states, int hidden_dtype, const void* w1,
                             const uint8_t* w1_scale, const void* w2, const uint8_t* w2_scale,
                             const float* topk_weights, const int32_t* topk_ids,
                             const int32_t* expert_mask, const int32_t* num_local_tokens,
                             void* out, int out_dtype, int64_t tokens, int64_t model_dim,
                             int64_t inter_dim, int64_t num_experts, int64_t global_experts,
                             int64_t topk, int64_t block_m, int64_t activation,
                             int64_t doweight_stage1, int64_t w_shuffled, void* workspace,
                             int64_t workspace_bytes, void* stream);

/* The whole layer with both GEMMs in ONE launch; replaces fused_moe_1stage
 * -> fmoe_fp8_blockscale_g1u1 (aiter/fused_moe.py:367-511,
 * csrc/py_itfs_cu/asm_fmoe.cu:858-922), which the reference picks per shape
 * from its tuned table (run_1stage). Each workgroup runs stage 1 for one
 * 128-wide slice of inter_dim of one M-block, keeps the slice's fp8 rows
 * (one 1x128 quant group each, as the reference's a2) on chip and adds their
 * down-GEMM share into the fp32 accumulator; then one pass writes out.
 * Arguments as aiter_amd_fused_moe_fp8_blockscale (same workspace size);
 * block_m must be 16 or 32 (0: the default, which must then be one of them)
 * and model_dim a multiple of 256 up to 8192. */
int aiter_amd_fused_moe_1stage_fp8_blockscale(
    const void* hidden_states, int hidden_dtype, const void* w1, const float* w1_scale,
    const void* w2, const float* w2_scale, const float* topk_weights, const int32_t* topk_ids,
    const int32_t* expert_mask, const int32_t* num_local_tokens, void* out, int out_dtype,
    int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t num_experts,
    int64_t global_experts, int64_t topk, int64_t block_m, int64_t activation,
    int64_t doweight_stage1, int64_t w_shuffled, void* workspace, int64_t workspace_bytes,
    void* stream);

/* The one-launch layer on MXFP4 weights (A8W4); arguments as
 * aiter_amd_fused_moe_a8w4, constraints as
 * aiter_amd_fused_moe_1stage_fp8_blockscale. Replaces the same reference
 * path with quant_type per_1x32 (aiter/fused_moe.py:367-511). */
int aiter_amd_fused_moe_1stage_a8w4(
    const void* hidden_states, int hidden_dtype, const void* w1, const uint8_t* w1_scale,
    const void* w2, const uint8_t* w2_scale, const float* topk_weights, const int32_t* topk_ids,
    const int32_t* expert_mask, const int32_t* num_local_tokens, void* out, int out_dtype,
    int64_t tokens, int64_t model_dim, int64_t inter_dim, int64_t num_experts,
    int64_t global_experts, int64_t topk, int64_t block_m, int64_t activation,
    int64_t doweight_stage1, int64_t w_shuffled, void* workspace, int64_t workspace_bytes,
    void* stream);

/* ---- routing: top-k experts per token from the router logits ----
 * gating [tokens, num_experts] fp32/bf16/fp16 (dtype code as above),
 * contiguous; outputs topk_weights f32 and topk_ids i32 with row strides
 * weights_stride / ids_stride (elements, >= topk). num_experts <= 1024,
 * topk <= 32. Ties rank the lower expert (group) index first; rows come out
 * in rank order. */

/* Replaces topk_softmax / topk_softmax_asm (aiter/ops/moe_op.py:15-36;
 * csrc/kernels/topk_softmax_kernels.cu:380-500), as called by fused_topk
 * (aiter/fused_moe.py:1853-1923): experts ranked by logit, weight
 * exp(x - rowmax) / (sum over the topk if need_renorm, else over the row).
 * token_expert_indices [tokens, topk] i32 (= rank * tokens + row) or NULL. */
int aiter_amd_topk_softmax(const void* gating, int gating_dtype, int64_t tokens,
                           int64_t num_experts, int64_t topk, float* topk_weights,
                           int64_t weights_stride, int32_t* topk_ids, int64_t ids_stride,
                           int32_t* token_expert_indices, int need_renorm, void* stream);

/* Replaces topk_softmax with its shared-expert fusion (num_shared_experts > 0,
 * shared_expert_scoring_func "sigmoid"; aiter/ops/moe_op.py:15-24,
 * csrc/kernels/topk_softmax_kernels.cu:326-353, 760-810): gating rows hold
 * num_experts routed logits then num_shared_experts shared ones (row stride
 * num_experts + num_shared_experts, contiguous); the routed experts are
 * ranked and weighted as aiter_amd_topk_softmax over the first num_experts
 * columns, and topk_weights[t, topk + j] = sigmoid(gating[t, num_experts +
 * j]) for j < num_shared_experts (weights_stride >= topk +
 * num_shared_experts); topk_ids holds the routed experts only. */
int aiter_amd_topk_softmax_shared(const void* gating, int gating_dtype, int64_t tokens,
                                  int64_t num_experts, int64_t num_shared_experts,
                                  int64_t topk, float* topk_weights, int64_t weights_stride,
                                  int32_t* topk_ids, int64_t ids_stride,
                                  int32_t* token_expert_indices, int need_renorm,
                                  void* stream);

/* Replaces topk_sigmoid (aiter/ops/moe_op.py:39-42; semantics
 * op_tests/test_moe_topk_sigmoid.py:28-32): experts ranked by logit, weight
 * sigmoid(logit). */
int aiter_amd_topk_sigmoid(const void* gating, int gating_dtype, int64_t tokens,
                           int64_t num_experts, int64_t topk, float* topk_weights,
                           int64_t weights_stride, int32_t* topk_ids, int64_t ids_stride,
                           void* stream);

/* Replaces grouped_topk (aiter/ops/topk.py:28-38, torch semantics 163-197)
 * when correction_bias is NULL, and biased_grouped_topk
 * (aiter/ops/topk.py:15-25,90-160) when it is an f32 [num_experts] array.
 *   grouped: scores = softmax (is_softmax != 0) or sigmoid of the logits;
 *     a group's score is its best expert score;
 *   biased: scores = sigmoid; choice = score + bias; a group's score is the
 *     sum of its two best choices (is_softmax must be 0).
 * The topk_group best groups are kept and their experts ranked by choice
 * (grouped: score); weight = score * routed_scaling_factor / (sum of the
 * topk scores if need_renorm, else 1). num_expert_group <= 32 divides
 * num_experts; topk_group <= num_expert_group; topk <= the experts kept. */
int aiter_amd_grouped_topk(const void* gating, int gating_dtype, const float* correction_bias,
                           int64_t tokens, int64_t num_experts, int64_t topk,
                           int64_t num_expert_group, int64_t topk_group, int need_renorm,
                           int is_softmax, float routed_scaling_factor, float* topk_weights,
                           int64_t weights_stride, int32_t* topk_ids, int64_t ids_stride,
                           void* stream);

/* Measurement hooks of the one-call entries, the per-kernel device times the
 * reference's perftest reads from a profiler trace (aiter/test_common.py:
 * 46-120).  Between begin and end, each of up to max_calls calls of
 * aiter_amd_fused_moe_* on this thread records HIP events on its stream
 * around its five steps: sorting (with the activation quant when it rides
 * in that launch), the separate activation quant, stage 1, stage 2, and the
 * finishing pass (slot sum or f32 -> 16-bit).  end waits for the last
 * event, writes step_ms[call * 5 + step] (a step that launched nothing
 * reads ~0) and returns the number of calls recorded, or -1 on error. */
int aiter_amd_layer_timing_begin(int64_t max_calls);
int64_t aiter_amd_layer_timing_end(float* step_ms, int64_t max_calls);

/* Default M-block (sorted rows per GEMM tile) for a token count: 16 / 32 / 64 by the average
 * rows per expert, tokens * topk / global_experts (<= 8, <= 20, else); 128 once experts average
 * >= 64 rows, the pairs this GPU holds (tokens * topk * num_experts / global_experts) times
 * inter_dim reach 2^26, and the dims allow 128-row tiles. global_experts: the expert_mask
 * entries of an expert-parallel share, or <= 0 (or num_experts) without one. The one-call
 * entries and the workspace query resolve block_m <= 0 with this rule.
 * Plays the part of the block_m choice in aiter's get_2stage_cfgs (aiter/fused_moe.py:830-905). */
int64_t aiter_amd_default_block_m(int64_t tokens, int64_t topk, int64_t num_experts,
                                  int64_t global_experts, int64_t model_dim, int64_t inter_dim);

#ifdef __cplusplus
}
#endif

#endif /* AITER_AMD_H */
