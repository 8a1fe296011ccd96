/*
 * aiter_ctypes.h — entry points of libaiter_amd.so in the shape of the
 * reference's torch-free ctypes FFI, so that its own binder,
 * compile_ops(..., ffi_type="ctypes") (aiter/jit/core.py:1105-1363), binds
 * them by name with no stub of its own:
 *   - each tensor argument is an aiter_tensor_t* (NULL for an optional tensor
 *     that is None); a Python int is int64_t, a bool int, a str const char*,
 *     and the hipStream_t (torch's current stream) is appended last;
 *   - each entry returns 0 on success and -1 on failure, with the message in
 *     a thread-local string read by aiter_get_last_error(), which returns
 *     NULL when there is none (csrc/include/aiter_ctypes_error.h:60-147);
 *     aiter_ctypes_abi_version() returns 2, the status-return convention;
 *   - tensor metadata (dtype, shape, strides, device) is validated before
 *     any device work, and the device is set from device_id for the call;
 *   - every buffer is owned by the caller; nothing here allocates device
 *     memory, except the workspace fmoe_fp8_blockscale_g1u1 needs and its
 *     signature does not carry (held by the library per device and stream,
 *     described there).
 * The error state is shared with the aiter_amd_* entry points of
 * include/aiter_amd.h, which these entries call after unpacking tensors.
 */
#ifndef AITER_AMD_CTYPES_H
#define AITER_AMD_CTYPES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The tensor descriptor of csrc/include/aiter_tensor.h:8-37 (a POD of 160
 * bytes whose size aiter/utility/aiter_types.py:68-86 asserts). dtype_ is an
 * AiterDtype code (csrc/include/aiter_enum.h:27-43): fp8 0, fp8_e8m0 1,
 * fp16 2, bf16 3, fp32 4, fp4x2 6, i32 8, u8 11. */
typedef struct aiter_tensor_t {
    void* ptr;
    size_t numel_;
    int ndim;
    int64_t shape[8];
    int64_t strides[8];
    int dtype_;
    int device_id;
} aiter_tensor_t;

/* aiter_ctypes_error.h:60-72 (AITER_CTYPES_ERROR_DEF). */
int aiter_ctypes_abi_version(void);
const char* aiter_get_last_error(void);
void aiter_clear_last_error(void);

/* Replaces moe_sorting_fwd (aiter/ops/moe_sorting.py:11-25, host
 * csrc/py_itfs_ck/moe_sorting_kernels.cu:10-70), same arguments and outputs
 * as aiter_amd_moe_sorting_fwd.
 *   topk_ids i32 [M, topk], topk_weights f32 [M, topk]; sorted_token_ids i32,
 *   sorted_weights f32 of >= M*topk + num_experts*unit_size - topk entries;
 *   sorted_expert_ids i32 of >= ceil(that / unit_size); num_valid_ids i32
 *   of >= 2; moe_buf [M, model_dim] (row bytes a multiple of 16), zeroed for
 *   the local token rows; local_expert_mask i32 [num_experts] or NULL;
 *   num_local_tokens i32 [1] or NULL; dispatch_policy is accepted and
 *   ignored.  The reference allocates a workspace with torch for more than
 *   one chunk of tokens; here the chunk counts are kept in moe_buf, which a
 *   last launch clears, so nothing is allocated.  moe_buf must then hold
 *   them: aiter_amd_moe_sorting_workspace_bytes(M, topk, num_experts) <=
 *   M * row bytes.  That is ceil(M / c) * num_experts * 4 bytes for the
 *   chunk size c sorting picks (0 when M fits one chunk); c is 16 tokens for
 *   129 to 2047 tokens at 256 experts, so rows need at least 4 * 256 / 16 =
 *   64 bytes there, plus one chunk's counts (80-byte rows suffice from 129
 *   tokens on; MiMo's 8192-byte rows always do); otherwise the call fails
 *   with an error and the caller uses aiter_amd_moe_sorting_fwd with a
 *   workspace. */
int moe_sorting_fwd(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights,
                    aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_weights,
                    aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                    aiter_tensor_t* moe_buf, int64_t num_experts, int64_t unit_size,
                    aiter_tensor_t* local_expert_mask, aiter_tensor_t* num_local_tokens,
                    int64_t dispatch_policy, void* stream);

/* Replaces dynamic_per_token_scaled_quant (aiter/ops/quant.py:472-481) as
 * per_group_quant_hip calls it for 1x128 groups (quant.py:260-292): input
 * bf16/fp16 viewed [groups, 128], out fp8 [rows, cols] (cols % 128 == 0),
 * scales f32 with rows*cols/128 entries, row-major [rows, cols/128] or, with
 * shuffle_scale, [cols/128, rows]; num_rows i32 [1] or NULL; scale_ub must
 * be NULL (only dynamic scales). */
int dynamic_per_token_scaled_quant(aiter_tensor_t* out, aiter_tensor_t* input,
                                   aiter_tensor_t* scales, aiter_tensor_t* scale_ub,
                                   int shuffle_scale, aiter_tensor_t* num_rows,
                                   int64_t num_rows_factor, void* stream);

/* Replaces moe_stage1_g1u1 for per_1x128 fp8 (aiter/ops/moe_op.py:196-213,
 * csrc/py_itfs_cu/asm_moe_2stage.cu:148-280), as asm_stage1 calls it
 * (aiter/fused_moe.py:1345-1406, 1213-1221, 1293-1301):
 *   input fp8 [T, model_dim]; a1_scale f32 of T*model_dim/128 entries in
 *   the transposed layout [model_dim/128, T] (per_group_quant_hip with
 *   transpose_scale, as fused_moe_2stages makes it for this kernel);
 *   w1 fp8 [E, 2*inter_dim, model_dim] in the (16,16) shuffled layout;
 *   w1_scale f32 [E, 2*inter_dim/128, model_dim/128];
 *   out fp8 [T + ceil(4T/128), topk, inter_dim]: the first T rows receive
 *   the requantised SiLU(gate)*up (or GELU) codes [T, topk, inter_dim], the
 *   bytes after them the f32 1x128 scales [T, topk * inter_dim/128];
 *   sorted_weights f32 or NULL (doweight_stage1); activation 0 Silu, 1 Gelu;
 *   quant_type must be per_1x128 (4); block_m 16, 32, 64 or 128; ksplit
 *   must be 0 (the library splits K itself where that pays); kernelName is
 *   accepted and ignored (kernel choice is by shape); w2 is unused. */
int moe_stage1_g1u1(aiter_tensor_t* input, aiter_tensor_t* w1, aiter_tensor_t* w2,
                    aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids,
                    aiter_tensor_t* num_valid_ids, aiter_tensor_t* out, int64_t inter_dim,
                    const char* kernelName, int64_t block_m, int64_t ksplit, int64_t activation,
                    int64_t quant_type, aiter_tensor_t* a1_scale, aiter_tensor_t* w1_scale,
                    aiter_tensor_t* sorted_weights, void* stream);

/* Replaces ck_moe_stage2 for per_1x128 fp8 a2 (aiter/ops/moe_op.py:319-340,
 * csrc/ck_gemm_moe_2stages_codegen/gemm_moe_ck2stages.cu:118-181), as
 * fused_moe_2stages calls it (aiter/fused_moe.py:1316-1332):
 *   inter_states fp8 [T, topk, inter_dim]; a2_scale f32 of
 *   T*topk*inter_dim/128 entries ([T, topk, inter_dim/128]); w2 fp8
 *   [E, model_dim, inter_dim] with w2_scale f32 [E, model_dim/128,
 *   inter_dim/128], or fp4x2 / u8 [E, model_dim, inter_dim/2] with e8m0 / u8
 *   w2_scale [E, model_dim, inter_dim/32] (A8W4); out = moe_buf [T, model_dim]
 *   bf16 / fp16 (or fp32), zeroed by moe_sorting_fwd, accumulates
 *   sorted_weight * row with atomics; sorted_weights NULL gives unit weights
 *   (doweight_stage1); is_shuffled: the (16,16) weight layout; quant_type
 *   per_1x128 (4) or, for fp4 weights, per_1x32 (3); splitk 0 or 1;
 *   kernelName, use_non_temporal_load and dst_type are accepted and ignored;
 *   activation and w1 are unused. */
int ck_moe_stage2(aiter_tensor_t* inter_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids,
                  aiter_tensor_t* num_valid_ids, aiter_tensor_t* out, int64_t topk,
                  const char* kernelName, aiter_tensor_t* w2_scale, aiter_tensor_t* a2_scale,
                  int64_t block_m, aiter_tensor_t* sorted_weights, int64_t quant_type,
                  int64_t activation, int64_t splitk, int use_non_temporal_load,
                  const char* dst_type, int is_shuffled, void* stream);

/* Replaces ck_moe_stage1 (aiter/ops/moe_op.py:295-316, host
 * csrc/ck_gemm_moe_2stages_codegen/gemm_moe_ck2stages.cu:46-116), as the
 * ck_moe_stage1 wrapper of aiter/fused_moe.py:1669-1725 calls it through
 * ck_moe_stage1_fwd (aiter/ops/moe_op.py:534-575):
 *   hidden_states fp8 [T, model_dim] with a1_scale f32 [T, model_dim/128]
 *   (row-major: fused_moe_2stages quantises without transpose_scale for
 *   this kernel); w1 fp8 [E, 2*inter_dim, model_dim] with w1_scale f32
 *   [E, 2*inter_dim/128, model_dim/128] and quant_type per_1x128 (4), or
 *   fp4x2 / u8 [E, 2*inter_dim, model_dim/2] with e8m0 / u8 w1_scale
 *   [E, 2*inter_dim, model_dim/32] and quant_type per_1x32 (3);
 *   splitk 0 or 1: out bf16 / fp16 [T, topk, inter_dim] receives
 *   act(gate) * up (activation 0 Silu, 1 Gelu) rounded once;
 *   splitk > 1 (a divisor of model_dim/128): out fp32 [>= T*topk,
 *   2*inter_dim] receives the gate | up sums before the activation in rows
 *   t*topk + slot (zeroed first, as the reference's KBatch > 1 kernel
 *   does), which silu_and_mul / gelu_and_mul then finish;
 *   sorted_weights f32 or NULL (doweight_stage1: gate and up scaled before
 *   the activation); block_m 16, 32, 64 or 128; is_shuffled: the (16,16)
 *   weight layout; kernelName, use_non_temporal_load and dst_type are
 *   accepted and ignored; w2 is unused. */
int ck_moe_stage1(aiter_tensor_t* hidden_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids,
                  aiter_tensor_t* num_valid_ids, aiter_tensor_t* out, int64_t topk,
                  const char* kernelName, aiter_tensor_t* w1_scale, aiter_tensor_t* a1_scale,
                  int64_t block_m, aiter_tensor_t* sorted_weights, int64_t quant_type,
                  int64_t activation, int64_t splitk, int use_non_temporal_load,
                  const char* dst_type, int is_shuffled, void* stream);

/* Replace silu_and_mul / gelu_and_mul (aiter/ops/activation.py:10-19,
 * csrc/kernels/activation_kernels.cu:24-90, 337-354): input [..., 2*d]
 * fp32 / bf16 / fp16, out [..., d] fp32 / bf16 / fp16 (same rows, both
 * contiguous), out = act(input[..., :d]) * input[..., d:], computed in fp32
 * and rounded once. */
int silu_and_mul(aiter_tensor_t* out, aiter_tensor_t* input, void* stream);
int gelu_and_mul(aiter_tensor_t* out, aiter_tensor_t* input, void* stream);

/* Replaces fmoe_fp8_blockscale_g1u1 (aiter/ops/moe_op.py:172-192,
 * csrc/py_itfs_cu/asm_fmoe.cu:858-922), as fused_moe_1stage calls it
 * (aiter/fused_moe.py:367-511), the reference's default for FP8 blockscale
 * above 32 tokens:
 *   out bf16 / fp16 [T, model_dim] = moe_buf, which moe_sorting_fwd zeroed:
 *   the layer is added to it (in fp32, rounded once) for the first
 *   num_valid_ids[1] rows; input fp8 [T, model_dim] with input_scale f32 in
 *   the transposed layout [model_dim/128, T] (per_group_quant_hip with
 *   transpose_scale); gate fp8 [E, 2*inter_dim, model_dim] and down fp8
 *   [E, model_dim, inter_dim] in the (16,16) shuffled layout (the layout
 *   the replaced kernel reads; the signature carries no flag); fc1_scale f32
 *   [E, 2*inter_dim/128, model_dim/128], fc2_scale f32 [E, model_dim/128,
 *   inter_dim/128]; sorted_* and num_valid_ids from moe_sorting at
 *   block_size_M; fc_scale_blkn = fc_scale_blkk = 128; fc2_smooth_scale
 *   NULL; activation 0 Silu, 1 Gelu; kernel_name accepted and ignored.
 * The pairs are recovered from the sorted entries and the layer runs as
 * aiter_amd_fused_moe_sorted_fp8_blockscale (include/aiter_amd.h): two GEMM
 * launches at this library's block size for the shape. Its intermediates
 * live in a device workspace the library holds per (device, stream) and
 * grows with hipMalloc when a larger layer arrives; growing is refused
 * during HIP graph capture (one call of that size on the same stream before
 * capturing avoids
 * it). About 0.7 GB at T = 8192 for MiMo dims (hidden 4096, inter 2048,
 * top-8). */
int fmoe_fp8_blockscale_g1u1(aiter_tensor_t* out, aiter_tensor_t* input, aiter_tensor_t* gate,
                             aiter_tensor_t* down, aiter_tensor_t* sorted_token_ids,
                             aiter_tensor_t* sorted_weights, aiter_tensor_t* sorted_expert_ids,
                             aiter_tensor_t* num_valid_ids, int64_t topk,
                             aiter_tensor_t* input_scale, aiter_tensor_t* fc1_scale,
                             aiter_tensor_t* fc2_scale, const char* kernel_name,
                             int64_t fc_scale_blkn, int64_t fc_scale_blkk,
                             aiter_tensor_t* fc2_smooth_scale, int64_t activation,
                             int64_t block_size_M, void* stream);

/* Replaces topk_softmax (aiter/ops/moe_op.py:15-24,
 * csrc/kernels/topk_softmax_kernels.cu:760-810): gating_output
 * [M, E + S] f32/bf16/fp16 (contiguous) -> topk_weights f32 [M, k + S],
 * topk_indices i32 [M, k] (row strides taken from the tensors),
 * token_expert_indices i32 [M, k] or NULL. The first E columns are ranked
 * by softmax top-k; with S = num_shared_experts > 0 and
 * shared_expert_scoring_func "sigmoid" (the only function the reference
 * supports), topk_weights[:, k + j] = sigmoid(gating_output[:, E + j]).
 * S > 0 with an empty function is an error, as is another function. */
int topk_softmax(aiter_tensor_t* topk_weights, aiter_tensor_t* topk_indices,
                 aiter_tensor_t* token_expert_indices, aiter_tensor_t* gating_output,
                 int need_renorm, int64_t num_shared_experts,
                 const char* shared_expert_scoring_func, void* stream);

/* Replaces topk_sigmoid (aiter/ops/moe_op.py:39-42). */
int topk_sigmoid(aiter_tensor_t* topk_weights, aiter_tensor_t* topk_indices,
                 aiter_tensor_t* gating_output, void* stream);

/* Replaces grouped_topk (aiter/ops/topk.py:28-38). */
int grouped_topk(aiter_tensor_t* gating_output, aiter_tensor_t* topk_weights,
                 aiter_tensor_t* topk_ids, int64_t num_expert_group, int64_t topk_group,
                 int need_renorm, int is_softmax, float routed_scaling_factor, void* stream);

/* Replaces biased_grouped_topk (aiter/ops/topk.py:15-25). */
int biased_grouped_topk(aiter_tensor_t* gating_output, aiter_tensor_t* correction_bias,
                        aiter_tensor_t* topk_weights, aiter_tensor_t* topk_ids,
                        int64_t num_expert_group, int64_t topk_grp, int need_renorm,
                        float routed_scaling_factor, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* AITER_AMD_CTYPES_H */
