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
 *     memory.
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
 *   M * row bytes (any row of 16 bytes or more at 256 experts and topk <= 8;
 *   about num_experts^2 / 8192 bytes per row for more experts); otherwise the
 *   call fails with an error and the caller uses aiter_amd_moe_sorting_fwd
 *   with a workspace. */
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

/* Replaces topk_softmax (aiter/ops/moe_op.py:15-24): gating_output
 * [M, E] f32/bf16/fp16 -> topk_weights f32 [M, k], topk_indices i32 [M, k]
 * (row strides taken from the tensors), token_expert_indices i32 [M, k] or
 * NULL; num_shared_experts must be 0 and shared_expert_scoring_func empty
 * or NULL (the shared-expert fusion is not provided). */
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
