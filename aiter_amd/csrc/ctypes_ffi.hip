// Entry points in the shape of the reference's torch-free ctypes FFI
// (aiter_tensor_t* arguments, 0/-1 status, hipStream_t last), declared in
// include/aiter_ctypes.h.  Each one checks the tensor descriptors -- dtype,
// shape, contiguity, device -- before any device work, unpacks pointers
// and sizes, and calls the plain-pointer entry of include/aiter_amd.h that
// does the work, so the two surfaces share validation, kernels and the
// thread-local error text.
#include "../../include/aiter_amd.h"
#include "../../include/aiter_ctypes.h"

#include <algorithm>
#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "common.h"

namespace aiter_amd {
namespace {

static_assert(sizeof(aiter_tensor_t) == 160, "aiter_tensor_t must keep the reference's layout");

constexpr int DT_U8 = 11;
constexpr int kQuantPer1x32 = 3;
constexpr int kQuantPer1x128 = 4;

const char* dtype_name(int d) {
    switch (d) {
        case DT_FP8: return "fp8";
        case DT_FP8_E8M0: return "fp8_e8m0";
        case DT_FP16: return "fp16";
        case DT_BF16: return "bf16";
        case DT_FP32: return "fp32";
        case DT_FP4X2: return "fp4x2";
        case DT_I32: return "i32";
        case DT_U8: return "u8";
        default: return "unsupported";
    }
}

// Raises (through safe_call) when a required tensor is missing.
const aiter_tensor_t& need(const aiter_tensor_t* t, const char* name) {
    AMD_CHECK(t != nullptr, std::string(name) + " is required");
    AMD_CHECK(t->ndim >= 0 && t->ndim <= 8, std::string(name) + " has an invalid ndim");
    return *t;
}

int64_t dim(const aiter_tensor_t& t, int i) { return i < 0 ? t.shape[t.ndim + i] : t.shape[i]; }

bool contiguous(const aiter_tensor_t& t) {
    int64_t expected = 1;
    for (int d = t.ndim - 1; d >= 0; --d) {
        if (t.shape[d] != 1 && t.strides[d] != expected) return false;
        expected *= t.shape[d];
    }
    return true;
}

void check_dtype(const aiter_tensor_t& t, const char* name, std::initializer_list<int> ok) {
    for (int d : ok)
        if (t.dtype_ == d) return;
    std::string want;
    for (int d : ok) want += std::string(want.empty() ? "" : " or ") + dtype_name(d);
    AMD_CHECK(false, std::string(name) + " must be " + want + ", got " + dtype_name(t.dtype_));
}

void check_contig(const aiter_tensor_t& t, const char* name) {
    AMD_CHECK(contiguous(t), std::string(name) + " must be contiguous");
}

void check_device(const aiter_tensor_t& t, int dev, const char* name) {
    AMD_CHECK(t.device_id == dev, std::string(name) + " is on device " +
                                      std::to_string(t.device_id) + ", expected " +
                                      std::to_string(dev));
}

void check_shape(const aiter_tensor_t& t, const char* name, std::initializer_list<int64_t> s) {
    bool ok = t.ndim == (int)s.size();
    int i = 0;
    for (int64_t v : s) ok = ok && t.shape[i++] == v;
    if (ok) return;
    std::string got, want;
    for (int d = 0; d < t.ndim; ++d) got += (d ? ", " : "") + std::to_string(t.shape[d]);
    i = 0;
    for (int64_t v : s) want += (i++ ? ", " : "") + std::to_string(v);
    AMD_CHECK(false, std::string(name) + " must be [" + want + "], got [" + got + "]");
}

void check_numel(const aiter_tensor_t& t, const char* name, int64_t at_least) {
    AMD_CHECK((int64_t)t.numel_ >= at_least, std::string(name) + " holds " +
                                                  std::to_string(t.numel_) + " elements, " +
                                                  std::to_string(at_least) + " needed");
}

// A checked, contiguous tensor on `dev` of one of the dtypes.
const aiter_tensor_t& tensor(const aiter_tensor_t* t, const char* name, int dev,
                             std::initializer_list<int> dtypes) {
    const aiter_tensor_t& r = need(t, name);
    check_dtype(r, name, dtypes);
    check_contig(r, name);
    check_device(r, dev, name);
    return r;
}

const aiter_tensor_t* optional(const aiter_tensor_t* t, const char* name, int dev,
                               std::initializer_list<int> dtypes) {
    return t ? &tensor(t, name, dev, dtypes) : nullptr;
}

const void* ptr(const aiter_tensor_t* t) { return t ? t->ptr : nullptr; }

int64_t row_bytes(const aiter_tensor_t& t) {
    int64_t es = t.dtype_ == DT_FP32 || t.dtype_ == DT_I32 ? 4
                 : t.dtype_ == DT_FP16 || t.dtype_ == DT_BF16 ? 2 : 1;
    return t.ndim ? dim(t, -1) * es : es;
}

// Sets the current device to `dev` for the call and restores the caller's.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        AMD_HIP_CHECK(hipGetDevice(&prev));
        if (prev != dev) AMD_HIP_CHECK(hipSetDevice(dev));
    }
    ~DeviceGuard() {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Runs a plain-pointer entry and turns its -1 into an exception carrying the
// message it left (safe_call stores it back).
void run(int rc) {
    if (rc != 0) throw AbiError(aiter_amd_get_last_error());
}

// Device workspace the library holds for the reference-shaped entries whose
// signatures carry none (fmoe_fp8_blockscale_g1u1): one buffer per (device,
// stream), grown on demand with hipMalloc and kept until the process ends.
// Growing waits for the stream's earlier work, frees the old buffer and is
// refused while the stream is being captured into a HIP graph (a call of
// the same or a larger size made before capture avoids it). Calls on one
// stream are ordered by the stream; calls on different streams use
// different buffers.
struct Pooled {
    void* p = nullptr;
    int64_t bytes = 0;
};
std::mutex g_pool_mu;
std::map<std::pair<int, void*>, Pooled> g_pool;

void* pooled_workspace(int dev, void* stream, int64_t bytes, const char* who) {
    std::lock_guard<std::mutex> lock(g_pool_mu);
    Pooled& w = g_pool[{dev, stream}];
    if (w.bytes >= bytes) return w.p;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    AMD_HIP_CHECK(hipStreamIsCapturing((hipStream_t)stream, &st));
    AMD_CHECK(st == hipStreamCaptureStatusNone,
              std::string(who) + " needs " + std::to_string(bytes) +
                  " bytes of library workspace on this stream, which cannot be allocated "
                  "during graph capture: make one call of this size before capturing");
    // grow by at least a quarter, in 2 MiB steps, so a slowly growing batch
    // does not reallocate on every call
    int64_t want = std::max(bytes, w.bytes + w.bytes / 4);
    want = (want + (2 << 20) - 1) / (2 << 20) * (2 << 20);
    if (w.p) {
        AMD_HIP_CHECK(hipStreamSynchronize((hipStream_t)stream));
        AMD_HIP_CHECK(hipFree(w.p));
        w.p = nullptr;
        w.bytes = 0;
    }
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, (size_t)want);
    AMD_CHECK(e == hipSuccess && p, std::string(who) + ": hipMalloc of " + std::to_string(want) +
                                        " bytes of workspace failed: " + hipGetErrorString(e));
    w.p = p;
    w.bytes = want;
    return p;
}

}  // namespace
}  // namespace aiter_amd

using namespace aiter_amd;

extern "C" {

int moe_sorting_fwd(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights,
                    aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_weights,
                    aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                    aiter_tensor_t* moe_buf, int64_t num_experts, int64_t unit_size,
                    aiter_tensor_t* local_expert_mask, aiter_tensor_t* num_local_tokens,
                    int64_t dispatch_policy, void* stream) {
    return safe_call([&] {
        const int dev = need(topk_ids, "topk_ids").device_id;
        const auto& ids = tensor(topk_ids, "topk_ids", dev, {DT_I32});
        AMD_CHECK(ids.ndim == 2, "topk_ids must be [M, topk]");
        const int64_t M = ids.shape[0], topk = ids.shape[1];
        const auto& w = tensor(topk_weights, "topk_weights", dev, {DT_FP32});
        check_shape(w, "topk_weights", {M, topk});
        const auto& sid = tensor(sorted_token_ids, "sorted_token_ids", dev, {DT_I32});
        const auto& sw = tensor(sorted_weights, "sorted_weights", dev, {DT_FP32});
        const auto& se = tensor(sorted_expert_ids, "sorted_expert_ids", dev, {DT_I32});
        const auto& nv = tensor(num_valid_ids, "num_valid_ids", dev, {DT_I32});
        check_numel(nv, "num_valid_ids", 2);
        const auto& buf = tensor(moe_buf, "moe_buf", dev,
                                 {DT_BF16, DT_FP16, DT_FP32, DT_FP8, DT_U8, DT_I32});
        AMD_CHECK(buf.ndim == 2 && buf.shape[0] == M, "moe_buf must be [M, model_dim]");
        const auto* mask = optional(local_expert_mask, "local_expert_mask", dev, {DT_I32});
        if (mask) check_numel(*mask, "local_expert_mask", num_experts);
        const auto* loc = optional(num_local_tokens, "num_local_tokens", dev, {DT_I32});
        if (loc) check_numel(*loc, "num_local_tokens", 1);
        const int64_t rb = row_bytes(buf);
        AMD_CHECK(rb % 16 == 0, "moe_buf rows must be a multiple of 16 bytes");
        DeviceGuard guard(dev);
        // more than one chunk of tokens: the chunk counts live in moe_buf
        const int64_t ws = aiter_amd_moe_sorting_workspace_bytes(M, topk, num_experts);
        AMD_CHECK(ws <= M * rb, "moe_buf is too small to hold the sorting counts (" +
                                    std::to_string(ws) + " bytes)");
        run(aiter_amd_moe_sorting_fwd(
            (const int32_t*)ids.ptr, (const float*)w.ptr, M, topk, (int32_t*)sid.ptr,
            (float*)sw.ptr, (int32_t*)se.ptr, (int32_t*)nv.ptr,
            std::min<int64_t>(sid.numel_, sw.numel_), se.numel_, buf.ptr, rb, num_experts,
            unit_size, (const int32_t*)ptr(mask), (const int32_t*)ptr(loc), dispatch_policy,
            ws ? buf.ptr : nullptr, ws ? M * rb : 0, stream));
    });
}

int dynamic_per_token_scaled_quant(aiter_tensor_t* out, aiter_tensor_t* input,
                                   aiter_tensor_t* scales, aiter_tensor_t* scale_ub,
                                   int shuffle_scale, aiter_tensor_t* num_rows,
                                   int64_t num_rows_factor, void* stream) {
    return safe_call([&] {
        const int dev = need(input, "input").device_id;
        const auto& x = tensor(input, "input", dev, {DT_BF16, DT_FP16});
        const auto& y = tensor(out, "out", dev, {DT_FP8});
        const auto& s = tensor(scales, "scales", dev, {DT_FP32});
        AMD_CHECK(scale_ub == nullptr, "scale_ub is not supported (only dynamic scales)");
        AMD_CHECK(x.ndim >= 1 && dim(x, -1) == 128,
                  "input must be viewed as [groups, 128]: only 1x128 group quant is provided");
        AMD_CHECK(y.ndim >= 1 && x.numel_ == y.numel_, "out must hold as many elements as input");
        const int64_t cols = dim(y, -1), rows = cols ? (int64_t)y.numel_ / cols : 0;
        AMD_CHECK(cols % 128 == 0, "out's last dimension must be a multiple of 128");
        check_numel(s, "scales", rows * (cols / 128));
        const auto* nr = optional(num_rows, "num_rows", dev, {DT_I32});
        DeviceGuard guard(dev);
        run(aiter_amd_dynamic_per_group_quant_fp8(x.ptr, x.dtype_, rows, cols, 128, y.ptr,
                                                  (float*)s.ptr, shuffle_scale != 0,
                                                  (const int32_t*)ptr(nr), num_rows_factor,
                                                  stream));
    });
}

int moe_stage1_g1u1(aiter_tensor_t* input, aiter_tensor_t* w1, aiter_tensor_t* w2,
                    aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids,
                    aiter_tensor_t* num_valid_ids, aiter_tensor_t* out, int64_t inter_dim,
                    const char* kernelName, int64_t block_m, int64_t ksplit, int64_t activation,
                    int64_t quant_type, aiter_tensor_t* a1_scale, aiter_tensor_t* w1_scale,
                    aiter_tensor_t* sorted_weights, void* stream) {
    (void)kernelName;
    (void)w2;
    return safe_call([&] {
        AMD_CHECK(quant_type == kQuantPer1x128,
                  "moe_stage1_g1u1: only QuantType.per_1x128 (fp8 blockscale) is provided, got " +
                      std::to_string(quant_type));
        AMD_CHECK(ksplit == 0, "ksplit must be 0: K splitting is chosen by the library");
        const int dev = need(input, "input").device_id;
        const auto& a = tensor(input, "input", dev, {DT_FP8});
        AMD_CHECK(a.ndim == 2, "input must be [tokens, model_dim]");
        const int64_t T = a.shape[0], H = a.shape[1], I = inter_dim;
        const auto& wt = tensor(w1, "w1", dev, {DT_FP8});
        AMD_CHECK(wt.ndim == 3 && wt.shape[1] == 2 * I && wt.shape[2] == H,
                  "w1 must be [E, 2*inter_dim, model_dim] (gate and up)");
        const int64_t E = wt.shape[0];
        const auto& ws = tensor(w1_scale, "w1_scale", dev, {DT_FP32});
        check_shape(ws, "w1_scale", {E, 2 * I / 128, H / 128});
        const auto& as = tensor(a1_scale, "a1_scale", dev, {DT_FP32});
        check_numel(as, "a1_scale", T * (H / 128));
        const auto& o = tensor(out, "out", dev, {DT_FP8});
        AMD_CHECK(o.ndim == 3 && o.shape[2] == I, "out must be [tokens + ceil(4 tokens / 128), "
                                                   "topk, inter_dim]");
        const int64_t topk = o.shape[1];
        check_shape(o, "out", {T + (4 * T + 127) / 128, topk, I});
        const auto& sid = tensor(sorted_token_ids, "sorted_token_ids", dev, {DT_I32});
        const auto& se = tensor(sorted_expert_ids, "sorted_expert_ids", dev, {DT_I32});
        const auto& nv = tensor(num_valid_ids, "num_valid_ids", dev, {DT_I32});
        const auto* sw = optional(sorted_weights, "sorted_weights", dev, {DT_FP32});
        DeviceGuard guard(dev);
        // codes in the first T rows, the f32 scales in the bytes after them
        uint8_t* a2 = (uint8_t*)o.ptr;
        float* a2s = reinterpret_cast<float*>(a2 + T * topk * I);
        run(aiter_amd_moe_stage1_fp8_blockscale(
            a.ptr, (const float*)as.ptr, 1, wt.ptr, (const float*)ws.ptr,
            (const int32_t*)sid.ptr, (const float*)ptr(sw), (const int32_t*)se.ptr,
            (const int32_t*)nv.ptr, a2, a2s, T, H, I, E, topk, block_m, se.numel_, activation, 1,
            stream));
    });
}

int ck_moe_stage2(aiter_tensor_t* inter_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids,
                  aiter_tensor_t* num_valid_ids, aiter_tensor_t* out, int64_t topk,
                  const char* kernelName, aiter_tensor_t* w2_scale, aiter_tensor_t* a2_scale,
                  int64_t block_m, aiter_tensor_t* sorted_weights, int64_t quant_type,
                  int64_t activation, int64_t splitk, int use_non_temporal_load,
                  const char* dst_type, int is_shuffled, void* stream) {
    (void)w1;
    (void)kernelName;
    (void)activation;
    (void)use_non_temporal_load;
    (void)dst_type;
    return safe_call([&] {
        AMD_CHECK(splitk == 0 || splitk == 1, "splitk must be 0 or 1 for stage 2");
        const int dev = need(inter_states, "inter_states").device_id;
        const auto& a = tensor(inter_states, "inter_states", dev, {DT_FP8});
        AMD_CHECK(a.ndim == 3 && a.shape[1] == topk, "inter_states must be [tokens, topk, "
                                                      "inter_dim]");
        const int64_t T = a.shape[0], I = a.shape[2];
        const auto& w = tensor(w2, "w2", dev, {DT_FP8, DT_FP4X2, DT_U8});
        AMD_CHECK(w.ndim == 3, "w2 must be [E, model_dim, inter_dim]");
        const bool w4 = w.dtype_ != DT_FP8;
        const int64_t E = w.shape[0], H = w.shape[1];
        AMD_CHECK(w.shape[2] == (w4 ? I / 2 : I), "w2's last dimension does not match inter_dim");
        AMD_CHECK(quant_type == (w4 ? kQuantPer1x32 : kQuantPer1x128),
                  w4 ? "fp4x2 w2 needs QuantType.per_1x32" : "fp8 w2 needs QuantType.per_1x128");
        const auto& ws = tensor(w2_scale, "w2_scale", dev,
                                w4 ? std::initializer_list<int>{DT_FP8_E8M0, DT_U8}
                                   : std::initializer_list<int>{DT_FP32});
        if (w4)
            check_shape(ws, "w2_scale", {E, H, I / 32});
        else
            check_shape(ws, "w2_scale", {E, H / 128, I / 128});
        const auto& as = tensor(a2_scale, "a2_scale", dev, {DT_FP32});
        check_numel(as, "a2_scale", T * topk * (I / 128));
        const auto& o = tensor(out, "out", dev, {DT_BF16, DT_FP16, DT_FP32});
        check_shape(o, "out", {T, H});
        const auto& sid = tensor(sorted_token_ids, "sorted_token_ids", dev, {DT_I32});
        const auto& se = tensor(sorted_expert_ids, "sorted_expert_ids", dev, {DT_I32});
        const auto& nv = tensor(num_valid_ids, "num_valid_ids", dev, {DT_I32});
        const auto* sw = optional(sorted_weights, "sorted_weights", dev, {DT_FP32});
        DeviceGuard guard(dev);
        if (w4)
            run(aiter_amd_moe_stage2_a8w4(
                a.ptr, (const float*)as.ptr, w.ptr, (const uint8_t*)ws.ptr,
                (const int32_t*)sid.ptr, (const float*)ptr(sw), (const int32_t*)se.ptr,
                (const int32_t*)nv.ptr, o.ptr, o.dtype_, T, H, I, E, topk, block_m, se.numel_,
                is_shuffled != 0, stream));
        else
            run(aiter_amd_moe_stage2_fp8_blockscale(
                a.ptr, (const float*)as.ptr, w.ptr, (const float*)ws.ptr,
                (const int32_t*)sid.ptr, (const float*)ptr(sw), (const int32_t*)se.ptr,
                (const int32_t*)nv.ptr, o.ptr, o.dtype_, T, H, I, E, topk, block_m, se.numel_,
                is_shuffled != 0, stream));
    });
}

int ck_moe_stage1(aiter_tensor_t* hidden_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids,
                  aiter_tensor_t* num_valid_ids, aiter_tensor_t* out, int64_t topk,
                  const char* kernelName, aiter_tensor_t* w1_scale, aiter_tensor_t* a1_scale,
                  int64_t block_m, aiter_tensor_t* sorted_weights, int64_t quant_type,
                  int64_t activation, int64_t splitk, int use_non_temporal_load,
                  const char* dst_type, int is_shuffled, void* stream) {
    (void)w2;
    (void)kernelName;
    (void)use_non_temporal_load;
    (void)dst_type;
    return safe_call([&] {
        const int dev = need(hidden_states, "hidden_states").device_id;
        const auto& a = tensor(hidden_states, "hidden_states", dev, {DT_FP8});
        AMD_CHECK(a.ndim == 2, "hidden_states must be [tokens, model_dim]");
        const int64_t T = a.shape[0], H = a.shape[1];
        const auto& w = tensor(w1, "w1", dev, {DT_FP8, DT_FP4X2, DT_U8});
        AMD_CHECK(w.ndim == 3 && w.shape[1] % 2 == 0, "w1 must be [E, 2*inter_dim, model_dim]");
        const bool w4 = w.dtype_ != DT_FP8;
        const int64_t E = w.shape[0], I = w.shape[1] / 2;
        AMD_CHECK(w.shape[2] == (w4 ? H / 2 : H), "w1's last dimension does not match model_dim");
        AMD_CHECK(quant_type == (w4 ? kQuantPer1x32 : kQuantPer1x128),
                  w4 ? "fp4x2 w1 needs QuantType.per_1x32 (fp8 1x128 activations)"
                     : "fp8 w1 needs QuantType.per_1x128");
        const auto& ws = tensor(w1_scale, "w1_scale", dev,
                                w4 ? std::initializer_list<int>{DT_FP8_E8M0, DT_U8}
                                   : std::initializer_list<int>{DT_FP32});
        if (w4)
            check_shape(ws, "w1_scale", {E, 2 * I, H / 32});
        else
            check_shape(ws, "w1_scale", {E, 2 * I / 128, H / 128});
        const auto& as = tensor(a1_scale, "a1_scale", dev, {DT_FP32});
        check_numel(as, "a1_scale", T * (H / 128));
        const bool split = splitk > 1;
        const auto& o = tensor(out, "out", dev,
                               split ? std::initializer_list<int>{DT_FP32}
                                     : std::initializer_list<int>{DT_BF16, DT_FP16});
        if (split) {
            AMD_CHECK(o.ndim == 2 && o.shape[1] == 2 * I && o.shape[0] >= T * topk,
                      "with splitk > 1, out must be fp32 [>= tokens*topk, 2*inter_dim]");
        } else {
            AMD_CHECK(o.ndim >= 1 && dim(o, -1) == I && (int64_t)o.numel_ == T * topk * I,
                      "out must be [tokens, topk, inter_dim] (or [tokens*topk, inter_dim])");
        }
        const auto& sid = tensor(sorted_token_ids, "sorted_token_ids", dev, {DT_I32});
        const auto& se = tensor(sorted_expert_ids, "sorted_expert_ids", dev, {DT_I32});
        const auto& nv = tensor(num_valid_ids, "num_valid_ids", dev, {DT_I32});
        check_numel(nv, "num_valid_ids", 2);
        const auto* sw = optional(sorted_weights, "sorted_weights", dev, {DT_FP32});
        AMD_CHECK(block_m == 16 || block_m == 32 || block_m == 64 || block_m == 128,
                  "block_m must be 16, 32, 64 or 128, got " + std::to_string(block_m));
        AMD_CHECK(activation == kActSilu || activation == kActGelu,
                  "only ActivationType.Silu (0) and Gelu (1) are supported, got " +
                      std::to_string(activation));
        AMD_CHECK(H % 128 == 0 && (!split || (H / 128) % splitk == 0),
                  "ksplit must divide model_dim / 128 = " + std::to_string(H / 128) + ", got " +
                      std::to_string(splitk));
        DeviceGuard guard(dev);
        run(aiter_amd_moe_stage1_rows(
            a.ptr, (const float*)as.ptr, 0, w.ptr, w4 ? nullptr : (const float*)ws.ptr,
            w4 ? (const uint8_t*)ws.ptr : nullptr, (const int32_t*)sid.ptr,
            (const float*)ptr(sw), (const int32_t*)se.ptr, (const int32_t*)nv.ptr, o.ptr,
            split ? kOutGateUp : kOutAct, o.dtype_, T, H, I, E, topk, block_m, se.numel_,
            activation, split ? splitk : 0, is_shuffled != 0, stream));
    });
}

static int act_and_mul(aiter_tensor_t* out, aiter_tensor_t* input, int act, void* stream) {
    return safe_call([&] {
        const int dev = need(input, "input").device_id;
        const auto& x = tensor(input, "input", dev, {DT_FP32, DT_BF16, DT_FP16});
        const auto& y = tensor(out, "out", dev, {DT_FP32, DT_BF16, DT_FP16});
        AMD_CHECK(x.ndim >= 1 && y.ndim >= 1, "input and out need a last dimension");
        const int64_t d = dim(y, -1);
        AMD_CHECK(dim(x, -1) == 2 * d, "input's last dimension must be twice out's");
        AMD_CHECK((int64_t)x.numel_ == 2 * (int64_t)y.numel_,
                  "input and out must hold the same rows");
        const int64_t rows = d ? (int64_t)y.numel_ / d : 0;
        DeviceGuard guard(dev);
        run(aiter_amd_act_and_mul(x.ptr, x.dtype_, y.ptr, y.dtype_, rows, d, act, stream));
    });
}

int silu_and_mul(aiter_tensor_t* out, aiter_tensor_t* input, void* stream) {
    return act_and_mul(out, input, kActSilu, stream);
}

int gelu_and_mul(aiter_tensor_t* out, aiter_tensor_t* input, void* stream) {
    return act_and_mul(out, input, kActGelu, stream);
}

int fmoe_fp8_blockscale_g1u1(aiter_tensor_t* out, aiter_tensor_t* input, aiter_tensor_t* gate,
                             aiter_tensor_t* down, aiter_tensor_t* sorted_token_ids,
                             aiter_tensor_t* sorted_weights, aiter_tensor_t* sorted_expert_ids,
                             aiter_tensor_t* num_valid_ids, int64_t topk,
                             aiter_tensor_t* input_scale, aiter_tensor_t* fc1_scale,
                             aiter_tensor_t* fc2_scale, const char* kernel_name,
                             int64_t fc_scale_blkn, int64_t fc_scale_blkk,
                             aiter_tensor_t* fc2_smooth_scale, int64_t activation,
                             int64_t block_size_M, void* stream) {
    (void)kernel_name;
    return safe_call([&] {
        AMD_CHECK(fc_scale_blkn == 128 && fc_scale_blkk == 128,
                  "fmoe_fp8_blockscale_g1u1: only 128x128 weight scale blocks are supported");
        AMD_CHECK(fc2_smooth_scale == nullptr, "fc2_smooth_scale is not supported");
        const int dev = need(input, "input").device_id;
        const auto& a = tensor(input, "input", dev, {DT_FP8});
        AMD_CHECK(a.ndim == 2, "input must be [tokens, model_dim]");
        const int64_t T = a.shape[0], H = a.shape[1];
        const auto& w1 = tensor(gate, "gate", dev, {DT_FP8});
        AMD_CHECK(w1.ndim == 3 && w1.shape[2] == H && w1.shape[1] % 2 == 0,
                  "gate must be [E, 2*inter_dim, model_dim] fp8");
        const int64_t E = w1.shape[0], I = w1.shape[1] / 2;
        const auto& w2 = tensor(down, "down", dev, {DT_FP8});
        check_shape(w2, "down", {E, H, I});
        const auto& s1 = tensor(fc1_scale, "fc1_scale", dev, {DT_FP32});
        check_numel(s1, "fc1_scale", E * (2 * I / 128) * (H / 128));
        const auto& s2 = tensor(fc2_scale, "fc2_scale", dev, {DT_FP32});
        check_numel(s2, "fc2_scale", E * (H / 128) * (I / 128));
        const auto& as = tensor(input_scale, "input_scale", dev, {DT_FP32});
        check_numel(as, "input_scale", T * (H / 128));
        const auto& o = tensor(out, "out", dev, {DT_BF16, DT_FP16});
        check_shape(o, "out", {T, H});
        const auto& sid = tensor(sorted_token_ids, "sorted_token_ids", dev, {DT_I32});
        const auto& sw = tensor(sorted_weights, "sorted_weights", dev, {DT_FP32});
        const auto& se = tensor(sorted_expert_ids, "sorted_expert_ids", dev, {DT_I32});
        const auto& nv = tensor(num_valid_ids, "num_valid_ids", dev, {DT_I32});
        check_numel(nv, "num_valid_ids", 2);
        AMD_CHECK(block_size_M >= 1 && block_size_M <= 256,
                  "block_size_M must be the sorting's block size, in [1, 256]");
        AMD_CHECK(topk >= 1 && topk <= 32, "topk must be in [1, 32]");
        AMD_CHECK(activation == kActSilu || activation == kActGelu,
                  "only ActivationType.Silu (0) and Gelu (1) are supported, got " +
                      std::to_string(activation));
        const int64_t cap = std::min<int64_t>(sid.numel_, sw.numel_);
        AMD_CHECK((int64_t)se.numel_ >= ceil_div(cap, block_size_M),
                  "sorted_expert_ids holds fewer blocks than sorted_token_ids needs");
        // the router's expert count, from moe_sorting's capacity
        // tokens*topk + experts*block - topk (a block-size hint only)
        const int64_t G = std::min<int64_t>(
            std::max<int64_t>((cap - T * topk + topk) / block_size_M, E), 4096);
        DeviceGuard guard(dev);
        const int64_t need_bytes =
            aiter_amd_fused_moe_sorted_workspace_bytes(T, H, I, E, G, topk);
        AMD_CHECK(need_bytes >= 0, "invalid layer dimensions");
        void* ws = T ? pooled_workspace(dev, stream, need_bytes, "fmoe_fp8_blockscale_g1u1")
                     : nullptr;
        // the asm kernel this replaces reads (16,16)-shuffled weights and the
        // transposed [model_dim/128, tokens] activation scales
        run(aiter_amd_fused_moe_sorted_fp8_blockscale(
            a.ptr, (const float*)as.ptr, 1, w1.ptr, (const float*)s1.ptr, w2.ptr,
            (const float*)s2.ptr, (const int32_t*)sid.ptr, (const float*)sw.ptr,
            (const int32_t*)se.ptr, (const int32_t*)nv.ptr, cap, block_size_M, o.ptr, o.dtype_, T,
            H, I, E, G, topk, activation, 1, ws, need_bytes, stream));
    });
}

// Routing: outputs may be row-strided views (the reference's kernels take
// the row stride of topk_weights / topk_ids); the gating rows are contiguous.
static void route_outputs(const aiter_tensor_t* w, const aiter_tensor_t* ids, int dev,
                          int64_t& M, int64_t& k) {
    const auto& tw = need(w, "topk_weights");
    const auto& ti = need(ids, "topk_ids");
    check_dtype(tw, "topk_weights", {DT_FP32});
    check_dtype(ti, "topk_ids", {DT_I32});
    check_device(tw, dev, "topk_weights");
    check_device(ti, dev, "topk_ids");
    AMD_CHECK(tw.ndim == 2 && ti.ndim == 2 && tw.shape[0] == ti.shape[0] &&
                  tw.shape[1] == ti.shape[1],
              "topk_weights and topk_ids must both be [M, topk]");
    AMD_CHECK(tw.strides[1] == 1 && ti.strides[1] == 1,
              "topk_weights / topk_ids rows must be contiguous");
    M = tw.shape[0];
    k = tw.shape[1];
}

static const aiter_tensor_t& gating(const aiter_tensor_t* g, int64_t M) {
    const auto& x = need(g, "gating_output");
    check_dtype(x, "gating_output", {DT_FP32, DT_BF16, DT_FP16});
    check_contig(x, "gating_output");
    AMD_CHECK(x.ndim == 2 && x.shape[0] == M, "gating_output must be [M, num_experts]");
    return x;
}

int topk_softmax(aiter_tensor_t* topk_weights, aiter_tensor_t* topk_indices,
                 aiter_tensor_t* token_expert_indices, aiter_tensor_t* gating_output,
                 int need_renorm, int64_t num_shared_experts,
                 const char* shared_expert_scoring_func, void* stream) {
    return safe_call([&] {
        const bool func = shared_expert_scoring_func && shared_expert_scoring_func[0];
        AMD_CHECK(num_shared_experts >= 0, "num_shared_experts must be >= 0");
        AMD_CHECK(!func || std::string(shared_expert_scoring_func) == "sigmoid",
                  std::string("Only 'sigmoid' scoring function is supported for shared experts, "
                              "got: ") + (func ? shared_expert_scoring_func : ""));
        AMD_CHECK(num_shared_experts == 0 || func,
                  "num_shared_experts > 0 needs shared_expert_scoring_func 'sigmoid'");
        const int dev = need(gating_output, "gating_output").device_id;
        const auto& tiw = need(topk_weights, "topk_weights");
        const auto& tii = need(topk_indices, "topk_indices");
        check_dtype(tiw, "topk_weights", {DT_FP32});
        check_dtype(tii, "topk_indices", {DT_I32});
        check_device(tiw, dev, "topk_weights");
        check_device(tii, dev, "topk_indices");
        // topk_weights [M, topk + shared], topk_indices [M, topk]
        AMD_CHECK(tiw.ndim == 2 && tii.ndim == 2 && tiw.shape[0] == tii.shape[0] &&
                      tiw.shape[1] == tii.shape[1] + num_shared_experts,
                  "topk_weights must be [M, topk + num_shared_experts] and topk_indices "
                  "[M, topk]");
        AMD_CHECK(tiw.strides[1] == 1 && tii.strides[1] == 1,
                  "topk_weights / topk_indices rows must be contiguous");
        const int64_t M = tii.shape[0], k = tii.shape[1];
        const auto& x = gating(gating_output, M);
        AMD_CHECK(x.shape[1] > num_shared_experts,
                  "gating_output must hold the routed experts, then the shared ones");
        const auto* tei = optional(token_expert_indices, "token_expert_indices", dev, {DT_I32});
        if (tei) check_shape(*tei, "token_expert_indices", {M, k});
        DeviceGuard guard(dev);
        run(aiter_amd_topk_softmax_shared(
            x.ptr, x.dtype_, M, x.shape[1] - num_shared_experts, num_shared_experts, k,
            (float*)tiw.ptr, tiw.strides[0], (int32_t*)tii.ptr, tii.strides[0],
            (int32_t*)(tei ? tei->ptr : nullptr), need_renorm, stream));
    });
}

int topk_sigmoid(aiter_tensor_t* topk_weights, aiter_tensor_t* topk_indices,
                 aiter_tensor_t* gating_output, void* stream) {
    return safe_call([&] {
        const int dev = need(gating_output, "gating_output").device_id;
        int64_t M, k;
        route_outputs(topk_weights, topk_indices, dev, M, k);
        const auto& x = gating(gating_output, M);
        DeviceGuard guard(dev);
        run(aiter_amd_topk_sigmoid(x.ptr, x.dtype_, M, x.shape[1], k, (float*)topk_weights->ptr,
                                   topk_weights->strides[0], (int32_t*)topk_indices->ptr,
                                   topk_indices->strides[0], stream));
    });
}

int grouped_topk(aiter_tensor_t* gating_output, aiter_tensor_t* topk_weights,
                 aiter_tensor_t* topk_ids, int64_t num_expert_group, int64_t topk_group,
                 int need_renorm, int is_softmax, float routed_scaling_factor, void* stream) {
    return safe_call([&] {
        const int dev = need(gating_output, "gating_output").device_id;
        int64_t M, k;
        route_outputs(topk_weights, topk_ids, dev, M, k);
        const auto& x = gating(gating_output, M);
        DeviceGuard guard(dev);
        run(aiter_amd_grouped_topk(x.ptr, x.dtype_, nullptr, M, x.shape[1], k, num_expert_group,
                                   topk_group, need_renorm, is_softmax, routed_scaling_factor,
                                   (float*)topk_weights->ptr, topk_weights->strides[0],
                                   (int32_t*)topk_ids->ptr, topk_ids->strides[0], stream));
    });
}

int biased_grouped_topk(aiter_tensor_t* gating_output, aiter_tensor_t* correction_bias,
                        aiter_tensor_t* topk_weights, aiter_tensor_t* topk_ids,
                        int64_t num_expert_group, int64_t topk_grp, int need_renorm,
                        float routed_scaling_factor, void* stream) {
    return safe_call([&] {
        const int dev = need(gating_output, "gating_output").device_id;
        int64_t M, k;
        route_outputs(topk_weights, topk_ids, dev, M, k);
        const auto& x = gating(gating_output, M);
        const auto& b = tensor(correction_bias, "correction_bias", dev, {DT_FP32});
        check_shape(b, "correction_bias", {x.shape[1]});
        DeviceGuard guard(dev);
        run(aiter_amd_grouped_topk(x.ptr, x.dtype_, (const float*)b.ptr, M, x.shape[1], k,
                                   num_expert_group, topk_grp, need_renorm, 0,
                                   routed_scaling_factor, (float*)topk_weights->ptr,
                                   topk_weights->strides[0], (int32_t*)topk_ids->ptr,
                                   topk_ids->strides[0], stream));
    });
}

}  // extern "C"
