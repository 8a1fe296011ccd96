// Per-token-group (1 x 128) dynamic FP8 e4m3fn quantisation of activations,
// and the fp32 -> bf16/fp16 conversion that finishes the down GEMM.
//
// Quantisation semantics follow the reference HIP kernel
// (csrc/kernels/quant_kernels.cu:16-133, host 710-757):
//   amax  = max(1e-10, max |x|) over the 128-element group
//   scale = amax * fp32(1/448)
//   q     = e4m3fn_rne(clamp(x * fp32(1/scale), -448, 448))
// The scale is stored row-major [rows, cols/128], or transposed
// [cols/128, rows] when transpose_scale is set (quant_kernels.cu:118-121).
// When num_rows is given (a device scalar), only *num_rows * num_rows_factor
// rows are processed (quant_kernels.cu:32-35).
//
// MI355X layout: 16 lanes x 8 elements (one 16-byte load each) cover a
// group; a 256-thread block quantises 16 groups; the group amax is a 4-step
// xor-shuffle inside the 16-lane quarter of the wave.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "quant_dev.h"

namespace aiter_amd {

template <bool kBf16>
__global__ __launch_bounds__(kQuantThreads) void per_group_quant_fp8_kernel(
    const uint16_t* __restrict__ x, uint8_t* __restrict__ q, float* __restrict__ scale,
    int64_t rows, int cols, int transpose_scale, const int32_t* __restrict__ num_rows,
    int num_rows_factor) {
    quant_groups_block<kBf16>(x, q, scale, rows, cols, transpose_scale, num_rows,
                              num_rows_factor, (int64_t)blockIdx.x);
}

void launch_per_group_quant_fp8(const void* x, int x_dtype, void* q, float* scale, int64_t rows,
                                int64_t cols, int transpose_scale, const int32_t* num_rows,
                                int64_t num_rows_factor, hipStream_t stream) {
    const int64_t groups = rows * (cols / 128);
    if (groups == 0) return;
    const int64_t blocks = ceil_div(groups, kQuantThreads / 16);
    AMD_CHECK(blocks < (1ll << 31), "too many rows");
    if (x_dtype == DT_BF16)
        hipLaunchKernelGGL(per_group_quant_fp8_kernel<true>, dim3((unsigned)blocks),
                           dim3(kQuantThreads), 0, stream, (const uint16_t*)x, (uint8_t*)q, scale,
                           rows, (int)cols, transpose_scale, num_rows, (int)num_rows_factor);
    else
        hipLaunchKernelGGL(per_group_quant_fp8_kernel<false>, dim3((unsigned)blocks),
                           dim3(kQuantThreads), 0, stream, (const uint16_t*)x, (uint8_t*)q, scale,
                           rows, (int)cols, transpose_scale, num_rows, (int)num_rows_factor);
    AMD_HIP_CHECK(hipGetLastError());
}

// ------------------------------------------- fp32 accumulator -> output ---
template <bool kBf16>
__device__ __forceinline__ float to_f32(uint16_t b) {
    return kBf16 ? bf16_bits_to_f32(b) : fp16_bits_to_f32(b);
}

// a[0..7] += the 8 bf16 / fp16 values at p (16-byte aligned)
template <bool kBf16>
__device__ __forceinline__ void add_row8(float (&a)[8], const uint16_t* p) {
    const v4i o = *reinterpret_cast<const v4i*>(p);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        a[2 * e] += to_f32<kBf16>((uint16_t)((uint32_t)o[e] & 0xFFFFu));
        a[2 * e + 1] += to_f32<kBf16>((uint16_t)((uint32_t)o[e] >> 16));
    }
}

// out[r, :] = round(acc[r, :] (+ addend[r, :])) for r < tokens (tokens =
// *num_valid[1]); 8 elements per thread. addend may alias out: each thread
// reads its own 8 elements before writing them.
template <bool kBf16>
__global__ __launch_bounds__(256) void acc_to_out_kernel(const float* __restrict__ acc,
                                                         uint16_t* out,
                                                         const int32_t* __restrict__ num_valid,
                                                         int64_t rows, int cols,
                                                         const uint16_t* addend) {
    int64_t tokens = num_valid ? (int64_t)num_valid[1] : rows;
    tokens = tokens < rows ? tokens : rows;
    const int64_t n8 = tokens * cols / 8;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8;
         i += (int64_t)gridDim.x * 256) {
        v4f a = *reinterpret_cast<const v4f*>(acc + i * 8);
        v4f b = *reinterpret_cast<const v4f*>(acc + i * 8 + 4);
        if (addend) {
            const v4i o = *reinterpret_cast<const v4i*>(addend + i * 8);
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                a[2 * e] += to_f32<kBf16>((uint16_t)((uint32_t)o[e] & 0xFFFFu));
                a[2 * e + 1] += to_f32<kBf16>((uint16_t)((uint32_t)o[e] >> 16));
                b[2 * e] += to_f32<kBf16>((uint16_t)((uint32_t)o[2 + e] & 0xFFFFu));
                b[2 * e + 1] += to_f32<kBf16>((uint16_t)((uint32_t)o[2 + e] >> 16));
            }
        }
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float x0 = a[2 * j], x1 = a[2 * j + 1];
            float y0 = b[2 * j], y1 = b[2 * j + 1];
            if (kBf16) {
                w[j] = f32_to_bf16_bits(x0) | ((uint32_t)f32_to_bf16_bits(x1) << 16);
                w[2 + j] = f32_to_bf16_bits(y0) | ((uint32_t)f32_to_bf16_bits(y1) << 16);
            } else {
                w[j] = f32_to_fp16_bits(x0) | ((uint32_t)f32_to_fp16_bits(x1) << 16);
                w[2 + j] = f32_to_fp16_bits(y0) | ((uint32_t)f32_to_fp16_bits(y1) << 16);
            }
        }
        v4i o = {(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        *reinterpret_cast<v4i*>(out + i * 8) = o;
    }
}

void launch_acc_to_out(const float* acc, void* out, int out_dtype, const int32_t* num_valid,
                       int64_t rows, int64_t cols, hipStream_t stream, const void* addend) {
    const int64_t n8 = rows * cols / 8;
    if (n8 == 0) return;
    const int blocks = (int)std::min<int64_t>(ceil_div(n8, 256), 8192);
    if (out_dtype == DT_BF16)
        hipLaunchKernelGGL(acc_to_out_kernel<true>, dim3(blocks), dim3(256), 0, stream, acc,
                           (uint16_t*)out, num_valid, rows, (int)cols, (const uint16_t*)addend);
    else
        hipLaunchKernelGGL(acc_to_out_kernel<false>, dim3(blocks), dim3(256), 0, stream, acc,
                           (uint16_t*)out, num_valid, rows, (int)cols, (const uint16_t*)addend);
    AMD_HIP_CHECK(hipGetLastError());
}

// ------------------------------------ per-pair bf16 rows -> output ---
// out[t, :] = round(sum over the token's routed slots j of part[t*topk + j, :])
// for t < tokens (= *num_valid[1]), summed in fp32 in slot order. A slot is
// routed when sorting kept its pair: expert id in [0, num_experts) and, with
// an expert mask, mask[id] != 0. topk <= 32. The token's valid slots are
// checked once (lane j checks slot j; a ballot gives the bit mask).
//
// slot_sum_kernel: one token per workgroup; each lane sums two 8-column
// pieces of a 4096-column row in one pass, the loads of 8 slots of both
// pieces in flight before any sum.
template <bool kBf16>
__global__ __launch_bounds__(256) void slot_sum_kernel(const uint16_t* __restrict__ part,
                                                       const int32_t* __restrict__ topk_ids,
                                                       const int32_t* __restrict__ mask,
                                                       int num_experts,
                                                       const int32_t* __restrict__ num_valid,
                                                       uint16_t* out, int64_t rows,
                                                       int topk, int cols,
                                                       const uint16_t* addend) {
    int64_t tokens = (int64_t)num_valid[1];
    tokens = tokens < rows ? tokens : rows;
    const int c8 = cols / 8;
    const int lane = threadIdx.x & 63;
    constexpr int kSpan = 256;                          // lanes that share a token
    const int tl = (int)threadIdx.x;
    for (int64_t t = (int64_t)blockIdx.x; t < tokens; t += (int64_t)gridDim.x) {
        int ok = 0;
        if (lane < topk) {
            const int id = topk_ids[t * topk + lane];
            ok = id >= 0 && id < num_experts && (!mask || mask[id] != 0);
        }
        const uint32_t valid = (uint32_t)__builtin_amdgcn_ballot_w64(ok);
        const uint16_t* src = part + t * topk * (int64_t)cols;
        for (int c0 = tl; c0 < c8; c0 += 2 * kSpan) {
            const int cc[2] = {c0, c0 + kSpan};
            float a[2][8] = {};
            for (int j0 = 0; j0 < topk; j0 += 8) {
                v4i v[2][8];
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int j = j0 + u;
                        v[h][u] = v4i{0, 0, 0, 0};
                        if (cc[h] < c8 && j < topk && ((valid >> j) & 1u))
                            v[h][u] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(
                                src + (int64_t)j * cols + cc[h] * 8));
                    }
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int j = j0 + u;
                        if (j >= topk || !((valid >> j) & 1u)) continue;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            a[h][2 * e] += bf16_bits_to_f32((uint16_t)((uint32_t)v[h][u][e] & 0xFFFFu));
                            a[h][2 * e + 1] += bf16_bits_to_f32((uint16_t)((uint32_t)v[h][u][e] >> 16));
                        }
                    }
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                if (cc[h] >= c8) continue;
                if (addend) add_row8<kBf16>(a[h], addend + t * cols + cc[h] * 8);
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[e] = kBf16 ? f32_to_bf16_bits(a[h][2 * e]) |
                                       ((uint32_t)f32_to_bf16_bits(a[h][2 * e + 1]) << 16)
                                 : f32_to_fp16_bits(a[h][2 * e]) |
                                       ((uint32_t)f32_to_fp16_bits(a[h][2 * e + 1]) << 16);
                *reinterpret_cast<v4i*>(out + t * cols + cc[h] * 8) =
                    v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            }
        }
    }
}

// slot_sum_wave_kernel: one token per wave, four per workgroup, so the short
// id -> mask -> row chains of an expert-parallel share's rows (about one
// routed slot in eight) overlap. Each lane holds kPieces 8-column pieces of
// the row (a 4096-column row in one pass) and, slot by slot in slot order,
// issues all of a slot's piece loads before summing them. Measured on MI355X,
// EP share (32 of 256 experts, 64-row blocks): T=4096 20.0 -> 18.9 us, T=2048
// 14.7 -> 13.7 us against two pieces per pass (the per-workgroup kernel took
// 21 us); 4 pieces per lane (two passes, 92 instead of 168 VGPRs) 20.5 us.
template <bool kBf16>
__global__ __launch_bounds__(256) void slot_sum_wave_kernel(
    const uint16_t* __restrict__ part, const int32_t* __restrict__ topk_ids,
    const int32_t* __restrict__ mask, int num_experts, const int32_t* __restrict__ num_valid,
    uint16_t* out, int64_t rows, int topk, int cols, const uint16_t* addend) {
    constexpr int kPieces = 8;
    int64_t tokens = (int64_t)num_valid[1];
    tokens = tokens < rows ? tokens : rows;
    const int c8 = cols / 8;
    const int lane = threadIdx.x & 63;
    for (int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); t < tokens;
         t += (int64_t)gridDim.x * 4) {
        int ok = 0;
        if (lane < topk) {
            const int id = topk_ids[t * topk + lane];
            ok = id >= 0 && id < num_experts && (!mask || mask[id] != 0);
        }
        const uint32_t valid = (uint32_t)__builtin_amdgcn_ballot_w64(ok);
        const uint16_t* src = part + t * topk * (int64_t)cols;
        for (int base = lane; base < c8; base += 64 * kPieces) {
            float a[kPieces][8] = {};
            uint32_t m = valid;
            while (m != 0) {
                const int j = __builtin_ctz(m);
                m &= m - 1;
                v4i v[kPieces];
#pragma unroll
                for (int i = 0; i < kPieces; ++i) {
                    const int cc = base + 64 * i;
                    v[i] = v4i{0, 0, 0, 0};
                    if (cc < c8)
                        v[i] = __builtin_nontemporal_load(
                            reinterpret_cast<const v4i*>(src + (int64_t)j * cols + cc * 8));
                }
#pragma unroll
                for (int i = 0; i < kPieces; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        a[i][2 * e] += bf16_bits_to_f32((uint16_t)((uint32_t)v[i][e] & 0xFFFFu));
                        a[i][2 * e + 1] += bf16_bits_to_f32((uint16_t)((uint32_t)v[i][e] >> 16));
                    }
            }
#pragma unroll
            for (int i = 0; i < kPieces; ++i) {
                const int cc = base + 64 * i;
                if (cc >= c8) continue;
                if (addend) add_row8<kBf16>(a[i], addend + t * cols + cc * 8);
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    w[e] = kBf16 ? f32_to_bf16_bits(a[i][2 * e]) |
                                       ((uint32_t)f32_to_bf16_bits(a[i][2 * e + 1]) << 16)
                                 : f32_to_fp16_bits(a[i][2 * e]) |
                                       ((uint32_t)f32_to_fp16_bits(a[i][2 * e + 1]) << 16);
                *reinterpret_cast<v4i*>(out + t * cols + cc * 8) =
                    v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            }
        }
    }
}

void launch_slot_sum(const uint16_t* part, const int32_t* topk_ids, const int32_t* mask,
                     int64_t num_experts, const int32_t* num_valid, void* out, int out_dtype,
                     int64_t rows, int64_t topk, int64_t cols, hipStream_t stream,
                     const void* addend) {
    if (rows == 0 || cols == 0) return;
    // an expert mask means an expert-parallel share: most slots are not routed here
    const bool per_wave = mask != nullptr;
    const int blocks = (int)std::min<int64_t>(ceil_div(rows, per_wave ? 4 : 1), 8192);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, stream, part, topk_ids, mask,
                           (int)num_experts, num_valid, (uint16_t*)out, rows, (int)topk,
                           (int)cols, (const uint16_t*)addend);
    };
    if (out_dtype == DT_BF16)
        per_wave ? go(slot_sum_wave_kernel<true>) : go(slot_sum_kernel<true>);
    else
        per_wave ? go(slot_sum_wave_kernel<false>) : go(slot_sum_kernel<false>);
    AMD_HIP_CHECK(hipGetLastError());
}

// ------------------------------------------- act(gate) * up of fp32 rows ---
// out[r, c] = act(x[r, c]) * x[r, d + c] for c < d: the gate | up rows of a
// split-K stage 1 finished into the activation's output (the reference's
// silu_and_mul / gelu_and_mul, csrc/kernels/activation_kernels.cu:24-90,
// 337-354). Computed in fp32, rounded once to the output dtype. Rows of x
// are 2d wide, rows of out d wide; 4 elements per thread when d % 4 == 0.
template <typename TI>
__device__ __forceinline__ float load_f32(const TI* p, int64_t i) {
    if constexpr (sizeof(TI) == 4)
        return p[i];
    else if constexpr (std::is_same_v<TI, __bf16>)
        return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
    else
        return fp16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[i]);
}

template <typename TO>
__device__ __forceinline__ void store_f32(TO* p, int64_t i, float v) {
    if constexpr (sizeof(TO) == 4)
        p[i] = v;
    else if constexpr (std::is_same_v<TO, __bf16>)
        reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
    else
        reinterpret_cast<uint16_t*>(p)[i] = f32_to_fp16_bits(v);
}

template <typename TI, typename TO, int ACT>
__global__ __launch_bounds__(256) void act_and_mul_kernel(const TI* __restrict__ x,
                                                          TO* __restrict__ out, int64_t rows,
                                                          int d) {
    const int64_t n = rows * d;
    for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < n;
         i += (int64_t)gridDim.x * 256 * 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t j = i + u;
            if (j >= n) break;
            const int64_t r = j / d;
            const int64_t c = j - r * d;
            const float g = load_f32(x, r * 2 * d + c);
            const float up = load_f32(x, r * 2 * d + d + c);
            store_f32(out, j, (ACT == kActGelu ? gelu_f32(g) : silu_f32(g)) * up);
        }
    }
}

void launch_act_and_mul(const void* in, int in_dtype, void* out, int out_dtype, int64_t rows,
                        int64_t d, int act, hipStream_t stream) {
    const int64_t n = rows * d;
    if (n == 0) return;
    const int blocks = (int)std::min<int64_t>(ceil_div(n, 1024), 16384);
    auto go = [&](auto ti, auto to) {
        using TI = decltype(ti);
        using TO = decltype(to);
        if (act == kActGelu)
            hipLaunchKernelGGL((act_and_mul_kernel<TI, TO, kActGelu>), dim3(blocks), dim3(256),
                               0, stream, (const TI*)in, (TO*)out, rows, (int)d);
        else
            hipLaunchKernelGGL((act_and_mul_kernel<TI, TO, kActSilu>), dim3(blocks), dim3(256),
                               0, stream, (const TI*)in, (TO*)out, rows, (int)d);
    };
    auto with_out = [&](auto ti) {
        if (out_dtype == DT_FP32)
            go(ti, float{});
        else if (out_dtype == DT_BF16)
            go(ti, __bf16{});
        else
            go(ti, _Float16{});
    };
    if (in_dtype == DT_FP32)
        with_out(float{});
    else if (in_dtype == DT_BF16)
        with_out(__bf16{});
    else
        with_out(_Float16{});
    AMD_HIP_CHECK(hipGetLastError());
}

// ------------------------------------------------------------- zero fill ---
// A kernel, not hipMemsetAsync: the memory may be cleared inside a captured
// HIP graph.
__global__ __launch_bounds__(256) void zero_kernel(v4i* __restrict__ p, int64_t n16) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16;
         i += (int64_t)gridDim.x * 256)
        p[i] = v4i{0, 0, 0, 0};
}

void launch_zero(void* p, int64_t bytes, hipStream_t stream) {
    AMD_CHECK(bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0,
              "zero fill needs 16-byte aligned memory and size");
    const int64_t n16 = bytes / 16;
    if (n16 == 0) return;
    const int blocks = (int)std::min<int64_t>(ceil_div(n16, 256), 8192);
    hipLaunchKernelGGL(zero_kernel, dim3(blocks), dim3(256), 0, stream, (v4i*)p, n16);
    AMD_HIP_CHECK(hipGetLastError());
}

}  // namespace aiter_amd
