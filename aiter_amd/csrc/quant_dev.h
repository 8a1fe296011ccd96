// 1 x 128 FP8 quantisation of one 256-thread block's 16 groups: the body of
// per_group_quant_fp8_kernel, shared with the sorting launch (which runs it
// in extra blocks at decode sizes). Semantics: quant.hip's header.
#pragma once
#include "common.h"

namespace aiter_amd {

constexpr int kQuantThreads = 256;

template <bool kBf16>
__device__ __forceinline__ void quant_groups_block(const uint16_t* __restrict__ x,
                                                   uint8_t* __restrict__ q,
                                                   float* __restrict__ scale, int64_t rows,
                                                   int cols, int transpose_scale,
                                                   const int32_t* __restrict__ num_rows,
                                                   int num_rows_factor, int64_t block) {
    int64_t rows_eff = rows;
    if (num_rows) {
        int64_t r = (int64_t)num_rows[0] * num_rows_factor;
        rows_eff = r < 0 ? 0 : (r < rows ? r : rows);
    }
    const int G = cols / 128;
    const int64_t g = block * (kQuantThreads / 16) + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    const int64_t row = g / G;
    const int gc = (int)(g - row * G);
    const bool active = row < rows_eff;
    const int64_t off = row * cols + (int64_t)gc * 128 + sub * 8;

    float v[8];
    float amax = 1e-10f;
    if (active) {
        v4i raw = *reinterpret_cast<const v4i*>(x + off);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t w = (uint32_t)raw[i];
            if (kBf16) {
                v[2 * i] = bf16_bits_to_f32((uint16_t)(w & 0xFFFFu));
                v[2 * i + 1] = bf16_bits_to_f32((uint16_t)(w >> 16));
            } else {
                v[2 * i] = fp16_bits_to_f32((uint16_t)(w & 0xFFFFu));
                v[2 * i + 1] = fp16_bits_to_f32((uint16_t)(w >> 16));
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
    }
    amax = warp_max_16(amax);
    if (!active) return;
    const float s = amax * kInvFp8Max;
    const float inv = 1.0f / s;
    uint32_t lo = f32x4_to_fp8x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    uint32_t hi = f32x4_to_fp8x4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
    uint2 packed;
    packed.x = lo;
    packed.y = hi;
    *reinterpret_cast<uint2*>(q + off) = packed;
    if (sub == 0) {
        if (transpose_scale)
            scale[(int64_t)gc * rows_eff + row] = s;
        else
            scale[row * G + gc] = s;
    }
}

}  // namespace aiter_amd
