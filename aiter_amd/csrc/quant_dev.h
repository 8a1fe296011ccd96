// 1 x 128 FP8 quantisation of one 256-thread block's 16 groups: the body of
// per_group_quant_fp8_kernel, shared with the sorting launch (which runs it
// in extra blocks at decode sizes). Semantics: quant.hip's header.
#pragma once
#include "common.h"

namespace aiter_amd {

constexpr int kQuantThreads = 256;

// A lane's 8 consecutive bf16 / fp16 elements of one 1x128 group as fp32.
template <bool kBf16>
__device__ __forceinline__ void load8_f32(const uint16_t* p, float (&v)[8]) {
    const v4i raw = *reinterpret_cast<const v4i*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = (uint32_t)raw[i];
        if (kBf16) {
            v[2 * i] = bf16_bits_to_f32((uint16_t)(w & 0xFFFFu));
            v[2 * i + 1] = bf16_bits_to_f32((uint16_t)(w >> 16));
        } else {
            v[2 * i] = fp16_bits_to_f32((uint16_t)(w & 0xFFFFu));
            v[2 * i + 1] = fp16_bits_to_f32((uint16_t)(w >> 16));
        }
    }
}

// The 1x128 quant of a group held by 16 consecutive lanes, 8 elements each
// (all 16 lanes must call it; `active` false contributes nothing): returns
// the group's scale amax / 448 (amax floored at 1e-10) and the lane's 8 fp8
// codes in *codes.
__device__ __forceinline__ float quant8(const float (&v)[8], bool active, uint2* codes) {
    float amax = 1e-10f;
    if (active) {
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(v[i]));
    }
    amax = warp_max_16(amax);
    const float s = amax * kInvFp8Max;
    const float inv = 1.0f / s;
    codes->x = f32x4_to_fp8x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    codes->y = f32x4_to_fp8x4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
    return s;
}

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

    float v[8] = {};
    if (active) load8_f32<kBf16>(x + off, v);
    uint2 packed;
    const float s = quant8(v, active, &packed);
    if (!active) return;
    *reinterpret_cast<uint2*>(q + off) = packed;
    if (sub == 0) {
        if (transpose_scale)
            scale[(int64_t)gc * rows_eff + row] = s;
        else
            scale[row * G + gc] = s;
    }
}

}  // namespace aiter_amd
