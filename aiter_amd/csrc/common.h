// Shared helpers for the aiter_amd fused-MoE library (gfx950 / CDNA4 only).
//
// Error handling follows the reference's ctypes bridge
// (csrc/include/aiter_ctypes_error.h:60-147): every extern "C" entry point
// returns 0 on success and -1 on failure, and the failure text is kept in a
// thread-local string that aiter_amd_get_last_error() returns.  No C++
// exception ever crosses the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

namespace aiter_amd {

// ---------------------------------------------------------------- errors ---
void set_last_error(const std::string& msg);
void clear_last_error();

struct AbiError : public std::runtime_error {
    explicit AbiError(const std::string& m) : std::runtime_error(m) {}
};

#define AMD_CHECK(cond, msg)                                                   \
    do {                                                                       \
        if (!(cond)) {                                                         \
            throw ::aiter_amd::AbiError(std::string(__func__) + ": " + (msg)); \
        }                                                                      \
    } while (0)

#define AMD_HIP_CHECK(expr)                                                    \
    do {                                                                       \
        hipError_t _e = (expr);                                                \
        if (_e != hipSuccess) {                                                \
            throw ::aiter_amd::AbiError(std::string(#expr) + " failed: " +     \
                                        hipGetErrorString(_e));                \
        }                                                                      \
    } while (0)

// Runs `fn` and converts any exception into the thread-local error + -1; a
// call clears the error left by an earlier one first.
template <typename F>
inline int safe_call(F&& fn) {
    clear_last_error();
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return -1;
    } catch (...) {
        set_last_error("unknown C++ exception");
        return -1;
    }
}

// dtype codes: identical to AiterDtype (csrc/include/aiter_enum.h:27-43).
enum DtypeCode : int {
    DT_FP8 = 0,
    DT_FP8_E8M0 = 1,
    DT_FP16 = 2,
    DT_BF16 = 3,
    DT_FP32 = 4,
    DT_FP4X2 = 6,
    DT_I32 = 8,
};

// ------------------------------------------------------- device helpers ---
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// 1/448 rounded to fp32, the e4m3fn maximum's reciprocal.  The reference
// kernel multiplies amax by this constant (quant_kernels.cu:67-69,98-100).
constexpr float kInvFp8Max = (float)(1.0 / 448.0);
constexpr float kFp8Max = 448.0f;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}

__device__ __forceinline__ float fp16_bits_to_f32(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// fp32 -> bf16, round to nearest even: gfx950's v_cvt_pk_bf16_f32 (one
// instruction; inputs here are finite).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ uint16_t f32_to_fp16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

__device__ __forceinline__ float bf16_round(float f) {
    return bf16_bits_to_f32(f32_to_bf16_bits(f));
}

// Two fp32 -> two e4m3fn bytes (low 16 bits of the result), saturated to
// +-448 first and then converted round-to-nearest-even by the hardware
// converter.
__device__ __forceinline__ uint32_t f32x2_to_fp8x2(float a, float b) {
    a = __builtin_fminf(__builtin_fmaxf(a, -kFp8Max), kFp8Max);
    b = __builtin_fminf(__builtin_fmaxf(b, -kFp8Max), kFp8Max);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

__device__ __forceinline__ uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
    return f32x2_to_fp8x2(a, b) | (f32x2_to_fp8x2(c, d) << 16);
}

// One 16x16x128 fp8 x fp8 MFMA with fresh (zero) accumulator.  Scale
// operands of zero select the unscaled gfx950 instruction
// v_mfma_f32_16x16x128_f8f6f4.
__device__ __forceinline__ v4f mfma16x16x128_fp8(const v8i& a, const v8i& b) {
    v4f z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 0, 0, 0, 0, 0);
}

// One 16x16x128 MFMA of fp8 e4m3 A against fp4 e2m1 B (two values per byte,
// even K in the low nibble) with an e8m0 scale per B lane taken from byte 0 of
// b_scale; the A scale is 127 = 1.0.  Only the low 4 dwords of b are used.
// K order of this operand pairing (measured on gfx950): the B lane of group
// q = lane/16 holds K 32q..32q+31 in nibble order -- one MX block, which its
// scale byte covers -- and the matching A lane must hold K 16q..16q+15 in
// bytes 0-15 and K 64+16q..64+16q+15 in bytes 16-31 of its 32-byte fragment.
__device__ __forceinline__ v4f mfma16x16x128_fp8_fp4(const v8i& a, const v8i& b, int b_scale) {
    v4f z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 0, 4, 0, 127, 0, b_scale);
}

// The same product with the operands' roles swapped: fp4 e2m1 weights as the
// MFMA's A operand (e8m0 scale per A lane from byte 0 of a_scale) and fp8 e4m3
// activations as B (scale 127 = 1.0), fragments laid out per lane as above.
__device__ __forceinline__ v4f mfma16x16x128_fp4_fp8(const v8i& a, const v8i& b, int a_scale) {
    v4f z = {0.f, 0.f, 0.f, 0.f};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, z, 4, 0, 0, a_scale, 0, 127);
}

template <typename T>
__device__ __forceinline__ T warp_max_16(T v) {
    // max over the 16 lanes that share lane/16 (xor over lane bits 0..3)
    v = __builtin_fmaxf(v, __shfl_xor(v, 1, 64));
    v = __builtin_fmaxf(v, __shfl_xor(v, 2, 64));
    v = __builtin_fmaxf(v, __shfl_xor(v, 4, 64));
    v = __builtin_fmaxf(v, __shfl_xor(v, 8, 64));
    return v;
}

// x * sigmoid(x) with the hardware reciprocal (1 ulp) instead of a correctly
// rounded division: for x -> -inf the reciprocal of inf is 0 (result -0), for
// x -> +inf it is 1
__device__ __forceinline__ float silu_f32(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// torch.nn.functional.gelu (approximate='none'): x/2 * (1 + erf(x/sqrt(2))),
// evaluated as x/2 * erfc(-x/sqrt(2)), which has no cancellation for x < 0
// (and in the unrolled GEMM epilogues needs fewer registers than erff)
__device__ __forceinline__ float gelu_f32(float x) {
    return 0.5f * x * erfcf(x * -0.70710678118654752f);
}

// Stage-2 accumulation: adds v to element i of the output, which is fp32
// (the hardware fp32 atomic) or, as the reference's moe_buf, bf16 / fp16:
// the packed 16-bit atomic on the aligned pair holding the element, with 0
// added to its neighbour (x + 0 = x), so every add rounds once to 16 bits.
typedef __bf16 v2bf16 __attribute__((ext_vector_type(2)));
typedef _Float16 v2f16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void acc_add(void* base, int dtype, int64_t i, float v) {
    if (dtype == DT_FP32) {
        unsafeAtomicAdd(reinterpret_cast<float*>(base) + i, v);
    } else if (dtype == DT_BF16) {
        const __bf16 b = (__bf16)v, z = (__bf16)0.0f;
        v2bf16* pair = reinterpret_cast<v2bf16*>(reinterpret_cast<uint16_t*>(base) + (i & ~int64_t(1)));
        __builtin_amdgcn_global_atomic_fadd_v2bf16(pair, (i & 1) ? v2bf16{z, b} : v2bf16{b, z});
    } else {
        const _Float16 h = (_Float16)v, z = (_Float16)0.0f;
        v2f16* pair = reinterpret_cast<v2f16*>(reinterpret_cast<uint16_t*>(base) + (i & ~int64_t(1)));
        __builtin_amdgcn_global_atomic_fadd_v2f16(pair, (i & 1) ? v2f16{z, h} : v2f16{h, z});
    }
}

// ActivationType values (csrc/include/aiter_enum.h:7-12) the GEMMs apply to gate
constexpr int kActSilu = 0;
constexpr int kActGelu = 1;

// Stage-1 output forms: the fp8 a2 with its 1x128 scales (the fused requant);
// act(gate) * up rows [pairs, inter] in bf16 / fp16 / fp32 (the reference's
// ck_moe_stage1 output, quantised by a separate launch); fp32 gate | up rows
// [pairs, 2 * inter] before the activation (its split-K output, which
// silu_and_mul / gelu_and_mul finish).
constexpr int kOutA2 = 0;
constexpr int kOutAct = 1;
constexpr int kOutGateUp = 2;

// Direct M-blocks for the decode kernel's stage 1 (a one-token layer, too
// small to be worth a sorting launch): M-block p holds routing pair p of
// `tokens` tokens, its expert ids[p]. Stage 1 may also quantise the
// activations xq (bf16 / fp16 [tokens, K]) itself.
struct StreamDirect {
    const int32_t* ids = nullptr;
    int tokens = 0;
    const void* xq = nullptr;
    int xq_dtype = 0;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// XCD-aware order of a 1-D grid of (M-tile, column group) workgroups.
// Workgroup L runs on XCD L % 8. With ng % 8 == 0 the 8 XCDs form ms groups
// along M x 8/ms along N: XCD x takes column groups [(x % (8/ms)) * per, +per)
// (per = ng / (8/ms)) of the valid M-tiles [(x / (8/ms)) * chunk, +chunk),
// M-major; with rot its walk starts (x % (8/ms)) / (8/ms) of the way into
// the range. m_slots is the grid's M-tiles per group (ceil(m_tiles / ms)),
// mv the valid M-tiles. Returns false for a workgroup with no tile.
__device__ __forceinline__ bool xcd_tile(int L, int ng, int m_slots, int mv, int ms, int rot,
                                         int& nt, int& mt) {
    if ((ng & 7) != 0) {
        nt = L % ng;
        mt = L / ng;
        return true;
    }
    const int nsplit = 8 / ms;
    const int per = ng / nsplit;
    const int idx = L >> 3;
    const int x = L & 7;
    const int chunk = (ms == 1 && !rot) ? m_slots : (mv + ms - 1) / ms;
    int ml = idx / per;
    if (ml >= chunk) return false;
    if (rot) {
        ml += ((x % nsplit) * chunk) / nsplit;
        if (ml >= chunk) ml -= chunk;
    }
    nt = (x % nsplit) * per + idx % per;
    mt = (x / nsplit) * chunk + ml;
    return true;
}

// Grid size of xcd_tile's order: every group gets ceil(m_tiles / ms) M-tiles' slots.
inline int64_t xcd_grid(int ng, int64_t m_tiles, int ms) {
    return (ng & 7) != 0 ? (int64_t)ng * m_tiles : (int64_t)ng * ceil_div(m_tiles, ms) * ms;
}

}  // namespace aiter_amd
