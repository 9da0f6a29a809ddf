// Shared definitions for the gfx950 kernels of the compressed-KV hot path: the page-record
// format (kushkash/kush/quant.mojo:16-87), the quantization arithmetic (quant.mojo:25-50), input
// dtype conversions, row loads and stores, and lane exchange.
//
// Page record of one (block, kv head), D channels, BITS in {4, 8}, DC = row bytes:
//   [ kq: 32*DC | vq: 32*DC | ks: D fp16 | kb: D fp16 | vs: 32 fp16 | vb: 32 fp16 ]
// int4 row byte j holds the code of dim j (low nibble) and of dim j + D/2 (high nibble).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kushkash_amd.h"   // the C ABI these sources implement

// Error reporting shared by the C entry points (kush_capi.hip): records a message for
// kush_last_error() and returns code.
int kush_fail(int code, const char* fmt, ...);
int kush_check_launch(const char* what);

namespace kush {

constexpr int PAGE = 32;
constexpr int WAVE = 64;

template <int D, int BITS>
struct Fmt {
    static_assert(D == 64 || D == 128 || D == 256, "head_dim must be 64, 128 or 256");
    static_assert(BITS == 4 || BITS == 8, "bits must be 4 or 8");
    static constexpr int DC = BITS == 8 ? D : D / 2;   // bytes per token row
    static constexpr int OFF_VQ = PAGE * DC;
    static constexpr int OFF_KS = 2 * PAGE * DC;
    static constexpr int OFF_KB = OFF_KS + 2 * D;
    static constexpr int OFF_VS = OFF_KS + 4 * D;
    static constexpr int OFF_VB = OFF_VS + 2 * PAGE;
    static constexpr int REC = OFF_VB + 2 * PAGE;       // record bytes, a multiple of 16
    static constexpr int HALF = 1 << (BITS - 1);
    static_assert(REC % 16 == 0, "records must stay 16-byte aligned");
};

// ------------------------------------------------------------------ vector types
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

// ------------------------------------------------------------------ input element types
// The kernels take q, k, v, out and the exact K tail in one of three dtypes.
struct bf16_t {
    uint16_t u;
};

// 8 consecutive elements as fp32: one or two 16-byte loads (p 16-byte aligned)
__device__ __forceinline__ void load8(const float* p, float (&x)[8]) {
    const f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[j] = a[j];
        x[j + 4] = b[j];
    }
}

__device__ __forceinline__ void load8(const _Float16* p, float (&x)[8]) {
    const h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (float)v[j];
}

__device__ __forceinline__ void load8(const bf16_t* p, float (&x)[8]) {
    const u4 v = *reinterpret_cast<const u4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(v[i] << 16);
        x[2 * i + 1] = __uint_as_float(v[i] & 0xFFFF0000u);
    }
}

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(_Float16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float((uint32_t)x.u << 16); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float x) { return (_Float16)x; }   // RNE
// RNE to bf16 (overflow to infinity, NaN stays NaN): gfx950's v_cvt_pk_bf16_f32, which converts
// two values per instruction when two conversions meet in one 32-bit word
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) {
    return bf16_t{__builtin_bit_cast(uint16_t, (__bf16)x)};
}

// 8 consecutive elements as fp32: 16-byte loads when the rows are 16-byte aligned, else per element
template <bool VEC, typename IN>
__device__ __forceinline__ void get8(const IN* p, float (&x)[8]) {
    if constexpr (VEC) {
        load8(p, x);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = to_f32(p[j]);
    }
}

template <bool VEC, typename IN>
__device__ __forceinline__ void copy8(IN* dst, const IN* src) {
    if constexpr (VEC && sizeof(IN) == 2) {
        *reinterpret_cast<u4*>(dst) = *reinterpret_cast<const u4*>(src);
    } else if constexpr (VEC) {
        reinterpret_cast<u4*>(dst)[0] = reinterpret_cast<const u4*>(src)[0];
        reinterpret_cast<u4*>(dst)[1] = reinterpret_cast<const u4*>(src)[1];
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = src[j];
    }
}

// 8 fp32 values rounded to IN at dst: 16-byte stores when dst is 16-byte aligned, else per element.
// The opaque copy keeps the compiler from folding a preceding fp32 multiply or fma into an fp16
// conversion (v_fma_mix*_f16 round once, straight to fp16; these kernels round to fp32 first, then
// to IN, as the reference does, and at fp16 ties the two differ).
template <typename IN>
__device__ __forceinline__ IN store_rounded(float x) {
    asm volatile("" : "+v"(x));
    return from_f32<IN>(x);
}

template <bool VEC, typename IN>
__device__ __forceinline__ void put8(IN* dst, const float* x) {
    if constexpr (VEC && sizeof(IN) == 4) {
        reinterpret_cast<f4*>(dst)[0] = f4{x[0], x[1], x[2], x[3]};
        reinterpret_cast<f4*>(dst)[1] = f4{x[4], x[5], x[6], x[7]};
    } else if constexpr (VEC) {
        u4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, store_rounded<IN>(x[2 * i])) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, store_rounded<IN>(x[2 * i + 1])) << 16);
        *reinterpret_cast<u4*>(dst) = w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) dst[j] = store_rounded<IN>(x[j]);
    }
}

__device__ __forceinline__ uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
__device__ __forceinline__ float f16_val(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// ------------------------------------------------------------------ quantization (quant.mojo:25-50)
// These must round exactly like the reference CPU path: IEEE fp32 division (the library is built
// with -fhip-fp32-correctly-rounded-divide-sqrt and without fast-math), RNE to fp16, codes
// against the fp16-rounded scale and bias, round half to even.
#pragma clang fp contract(off)

template <int BITS>
__device__ __forceinline__ void qparams(float mn, float mx, float& s, float& b, float& inv) {
    constexpr float LEVELS = float((1 << BITS) - 1);
    constexpr float HALF = float(1 << (BITS - 1));
    s = (float)(_Float16)((mx - mn) / LEVELS);
    b = (float)(_Float16)(mn + s * HALF);
    inv = s > 0.0f ? 1.0f / s : 0.0f;
}

template <int BITS>
__device__ __forceinline__ int qcode(float x, float b, float inv) {
    constexpr float HALF = float(1 << (BITS - 1));
    float r = __builtin_rintf((x - b) * inv);
    r = __builtin_fminf(__builtin_fmaxf(r, -HALF), HALF - 1.0f);
    return (int)r;
}

__device__ __forceinline__ uint8_t pack4(int lo, int hi) { return (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4)); }

#pragma clang fp contract(on)

// ------------------------------------------------------------------ lane exchange
// x of lane (l ^ m) for m in {1, 2, 4, 8}, by DPP within each 16-lane row: quad_perm swaps for 1
// and 2; 4 and 8 compose two mirrors (half-row mirror l -> l ^ 7 and quad reversal l -> l ^ 3
// give l ^ 4; row mirror l -> l ^ 15 and half-row mirror give l ^ 8)
template <int M>
__device__ __forceinline__ float lane_xor(float x) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8, "DPP xor within a 16-lane row");
    int v = __float_as_int(x);
    if constexpr (M == 1) {
        v = __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);       // quad_perm [1, 0, 3, 2]
    } else if constexpr (M == 2) {
        v = __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);       // quad_perm [2, 3, 0, 1]
    } else if constexpr (M == 4) {
        v = __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);      // row_half_mirror
        v = __builtin_amdgcn_mov_dpp(v, 0x1B, 0xF, 0xF, true);       // quad_perm [3, 2, 1, 0]
    } else {
        v = __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true);      // row_mirror
        v = __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);      // row_half_mirror
    }
    return __int_as_float(v);
}

// ------------------------------------------------------------------ shape dispatch
template <int V>
using ic = std::integral_constant<int, V>;

template <typename Fn>
static inline int dispatch_shape(int D, int bits, int dtype, const char* what, Fn&& fn) {
    auto by_dtype = [&](auto dd, auto bb) -> int {
        switch (dtype) {
            case 0: return fn(dd, bb, float{});
            case 1: return fn(dd, bb, _Float16{});
            case 2: return fn(dd, bb, bf16_t{});
        }
        return kush_fail(-1, "%s: unsupported dtype code %d (0 fp32, 1 fp16, 2 bf16)", what, dtype);
    };
    auto by_bits = [&](auto dd) -> int {
        if (bits == 4) return by_dtype(dd, ic<4>{});
        if (bits == 8) return by_dtype(dd, ic<8>{});
        return kush_fail(-1, "%s: unsupported bits %d (4 or 8)", what, bits);
    };
    switch (D) {
        case 64: return by_bits(ic<64>{});
        case 128: return by_bits(ic<128>{});
        case 256: return by_bits(ic<256>{});
    }
    return kush_fail(-1, "%s: unsupported head_dim %d (64, 128 or 256)", what, D);
}

}  // namespace kush

