// Walsh-Hadamard rotation of D-element rows for gfx950, in the kernels' canonical evaluation order:
// butterflies at strides 1, 2, ..., D/2 in that order (the element with stride bit h set becomes
// partner - self, the other self + partner), then one fp32 multiply by 1/sqrt(D), then one rounding
// to the row dtype. Contract: kush_fwht, kushkash/kush/gpu.mojo:95-112 (warp butterflies
// gpu.mojo:57-93), order kushkash/kush/quant.mojo:95-110, launched by Ops.fwht
// (kushkash/_ops.py:104-126); bit-identical to the reference CPU path (cpu.mojo:83-107).
//
// One wave64 per row: lane l holds row[l + 64 i], i < D / 64. Strides 1..32 pair lanes (xor
// shuffles), strides 64 and 128 pair the lane's own registers. fp32 adds are exact regardless of
// which lane computes them, so any layout that keeps the stage order gives the same bits.
#include "kush_common.h"

namespace kush {

// fp32 1/sqrt(D) (its exact bits: quant.mojo:101-110)
template <int D>
__device__ __forceinline__ float fwht_scale() {
    return __uint_as_float(D == 64 ? 0x3E000000u : (D == 128 ? 0x3DB504F3u : 0x3D800000u));
}

#pragma clang fp contract(off)
template <int D>
__device__ __forceinline__ void fwht_wave(float (&v)[D / WAVE], int lane) {
    constexpr int R = D / WAVE;
#pragma unroll
    for (int h = 1; h < WAVE; h <<= 1) {
        const bool upper = (lane & h) != 0;
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const float other = __shfl_xor(v[i], h, WAVE);
            v[i] = upper ? other - v[i] : v[i] + other;
        }
    }
#pragma unroll
    for (int hb = 1; hb < R; hb <<= 1) {              // stride 64 hb: register bit hb
#pragma unroll
        for (int i = 0; i < R; ++i) {
            if (i & hb) continue;
            const float a = v[i], b = v[i + hb];
            v[i] = a + b;
            v[i + hb] = a - b;
        }
    }
    const float sc = fwht_scale<D>();
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = v[i] * sc;
}

// rounds x (already rounded to fp32) to IN. The opaque copy keeps the compiler from folding the
// preceding fp32 multiply into the conversion (v_fma_mixlo_f16 rounds x * s once, straight to fp16;
// the reference rounds twice, fp32 then fp16, and at fp16 ties the two differ)
template <typename IN>
__device__ __forceinline__ IN store_rounded(float x) {
    asm volatile("" : "+v"(x));
    return from_f32<IN>(x);
}
#pragma clang fp contract(on)

// grid (ceil(rows / 4)), block 256: one wave per row; y may alias x (a wave reads its whole row first)
template <int D, typename IN>
__global__ __launch_bounds__(256) void fwht_kernel(const IN* x, IN* y, int64_t x_stride, int64_t y_stride,
                                                   int64_t rows) {
    const int lane = threadIdx.x % WAVE;
    const int64_t r = (int64_t)blockIdx.x * 4 + threadIdx.x / WAVE;
    if (r >= rows) return;
    constexpr int R = D / WAVE;
    float v[R];
#pragma unroll
    for (int i = 0; i < R; ++i) v[i] = to_f32(x[r * x_stride + lane + WAVE * i]);
    fwht_wave<D>(v, lane);
#pragma unroll
    for (int i = 0; i < R; ++i) y[r * y_stride + lane + WAVE * i] = store_rounded<IN>(v[i]);
}

}  // namespace kush

using namespace kush;

extern "C" int kush_fwht(int head_dim, int dtype, const void* x, void* y, int64_t x_row_stride, int64_t y_row_stride,
                         int64_t rows, void* stream) {
    if (rows < 0) return kush_fail(-2, "kush_fwht: bad rows %lld", (long long)rows);
    return dispatch_shape(head_dim, 4, dtype, "kush_fwht", [&](auto dd, auto, auto in) -> int {
        constexpr int D = decltype(dd)::value;
        using IN = decltype(in);
        if (rows == 0) return 0;
        const int64_t blocks = (rows + 3) / 4;
        if (blocks > 0x7fffffff) return kush_fail(-2, "kush_fwht: %lld rows is too many", (long long)rows);
        fwht_kernel<D, IN><<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
            (const IN*)x, (IN*)y, x_row_stride, y_row_stride, rows);
        return kush_check_launch("kush_fwht");
    });
}
