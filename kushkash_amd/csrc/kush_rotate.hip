// Walsh-Hadamard rotation of D-element rows for gfx950, in the kernels' canonical evaluation order:
// butterflies at strides 1, 2, ..., D/2 in that order (the element with stride bit h set becomes
// partner - self, the other self + partner), then one fp32 multiply by 1/sqrt(D), then one rounding
// to the row dtype. Contract: kush_fwht, kushkash/kush/gpu.mojo:95-112 (warp butterflies
// gpu.mojo:57-93), order kushkash/kush/quant.mojo:95-110, launched by Ops.fwht
// (kushkash/_ops.py:104-126); bit-identical to the reference CPU path (cpu.mojo:83-107).
//
// One wave64 per row (fwht_wave): lane l holds row[l + 64 i], i < D / 64.
#include "kush_fwht.h"

namespace kush {

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
