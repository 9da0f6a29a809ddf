// Walsh-Hadamard rotation of D-element rows for gfx950, in the kernels' canonical evaluation order:
// butterflies at strides 1, 2, ..., D/2 in that order (the element with stride bit h set becomes
// partner - self, the other self + partner), then one fp32 multiply by 1/sqrt(D), then one rounding
// to the row dtype. Contract: kush_fwht, kushkash/kush/gpu.mojo:95-112 (warp butterflies
// gpu.mojo:57-93), order kushkash/kush/quant.mojo:95-110, launched by Ops.fwht
// (kushkash/_ops.py:104-126); bit-identical to the reference CPU path (cpu.mojo:83-107).
//
// A streaming kernel (each row read once, written once): a row is D / 16 consecutive lanes, each
// holding two runs of 8 dims (fwht_runs) moved with 16-byte accesses when the rows are 16-byte
// aligned, so a 256-thread workgroup covers 4096 elements per pass.
#include "kush_fwht.h"

namespace kush {

// grid (ceil(rows / (256 / (D / 16)))), block 256; y may alias x (a row's lanes read it whole
// before any of them writes)
template <int D, typename IN, bool VEC>
__global__ __launch_bounds__(256) void fwht_kernel(const IN* x, IN* y, int64_t x_stride, int64_t y_stride,
                                                   int64_t rows) {
    constexpr int CG = D / 16, RPB = 256 / CG;
    const int c = threadIdx.x % CG;
    const int64_t r = (int64_t)blockIdx.x * RPB + threadIdx.x / CG;
    if (r >= rows) return;                            // a row's lanes leave together
    const int lo = 8 * c, hi = D / 2 + 8 * c;
    float v[16];
    get8<VEC>(x + r * x_stride + lo, reinterpret_cast<float(&)[8]>(v[0]));
    get8<VEC>(x + r * x_stride + hi, reinterpret_cast<float(&)[8]>(v[8]));
    fwht_runs<D>(v, c);
    put8<VEC>(y + r * y_stride + lo, v);
    put8<VEC>(y + r * y_stride + hi, v + 8);
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
        constexpr int RPB = 256 / (D / 16);
        const int64_t blocks = (rows + RPB - 1) / RPB;
        if (blocks > 0x7fffffff) return kush_fail(-2, "kush_fwht: %lld rows is too many", (long long)rows);
        const uint64_t e = sizeof(IN);
        const bool vec = (((uintptr_t)x | (uintptr_t)y | (uint64_t)(x_row_stride * e) | (uint64_t)(y_row_stride * e)) &
                          15) == 0;
        auto kern = vec ? fwht_kernel<D, IN, true> : fwht_kernel<D, IN, false>;
        kern<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>((const IN*)x, (IN*)y, x_row_stride,
                                                                             y_row_stride, rows);
        return kush_check_launch("kush_fwht");
    });
}
