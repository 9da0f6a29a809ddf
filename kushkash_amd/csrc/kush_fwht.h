// Walsh-Hadamard rotation of D-element rows in the kernels' canonical evaluation order
// (kushkash/kush/quant.mojo:90-110, GPU butterflies gpu.mojo:57-93): butterflies at strides
// 1, 2, ..., D/2 in that order (of each pair, the element with the stride bit set becomes
// partner - self, the other self + partner), then one fp32 multiply by 1/sqrt(D). Every add is an
// exact-order fp32 add, so any data layout that keeps the stage order gives the same bits. The
// layout here (fwht_runs): D / 16 consecutive lanes per row, lane c of the row holds two runs of 8
// dims, x[j] = dim 8c + j and x[8 + j] = dim D/2 + 8c + j (the record's int4 byte order); strides
// 1..4 stay in a run, 8..D/4 cross lanes (DPP within 16-lane rows), D/2 pairs the two runs.
#pragma once

#include "kush_common.h"

namespace kush {

// fp32 1/sqrt(D) (its exact bits: quant.mojo:101-110)
template <int D>
__device__ __forceinline__ float fwht_scale() {
    return __uint_as_float(D == 64 ? 0x3E000000u : (D == 128 ? 0x3DB504F3u : 0x3D800000u));
}

#pragma clang fp contract(off)
// one butterfly stage across lanes (lane bit M of l): the lower lane keeps self + partner, the upper
// one partner - self, written partner + (-self) (the same IEEE result) so that every lane does one
// sign xor and one add, into which the compiler folds the DPP move
template <int M, int N>
__device__ __forceinline__ void butterfly_lanes(float (&x)[N], int l) {
    const uint32_t sign = (l & M) ? 0x80000000u : 0u;
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = lane_xor<M>(x[i]) + __uint_as_float(__float_as_uint(x[i]) ^ sign);
}

// c = the lane's index within its row's D / 16 lanes (those lanes are consecutive and aligned)
template <int D>
__device__ __forceinline__ void fwht_runs(float (&x)[16], int c) {
    constexpr int CG = D / 16;
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {                 // strides 1, 2, 4: within a run
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i & h) continue;
            const float a = x[i], b = x[i + h];
            x[i] = a + b;
            x[i + h] = a - b;
        }
    }
    butterfly_lanes<1>(x, c);                        // strides 8 .. D/4: lane bits 1 .. CG/2
    butterfly_lanes<2>(x, c);
    if constexpr (CG > 4) butterfly_lanes<4>(x, c);
    if constexpr (CG > 8) butterfly_lanes<8>(x, c);
#pragma unroll
    for (int i = 0; i < 8; ++i) {                     // stride D/2: the two runs
        const float a = x[i], b = x[i + 8];
        x[i] = a + b;
        x[i + 8] = a - b;
    }
    const float sc = fwht_scale<D>();
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = x[i] * sc;
}
#pragma clang fp contract(on)

}  // namespace kush
