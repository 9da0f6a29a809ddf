// The page quantizer shared by the write kernels and the fused append + decode: one (page, kv head)
// task quantized by one workgroup, K page and V rows, with the quantizer arithmetic of
// kushkash/kush/quant.mojo:25-50 (bit-identical to the reference CPU path, cpu.mojo:173-245).
//
// Thread t owns row t / CG of each pass over the page (CG = D / 16 threads per row) and the 16 dims
// [8c, 8c + 8) and [D/2 + 8c, D/2 + 8c + 8), c = t % CG: exactly the dims whose codes make bytes
// [8c, 8c + 8) of an int4 row (low nibble dim j, high nibble dim j + D/2), so rows are loaded with
// 16-byte loads and stored with 8-byte stores, both coalesced. A V row's range is reduced over the
// CG lanes of its row (xor shuffles); a K channel's range over the 32 rows goes through a tile of
// the K rows in LDS, kept in the input dtype (exact), one channel per thread.
//
// Rotated caches (rot): the rows a cache quantizes or stashes may be rotated by the canonical
// Walsh-Hadamard transform first, in registers: a thread's 16 dims of a row are exactly the
// butterfly layout of fwht_runs, and the rotated values are rounded to the input dtype, so a rotated
// write stores the bytes that Ops.fwht on the rows followed by an unrotated write would. Rows that
// come from a K tail are rotated already.
#pragma once

#include "kush_fwht.h"

namespace kush {

constexpr int WRITE_THREADS = 256;

// threads of a chunk-write workgroup
template <int D>
constexpr int write_threads() { return D == 256 ? 256 : 128; }

// Record bytes are written non-temporally: a chunk write leaves megabytes of records that no kernel
// of the write reads back, and as ordinary writes they sit dirty in L2 until the end of the launch,
// whose release then writes them back while nothing else runs (C4 write: 22.5 -> 19.3 us).
__device__ __forceinline__ void put_rec8(uint8_t* p, u2 v) {
    __builtin_nontemporal_store((uint64_t)v[0] | ((uint64_t)v[1] << 32), reinterpret_cast<uint64_t*>(p));
}
__device__ __forceinline__ void put_rec2(uint8_t* p, uint16_t x) {
    __builtin_nontemporal_store(x, reinterpret_cast<uint16_t*>(p));
}

template <int D, int THREADS>
struct Rows {
    static constexpr int CG = D / 16;                        // threads per row
    static constexpr int RP = THREADS / CG;                  // rows per pass
    static constexpr int PASSES = RP >= PAGE ? 1 : PAGE / RP;
};

// LDS of a page task: the K tile (PAGE x D in the input dtype), then the channels' fp32 bias and
// reciprocal scale
template <int D, typename IN>
constexpr int tile_bytes() { return PAGE * D * (int)sizeof(IN) + 2 * D * 4; }

// A thread's 16 values of one row (two runs of 8: dims 8c.. and D/2 + 8c..) as loaded, in 16-byte
// words (2 for 16-bit inputs, 4 for fp32): half the registers of fp32 values for bf16 / fp16
template <typename IN, bool VEC>
struct Row16 {
    static constexpr int W = (int)sizeof(IN) * 16 / 16;
    u4 w[W];
    __device__ __forceinline__ void load(const IN* row, int lo, int hi) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < W / 2; ++i) {
                w[i] = reinterpret_cast<const u4*>(row + lo)[i];
                w[W / 2 + i] = reinterpret_cast<const u4*>(row + hi)[i];
            }
        } else {
            IN v[16];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v[j] = row[lo + j];
                v[8 + j] = row[hi + j];
            }
            __builtin_memcpy(w, v, sizeof(w));
        }
    }
    __device__ __forceinline__ void floats(float (&x)[16]) const {
        const IN* v = reinterpret_cast<const IN*>(w);
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] = to_f32(v[j]);
    }
    // the 16 values back as IN (values already representable in IN: rotate16's output)
    __device__ __forceinline__ void set(const float (&x)[16]) {
        IN v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) v[j] = from_f32<IN>(x[j]);
        __builtin_memcpy(w, v, sizeof(w));
    }
    // both runs into the tile row (16-byte aligned)
    __device__ __forceinline__ void store(IN* row, int lo, int hi) const {
#pragma unroll
        for (int i = 0; i < W / 2; ++i) {
            reinterpret_cast<u4*>(row + lo)[i] = w[i];
            reinterpret_cast<u4*>(row + hi)[i] = w[W / 2 + i];
        }
    }
};

// This lane's 16 values of a row (lane c of the row's D / 16 lanes) rotated by the canonical
// Walsh-Hadamard transform and rounded to IN, as Ops.fwht writes the row
template <int D, typename IN>
__device__ __forceinline__ void rotate16(float (&x)[16], int c) {
    fwht_runs<D>(x, c);
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = to_f32(store_rounded<IN>(x[j]));
}

template <int D, typename IN, bool VEC>
__device__ __forceinline__ void rotate_row(Row16<IN, VEC>& row, int c) {
    float x[16];
    row.floats(x);
    rotate16<D, IN>(x, c);
    row.set(x);
}

// codes of the 16 values of a thread (x[0..8): dims 8c.., x[8..16): dims D/2 + 8c..) -> the bytes
// they make: int4 byte i = code(x[i]) & 15 | (code(x[8 + i]) & 15) << 4 (row bytes 8c + i, in lo);
// int8 bytes in dim order (row bytes 8c + i in lo, D/2 + 8c + i in hi). The codes stay floats
// (exact small integers): an offset byte (code + 8 per nibble, code + 128) is inserted by
// v_cvt_pk_u8_f32 and the offset taken out of the whole word by one xor.
#pragma clang fp contract(off)
template <int BITS>
__device__ __forceinline__ float qcode_f(float x, float b, float inv) {
    constexpr float HALF = float(1 << (BITS - 1));
    const float r = __builtin_rintf((x - b) * inv);
    return __builtin_fminf(__builtin_fmaxf(r, -HALF), HALF - 1.0f);
}

template <int BITS>
__device__ __forceinline__ void pack16(const float (&x)[16], const float (&b)[16], const float (&inv)[16], u2& lo,
                                       u2& hi) {
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float c0 = qcode_f<BITS>(x[i], b[i], inv[i]);
        const float c1 = qcode_f<BITS>(x[8 + i], b[8 + i], inv[8 + i]);
        if constexpr (BITS == 4) {
            w[i / 4] = __builtin_amdgcn_cvt_pk_u8_f32(__builtin_fmaf(c1, 16.0f, c0) + 136.0f, i % 4, w[i / 4]);
        } else {
            w[i / 4] = __builtin_amdgcn_cvt_pk_u8_f32(c0 + 128.0f, i % 4, w[i / 4]);
            w[2 + i / 4] = __builtin_amdgcn_cvt_pk_u8_f32(c1 + 128.0f, i % 4, w[2 + i / 4]);
        }
    }
    constexpr uint32_t OFF = BITS == 4 ? 0x88888888u : 0x80808080u;
    lo = u2{w[0] ^ OFF, w[1] ^ OFF};
    hi = u2{w[2] ^ OFF, w[3] ^ OFF};
}
#pragma clang fp contract(on)

// min / max over the CG consecutive lanes of a row (xor butterflies by DPP within 16-lane rows)
template <int CG>
__device__ __forceinline__ void row_range(float& mn, float& mx) {
    mn = __builtin_fminf(mn, lane_xor<1>(mn));
    mx = __builtin_fmaxf(mx, lane_xor<1>(mx));
    mn = __builtin_fminf(mn, lane_xor<2>(mn));
    mx = __builtin_fmaxf(mx, lane_xor<2>(mx));
    if constexpr (CG > 4) {
        mn = __builtin_fminf(mn, lane_xor<4>(mn));
        mx = __builtin_fmaxf(mx, lane_xor<4>(mx));
    }
    if constexpr (CG > 8) {
        mn = __builtin_fminf(mn, lane_xor<8>(mn));
        mx = __builtin_fmaxf(mx, lane_xor<8>(mx));
    }
}

// One (page, kv head) by THREADS threads (t = 0 .. THREADS - 1, this thread's index among them): V
// rows [vlo, vhi) of the page (row r from v_new + (r - vlo) * v_stride) and, when do_k, the K page:
// rows r < split from k_tail (stride D), the others from k_new + (r - split) * k_stride. rec: the
// page's record. lds: tile_bytes<D, IN>() bytes of this task. Every thread of the workgroup calls
// this: it has three barriers when do_k; with SYNC_ALWAYS it has them in any case, so that tasks
// packed into one workgroup (some without a K page) pass the same barriers.
template <int D, int BITS, typename IN, bool VEC, int THREADS, bool ROT, bool SYNC_ALWAYS = false>
__device__ __forceinline__ void page_task(const IN* __restrict__ k_tail, const IN* __restrict__ k_new, int64_t k_stride,
                                          int split, bool do_k, const IN* __restrict__ v_new, int64_t v_stride,
                                          int vlo, int vhi, uint8_t* __restrict__ rec, uint8_t* lds,
                                          int t = (int)threadIdx.x) {
    using F = Fmt<D, BITS>;
    using RW = Rows<D, THREADS>;
    constexpr int CG = RW::CG;
    const int c = t % CG, r0 = t / CG;
    const auto has_v = [&](int r) { return r >= vlo && r < vhi && r < PAGE; };

    // V rows: each row's final encoding, per-token range over the CG lanes of the row (consecutive
    // lanes of one wave, all taking the same branch). Their loads go out first, the K rows' behind
    // them, and the V work runs while the K rows land (C4 write: 19.3 -> 17.1 us).
    Row16<IN, VEC> vrow[RW::PASSES];
#pragma unroll
    for (int pp = 0; pp < RW::PASSES; ++pp) {
        const int r = r0 + pp * RW::RP;
        if (has_v(r)) vrow[pp].load(v_new + (int64_t)(r - vlo) * v_stride, 8 * c, D / 2 + 8 * c);
    }
    const auto v_rows = [&]() {
#pragma unroll
        for (int pp = 0; pp < RW::PASSES; ++pp) {
            const int r = r0 + pp * RW::RP;
            if (!has_v(r)) continue;
            float x[16];
            vrow[pp].floats(x);
            if constexpr (ROT) rotate16<D, IN>(x, c);
            float mn = x[0], mx = x[0];
#pragma unroll
            for (int j = 1; j < 16; ++j) {
                mn = __builtin_fminf(mn, x[j]);
                mx = __builtin_fmaxf(mx, x[j]);
            }
            row_range<CG>(mn, mx);
            float s, b, inv;
            qparams<BITS>(mn, mx, s, b, inv);
            float bb[16], ii[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                bb[j] = b;
                ii[j] = inv;
            }
            u2 lo, hi;
            pack16<BITS>(x, bb, ii, lo, hi);
            uint8_t* dst = rec + F::OFF_VQ + r * F::DC + 8 * c;
            put_rec8(dst, lo);
            if constexpr (BITS == 8) put_rec8(dst + D / 2, hi);
            if (c == 0) {
                put_rec2(rec + F::OFF_VS + 2 * r, f16_bits(s));
                put_rec2(rec + F::OFF_VB + 2 * r, f16_bits(b));
            }
        }
    };
    if (!do_k) {
        v_rows();
        if constexpr (SYNC_ALWAYS) {
            __syncthreads();
            __syncthreads();
            __syncthreads();
        }
        return;
    }

    // K rows into registers, the V work while they land, then the rows into the tile
    IN* const tile = reinterpret_cast<IN*>(lds);
    Row16<IN, VEC> kr[RW::PASSES];
#pragma unroll
    for (int pp = 0; pp < RW::PASSES; ++pp) {
        const int r = r0 + pp * RW::RP;
        if (r < PAGE) kr[pp].load(r < split ? k_tail + r * D : k_new + (int64_t)(r - split) * k_stride, 8 * c, D / 2 + 8 * c);
    }
    v_rows();
#pragma unroll
    for (int pp = 0; pp < RW::PASSES; ++pp) {
        const int r = r0 + pp * RW::RP;
        if (r >= PAGE) continue;
        if constexpr (ROT) {
            if (r >= split) rotate_row<D>(kr[pp], c);                   // a whole row's lanes branch together
        }
        kr[pp].store(tile + r * D, 8 * c, D / 2 + 8 * c);
    }

    // K: per-channel range over the 32 rows (one channel per thread), then the codes
    float* kbias = reinterpret_cast<float*>(lds + PAGE * D * sizeof(IN));
    float* kinv = kbias + D;
    __syncthreads();
    for (int ch = t; ch < D; ch += THREADS) {
        float mn = __builtin_inff(), mx = -__builtin_inff();
#pragma unroll 8
        for (int r = 0; r < PAGE; ++r) {
            const float x = to_f32(tile[r * D + ch]);
            mn = __builtin_fminf(mn, x);
            mx = __builtin_fmaxf(mx, x);
        }
        float s, b, inv;
        qparams<BITS>(mn, mx, s, b, inv);
        put_rec2(rec + F::OFF_KS + 2 * ch, f16_bits(s));
        put_rec2(rec + F::OFF_KB + 2 * ch, f16_bits(b));
        kbias[ch] = b;
        kinv[ch] = inv;
    }
    __syncthreads();
    float bb[16], ii[16];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
        const f4 b0 = *reinterpret_cast<const f4*>(kbias + hh * (D / 2) + 8 * c);
        const f4 b1 = *reinterpret_cast<const f4*>(kbias + hh * (D / 2) + 8 * c + 4);
        const f4 i0 = *reinterpret_cast<const f4*>(kinv + hh * (D / 2) + 8 * c);
        const f4 i1 = *reinterpret_cast<const f4*>(kinv + hh * (D / 2) + 8 * c + 4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bb[8 * hh + j] = b0[j];
            bb[8 * hh + 4 + j] = b1[j];
            ii[8 * hh + j] = i0[j];
            ii[8 * hh + 4 + j] = i1[j];
        }
    }
#pragma unroll
    for (int pp = 0; pp < RW::PASSES; ++pp) {
        const int r = r0 + pp * RW::RP;
        if (r >= PAGE) continue;
        float kx[16];
        kr[pp].floats(kx);
        u2 lo, hi;
        pack16<BITS>(kx, bb, ii, lo, hi);
        uint8_t* dst = rec + r * F::DC + 8 * c;
        put_rec8(dst, lo);
        if constexpr (BITS == 8) put_rec8(dst + D / 2, hi);
    }
    __syncthreads();   // tile is free again
}

// n K rows from src (row stride src_stride) into a tail at dst (row stride D), rotated when ROT, by
// THREADS threads: without rotation a plain copy, with it D / 16 lanes per row in the butterfly layout
template <int D, typename IN, bool VEC, bool ROT, int THREADS>
__device__ __forceinline__ void stash_rows(IN* __restrict__ dst, const IN* __restrict__ src, int64_t src_stride, int n,
                                           int tid) {
    if constexpr (!ROT) {
        for (int i = tid; i < n * (D / 8); i += THREADS) {
            const int r = i / (D / 8), j = 8 * (i % (D / 8));
            copy8<VEC>(dst + r * D + j, src + (int64_t)r * src_stride + j);
        }
    } else {
        constexpr int CG = D / 16, RP = THREADS / CG;
        static_assert(THREADS % CG == 0, "whole rows per pass");
        const int c = tid % CG;
        for (int r = tid / CG; r < n; r += RP) {                   // a row's lanes iterate together
            Row16<IN, VEC> row;
            row.load(src + (int64_t)r * src_stride, 8 * c, D / 2 + 8 * c);
            rotate_row<D>(row, c);
            float x[16];
            row.floats(x);
            put8<VEC>(dst + r * D + 8 * c, x);
            put8<VEC>(dst + r * D + D / 2 + 8 * c, x + 8);
        }
    }
}

}  // namespace kush
