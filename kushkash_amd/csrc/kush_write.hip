// Quantize-and-pack on write for gfx950: one token per sequence (append) and ragged
// multi-token chunks (write). Reference contract: kushkash/kush/gpu.mojo:207-276 (kernels),
// kushkash/_ops.py:66-101 (launch), arithmetic kushkash/kush/quant.mojo:25-50. Pages are
// bit-identical to the reference CPU path (kushkash/kush/cpu.mojo:173-304).
//
// Work split on CDNA4: one workgroup per (page, kv head), of 256 threads for the append and of
// 128 (D <= 128) or 256 threads for the chunk write, small enough in threads and LDS that a CU
// holds 16 of them: a chunk's pages then mostly run as one round, all their row loads in flight
// together. Thread t owns row t / CG of each pass over the page (CG = D / 16 threads per row)
// and the 16 dims [8c, 8c + 8) and [D/2 + 8c, D/2 + 8c + 8), c = t % CG: exactly the dims whose
// codes make bytes [8c, 8c + 8) of an int4 row (low nibble dim j, high nibble dim j + D/2), so
// rows are loaded with 16-byte loads and stored with 8-byte stores, both coalesced. A V row's
// range is reduced over the CG lanes of its row (xor shuffles); a K channel's range over the 32
// rows goes through a tile of the K rows in LDS, kept in the input dtype (exact), one channel
// per thread.
//
// Rotated caches (rot): the rows a cache quantizes or stashes may be rotated by the canonical
// Walsh-Hadamard transform first, in registers: a thread's 16 dims of a row are exactly the
// butterfly layout of fwht_runs (D / 16 consecutive lanes per row, dims 8c.. and D/2 + 8c..), and the
// rotated values are rounded to the input dtype, so a rotated write stores the bytes that Ops.fwht
// on the rows followed by an unrotated write would. Rows that come from a K tail are rotated already.
#include "kush_fwht.h"

namespace kush {

constexpr int WRITE_THREADS = 256;

// threads of a chunk-write workgroup
template <int D>
constexpr int write_threads() { return D == 256 ? 256 : 128; }

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

// One (page, kv head) by the workgroup of THREADS threads: V rows [vlo, vhi) of the page (row t
// from v_new + (t - vlo) * v_stride) and, when do_k, the K page: rows t < split from k_tail
// (stride D), the others from k_new + (t - split) * k_stride. rec: the page's record. lds:
// tile_bytes<D, IN>() bytes. Every thread of the workgroup calls this (it has barriers when do_k).
template <int D, int BITS, typename IN, bool VEC, int THREADS, bool ROT>
__device__ __forceinline__ void page_task(const IN* __restrict__ k_tail, const IN* __restrict__ k_new, int64_t k_stride,
                                          int split, bool do_k, const IN* __restrict__ v_new, int64_t v_stride,
                                          int vlo, int vhi, uint8_t* __restrict__ rec, uint8_t* lds) {
    using F = Fmt<D, BITS>;
    using RW = Rows<D, THREADS>;
    constexpr int CG = RW::CG;
    const int t = threadIdx.x, c = t % CG, r0 = t / CG;
    const auto has_v = [&](int r) { return r >= vlo && r < vhi && r < PAGE; };

    // V rows: each row's final encoding, per-token range over the CG lanes of the row (consecutive
    // lanes of one wave, all taking the same branch)
    const auto v_rows = [&]() {
#pragma unroll
        for (int pp = 0; pp < RW::PASSES; ++pp) {
            const int r = r0 + pp * RW::RP;
            if (!has_v(r)) continue;
            Row16<IN, VEC> vr;
            vr.load(v_new + (int64_t)(r - vlo) * v_stride, 8 * c, D / 2 + 8 * c);
            float x[16];
            vr.floats(x);
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
            *reinterpret_cast<u2*>(dst) = lo;
            if constexpr (BITS == 8) *reinterpret_cast<u2*>(dst + D / 2) = hi;
            if (c == 0) {
                reinterpret_cast<uint16_t*>(rec + F::OFF_VS)[r] = f16_bits(s);
                reinterpret_cast<uint16_t*>(rec + F::OFF_VB)[r] = f16_bits(b);
            }
        }
    };
    if (!do_k) {
        v_rows();
        return;
    }

    // K rows into registers as loaded and into the tile (loads issued before the V work)
    IN* const tile = reinterpret_cast<IN*>(lds);
    Row16<IN, VEC> kr[RW::PASSES];
#pragma unroll
    for (int pp = 0; pp < RW::PASSES; ++pp) {
        const int r = r0 + pp * RW::RP;
        if (r >= PAGE) continue;
        kr[pp].load(r < split ? k_tail + r * D : k_new + (int64_t)(r - split) * k_stride, 8 * c, D / 2 + 8 * c);
        if constexpr (ROT) {
            if (r >= split) rotate_row<D>(kr[pp], c);                   // a whole row's lanes branch together
        }
        kr[pp].store(tile + r * D, 8 * c, D / 2 + 8 * c);
    }
    v_rows();

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
        reinterpret_cast<uint16_t*>(rec + F::OFF_KS)[ch] = f16_bits(s);
        reinterpret_cast<uint16_t*>(rec + F::OFF_KB)[ch] = f16_bits(b);
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
        *reinterpret_cast<u2*>(dst) = lo;
        if constexpr (BITS == 8) *reinterpret_cast<u2*>(dst + D / 2) = hi;
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

// grid (S, Hkv), block 256: one (sequence, kv head). One token per sequence at position
// seq_lens[s] + pos_offset; negative positions (padding rows) are skipped. K goes to the exact
// tail (quantized when its page fills: rows 0..30 from the tail, row 31 this token, read from k),
// V straight into its record row. Contract: gpu.mojo:207-238, cpu.mojo:248-270 (seq_lens
// advances in advance_kernel, launched after this one).
template <int D, int BITS, typename IN, bool VEC, bool ROT>
__global__ __launch_bounds__(WRITE_THREADS) void append_kernel(
    const IN* __restrict__ k, const IN* __restrict__ v, int64_t k_stride, int64_t v_stride,
    const int32_t* __restrict__ seq_lens, int pos_offset, const int32_t* __restrict__ tail_idx,
    uint8_t* __restrict__ cache, int64_t bs, int64_t hs, IN* __restrict__ tail_k,
    const int32_t* __restrict__ block_table, int64_t bt_stride, int H) {
    __shared__ __align__(16) uint8_t lds[tile_bytes<D, IN>()];
    const int s = blockIdx.x, h = blockIdx.y;
    const int pos = seq_lens[s] + pos_offset;
    if (pos < 0) return;
    const int slot = pos % PAGE;
    const int64_t blk = block_table[(int64_t)s * bt_stride + pos / PAGE];
    IN* tail = tail_k + ((int64_t)tail_idx[s] * H + h) * PAGE * D;
    const IN* krow = k + (int64_t)s * k_stride + (int64_t)h * D;
    uint8_t* rec = cache + blk * bs + (int64_t)h * hs;
    stash_rows<D, IN, VEC, ROT, WRITE_THREADS>(tail + slot * D, krow, 0, 1, threadIdx.x);
    page_task<D, BITS, IN, VEC, WRITE_THREADS, ROT>(tail, krow, 0, PAGE - 1, slot == PAGE - 1,
                                               v + (int64_t)s * v_stride + (int64_t)h * D, 0, slot, slot + 1, rec, lds);
}

// seq_lens[s] = seq_lens[s] + pos_offset + 1 where that position is >= 0 (the appended token)
__global__ __launch_bounds__(256) void advance_kernel(int32_t* seq_lens, int pos_offset, int S) {
    const int s = blockIdx.x * 256 + threadIdx.x;
    if (s < S) {
        const int pos = seq_lens[s] + pos_offset;
        if (pos >= 0) seq_lens[s] = pos + 1;
    }
}

// grid (n_jobs, Hkv), block write_threads<D>(): the write's mode 0. Job j covers logical page job_page[j] of
// sequence job_seq[j], whose new rows [qsl[s], qsl[s+1]) sit at positions [ctx, seq_lens[s]):
// write the page's new V rows and, if the page is complete, quantize its K (older rows from the
// tail, newer from the chunk). Mode 1 (tail_kernel) then stashes the new K rows of still-partial
// pages in the tail: two launches, so no tail is read and written by the same one.
// FUSE (mode 2): mode 1 in the same launch. A sequence's tail is read only by the job of its first
// touched page (page ctx / 32, when ctx % 32 != 0 and the page completes) and written only for its
// last page (seq_lens / 32, when left partial). When both happen on different pages, the first
// page's job writes the tail after its own reads (same workgroup, behind page_task's last barrier);
// otherwise the partial page's job does. Needs a job for every page the chunk touches.
// Contract: gpu.mojo:241-276, cpu.mojo:273-304.
template <int D, int BITS, typename IN, bool VEC, bool FUSE, bool ROT>
__global__ __launch_bounds__(write_threads<D>()) void write_kernel(
    const IN* __restrict__ k, const IN* __restrict__ v, int64_t k_stride, int64_t v_stride,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ tail_idx,
    const int32_t* __restrict__ job_seq, const int32_t* __restrict__ job_page, uint8_t* __restrict__ cache,
    int64_t bs, int64_t hs, IN* __restrict__ tail_k, const int32_t* __restrict__ block_table, int64_t bt_stride, int H) {
    __shared__ __align__(16) uint8_t lds[tile_bytes<D, IN>()];
    const int j = blockIdx.x, h = blockIdx.y;
    const int s = job_seq[j];
    const int ps = job_page[j] * PAGE;
    const int q0 = qsl[s];
    const int total = seq_lens[s];
    const int ctx = total - (qsl[s + 1] - q0);
    const bool complete = ps + PAGE <= total;
    IN* tail = tail_k + ((int64_t)tail_idx[s] * H + h) * PAGE * D;
    const int lo = ps > ctx ? ps : ctx;                     // first new position in the page
    const int64_t hoff = (int64_t)h * D;
    {
        uint8_t* rec = cache + (int64_t)block_table[(int64_t)s * bt_stride + ps / PAGE] * bs + (int64_t)h * hs;
        const int hi = ps + PAGE < total ? ps + PAGE : total;
        int split = ctx - ps;                               // K rows before it come from the tail
        split = split < 0 ? 0 : (split > PAGE ? PAGE : split);
        page_task<D, BITS, IN, VEC, write_threads<D>(), ROT>(tail, k + (int64_t)(q0 + ps + split - ctx) * k_stride + hoff,
                                                        k_stride, split, complete,
                                                        v + (int64_t)(q0 + lo - ctx) * v_stride + hoff, v_stride,
                                                        lo - ps, hi - ps, rec, lds);
    }
    if constexpr (FUSE) {
        const int last = total / PAGE, first = ctx / PAGE;
        const int owner = (ctx % PAGE != 0 && last != first) ? first : last;
        if (total % PAGE != 0 && ps / PAGE == owner) {
            const int pl = last * PAGE;
            const int lo2 = pl > ctx ? pl : ctx;
            stash_rows<D, IN, VEC, ROT, write_threads<D>()>(tail + (lo2 - pl) * D,
                                                             k + (int64_t)(q0 + lo2 - ctx) * k_stride + hoff, k_stride,
                                                             total - lo2, threadIdx.x);
        }
    }
}

// grid (ceil(n_jobs * Hkv / 4)), block 256: the write's mode 1, one wave per (job, kv head): stash
// the new K rows of a still-partial page in the tail (a complete page's wave returns at once).
template <int D, typename IN, bool VEC, bool ROT>
__global__ __launch_bounds__(256) void tail_kernel(const IN* __restrict__ k, int64_t k_stride,
                                                   const int32_t* __restrict__ qsl, const int32_t* __restrict__ seq_lens,
                                                   const int32_t* __restrict__ tail_idx,
                                                   const int32_t* __restrict__ job_seq,
                                                   const int32_t* __restrict__ job_page, int n_jobs,
                                                   IN* __restrict__ tail_k, int H) {
    const int gw = blockIdx.x * 4 + (int)(threadIdx.x / WAVE), lane = threadIdx.x % WAVE;
    const int j = gw / H, h = gw % H;
    if (j >= n_jobs) return;
    const int s = job_seq[j];
    const int ps = job_page[j] * PAGE;
    const int total = seq_lens[s];
    if (ps + PAGE <= total) return;
    const int q0 = qsl[s];
    const int ctx = total - (qsl[s + 1] - q0);
    const int lo = ps > ctx ? ps : ctx;
    IN* dst = tail_k + (((int64_t)tail_idx[s] * H + h) * PAGE + (lo - ps)) * D;
    const IN* src = k + (int64_t)(q0 + lo - ctx) * k_stride + (int64_t)h * D;
    stash_rows<D, IN, VEC, ROT, WAVE>(dst, src, k_stride, total - lo, lane);
}

// 16-byte loads and stores when k / v rows (pointer and row stride) and tail_k are 16-byte aligned
template <typename IN>
static bool rows_aligned(const void* k, const void* v, int64_t k_stride, int64_t v_stride, const void* tail_k) {
    const uint64_t e = sizeof(IN);
    return (((uintptr_t)k | (uintptr_t)v | (uintptr_t)tail_k | (uint64_t)(k_stride * e) | (uint64_t)(v_stride * e)) &
            15) == 0;
}

}  // namespace kush

using namespace kush;

extern "C" int kush_append(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                           int64_t v_stride, int32_t* seq_lens, int32_t pos_offset, int32_t advance,
                           const int32_t* tail_idx, void* cache, int64_t block_stride, int64_t head_stride,
                           void* tail_k, const int32_t* block_table, int64_t bt_stride, int32_t hkv, int32_t n_seqs,
                           int32_t rot, void* stream) {
    if (n_seqs < 0 || hkv <= 0 || rot < 0 || rot > 1)
        return kush_fail(-2, "kush_append: bad n_seqs %d / hkv %d / rot %d", n_seqs, hkv, rot);
    return dispatch_shape(head_dim, bits, dtype, "kush_append", [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        if (n_seqs == 0) return 0;
        hipStream_t st = (hipStream_t)stream;
        const bool vec = rows_aligned<IN>(k, v, k_stride, v_stride, tail_k);
        auto kern = rot ? (vec ? append_kernel<D, BITS, IN, true, true> : append_kernel<D, BITS, IN, false, true>)
                        : (vec ? append_kernel<D, BITS, IN, true, false> : append_kernel<D, BITS, IN, false, false>);
        kern<<<dim3(n_seqs, hkv), dim3(WRITE_THREADS), 0, st>>>((const IN*)k, (const IN*)v, k_stride, v_stride,
                                                                seq_lens, pos_offset, tail_idx, (uint8_t*)cache,
                                                                block_stride, head_stride, (IN*)tail_k, block_table,
                                                                bt_stride, hkv);
        if (advance) advance_kernel<<<dim3((n_seqs + 255) / 256), dim3(256), 0, st>>>(seq_lens, pos_offset, n_seqs);
        return kush_check_launch("kush_append");
    });
}

extern "C" int kush_write(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                          int64_t v_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                          const int32_t* tail_idx, const int32_t* job_seq, const int32_t* job_page, int32_t n_jobs,
                          int32_t mode, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                          const int32_t* block_table, int64_t bt_stride, int32_t hkv, int32_t rot, void* stream) {
    if (n_jobs < 0 || hkv <= 0 || mode < 0 || mode > 2 || rot < 0 || rot > 1)
        return kush_fail(-2, "kush_write: bad n_jobs %d / hkv %d / mode %d / rot %d", n_jobs, hkv, mode, rot);
    return dispatch_shape(head_dim, bits, dtype, "kush_write", [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        if (n_jobs == 0) return 0;
        const bool vec = rows_aligned<IN>(k, v, k_stride, v_stride, tail_k);
        hipStream_t st = (hipStream_t)stream;
        if (mode != 1) {
            using K = decltype(&write_kernel<D, BITS, IN, true, true, true>);
            const K table[2][2][2] = {                                  // [vec][fuse][rot]
                {{write_kernel<D, BITS, IN, false, false, false>, write_kernel<D, BITS, IN, false, false, true>},
                 {write_kernel<D, BITS, IN, false, true, false>, write_kernel<D, BITS, IN, false, true, true>}},
                {{write_kernel<D, BITS, IN, true, false, false>, write_kernel<D, BITS, IN, true, false, true>},
                 {write_kernel<D, BITS, IN, true, true, false>, write_kernel<D, BITS, IN, true, true, true>}}};
            auto kern = table[vec][mode == 2][rot];
            kern<<<dim3(n_jobs, hkv), dim3(write_threads<D>()), 0, st>>>(
                (const IN*)k, (const IN*)v, k_stride, v_stride, query_start_loc, seq_lens, tail_idx, job_seq, job_page,
                (uint8_t*)cache, block_stride, head_stride, (IN*)tail_k, block_table, bt_stride, hkv);
        } else {
            auto kern = rot ? (vec ? tail_kernel<D, IN, true, true> : tail_kernel<D, IN, false, true>)
                            : (vec ? tail_kernel<D, IN, true, false> : tail_kernel<D, IN, false, false>);
            kern<<<dim3(((int64_t)n_jobs * hkv + 3) / 4), dim3(256), 0, st>>>(
                (const IN*)k, k_stride, query_start_loc, seq_lens, tail_idx, job_seq, job_page, n_jobs, (IN*)tail_k, hkv);
        }
        return kush_check_launch("kush_write");
    });
}
