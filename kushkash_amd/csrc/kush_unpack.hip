// Packed-prefill unpack for gfx950: one launch builds a prefill group's keys and values,
// kp / vp [rows, Hkv, D] in the input dtype, from (1) full history pages, (2) partial history
// pages (K rows from the exact tail, V rows from the record) and (3) the new chunk's rows, copied.
// Contract: kush_unpack, kushkash/kush/gpu.mojo:303-375, launched by Ops.unpack
// (kushkash/_ops.py:128-180); bit-identical to the reference CPU path (cpu.mojo:122-169).
//
// Dequantization is fma(code, scale, bias) in fp32 (fp16 scales and biases are exact in fp32),
// optionally rotated back by the canonical Walsh-Hadamard transform, then rounded once to the
// output dtype.
//
// The work is HBM-bound and write-heavy: a D = 128 int4 page of one kv head reads a 4,736-byte
// record and writes 32 K + 32 V rows (16 KB in bf16). A task is one (item, kv head), numbered
// with the heads fastest (neighbouring tasks read neighbouring records and write neighbouring
// 2*D-byte row pieces). A workgroup takes TASKS consecutive tasks: it first loads all their
// records into LDS (loads only, all issued before the first wait, so a workgroup keeps several
// records in flight), then dequantizes from LDS and streams the rows out with non-temporal
// stores, row by row across its tasks when they are heads of one page. A token row is D / 16 consecutive lanes; lane c of the row holds dims 8c.. and
// D/2 + 8c.. (the int4 record's byte order: byte 8c + j carries dims 8c + j and D/2 + 8c + j).
#include "kush_fwht.h"

namespace kush {

// record bytes a workgroup stages in LDS (whole records, at least one)
constexpr int UNPACK_STAGE_BYTES = 19 * 1024;

template <int D, int BITS>
struct Unpack {
    static constexpr int CG = D / 16;                                 // lanes per token row
    static constexpr int THREADS = PAGE * CG < 256 ? PAGE * CG : 256;
    static constexpr int RP = THREADS / CG;                           // rows per pass
    static constexpr int REC = Fmt<D, BITS>::REC;
    static constexpr int TASKS = UNPACK_STAGE_BYTES / REC > 1 ? UNPACK_STAGE_BYTES / REC : 1;
    static constexpr int CHUNKS = REC / 16;                           // 16-byte pieces of a record
    static constexpr int LOADS = (CHUNKS + THREADS - 1) / THREADS;    // per thread and record
};

// the 16 codes of lane c in the token row at `row` (LDS): x[j] = code of dim 8c + j, x[8 + j] =
// code of dim D/2 + 8c + j, as fp32 (exact small integers)
template <int D, int BITS>
__device__ __forceinline__ void row_codes(const uint8_t* row, int c, float (&x)[16]) {
    if constexpr (BITS == 4) {
        const u2 w = *reinterpret_cast<const u2*>(row + 8 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int32_t word = (int32_t)w[j / 4];
            x[j] = (float)((word << (28 - 8 * (j % 4))) >> 28);       // low nibble, sign-extended
            x[8 + j] = (float)((word << (24 - 8 * (j % 4))) >> 28);   // high nibble
        }
    } else {
        const u2 lo = *reinterpret_cast<const u2*>(row + 8 * c);
        const u2 hi = *reinterpret_cast<const u2*>(row + D / 2 + 8 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[j] = (float)(((int32_t)lo[j / 4] << (24 - 8 * (j % 4))) >> 24);
            x[8 + j] = (float)(((int32_t)hi[j / 4] << (24 - 8 * (j % 4))) >> 24);
        }
    }
}

// 8 fp16 values at p (16-byte aligned) as fp32
__device__ __forceinline__ void f16x8(const uint8_t* p, float* x) {
    const h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = (float)v[j];
}

// Token row t of a page record in LDS, dequantized for lane c (dims lo.. and hi..): V always from
// the record; K from the record when k_src is null, else copied from the exact K row k_src + t * D.
// fma(code, scale, bias) in fp32, then the rotation back when rot.
#pragma clang fp contract(off)
template <int D, int BITS, typename IN, bool VEC>
__device__ __forceinline__ void dequant_row(const uint8_t* rec, int t, int c, int lo, int hi, const IN* k_src, int rot,
                                            float (&kx)[16], float (&vx)[16]) {
    using F = Fmt<D, BITS>;
    if (k_src == nullptr) {
        float ks[16], kb[16];
        f16x8(rec + F::OFF_KS + 2 * lo, ks);
        f16x8(rec + F::OFF_KS + 2 * hi, ks + 8);
        f16x8(rec + F::OFF_KB + 2 * lo, kb);
        f16x8(rec + F::OFF_KB + 2 * hi, kb + 8);
        row_codes<D, BITS>(rec + t * F::DC, c, kx);
#pragma unroll
        for (int j = 0; j < 16; ++j) kx[j] = __builtin_fmaf(kx[j], ks[j], kb[j]);
    } else {
        get8<VEC>(k_src + t * D + lo, reinterpret_cast<float(&)[8]>(kx[0]));
        get8<VEC>(k_src + t * D + hi, reinterpret_cast<float(&)[8]>(kx[8]));
    }
    row_codes<D, BITS>(rec + F::OFF_VQ + t * F::DC, c, vx);
    const float vs = f16_val(*reinterpret_cast<const uint16_t*>(rec + F::OFF_VS + 2 * t));
    const float vb = f16_val(*reinterpret_cast<const uint16_t*>(rec + F::OFF_VB + 2 * t));
#pragma unroll
    for (int j = 0; j < 16; ++j) vx[j] = __builtin_fmaf(vx[j], vs, vb);
    if (rot) {
        fwht_runs<D>(kx, c);
        fwht_runs<D>(vx, c);
    }
}
#pragma clang fp contract(on)

// 8 fp32 values rounded to IN at dst, 16-byte non-temporal stores when VEC (the rows are not
// read again by this kernel, and a group's rows exceed the caches)
template <bool VEC, typename IN>
__device__ __forceinline__ void stream8(IN* dst, const float* x) {
    if constexpr (VEC && sizeof(IN) == 4) {
        __builtin_nontemporal_store(f4{x[0], x[1], x[2], x[3]}, reinterpret_cast<f4*>(dst));
        __builtin_nontemporal_store(f4{x[4], x[5], x[6], x[7]}, reinterpret_cast<f4*>(dst) + 1);
    } else if constexpr (VEC) {
        u4 w;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, store_rounded<IN>(x[2 * i])) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, store_rounded<IN>(x[2 * i + 1])) << 16);
        __builtin_nontemporal_store(w, reinterpret_cast<u4*>(dst));
    } else {
        put8<false>(dst, x);
    }
}

// grid (ceil(tasks / TASKS)), block Unpack::THREADS; task = item * H + kv head, item:
//   item < n_pages:            record of block page_blk[item] -> rows page_dst[item] + t, t < 32
//   item < n_pages + n_tail:   partial page i = item - n_pages, tail_info[3i..3i+2] = (first row,
//                              tokens n, tail slot): K from tail_k[slot], V from record tail_blk[i]
//   otherwise:                 32 new rows: row j of k_new / v_new -> row new_dst[j]
// Rows no item names are not written. VEC: 16-byte accesses (host-checked alignment).
#pragma clang fp contract(off)
template <int D, int BITS, typename IN, bool VEC>
__global__ __launch_bounds__((Unpack<D, BITS>::THREADS)) void unpack_kernel(
    const uint8_t* __restrict__ cache, int64_t bs, int64_t hs, int H, const int32_t* __restrict__ page_blk,
    const int32_t* __restrict__ page_dst, int n_pages, const int32_t* __restrict__ tail_blk,
    const int32_t* __restrict__ tail_info, int n_tail, const IN* __restrict__ tail_k, const IN* __restrict__ k_new,
    const IN* __restrict__ v_new, int64_t k_stride, int64_t v_stride, const int32_t* __restrict__ new_dst, int n_new,
    IN* __restrict__ kp, IN* __restrict__ vp, int rot, int n_tasks) {
    using F = Fmt<D, BITS>;
    using U = Unpack<D, BITS>;
    __shared__ __align__(16) uint8_t stage[U::TASKS][U::REC];
    const int tid = threadIdx.x;
    const int c = tid % U::CG, r0 = tid / U::CG;
    const int64_t rs = (int64_t)H * D;                                // kp / vp row stride
    const int lo = 8 * c, hi = D / 2 + 8 * c;                         // the lane's two runs of dims
    const int task0 = blockIdx.x * U::TASKS;
    const int rec_tasks = (n_pages + n_tail) * H;                    // < n_tasks < 2^31

    // the records of this workgroup's page tasks -> LDS: every load issued before the first wait
    u4 buf[U::TASKS][U::LOADS];
#pragma unroll
    for (int k = 0; k < U::TASKS; ++k) {
        const int task = task0 + k;
        if (task < rec_tasks) {
            const int item = task / H, h = task - item * H;
            const int64_t blk = item < n_pages ? page_blk[item] : tail_blk[item - n_pages];
            const u4* src = reinterpret_cast<const u4*>(cache + blk * bs + (int64_t)h * hs);
#pragma unroll
            for (int j = 0; j < U::LOADS; ++j) {
                const int i = tid + U::THREADS * j;
                if (i < U::CHUNKS) buf[k][j] = src[i];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < U::TASKS; ++k) {
        if (task0 + k < rec_tasks) {
#pragma unroll
            for (int j = 0; j < U::LOADS; ++j) {
                const int i = tid + U::THREADS * j;
                if (i < U::CHUNKS) reinterpret_cast<u4*>(stage[k])[i] = buf[k][j];
            }
        }
    }
    __syncthreads();

    // The common case, every task of the workgroup a full page of one item (TASKS consecutive kv heads
    // of one page): rows outside, heads inside, so a wave's consecutive stores fill the TASKS heads'
    // pieces of each row back to back (C4 group 129.7 -> 125.7 us, rotated back 143.9 -> 134.0)
    // rather than coming back to every row once per head.
    {
        const int item0 = task0 / H, h0 = task0 - item0 * H;
        if (h0 + U::TASKS <= H && item0 < n_pages && task0 + U::TASKS <= rec_tasks) {
            const int64_t dst0 = page_dst[item0];
            for (int t = r0; t < PAGE; t += U::RP) {
                IN* ko = kp + (dst0 + t) * rs + (int64_t)h0 * D;
                IN* vo = vp + (dst0 + t) * rs + (int64_t)h0 * D;
#pragma unroll
                for (int k = 0; k < U::TASKS; ++k) {
                    float kx[16], vx[16];
                    dequant_row<D, BITS, IN, VEC>(stage[k], t, c, lo, hi, nullptr, rot, kx, vx);
                    stream8<VEC>(ko + k * D + lo, kx);
                    stream8<VEC>(ko + k * D + hi, kx + 8);
                    stream8<VEC>(vo + k * D + lo, vx);
                    stream8<VEC>(vo + k * D + hi, vx + 8);
                }
            }
            return;
        }
    }
    for (int k = 0; k < U::TASKS; ++k) {
        const int task = task0 + k;
        if (task >= n_tasks) break;
        const int item = task / H, h = task - item * H;
        if (task < rec_tasks) {
            const uint8_t* rec = stage[k];
            const bool page = item < n_pages;
            const int i = item - n_pages;
            const int64_t dst0 = page ? page_dst[item] : tail_info[3 * i];
            const int n = page ? PAGE : tail_info[3 * i + 1];
            const IN* tk = page ? nullptr : tail_k + ((int64_t)tail_info[3 * i + 2] * H + h) * PAGE * D;
            for (int t = r0; t < n; t += U::RP) {
                float kx[16], vx[16];
                dequant_row<D, BITS, IN, VEC>(rec, t, c, lo, hi, tk, rot, kx, vx);
                IN* ko = kp + (dst0 + t) * rs + (int64_t)h * D;
                IN* vo = vp + (dst0 + t) * rs + (int64_t)h * D;
                stream8<VEC>(ko + lo, kx);
                stream8<VEC>(ko + hi, kx + 8);
                stream8<VEC>(vo + lo, vx);
                stream8<VEC>(vo + hi, vx + 8);
            }
        } else {
            const int j0 = (item - n_pages - n_tail) * PAGE;
            for (int t = r0; t < PAGE; t += U::RP) {
                const int j = j0 + t;
                if (j >= n_new) break;
                const int64_t o = (int64_t)new_dst[j] * rs + (int64_t)h * D;
                const IN* kr = k_new + (int64_t)j * k_stride + (int64_t)h * D;
                const IN* vr = v_new + (int64_t)j * v_stride + (int64_t)h * D;
                copy8<VEC>(kp + o + lo, kr + lo);
                copy8<VEC>(kp + o + hi, kr + hi);
                copy8<VEC>(vp + o + lo, vr + lo);
                copy8<VEC>(vp + o + hi, vr + hi);
            }
        }
    }
}
#pragma clang fp contract(on)

}  // namespace kush

using namespace kush;

extern "C" int kush_unpack(int head_dim, int bits, int dtype, const void* cache, int64_t block_stride,
                           int64_t head_stride, int32_t hkv, const int32_t* page_blk, const int32_t* page_dst,
                           int64_t n_pages, const int32_t* tail_blk, const int32_t* tail_info, int64_t n_tail,
                           const void* tail_k, const void* k_new, const void* v_new, int64_t k_stride,
                           int64_t v_stride, const int32_t* new_dst, int64_t n_new, void* kp, void* vp, int32_t rot,
                           void* stream) {
    if (n_pages < 0 || n_tail < 0 || n_new < 0)
        return kush_fail(-2, "kush_unpack: negative item count (pages %lld, tails %lld, new rows %lld)",
                         (long long)n_pages, (long long)n_tail, (long long)n_new);
    if (hkv < 1 || hkv > 65535) return kush_fail(-2, "kush_unpack: hkv %d out of range", hkv);
    if (((uintptr_t)cache | (uint64_t)block_stride | (uint64_t)head_stride) & 15)
        return kush_fail(-2, "kush_unpack: cache records must be 16-byte aligned");
    return dispatch_shape(head_dim, bits, dtype, "kush_unpack", [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        using U = Unpack<D, BITS>;
        const int64_t items = n_pages + n_tail + (n_new + PAGE - 1) / PAGE;
        if (items == 0) return 0;
        const int64_t tasks = items * hkv, blocks = (tasks + U::TASKS - 1) / U::TASKS;
        if (tasks > 0x7fffffff)
            return kush_fail(-2, "kush_unpack: %lld items x %d kv heads is too many", (long long)items, hkv);
        const uint64_t e = sizeof(IN);
        const bool vec = (((uintptr_t)tail_k | (uintptr_t)k_new | (uintptr_t)v_new | (uintptr_t)kp | (uintptr_t)vp |
                           (uint64_t)(k_stride * e) | (uint64_t)(v_stride * e)) & 15) == 0;
        auto kern = vec ? unpack_kernel<D, BITS, IN, true> : unpack_kernel<D, BITS, IN, false>;
        kern<<<dim3((unsigned)blocks), dim3(U::THREADS), 0, (hipStream_t)stream>>>(
            (const uint8_t*)cache, block_stride, head_stride, hkv, page_blk, page_dst, (int)n_pages, tail_blk,
            tail_info, (int)n_tail, (const IN*)tail_k, (const IN*)k_new, (const IN*)v_new, k_stride, v_stride,
            new_dst, (int)n_new, (IN*)kp, (IN*)vp, rot, (int)tasks);
        return kush_check_launch("kush_unpack");
    });
}
