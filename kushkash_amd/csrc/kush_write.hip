// Quantize-and-pack on write for gfx950: one token per sequence (append) and ragged
// multi-token chunks (write). Reference contract: kushkash/kush/gpu.mojo:207-276 (kernels),
// kushkash/_ops.py:66-101 (launch), arithmetic kushkash/kush/quant.mojo:25-50. Pages are
// bit-identical to the reference CPU path (kushkash/kush/cpu.mojo:173-304).
//
// Work split on CDNA4: a page task is one (page, kv head), of 256 threads for the append and of
// 128 (D <= 128) or 256 threads for the chunk write, whose 256-thread workgroups take two
// neighbouring kv heads of a page at D <= 128. A task's indices come in by scalar loads (two round
// trips), and every task's row loads are issued before its first wait. The page quantizer itself (thread layout, K tile, rotation) is in
// kush_page.h.
#include "kush_page.h"

namespace kush {

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

// Page tasks per chunk-write workgroup (256 threads): neighbouring kv heads of one page side by side.
// A chunk write has thousands of small page tasks that the dispatcher starts over ~10 us; two per
// workgroup halve the dispatches (C4 write 17.05 -> 16.86 us). More per workgroup lose: every
// task then waits at each barrier for the slowest of them (8 per workgroup: 19.3 -> 20.3 us).
template <int D>
constexpr int write_tpb() { return 256 / write_threads<D>(); }

// grid (ceil(n_jobs * Hkv / TPB)), block TPB * write_threads<D>(): the write's mode 0, task i =
// (job i / Hkv, kv head i % Hkv). Job j covers logical page job_page[j] of sequence job_seq[j],
// whose new rows [qsl[s], qsl[s+1]) sit at positions [ctx, seq_lens[s]): write the page's new V rows
// and, if the page is complete, quantize its K (older rows from the tail, newer from the chunk).
// Mode 1 (tail_kernel) then stashes the new K rows of still-partial pages in the tail: two
// launches, so no tail is read and written by the same one.
// FUSE (mode 2): mode 1 in the same launch. A sequence's tail is read only by the job of its first
// touched page (page ctx / 32, when ctx % 32 != 0 and the page completes) and written only for its
// last page (seq_lens / 32, when left partial). When both happen on different pages, the first
// page's job writes the tail after its own reads (same task, behind page_task's last barrier);
// otherwise the partial page's job does. Needs a job for every page the chunk touches.
// Contract: gpu.mojo:241-276, cpu.mojo:273-304.
template <int D, int BITS, typename IN, bool VEC, bool FUSE, bool ROT>
__global__ __launch_bounds__(256) void write_kernel(
    const IN* __restrict__ k, const IN* __restrict__ v, int64_t k_stride, int64_t v_stride,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ tail_idx,
    const int32_t* __restrict__ job_seq, const int32_t* __restrict__ job_page, int n_jobs, uint8_t* __restrict__ cache,
    int64_t bs, int64_t hs, IN* __restrict__ tail_k, const int32_t* __restrict__ block_table, int64_t bt_stride, int H) {
    constexpr int TH = write_threads<D>(), TPB = write_tpb<D>();
    __shared__ __align__(16) uint8_t lds[TPB * tile_bytes<D, IN>()];
    // the task's indices are wave-uniform (a task is whole waves): scalar loads, in two round trips --
    // the job's sequence and page, then everything of the sequence at once (the empty asm statements
    // take each group's values together, so no load waits for another of its group)
    const int sub = __builtin_amdgcn_readfirstlane((int)threadIdx.x / TH), tid = (int)threadIdx.x % TH;
    const int task = (int)blockIdx.x * TPB + sub;     // n_jobs H < 2^31 (checked by the entry point)
    const bool live = task < n_jobs * H;              // a task past the end still passes the barriers
    const int j = live ? task / H : 0, h = live ? task % H : 0;
    int s = job_seq[j], pg = job_page[j];
    asm volatile("" : "+s"(s), "+s"(pg));
    int q0 = qsl[s], q1 = qsl[s + 1], total = seq_lens[s], ti = tail_idx[s];
    int blk = block_table[(int64_t)s * bt_stride + pg];
    asm volatile("" : "+s"(q0), "+s"(q1), "+s"(total), "+s"(ti), "+s"(blk));
    const int ps = pg * PAGE;
    const int ctx = total - (q1 - q0);
    const bool complete = ps + PAGE <= total;
    IN* tail = tail_k + ((int64_t)ti * H + h) * PAGE * D;
    const int lo = ps > ctx ? ps : ctx;                     // first new position in the page
    const int64_t hoff = (int64_t)h * D;
    {
        uint8_t* rec = cache + (int64_t)blk * bs + (int64_t)h * hs;
        const int hi = !live ? lo : (ps + PAGE < total ? ps + PAGE : total);
        int split = ctx - ps;                               // K rows before it come from the tail
        split = split < 0 ? 0 : (split > PAGE ? PAGE : split);
        page_task<D, BITS, IN, VEC, TH, ROT, true>(tail, k + (int64_t)(q0 + ps + split - ctx) * k_stride + hoff,
                                                   k_stride, split, live && complete,
                                                   v + (int64_t)(q0 + lo - ctx) * v_stride + hoff, v_stride, lo - ps,
                                                   hi - ps, rec, lds + sub * tile_bytes<D, IN>(), tid);
    }
    if constexpr (FUSE) {
        const int last = total / PAGE, first = ctx / PAGE;
        const int owner = (ctx % PAGE != 0 && last != first) ? first : last;
        if (live && total % PAGE != 0 && ps / PAGE == owner) {
            const int pl = last * PAGE;
            const int lo2 = pl > ctx ? pl : ctx;
            stash_rows<D, IN, VEC, ROT, TH>(tail + (lo2 - pl) * D, k + (int64_t)(q0 + lo2 - ctx) * k_stride + hoff,
                                            k_stride, total - lo2, tid);
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

extern "C" int kush_append_ex(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                              int64_t v_stride, int32_t* seq_lens, int32_t pos_offset, int32_t advance,
                              const int32_t* tail_idx, void* cache, int64_t block_stride, int64_t head_stride,
                              void* tail_k, const int32_t* block_table, int64_t bt_stride, int32_t hkv, int32_t n_seqs,
                              void* stream, int32_t rot) {
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

extern "C" int kush_write_ex(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                             int64_t v_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                             const int32_t* tail_idx, const int32_t* job_seq, const int32_t* job_page, int32_t n_jobs,
                             int32_t mode, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                             const int32_t* block_table, int64_t bt_stride, int32_t hkv, void* stream, int32_t rot) {
    if (n_jobs < 0 || hkv <= 0 || mode < 0 || mode > 2 || rot < 0 || rot > 1)
        return kush_fail(-2, "kush_write: bad n_jobs %d / hkv %d / mode %d / rot %d", n_jobs, hkv, mode, rot);
    if ((int64_t)n_jobs * hkv >= (int64_t)1 << 31)
        return kush_fail(-2, "kush_write: %d jobs x %d kv heads is 2^31 page tasks or more", n_jobs, hkv);
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
            constexpr int TPB = write_tpb<D>();
            const int64_t tasks = (int64_t)n_jobs * hkv;
            kern<<<dim3((unsigned)((tasks + TPB - 1) / TPB)), dim3(TPB * write_threads<D>()), 0, st>>>(
                (const IN*)k, (const IN*)v, k_stride, v_stride, query_start_loc, seq_lens, tail_idx, job_seq, job_page,
                n_jobs, (uint8_t*)cache, block_stride, head_stride, (IN*)tail_k, block_table, bt_stride, hkv);
        } else {
            auto kern = rot ? (vec ? tail_kernel<D, IN, true, true> : tail_kernel<D, IN, false, true>)
                            : (vec ? tail_kernel<D, IN, true, false> : tail_kernel<D, IN, false, false>);
            kern<<<dim3(((int64_t)n_jobs * hkv + 3) / 4), dim3(256), 0, st>>>(
                (const IN*)k, k_stride, query_start_loc, seq_lens, tail_idx, job_seq, job_page, n_jobs, (IN*)tail_k, hkv);
        }
        return kush_check_launch("kush_write");
    });
}

// The reference's argument lists exactly (rot = 0): a binding written from the reference's launch
// arguments works by position.
extern "C" int kush_append(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                           int64_t v_stride, int32_t* seq_lens, int32_t pos_offset, int32_t advance,
                           const int32_t* tail_idx, void* cache, int64_t block_stride, int64_t head_stride,
                           void* tail_k, const int32_t* block_table, int64_t bt_stride, int32_t hkv, int32_t n_seqs,
                           void* stream) {
    return kush_append_ex(head_dim, bits, dtype, k, v, k_stride, v_stride, seq_lens, pos_offset, advance, tail_idx,
                          cache, block_stride, head_stride, tail_k, block_table, bt_stride, hkv, n_seqs, stream, 0);
}

extern "C" int kush_write(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                          int64_t v_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                          const int32_t* tail_idx, const int32_t* job_seq, const int32_t* job_page, int32_t n_jobs,
                          int32_t mode, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                          const int32_t* block_table, int64_t bt_stride, int32_t hkv, void* stream) {
    return kush_write_ex(head_dim, bits, dtype, k, v, k_stride, v_stride, query_start_loc, seq_lens, tail_idx, job_seq,
                         job_page, n_jobs, mode, cache, block_stride, head_stride, tail_k, block_table, bt_stride, hkv,
                         stream, 0);
}
