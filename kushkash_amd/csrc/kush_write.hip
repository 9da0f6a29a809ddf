// Quantize-and-pack on write for gfx950: one token per sequence (append) and ragged
// multi-token chunks (write). Reference contract: kushkash/kush/gpu.mojo:207-276 (kernels),
// kushkash/_ops.py:66-101 (launch), arithmetic kushkash/kush/quant.mojo:25-50. Pages are
// bit-identical to the reference CPU path (kushkash/kush/cpu.mojo:173-304).
//
// Work split on CDNA4 (wave64): a V token row is one wave (per-token range: wave min/max
// reduction, then each lane packs the bytes of its dims); a K page is one workgroup that stages
// the page's 32 x D values in LDS as fp32, reduces one channel per thread, and packs the codes
// with consecutive lanes writing consecutive bytes.
#include "kush_common.h"

namespace kush {

constexpr int WRITE_THREADS = 256;

// V token row src[0:D] -> row t of a record (its final encoding: per-token range).
template <int D, int BITS, typename IN>
__device__ __forceinline__ void quantize_v_row(const IN* __restrict__ src, uint8_t* __restrict__ rec, int t, int lane) {
    using F = Fmt<D, BITS>;
    constexpr int R = D / WAVE;            // values per lane: 1, 2 or 4
    float x[R];
    float mn = __builtin_inff(), mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        x[r] = to_f32(src[lane + WAVE * r]);
        mn = __builtin_fminf(mn, x[r]);
        mx = __builtin_fmaxf(mx, x[r]);
    }
    mn = wave_min(mn);
    mx = wave_max(mx);
    float s, b, inv;
    qparams<BITS>(mn, mx, s, b, inv);
    if (lane == 0) {
        reinterpret_cast<uint16_t*>(rec + F::OFF_VS)[t] = f16_bits(s);
        reinterpret_cast<uint16_t*>(rec + F::OFF_VB)[t] = f16_bits(b);
    }
    uint8_t* dst = rec + F::OFF_VQ + t * F::DC;
    if constexpr (BITS == 8) {
#pragma unroll
        for (int r = 0; r < R; ++r) dst[lane + WAVE * r] = (uint8_t)qcode<8>(x[r], b, inv);
    } else if constexpr (D == 64) {
        // byte j < 32 pairs dim j (this lane) with dim j + 32 (lane j + 32)
        float hi = __shfl_down(x[0], 32, WAVE);
        if (lane < 32) dst[lane] = pack4(qcode<4>(x[0], b, inv), qcode<4>(hi, b, inv));
    } else {
        // byte j = lane + 64 r pairs dim j with dim j + D/2 = lane + 64 (r + R/2): same lane
#pragma unroll
        for (int r = 0; r < R / 2; ++r)
            dst[lane + WAVE * r] = pack4(qcode<4>(x[r], b, inv), qcode<4>(x[r + R / 2], b, inv));
    }
}

// K of one page by a workgroup: per-channel range over its 32 rows. Row t < split comes from
// ka + t*sa (the exact tail), the rest from kb_src + (t - split)*skb (new rows). tile holds
// PAGE*D + 2*D floats of LDS.
template <int D, int BITS, typename IN, int NT>
__device__ __forceinline__ void quantize_k_page(const IN* __restrict__ ka, int64_t sa, const IN* __restrict__ kb_src,
                                                int64_t skb, int split, uint8_t* __restrict__ rec, float* tile) {
    using F = Fmt<D, BITS>;
    float* kbias = tile + PAGE * D;
    float* kinv = kbias + D;
    const int tid = threadIdx.x;
    for (int i = tid; i < PAGE * D; i += NT) {
        const int t = i / D, d = i % D;
        const IN* row = t < split ? ka + t * sa : kb_src + (t - split) * skb;
        tile[i] = to_f32(row[d]);
    }
    __syncthreads();
    for (int c = tid; c < D; c += NT) {
        float mn = __builtin_inff(), mx = -__builtin_inff();
#pragma unroll 8
        for (int t = 0; t < PAGE; ++t) {
            const float x = tile[t * D + c];
            mn = __builtin_fminf(mn, x);
            mx = __builtin_fmaxf(mx, x);
        }
        float s, b, inv;
        qparams<BITS>(mn, mx, s, b, inv);
        reinterpret_cast<uint16_t*>(rec + F::OFF_KS)[c] = f16_bits(s);
        reinterpret_cast<uint16_t*>(rec + F::OFF_KB)[c] = f16_bits(b);
        kbias[c] = b;
        kinv[c] = inv;
    }
    __syncthreads();
    for (int i = tid; i < PAGE * F::DC; i += NT) {
        const int t = i / F::DC, j = i % F::DC;
        uint8_t byte;
        if constexpr (BITS == 8) {
            byte = (uint8_t)qcode<8>(tile[t * D + j], kbias[j], kinv[j]);
        } else {
            byte = pack4(qcode<4>(tile[t * D + j], kbias[j], kinv[j]),
                         qcode<4>(tile[t * D + j + D / 2], kbias[j + D / 2], kinv[j + D / 2]));
        }
        rec[t * F::DC + j] = byte;
    }
    __syncthreads();   // tile is reused by the next call
}

// grid (S), block 256. One token per sequence at position seq_lens[s] + pos_offset; negative
// positions (padding rows) are skipped. K goes to the exact tail (quantized when its page
// fills), V straight into its record row. Contract: gpu.mojo:207-238, cpu.mojo:248-270.
template <int D, int BITS, typename IN>
__global__ __launch_bounds__(WRITE_THREADS) void append_kernel(
    const IN* __restrict__ k, const IN* __restrict__ v, int64_t k_stride, int64_t v_stride, int32_t* seq_lens,
    int pos_offset, int advance, const int32_t* __restrict__ tail_idx, uint8_t* __restrict__ cache, int64_t bs,
    int64_t hs, IN* __restrict__ tail_k, const int32_t* __restrict__ block_table, int64_t bt_stride, int H) {
    __shared__ float tile[PAGE * D + 2 * D];
    const int s = blockIdx.x;
    const int pos = seq_lens[s] + pos_offset;
    if (pos < 0) return;
    const int slot = pos % PAGE;
    const int64_t blk = block_table[(int64_t)s * bt_stride + pos / PAGE];
    const int64_t tb = (int64_t)tail_idx[s] * H * PAGE * D;
    const IN* krow = k + (int64_t)s * k_stride;
    const IN* vrow = v + (int64_t)s * v_stride;
    for (int i = threadIdx.x; i < H * D; i += WRITE_THREADS) {
        const int h = i / D, d = i % D;
        tail_k[tb + ((int64_t)h * PAGE + slot) * D + d] = krow[(int64_t)h * D + d];
    }
    const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    for (int h = wave; h < H; h += WRITE_THREADS / WAVE)
        quantize_v_row<D, BITS, IN>(vrow + (int64_t)h * D, cache + blk * bs + (int64_t)h * hs, slot, lane);
    if (slot == PAGE - 1) {
        // rows 0..30 were stashed in the tail by earlier steps; row 31 is this token
        for (int h = 0; h < H; ++h)
            quantize_k_page<D, BITS, IN, WRITE_THREADS>(tail_k + tb + (int64_t)h * PAGE * D, D, krow + (int64_t)h * D, 0,
                                                        PAGE - 1, cache + blk * bs + (int64_t)h * hs, tile);
    }
    __syncthreads();   // every thread has read seq_lens[s]
    if (advance && threadIdx.x == 0) seq_lens[s] = pos + 1;
}

// grid (n_jobs, Hkv), block 256. Job j covers logical page job_page[j] of sequence job_seq[j],
// whose new rows [qsl[s], qsl[s+1]) sit at positions [ctx, seq_lens[s]).
// mode 0: write the page's new V rows; if the page is complete, quantize its K (older rows from
// the tail, newer from the chunk). mode 1: stash the new K rows of a still-partial page in the
// tail. Launched as mode 0 then mode 1 so no tail is read and written by the same launch.
// Contract: gpu.mojo:241-276, cpu.mojo:273-304.
template <int D, int BITS, typename IN>
__global__ __launch_bounds__(WRITE_THREADS) void write_kernel(
    const IN* __restrict__ k, const IN* __restrict__ v, int64_t k_stride, int64_t v_stride,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ seq_lens, const int32_t* __restrict__ tail_idx,
    const int32_t* __restrict__ job_seq, const int32_t* __restrict__ job_page, int mode, uint8_t* __restrict__ cache,
    int64_t bs, int64_t hs, IN* __restrict__ tail_k, const int32_t* __restrict__ block_table, int64_t bt_stride, int H) {
    __shared__ float tile[PAGE * D + 2 * D];
    const int j = blockIdx.x, h = blockIdx.y;
    const int s = job_seq[j];
    const int ps = job_page[j] * PAGE;
    const int q0 = qsl[s];
    const int total = seq_lens[s];
    const int ctx = total - (qsl[s + 1] - q0);
    const bool complete = ps + PAGE <= total;
    const int64_t tb = ((int64_t)tail_idx[s] * H + h) * PAGE * D;
    const int lo = ps > ctx ? ps : ctx;
    if (mode == 0) {
        uint8_t* rec = cache + (int64_t)block_table[(int64_t)s * bt_stride + ps / PAGE] * bs + (int64_t)h * hs;
        const int hi = ps + PAGE < total ? ps + PAGE : total;
        const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
        for (int t = lo + wave; t < hi; t += WRITE_THREADS / WAVE)
            quantize_v_row<D, BITS, IN>(v + (int64_t)(q0 + t - ctx) * v_stride + (int64_t)h * D, rec, t - ps, lane);
        if (complete) {
            int split = ctx - ps;
            split = split < 0 ? 0 : (split > PAGE ? PAGE : split);
            quantize_k_page<D, BITS, IN, WRITE_THREADS>(tail_k + tb, D,
                                                        k + (int64_t)(q0 + ps + split - ctx) * k_stride + (int64_t)h * D,
                                                        k_stride, split, rec, tile);
        }
    } else {
        if (complete) return;
        const int n = total - lo;
        for (int i = threadIdx.x; i < n * D; i += WRITE_THREADS) {
            const int t = lo + i / D, d = i % D;
            tail_k[tb + (int64_t)(t - ps) * D + d] = k[(int64_t)(q0 + t - ctx) * k_stride + (int64_t)h * D + d];
        }
    }
}

}  // namespace kush

using namespace kush;

extern "C" int kush_append(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                           int64_t v_stride, int32_t* seq_lens, int32_t pos_offset, int32_t advance,
                           const int32_t* tail_idx, void* cache, int64_t block_stride, int64_t head_stride,
                           void* tail_k, const int32_t* block_table, int64_t bt_stride, int32_t hkv, int32_t n_seqs,
                           void* stream) {
    if (n_seqs < 0 || hkv <= 0) return kush_fail(-2, "kush_append: bad n_seqs %d / hkv %d", n_seqs, hkv);
    return dispatch_shape(head_dim, bits, dtype, "kush_append", [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        if (n_seqs == 0) return 0;
        append_kernel<D, BITS, IN><<<dim3(n_seqs), dim3(WRITE_THREADS), 0, (hipStream_t)stream>>>(
            (const IN*)k, (const IN*)v, k_stride, v_stride, seq_lens, pos_offset, advance, tail_idx, (uint8_t*)cache,
            block_stride, head_stride, (IN*)tail_k, block_table, bt_stride, hkv);
        return kush_check_launch("kush_append");
    });
}

extern "C" int kush_write(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_stride,
                          int64_t v_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                          const int32_t* tail_idx, const int32_t* job_seq, const int32_t* job_page, int32_t n_jobs,
                          int32_t mode, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                          const int32_t* block_table, int64_t bt_stride, int32_t hkv, void* stream) {
    if (n_jobs < 0 || hkv <= 0 || (mode != 0 && mode != 1))
        return kush_fail(-2, "kush_write: bad n_jobs %d / hkv %d / mode %d", n_jobs, hkv, mode);
    return dispatch_shape(head_dim, bits, dtype, "kush_write", [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        if (n_jobs == 0) return 0;
        write_kernel<D, BITS, IN><<<dim3(n_jobs, hkv), dim3(WRITE_THREADS), 0, (hipStream_t)stream>>>(
            (const IN*)k, (const IN*)v, k_stride, v_stride, query_start_loc, seq_lens, tail_idx, job_seq, job_page,
            mode, (uint8_t*)cache, block_stride, head_stride, (IN*)tail_k, block_table, bt_stride, hkv);
        return kush_check_launch("kush_write");
    });
}
