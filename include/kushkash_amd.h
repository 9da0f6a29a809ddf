/*
 * kushkash_amd.h — C ABI of the MI355X (gfx950) compressed-KV hot path: quantize-and-pack on
 * write and fused dequant decode attention over int4 / int8 page records.
 *
 * Library: kushkash_amd/libkushhip.so (hipcc, --offload-arch=gfx950). These entry points replace
 * the reference's kernel dispatch (kushkash/_cuda.py:60-103 Kernel(grid, block, *args) launching
 * Mojo PTX, and kushkash/_ops.py:42-213 Ops). Each argument keeps the meaning of the reference
 * kernel parameter it replaces; the reference's per-config specialisation (GpuConfig(head_dim,
 * bits, group, dtype), _build.py:112-149) becomes the leading head_dim / bits / group / dtype
 * arguments.
 *
 * Conventions (reference: _ops.py:6-15, gpu.mojo:1-12):
 *   - The caller owns every buffer; pointers are device addresses. No entry point allocates,
 *     synchronizes or checks index values: launches are asynchronous on `stream` (a hipStream_t,
 *     NULL = default stream) and safe to record into a HIP graph.
 *   - cache: record of (block b, kv head h) at cache + b*block_stride + h*head_stride (bytes);
 *     records, block_stride and head_stride must be 16-byte aligned.
 *   - Record layout [kq 32*DC | vq 32*DC | ks D fp16 | kb D fp16 | vs 32 fp16 | vb 32 fp16],
 *     DC = D (int8) or D/2 (int4); record bytes = 64*DC + 4*D + 128.
 *   - tail_k: [slots][hkv][32][D] in dtype, exact K of each sequence's partial page; sequence s
 *     uses slot tail_idx[s].
 *   - k, v rows: row r, kv head h at base + r*row_stride + h*D (elements); q, out contiguous
 *     [n_seqs][hkv*group][D] (q head = kv_head*group + g).
 *   - block_table: int32 [n_seqs][bt_row_stride]; seq_lens int32 [n_seqs].
 *   - dtype codes: 0 fp32, 1 fp16, 2 bf16 (for q, k, v, out and tail_k).
 *   - head_dim 64, 128 or 256; bits 4 or 8; any group >= 1.
 *
 * Return values: 0 success; KUSH_EUNSUPPORTED for a head_dim / bits / dtype outside the
 * supported set (the reference's -1 -> ValueError, _cpu.py:38-40); KUSH_EINVAL for a rejected
 * argument; KUSH_EHIP for a launch error (the reference's RuntimeError with the driver string,
 * _cuda.py:39-43). kush_last_error() returns the message of the last failure on this thread.
 */
#ifndef KUSHKASH_AMD_H
#define KUSHKASH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KUSH_OK 0
#define KUSH_EUNSUPPORTED (-1)
#define KUSH_EINVAL (-2)
#define KUSH_EHIP (-3)

#define KUSH_DTYPE_F32 0
#define KUSH_DTYPE_F16 1
#define KUSH_DTYPE_BF16 2

/* Argument lists. Each entry point that replaces a reference kernel takes the reference's launch
 * arguments in the reference's order, ending with the stream (the argument sets of the reference's
 * kernels, gpu.mojo:207-212, :241-246, :566-572, :469-471, and of its CPU library, _cpu.py:12-19).
 * Where this library offers more, an `_ex` variant takes the same list followed by the extensions,
 * after the stream; the plain entry point is the `_ex` one with every extension at its default. */

/* One new token per sequence (decode step): row s of k / v goes to position
 * seq_lens[s] + pos_offset; negative positions (padding rows) are skipped. K goes to the exact
 * tail and its page is quantized when the token fills it; V is quantized straight into its
 * record row. advance != 0 stores pos + 1 back into seq_lens[s].
 * Replaces kush_append (gpu.mojo:207-238) as launched by Ops.append (_ops.py:66-80). */
int kush_append(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_row_stride,
                int64_t v_row_stride, int32_t* seq_lens, int32_t pos_offset, int32_t advance,
                const int32_t* tail_idx, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                const int32_t* block_table, int64_t bt_row_stride, int32_t hkv, int32_t n_seqs, void* stream);

/* kush_append plus rot (no counterpart in the reference, which rotates with a GEMM outside the
 * kernels): 1 rotates each k / v row by the canonical Walsh-Hadamard transform, rounded to dtype,
 * before it is quantized or stashed (the bytes of kush_fwht on the rows followed by rot = 0); 0 is
 * kush_append. */
int kush_append_ex(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_row_stride,
                   int64_t v_row_stride, int32_t* seq_lens, int32_t pos_offset, int32_t advance,
                   const int32_t* tail_idx, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                   const int32_t* block_table, int64_t bt_row_stride, int32_t hkv, int32_t n_seqs, void* stream,
                   int32_t rot);

/* Ragged multi-token write, one launch per mode: sequence s owns rows
 * [query_start_loc[s], query_start_loc[s+1]) at positions ending at seq_lens[s] (already
 * counting them); job j covers logical page job_page[j] of sequence job_seq[j]. mode 0 writes V
 * rows and quantizes pages the chunk completes; mode 1 stashes the K rows of still-partial pages
 * in the tail. Call mode 0 for all jobs, then mode 1, on the same stream. mode 2 (no counterpart
 * in the reference) does both in one launch; it needs a job for every page each sequence's chunk
 * touches (the job list every caller of the reference builds, _ops.py:342-344).
 * Replaces kush_write (gpu.mojo:241-276) as launched by Ops.write (_ops.py:82-101). */
int kush_write(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_row_stride,
               int64_t v_row_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
               const int32_t* tail_idx, const int32_t* job_seq, const int32_t* job_page, int32_t n_jobs,
               int32_t mode, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
               const int32_t* block_table, int64_t bt_row_stride, int32_t hkv, void* stream);

/* kush_write plus rot, as in kush_append_ex (rows from the chunk are rotated; rows read back from a
 * tail are rotated already). */
int kush_write_ex(int head_dim, int bits, int dtype, const void* k, const void* v, int64_t k_row_stride,
                  int64_t v_row_stride, const int32_t* query_start_loc, const int32_t* seq_lens,
                  const int32_t* tail_idx, const int32_t* job_seq, const int32_t* job_page, int32_t n_jobs,
                  int32_t mode, void* cache, int64_t block_stride, int64_t head_stride, void* tail_k,
                  const int32_t* block_table, int64_t bt_row_stride, int32_t hkv, void* stream, int32_t rot);

/* Decode attention of one query per sequence over its seq_lens[s] cached tokens, softmax scale
 * `scale`. n_splits == 1 writes out. n_splits > 1 splits every sequence's pages into n_splits
 * contiguous ranges (ceil(full pages / n_splits) each, the partial page in the last) and writes
 * per-split partials: part_ml fp32 [n_seqs*hkv*n_splits*group][2] (running max in log2 units, sum)
 * and part_o fp32 [n_seqs*hkv*n_splits*group][head_dim] (unnormalized), the reference's `work`
 * layout (_ops.py:204-208); kush_combine then writes out. q and tail_k must be 16-byte aligned.
 * Replaces kush_decode_tc / kush_decode (gpu.mojo:566-807, :840-1040) as issued by Ops.decode
 * (_ops.py:191-213). */
int kush_decode(int head_dim, int bits, int group, int dtype, const void* q, void* out, const void* cache,
                int64_t block_stride, int64_t head_stride, const void* tail_k, const int32_t* tail_idx,
                const int32_t* block_table, const int32_t* seq_lens, int64_t bt_row_stride, int32_t hkv, float scale,
                int32_t n_splits, float* part_ml, float* part_o, int32_t n_seqs, void* stream);

/* kush_decode plus (none has a reference counterpart; kush_decode passes 0 / NULL for each):
 * bt_cols: entries per block_table row that may be read (the table's column count), or 0 when
 *   unknown; with it the first block ids of split 0 are fetched before seq_lens is read (a shorter
 *   dependent chain at the start of every workgroup); with 0 only entries below seq_lens are read.
 * split_sync: NULL, or int32 [n_seqs*hkv*ceil(group/16)], zero before the first call: the last
 *   workgroup of each (sequence, kv head) merges the splits into out itself and resets its counter,
 *   so the buffer stays zero between calls and no kush_combine is needed; calls that share
 *   split_sync must not overlap.
 * waves: 2, 4 or 8 waves per workgroup (0 = 4; a configuration whose page ring does not fit in LDS
 *   runs fewer). Every choice is deterministic: the same call gives the same bits.
 * seq_order: NULL, or int32 [n_seqs] holding a permutation of the sequences: their workgroups start
 *   in that order (longest first balances a ragged batch); the results do not depend on it.
 * rot: 1 for a cache written with rot = 1: q is rotated by the canonical Walsh-Hadamard transform
 *   (rounded to dtype, as kush_fwht) on load and the output rotated back before its one rounding to
 *   dtype; the split partials stay unrotated (kush_combine_ex takes the same rot). */
int kush_decode_ex(int head_dim, int bits, int group, int dtype, const void* q, void* out, const void* cache,
                   int64_t block_stride, int64_t head_stride, const void* tail_k, const int32_t* tail_idx,
                   const int32_t* block_table, const int32_t* seq_lens, int64_t bt_row_stride, int32_t hkv,
                   float scale, int32_t n_splits, float* part_ml, float* part_o, int32_t n_seqs, void* stream,
                   int32_t bt_cols, int32_t* split_sync, int32_t waves, const int32_t* seq_order, int32_t rot);

/* kush_append (pos_offset = -1, advance = 0: row s of k / v is the token at position seq_lens[s] - 1,
 * which seq_lens already counts, the serving engines' convention) followed by kush_decode_ex, in one
 * launch: the workgroup that reads the token's page appends it first (same bytes as kush_append).
 * group <= 16 and 16-byte aligned k / v rows (otherwise -2: call the two entry points). No
 * reference counterpart (the reference launches kush_append then a decode kernel, gpu.mojo:207-238,
 * :566-807, as _ops.py:66-80 and :191-213 issue them); the arguments are kush_decode's, then the new
 * token's rows, then kush_decode_ex's extensions. */
int kush_append_decode(int head_dim, int bits, int group, int dtype, const void* q, void* out, void* cache,
                       int64_t block_stride, int64_t head_stride, void* tail_k, const int32_t* tail_idx,
                       const int32_t* block_table, const int32_t* seq_lens, int64_t bt_row_stride, int32_t hkv,
                       float scale, int32_t n_splits, float* part_ml, float* part_o, int32_t n_seqs, void* stream,
                       const void* k, const void* v, int64_t k_row_stride, int64_t v_row_stride, int32_t bt_cols,
                       int32_t* split_sync, int32_t waves, const int32_t* seq_order, int32_t rot);

/* kush_decode_ex without caller buffers: the split-K merge counters and partials live in a static
 * device array of the library (64 MiB per device, held until the process ends; its counters are
 * cleared once, by a fill kernel on `stream`, at the first call on each device). n_splits > 1 needs
 * n_seqs*hkv*ceil(group/16) <= 65536 counters and 262144 + 4*(head_dim+2)*n_seqs*hkv*n_splits*group
 * bytes <= 64 MiB (otherwise -2: use kush_decode_ex); the splits are always merged in the launch.
 * Calls share the array and must not overlap on one device; for graph capture, make the first call
 * on a device outside the capture. No counterpart in the reference: for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). */
int kush_decode_noalloc(int head_dim, int bits, int group, int dtype, const void* q, void* out, const void* cache,
                        int64_t block_stride, int64_t head_stride, const void* tail_k, const int32_t* tail_idx,
                        const int32_t* block_table, const int32_t* seq_lens, int64_t bt_row_stride, int32_t hkv,
                        float scale, int32_t n_splits, int32_t n_seqs, void* stream, int32_t bt_cols, int32_t waves,
                        const int32_t* seq_order, int32_t rot);

/* Walsh-Hadamard rotation of rows of head_dim elements: y[r] = fwht(x[r]) for r < rows (row strides
 * in elements; y may alias x), in the canonical order — butterflies at strides 1, 2, ..., D/2, then
 * one fp32 multiply by 1/sqrt(D), rounded once to dtype — bit-identical to the reference's CPU
 * and GPU rotation. bits is not a parameter (any record format).
 * Replaces kush_fwht (gpu.mojo:95-112) as launched by Ops.fwht (_ops.py:104-126). */
int kush_fwht(int head_dim, int dtype, const void* x, void* y, int64_t x_row_stride, int64_t y_row_stride,
              int64_t rows, void* stream);

/* Build one packed-prefill group's keys and values, kp / vp [rows][hkv][head_dim] in dtype
 * (contiguous), in one launch: full history pages (record of block page_blk[i] -> rows
 * page_dst[i] + 0..31), partial pages (tail_info[3i..3i+2] = first row, tokens 1..32, tail slot:
 * K rows from tail_k [slots][hkv][32][head_dim], V rows from the record of block tail_blk[i]) and
 * the new chunk (row j of k_new / v_new, element row strides k_stride / v_stride, head stride
 * head_dim -> row new_dst[j]). Dequantization is fma(code, scale, bias) in fp32; rot != 0 rotates
 * history rows back (canonical Walsh-Hadamard) before the one rounding to dtype; new rows are
 * copied. Rows no entry names are left untouched. Indices are not bounds-checked (the caller's
 * contract, as in the reference).
 * Replaces kush_unpack (gpu.mojo:303-375) as launched by Ops.unpack (_ops.py:128-180). */
int kush_unpack(int head_dim, int bits, int dtype, const void* cache, int64_t block_stride, int64_t head_stride,
                int32_t hkv, const int32_t* page_blk, const int32_t* page_dst, int64_t n_pages,
                const int32_t* tail_blk, const int32_t* tail_info, int64_t n_tail, const void* tail_k,
                const void* k_new, const void* v_new, int64_t k_stride, int64_t v_stride, const int32_t* new_dst,
                int64_t n_new, void* kp, void* vp, int32_t rot, void* stream);

/* Merge kush_decode's split partials into out [n_seqs][hkv*group][head_dim].
 * Replaces kush_combine (gpu.mojo:469-491) as launched by Ops.decode (_ops.py:212-213). */
int kush_combine(int head_dim, int group, int dtype, void* out, const float* part_ml, const float* part_o,
                 int32_t n_splits, int32_t hkv, int32_t n_seqs, void* stream);

/* kush_combine plus rot (as kush_decode_ex: the merged rows are rotated back before their rounding). */
int kush_combine_ex(int head_dim, int group, int dtype, void* out, const float* part_ml, const float* part_o,
                    int32_t n_splits, int32_t hkv, int32_t n_seqs, void* stream, int32_t rot);

/* Message of the last failing call on this thread ("" if none). No reference counterpart: the
 * reference raises the driver's error string directly (_cuda.py:39-43). */
const char* kush_last_error(void);

/* ABI revision of this header (8). No reference counterpart. */
int kush_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KUSHKASH_AMD_H */
