/* kushkash_amd host library (kushkash_amd/libkushcpu.so, built from csrc/kush_cpu.cpp with g++ and
 * OpenMP): the page-record kernels on the CPU, for Ops and KushCache on device "cpu".
 *
 * It keeps the C ABI of the reference's CPU library, libkush_cpu.so (kush/cpu.mojo:476-562, bound by
 * kushkash/_cpu.py:10-25), so a binding written for that library loads this one unchanged: every
 * argument is an int64 (addresses as integers) except the decode's softmax scale (float), inputs and
 * outputs are fp32, and each entry point returns 0, or -1 for a head dim other than 64 / 128 / 256 or
 * bits other than 4 / 8 (the reference raises ValueError on it, kushkash/_cpu.py:38-40).
 *
 * Records, K tails, block tables and lengths have the GPU library's layout (kushkash_amd.h), with the
 * K tail in fp32. Records are byte-identical to the GPU kernels' for the same fp32 input.
 */
#ifndef KUSHKASH_AMD_CPU_H
#define KUSHKASH_AMD_CPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One new token per sequence: K row into the tail, V row into the record, the K page on completion.
 * Replaces kush_cpu_append (cpu.mojo:476-495). */
int32_t kush_cpu_append(int64_t head_dim, int64_t bits, int64_t k, int64_t v, int64_t k_row_stride,
                        int64_t v_row_stride, int64_t seq_lens, int64_t pos_offset, int64_t advance, int64_t cache,
                        int64_t block_stride, int64_t head_stride, int64_t tail_k, int64_t tail_idx,
                        int64_t block_table, int64_t bt_row_stride, int64_t hkv, int64_t n_seqs);

/* Ragged chunk write over page jobs: mode 0 completed pages and V rows, mode 1 K rows of partial pages
 * into the tail. Replaces kush_cpu_write (cpu.mojo:497-515). */
int32_t kush_cpu_write(int64_t head_dim, int64_t bits, int64_t k, int64_t v, int64_t k_row_stride,
                       int64_t v_row_stride, int64_t query_start_loc, int64_t seq_lens, int64_t job_seq,
                       int64_t job_page, int64_t n_jobs, int64_t mode, int64_t cache, int64_t block_stride,
                       int64_t head_stride, int64_t tail_k, int64_t tail_idx, int64_t block_table,
                       int64_t bt_row_stride, int64_t hkv);

/* Decode attention of one query row per q head over each sequence's records and K tail.
 * Replaces kush_cpu_decode (cpu.mojo:517-532). */
int32_t kush_cpu_decode(int64_t head_dim, int64_t bits, int64_t q, int64_t out, int64_t cache,
                        int64_t block_stride, int64_t head_stride, int64_t tail_k, int64_t tail_idx,
                        int64_t block_table, int64_t seq_lens, int64_t bt_row_stride, int64_t hkv, int64_t group,
                        float scale, int64_t n_seqs);

/* Walsh-Hadamard rotation of `rows` contiguous fp32 rows in place (its own inverse).
 * Replaces kush_cpu_fwht (cpu.mojo:534-543). */
int32_t kush_cpu_fwht(int64_t head_dim, int64_t x, int64_t rows);

/* Prefill unpack of records, partial pages and new rows into packed fp32 K / V rows.
 * Replaces kush_cpu_unpack (cpu.mojo:545-562). */
int32_t kush_cpu_unpack(int64_t head_dim, int64_t bits, int64_t cache, int64_t block_stride, int64_t head_stride,
                        int64_t hkv, int64_t page_blk, int64_t page_dst, int64_t n_pages, int64_t tail_blk,
                        int64_t tail_info, int64_t n_tail, int64_t tail_k, int64_t k_new, int64_t v_new,
                        int64_t k_row_stride, int64_t v_row_stride, int64_t new_dst, int64_t n_new, int64_t kp,
                        int64_t vp, int64_t rot);

/* No counterpart in the reference: the library's fp32 -> fp16 rounding (round to nearest even) of n
 * values into their bit patterns, so tests can pin the scales' conversion. */
int32_t kush_cpu_half_bits(int64_t x, int64_t out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif /* KUSHKASH_AMD_CPU_H */
