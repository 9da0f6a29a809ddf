// Fused dequant decode attention over int4/int8 page records for gfx950 (CDNA4), with split-K
// partials and a log-sum-exp combine. Contract: kushkash/kush/gpu.mojo:566-807 (decode),
// :418-491 (split ranges, merge, combine), kushkash/_ops.py:182-213 (launch), arithmetic of the
// reference CPU path kushkash/kush/cpu.mojo:320-451.
//
// Mapping onto CDNA4. One workgroup = NW waves for one (sequence, kv head, split, 16-head
// chunk); its waves take the split's pages round-robin, each keeping its own online-softmax
// state, and merge through LDS at the end. Per page a wave:
//   1. loads its K code slice straight into registers (lane (t, q): row t of a 16-token tile,
//      bytes [q*DC/4, (q+1)*DC/4): the 64 lanes read 16 contiguous rows) and copies the V codes
//      and the page's scales / biases into a wave-private LDS stage with 16-byte loads;
//   2. turns codes into exact fp16 with v_perm (byte under the fp16 exponent of 1024) and one
//      packed subtract, and computes S^T = K . Q'^T on MFMA 16x16x32 f16, where
//      Q' = fp16(q * sm * log2 e) * k_scale (fp16) and the K bias dot stays fp32 (v_dot2 on a
//      hi/lo fp16 split of q);
//   3. runs a page-granular online softmax in base 2 (wave shuffles over the 4 lane groups);
//   4. reads V codes column-wise from LDS (8 tokens per lane) into V^T operands and
//      accumulates O^T += V^T . P'^T on MFMA, with P' = e * v_scale in fp16 and the V bias
//      folded into one scalar per head.
// The partial last page takes K from the exact tail (fp32 dot products) and V rows from its
// record, masked beyond the tail length.
//
// MFMA 16x16x32 f16 operand layout used throughout (lane l, r = l % 16, q = l / 16):
//   A: row r, 8 contraction slots of lane group q;  B: column r, the same 8 slots;
//   C: rows 4q .. 4q+3 of column r.
// Which physical dim or token a slot stands for is chosen here (kdim, tok), identically for A
// and B, so only the C layout is relied upon.
#include "kush_common.h"

namespace kush {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4v __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));

constexpr float LOG2E = 1.4426950408889634f;

__device__ __forceinline__ h2 as_h2(uint32_t x) { return __builtin_bit_cast(h2, x); }

// Four two's-complement nibble codes per byte pair of w -> exact fp16. Slots 0-3: low nibbles of
// bytes 0-3, slots 4-7: high nibbles. n ^ 8 = c + 8 for a signed nibble c; placed under the fp16
// exponent of 1024 it reads 1024 + c + 8, and one packed subtract leaves c.
__device__ __forceinline__ h8 int4_codes(uint32_t w) {
    const uint32_t x = w ^ 0x88888888u;
    const uint32_t lo = x & 0x0F0F0F0Fu, hi = (x >> 4) & 0x0F0F0F0Fu;
    const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const h2 a = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04010400u)) + off;
    const h2 b = as_h2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030402u)) + off;
    const h2 c = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04010400u)) + off;
    const h2 d = as_h2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030402u)) + off;
    return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Eight signed int8 codes (two words) -> exact fp16 (c + 128 under the exponent of 1024).
__device__ __forceinline__ h8 int8_codes(uint32_t w0, uint32_t w1) {
    const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
    const h2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const h2 a = as_h2(__builtin_amdgcn_perm(0x64646464u, x0, 0x04010400u)) + off;
    const h2 b = as_h2(__builtin_amdgcn_perm(0x64646464u, x0, 0x04030402u)) + off;
    const h2 c = as_h2(__builtin_amdgcn_perm(0x64646464u, x1, 0x04010400u)) + off;
    const h2 d = as_h2(__builtin_amdgcn_perm(0x64646464u, x1, 0x04030402u)) + off;
    return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// Physical dim of contraction slot j of lane group q in K-step kk (QK^T). int4: the lane's 16-byte
// slice of a row holds dims [q D/8, (q+1) D/8) in low nibbles and the same + D/2 in high nibbles;
// K-step kk takes bytes 4kk..4kk+3 of it. int8: dims q D/4 + 8 kk + j.
template <int D, int BITS>
__device__ __forceinline__ int kdim(int kk, int q, int j) {
    if constexpr (BITS == 4)
        return (j < 4 ? 0 : D / 2) + q * (D / 8) + 4 * kk + (j & 3);
    else
        return q * (D / 4) + 8 * kk + j;
}

// Token of slot j of lane group q in the PV contraction: the token the QK^T accumulators of lane
// group q hold in register j % 4 of tile j / 4.
__device__ __forceinline__ int tok(int q, int j) { return 16 * (j >> 2) + 4 * q + (j & 3); }

template <int D, int BITS>
struct Stage {                                     // wave-private LDS copy of a record's tail part
    using F = Fmt<D, BITS>;
    static constexpr int BYTES = F::REC - F::OFF_VQ;   // V codes + ks + kb + vs + vb
    static constexpr int CHUNKS = BYTES / 16;
    static constexpr int KS = F::OFF_KS - F::OFF_VQ;
    static constexpr int KB = F::OFF_KB - F::OFF_VQ;
    static constexpr int VS = F::OFF_VS - F::OFF_VQ;
    static constexpr int VB = F::OFF_VB - F::OFF_VQ;
};

template <int D, int BITS>
__device__ __forceinline__ void stage_record(const uint8_t* __restrict__ rec, uint8_t* st, int lane) {
    using F = Fmt<D, BITS>;
    using S = Stage<D, BITS>;
    const uint4* src = reinterpret_cast<const uint4*>(rec + F::OFF_VQ);
    uint4* dst = reinterpret_cast<uint4*>(st);
#pragma unroll
    for (int i = 0; i < (S::CHUNKS + WAVE - 1) / WAVE; ++i) {
        const int c = lane + WAVE * i;
        if (c < S::CHUNKS) dst[c] = src[c];
    }
}

// max / sum over the 4 lanes l, l ^ 16, l ^ 32, l ^ 48 (one q head's lane groups), on the VALU
__device__ __forceinline__ float rows_max(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __builtin_fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows_sum(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

// V^T operand gather: within each 16-lane group, ds_read_b64_tr_b8 hands output lane i byte
// (i % 8) of the 8-byte rows supplied by lanes 2k + (i % 16) / 8, k = 0..7. Lane (2k + half) of
// group q supplies token tok(q, k) at byte column 16 ct + 8 half, so lane r of the group receives
// byte column 16 ct + r of its 8 tokens, in PV slot order.
__device__ __forceinline__ v2i gather_vt(const uint8_t* st, int dc, int ct, int lane) {
    const int s16 = lane & 15, q = lane >> 4;
    const uint8_t* src = st + tok(q, s16 >> 1) * dc + 16 * ct + 8 * (s16 & 1);
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(src));
}

// Softmax update of one page (scores x in log2 units, tokens tok(q, j); tokens >= valid masked)
// and its PV accumulation from the staged V codes.
template <int D, int BITS>
__device__ __forceinline__ void consume_page(const uint8_t* st, f4 (&o)[D / 16], const float (&x)[8], int valid,
                                             float& m_run, float& l_run, float& vb_run, int lane) {
    using F = Fmt<D, BITS>;
    using S = Stage<D, BITS>;
    const int q = lane >> 4;
    float pm = x[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) pm = __builtin_fmaxf(pm, x[j]);
    const float m_new = __builtin_fmaxf(m_run, rows_max(pm));
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);   // first page: exp2(-inf) = 0

    const h4v vs0 = *reinterpret_cast<const h4v*>(st + S::VS + 8 * q);
    const h4v vs1 = *reinterpret_cast<const h4v*>(st + S::VS + 32 + 8 * q);
    const h4v vb0 = *reinterpret_cast<const h4v*>(st + S::VB + 8 * q);
    const h4v vb1 = *reinterpret_cast<const h4v*>(st + S::VB + 32 + 8 * q);
    float lsum = 0.0f, vbsum = 0.0f;
    h8 pw;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const bool ok = tok(q, j) < valid;
        const float vsj = (float)(j < 4 ? vs0[j] : vs1[j - 4]);
        const float vbj = (float)(j < 4 ? vb0[j] : vb1[j - 4]);
        const float e = ok ? __builtin_amdgcn_exp2f(x[j] - m_new) : 0.0f;
        lsum += e;
        vbsum += ok ? e * vbj : 0.0f;
        pw[j] = (_Float16)(ok ? e * vsj : 0.0f);
    }
    l_run = l_run * corr + lsum;
    vb_run = vb_run * corr + vbsum;
    m_run = m_new;
    if (corr != 1.0f) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) o[dt] *= corr;
    }

    constexpr int NCOL = BITS == 4 ? D / 32 : D / 16;
#pragma unroll
    for (int ct = 0; ct < NCOL; ++ct) {
        const v2i w = gather_vt(st, F::DC, ct, lane);
        if constexpr (BITS == 4) {
            const uint32_t x0 = (uint32_t)w[0] ^ 0x88888888u, x1 = (uint32_t)w[1] ^ 0x88888888u;
            const uint32_t l0 = x0 & 0x0F0F0F0Fu, l1 = x1 & 0x0F0F0F0Fu;
            const uint32_t u0 = (x0 >> 4) & 0x0F0F0F0Fu, u1 = (x1 >> 4) & 0x0F0F0F0Fu;
            const h2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
            const h2 a = as_h2(__builtin_amdgcn_perm(0x64646464u, l0, 0x04010400u)) + off;
            const h2 b = as_h2(__builtin_amdgcn_perm(0x64646464u, l0, 0x04030402u)) + off;
            const h2 c = as_h2(__builtin_amdgcn_perm(0x64646464u, l1, 0x04010400u)) + off;
            const h2 d = as_h2(__builtin_amdgcn_perm(0x64646464u, l1, 0x04030402u)) + off;
            const h2 e = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) + off;
            const h2 f = as_h2(__builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) + off;
            const h2 g = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) + off;
            const h2 hh = as_h2(__builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) + off;
            o[ct] = mfma16(h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]}, pw, o[ct]);
            o[ct + D / 32] = mfma16(h8{e[0], e[1], f[0], f[1], g[0], g[1], hh[0], hh[1]}, pw, o[ct + D / 32]);
        } else {
            o[ct] = mfma16(int8_codes((uint32_t)w[0], (uint32_t)w[1]), pw, o[ct]);
        }
    }
}

// grid (S, Hkv, n_splits * ceil(G / 16)), block NW * 64.
// NS > 1: each workgroup writes its split's partials; with `sync` (one zeroed int32 per
// (sequence, kv head, head chunk)), the last workgroup of a (sequence, kv head, head chunk) to
// finish merges all splits into `out` and resets its counter, so no second launch is needed.
template <int D, int BITS, typename IN, int NW, int PF>
__global__ __launch_bounds__(NW * WAVE) void decode_kernel(
    const IN* __restrict__ qg, IN* __restrict__ out, const uint8_t* __restrict__ cache, int64_t bs, int64_t hs,
    const IN* __restrict__ tail_k, const int32_t* __restrict__ tail_idx, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ seq_lens, int64_t bt_stride, int H, int G, float sm_log2, int NS,
    float* __restrict__ part_ml, float* __restrict__ part_o, int32_t* __restrict__ sync) {
    using F = Fmt<D, BITS>;
    using S = Stage<D, BITS>;
    constexpr int KSTEPS = D / 32;
    constexpr int DT = D / 16;
    constexpr int KBYTES = F::DC / 4;                // K code bytes per lane per 16-token tile
    constexpr int KW = KBYTES / 4;
    constexpr int STAGE = S::BYTES;
    constexpr int VCPL = (S::CHUNKS + WAVE - 1) / WAVE;

    __shared__ __align__(16) uint8_t stage_all[NW * STAGE];
    __shared__ __align__(16) h8 qhl[KSTEPS * WAVE];   // fp16(q sm log2e) in each lane's contraction order
    __shared__ __align__(16) h8 qll[KSTEPS * WAVE];   // fp16 remainder: hi + lo carries q to ~2^-22
    __shared__ __align__(16) float qs_l[16 * D];     // fp32 q sm log2e for the exact-K tail; then merge buffer
    __shared__ float sc_l[16 * PAGE];                // tail scores
    __shared__ float m_l[NW * 16], l_l[NW * 16];
    __shared__ int last_flag;

    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);   // wave-uniform: scalar page loop
    const int r16 = lane & 15, q = lane >> 4;
    const int s = blockIdx.x, h = blockIdx.y;
    const int z = blockIdx.z % NS, gc = blockIdx.z / NS, g0 = gc * 16;
    const int Gc = min(16, G - g0);

    const int n = seq_lens[s];
    const int full = n / PAGE, tail_n = n % PAGE;
    const int pps = (full + NS - 1) / NS;
    const int p0 = min(full, z * pps), p1 = min(full, p0 + pps);
    const int32_t* bt = block_table + (int64_t)s * bt_stride;
    const uint8_t* head_base = cache + (int64_t)h * hs;
    const int64_t qbase = ((int64_t)s * H + h) * G * D + (int64_t)g0 * D;
    const bool has_tail = tail_n > 0 && z == NS - 1;
    uint8_t* st = stage_all + w * STAGE;

    // PF pages in flight per wave: K code slices in registers, V codes + scales staged through
    // registers, one ring slot per page; the loop is unrolled over the ring so slots stay in VGPRs.
    uint32_t kwn[PF][2][KW];
    u4 vn[PF][VCPL];
#define KUSH_ISSUE(SLOT_, BLK_)                                                                          \
    do {                                                                                                 \
        const uint8_t* rec_ = head_base + (int64_t)(BLK_) * bs;                                          \
        _Pragma("unroll") for (int tt = 0; tt < 2; ++tt) {                                               \
            const uint8_t* src_ = rec_ + (16 * tt + r16) * F::DC + q * KBYTES;                           \
            if constexpr (KBYTES == 8) {                                                                 \
                const u2 v2_ = *reinterpret_cast<const u2*>(src_);                                       \
                kwn[SLOT_][tt][0] = v2_[0];                                                              \
                kwn[SLOT_][tt][1] = v2_[1];                                                              \
            } else {                                                                                     \
                _Pragma("unroll") for (int c = 0; c < KBYTES / 16; ++c) {                                \
                    const u4 v4_ = reinterpret_cast<const u4*>(src_)[c];                                 \
                    kwn[SLOT_][tt][4 * c + 0] = v4_[0];                                                  \
                    kwn[SLOT_][tt][4 * c + 1] = v4_[1];                                                  \
                    kwn[SLOT_][tt][4 * c + 2] = v4_[2];                                                  \
                    kwn[SLOT_][tt][4 * c + 3] = v4_[3];                                                  \
                }                                                                                        \
            }                                                                                            \
        }                                                                                                \
        const u4* vsrc_ = reinterpret_cast<const u4*>(rec_ + F::OFF_VQ);                                 \
        _Pragma("unroll") for (int i = 0; i < VCPL; ++i) {                                               \
            const int c = lane + WAVE * i;                                                               \
            vn[SLOT_][i] = c < S::CHUNKS ? vsrc_[c < S::CHUNKS ? c : 0] : u4{0u, 0u, 0u, 0u};            \
        }                                                                                                \
    } while (0)

    // the first pages are requested before the q prologue so their latency overlaps it
    int32_t bnext[PF];                       // block ids of the round after the one in flight
#pragma unroll
    for (int slot = 0; slot < PF; ++slot) {
        const int pp = p0 + w + slot * NW, pn = pp + PF * NW;
        if (pp < p1) KUSH_ISSUE(slot, bt[pp]);
        bnext[slot] = pn < p1 ? bt[pn] : 0;
    }

    for (int i = threadIdx.x; i < KSTEPS * WAVE * 8; i += NW * WAVE) {
        const int kk = i / (WAVE * 8), l = (i / 8) % WAVE, j = i % 8;
        const int g = l & 15;
        const float xq = g < Gc ? to_f32(qg[qbase + (int64_t)g * D + kdim<D, BITS>(kk, l >> 4, j)]) * sm_log2 : 0.0f;
        const _Float16 hi = (_Float16)xq;
        reinterpret_cast<_Float16*>(&qhl[kk * WAVE + l])[j] = hi;
        reinterpret_cast<_Float16*>(&qll[kk * WAVE + l])[j] = (_Float16)(xq - (float)hi);
    }
    if (has_tail) {
        for (int i = threadIdx.x; i < 16 * D; i += NW * WAVE)
            qs_l[i] = i / D < Gc ? to_f32(qg[qbase + i]) * sm_log2 : 0.0f;
    }
    __syncthreads();

    f4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -__builtin_inff(), l_run = 0.0f, vb_run = 0.0f;

    for (int pb = p0 + w; pb < p1; pb += PF * NW) {
#pragma unroll
        for (int slot = 0; slot < PF; ++slot) {
            const int p = pb + slot * NW;
            if (p >= p1) break;
            uint32_t kw[2][KW];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt)
#pragma unroll
                for (int i = 0; i < KW; ++i) kw[tt][i] = kwn[slot][tt][i];
#pragma unroll
            for (int i = 0; i < VCPL; ++i) {
                const int c = lane + WAVE * i;
                if (c < S::CHUNKS) reinterpret_cast<u4*>(st)[c] = vn[slot][i];
            }
            const int pn = p + PF * NW;
            if (pn < p1) {
                KUSH_ISSUE(slot, bnext[slot]);
                const int pnn = pn + PF * NW;
                bnext[slot] = pnn < p1 ? bt[pnn] : 0;
            }

            f4 sacc[2] = {f4{0.0f, 0.0f, 0.0f, 0.0f}, f4{0.0f, 0.0f, 0.0f, 0.0f}};
            f4 kacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) {
                h8 ks8, kb8;
                if constexpr (BITS == 4) {
                    const int d0 = q * (D / 8) + 4 * kk;
                    const h4v a = *reinterpret_cast<const h4v*>(st + S::KS + 2 * d0);
                    const h4v b = *reinterpret_cast<const h4v*>(st + S::KS + 2 * (d0 + D / 2));
                    const h4v c = *reinterpret_cast<const h4v*>(st + S::KB + 2 * d0);
                    const h4v d = *reinterpret_cast<const h4v*>(st + S::KB + 2 * (d0 + D / 2));
                    ks8 = h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
                    kb8 = h8{c[0], c[1], c[2], c[3], d[0], d[1], d[2], d[3]};
                } else {
                    const int d0 = q * (D / 4) + 8 * kk;
                    ks8 = *reinterpret_cast<const h8*>(st + S::KS + 2 * d0);
                    kb8 = *reinterpret_cast<const h8*>(st + S::KB + 2 * d0);
                }
                const h8 qh = qhl[kk * WAVE + lane];
                const h8 ql = qll[kk * WAVE + lane];
                // K bias dot: every row of A is this lane group's k_bias slice, so every output row is
                // sum_d kb[d] q[g][d]: all four accumulators of lane (q, g) hold it, no reduction needed
                kacc = mfma16(kb8, qh, kacc);
                kacc = mfma16(kb8, ql, kacc);
                const h8 qp = qh * ks8;                           // fp16 multiply, as the reference TC path
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    h8 a;
                    if constexpr (BITS == 4)
                        a = int4_codes(kw[tt][kk]);
                    else
                        a = int8_codes(kw[tt][2 * kk], kw[tt][2 * kk + 1]);
                    sacc[tt] = mfma16(a, qp, sacc[tt]);
                }
            }
            float x[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) x[j] = sacc[j >> 2][j & 3] + kacc[0];
            consume_page<D, BITS>(st, o, x, PAGE, m_run, l_run, vb_run, lane);
        }
    }
#undef KUSH_ISSUE

    // partial last page: exact K from the tail, V rows from its record (last split only)
    if (has_tail && w == (p1 - p0) % NW) {
        const IN* tk = tail_k + ((int64_t)tail_idx[s] * H + h) * PAGE * D;
        const int t = lane & 31, hf = lane >> 5;
        float acc[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) acc[g] = 0.0f;
        if (t < tail_n) {
            for (int d = hf * (D / 2); d < (hf + 1) * (D / 2); d += 4) {
                const float k0 = to_f32(tk[t * D + d]), k1 = to_f32(tk[t * D + d + 1]);
                const float k2 = to_f32(tk[t * D + d + 2]), k3 = to_f32(tk[t * D + d + 3]);
#pragma unroll
                for (int g = 0; g < 16; ++g) {
                    const float4 q4 = *reinterpret_cast<const float4*>(&qs_l[g * D + d]);
                    acc[g] += q4.x * k0 + q4.y * k1 + q4.z * k2 + q4.w * k3;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < 16; ++g) {
            acc[g] += __shfl_xor(acc[g], 32, WAVE);
            if (hf == 0) sc_l[g * PAGE + t] = t < tail_n ? acc[g] : -__builtin_inff();
        }
        const u4* vsrc = reinterpret_cast<const u4*>(head_base + (int64_t)bt[full] * bs + F::OFF_VQ);
#pragma unroll
        for (int i = 0; i < VCPL; ++i) {
            const int c = lane + WAVE * i;
            if (c < S::CHUNKS) reinterpret_cast<u4*>(st)[c] = vsrc[c];
        }
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = sc_l[r16 * PAGE + tok(q, j)];
        consume_page<D, BITS>(st, o, x, tail_n, m_run, l_run, vb_run, lane);
    }

    // merge the waves: every wave rescales to the workgroup max and adds into LDS in turn
    l_run = rows_sum(l_run);
    vb_run = rows_sum(vb_run);
    __syncthreads();
    if (q == 0) {
        m_l[w * 16 + r16] = m_run;
        l_l[w * 16 + r16] = l_run;
    }
    __syncthreads();
    float M = -__builtin_inff();
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) M = __builtin_fmaxf(M, m_l[ww * 16 + r16]);
    const float f = m_run == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - M);
    float* mbuf = qs_l;
#pragma unroll 1
    for (int ww = 0; ww < NW; ++ww) {
        if (w == ww) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = r16 * D + 16 * dt + 4 * q + i;
                    const float val = (o[dt][i] + vb_run) * f;
                    mbuf[idx] = ww == 0 ? val : mbuf[idx] + val;
                }
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < Gc * D; i += NW * WAVE) {
        const int g = i / D, d = i % D;
        float Mg = -__builtin_inff();
#pragma unroll
        for (int ww = 0; ww < NW; ++ww) Mg = __builtin_fmaxf(Mg, m_l[ww * 16 + g]);
        float L = 0.0f;
        if (Mg > -__builtin_inff()) {
#pragma unroll
            for (int ww = 0; ww < NW; ++ww) {
                const float mw = m_l[ww * 16 + g];
                if (mw > -__builtin_inff()) L += l_l[ww * 16 + g] * __builtin_amdgcn_exp2f(mw - Mg);
            }
        }
        const float val = mbuf[g * D + d];
        if (NS == 1) {
            out[qbase + i] = from_f32<IN>(L > 0.0f ? val / L : 0.0f);
        } else {
            const int64_t pb = (((int64_t)s * H + h) * NS + z) * G + g0 + g;
            part_o[pb * D + d] = val;
            if (d == 0) {
                part_ml[2 * pb] = Mg;
                part_ml[2 * pb + 1] = L;
            }
        }
    }
    if (NS == 1 || sync == nullptr) return;

    // split-K: the last workgroup of this (sequence, kv head, head chunk) merges every split. The
    // barrier completes every wave's partial stores; one agent-scope release (L2 writeback) by thread
    // 0 then publishes them before the counter moves, and the last workgroup's thread 0 acquires
    // (L2 invalidate) before its waves read the other splits.
    __syncthreads();
    if (threadIdx.x == 0) {
        const int n_gc = gridDim.z / NS;
        int32_t* ctr = sync + ((int64_t)s * H + h) * n_gc + gc;
        const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = prev == NS - 1;
        if (prev == NS - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_flag) return;
    const int64_t base = ((int64_t)s * H + h) * NS;
    for (int i = threadIdx.x; i < Gc * D; i += NW * WAVE) {
        const int g = g0 + i / D, d = i % D;
        float Mg = -__builtin_inff();
        for (int zz = 0; zz < NS; ++zz) Mg = __builtin_fmaxf(Mg, part_ml[2 * ((base + zz) * G + g)]);
        float L = 0.0f, acc = 0.0f;
        if (Mg > -__builtin_inff()) {
            for (int zz = 0; zz < NS; ++zz) {
                const int64_t pb = (base + zz) * G + g;
                const float mz = part_ml[2 * pb];
                if (mz > -__builtin_inff()) {
                    const float fz = __builtin_amdgcn_exp2f(mz - Mg);
                    L += part_ml[2 * pb + 1] * fz;
                    acc += fz * part_o[pb * D + d];
                }
            }
        }
        out[qbase + i] = from_f32<IN>(L > 0.0f ? acc / L : 0.0f);
    }
}

// grid (S, Hkv), block 256: merge split-K partials (M, L, unnormalized O) into the output.
// M is in log2 units. Splits with no tokens (M = -inf) are skipped (gpu.mojo:469-491).
template <typename IN>
__global__ __launch_bounds__(256) void combine_kernel(IN* __restrict__ out, const float* __restrict__ part_ml,
                                                      const float* __restrict__ part_o, int NS, int H, int G, int D) {
    const int s = blockIdx.x, h = blockIdx.y;
    const int64_t base = ((int64_t)s * H + h) * NS;
    for (int i = threadIdx.x; i < G * D; i += 256) {
        const int g = i / D, d = i % D;
        float M = -__builtin_inff();
        for (int z = 0; z < NS; ++z) M = __builtin_fmaxf(M, part_ml[2 * ((base + z) * G + g)]);
        float L = 0.0f, o = 0.0f;
        if (M > -__builtin_inff()) {
            for (int z = 0; z < NS; ++z) {
                const int64_t pb = (base + z) * G + g;
                const float mz = part_ml[2 * pb];
                if (mz > -__builtin_inff()) {
                    const float fz = __builtin_amdgcn_exp2f(mz - M);
                    L += part_ml[2 * pb + 1] * fz;
                    o += fz * part_o[pb * D + d];
                }
            }
        }
        out[((int64_t)s * H + h) * G * D + i] = from_f32<IN>(L > 0.0f ? o / L : 0.0f);
    }
}

// Static LDS of one decode workgroup (must stay within the 160 KB of a gfx950 CU).
template <int D, int BITS, int NW>
constexpr int decode_lds_bytes() {
    return NW * Stage<D, BITS>::BYTES + 2 * (D / 32) * WAVE * 16 + 16 * D * 4 + 16 * PAGE * 4 + 2 * NW * 16 * 4 + 16;
}

template <int D, int BITS, typename IN, int NW, int PF>
static int launch_decode(dim3 grid, hipStream_t stream, const void* q, void* out, const void* cache, int64_t bs,
                         int64_t hs, const void* tail_k, const int32_t* tail_idx, const int32_t* block_table,
                         const int32_t* seq_lens, int64_t bt_stride, int hkv, int group, float sm_log2, int n_splits,
                         float* part_ml, float* part_o, int32_t* sync) {
    decode_kernel<D, BITS, IN, NW, PF><<<grid, dim3(NW * WAVE), 0, stream>>>(
        (const IN*)q, (IN*)out, (const uint8_t*)cache, bs, hs, (const IN*)tail_k, tail_idx, block_table, seq_lens,
        bt_stride, hkv, group, sm_log2, n_splits, part_ml, part_o, sync);
    return kush_check_launch("kush_decode");
}

}  // namespace kush

using namespace kush;

extern "C" int kush_decode(int head_dim, int bits, int group, int dtype, const void* q, void* out, const void* cache,
                           int64_t block_stride, int64_t head_stride, const void* tail_k, const int32_t* tail_idx,
                           const int32_t* block_table, const int32_t* seq_lens, int64_t bt_stride, int32_t hkv,
                           float scale, int32_t n_splits, float* part_ml, float* part_o, int32_t* split_sync,
                           int32_t waves, int32_t n_seqs, void* stream) {
    if (n_seqs < 0 || hkv <= 0 || group <= 0 || n_splits <= 0)
        return kush_fail(-2, "kush_decode: bad n_seqs %d / hkv %d / group %d / n_splits %d", n_seqs, hkv, group,
                         n_splits);
    if (n_splits > 1 && (part_ml == nullptr || part_o == nullptr))
        return kush_fail(-2, "kush_decode: n_splits %d needs the partial buffers", n_splits);
    if (((uintptr_t)cache | (uint64_t)block_stride | (uint64_t)head_stride) & 15)
        return kush_fail(-2, "kush_decode: cache records must be 16-byte aligned");
    // waves: low byte = waves per workgroup (4, 8, 16; 0 = 4), next byte = pages in flight per wave
    int depth = (waves >> 8) & 0xff;
    waves &= 0xff;
    if (waves == 0) waves = 4;
    if (depth == 0) depth = 1;
    if (waves != 4 && waves != 8 && waves != 16) return kush_fail(-2, "kush_decode: waves must be 0, 4, 8 or 16");
    if (depth < 1 || depth > 3) return kush_fail(-2, "kush_decode: prefetch depth must be 1, 2 or 3");
    const int n_gc = (group + 15) / 16;
    if ((int64_t)n_splits * n_gc > 65535) return kush_fail(-2, "kush_decode: n_splits %d too large", n_splits);
    const float sm_log2 = (float)((double)scale * 1.4426950408889634);
    const dim3 grid(n_seqs, hkv, n_splits * n_gc);
    hipStream_t st = (hipStream_t)stream;
    return dispatch_shape(head_dim, bits, dtype, "kush_decode", [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        if (n_seqs == 0) return 0;
#define KUSH_DECODE_ARGS grid, st, q, out, cache, block_stride, head_stride, tail_k, tail_idx, block_table, seq_lens, \
                         bt_stride, hkv, group, sm_log2, n_splits, part_ml, part_o, split_sync
        if (waves == 16) {
            if constexpr (decode_lds_bytes<D, BITS, 16>() <= 160 * 1024)
                return launch_decode<D, BITS, IN, 16, 1>(KUSH_DECODE_ARGS);
            else
                return launch_decode<D, BITS, IN, 8, 1>(KUSH_DECODE_ARGS);
        }
        if (waves == 8) {
            if (depth == 3) return launch_decode<D, BITS, IN, 8, 3>(KUSH_DECODE_ARGS);
            if (depth == 2) return launch_decode<D, BITS, IN, 8, 2>(KUSH_DECODE_ARGS);
            return launch_decode<D, BITS, IN, 8, 1>(KUSH_DECODE_ARGS);
        }
        if (depth == 2) return launch_decode<D, BITS, IN, 4, 2>(KUSH_DECODE_ARGS);
        return launch_decode<D, BITS, IN, 4, 1>(KUSH_DECODE_ARGS);
#undef KUSH_DECODE_ARGS
    });
}

extern "C" int kush_combine(int head_dim, int group, int dtype, void* out, const float* part_ml, const float* part_o,
                            int32_t n_splits, int32_t hkv, int32_t n_seqs, void* stream) {
    if (n_seqs < 0 || hkv <= 0 || group <= 0 || n_splits <= 0)
        return kush_fail(-2, "kush_combine: bad arguments");
    if (head_dim != 64 && head_dim != 128 && head_dim != 256)
        return kush_fail(-1, "kush_combine: unsupported head_dim %d", head_dim);
    if (n_seqs == 0) return 0;
    const dim3 grid(n_seqs, hkv);
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case 0: combine_kernel<float><<<grid, 256, 0, st>>>((float*)out, part_ml, part_o, n_splits, hkv, group, head_dim); break;
        case 1: combine_kernel<_Float16><<<grid, 256, 0, st>>>((_Float16*)out, part_ml, part_o, n_splits, hkv, group, head_dim); break;
        case 2: combine_kernel<bf16_t><<<grid, 256, 0, st>>>((bf16_t*)out, part_ml, part_o, n_splits, hkv, group, head_dim); break;
        default: return kush_fail(-1, "kush_combine: unsupported dtype code %d", dtype);
    }
    return kush_check_launch("kush_combine");
}
