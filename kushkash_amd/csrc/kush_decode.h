// Fused dequant decode attention over int4/int8 page records for gfx950 (CDNA4), with split-K
// partials and a log-sum-exp combine. Contract: kushkash/kush/gpu.mojo:566-807 (decode),
// :418-491 (split ranges, merge, combine), kushkash/_ops.py:182-213 (launch), arithmetic of the
// reference CPU path kushkash/kush/cpu.mojo:320-451.
//
// Mapping onto CDNA4. One workgroup = NW waves (2, 4 or 8) for one (sequence, kv head, split,
// 16-head chunk). The split's pages go out in pairs over windows of up to 1,024 pages whose block
// ids sit in an LDS table; wave w takes pairs w, w + NW, ... (a fixed assignment: the same call
// always sums the same pages in the same order, so its output bits are reproducible). Per pair a wave:
//   1. has both records staged in its private LDS ring by buffer-to-LDS DMA (whole records, 1 KB
//      per instruction, issued one pair ahead and waited on with explicit vmcnt counts);
//   2. reads K code rows from the ring and turns them into exact subnormal fp16 operands (one
//      v_perm and one v_bitop3 per pair of codes), and computes the scores S^T = K . Q'^T on MFMA
//      16x16x32 f16 with Q' = fp16(q' * k_scale) (q' = q times a power of two; the rest of
//      scale * log2 e multiplies the fp32 scores); the K-bias and -HALF * k_scale terms of both pages
//      come from one more MFMA per K-step;
//   3. runs a page-granular online softmax in base 2 per MFMA column (with G <= 8 two page
//      streams share the 16 columns: page A in 0-7, page B in 8-15), moving the running max only
//      when a page exceeds it by more than 2^3;
//   4. gathers V codes column-wise from the ring (ds_read_b64_tr_b8) into V^T operands and
//      accumulates O^T += V^T . P'^T on MFMA, with P' = fp16(e * v_scale); -HALF * sum P' comes
//      from one MFMA and the V bias sum e * v_bias stays in fp32.
// The partial last page takes exact fp32 K . q scores from the tail (spread over all waves) and V
// rows from its record. A rotated cache (ROT) gets q rotated by the canonical Walsh-Hadamard
// transform on load (rows of the chunk's heads in the butterfly layout, through LDS) and the output
// rotated back before its one rounding; split partials stay unrotated. With app_k (the fused append
// + decode), the workgroup that reads the new token's page first appends the token (row s of app_k /
// app_v at position seq_lens[s] - 1): K to the tail, V into its record row, the K page quantized
// when the token completes it -- the page quantizer of kush_page.h over the idle ring LDS. The waves (and streams) merge through the idle ring at the end; with
// split-K, partials are published write-through and the last workgroup of a (sequence, kv head)
// merges them in the same launch.
//
// MFMA 16x16x32 f16 operand layout used throughout (lane l, r = l % 16, q = l / 16):
//   A: row r, 8 contraction slots of lane group q;  B: column r, the same 8 slots;
//   C: rows 4q .. 4q+3 of column r.
// Which physical dim or token a slot stands for is chosen here (kdim, tok), identically for A
// and B, so only the C layout is relied upon.
#pragma once

#include <cmath>
#include <cstdlib>

#include "kush_page.h"

namespace kush {

// Timeline build (-DKUSH_TIMELINE: the instrumented copy of one instantiation unit linked into
// libkushhip_timeline.so, never the product library). Each workgroup has a row of TIMELINE_COLS
// int64 per launch. Wave 0 records the 100 MHz wall clock at five points -- 0 start, 1 prologue done
// (first page DMAs about to go out), 2 its first page pair landed, 3 its pages done, 4 output stored --
// in slots 0-4, the shader clock at points 2 and 3 in slots 5 and 6, and the XCD it ran on (hardware
// register XCC_ID) in slot 7; every wave w records the wall clock at which it consumed its last page
// pair (before the workgroup's barrier; the last window's, with several) in slot 8 + w. Rows
// beyond TIMELINE_ROWS are not recorded. The stores are ordinary vector stores (every lane of the
// wave the same value), made once the output is stored.
#ifdef KUSH_TIMELINE
constexpr int TIMELINE_ROWS = 1 << 16, TIMELINE_COLS = 16;
static __device__ long long g_timeline[TIMELINE_ROWS * TIMELINE_COLS];
__device__ __forceinline__ long long* timeline_row() {
    const long long row = ((long long)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    return row < TIMELINE_ROWS ? g_timeline + row * TIMELINE_COLS : nullptr;
}
// The marks are held in registers and stored once, after the output (KUSH_MARK_FLUSH): a store
// inside the page loop would count in the vmcnt the loop waits on and hold the marking wave back.
struct TimelineMarks {
    long long v[8] = {};
    long long wave_done = 0;
    __device__ __forceinline__ void mark(int k) {
        v[k] = wall_clock64();
        if (k == 0) v[7] = __builtin_amdgcn_s_getreg((3 << 11) | 20);         // XCC_ID bits [3:0]
        if (k == 2) v[5] = clock64();
        if (k == 3) v[6] = clock64();
    }
    __device__ __forceinline__ void flush(int w) {
        long long* const r = timeline_row();
        if (r == nullptr) return;
        if (w == 0) {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[k] = v[k];
        }
        r[8 + w] = wave_done;
    }
};
#define KUSH_TIMELINE_DECL TimelineMarks tl_marks
#define KUSH_MARK(k) tl_marks.mark(k)
#define KUSH_MARK_WAVE() (tl_marks.wave_done = wall_clock64())
#define KUSH_MARK_FLUSH() tl_marks.flush(w)
#else
#define KUSH_TIMELINE_DECL
#define KUSH_MARK(k) ((void)0)
#define KUSH_MARK_WAVE() ((void)0)
#define KUSH_MARK_FLUSH() ((void)0)
#endif

typedef _Float16 h4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }

// Physical dim of contraction slot j of lane group q in K-step kk (QK^T). The lane owns bytes
// [q KB, (q+1) KB) of each code row (KB = DC / 4). int4: K-steps come in pairs over 8 of those
// bytes, 2 pr and 2 pr + 1 taking their low and high nibbles, so the 8 dims of a K-step are
// consecutive and its scales and biases are one 16-byte read. int8: dims q D/4 + 8 kk + j.
template <int D, int BITS>
__device__ __forceinline__ int kdim(int kk, int q, int j) {
    if constexpr (BITS == 4)
        return (kk & 1) * (D / 2) + q * (D / 8) + 8 * (kk >> 1) + j;
    else
        return q * (D / 4) + 8 * kk + j;
}

// Token of slot j of lane group q in the PV contraction: the token the QK^T accumulators of lane
// group q hold in register j % 4 of tile j / 4.
__device__ __forceinline__ int tok(int q, int j) { return 16 * (j >> 2) + 4 * q + (j & 3); }

// ------------------------------------------------------------------ LDS page stage
// A wave stages whole records in a ring of LDS slots with buffer-to-LDS DMA (64 lanes x 16 bytes per
// instruction, lane l -> 16-byte chunk l of the instruction's 1 KB). Chunks of the 64 code rows are
// placed XOR-swizzled within their row, chunk c of row r at position c ^ swz(r), so the column-wise
// V gathers and the K row reads spread over the 64 LDS banks; the scales and biases stay in place.
// The swizzle is applied on the source side: the lane that fills LDS chunk L loads record chunk
// src_chunk(L). A slot is exactly one record: instruction i covers chunks [64 i, 64 i + 64), except
// the last, which covers the record's last 64 chunks and so rewrites the overlap with the same bytes
// (a lane past the end of its 1 KB would write zeros beyond the slot).
template <int D, int BITS>
struct Ring {
    using F = Fmt<D, BITS>;
    static constexpr int CPR = F::DC / 16;                  // 16-byte chunks per code row
    static constexpr int CODE_CHUNKS = 64 * CPR;            // K rows then V rows
    static constexpr int CHUNKS = F::REC / 16;
    static constexpr int DMA = (CHUNKS + WAVE - 1) / WAVE;   // 1 KB instructions per page
    static constexpr int SLOT = F::REC;                     // LDS bytes per ring slot
    static constexpr int RSHIFT = F::DC >= 256 ? 0 : (F::DC == 128 ? 1 : (F::DC == 64 ? 2 : 3));
    static_assert(CHUNKS >= WAVE, "a record spans at least one full instruction");
    // first LDS chunk filled by instruction i
    static constexpr int chunk0(int i) { return i < DMA - 1 ? WAVE * i : CHUNKS - WAVE; }
};

// Swizzle of code row r (0-31 K, 32-63 V). K rows are read row-wise (16 rows by 16 lanes):
// rows r and r + 4 (DC = 64) must land on different banks, so the swizzle takes the row bits
// above those that already select the bank. V rows are gathered column-wise, 16 tokens per half
// wave, t = 16 a + 4 q + b (b < 4, q the lane group, a the tile); u = b | (q & 1) << 2 | a << 3
// indexes them, and the swizzle takes the bits of u that the row address leaves on one bank.
template <int D, int BITS>
__device__ __forceinline__ int swz(int r) {
    using R = Ring<D, BITS>;
    if (r < 32) return (r >> R::RSHIFT) & (R::CPR - 1);
    const int t = r - 32;
    const int u = (t & 3) | (((t >> 2) & 1) << 2) | (((t >> 4) & 1) << 3);
    return (u >> R::RSHIFT) & (R::CPR - 1);
}

// byte offset in a slot of record chunk c (16 bytes) of code row r (0-31 K, 32-63 V)
template <int D, int BITS>
__device__ __forceinline__ int slot_chunk(int r, int c) {
    using R = Ring<D, BITS>;
    return (r * R::CPR + (c ^ swz<D, BITS>(r))) * 16;
}

template <int D, int BITS>
__device__ __forceinline__ uint32_t src_chunk(int L) {
    using R = Ring<D, BITS>;
    if (L >= R::CODE_CHUNKS) return (uint32_t)L;             // scales / biases (and padding) in place
    const int r = L / R::CPR, j = L % R::CPR;
    return (uint32_t)(r * R::CPR + (j ^ swz<D, BITS>(r)));
}

// s_waitcnt with only vmcnt(N) (gfx9 encoding: vmcnt [3:0] + [15:14], expcnt [6:4], lgkmcnt [11:8]),
// then a compiler barrier: no LDS read of the landed data is moved above the wait
#define KUSH_WAIT_VM(N)                                                                          \
    do {                                                                                         \
        __builtin_amdgcn_s_waitcnt(((N) & 15) | (((N) >> 4) << 14) | (7 << 4) | (15 << 8));      \
        asm volatile("" ::: "memory");                                                           \
    } while (0)

// Subnormal fp16 codes: the bit pattern n (0..255) is the fp16 value n * 2^-24, exact, so unsigned
// code bytes become MFMA operands with one byte shuffle and no arithmetic; the products are exact in
// fp32 and the 2^24 is applied to the fp32 results. n = c + HALF: the HALF offset is removed through
// the bias terms. perm(x, 0, 0x0C010C00) = bytes [x0, 0, x1, 0].
__device__ __forceinline__ h8 sub_codes4(uint32_t lo, uint32_t hi) {    // 4 + 4 nibble values, masked
    return __builtin_bit_cast(h8, u4{__builtin_amdgcn_perm(0u, lo, 0x0C010C00u), __builtin_amdgcn_perm(0u, lo, 0x0C030C02u),
                                     __builtin_amdgcn_perm(0u, hi, 0x0C010C00u), __builtin_amdgcn_perm(0u, hi, 0x0C030C02u)});
}

// int4 codes to operands. The xor with 0x88 turns a two's-complement nibble into n = c + 8; a
// nibble is then masked in place: a low nibble is the subnormal n, a high nibble lands 4 bits up,
// as 16 n. Each of (x ^ 0x88888888) & mask is one v_bitop3.
constexpr uint32_t NIB_XOR = 0x88888888u, NIB_LO = 0x000F000Fu, NIB_HI = 0x00F000F0u;

// K: two words (8 code bytes of a row, dims in order) -> the low nibbles (n) and the high nibbles
// (16 n) of the 8 bytes, in byte order: v_perm spreads two bytes into the low bytes of the halves.
__device__ __forceinline__ void k_codes4(uint32_t w0, uint32_t w1, h8& lo, h8& hi) {
    const uint32_t p[4] = {__builtin_amdgcn_perm(0u, w0, 0x0C010C00u), __builtin_amdgcn_perm(0u, w0, 0x0C030C02u),
                           __builtin_amdgcn_perm(0u, w1, 0x0C010C00u), __builtin_amdgcn_perm(0u, w1, 0x0C030C02u)};
    u4 l, h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        l[i] = (p[i] ^ NIB_XOR) & NIB_LO;
        h[i] = (p[i] ^ NIB_XOR) & NIB_HI;
    }
    lo = __builtin_bit_cast(h8, l);
    hi = __builtin_bit_cast(h8, h);
}

// V^T: two words of 4 token bytes each (PV slots 0-3, 4-7) -> low nibbles (n) and high nibbles
// (16 n) in slot order 0 2 1 3 4 6 5 7: bytes 0 and 2 of a word are masked in place, bytes 1 and 3
// after a shift by 8. The P' operand takes the same order (VSLOT).
__device__ __forceinline__ void v_codes4(uint32_t w0, uint32_t w1, h8& lo, h8& hi) {
    const uint32_t p[4] = {w0, w0 >> 8, w1, w1 >> 8};
    u4 l, h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        l[i] = (p[i] ^ NIB_XOR) & NIB_LO;
        h[i] = (p[i] ^ NIB_XOR) & NIB_HI;
    }
    lo = __builtin_bit_cast(h8, l);
    hi = __builtin_bit_cast(h8, h);
}

// PV slot held by operand position k (int4: the v_codes4 order; int8: in order)
template <int BITS>
__device__ __forceinline__ constexpr int vslot(int k) {
    return BITS == 4 ? (k & 4) | ((k & 1) << 1) | ((k >> 1) & 1) : k;
}

// two int8 words (8 codes) -> n = c + 128
__device__ __forceinline__ h8 int8_sub(uint32_t w0, uint32_t w1) {
    return sub_codes4(w0 ^ 0x80808080u, w1 ^ 0x80808080u);
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
typedef __attribute__((address_space(3))) void lds_void;

// V^T operand gather: within each 16-lane group, ds_read_b64_tr_b8 hands output lane i byte
// (i % 8) of the 8-byte rows supplied by lanes 2k + (i % 16) / 8, k = 0..7. Lane (2k + half) of
// group q supplies V token tok(q, k) at byte column 16 ct + 8 half, so lane r of the group receives
// byte column 16 ct + r of its 8 tokens, in PV slot order.
template <int D, int BITS>
__device__ __forceinline__ v2i gather_vt(const uint8_t* slot, int ct, int lane) {
    const int s16 = lane & 15, q = lane >> 4;
    const uint8_t* src = slot + slot_chunk<D, BITS>(32 + tok(q, s16 >> 1), ct) + 8 * (s16 & 1);
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(src));
}

// Softmax update over NP staged pages at once and their PV accumulation from the staged V codes.
// Scores in log2 units are x = a s[p][j] + b[p] (a > 0) for tokens tok(q, j); masked tokens carry
// s = -inf. o accumulates in units of 2^-24 (subnormal codes; int4 high-nibble tiles, o[D/32 ..],
// in units of 2^-20); with P' = fp16(e vs) a page adds sum P' n (MFMA), -HALF sum P' (MFMA into
// vacc, units of 2^-24) and sum e vb (vb_run), i.e. sum e (vs' c + vb) with vs' = P' / e.
template <int D, int BITS, int NP>
__device__ __forceinline__ void consume_pages(const uint8_t* const (&slot)[NP], f4 (&o)[D / 16], f4& vacc,
                                              const float (&sv)[NP][8], float a, const float (&b)[NP],
                                              float& m_run, float& l_run, float& vb_run, int lane) {
    using F = Fmt<D, BITS>;
    const int q = lane >> 4;
    float pm = -__builtin_inff();
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        float mx = sv[p][0];
#pragma unroll
        for (int j = 1; j < 8; ++j) mx = __builtin_fmaxf(mx, sv[p][j]);
        pm = __builtin_fmaxf(pm, __builtin_fmaf(mx, a, b[p]));
    }
    // the reference point of the exponentials moves only when the max exceeds it by more than 2^3:
    // weights stay <= 8 (P' = e vs stays far from fp16 overflow) and most steps skip the O rescale
    pm = rows_max(pm);
    const float m_new = pm > m_run + 3.0f ? pm : m_run;
    const float corr = __builtin_amdgcn_exp2f(m_run - m_new);   // first step: exp2(-inf) = 0

    float lsum = 0.0f, vbsum = 0.0f;
    h8 pw[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        const float bp = b[p] - m_new;
        const h4v vs0 = *reinterpret_cast<const h4v*>(slot[p] + F::OFF_VS + 8 * q);
        const h4v vs1 = *reinterpret_cast<const h4v*>(slot[p] + F::OFF_VS + 32 + 8 * q);
        const h4v vb0 = *reinterpret_cast<const h4v*>(slot[p] + F::OFF_VB + 8 * q);
        const h4v vb1 = *reinterpret_cast<const h4v*>(slot[p] + F::OFF_VB + 32 + 8 * q);
        _Float16 pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float vsj = (float)(j < 4 ? vs0[j] : vs1[j - 4]);
            const float vbj = (float)(j < 4 ? vb0[j] : vb1[j - 4]);
            const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[p][j], a, bp));
            pv[j] = (_Float16)__builtin_fmaf(e, vsj, 0.0f);   // e vs (fma_mix, then one pack per pair)
            lsum += e;
            vbsum = __builtin_fmaf(e, vbj, vbsum);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) pw[p][k] = pv[vslot<BITS>(k)];
    }
    l_run = l_run * corr + lsum;
    vb_run = vb_run * corr + vbsum;
    m_run = m_new;
    if (corr != 1.0f) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) o[dt] *= corr;
        vacc *= corr;
    }

    constexpr int NCOL = BITS == 4 ? D / 32 : D / 16;
#pragma unroll
    for (int ct = 0; ct < NCOL; ++ct)
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const v2i w = gather_vt<D, BITS>(slot[p], ct, lane);
            if constexpr (BITS == 4) {
                h8 lo, hi;
                v_codes4((uint32_t)w[0], (uint32_t)w[1], lo, hi);
                o[ct] = mfma16(lo, pw[p], o[ct]);
                o[ct + D / 32] = mfma16(hi, pw[p], o[ct + D / 32]);
            } else {
                o[ct] = mfma16(int8_sub((uint32_t)w[0], (uint32_t)w[1]), pw[p], o[ct]);
            }
        }
    // -HALF sum P' per head: A rows all -HALF 2^-24 (fp16 bits 0x8000 | HALF, exact)
    const _Float16 nh = __builtin_bit_cast(_Float16, (uint16_t)(0x8000u | (uint32_t)F::HALF));
    const h8 neg_half = h8{nh, nh, nh, nh, nh, nh, nh, nh};
#pragma unroll
    for (int p = 0; p < NP; ++p) vacc = mfma16(neg_half, pw[p], vacc);
}

// Wave splits: one wave stores the n (<= N * 64) block ids of its window, ids[0 .. n), into its own
// table region tb, every id load in flight at once. Kept out of the workgroup's window lambda, whose
// code the other kernels share unchanged.
template <int N>
__device__ __forceinline__ void load_wave_window(int* tb, const int32_t* ids, int n, int lane) {
    int v[N];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int i = lane + k * WAVE;
        v[k] = i < n ? ids[i] : 0;
    }
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int i = lane + k * WAVE;
        if (i < n) tb[i] = v[k];
    }
}

// Stage the record of block blk into LDS at dst: R::DMA buffer-to-LDS loads of 1 KB. An invalid page
// (past the window's last) gets an empty buffer range: the loads then fill the slot with zeros and
// touch no memory, and still count in vmcnt like a real page.
// The loads are written in asm so that the compiler does not track them: the page loop waits for
// them with explicit vmcnt counts alone. Vector loads complete in order, so any vector memory op the
// compiler adds (issued later) only makes those waits stricter.
template <int D, int BITS>
__device__ __forceinline__ void issue_page(uint8_t* dst, bool valid, int blk, const uint8_t* head_base, int64_t bs,
                                           const uint32_t* voff) {
    using F = Fmt<D, BITS>;
    using R = Ring<D, BITS>;
    const uint64_t rec = (uint64_t)(uintptr_t)(head_base + (int64_t)blk * bs);
    // raw buffer descriptor: base, stride 0, num_records (0: every lane out of range), dword format
    const u4 rsrc = u4{(uint32_t)rec, (uint32_t)(rec >> 32) & 0xFFFFu, valid ? (uint32_t)F::REC : 0u, 0x00020000u};
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_void*)dst;
    // m0 is reserved by the compiler; nothing else in the decode kernels uses it (checked on their
    // assembly by tests/test_isa.py), so setting it here is safe. An LDS DMA reads m0 one wait state
    // after a scalar write of it at the earliest (the compiler puts one between its own m0 writes and
    // LDS DMAs, and cannot see inside this asm), hence the s_nop: without it the load can take the
    // previous m0, the previous chunk's LDS address, depending on how the two instructions issue.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
#pragma unroll
    for (int i = 0; i < R::DMA; ++i)
        asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                     :: "s"(lds + R::chunk0(i) * 16), "v"(voff[i]), "s"(rsrc) : "memory", "m0");
#pragma clang diagnostic pop
}

// Scores of the 64 tokens of a staged page pair (page 0 at s0, page 1 in the next slot):
// x = a sacc[p][j / 4][j % 4] + kx[p] in log2 units for token tok(q, j) of page p, head r16, with
// a = rs 2^24.
// sacc = K . Q'^T on codes n = c + HALF as subnormal fp16 (units of 2^-24) and Q' = q' ks as an fp16
// pair qp + qr, q' = q p2 (p2 a power of two: q' is exact in fp16 for bf16 / fp16 q; fp32 q adds
// its low fp16 part ql): fp32-grade scores for more than 8 q heads per kv head, the reference's
// CUDA-core domain (its tensor-core path takes G <= 8, gpu.mojo:576). int4 high nibbles enter as
// 16 n against Q' / 16 (qa holds q' / 16 there). kx = rs (sum_d kb[d] q'[d] - HALF sum_d ks[d] q'[d]): one
// MFMA per K-step for both pages, A row r holding page r % 2's biases (r % 4 < 2) or scales, so C
// register i holds page i % 2's bias dot (i < 2) or scale dot (i >= 2).
template <int D, int BITS, bool QLO>
__device__ __forceinline__ void pair_scores(const uint8_t* s0, const h8 (&qa)[D / 32],
                                            const h8 (&qla)[D / 32], const h8 (&qh)[D / 32], const h8 (&ql)[D / 32],
                                            float (&sv)[2][8], float (&kx)[2], float rs, int lane) {
    using F = Fmt<D, BITS>;
    constexpr int KSTEPS = D / 32;
    constexpr int KBYTES = F::DC / 4;                // K code bytes per lane per 16-token tile
    const int r16 = lane & 15, q = lane >> 4;
    const uint8_t* const sl[2] = {s0, s0 + Ring<D, BITS>::SLOT};
    // A row r16 of the bias MFMA: page r16 & 1, k bias (r16 & 2 == 0) or k scale
    const uint8_t* const brow = s0 + (r16 & 1) * Ring<D, BITS>::SLOT + ((r16 & 2) ? F::OFF_KS : F::OFF_KB);
    f4 sacc[2][2];
#pragma unroll
    for (int p = 0; p < 2; ++p) sacc[p][0] = sacc[p][1] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    f4 bacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
        const int d0 = kdim<D, BITS>(kk, q, 0);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            h8 a[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                // code bytes of row 16 tt + r16 for this K-step, from the swizzled slot
                const int row = 16 * tt + r16;
                const int byte = q * KBYTES + 8 * (BITS == 4 ? kk >> 1 : kk);
                const u2 wv = *reinterpret_cast<const u2*>(sl[p] + slot_chunk<D, BITS>(row, byte / 16) + byte % 16);
                if constexpr (BITS == 4) {
                    h8 lo, hi;
                    k_codes4(wv[0], wv[1], lo, hi);
                    a[tt] = (kk & 1) ? hi : lo;
                } else {
                    a[tt] = int8_sub(wv[0], wv[1]);
                }
            }
            const h8 ks8 = *reinterpret_cast<const h8*>(sl[p] + F::OFF_KS + 2 * d0);
            // Q' = q' ks as an fp16 pair: qp = fp16(q' ks), qr = the exact residual of that product
            // (plus ql ks for fp32 q), rounded once
            const h8 qp = qa[kk] * ks8;
            h8 qr = __builtin_elementwise_fma(qa[kk], ks8, -qp);
            if constexpr (QLO) qr = __builtin_elementwise_fma(qla[kk], ks8, qr);
            sacc[p][0] = mfma16(a[0], qp, sacc[p][0]);
            sacc[p][1] = mfma16(a[1], qp, sacc[p][1]);
            sacc[p][0] = mfma16(a[0], qr, sacc[p][0]);
            sacc[p][1] = mfma16(a[1], qr, sacc[p][1]);
        }
        const h8 b8 = *reinterpret_cast<const h8*>(brow + 2 * d0);
        bacc = mfma16(b8, qh[kk], bacc);
        if constexpr (QLO) bacc = mfma16(b8, ql[kk], bacc);
    }
    // C register i is row 4 q + i: page i & 1, the k bias dot (i < 2) or the k scale dot
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int j = 0; j < 8; ++j) sv[p][j] = sacc[p][j >> 2][j & 3];
        kx[p] = rs * __builtin_fmaf(-(float)F::HALF, bacc[2 + p], bacc[p]);
    }
}

// ------------------------------------------------------------------ two page streams (G <= 8)
// With at most 8 q heads per kv head, MFMA column c stands for head c % 8 of page stream c / 8: a
// page pair puts page A in columns 0-7 and page B in columns 8-15, so each lane's Q', softmax and
// P' work covers one (head, page) and no column is idle. Each column keeps its own online-softmax
// state; the streams of a head are merged with the waves at the end.

// Scores of a staged pair (page A at s0, page B in the next slot) for this lane's column: sv[j] for
// token tok(q, j) of its page, x = a sv[j] + kx. The Q' operand is built once for both pages (each
// column from its own page's scales); K of page A and of page B each meet it in their own MFMAs,
// and a column keeps the product with its page. Q' enters as the fp16 pair qp + qr: qp = fp16(q' ks),
// the operand the reference's tensor-core path (G <= 8) forms (gpu.mojo:660-675, rounded twice
// there), and qr the residual of that product (plus q's low part ql times ks for fp32 q), in a
// second MFMA, so the scores are fp32-grade here as in the one-stream form.
template <int D, int BITS, bool QLO>
__device__ __forceinline__ void pair_scores2(const uint8_t* s0, const h8 (&qa)[D / 32], const h8 (&qla)[D / 32],
                                             const h8 (&qh)[D / 32], const h8 (&ql)[D / 32], float (&sv)[8],
                                             float& kx, float rs, int lane) {
    using F = Fmt<D, BITS>;
    constexpr int KSTEPS = D / 32;
    constexpr int KBYTES = F::DC / 4;
    constexpr int SLOT = Ring<D, BITS>::SLOT;
    const int r16 = lane & 15, q = lane >> 4, st = r16 >> 3;
    const uint8_t* const sl[2] = {s0, s0 + SLOT};
    const uint8_t* const mine = s0 + st * SLOT;                 // the page of this lane's column
    // A row r16 of the bias MFMA: page r16 & 1, k bias (r16 & 2 == 0) or k scale
    const uint8_t* const brow = s0 + (r16 & 1) * SLOT + ((r16 & 2) ? F::OFF_KS : F::OFF_KB);
    f4 sacc[2][2];
#pragma unroll
    for (int p = 0; p < 2; ++p) sacc[p][0] = sacc[p][1] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    f4 bacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
        const int d0 = kdim<D, BITS>(kk, q, 0);
        const h8 ks8 = *reinterpret_cast<const h8*>(mine + F::OFF_KS + 2 * d0);
        // Q' as an fp16 pair: qp = fp16(q' ks) and qr, the residual of that product (plus ql ks for
        // fp32 q), so the scores carry no fp16 rounding of Q'. With qp alone (the reference's
        // tensor-core operand, which it rounds twice) a few outputs in a thousand exceeded 2e-3
        // plus their own rounding; the residual's MFMAs cost C2 ~0.5 us of 31.7.
        const h8 qp = qa[kk] * ks8;
        h8 qr = __builtin_elementwise_fma(qa[kk], ks8, -qp);
        if constexpr (QLO) qr = __builtin_elementwise_fma(qla[kk], ks8, qr);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            h8 a[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int row = 16 * tt + r16;
                const int byte = q * KBYTES + 8 * (BITS == 4 ? kk >> 1 : kk);
                const u2 wv = *reinterpret_cast<const u2*>(sl[p] + slot_chunk<D, BITS>(row, byte / 16) + byte % 16);
                if constexpr (BITS == 4) {
                    h8 lo, hi;
                    k_codes4(wv[0], wv[1], lo, hi);
                    a[tt] = (kk & 1) ? hi : lo;
                } else {
                    a[tt] = int8_sub(wv[0], wv[1]);
                }
            }
            sacc[p][0] = mfma16(a[0], qp, sacc[p][0]);
            sacc[p][1] = mfma16(a[1], qp, sacc[p][1]);
            sacc[p][0] = mfma16(a[0], qr, sacc[p][0]);
            sacc[p][1] = mfma16(a[1], qr, sacc[p][1]);
        }
        const h8 b8 = *reinterpret_cast<const h8*>(brow + 2 * d0);
        bacc = mfma16(b8, qh[kk], bacc);
        if constexpr (QLO) bacc = mfma16(b8, ql[kk], bacc);
    }
    // C register i is row 4 q + i: page i & 1, the k bias dot (i < 2) or the k scale dot
#pragma unroll
    for (int j = 0; j < 8; ++j) sv[j] = st ? sacc[1][j >> 2][j & 3] : sacc[0][j >> 2][j & 3];
    kx = rs * __builtin_fmaf(-(float)F::HALF, st ? bacc[3] : bacc[2], st ? bacc[1] : bacc[0]);
}

// Softmax update of this lane's column over its page (scores x = a sv[j] + kx; masked tokens
// sv = -inf; a column may be masked whole) and the PV accumulation of page A (at s0) into columns
// 0-7 and page B (at s0 + ds) into columns 8-15: each MFMA takes P' with the other stream's
// columns zeroed. Units as in consume_pages.
template <int D, int BITS>
__device__ __forceinline__ void consume2(const uint8_t* s0, int ds, f4 (&o)[D / 16], f4& vacc, const float (&sv)[8],
                                         float a, float kx, float& m_run, float& l_run, float& vb_run, int lane) {
    using F = Fmt<D, BITS>;
    const int r16 = lane & 15, q = lane >> 4, st = r16 >> 3;
    const uint8_t* const mine = s0 + st * ds;
    float pm = sv[0];
#pragma unroll
    for (int j = 1; j < 8; ++j) pm = __builtin_fmaxf(pm, sv[j]);
    pm = rows_max(__builtin_fmaf(pm, a, kx));
    const float m_new = pm > m_run + 3.0f ? pm : m_run;
    // A masked page (every token's sv = -inf, or the whole column's kx = -inf with finite sv from a
    // zero-filled slot) moves nothing: its x = -inf, so its weights are exp2(-inf) = 0, also in a
    // column that has seen nothing yet (m_new = -inf, where the reference point is -inf as well)
    const bool none = m_new == -__builtin_inff();                 // nothing seen yet in this column
    const float corr = none ? 1.0f : __builtin_amdgcn_exp2f(m_run - m_new);
    const float bp = none ? -__builtin_inff() : kx - m_new;

    const h4v vs0 = *reinterpret_cast<const h4v*>(mine + F::OFF_VS + 8 * q);
    const h4v vs1 = *reinterpret_cast<const h4v*>(mine + F::OFF_VS + 32 + 8 * q);
    const h4v vb0 = *reinterpret_cast<const h4v*>(mine + F::OFF_VB + 8 * q);
    const h4v vb1 = *reinterpret_cast<const h4v*>(mine + F::OFF_VB + 32 + 8 * q);
    float lsum = 0.0f, vbsum = 0.0f;
    _Float16 pv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float vsj = (float)(j < 4 ? vs0[j] : vs1[j - 4]);
        const float vbj = (float)(j < 4 ? vb0[j] : vb1[j - 4]);
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], a, bp));
        pv[j] = (_Float16)__builtin_fmaf(e, vsj, 0.0f);
        lsum += e;
        vbsum = __builtin_fmaf(e, vbj, vbsum);
    }
    h8 pw;
#pragma unroll
    for (int k = 0; k < 8; ++k) pw[k] = pv[vslot<BITS>(k)];
    const u4 pu = __builtin_bit_cast(u4, pw);
    const uint32_t keep_a = st ? 0u : ~0u;
    const h8 pwa = __builtin_bit_cast(h8, pu & keep_a), pwb = __builtin_bit_cast(h8, pu & ~keep_a);
    l_run = l_run * corr + lsum;
    vb_run = vb_run * corr + vbsum;
    m_run = m_new;
    if (corr != 1.0f) {
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) o[dt] *= corr;
        vacc *= corr;
    }

    constexpr int NCOL = BITS == 4 ? D / 32 : D / 16;
#pragma unroll
    for (int ct = 0; ct < NCOL; ++ct) {
        const v2i wa = gather_vt<D, BITS>(s0, ct, lane);
        const v2i wb = gather_vt<D, BITS>(s0 + ds, ct, lane);
        if constexpr (BITS == 4) {
            h8 lo, hi;
            v_codes4((uint32_t)wa[0], (uint32_t)wa[1], lo, hi);
            o[ct] = mfma16(lo, pwa, o[ct]);
            o[ct + D / 32] = mfma16(hi, pwa, o[ct + D / 32]);
            v_codes4((uint32_t)wb[0], (uint32_t)wb[1], lo, hi);
            o[ct] = mfma16(lo, pwb, o[ct]);
            o[ct + D / 32] = mfma16(hi, pwb, o[ct + D / 32]);
        } else {
            o[ct] = mfma16(int8_sub((uint32_t)wa[0], (uint32_t)wa[1]), pwa, o[ct]);
            o[ct] = mfma16(int8_sub((uint32_t)wb[0], (uint32_t)wb[1]), pwb, o[ct]);
        }
    }
    const _Float16 nh = __builtin_bit_cast(_Float16, (uint16_t)(0x8000u | (uint32_t)F::HALF));
    vacc = mfma16(h8{nh, nh, nh, nh, nh, nh, nh, nh}, pw, vacc);   // column c sums its own P'
}

// Pages per window of the page loop: the block ids of a window sit in an LDS table.
constexpr int WIN = 1024;

// Static LDS of one decode workgroup: two arrays, each holding one page pair per wave (wave w at
// 2 w SLOT) and the window's block-id table. After the page loop the idle arrays
// hold everything else: the cross-wave merge in the first; the exact-K tail's q and scores, the
// waves' softmax state and the split-K flag in the second.
template <int D, int BITS, int NW>
constexpr int decode_lds_bytes() {
    return 4 * NW * Ring<D, BITS>::SLOT + 4 * WIN + 16;
}

template <int D, int BITS, int NW>
constexpr bool decode_fits() {
    return decode_lds_bytes<D, BITS, NW>() <= 160 * 1024;
}

// A third ring array (DEP = 3: each wave holds three page pairs, one consumed while two are in flight)
// where it fits in LDS and in vmcnt's 63 outstanding loads.
template <int D, int BITS, int NW>
constexpr bool decode_fits3() {
    return decode_lds_bytes<D, BITS, NW>() + 2 * NW * Ring<D, BITS>::SLOT <= 160 * 1024 && 4 * Ring<D, BITS>::DMA <= 63;
}

// byte offsets in the second array of the after-loop scratch: q [16][QS] fp32 (rows padded by 4
// floats, so the 16 rows of one MFMA operand read fall on different banks), tail scores [16][PAGE],
// m and l per wave and head [NW][16] each, the split-K flag
template <int D, int NW>
struct AfterLoop {
    static constexpr int QS = D + 4;
    static constexpr int NKP = NW / 2;                   // tail-score parts (contraction split NW / 2 ways)
    static constexpr int Q_OFF = 0, SC_OFF = 16 * QS * 4, ML_OFF = SC_OFF + NKP * 16 * PAGE * 4;
};

// N consecutive IN values kept packed in 32-bit words (a register-lean copy of a row slice)
template <typename IN, int N>
struct Packed {
    static constexpr int BYTES = N * (int)sizeof(IN), WORDS = BYTES / 4;
    static_assert(BYTES % 16 == 0 || BYTES == 8, "16-byte pieces, or one 8-byte piece");
    // zero at first: set() of a half-width element keeps the other half of its word, which must
    // then be a defined value (an uninitialized one lets the optimizer fold the word away)
    uint32_t wd[WORDS] = {};
    __device__ __forceinline__ void load(const IN* p) {          // p aligned to min(16, BYTES)
        if constexpr (BYTES % 16 == 0) {
#pragma unroll
            for (int i = 0; i < BYTES / 16; ++i) {
                const u4 v = reinterpret_cast<const u4*>(p)[i];
#pragma unroll
                for (int j = 0; j < 4; ++j) wd[4 * i + j] = v[j];
            }
        } else {
            const u2 v = *reinterpret_cast<const u2*>(p);
            wd[0] = v[0];
            wd[1] = v[1];
        }
    }
    __device__ __forceinline__ float get(int k) const {          // k a constant after unrolling
        if constexpr (sizeof(IN) == 4) {
            return __uint_as_float(wd[k]);
        } else {
            const uint16_t b = (uint16_t)((k & 1) ? wd[k / 2] >> 16 : wd[k / 2] & 0xFFFFu);
            return to_f32(__builtin_bit_cast(IN, b));
        }
    }
    __device__ __forceinline__ void set(int k, float x) {        // x exactly representable in IN
        if constexpr (sizeof(IN) == 4) {
            wd[k] = __float_as_uint(x);
        } else {
            const uint32_t b = __builtin_bit_cast(uint16_t, from_f32<IN>(x));
            wd[k / 2] = (k & 1) ? ((wd[k / 2] & 0xFFFFu) | (b << 16)) : ((wd[k / 2] & 0xFFFF0000u) | b);
        }
    }
};

// Rows r < n of an fp32 staging area [.][D] in LDS rotated back by the canonical Walsh-Hadamard
// transform and rounded once into out (row stride D), by THREADS threads: D / 16 lanes per row in the
// butterfly layout (a row's lanes iterate together).
template <int D, typename IN, int THREADS>
__device__ __forceinline__ void store_rotated(IN* __restrict__ out, const float* stage, int n, bool vec) {
    constexpr int CG = D / 16, RP = THREADS / CG;
    static_assert(THREADS % CG == 0, "whole rows per pass");
    const int c = (int)threadIdx.x % CG;
    for (int r = (int)threadIdx.x / CG; r < n; r += RP) {
        float x[16];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[j] = stage[r * D + 8 * c + j];
            x[8 + j] = stage[r * D + D / 2 + 8 * c + j];
        }
        fwht_runs<D>(x, c);
        if (vec) {
            put8<true>(out + (int64_t)r * D + 8 * c, x);
            put8<true>(out + (int64_t)r * D + D / 2 + 8 * c, x + 8);
        } else {
            put8<false>(out + (int64_t)r * D + 8 * c, x);
            put8<false>(out + (int64_t)r * D + D / 2 + 8 * c, x + 8);
        }
    }
}

// Split-K partials cross XCDs (separate L2s): stored write-through and read past the local L2, as
// relaxed device-scope atomics (global_store / global_load with sc1).
__device__ __forceinline__ void publish(float* p, float x) {
    __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float fetch(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two or four consecutive partial floats past the local L2 (64-bit relaxed agent-scope loads).
__device__ __forceinline__ void fetch2(const float* p, float& a, float& b) {
    const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    a = __uint_as_float((uint32_t)v);
    b = __uint_as_float((uint32_t)(v >> 32));
}
__device__ __forceinline__ f4 fetch4(const float* p) {
    float a, b, c, d;
    fetch2(p, a, b);
    fetch2(p + 2, c, d);
    return f4{a, b, c, d};
}

// The splits a wave has finished (wave splits with several splits per wave), folded in split order:
// a finished split's own softmax state (m, l, vb and its O and -HALF sum P' accumulators, per MFMA
// column) is merged into the folded one by log-sum-exp -- both rescaled to the larger max, a side over
// no keys adding nothing -- and the split's state starts afresh for the next split. Every accumulator
// is in the same units in every split, so the fold is the same weighted sum the merge of split
// partials forms, in a fixed order.
template <int DT>
struct SplitFold {
    f4 o[DT];
    f4 vacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = -__builtin_inff(), l = 0.0f, vb = 0.0f;
    __device__ __forceinline__ SplitFold() {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    __device__ __forceinline__ void fold(f4 (&so)[DT], f4& svacc, float& sm, float& sl, float& svb, bool reset) {
        const float M = __builtin_fmaxf(m, sm);
        const float a = m == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m - M);
        const float b = sm == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(sm - M);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] = o[dt] * a + so[dt] * b;
        vacc = vacc * a + svacc * b;
        l = l * a + sl * b;
        vb = vb * a + svb * b;
        m = M;
        if (reset) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) so[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
            svacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
            sm = -__builtin_inff();
            sl = 0.0f;
            svb = 0.0f;
        }
    }
    // the folded state back into the wave's running state (after its last split)
    __device__ __forceinline__ void restore(f4 (&so)[DT], f4& svacc, float& sm, float& sl, float& svb) const {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) so[dt] = o[dt];
        svacc = vacc;
        sm = m;
        sl = l;
        svb = vb;
    }
};

// (m, l) of two disjoint key sets in log2 units folded into one: the sums rescaled to the larger
// max; a side over no keys (m = -inf) adds nothing.
__device__ __forceinline__ void fold_ml(float& m, float& l, float m2, float l2) {
    const float M = __builtin_fmaxf(m, m2);
    const float a = m == -__builtin_inff() ? 0.0f : l * __builtin_amdgcn_exp2f(m - M);
    const float b = m2 == -__builtin_inff() ? 0.0f : l2 * __builtin_amdgcn_exp2f(m2 - M);
    m = M;
    l = a + b;
}

// LDS floats the split merge needs: m and l of every (split, head), each head's (M, L), and the
// threads' partial sums.
__host__ __device__ constexpr int merge_red_offset(int NS, int gn) {      // 16-byte aligned partial sums
    return (2 * NS * gn + 2 * 16 + 3) & ~3;
}
__host__ __device__ constexpr int merge_smem_floats(int NS, int gn, int NW) {
    return merge_red_offset(NS, gn) + NW * WAVE * 4;
}

// Merge of the NS split partials of one (sequence, kv head) -- rows (base + z) * G + g of part_ml
// [..][2] and part_o [..][D] -- for the heads g0 .. g0 + gn - 1 (gn <= 16), by the NW * 64 threads of
// the calling workgroup, in a fixed order (the same bits on every call), with many loads in flight
// instead of one dependent chain per split:
//   1. every (split, head)'s (m, l) is loaded (batches of independent loads) into smem; per head,
//      ZG1 = min(T / gn, NS) thread groups fold the splits zg, zg + ZG1, ... and the groups' results
//      fold in group order into (M_g, L_g);
//   2. out[g][d..d+3] = sum_z exp2(m_z - M_g) o_z[g][d..d+3] / L_g: thread j owns output quad j % NQ
//      over the splits z = j / NQ + k ZG (ZG = min(T / NQ, NS) groups), loads in batches, summed in z
//      order; the groups' sums add in group order.
// emit(g, d, f4) receives each merged quad (zeros for a head no split saw). smem holds
// merge_smem_floats(NS, gn, NW) floats. Ends with the workgroup synchronized.
template <int D, int NW, typename Emit>
__device__ void merge_splits(const float* __restrict__ part_ml, const float* __restrict__ part_o, int64_t base,
                             int NS, int G, int g0, int gn, float* smem, Emit&& emit) {
    constexpr int T = NW * WAVE, NQ1 = D / 4, B = 8;
    const int t = (int)threadIdx.x;
    const int P = NS * gn;
    float* const ms = smem;                        // [NS][gn]
    float* const ls = smem + P;                    // [NS][gn]
    float* const ML = smem + 2 * P;                // [16][2]
    float* const red = smem + merge_red_offset(NS, gn);   // [T][4]
    for (int p0 = t; p0 < P; p0 += B * T) {
        float bm[B], bl[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int p = p0 + u * T;
            bm[u] = -__builtin_inff();
            bl[u] = 0.0f;
            if (p < P) fetch2(part_ml + 2 * ((base + p / gn) * G + g0 + p % gn), bm[u], bl[u]);
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
            const int p = p0 + u * T;
            if (p < P) {
                ms[p] = bm[u];
                ls[p] = bl[u];
            }
        }
    }
    __syncthreads();
    const int ZG1 = max(1, min(T / gn, NS));       // split groups of phase 1 (no more than splits)
    if (t < gn * ZG1) {
        const int g = t % gn, zg = t / gn;
        float m = -__builtin_inff(), l = 0.0f;
        for (int z = zg; z < NS; z += ZG1) fold_ml(m, l, ms[z * gn + g], ls[z * gn + g]);
        red[2 * t] = m;
        red[2 * t + 1] = l;
    }
    __syncthreads();
    if (t < gn) {
        float m = -__builtin_inff(), l = 0.0f;
        for (int zg = 0; zg < ZG1; ++zg) fold_ml(m, l, red[2 * (zg * gn + t)], red[2 * (zg * gn + t) + 1]);
        ML[2 * t] = m;
        ML[2 * t + 1] = l;
    }
    __syncthreads();

    const int NQ = gn * NQ1;                       // output quads
    const int ZG = NQ >= T ? 1 : max(1, min(T / NQ, NS));     // split groups of phase 2
    for (int j = t; j < NQ * ZG; j += T) {
        const int q = j % NQ, zg = j / NQ, g = q / NQ1, d = 4 * (q % NQ1);
        const float M = ML[2 * g], L = ML[2 * g + 1];
        f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if (M > -__builtin_inff()) {
            for (int z0 = zg; z0 < NS; z0 += B * ZG) {
                f4 v[B];
                float wz[B];
#pragma unroll
                for (int u = 0; u < B; ++u) {
                    const int z = z0 + u * ZG;
                    v[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                    wz[u] = 0.0f;
                    if (z < NS) {
                        const float mzg = ms[z * gn + g];
                        if (mzg > -__builtin_inff()) {
                            v[u] = fetch4(part_o + ((base + z) * G + g0 + g) * D + d);
                            wz[u] = __builtin_amdgcn_exp2f(mzg - M);
                        }
                    }
                }
#pragma unroll
                for (int u = 0; u < B; ++u) acc += wz[u] * v[u];
            }
        }
        const float inv = L > 0.0f ? 1.0f / L : 0.0f;
        if (ZG == 1) {
            emit(g, d, acc * inv);
        } else {
            *reinterpret_cast<f4*>(red + 4 * j) = acc * inv;
        }
    }
    __syncthreads();
    if (ZG > 1 && t < NQ) {
        f4 sum = f4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int zg = 0; zg < ZG; ++zg) sum += *reinterpret_cast<const f4*>(red + 4 * (zg * NQ + t));
        emit(t / NQ1, 4 * (t % NQ1), sum);
    }
    __syncthreads();
}

// grid (S, Hkv, n_splits * ceil(G / 16)), block NW * 64. Registers are budgeted for two waves per SIMD
// (amdgpu_waves_per_eu(2); the library is built with MFMA accumulators in VGPRs): with a 512-register
// budget the 4-wave variant used 236 VGPRs + 76 AGPRs and spent 46 v_accvgpr moves per page in its
// loop; at <= 256 it needs none, and two 4-wave workgroups fit on one CU. ST = 2 (G <= 8): two page streams share the
// MFMA columns (page A of each pair in columns 0-7, page B in 8-15); ST = 1: one page's 16 heads.
// NS > 1: each workgroup writes its split's partials; with `sync` (one zeroed int32 per
// (sequence, kv head, head chunk)), the last workgroup of a (sequence, kv head, head chunk) to
// finish merges all splits into `out` and resets its counter, so no second launch is needed.
template <int D, int BITS, typename IN, int NW, int ST, bool ROT, bool WS, int DEP>
__global__ __launch_bounds__(NW * WAVE) __attribute__((amdgpu_waves_per_eu(2))) void decode_kernel(
    const IN* __restrict__ qg, IN* __restrict__ out, uint8_t* __restrict__ cache, int64_t bs, int64_t hs,
    IN* __restrict__ tail_k, const int32_t* __restrict__ tail_idx, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ seq_lens, int64_t bt_stride, int bt_cols, int H, int G, float p2, float rs, int NS,
    float* __restrict__ part_ml, float* __restrict__ part_o, int32_t* __restrict__ sync,
    const int32_t* __restrict__ seq_order, const IN* __restrict__ app_k, const IN* __restrict__ app_v, int64_t app_ks,
    int64_t app_vs, int KW) {
    constexpr bool ws = WS;
    using F = Fmt<D, BITS>;
    using R = Ring<D, BITS>;
    constexpr int KSTEPS = D / 32;
    constexpr int DT = D / 16;
    constexpr int NLO = BITS == 4 ? D / 32 : D / 16;          // O tiles in units of 2^-24 (the rest 2^-20)
    constexpr float TWO24 = 16777216.0f, TWO20 = 1048576.0f;
    constexpr bool QLO = std::is_same<IN, float>::value;      // q needs a low fp16 part
    const float sm_log2 = p2 * rs;                            // exact: p2 is a power of two
    static_assert(NW == 2 || NW == 4 || NW == 8, "the tail splits 16 heads over 2 NW lane halves");
    static_assert(ST == 1 || ST == 2, "one or two page streams");
    using AL = AfterLoop<D, NW>;
    static_assert(2 * NW * R::SLOT >= AL::ML_OFF + 2 * NW * 16 * 4 + 16, "the after-loop scratch must fit");
    static_assert(2 * R::DMA <= 63, "vmcnt holds at most 63 loads");
    static_assert(DEP == 2 || (DEP == 3 && !ROT && !WS && decode_fits3<D, BITS, NW>()),
                  "three pairs per wave: unrotated, shared splits, where the third array fits");
    static_assert(2 * NW * R::SLOT >= 16 * D * 4, "ROT stages the chunk's q rows in the second array");
    static_assert(2 * NW * R::SLOT >= tile_bytes<D, IN>(), "the fused append's K tile lives in the first array");

    // one array per page pair (wave w at 2 w R::SLOT): the compiler tells the pairs apart and leaves
    // the DMA waits to the explicit vmcnt below (it need not tell the two pages of a pair apart: a
    // pair is only read once both have landed)
    __shared__ __align__(16) uint8_t ringA[2 * NW * R::SLOT];
    __shared__ __align__(16) uint8_t ringB[2 * NW * R::SLOT];
    __shared__ __align__(16) uint8_t ringC[DEP == 3 ? 2 * NW * R::SLOT : 16];   // DEP = 3 only
    __shared__ __align__(16) int tbl[WIN];                               // block ids of the window
    float* const m_l = reinterpret_cast<float*>(ringB + AL::ML_OFF);      // after the loop only
    float* const l_l = m_l + NW * 16;
    int* const last_flag = reinterpret_cast<int*>(l_l + NW * 16);

    KUSH_TIMELINE_DECL;
    KUSH_MARK(0);
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);   // wave-uniform: scalar page loop
    const int r16 = lane & 15, q = lane >> 4;
    // with seq_order, workgroups go out sequence by sequence (all kv heads of one, then the next) in
    // the given order: the hardware starts workgroups in linear order
    int s = blockIdx.x, h = blockIdx.y;
    if (seq_order != nullptr) {
        const int L = blockIdx.x + gridDim.x * blockIdx.y;
        s = seq_order[L / H];
        h = L % H;
    }
    // ws (wave splits, NS a multiple of NW KW): each wave takes KW whole consecutive splits of its own --
    // splits (zg NW + w) KW .. + KW - 1 of workgroup zg, one contiguous run of pages -- with its own
    // block-id table and no merge with the other waves until the end; else the waves of a workgroup
    // share its split's pages. With KW > 1 a wave starts a fresh softmax state at each of its splits
    // and folds the finished split into its running state in split order (a log-sum-exp merge).
    const int NSG = ws ? NS / (NW * KW) : NS;                             // workgroups per head chunk
    const int zg = blockIdx.z % NSG, gc = blockIdx.z / NSG, g0 = gc * 16;
    const int z = ws ? (zg * NW + w) * KW : zg;                           // this wave's (first) split
    const int tw = ws ? NW - 1 : 0;                                       // the wave taking the partial page
    // ws with the in-launch merge (sync): the workgroup first merges its NW splits in LDS and writes one
    // partial (index zg of NSG), so the last workgroup merges NSG partials; without sync every wave
    // writes its own (index z of NS) for the caller's combine over NS
    const bool wmerge = ws && sync != nullptr, own = ws && !wmerge;
    const int NSP = wmerge ? NSG : NS, zp = wmerge ? zg : z;                   // partials per head chunk, this one's
    const int Gc = min(16, G - g0);

    const int32_t* bt = block_table + (int64_t)s * bt_stride;
    const int64_t qbase = ((int64_t)s * H + h) * G * D + (int64_t)g0 * D;
    // Issued before the length is read, which neither depends on: this lane's q head (B column r16)
    // over its contraction dims (8 consecutive dims per K-step; lanes of heads past the chunk read
    // the chunk's last head and zero it later) and, for split 0 (whose pages start at 0), the first
    // window's block ids up to the table's column count bt_cols (entries past the length are never
    // used). The length then arrives with them instead of before them.
    const int hq = ST == 2 ? (r16 & 7) : r16;                            // the head of this lane's column
    const bool gv = hq < Gc;
    float qv[KSTEPS][8];
    // ROT: the q rows in the butterfly layout instead (thread t: head t / QCG + QRP pp, dims 8 qc.. and
    // D/2 + 8 qc..), rotated once the length is known
    constexpr int QCG = D / 16, QRP = NW * WAVE / QCG, QPASS = (16 + QRP - 1) / QRP;
    const int qc = (int)threadIdx.x % QCG;
    float qrow[ROT ? QPASS : 1][16];
    if constexpr (ROT) {
#pragma unroll
        for (int pp = 0; pp < QPASS; ++pp) {
            const int rr = min((int)threadIdx.x / QCG + pp * QRP, Gc - 1);
            load8(qg + qbase + (int64_t)rr * D + 8 * qc, reinterpret_cast<float(&)[8]>(qrow[pp][0]));
            load8(qg + qbase + (int64_t)rr * D + D / 2 + 8 * qc, reinterpret_cast<float(&)[8]>(qrow[pp][8]));
        }
    } else {
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk) load8(qg + qbase + (int64_t)min(hq, Gc - 1) * D + kdim<D, BITS>(kk, q, 0), qv[kk]);
    }
    constexpr int PRE = WIN / (NW * WAVE);                               // prefetched ids per thread
    const int npre = !ws && z == 0 ? min(WIN, bt_cols) : 0;
    int pre[PRE];
#pragma unroll
    for (int k = 0; k < PRE; ++k) {
        const int i = (int)threadIdx.x + k * NW * WAVE;
        pre[k] = i < npre ? bt[i] : 0;
    }

    const int n = seq_lens[s];
    const int tix = tail_idx != nullptr ? tail_idx[s] : 0;              // the tail slot, with the length
    const int full = n / PAGE, tail_n = n % PAGE;
    const int pps = (full + NS - 1) / NS;
    const int p0 = min(full, z * pps), p1 = min(full, p0 + (ws ? KW : 1) * pps);
    const int wp1 = ws ? min(full, (zg + 1) * NW * KW * pps) : p1, wp0 = ws ? min(full, zg * NW * KW * pps) : p0;
    const uint8_t* head_base = cache + (int64_t)h * hs;

    // Fused append (app_k): the token at position n - 1 of sequence s, kv head h, is written by the one
    // workgroup that reads its page -- the split holding the page when the token completes it, else
    // the last split (which takes the partial page) -- of the first head chunk (the entry point takes
    // at most 16 q heads per kv head). Its stores are complete and visible to its own page loads after
    // the barrier; no other workgroup reads that page or the sequence's tail.
    if (app_k != nullptr) {
        if (gc == 0 && n > 0) {
            const int pos = n - 1, slot = pos % PAGE, pg = pos / PAGE;
            const int owner = slot == PAGE - 1 ? pg / max(pps, 1) : NS - 1;
            if (zg == (ws ? owner / (NW * KW) : owner)) {           // the whole workgroup
                const IN* krow = app_k + (int64_t)s * app_ks + (int64_t)h * D;
                IN* tail = tail_k + ((int64_t)tix * H + h) * PAGE * D;
                uint8_t* rec = cache + (int64_t)bt[pg] * bs + (int64_t)h * hs;
                stash_rows<D, IN, true, ROT, NW * WAVE>(tail + slot * D, krow, 0, 1, (int)threadIdx.x);
                page_task<D, BITS, IN, true, NW * WAVE, ROT>(tail, krow, 0, PAGE - 1, slot == PAGE - 1,
                                                             app_v + (int64_t)s * app_vs + (int64_t)h * D, 0, slot,
                                                             slot + 1, rec, ringA);
            }
        }
        __syncthreads();
    }
    const bool has_tail = tail_n > 0 && zg == NSG - 1;                 // the workgroup holds the last split
    const int tail_blk = has_tail ? bt[full] : 0;                      // in before the page loop starts
    uint8_t* const sl0 = ringA + 2 * w * R::SLOT;
    uint8_t* const sl1 = sl0 + R::SLOT;
    uint8_t* const sl2 = ringB + 2 * w * R::SLOT;
    uint8_t* const sl3 = sl2 + R::SLOT;
    uint8_t* const sl4 = ringC + 2 * w * R::SLOT;                      // DEP = 3 only
    uint8_t* const sl5 = sl4 + R::SLOT;

    // per-lane DMA source offsets (swizzled code rows), fixed for every page
    uint32_t voff[R::DMA];
#pragma unroll
    for (int i = 0; i < R::DMA; ++i) voff[i] = src_chunk<D, BITS>(R::chunk0(i) + lane) * 16u;

    f4 o[DT], vacc = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = f4{0.0f, 0.0f, 0.0f, 0.0f};
    float m_run = -__builtin_inff(), l_run = 0.0f, vb_run = 0.0f;
    // ws, KW > 1: the splits this wave finished, folded in split order (fold_split), and the pages left
    // in the split being streamed
    SplitFold<DT> folded;
    int split_left = pps;

    // Partial page (last split): its exact-K scores are 16 x 16 x 4 fp32 MFMAs (fp32 products and
    // sums) over all waves: wave w takes tokens 16 (w & 1) .. + 15 and part w >> 1 of the contraction
    // (NKP = NW / 2 parts); lane: head (A row) and token (B column) lane % 16, dims [sdim, sdim + DS)
    // (the 4 lane groups are the MFMA's contraction). The lane's K and q slices go out right after the
    // first page DMAs and wait in registers until the loop ends (when they fit in 16 VGPRs, 32 at two
    // waves); wave 0 issues the page's DMA into its slot 0 in place of its first empty issue of the
    // last window, so both are in when the loop ends.
    constexpr int NKP = AL::NKP, DS = D / (4 * NKP);
    constexpr bool TPRE = 2 * Packed<IN, DS>::WORDS <= (NW == 2 ? 32 : 16);
    const int tt = 16 * (w & 1) + r16, kp = w >> 1;
    const int sdim = kp * (D / NKP) + q * DS;                          // first dim of the lane's slices
    const IN* const ktail = tail_k + (((int64_t)tix * H + h) * PAGE + min(tt, tail_n - 1)) * D + sdim;
    Packed<IN, DS> kpk, qpk;
    bool tpre = false, tdma = false;                                   // slices loaded, page DMA issued

    // The split's pages go out in pairs (k: pages 2k, 2k + 1 of the window), over windows of WIN pages
    // whose block ids are first copied to an LDS table. Wave w takes pairs w, w + NW, ...: a fixed
    // assignment, so which wave sums which page, and in which order, never changes between calls
    // (a counter handing pairs to whichever wave asks first balances two waves per SIMD better, but
    // then the sums, and so the output bits, vary from call to call). A wave holds two pairs,
    // in slots (0, 1) and (2, 3): one is consumed while the other is in flight. A wave's pairs only
    // grow, so once the pair it would consume is past the window's end, so is the one in flight. Each
    // pair issue is 2 R::DMA instructions, also for a pair past the end (an empty buffer range: no
    // memory access), so vmcnt counts stay exact.
    if (wp1 > wp0) {                                                     // the workgroup has pages (uniform)
        // windows of TW pages in the table region tb: the workgroup's (ws: the wave's own, a wave with
        // no pages of its own runs empty pairs)
        constexpr int TWS = WIN / NW;
        const int TW = ws ? TWS : WIN;
        int* const tb = tbl + (ws ? w * TWS : 0);
        const int PS = ws ? 1 : NW;                                      // the wave's pair stride
        int wb = p0, wn = min(TW, p1 - p0), pairs = (wn + 1) / 2;
        const auto load_window = [&]() {
            if (wb == 0 && wn <= npre) {                                 // split 0's first window, prefetched
#pragma unroll
                for (int k = 0; k < PRE; ++k) {
                    const int i = (int)threadIdx.x + k * NW * WAVE;
                    if (i < wn) tbl[i] = pre[k];
                }
            } else {                                                     // every id load in flight at once
                int ids[PRE];
#pragma unroll
                for (int k = 0; k < PRE; ++k) {
                    const int i = (int)threadIdx.x + k * NW * WAVE;
                    ids[k] = i < wn ? bt[wb + i] : 0;
                }
#pragma unroll
                for (int k = 0; k < PRE; ++k) {
                    const int i = (int)threadIdx.x + k * NW * WAVE;
                    if (i < wn) tbl[i] = ids[k];
                }
            }
        };
#define KUSH_ISSUE_PAIR(SA, SB, P)                                                                 \
    {                                                                                              \
        const int2 id2 = *reinterpret_cast<const int2*>(tb + min(2 * (P), TW - 2));                \
        issue_page<D, BITS>(SA, (P) < pairs, __builtin_amdgcn_readfirstlane(id2.x), head_base, bs, voff);  \
        issue_page<D, BITS>(SB, 2 * (P) + 1 < wn, __builtin_amdgcn_readfirstlane(id2.y), head_base, bs, voff); \
    }
        // the window's ids are stored and every load of the compiler's is in before the barrier: no
        // vector memory load of the compiler's is outstanding once the page DMAs start
        if constexpr (WS) load_wave_window<PRE>(tb, bt + wb, wn, lane);
        else load_window();
        int pa = ws ? 0 : w, pb = pa + PS, pc = pb + PS;                 // the pairs in slots (0, 1), (2, 3), (4, 5)
        // The first pairs go out before q is prepared: every compiler load in (vmcnt 0, so no later
        // wait of the compiler's counts the DMAs), the table's barrier, pair pa's DMAs into the first
        // array and pair pb's into the second; a rotated q is staged in the second array instead,
        // and pair pb waits until every wave has read it back.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        KUSH_MARK(1);
        KUSH_ISSUE_PAIR(sl0, sl1, pa)
        // the tail's slices between the first pair and the rest: the first step's wait (the later
        // pairs outstanding) then completes exactly the first pair and the slices, as with ROT
        if (!ROT && TPRE && has_tail) {
            kpk.load(ktail);
            qpk.load(qg + qbase + (int64_t)min(r16, Gc - 1) * D + sdim);
            tpre = true;
        }
        if constexpr (!ROT) KUSH_ISSUE_PAIR(sl2, sl3, pb)
        if constexpr (DEP == 3) KUSH_ISSUE_PAIR(sl4, sl5, pc)
        if constexpr (ROT) {                                             // rotate, round to IN, regather
            float* const qst = reinterpret_cast<float*>(ringB);          // [16][D]
#pragma unroll
            for (int pp = 0; pp < QPASS; ++pp) {
                const int rr = (int)threadIdx.x / QCG + pp * QRP;
                if (rr < 16) {                                           // a row's lanes branch together
                    fwht_runs<D>(qrow[pp], qc);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        qst[rr * D + 8 * qc + j] = to_f32(store_rounded<IN>(qrow[pp][j]));
                        qst[rr * D + D / 2 + 8 * qc + j] = to_f32(store_rounded<IN>(qrow[pp][8 + j]));
                    }
                }
            }
            __syncthreads();
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
                for (int j = 0; j < 8; ++j) qv[kk][j] = qst[min(hq, Gc - 1) * D + kdim<D, BITS>(kk, q, 0) + j];
            if (TPRE && has_tail) {
                kpk.load(ktail);
#pragma unroll
                for (int e = 0; e < DS; ++e) qpk.set(e, qst[min(r16, Gc - 1) * D + sdim + e]);
                tpre = true;
            }
        }
        // q' = q p2 as fp16 (+ its low part for fp32 q): qh, ql for the bias MFMAs; qa, qla the Q'
        // sources, divided by 16 in the int4 K-steps of high nibbles
        h8 qh[KSTEPS], ql[KSTEPS], qa[KSTEPS], qla[KSTEPS];
#pragma unroll
        for (int kk = 0; kk < KSTEPS; ++kk)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float xq = gv ? qv[kk][j] * p2 : 0.0f;
                const _Float16 hi = (_Float16)xq;
                const _Float16 lo = QLO ? (_Float16)(xq - (float)hi) : (_Float16)0.0f;
                const bool hin = BITS == 4 && (kk & 1);
                qh[kk][j] = hi;
                ql[kk][j] = lo;
                qa[kk][j] = hin ? (_Float16)((float)hi * 0.0625f) : hi;
                qla[kk][j] = hin ? (_Float16)((float)lo * 0.0625f) : lo;
            }
        const float sa = rs * TWO24;                             // x = sa s + kx
        if constexpr (ROT) {
            __syncthreads();                                     // every wave done with the staged q
            KUSH_ISSUE_PAIR(sl2, sl3, pb)
        }

        // One pair step: the pair has landed once at most the other pair's loads are outstanding;
        // scores of both pages (the next pair's table read hides behind them), one softmax update,
        // PV of both; then, every read of the
        // two slots complete (lgkmcnt 0), they take the next pair. The second page of a window's odd
        // last pair is masked.
#define KUSH_STEP(SA, SB, P, FIRST)                                                                \
    {                                                                                              \
        if ((P) >= pairs) break;                                                                   \
        KUSH_WAIT_VM((DEP - 1) * 2 * R::DMA);                                                      \
        if ((P) == 0) KUSH_MARK(2);                                                                \
        const int nx = (P) + DEP * PS;                   /* this wave's next pair in these slots */ \
        int2 id2;                                                                                  \
        if constexpr (ST == 2) {                                                                   \
            float sv[8], kx;                                                                       \
            pair_scores2<D, BITS, QLO>(SA, qa, qla, qh, ql, sv, kx, rs, lane);                     \
            if (2 * (P) + 1 >= wn && r16 >= 8) kx = -__builtin_inff();   /* page B masked */        \
            id2 = *reinterpret_cast<const int2*>(tb + min(2 * nx, TW - 2));                        \
            consume2<D, BITS>(SA, R::SLOT, o, vacc, sv, sa, kx, m_run, l_run, vb_run, lane);       \
        } else {                                                                                   \
            const uint8_t* const sp[2] = {SA, SB};                                                 \
            float sv[2][8], kx[2];                                                                 \
            pair_scores<D, BITS, QLO>(SA, qa, qla, qh, ql, sv, kx, rs, lane);                      \
            /* page B masked without a branch: a uniform branch here put the reads of the last  */ \
            /* bias MFMA's results (kx) 3 wait states after it on the taken path (8 needed), a  */ \
            /* join the compiler's hazard check does not cover (tests/test_isa.py checks every  */ \
            /* path)                                                                            */ \
            const float pbm = 2 * (P) + 1 >= wn ? -__builtin_inff() : 0.0f;                        \
            _Pragma("unroll") for (int jj = 0; jj < 8; ++jj) sv[1][jj] += pbm;                     \
            id2 = *reinterpret_cast<const int2*>(tb + min(2 * nx, TW - 2));                        \
            consume_pages<D, BITS, 2>(sp, o, vacc, sv, sa, kx, m_run, l_run, vb_run, lane);        \
        }                                                                                          \
        __builtin_amdgcn_s_waitcnt(0xC07F);                    /* lgkmcnt(0): slot reads done */    \
        const bool tl = (FIRST) && w == tw && has_tail && !tdma && nx >= pairs && wb + TW >= p1;       \
        issue_page<D, BITS>(SA, nx < pairs || tl, tl ? tail_blk : __builtin_amdgcn_readfirstlane(id2.x), \
                            head_base, bs, voff);                                                  \
        issue_page<D, BITS>(SB, 2 * nx + 1 < wn, __builtin_amdgcn_readfirstlane(id2.y), head_base, bs, voff); \
        tdma = tdma || tl;                                                                         \
        if constexpr (WS) {                                                                        \
            split_left -= 2;                                 /* a split holds an even page count */ \
            if (split_left == 0 && KW > 1) {                                                       \
                split_left = pps;                                                                  \
                if (wb + 2 * (P) + 2 < p1) folded.fold(o, vacc, m_run, l_run, vb_run, true);       \
            }                                                                                      \
        }                                                                                          \
        (P) = nx;                                                                                  \
    }
        for (;;) {
            for (;;) {
                KUSH_STEP(sl0, sl1, pa, true)
                KUSH_STEP(sl2, sl3, pb, false)
                if constexpr (DEP == 3) KUSH_STEP(sl4, sl5, pc, false)
            }
            KUSH_MARK_WAVE();
            KUSH_WAIT_VM(0);                                     // drain the trailing (empty) issues
            if (!ws) __syncthreads();                            // table and rings idle (ws: the wave's own)
            wb += TW;
            if (wb >= p1) break;
            wn = min(TW, p1 - wb);
            pairs = (wn + 1) / 2;
            pa = ws ? 0 : w;
            pb = pa + PS;
            pc = pb + PS;
            if constexpr (WS) load_wave_window<PRE>(tb, bt + wb, wn, lane);   // a wave's DS operations stay in order
            else load_window();
            if (!ws) __syncthreads();
            KUSH_ISSUE_PAIR(sl0, sl1, pa)
            KUSH_ISSUE_PAIR(sl2, sl3, pb)
            if constexpr (DEP == 3) KUSH_ISSUE_PAIR(sl4, sl5, pc)
        }
        if (ws) __syncthreads();                                 // every wave's pages done: rings idle
#undef KUSH_STEP
#undef KUSH_ISSUE_PAIR
    }
    KUSH_MARK(3);

    // partial last page (last split only): V rows from its record in wave tw's slot 0 (issued in the
    // loop, else now); the exact-K scores as set out before the loop, their NKP parts summed in order
    if (has_tail) {
        constexpr int QS = AL::QS;
        float* const qs = reinterpret_cast<float*>(ringB + AL::Q_OFF);    // [16][QS] rotated q (no prefetch)
        float* const sc = reinterpret_cast<float*>(ringB + AL::SC_OFF);   // [NKP][16][PAGE] score parts
        uint8_t* const tslot = ringA + 2 * tw * R::SLOT;                   // wave tw's slot 0
        if (w == tw && !tdma) issue_page<D, BITS>(tslot, true, tail_blk, head_base, bs, voff);
        if (!tpre) {                                                       // the slices now
            kpk.load(ktail);
            if constexpr (ROT) {                                           // rotated q rows, as in the prologue
                for (int rr = (int)threadIdx.x / QCG; rr < 16; rr += QRP) {  // a row's lanes iterate together
                    float x[16];
                    load8(qg + qbase + (int64_t)min(rr, Gc - 1) * D + 8 * qc, reinterpret_cast<float(&)[8]>(x[0]));
                    load8(qg + qbase + (int64_t)min(rr, Gc - 1) * D + D / 2 + 8 * qc,
                          reinterpret_cast<float(&)[8]>(x[8]));
                    fwht_runs<D>(x, qc);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        qs[rr * QS + 8 * qc + j] = to_f32(store_rounded<IN>(x[j]));
                        qs[rr * QS + D / 2 + 8 * qc + j] = to_f32(store_rounded<IN>(x[8 + j]));
                    }
                }
                __syncthreads();
#pragma unroll
                for (int e = 0; e < DS; ++e) qpk.set(e, qs[min(r16, Gc - 1) * QS + sdim + e]);
            } else {
                qpk.load(qg + qbase + (int64_t)min(r16, Gc - 1) * D + sdim);
            }
        }
        f4 c = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < DS; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(qpk.get(e) * sm_log2, kpk.get(e), c, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[(kp * 16 + 4 * q + i) * PAGE + tt] = tt < tail_n ? c[i] : -__builtin_inff();
        __syncthreads();
        if (w == tw) {
            float x[1][8];
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                float v = 0.0f;
#pragma unroll
                for (int k = 0; k < NKP; ++k) v += sc[(k * 16 + r16) * PAGE + tok(q, jj)];
                x[0][jj] = ST == 2 && r16 >= 8 ? -__builtin_inff() : v;
            }
            KUSH_WAIT_VM(0);
            if constexpr (ST == 2) {                             // stream 0 takes the page
                consume2<D, BITS>(tslot, 0, o, vacc, x[0], 1.0f, 0.0f, m_run, l_run, vb_run, lane);
            } else {
                const uint8_t* const sp[1] = {tslot};
                const float b0[1] = {0.0f};
                consume_pages<D, BITS, 1>(sp, o, vacc, x, 1.0f, b0, m_run, l_run, vb_run, lane);
            }
        }
    }

    if constexpr (WS) {                                          // the wave's last split, folded in last
        // The fold reuses registers the partial page's last MFMAs still write, behind a uniform branch:
        // on its taken path the compiler kept 7 wait states after them (8 needed), a join its hazard
        // check does not cover. Nothing sinks below this point, and 8 wait states follow it.
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7");
        if (KW > 1) {
            folded.fold(o, vacc, m_run, l_run, vb_run, false);
            folded.restore(o, vacc, m_run, l_run, vb_run);
        }
    }

    // Merge the waves (and, ST = 2, the two streams of a head: columns c and c ^ 8). After one
    // barrier every wave has the workgroup max M and denominator L of its columns' heads from the
    // waves' (m, l); it scales its O by exp2(m - M) (and, without splits, by 1 / L) and stores all 16
    // columns in the idle rings (region of wave ww: 16 D floats, dims d as [d / 4][column][d % 4],
    // one 16-byte store per lane and tile). After a second barrier wave w sums tiles w, w + NW, ...
    // over the waves (and a head's two stream columns) and writes them out. No lane shuffles or
    // masked stores: on one wave per SIMD this tail is latency-bound. ws: every wave its own split,
    // so the same steps over its own columns only, all its tiles.
    constexpr int OBYTES = 16 * D * 4;
    static_assert(NW * OBYTES <= 2 * NW * R::SLOT, "the merge needs 16 D floats per wave in the first array");
    l_run = rows_sum(l_run);
    vb_run = __builtin_fmaf(vacc[0], TWO24, rows_sum(vb_run));   // every row of vacc holds the head's sum
    if (q == 0) {
        m_l[w * 16 + r16] = m_run;
        l_l[w * 16 + r16] = l_run;
    }
    __syncthreads();                                             // rings idle, m_l / l_l complete
    const int rx = ST == 2 ? (r16 ^ 8) : r16;                    // the other stream's column of this head
    // M and the softmax denominator of this column's head: every wave's (and stream's) l at the
    // workgroup max. A column that saw no token holds m = -inf and l = 0, and exp2(-inf) = 0, so no
    // term needs a branch and all the LDS reads go out together (the sum keeps its order)
    float mv[NW][ST], lv[NW][ST];
#pragma unroll
    for (int ww = 0; ww < NW; ++ww)
#pragma unroll
        for (int c2 = 0; c2 < ST; ++c2) {
            mv[ww][c2] = m_l[ww * 16 + (c2 ? rx : r16)];
            lv[ww][c2] = l_l[ww * 16 + (c2 ? rx : r16)];
        }
    float M = -__builtin_inff();
#pragma unroll
    for (int ww = 0; ww < NW; ++ww)
#pragma unroll
        for (int c2 = 0; c2 < ST; ++c2)
            if (!ws || wmerge || ww == w) M = __builtin_fmaxf(M, mv[ww][c2]);
    float L = 0.0f;
    if (M > -__builtin_inff()) {
#pragma unroll
        for (int ww = 0; ww < NW; ++ww)
#pragma unroll
            for (int c2 = 0; c2 < ST; ++c2)
                if (!ws || wmerge || ww == w) L += lv[ww][c2] * __builtin_amdgcn_exp2f(mv[ww][c2] - M);
    }
    const float inv_l = L > 0.0f ? 1.0f / L : 0.0f;
    {
        // split partials stay unnormalized (L goes out beside them)
        const float f = m_run == -__builtin_inff() ? 0.0f : __builtin_amdgcn_exp2f(m_run - M) * (NS == 1 ? inv_l : 1.0f);
        uint8_t* reg = ringA + w * OBYTES;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            f4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = __builtin_fmaf(o[dt][i], dt < NLO ? TWO24 : TWO20, vb_run) * f;
            *reinterpret_cast<f4*>(reg + (((4 * dt + q) * 16 + r16) * 4) * 4) = v;
        }
    }
    __syncthreads();
    const int64_t pb = (((int64_t)s * H + h) * NSP + zp) * G + g0 + r16; // partials row of head r16
    const bool out_vec = (((uintptr_t)out) & 15) == 0;
    const int hcol = ST == 2 ? (r16 & 7) : r16;                  // the (first) column of head r16
    float* const ostage = reinterpret_cast<float*>(ringB + AL::Q_OFF);   // ROT: [16][D] output rows
    for (int dt = own ? 0 : w; dt < DT; dt += own ? 1 : NW) {
        f4 acc = f4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (WS) {
            if (own) {                                           // this wave's own pieces
                f4 part[ST];
#pragma unroll
                for (int c2 = 0; c2 < ST; ++c2)
                    part[c2] = *reinterpret_cast<const f4*>(ringA + w * OBYTES + (((4 * dt + q) * 16 + hcol + 8 * c2) * 4) * 4);
#pragma unroll
                for (int c2 = 0; c2 < ST; ++c2) acc += part[c2];
            } else {                                             // the workgroup's NW splits, merged here
                f4 part[NW][ST];
#pragma unroll
                for (int ww = 0; ww < NW; ++ww)
#pragma unroll
                    for (int c2 = 0; c2 < ST; ++c2)
                        part[ww][c2] = *reinterpret_cast<const f4*>(ringA + ww * OBYTES +
                                                                    (((4 * dt + q) * 16 + hcol + 8 * c2) * 4) * 4);
#pragma unroll
                for (int ww = 0; ww < NW; ++ww)
#pragma unroll
                    for (int c2 = 0; c2 < ST; ++c2) acc += part[ww][c2];
            }
        } else {
            f4 part[NW][ST];                                     // every wave's pieces, read together
#pragma unroll
            for (int ww = 0; ww < NW; ++ww)
#pragma unroll
                for (int c2 = 0; c2 < ST; ++c2)
                    part[ww][c2] = *reinterpret_cast<const f4*>(ringA + ww * OBYTES +
                                                                (((4 * dt + q) * 16 + hcol + 8 * c2) * 4) * 4);
#pragma unroll
            for (int ww = 0; ww < NW; ++ww)
#pragma unroll
                for (int c2 = 0; c2 < ST; ++c2) acc += part[ww][c2];
        }
        if (r16 < Gc) {
            const int d0 = 16 * dt + 4 * q;
            if (ROT && NS == 1) {                                // fp32 rows, rotated below
                *reinterpret_cast<f4*>(ostage + r16 * D + d0) = acc;
            } else if (NS == 1) {
                IN* dst = out + qbase + r16 * D + d0;
                if (out_vec) {                                   // one 8- or 16-byte store
                    IN v4[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) v4[i] = from_f32<IN>(acc[i]);
                    if constexpr (sizeof(IN) == 2) {
                        *reinterpret_cast<u2*>(dst) = __builtin_bit_cast(u2, v4);
                    } else {
                        *reinterpret_cast<f4*>(dst) = __builtin_bit_cast(f4, v4);
                    }
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) dst[i] = from_f32<IN>(acc[i]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) publish(part_o + pb * D + d0 + i, acc[i]);
            }
        }
    }
    if (ROT && NS == 1) {
        __syncthreads();
        store_rotated<D, IN, NW * WAVE>(out + qbase, ostage, Gc, out_vec);
    }
    KUSH_MARK(4);
    KUSH_MARK_FLUSH();
    if (NS > 1 && (own || w == 0) && q == 0 && r16 < Gc) {
        publish(part_ml + 2 * pb, M);
        publish(part_ml + 2 * pb + 1, L);
    }
    if (NS == 1 || sync == nullptr) return;

    // split-K: the last workgroup of this (sequence, kv head, head chunk) merges every split. The
    // partials went out as write-through stores (publish); once every wave has seen them complete
    // (vmcnt 0, then the barrier), thread 0 counts the split in at the device's coherence point, and
    // the last workgroup reads the other splits' partials past its own XCD's L2 (fetch). No L2-wide
    // write-back or invalidate, which would stall every other workgroup streaming on the XCD.
    KUSH_WAIT_VM(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int n_gc = gridDim.z / NSG;
        int32_t* ctr = sync + ((int64_t)s * H + h) * n_gc + gc;
        const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last_flag = prev == NSG - 1;                            // one count per workgroup (ws: NW splits)
        if (prev == NSG - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last_flag) return;
    const int64_t base = ((int64_t)s * H + h) * NSP;
    if (merge_smem_floats(NSP, Gc, NW) * 4 <= 2 * NW * R::SLOT) {      // the idle first ring holds the scratch
        merge_splits<D, NW>(part_ml, part_o, base, NSP, G, g0, Gc, reinterpret_cast<float*>(ringA),
                            [&](int g, int d, f4 v) {
                                if constexpr (ROT) {
                                    *reinterpret_cast<f4*>(ostage + g * D + d) = v;
                                } else {
#pragma unroll
                                    for (int i = 0; i < 4; ++i) out[qbase + g * D + d + i] = from_f32<IN>(v[i]);
                                }
                            });
        if constexpr (ROT) store_rotated<D, IN, NW * WAVE>(out + qbase, ostage, Gc, out_vec);
        return;
    }
    for (int i = threadIdx.x; i < Gc * D; i += NW * WAVE) {      // one dependent chain per split (large NS)
        const int g = g0 + i / D, d = i % D;
        float Mg = -__builtin_inff();
        for (int zz = 0; zz < NSP; ++zz) Mg = __builtin_fmaxf(Mg, fetch(part_ml + 2 * ((base + zz) * G + g)));
        float L = 0.0f, acc = 0.0f;
        if (Mg > -__builtin_inff()) {
            for (int zz = 0; zz < NSP; ++zz) {
                const int64_t pb = (base + zz) * G + g;
                const float mz = fetch(part_ml + 2 * pb);
                if (mz > -__builtin_inff()) {
                    const float fz = __builtin_amdgcn_exp2f(mz - Mg);
                    L += fetch(part_ml + 2 * pb + 1) * fz;
                    acc += fz * fetch(part_o + pb * D + d);
                }
            }
        }
        const float val = L > 0.0f ? acc / L : 0.0f;
        if constexpr (ROT) {
            ostage[i] = val;
        } else {
            out[qbase + i] = from_f32<IN>(val);
        }
    }
    if constexpr (ROT) {
        __syncthreads();
        store_rotated<D, IN, NW * WAVE>(out + qbase, ostage, Gc, out_vec);
    }
}

// Merged output of head g, dim d of (sequence, kv head) `base / NS` from its NS split partials
__device__ __forceinline__ float combine_one(const float* __restrict__ part_ml, const float* __restrict__ part_o,
                                             int64_t base, int NS, int G, int D, int g, int d) {
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
    return L > 0.0f ? o / L : 0.0f;
}

// grid (S, Hkv), block 256: merge split-K partials (M, L, unnormalized O) into the output, 16 heads
// at a time. M is in log2 units; splits with no tokens (M = -inf) add nothing (gpu.mojo:469-491).
// parallel: merge_splits over the dynamic LDS (merge_smem_floats(NS, 16, 4) floats at most); else one
// dependent chain per element (very large NS). ROT: each chunk's merged rows are rotated back through
// LDS before their one rounding.
template <int D, typename IN, bool ROT>
__global__ __launch_bounds__(256) void combine_kernel(IN* __restrict__ out, const float* __restrict__ part_ml,
                                                      const float* __restrict__ part_o, int NS, int H, int G,
                                                      int parallel) {
    extern __shared__ float merge_lds[];
    __shared__ float stage[ROT ? 16 * D : 1];
    const int s = blockIdx.x, h = blockIdx.y;
    const int64_t base = ((int64_t)s * H + h) * NS;
    IN* const orow = out + ((int64_t)s * H + h) * G * D;
    const bool vec = (((uintptr_t)out) & 15) == 0;
    for (int g0 = 0; g0 < G; g0 += 16) {
        const int gn = min(16, G - g0);
        if (parallel) {
            merge_splits<D, 4>(part_ml, part_o, base, NS, G, g0, gn, merge_lds, [&](int g, int d, f4 v) {
                if constexpr (ROT) {
                    *reinterpret_cast<f4*>(stage + g * D + d) = v;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) orow[(int64_t)(g0 + g) * D + d + i] = from_f32<IN>(v[i]);
                }
            });
        } else {
            for (int i = threadIdx.x; i < gn * D; i += 256) {
                const float val = combine_one(part_ml, part_o, base, NS, G, D, g0 + i / D, i % D);
                if constexpr (ROT) {
                    stage[i] = val;
                } else {
                    orow[(int64_t)g0 * D + i] = from_f32<IN>(val);
                }
            }
            __syncthreads();
        }
        if constexpr (ROT) {
            store_rotated<D, IN, 256>(orow + (int64_t)g0 * D, stage, gn, vec);
            __syncthreads();
        }
    }
}

// Launch of one decode configuration. Defined (and instantiated) only in kush_decode_inst.hip, compiled
// once per (input dtype, rot) pair, so the ~200 kernel instantiations build in parallel objects; the
// entry points in kush_decode.hip only call it.
template <int D, int BITS, typename IN, int NW, bool ROT>
int launch_decode(dim3 grid, hipStream_t stream, const void* q, void* out, const void* cache, int64_t bs,
                         int64_t hs, const void* tail_k, const int32_t* tail_idx, const int32_t* block_table,
                         const int32_t* seq_lens, int64_t bt_stride, int bt_cols, int hkv, int group, float p2, float rs,
                         int n_splits, float* part_ml, float* part_o, int32_t* sync, const int32_t* seq_order,
                         const void* app_k, const void* app_v, int64_t app_ks, int64_t app_vs, int ws);

#ifdef KUSH_DECODE_INSTANTIATE
// Page pairs each wave holds in its ring where a third array fits (KUSHKASH_AMD_RING=2 | 3)
inline int ring_depth() {
    const char* env = std::getenv("KUSHKASH_AMD_RING");
    return env != nullptr && env[0] == '3' ? 3 : 2;
}

template <int D, int BITS, typename IN, int NW, bool ROT>
int launch_decode(dim3 grid, hipStream_t stream, const void* q, void* out, const void* cache, int64_t bs,
                         int64_t hs, const void* tail_k, const int32_t* tail_idx, const int32_t* block_table,
                         const int32_t* seq_lens, int64_t bt_stride, int bt_cols, int hkv, int group, float p2, float rs,
                         int n_splits, float* part_ml, float* part_o, int32_t* sync, const int32_t* seq_order,
                         const void* app_k, const void* app_v, int64_t app_ks, int64_t app_vs, int ws) {
    // two page streams whenever the heads of a kv head fit in half the MFMA columns; wave splits are
    // built for 4 waves only (the policy's choice for the split counts that take them)
    auto kern = group <= 8 ? decode_kernel<D, BITS, IN, NW, 2, ROT, false, 2> : decode_kernel<D, BITS, IN, NW, 1, ROT, false, 2>;
    if constexpr (NW == 4) {
        if (ws) kern = group <= 8 ? decode_kernel<D, BITS, IN, NW, 2, ROT, true, 2> : decode_kernel<D, BITS, IN, NW, 1, ROT, true, 2>;
    }
    if constexpr (NW == 4 && !ROT && decode_fits3<D, BITS, NW>()) {
        if (!ws && ring_depth() == 3)
            kern = group <= 8 ? decode_kernel<D, BITS, IN, NW, 2, ROT, false, 3> : decode_kernel<D, BITS, IN, NW, 1, ROT, false, 3>;
    }
    kern<<<grid, dim3(NW * WAVE), 0, stream>>>(
        (const IN*)q, (IN*)out, (uint8_t*)cache, bs, hs, (IN*)tail_k, tail_idx, block_table, seq_lens, bt_stride,
        bt_cols, hkv, group, p2, rs, n_splits, part_ml, part_o, sync, seq_order, (const IN*)app_k, (const IN*)app_v,
        app_ks, app_vs, ws > 0 ? ws : 1);
    return kush_check_launch("kush_decode");
}
#endif

}  // namespace kush
