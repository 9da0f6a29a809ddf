/*
 * kush_oracle.c — TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * A plain-C restatement of the reference's CPU path for the compressed-KV hot path
 * (kushkash v0.6.0, kushkash/kush/cpu.mojo + kushkash/kush/quant.mojo), used only as the
 * checker in tests/, in __graft_entry__.smoke() and as the timed CPU baseline in bench.py.
 * Nothing in the kushkash_amd package loads or calls it.
 *
 * Exported entry points keep the C ABI of the reference's CPU library (cpu.mojo:476-562):
 * every argument is an int64 (addresses, strides, counts) except the softmax scale (float);
 * each returns 0, or -1 for an unsupported head_dim / bits.
 *
 *   kush_cpu_append  <- cpu.mojo:476-494  (_append      cpu.mojo:248-270)
 *   kush_cpu_write   <- cpu.mojo:497-514  (_write       cpu.mojo:273-304)
 *   kush_cpu_decode  <- cpu.mojo:517-531  (_decode      cpu.mojo:454-466, _decode_task :320-451)
 *   kush_cpu_fwht    <- cpu.mojo:534-542  (_fwht_rows   cpu.mojo:83-107)
 *   kush_cpu_unpack  <- cpu.mojo:545-562  (_unpack      cpu.mojo:122-169)
 *
 * Arithmetic is fp32 with IEEE-correct division, no FMA contraction (build with
 * -ffp-contract=off), round-half-to-even for codes (the reference's own test restatement,
 * tests/test_cpu.py:16-24, uses torch.round), RNE fp32->fp16 for scales and biases.
 *
 * Parity status (what pins each function):
 *   quantization (qparams/qcode/pack4, record layout): by-construction known answers
 *     (tests/golden/known_answers.npz via tests/test_known_answers.py: exact dyadic scales and
 *     codes, constant groups, the clamp at a subnormal fp16 scale), the reference test's own
 *     restatement ref_quantize/split_record (test_cpu.py:16-37; tests/test_oracle.py) and a
 *     brute-force nearest-level search with clamp.
 *     Exact round ties: pinned only to torch.round (half-to-even), the reference test's oracle;
 *     Mojo's own tie rule is not visible in the reference: parity unpinned for ties.
 *   append / write: the ragged vLLM simulation (test_ragged.py semantics), bulk-vs-append
 *     equality (test_cpu.py:40-76) and padding rows (tests/test_known_answers.py).
 *   decode: softmax attention over the dequantized cache (test_cpu.py:79-96) and float64 attention
 *     over exactly dequantizable records; exp only through those tolerances.
 *   fwht: bit-exact against the canonical torch order (_ops.py:383-395), close to the dense
 *     Hadamard product (tests/test_host.py).
 *   unpack: the reference test's fp64 restatement (test_cpu.py:458-477 over _ops.py:398-436:
 *     dequantize in fp64, round once, then the canonical rotation), records built from chosen
 *     codes and dyadic scales with closed-form values, and rot = plain unpack then the rotation
 *     of every history row (tests/test_unpack.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PAGE 32

typedef int64_t i64;

/* ------------------------------------------------------------------ fp16 helpers */
/* fp32 -> fp16 bits, round to nearest even (what a hardware cvt does). */
static uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                      /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* rounds to >= 65520: inf */
    if (ax < 0x38800000u) {                       /* result is subnormal (or zero) in fp16 */
        if (ax < 0x33000000u) return (uint16_t)sign;            /* < 2^-25: rounds to 0 */
        uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
        int e = (int)(ax >> 23);                  /* biased fp32 exponent, 102..112 */
        int shift = 126 - e;                      /* value = mant * 2^(e-150); fp16 sub unit 2^-24 */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u;               /* rebias 127 -> 15 */
    uint32_t m = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;   /* carry into the exponent is fine */
    return (uint16_t)(sign | h);
}

static float f16_bits_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {                                  /* subnormal: m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-08f;
            memcpy(&x, &v, 4);
            x |= sign;
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

static float round_f16(float f) { return f16_bits_to_f32(f32_to_f16_bits(f)); }

/* ------------------------------------------------------------------ format (quant.mojo) */
static inline int row_bytes(int D, int bits) { return bits == 8 ? D : D / 2; }          /* quant.mojo:19-22 */
static inline int off_vq(int D, int bits) { return PAGE * row_bytes(D, bits); }          /* quant.mojo:66-68 */
static inline int off_ks(int D, int bits) { return 2 * PAGE * row_bytes(D, bits); }      /* quant.mojo:71-73 */
static inline int off_kb(int D, int bits) { return off_ks(D, bits) + 2 * D; }            /* quant.mojo:76-78 */
static inline int off_vs(int D, int bits) { return off_ks(D, bits) + 4 * D; }            /* quant.mojo:81-83 */
static inline int off_vb(int D, int bits) { return off_ks(D, bits) + 4 * D + 2 * PAGE; } /* quant.mojo:86-87 */

/* (scale, bias, 1/scale) for a group with range [mn, mx]; scale and bias fp16-rounded (quant.mojo:25-35). */
static void qparams(int bits, float mn, float mx, float *s, float *b, float *inv) {
    const float levels = (float)((1 << bits) - 1);
    const float half = (float)(1 << (bits - 1));
    float sc = round_f16((mx - mn) / levels);
    float hs = sc * half;                         /* exact: power-of-two multiply */
    *s = sc;
    *b = round_f16(mn + hs);
    *inv = sc > 0.0f ? 1.0f / sc : 0.0f;
}

/* Signed code of x: clamp(round_half_even((x - b) * inv), -HALF, HALF - 1) (quant.mojo:38-44). */
static inline int8_t qcode(int bits, float x, float b, float inv) {
    const float half = (float)(1 << (bits - 1));
    float r = rintf((x - b) * inv);               /* default rounding mode: nearest-even */
    if (r < -half) r = -half;
    if (r > half - 1.0f) r = half - 1.0f;
    return (int8_t)(int)r;
}

/* lo in bits 0-3, hi in bits 4-7 (quant.mojo:47-50). */
static inline uint8_t pack4(int8_t lo, int8_t hi) { return (uint8_t)(((uint8_t)lo & 0x0Fu) | ((uint8_t)hi << 4)); }

/* Code of dim c in one page row as a float (cpu.mojo:112-119): int4 dim c < D/2 is the low nibble
 * of byte c, dim c >= D/2 the high nibble of byte c - D/2, both two's complement. */
static inline float code_at(const int8_t *row, int D, int bits, int c) {
    if (bits == 8) return (float)row[c];
    int8_t byte = row[c % (D / 2)];
    int v = c < D / 2 ? (int8_t)(byte << 4) >> 4 : byte >> 4;
    return (float)v;
}

/* ------------------------------------------------------------------ cache addressing */
typedef struct {
    int8_t *cache;
    i64 bs, hs;            /* block / head stride in bytes */
    float *tail_k;         /* [slots][hkv][PAGE][D] fp32 */
    const int32_t *tail_idx;
    const int32_t *block_table;
    i64 max_pages;         /* block_table row stride, elements */
    int hkv;
} Cache;

static inline int8_t *rec_of(const Cache *cc, int s, int lp, int h) {   /* cpu.mojo:62-66 */
    i64 blk = cc->block_table[(i64)s * cc->max_pages + lp];
    return cc->cache + blk * cc->bs + (i64)h * cc->hs;
}

static inline i64 tail_of(const Cache *cc, int s, int h, int D) {       /* cpu.mojo:68-71, in elements */
    return (((i64)cc->tail_idx[s] * cc->hkv + h) * PAGE) * D;
}

/* ------------------------------------------------------------------ write path */
/* K of one page: per-channel range over its 32 rows; rows t < split from ka + t*sa, the others from
 * kb_src + (t - split)*skb (cpu.mojo:173-218). */
static void quantize_k_page(int D, int bits, const float *ka, i64 sa, const float *kb_src, i64 skb, int split,
                            int8_t *rec) {
    const int DC = row_bytes(D, bits);
    uint16_t *ksp = (uint16_t *)(rec + off_ks(D, bits));
    uint16_t *kbp = (uint16_t *)(rec + off_kb(D, bits));
    float kbias[256], kinv[256];
    for (int d = 0; d < D; d++) {
        float mn = INFINITY, mx = -INFINITY;
        for (int t = 0; t < PAGE; t++) {
            const float *row = t < split ? ka + t * sa : kb_src + (t - split) * skb;
            float x = row[d];
            mn = x < mn ? x : mn;
            mx = x > mx ? x : mx;
        }
        float s, b, inv;
        qparams(bits, mn, mx, &s, &b, &inv);
        ksp[d] = f32_to_f16_bits(s);
        kbp[d] = f32_to_f16_bits(b);
        kbias[d] = b;
        kinv[d] = inv;
    }
    for (int t = 0; t < PAGE; t++) {
        const float *row = t < split ? ka + t * sa : kb_src + (t - split) * skb;
        int8_t *dst = rec + t * DC;
        if (bits == 8) {
            for (int j = 0; j < D; j++) dst[j] = qcode(8, row[j], kbias[j], kinv[j]);
        } else {
            for (int j = 0; j < D / 2; j++)
                dst[j] = (int8_t)pack4(qcode(4, row[j], kbias[j], kinv[j]),
                                       qcode(4, row[j + D / 2], kbias[j + D / 2], kinv[j + D / 2]));
        }
    }
}

/* V token row -> row t of a record, per-token range over the D channels (cpu.mojo:221-245). */
static void quantize_v_row(int D, int bits, const float *row, int8_t *rec, int t) {
    const int DC = row_bytes(D, bits);
    float mn = INFINITY, mx = -INFINITY;
    for (int j = 0; j < D; j++) {
        mn = row[j] < mn ? row[j] : mn;
        mx = row[j] > mx ? row[j] : mx;
    }
    float s, b, inv;
    qparams(bits, mn, mx, &s, &b, &inv);
    ((uint16_t *)(rec + off_vs(D, bits)))[t] = f32_to_f16_bits(s);
    ((uint16_t *)(rec + off_vb(D, bits)))[t] = f32_to_f16_bits(b);
    int8_t *dst = rec + off_vq(D, bits) + t * DC;
    if (bits == 8) {
        for (int j = 0; j < D; j++) dst[j] = qcode(8, row[j], b, inv);
    } else {
        for (int j = 0; j < D / 2; j++) dst[j] = (int8_t)pack4(qcode(4, row[j], b, inv), qcode(4, row[j + D / 2], b, inv));
    }
}

/* One token per sequence at position seq_lens[s] + pos_offset (cpu.mojo:248-270). */
static void do_append(int D, int bits, const float *k_new, const float *v_new, i64 ks, i64 vs, int32_t *seq_lens,
                      int pos_offset, int advance, const Cache *cc, int S) {
    for (int s = 0; s < S; s++) {
        int pos = seq_lens[s] + pos_offset;
        if (pos < 0) continue;
        int slot = pos % PAGE;
        for (int h = 0; h < cc->hkv; h++) {
            float *dst = cc->tail_k + tail_of(cc, s, h, D) + (i64)slot * D;
            memcpy(dst, k_new + s * ks + (i64)h * D, sizeof(float) * D);
            quantize_v_row(D, bits, v_new + s * vs + (i64)h * D, rec_of(cc, s, pos / PAGE, h), slot);
            if (slot == PAGE - 1) {
                const float *tk = cc->tail_k + tail_of(cc, s, h, D);
                quantize_k_page(D, bits, tk, D, tk, D, PAGE, rec_of(cc, s, pos / PAGE, h));
            }
        }
        if (advance) seq_lens[s] = pos + 1;
    }
}

/* Ragged write, one call per mode (cpu.mojo:273-304). */
static void do_write(int D, int bits, const float *k_new, const float *v_new, i64 ks, i64 vs, const int32_t *qsl,
                     const int32_t *seq_lens, const int32_t *job_seq, const int32_t *job_page, i64 n_jobs, int mode,
                     const Cache *cc) {
    for (i64 j = 0; j < n_jobs; j++) {
        int s = job_seq[j];
        int ps = job_page[j] * PAGE;
        int q0 = qsl[s];
        int total = seq_lens[s];
        int ctx = total - (qsl[s + 1] - q0);
        int complete = ps + PAGE <= total;
        if (mode != 0 && complete) continue;
        for (int h = 0; h < cc->hkv; h++) {
            i64 tb = tail_of(cc, s, h, D);
            int lo = ps > ctx ? ps : ctx;
            if (mode == 0) {
                int8_t *rec = rec_of(cc, s, ps / PAGE, h);
                int hi = ps + PAGE < total ? ps + PAGE : total;
                for (int t = lo; t < hi; t++)
                    quantize_v_row(D, bits, v_new + (i64)(q0 + t - ctx) * vs + (i64)h * D, rec, t - ps);
                if (complete) {
                    int split = ctx - ps;
                    split = split < 0 ? 0 : (split > PAGE ? PAGE : split);
                    quantize_k_page(D, bits, cc->tail_k + tb, D, k_new + (i64)(q0 + ps + split - ctx) * ks + (i64)h * D,
                                    ks, split, rec);
                }
            } else {
                for (int t = lo; t < total; t++)
                    memcpy(cc->tail_k + tb + (i64)(t - ps) * D, k_new + (i64)(q0 + t - ctx) * ks + (i64)h * D,
                           sizeof(float) * D);
            }
        }
    }
}

/* ------------------------------------------------------------------ decode */
/* Page-granular online softmax over cnt scores (cpu.mojo:352-368); returns the correction factor. */
static float softmax_page(float *row, int cnt, float *m, float *l) {
    float pm = -INFINITY;
    for (int t = 0; t < cnt; t++) pm = row[t] > pm ? row[t] : pm;
    float mo = *m;
    float mn = mo > pm ? mo : pm;
    float corr = expf(mo - mn);
    float tot = 0.0f;
    for (int t = 0; t < cnt; t++) {
        float e = expf(row[t] - mn);
        row[t] = e;
        tot += e;
    }
    *m = mn;
    *l = *l * corr + tot;
    return corr;
}

/* Dot product with W = 8 lane partial sums reduced at the end, the shape of the reference's
 * SIMD accumulators (cpu.mojo:397-400); D is a multiple of 8. */
static inline float dot_w(const float *a, const float *b, int D) {
    float part[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int d = 0; d < D; d += 8)
        for (int w = 0; w < 8; w++) part[w] += a[d + w] * b[d + w];
    return ((part[0] + part[1]) + (part[2] + part[3])) + ((part[4] + part[5]) + (part[6] + part[7]));
}

/* Attention of the G q heads of (sequence s, kv head h) over its whole cache (cpu.mojo:320-451):
 * per full page the K scale folds into q, the K bias into one scalar per head, the V scale into the
 * weights and the V bias into one scalar per head; the partial last page takes its K from the exact
 * tail and its V rows from the record. */
static void decode_task(int D, int bits, const float *q, float *o, const Cache *cc, const int32_t *seq_lens, int G,
                        float sm, int s, int h) {
    const int DC = row_bytes(D, bits);
    const int H = cc->hkv;
    const int n = seq_lens[s];
    const i64 qb = ((i64)s * H + h) * G * D;
    float *scr = (float *)malloc(sizeof(float) * ((size_t)G * D * 3 + D + (size_t)G * (PAGE + 4)));
    float *qsm = scr, *qs = scr + G * D, *acc = scr + 2 * G * D, *crow = scr + 3 * G * D;
    float *sc = crow + D, *m = sc + G * PAGE, *l = m + G, *vbacc = l + G, *kbs = vbacc + G;
    float kscale[256], kbiasv[256];
    for (int g = 0; g < G; g++) {
        for (int d = 0; d < D; d++) {
            qsm[g * D + d] = q[qb + g * D + d] * sm;
            acc[g * D + d] = 0.0f;
        }
        m[g] = -INFINITY;
        l[g] = 0.0f;
        vbacc[g] = 0.0f;
    }
    for (int lp = 0; lp < n / PAGE; lp++) {
        const int8_t *kc = rec_of(cc, s, lp, h);
        const int8_t *vc = kc + off_vq(D, bits);
        const uint16_t *ksp = (const uint16_t *)(kc + off_ks(D, bits));
        const uint16_t *kbp = (const uint16_t *)(kc + off_kb(D, bits));
        const uint16_t *vsp = (const uint16_t *)(kc + off_vs(D, bits));
        const uint16_t *vbp = (const uint16_t *)(kc + off_vb(D, bits));
        for (int d = 0; d < D; d++) {
            kscale[d] = f16_bits_to_f32(ksp[d]);
            kbiasv[d] = f16_bits_to_f32(kbp[d]);
        }
        for (int g = 0; g < G; g++) {
            for (int d = 0; d < D; d++) qs[g * D + d] = qsm[g * D + d] * kscale[d];
            kbs[g] = dot_w(qsm + g * D, kbiasv, D);
        }
        for (int t = 0; t < PAGE; t++) {
            for (int d = 0; d < D; d++) crow[d] = code_at(kc + t * DC, D, bits, d);
            for (int g = 0; g < G; g++) sc[g * PAGE + t] = dot_w(qs + g * D, crow, D) + kbs[g];
        }
        for (int g = 0; g < G; g++) {
            float corr = softmax_page(sc + g * PAGE, PAGE, m + g, l + g);
            vbacc[g] *= corr;
            for (int d = 0; d < D; d++) acc[g * D + d] *= corr;
        }
        for (int t = 0; t < PAGE; t++) {
            for (int d = 0; d < D; d++) crow[d] = code_at(vc + t * DC, D, bits, d);
            float vst = f16_bits_to_f32(vsp[t]), vbt = f16_bits_to_f32(vbp[t]);
            for (int g = 0; g < G; g++) {
                float e = sc[g * PAGE + t];
                vbacc[g] += e * vbt;
                float wv = e * vst;
                for (int d = 0; d < D; d++) acc[g * D + d] += wv * crow[d];
            }
        }
    }
    int tail_n = n % PAGE;
    if (tail_n > 0) {
        const float *tk = cc->tail_k + tail_of(cc, s, h, D);
        const int8_t *vrec = rec_of(cc, s, n / PAGE, h);
        const int8_t *vc = vrec + off_vq(D, bits);
        const uint16_t *vsp = (const uint16_t *)(vrec + off_vs(D, bits));
        const uint16_t *vbp = (const uint16_t *)(vrec + off_vb(D, bits));
        for (int g = 0; g < G; g++) {
            for (int t = 0; t < tail_n; t++) sc[g * PAGE + t] = dot_w(qsm + g * D, tk + t * D, D);
            float corr = softmax_page(sc + g * PAGE, tail_n, m + g, l + g);
            vbacc[g] *= corr;
            for (int d = 0; d < D; d++) acc[g * D + d] *= corr;
        }
        for (int t = 0; t < tail_n; t++) {
            for (int d = 0; d < D; d++) crow[d] = code_at(vc + t * DC, D, bits, d);
            float vst = f16_bits_to_f32(vsp[t]), vbt = f16_bits_to_f32(vbp[t]);
            for (int g = 0; g < G; g++) {
                float e = sc[g * PAGE + t];
                vbacc[g] += e * vbt;
                float wv = e * vst;
                for (int d = 0; d < D; d++) acc[g * D + d] += wv * crow[d];
            }
        }
    }
    for (int g = 0; g < G; g++) {
        float inv_l = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
        for (int d = 0; d < D; d++) o[qb + g * D + d] = (acc[g * D + d] + vbacc[g]) * inv_l;
    }
    free(scr);
}

static int g_threads = 0;   /* 0: all available */

/* One task per (sequence, kv head); inline below 256 page-tasks (cpu.mojo:454-466). */
static void do_decode(int D, int bits, const float *q, float *o, const Cache *cc, const int32_t *seq_lens, int G,
                      float sm, int S) {
    const int tasks = S * cc->hkv;
    i64 pages = 0;
    for (int s = 0; s < S; s++) pages += seq_lens[s] / PAGE + 1;
    if (pages * cc->hkv < 256 || g_threads == 1) {
        for (int i = 0; i < tasks; i++) decode_task(D, bits, q, o, cc, seq_lens, G, sm, i / cc->hkv, i % cc->hkv);
        return;
    }
#ifdef _OPENMP
    int nt = g_threads > 0 ? g_threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int i = 0; i < tasks; i++) decode_task(D, bits, q, o, cc, seq_lens, G, sm, i / cc->hkv, i % cc->hkv);
}

/* ------------------------------------------------------------------ rotation */
static float fwht_scale(int D) {      /* quant.mojo:101-110: 1/sqrt(D) as exact fp32 bits */
    uint32_t bits = D == 64 ? 0x3E000000u : D == 128 ? 0x3DB504F3u : 0x3D800000u;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Canonical Walsh-Hadamard order: butterflies over strides 1, 2, ..., D/2, then one separate
 * multiply (quant.mojo:90-99, cpu.mojo:83-107). */
static void fwht_rows(int D, float *x, i64 rows) {
    const float sc = fwht_scale(D);
    for (i64 r = 0; r < rows; r++) {
        float *p = x + r * D;
        for (int h = 1; h < D; h <<= 1)
            for (int i = 0; i < D; i++)
                if ((i & h) == 0) {
                    float a = p[i], b = p[i + h];
                    p[i] = a + b;
                    p[i + h] = a - b;
                }
        for (int j = 0; j < D; j++) {
            volatile float y = p[j] * sc;   /* one rounding, never fused */
            p[j] = y;
        }
    }
}

/* ------------------------------------------------------------------ unpack */
/* Packed prefill rows from history pages, partial pages and the new chunk (cpu.mojo:122-169). */
static void do_unpack(int D, int bits, const int8_t *cache, i64 bs, i64 hs, int H, const int32_t *page_blk,
                      const int32_t *page_dst, i64 n_pages, const int32_t *tail_blk, const int32_t *tail_info, i64 n_tail,
                      const float *tail_k, const float *k_new, const float *v_new, i64 ks_new, i64 vs_new,
                      const int32_t *new_dst, i64 n_new, float *kp, float *vp, int rot) {
    const int DC = row_bytes(D, bits);
    const i64 rs = (i64)H * D;
    float kx[256], vx[256];
    for (i64 b = 0; b < n_pages + n_tail; b++) {
        int page = b < n_pages;
        i64 i = b - n_pages;
        i64 blk = page ? page_blk[b] : tail_blk[i];
        i64 dst0 = page ? page_dst[b] : tail_info[3 * i];
        int n = page ? PAGE : tail_info[3 * i + 1];
        for (int h = 0; h < H; h++) {
            const int8_t *rec = cache + blk * bs + (i64)h * hs;
            const uint16_t *ksp = (const uint16_t *)(rec + off_ks(D, bits));
            const uint16_t *kbp = (const uint16_t *)(rec + off_kb(D, bits));
            const uint16_t *vsp = (const uint16_t *)(rec + off_vs(D, bits));
            const uint16_t *vbp = (const uint16_t *)(rec + off_vb(D, bits));
            i64 tk = page ? 0 : (((i64)tail_info[3 * i + 2] * H + h) * PAGE) * D;
            for (int t = 0; t < n; t++) {
                float vs = f16_bits_to_f32(vsp[t]), vb = f16_bits_to_f32(vbp[t]);
                for (int c = 0; c < D; c++) {
                    kx[c] = page ? fmaf(code_at(rec + t * DC, D, bits, c), f16_bits_to_f32(ksp[c]), f16_bits_to_f32(kbp[c]))
                                 : tail_k[tk + (i64)t * D + c];
                    vx[c] = fmaf(code_at(rec + off_vq(D, bits) + t * DC, D, bits, c), vs, vb);
                }
                if (rot) {
                    fwht_rows(D, kx, 1);
                    fwht_rows(D, vx, 1);
                }
                i64 o = (dst0 + t) * rs + (i64)h * D;
                memcpy(kp + o, kx, sizeof(float) * D);
                memcpy(vp + o, vx, sizeof(float) * D);
            }
        }
    }
    for (i64 j = 0; j < n_new; j++) {
        i64 o = (i64)new_dst[j] * rs;
        for (int h = 0; h < H; h++) {
            memcpy(kp + o + (i64)h * D, k_new + j * ks_new + (i64)h * D, sizeof(float) * D);
            memcpy(vp + o + (i64)h * D, v_new + j * vs_new + (i64)h * D, sizeof(float) * D);
        }
    }
}

/* ------------------------------------------------------------------ C ABI (cpu.mojo:476-562) */
#define P_(T, a) ((T)(intptr_t)(a))
static int ok_shape(i64 d, i64 bits) { return (d == 64 || d == 128 || d == 256) && (bits == 4 || bits == 8); }

static Cache make_cache(i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx, i64 block_table, i64 max_pages, i64 hkv) {
    Cache c = {P_(int8_t *, cache), bs, hs, P_(float *, tail_k), P_(const int32_t *, tail_idx),
               P_(const int32_t *, block_table), max_pages, (int)hkv};
    return c;
}

int kush_cpu_append(i64 d, i64 bits, i64 k_new, i64 v_new, i64 k_stride, i64 v_stride, i64 seq_lens, i64 pos_offset,
                    i64 advance, i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx, i64 block_table, i64 max_pages,
                    i64 hkv, i64 n_seqs) {
    if (!ok_shape(d, bits)) return -1;
    Cache cc = make_cache(cache, bs, hs, tail_k, tail_idx, block_table, max_pages, hkv);
    do_append((int)d, (int)bits, P_(const float *, k_new), P_(const float *, v_new), k_stride, v_stride,
              P_(int32_t *, seq_lens), (int)pos_offset, advance != 0, &cc, (int)n_seqs);
    return 0;
}

int kush_cpu_write(i64 d, i64 bits, i64 k_new, i64 v_new, i64 k_stride, i64 v_stride, i64 qsl, i64 seq_lens,
                   i64 job_seq, i64 job_page, i64 n_jobs, i64 mode, i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx,
                   i64 block_table, i64 max_pages, i64 hkv) {
    if (!ok_shape(d, bits)) return -1;
    Cache cc = make_cache(cache, bs, hs, tail_k, tail_idx, block_table, max_pages, hkv);
    do_write((int)d, (int)bits, P_(const float *, k_new), P_(const float *, v_new), k_stride, v_stride,
             P_(const int32_t *, qsl), P_(const int32_t *, seq_lens), P_(const int32_t *, job_seq),
             P_(const int32_t *, job_page), n_jobs, (int)mode, &cc);
    return 0;
}

int kush_cpu_decode(i64 d, i64 bits, i64 q, i64 o, i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx,
                    i64 block_table, i64 seq_lens, i64 max_pages, i64 hkv, i64 group, float sm, i64 n_seqs) {
    if (!ok_shape(d, bits)) return -1;
    Cache cc = make_cache(cache, bs, hs, tail_k, tail_idx, block_table, max_pages, hkv);
    do_decode((int)d, (int)bits, P_(const float *, q), P_(float *, o), &cc, P_(const int32_t *, seq_lens), (int)group,
              sm, (int)n_seqs);
    return 0;
}

int kush_cpu_fwht(i64 d, i64 x, i64 rows) {
    if (!(d == 64 || d == 128 || d == 256)) return -1;
    fwht_rows((int)d, P_(float *, x), rows);
    return 0;
}

int kush_cpu_unpack(i64 d, i64 bits, i64 cache, i64 bs, i64 hs, i64 hkv, i64 page_blk, i64 page_dst, i64 n_pages,
                    i64 tail_blk, i64 tail_info, i64 n_tail, i64 tail_k, i64 k_new, i64 v_new, i64 k_stride,
                    i64 v_stride, i64 new_dst, i64 n_new, i64 kp, i64 vp, i64 rot) {
    if (!ok_shape(d, bits)) return -1;
    do_unpack((int)d, (int)bits, P_(const int8_t *, cache), bs, hs, (int)hkv, P_(const int32_t *, page_blk),
              P_(const int32_t *, page_dst), n_pages, P_(const int32_t *, tail_blk), P_(const int32_t *, tail_info),
              n_tail, P_(const float *, tail_k), P_(const float *, k_new), P_(const float *, v_new), k_stride, v_stride,
              P_(const int32_t *, new_dst), n_new, P_(float *, kp), P_(float *, vp), rot != 0);
    return 0;
}

/* Thread count for kush_cpu_decode (0 = all available); not part of the reference ABI. */
int kush_oracle_set_threads(i64 n) {
    g_threads = (int)n;
    return 0;
}

int kush_oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
