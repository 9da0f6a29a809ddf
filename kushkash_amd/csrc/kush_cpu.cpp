// The package's CPU path: the compressed-KV hot path on the host, behind Ops and KushCache on device
// "cpu" -- the reference's CPU library (kushkash/kush/cpu.mojo, bound by kushkash/_cpu.py:10-40 and
// dispatched by kushkash/_ops.py:49-57). The entry points keep that library's C ABI: every argument
// an int64 (address, stride or count) except the decode's softmax scale (float); each returns 0, or
// -1 for an unsupported head_dim / bits. Tensors are fp32; records follow the page-record format of
// the GPU kernels (kush_common.h):
//   [ kq: 32 DC | vq: 32 DC | ks: D fp16 | kb: D fp16 | vs: 32 fp16 | vb: 32 fp16 ]
// and are byte-identical to theirs: the quantization arithmetic of kushkash/kush/quant.mojo:25-50 in
// IEEE fp32 (correctly rounded division, no fused multiply-add: this file is built with
// -ffp-contract=off), codes rounded half to even, scales and biases rounded to fp16 to nearest even.
//
// Host work split: OpenMP over (page, kv head) tasks for the writes, over (sequence, kv head) for the
// decode and over pages for the unpack. The decode dequantizes each page's codes once per kv head and
// scores it for every q head of the group with the K scales folded into q (score = sum_d q_d ks_d
// c_td + sum_d q_d kb_d) and the V scales into the softmax weights (o_d += sum_t (p_t vs_t) c_td,
// plus sum_t p_t vb_t once per head), with a page-granular online softmax in fp32.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <type_traits>
#include <vector>

#include "kushkash_amd_cpu.h"

namespace {

using i64 = int64_t;
constexpr int PAGE = 32;

// fp32 -> fp16 bit pattern, rounded to nearest even; overflow to infinity, NaN stays a quiet NaN
inline uint16_t half_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u);
    if (ax >= 0x477FF000u) return sign | 0x7C00u;                 // >= 65520: past the largest half
    if (ax < 0x38800000u) {                                       // below 2^-14: a subnormal half or zero
        float a;
        std::memcpy(&a, &ax, 4);
        return sign | (uint16_t)std::nearbyint(a * 16777216.0f);   // units of 2^-24 (exact scaling)
    }
    const uint32_t r = ax + 0xFFFu + ((ax >> 13) & 1u);            // round the 13 dropped bits to even
    return sign | (uint16_t)((r >> 13) - (112u << 10));            // rebias the exponent (127 -> 15)
}

inline float half_value(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-8f;         // m 2^-24, exact
        return sign ? -v : v;
    }
    const uint32_t x = sign | (e == 31 ? (0xFFu << 23) | (m << 13) : ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

inline void put_half(uint8_t* p, float f) {
    const uint16_t h = half_bits(f);
    std::memcpy(p, &h, 2);
}

inline float get_half(const uint8_t* p) {
    uint16_t h;
    std::memcpy(&h, p, 2);
    return half_value(h);
}

template <int D, int BITS>
struct Rec {
    static constexpr int DC = BITS == 8 ? D : D / 2;
    static constexpr i64 VQ = (i64)PAGE * DC, KS = 2 * (i64)PAGE * DC, KB = KS + 2 * D, VS = KS + 4 * D,
                         VB = VS + 2 * PAGE;
    static constexpr float LEVELS = float((1 << BITS) - 1), HALF = float(1 << (BITS - 1));
};

// one quantization group's scale s, bias b and 1 / s from its range (quant.mojo:25-37)
template <int BITS>
inline void group_params(float mn, float mx, float& s, float& b, float& inv) {
    constexpr float LEVELS = float((1 << BITS) - 1), HALF = float(1 << (BITS - 1));
    s = half_value(half_bits((mx - mn) / LEVELS));
    b = half_value(half_bits(mn + s * HALF));
    inv = s > 0.0f ? 1.0f / s : 0.0f;
}

// the code of x: rint((x - b) / s) through the reciprocal, clamped to [-HALF, HALF - 1] (quant.mojo:40-50)
template <int BITS>
inline int code_of(float x, float b, float inv) {
    constexpr float HALF = float(1 << (BITS - 1));
    const float r = std::nearbyint((x - b) * inv);
    return (int)std::fmin(std::fmax(r, -HALF), HALF - 1.0f);
}

// a row's codes into its DC record bytes (int4: byte j = dim j low nibble, dim j + D/2 high nibble)
template <int D, int BITS>
inline void put_codes(uint8_t* dst, const float* x, const float* b, const float* inv, bool per_dim) {
    if constexpr (BITS == 8) {
        for (int j = 0; j < D; ++j) dst[j] = (uint8_t)code_of<8>(x[j], b[per_dim ? j : 0], inv[per_dim ? j : 0]);
    } else {
        for (int j = 0; j < D / 2; ++j) {
            const int k = j + D / 2;
            const int lo = code_of<4>(x[j], b[per_dim ? j : 0], inv[per_dim ? j : 0]);
            const int hi = code_of<4>(x[k], b[per_dim ? k : 0], inv[per_dim ? k : 0]);
            dst[j] = (uint8_t)((lo & 15) | ((hi & 15) << 4));
        }
    }
}

// a V token row into row t of a record: its own range over the D channels (quant.mojo, cpu.mojo:221-245)
template <int D, int BITS>
void put_v_row(const float* x, uint8_t* rec, int t) {
    using R = Rec<D, BITS>;
    float mn = x[0], mx = x[0];
    for (int j = 1; j < D; ++j) {
        mn = std::fmin(mn, x[j]);
        mx = std::fmax(mx, x[j]);
    }
    float s, b, inv;
    group_params<BITS>(mn, mx, s, b, inv);
    put_half(rec + R::VS + 2 * t, s);
    put_half(rec + R::VB + 2 * t, b);
    put_codes<D, BITS>(rec + R::VQ + (i64)t * R::DC, x, &b, &inv, false);
}

// a K page into a record: per-channel ranges over its 32 rows, row t at row(t) (cpu.mojo:173-218)
template <int D, int BITS, typename Row>
void put_k_page(Row row, uint8_t* rec) {
    using R = Rec<D, BITS>;
    float mn[D], mx[D], b[D], inv[D];
    std::memcpy(mn, row(0), sizeof(mn));
    std::memcpy(mx, row(0), sizeof(mx));
    for (int t = 1; t < PAGE; ++t) {
        const float* x = row(t);
        for (int d = 0; d < D; ++d) {
            mn[d] = std::fmin(mn[d], x[d]);
            mx[d] = std::fmax(mx[d], x[d]);
        }
    }
    for (int d = 0; d < D; ++d) {
        float s;
        group_params<BITS>(mn[d], mx[d], s, b[d], inv[d]);
        put_half(rec + R::KS + 2 * d, s);
        put_half(rec + R::KB + 2 * d, b[d]);
    }
    for (int t = 0; t < PAGE; ++t) put_codes<D, BITS>(rec + (i64)t * R::DC, row(t), b, inv, true);
}

// the codes of rows [0, n) of a K (v = false) or V (v = true) page as floats [n][D]
template <int D, int BITS>
void read_codes(const uint8_t* rec, bool v, int n, float* out) {
    using R = Rec<D, BITS>;
    const int8_t* c = reinterpret_cast<const int8_t*>(rec + (v ? R::VQ : 0));
    for (int t = 0; t < n; ++t, c += R::DC, out += D) {
        if constexpr (BITS == 8) {
            for (int d = 0; d < D; ++d) out[d] = (float)c[d];
        } else {
            for (int j = 0; j < D / 2; ++j) {
                out[j] = (float)(int8_t)(c[j] << 4) / 16.0f;             // low nibble, sign-extended
                out[j + D / 2] = (float)(c[j] >> 4);                      // high nibble (arithmetic shift)
            }
        }
    }
}

// A full page's K codes by dimension: out[d * PAGE + t] (the scores then run over 32 tokens at a time)
template <int D, int BITS>
void read_k_codes_by_dim(const uint8_t* rec, float* out) {
    using R = Rec<D, BITS>;
    const int8_t* c = reinterpret_cast<const int8_t*>(rec);
    for (int t = 0; t < PAGE; ++t, c += R::DC) {
        if constexpr (BITS == 8) {
            for (int d = 0; d < D; ++d) out[d * PAGE + t] = (float)c[d];
        } else {
            for (int j = 0; j < D / 2; ++j) {
                out[j * PAGE + t] = (float)(int8_t)(c[j] << 4) / 16.0f;
                out[(j + D / 2) * PAGE + t] = (float)(c[j] >> 4);
            }
        }
    }
}

struct Cache {
    uint8_t* base;
    i64 bs, hs;
    float* tail_k;
    const int32_t* tail_idx;
    const int32_t* table;
    i64 bt_stride;
    int hkv;
    uint8_t* rec(int s, int page, int h) const {
        return base + (i64)table[(i64)s * bt_stride + page] * bs + (i64)h * hs;
    }
    float* tail(int s, int h, int D) const { return tail_k + ((i64)tail_idx[s] * hkv + h) * PAGE * D; }
};

// ------------------------------------------------------------------ writes
// One token per sequence at position seq_lens[s] + pos_offset (negative: a padding row, skipped): its K
// row to the exact tail, its V row to its record row; the K page is quantized when the token fills it.
// seq_lens advances after every head is written (cpu.mojo:248-270, gpu.mojo:207-238).
template <int D, int BITS>
void append(const float* k, const float* v, i64 ks, i64 vs, int32_t* seq_lens, int pos_offset, bool advance,
            const Cache& c, int S) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int s = 0; s < S; ++s)
        for (int h = 0; h < c.hkv; ++h) {
            const int pos = seq_lens[s] + pos_offset;
            if (pos < 0) continue;
            const int slot = pos % PAGE;
            float* tail = c.tail(s, h, D);
            std::memcpy(tail + (i64)slot * D, k + s * ks + (i64)h * D, sizeof(float) * D);
            uint8_t* rec = c.rec(s, pos / PAGE, h);
            put_v_row<D, BITS>(v + s * vs + (i64)h * D, rec, slot);
            if (slot == PAGE - 1) put_k_page<D, BITS>([&](int t) { return tail + (i64)t * D; }, rec);
        }
    if (advance)
        for (int s = 0; s < S; ++s) {
            const int pos = seq_lens[s] + pos_offset;
            if (pos >= 0) seq_lens[s] = pos + 1;
        }
}

// Ragged chunk write, one mode per call (cpu.mojo:273-304, gpu.mojo:241-276). Job j: logical page
// job_page[j] of sequence job_seq[j], whose new rows [qsl[s], qsl[s+1]) sit at positions [ctx, seq_lens[s]).
// Mode 0: the page's new V rows and, when the page is complete, its K (rows before ctx from the tail);
// mode 1: the new K rows of a page left partial, into the tail.
template <int D, int BITS>
void write(const float* k, const float* v, i64 ks, i64 vs, const int32_t* qsl, const int32_t* seq_lens,
           const int32_t* job_seq, const int32_t* job_page, i64 n_jobs, int mode, const Cache& c) {
#pragma omp parallel for collapse(2) schedule(static)
    for (i64 j = 0; j < n_jobs; ++j)
        for (int h = 0; h < c.hkv; ++h) {
            const int s = job_seq[j], ps = job_page[j] * PAGE;
            const int q0 = qsl[s], total = seq_lens[s], ctx = total - (qsl[s + 1] - q0);
            const bool complete = ps + PAGE <= total;
            const int lo = std::max(ps, ctx);
            const i64 hoff = (i64)h * D;
            float* tail = c.tail(s, h, D);
            if (mode == 0) {
                uint8_t* rec = c.rec(s, ps / PAGE, h);
                const int hi = std::min(ps + PAGE, total);
                for (int t = lo; t < hi; ++t) put_v_row<D, BITS>(v + (i64)(q0 + t - ctx) * vs + hoff, rec, t - ps);
                if (complete) {
                    const int split = std::min(PAGE, std::max(0, ctx - ps));
                    const float* first_new = k + (i64)(q0 + ps + split - ctx) * ks + hoff;
                    put_k_page<D, BITS>(
                        [&](int t) { return t < split ? tail + (i64)t * D : first_new + (i64)(t - split) * ks; }, rec);
                }
            } else if (!complete) {
                for (int t = lo; t < total; ++t)
                    std::memcpy(tail + (i64)(t - ps) * D, k + (i64)(q0 + t - ctx) * ks + hoff, sizeof(float) * D);
            }
        }
}

// ------------------------------------------------------------------ decode
// out[s] = softmax(scale q k^T) v over the seq_lens[s] cached tokens of sequence s, for the G q heads
// of every kv head (q head h G + g reads kv head h): full pages from their records, the partial last
// page's K exact from the tail and its V from its record (cpu.mojo:320-466).
template <int D, int BITS>
void decode(const float* q, float* out, const Cache& c, const int32_t* seq_lens, int G, float scale, int S) {
    using R = Rec<D, BITS>;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int s = 0; s < S; ++s)
        for (int h = 0; h < c.hkv; ++h) {
            const int n = seq_lens[s], full = n / PAGE, tn = n % PAGE;
            const i64 row0 = ((i64)s * c.hkv + h) * G;                    // first q / out row of this kv head
            std::vector<float> codes((size_t)PAGE * D), o((size_t)G * D, 0.0f), p((size_t)G * PAGE);
            std::vector<float> m(G, -INFINITY), l(G, 0.0f), vbs(G, 0.0f);
            float ksv[D], kbv[D], vsv[PAGE], vbv[PAGE];
            const float* tail = c.tail(s, h, D);
            for (int pg = 0; pg < full + (tn > 0 ? 1 : 0); ++pg) {
                const bool part = pg == full;
                const int cnt = part ? tn : PAGE;
                const uint8_t* rec = c.rec(s, pg, h);
                if (!part) {
                    read_k_codes_by_dim<D, BITS>(rec, codes.data());
                    for (int d = 0; d < D; ++d) {
                        ksv[d] = get_half(rec + R::KS + 2 * d);
                        kbv[d] = get_half(rec + R::KB + 2 * d);
                    }
                }
                for (int g = 0; g < G; ++g) {                          // scores, then the softmax update
                    const float* qg = q + (row0 + g) * D;
                    float* pg_ = p.data() + (size_t)g * PAGE;
                    if (!part) {                                       // K scales folded into q
                        float bias = 0.0f, acc[PAGE] = {};
                        for (int d = 0; d < D; ++d) {                  // each token's sum over d in order,
                            const float w = qg[d] * ksv[d];            // 32 tokens side by side
                            const float* col = codes.data() + (size_t)d * PAGE;
                            for (int t = 0; t < PAGE; ++t) acc[t] += w * col[t];
                            bias += qg[d] * kbv[d];
                        }
                        for (int t = 0; t < PAGE; ++t) pg_[t] = (acc[t] + bias) * scale;
                    } else {                                           // exact K rows from the tail
                        for (int t = 0; t < cnt; ++t) {
                            const float* kt = tail + (i64)t * D;
                            float acc = 0.0f;
                            for (int d = 0; d < D; ++d) acc += qg[d] * kt[d];
                            pg_[t] = acc * scale;
                        }
                    }
                    float pm = -INFINITY;
                    for (int t = 0; t < cnt; ++t) pm = std::fmax(pm, pg_[t]);
                    const float mn = std::fmax(m[g], pm);
                    const float corr = m[g] == -INFINITY ? 0.0f : std::exp(m[g] - mn);
                    float tot = 0.0f;
                    for (int t = 0; t < cnt; ++t) {
                        pg_[t] = std::exp(pg_[t] - mn);
                        tot += pg_[t];
                    }
                    m[g] = mn;
                    l[g] = l[g] * corr + tot;
                    vbs[g] *= corr;
                    float* og = o.data() + (size_t)g * D;
                    for (int d = 0; d < D; ++d) og[d] *= corr;
                }
                read_codes<D, BITS>(rec, true, cnt, codes.data());     // V: codes once for every head
                for (int t = 0; t < cnt; ++t) {
                    vsv[t] = get_half(rec + R::VS + 2 * t);
                    vbv[t] = get_half(rec + R::VB + 2 * t);
                }
                for (int g = 0; g < G; ++g) {
                    const float* pg_ = p.data() + (size_t)g * PAGE;
                    float* og = o.data() + (size_t)g * D;
                    float bsum = 0.0f;
                    for (int t = 0; t < cnt; ++t) {
                        const float wt = pg_[t] * vsv[t];
                        const float* ct = codes.data() + (size_t)t * D;
                        for (int d = 0; d < D; ++d) og[d] += wt * ct[d];
                        bsum += pg_[t] * vbv[t];
                    }
                    vbs[g] += bsum;
                }
            }
            for (int g = 0; g < G; ++g) {
                float* dst = out + (row0 + g) * D;
                const float inv = l[g] > 0.0f ? 1.0f / l[g] : 0.0f;
                for (int d = 0; d < D; ++d) dst[d] = (o[(size_t)g * D + d] + vbs[g]) * inv;
            }
        }
}

// ------------------------------------------------------------------ rotation
// fp32 1/sqrt(D), exact bits (quant.mojo:101-110)
template <int D>
constexpr uint32_t rsqrt_bits() { return D == 64 ? 0x3E000000u : (D == 128 ? 0x3DB504F3u : 0x3D800000u); }

// the canonical Walsh-Hadamard rotation of one row in place: butterflies at strides 1, 2, .., D/2 in
// that order (of each pair, the element with the stride bit set becomes partner - self, the other
// self + partner), then one multiply by 1/sqrt(D) (quant.mojo:90-110)
template <int D>
void rotate_row(float* x) {
    for (int hstride = 1; hstride < D; hstride <<= 1)
        for (int i = 0; i < D; ++i)
            if (!(i & hstride)) {
                const float a = x[i], b = x[i + hstride];
                x[i] = a + b;
                x[i + hstride] = a - b;
            }
    uint32_t bits = rsqrt_bits<D>();
    float sc;
    std::memcpy(&sc, &bits, 4);
    for (int i = 0; i < D; ++i) x[i] *= sc;
}

template <int D>
void fwht(float* x, i64 rows) {
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < rows; ++r) rotate_row<D>(x + r * D);
}

// ------------------------------------------------------------------ unpack
// One packed-prefill group's keys / values into kp, vp [rows, Hkv, D] (cpu.mojo:122-169, gpu.mojo:303-375):
// full history pages (block page_blk[i] -> rows page_dst[i] + 0..31), partial pages (block tail_blk[i],
// tail_info[i] = (first row, tokens, tail slot): K exact from tail_k, V from the record), the new rows
// (row j of k_new / v_new -> row new_dst[j]). Dequantization fma(code, scale, bias) in fp32; rot rotates
// every history row back (the rotation is its own inverse); new rows are copied as they are.
template <int D, int BITS>
void unpack(const uint8_t* cache, i64 bs, i64 hs, int H, const int32_t* page_blk, const int32_t* page_dst,
            i64 n_pages, const int32_t* tail_blk, const int32_t* tail_info, i64 n_tail, const float* tail_k,
            const float* k_new, const float* v_new, i64 k_stride, i64 v_stride, const int32_t* new_dst, i64 n_new,
            float* kp, float* vp, bool rot) {
    using R = Rec<D, BITS>;
    const auto rows_of = [&](const uint8_t* rec, int first, int cnt, const float* ktail, int h) {
        float codes[PAGE * D];
        for (int half = 0; half < 2; ++half) {                         // K (unless exact), then V
            const bool v = half == 1;
            float* dst = v ? vp : kp;
            if (!v && ktail != nullptr) {
                for (int t = 0; t < cnt; ++t) {
                    float* row = dst + ((i64)(first + t) * H + h) * D;
                    std::memcpy(row, ktail + (i64)t * D, sizeof(float) * D);
                    if (rot) rotate_row<D>(row);
                }
                continue;
            }
            read_codes<D, BITS>(rec, v, cnt, codes);
            for (int t = 0; t < cnt; ++t) {
                float* row = dst + ((i64)(first + t) * H + h) * D;
                const float* ct = codes + t * D;
                if (v) {
                    const float sc = get_half(rec + R::VS + 2 * t), bi = get_half(rec + R::VB + 2 * t);
                    for (int d = 0; d < D; ++d) row[d] = std::fma(ct[d], sc, bi);
                } else {
                    for (int d = 0; d < D; ++d) row[d] = std::fma(ct[d], get_half(rec + R::KS + 2 * d), get_half(rec + R::KB + 2 * d));
                }
                if (rot) rotate_row<D>(row);
            }
        }
    };
#pragma omp parallel for collapse(2) schedule(static)
    for (i64 i = 0; i < n_pages; ++i)
        for (int h = 0; h < H; ++h) rows_of(cache + (i64)page_blk[i] * bs + (i64)h * hs, page_dst[i], PAGE, nullptr, h);
#pragma omp parallel for collapse(2) schedule(static)
    for (i64 i = 0; i < n_tail; ++i)
        for (int h = 0; h < H; ++h) {
            const int first = tail_info[3 * i], cnt = tail_info[3 * i + 1], slot = tail_info[3 * i + 2];
            rows_of(cache + (i64)tail_blk[i] * bs + (i64)h * hs, first, cnt, tail_k + ((i64)slot * H + h) * PAGE * D, h);
        }
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < n_new; ++j)
        for (int h = 0; h < H; ++h) {
            std::memcpy(kp + ((i64)new_dst[j] * H + h) * D, k_new + j * k_stride + (i64)h * D, sizeof(float) * D);
            std::memcpy(vp + ((i64)new_dst[j] * H + h) * D, v_new + j * v_stride + (i64)h * D, sizeof(float) * D);
        }
}

// the (D, bits) instance of fn, or -1
template <typename Fn>
int by_shape(i64 D, i64 bits, Fn&& fn) {
    if (bits != 4 && bits != 8) return -1;
    const bool b8 = bits == 8;
    switch (D) {
        case 64: return b8 ? fn(std::integral_constant<int, 64>{}, std::integral_constant<int, 8>{})
                           : fn(std::integral_constant<int, 64>{}, std::integral_constant<int, 4>{});
        case 128: return b8 ? fn(std::integral_constant<int, 128>{}, std::integral_constant<int, 8>{})
                            : fn(std::integral_constant<int, 128>{}, std::integral_constant<int, 4>{});
        case 256: return b8 ? fn(std::integral_constant<int, 256>{}, std::integral_constant<int, 8>{})
                            : fn(std::integral_constant<int, 256>{}, std::integral_constant<int, 4>{});
    }
    return -1;
}

template <typename T>
T* ptr(i64 a) { return reinterpret_cast<T*>((uintptr_t)a); }

Cache make_cache(i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx, i64 table, i64 bt_stride, i64 hkv) {
    return Cache{ptr<uint8_t>(cache), bs, hs, ptr<float>(tail_k), ptr<const int32_t>(tail_idx),
                 ptr<const int32_t>(table), bt_stride, (int)hkv};
}

}  // namespace

// ------------------------------------------------------------------ C ABI (kushkash_amd_cpu.h; kushkash/_cpu.py:10-25)
extern "C" {

// d, bits, k, v, k_stride, v_stride, seq_lens, pos_offset, advance, cache, block_stride, head_stride,
// tail_k, tail_idx, block_table, max_pages (the table's row stride), hkv, n_seqs
int kush_cpu_append(i64 d, i64 bits, i64 k, i64 v, i64 k_stride, i64 v_stride, i64 seq_lens, i64 pos_offset,
                    i64 advance, i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx, i64 block_table, i64 max_pages,
                    i64 hkv, i64 n_seqs) {
    const Cache c = make_cache(cache, bs, hs, tail_k, tail_idx, block_table, max_pages, hkv);
    return by_shape(d, bits, [&](auto dd, auto bb) {
        append<decltype(dd)::value, decltype(bb)::value>(ptr<const float>(k), ptr<const float>(v), k_stride, v_stride,
                                                         ptr<int32_t>(seq_lens), (int)pos_offset, advance != 0, c,
                                                         (int)n_seqs);
        return 0;
    });
}

// d, bits, k, v, k_stride, v_stride, query_start_loc, seq_lens, job_seq, job_page, n_jobs, mode, cache,
// block_stride, head_stride, tail_k, tail_idx, block_table, max_pages, hkv
int kush_cpu_write(i64 d, i64 bits, i64 k, i64 v, i64 k_stride, i64 v_stride, i64 qsl, i64 seq_lens, i64 job_seq,
                   i64 job_page, i64 n_jobs, i64 mode, i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx,
                   i64 block_table, i64 max_pages, i64 hkv) {
    const Cache c = make_cache(cache, bs, hs, tail_k, tail_idx, block_table, max_pages, hkv);
    return by_shape(d, bits, [&](auto dd, auto bb) {
        write<decltype(dd)::value, decltype(bb)::value>(ptr<const float>(k), ptr<const float>(v), k_stride, v_stride,
                                                        ptr<const int32_t>(qsl), ptr<const int32_t>(seq_lens),
                                                        ptr<const int32_t>(job_seq), ptr<const int32_t>(job_page),
                                                        n_jobs, (int)mode, c);
        return 0;
    });
}

// d, bits, q, o, cache, block_stride, head_stride, tail_k, tail_idx, block_table, seq_lens, max_pages, hkv,
// group, scale, n_seqs
int kush_cpu_decode(i64 d, i64 bits, i64 q, i64 o, i64 cache, i64 bs, i64 hs, i64 tail_k, i64 tail_idx,
                    i64 block_table, i64 seq_lens, i64 max_pages, i64 hkv, i64 group, float scale, i64 n_seqs) {
    const Cache c = make_cache(cache, bs, hs, tail_k, tail_idx, block_table, max_pages, hkv);
    return by_shape(d, bits, [&](auto dd, auto bb) {
        decode<decltype(dd)::value, decltype(bb)::value>(ptr<const float>(q), ptr<float>(o), c,
                                                         ptr<const int32_t>(seq_lens), (int)group, scale, (int)n_seqs);
        return 0;
    });
}

// d, x (fp32 rows, rotated in place), rows
int kush_cpu_fwht(i64 d, i64 x, i64 rows) {
    return by_shape(d, 4, [&](auto dd, auto) {
        fwht<decltype(dd)::value>(ptr<float>(x), rows);
        return 0;
    });
}

// d, bits, cache, block_stride, head_stride, hkv, page_blk, page_dst, n_pages, tail_blk, tail_info, n_tail,
// tail_k, k_new, v_new, k_stride, v_stride, new_dst, n_new, kp, vp, rot
int kush_cpu_unpack(i64 d, i64 bits, i64 cache, i64 bs, i64 hs, i64 hkv, i64 page_blk, i64 page_dst, i64 n_pages,
                    i64 tail_blk, i64 tail_info, i64 n_tail, i64 tail_k, i64 k_new, i64 v_new, i64 k_stride,
                    i64 v_stride, i64 new_dst, i64 n_new, i64 kp, i64 vp, i64 rot) {
    return by_shape(d, bits, [&](auto dd, auto bb) {
        unpack<decltype(dd)::value, decltype(bb)::value>(
            ptr<const uint8_t>(cache), bs, hs, (int)hkv, ptr<const int32_t>(page_blk), ptr<const int32_t>(page_dst),
            n_pages, ptr<const int32_t>(tail_blk), ptr<const int32_t>(tail_info), n_tail, ptr<const float>(tail_k),
            ptr<const float>(k_new), ptr<const float>(v_new), k_stride, v_stride, ptr<const int32_t>(new_dst), n_new,
            ptr<float>(kp), ptr<float>(vp), rot != 0);
        return 0;
    });
}

// fp16 rounding of this library (the scales' and biases' conversion), for tests: n floats -> n half bits
int kush_cpu_half_bits(i64 x, i64 out, i64 n) {
    const float* src = ptr<const float>(x);
    uint16_t* dst = ptr<uint16_t>(out);
    for (i64 i = 0; i < n; ++i) dst[i] = half_bits(src[i]);
    return 0;
}

}  // extern "C"
