// C entry points of the fused dequant decode attention (kush_decode), the same launch with the
// step's token appended first (kush_append_decode) and the split-K combine (kush_combine); the
// kernels and their launch are in kush_decode.h (contract and design notes there).
#include <cstdlib>
#include <mutex>

#include "kush_decode.h"

using namespace kush;

namespace {

// The new tokens of a fused append + decode (row s of k / v at position seq_lens[s] - 1), or none
struct Append {
    const void* k = nullptr;
    const void* v = nullptr;
    int64_t k_stride = 0, v_stride = 0;
};

// Wave splits (decode_kernel WS: every wave a whole split of its own, the workgroup's q and launch
// cost shared by its 4 splits; with the in-launch merge the workgroup merges its 4 splits in LDS and
// writes one partial, so the last workgroup merges NS / 4): at 4 waves, whenever 4 divides NS,
// NS >= 8 and the workgroups still fill MI355X's 256 CUs. C4 (8 x 131,072 tokens) at 4 waves:
// NS 32 / 64 / 128 / 256 232 / 243 / 280 / 373 us -> 222 / 226 / 234 / 242 us.
// KUSHKASH_AMD_WAVE_SPLITS=0 / 1 turns it off / on wherever NS allows it.
//
// Returns 0 (no wave splits) or KW, the splits each wave takes: with the in-launch merge, as many
// consecutive splits per wave as keep at least 256 workgroups (one per CU of MI355X), so a large NS
// no longer multiplies the workgroups and their fixed costs (launch, q, window loads, the ramp of
// the first pages, the merge in LDS) -- C4 at NS 64 / 128 / 256 runs 256 workgroups of 4 waves,
// each wave streaming its 4 / 8 / 16 splits as one run of pages and folding each finished split
// into its running state. KUSHKASH_AMD_SPLITS_PER_WAVE=k takes k splits per wave wherever NS allows
// it (k = 1: one split per wave, as without the fold).
int wave_splits(int ns, int nw, int64_t chunks, bool fused_merge) {
    if (nw != 4 || ns % nw != 0 || ns < 2 * nw) return 0;             // built for 4 waves
    const char* env = std::getenv("KUSHKASH_AMD_WAVE_SPLITS");
    if (env != nullptr && env[0] == '0') return 0;
    if (!(env != nullptr && env[0] == '1') && chunks * (ns / nw) < 256) return 0;
    if (!fused_merge) return 1;                                      // the caller's combine reads NS partials
    const char* per = std::getenv("KUSHKASH_AMD_SPLITS_PER_WAVE");
    const int forced = per != nullptr ? std::atoi(per) : 0;
    if (forced >= 1) return ns % (nw * forced) == 0 ? forced : 1;
    int kw = 1;
    while ((ns / nw) % (2 * kw) == 0 && chunks * (ns / (nw * 2 * kw)) >= 256) kw *= 2;
    return kw;
}

int decode_impl(const char* what, int head_dim, int bits, int group, int dtype, const void* q, void* out,
                const void* cache, int64_t block_stride, int64_t head_stride, const void* tail_k, const int32_t* tail_idx,
                const int32_t* block_table, const int32_t* seq_lens, int64_t bt_stride, int32_t bt_cols, int32_t hkv,
                float scale, int32_t n_splits, float* part_ml, float* part_o, int32_t* split_sync, int32_t waves,
                const int32_t* seq_order, int32_t n_seqs, int32_t rot, const Append& app, void* stream) {
    if (n_seqs < 0 || hkv <= 0 || group <= 0 || n_splits <= 0 || bt_cols < 0 || rot < 0 || rot > 1)
        return kush_fail(-2, "%s: bad n_seqs %d / hkv %d / group %d / n_splits %d / bt_cols %d / rot %d", what, n_seqs,
                         hkv, group, n_splits, bt_cols, rot);
    if (n_splits > 1 && (part_ml == nullptr || part_o == nullptr))
        return kush_fail(-2, "%s: n_splits %d needs the partial buffers", what, n_splits);
    if (((uintptr_t)cache | (uint64_t)block_stride | (uint64_t)head_stride) & 15)
        return kush_fail(-2, "%s: cache records must be 16-byte aligned", what);
    if (((uintptr_t)q | (uintptr_t)tail_k) & 15) return kush_fail(-2, "%s: q and tail_k must be 16-byte aligned", what);
    if (waves == 0) waves = 4;
    if (waves != 2 && waves != 4 && waves != 8) return kush_fail(-2, "%s: waves must be 0, 2, 4 or 8", what);
    const int n_gc = (group + 15) / 16;
    if ((int64_t)n_splits * n_gc > 65535) return kush_fail(-2, "%s: n_splits %d too large", what, n_splits);
    // scores in log2 units: scale log2 e = p2 rs with p2 a signed power of two (q p2 is exact in fp16
    // for bf16 / fp16 q) and rs in [2^-0.5, 2^0.5] (a zero scale becomes 2^-120: x ~ 0, masks stay -inf)
    const float sm_log2 = (float)((double)scale * 1.4426950408889634);
    float p2 = 1.0f, rs = 0x1p-120f;
    if (!std::isfinite(sm_log2)) {
        rs = sm_log2;
    } else if (sm_log2 != 0.0f) {
        int e2 = 0;
        const float m = std::frexp(std::fabs(sm_log2), &e2);          // |sm_log2| = m 2^e2, m in [0.5, 1)
        if (m < 0.70710678f) --e2;
        p2 = std::copysign(std::ldexp(1.0f, e2), sm_log2);
        rs = sm_log2 / p2;
    }
    hipStream_t st = (hipStream_t)stream;
    return dispatch_shape(head_dim, bits, dtype, what, [&](auto dd, auto bb, auto in) -> int {
        constexpr int D = decltype(dd)::value, BITS = decltype(bb)::value;
        using IN = decltype(in);
        if (n_seqs == 0) return 0;
#define KUSH_DECODE_ARGS st, q, out, cache, block_stride, head_stride, tail_k, tail_idx, block_table, seq_lens, \
                         bt_stride, bt_cols, hkv, group, p2, rs, n_splits, part_ml, part_o, split_sync, seq_order, app.k, \
                         app.v, app.k_stride, app.v_stride
        // the largest of the requested, 4 and 2 waves whose rings fit in LDS
        const auto launch = [&](auto nw) -> int {
            constexpr int NW = decltype(nw)::value;
            const int ws = wave_splits(n_splits, NW, (int64_t)n_seqs * hkv * n_gc, split_sync != nullptr);
            const dim3 g(n_seqs, hkv, (ws ? n_splits / (NW * ws) : n_splits) * n_gc);
            return rot ? launch_decode<D, BITS, IN, NW, true>(g, KUSH_DECODE_ARGS, ws)
                       : launch_decode<D, BITS, IN, NW, false>(g, KUSH_DECODE_ARGS, ws);
        };
        if (waves >= 8) {
            if constexpr (decode_fits<D, BITS, 8>()) return launch(std::integral_constant<int, 8>{});
        }
        if (waves >= 4) {
            if constexpr (decode_fits<D, BITS, 4>()) return launch(std::integral_constant<int, 4>{});
        }
        static_assert(decode_fits<D, BITS, 2>(), "two waves' rings must fit in LDS");
        return launch(std::integral_constant<int, 2>{});
#undef KUSH_DECODE_ARGS
    });
}

}  // namespace

extern "C" int kush_decode_ex(int head_dim, int bits, int group, int dtype, const void* q, void* out,
                              const void* cache, int64_t block_stride, int64_t head_stride, const void* tail_k,
                              const int32_t* tail_idx, const int32_t* block_table, const int32_t* seq_lens,
                              int64_t bt_stride, int32_t hkv, float scale, int32_t n_splits, float* part_ml,
                              float* part_o, int32_t n_seqs, void* stream, int32_t bt_cols, int32_t* split_sync,
                              int32_t waves, const int32_t* seq_order, int32_t rot) {
    return decode_impl("kush_decode", head_dim, bits, group, dtype, q, out, cache, block_stride, head_stride, tail_k,
                       tail_idx, block_table, seq_lens, bt_stride, bt_cols, hkv, scale, n_splits, part_ml, part_o,
                       split_sync, waves, seq_order, n_seqs, rot, Append{}, stream);
}

// The reference's argument list exactly: no table prefetch, no in-launch merge (n_splits > 1 leaves
// the partials for kush_combine, as the reference's second launch), the default waves, no rotation.
extern "C" int kush_decode(int head_dim, int bits, int group, int dtype, const void* q, void* out, const void* cache,
                           int64_t block_stride, int64_t head_stride, const void* tail_k, const int32_t* tail_idx,
                           const int32_t* block_table, const int32_t* seq_lens, int64_t bt_stride, int32_t hkv,
                           float scale, int32_t n_splits, float* part_ml, float* part_o, int32_t n_seqs, void* stream) {
    return decode_impl("kush_decode", head_dim, bits, group, dtype, q, out, cache, block_stride, head_stride, tail_k,
                       tail_idx, block_table, seq_lens, bt_stride, 0, hkv, scale, n_splits, part_ml, part_o, nullptr, 0,
                       nullptr, n_seqs, 0, Append{}, stream);
}

extern "C" int kush_append_decode(int head_dim, int bits, int group, int dtype, const void* q, void* out, void* cache,
                                  int64_t block_stride, int64_t head_stride, void* tail_k, const int32_t* tail_idx,
                                  const int32_t* block_table, const int32_t* seq_lens, int64_t bt_stride, int32_t hkv,
                                  float scale, int32_t n_splits, float* part_ml, float* part_o, int32_t n_seqs,
                                  void* stream, const void* k, const void* v, int64_t k_row_stride,
                                  int64_t v_row_stride, int32_t bt_cols, int32_t* split_sync, int32_t waves,
                                  const int32_t* seq_order, int32_t rot) {
    if (group > 16) return kush_fail(-2, "kush_append_decode: group %d > 16 (use kush_append, then kush_decode)", group);
    if (k == nullptr || v == nullptr) return kush_fail(-2, "kush_append_decode: k and v are required");
    const int64_t e = dtype == 0 ? 4 : 2;
    if (((uintptr_t)k | (uintptr_t)v | (uint64_t)(k_row_stride * e) | (uint64_t)(v_row_stride * e)) & 15)
        return kush_fail(-2, "kush_append_decode: k / v rows must be 16-byte aligned (use kush_append, then kush_decode)");
    return decode_impl("kush_append_decode", head_dim, bits, group, dtype, q, out, cache, block_stride, head_stride,
                       tail_k, tail_idx, block_table, seq_lens, bt_stride, bt_cols, hkv, scale, n_splits, part_ml, part_o,
                       split_sync, waves, seq_order, n_seqs, rot, Append{k, v, k_row_stride, v_row_stride}, stream);
}

extern "C" int kush_combine_ex(int head_dim, int group, int dtype, void* out, const float* part_ml, const float* part_o,
                               int32_t n_splits, int32_t hkv, int32_t n_seqs, void* stream, int32_t rot) {
    if (n_seqs < 0 || hkv <= 0 || group <= 0 || n_splits <= 0 || rot < 0 || rot > 1)
        return kush_fail(-2, "kush_combine: bad arguments");
    // bits does not matter here: any record format's partials
    return dispatch_shape(head_dim, 4, dtype, "kush_combine", [&](auto dd, auto, auto in) -> int {
        constexpr int D = decltype(dd)::value;
        using IN = decltype(in);
        if (n_seqs == 0) return 0;
        auto kern = rot ? combine_kernel<D, IN, true> : combine_kernel<D, IN, false>;
        // the parallel merge when its LDS scratch fits in 48 KB of dynamic LDS
        const int64_t lds = (int64_t)merge_smem_floats(n_splits, group < 16 ? group : 16, 4) * 4;
        const int parallel = lds <= 48 * 1024;
        kern<<<dim3(n_seqs, hkv), dim3(256), parallel ? (size_t)lds : 0, (hipStream_t)stream>>>(
            (IN*)out, part_ml, part_o, n_splits, hkv, group, parallel);
        return kush_check_launch("kush_combine");
    });
}

extern "C" int kush_combine(int head_dim, int group, int dtype, void* out, const float* part_ml, const float* part_o,
                            int32_t n_splits, int32_t hkv, int32_t n_seqs, void* stream) {
    return kush_combine_ex(head_dim, group, dtype, out, part_ml, part_o, n_splits, hkv, n_seqs, stream, 0);
}

// ------------------------------------------------------------------ allocation-free decode
// kush_decode_noalloc: kush_decode_ex whose split-K scratch -- the merge counters, then the partials
// (part_ml, part_o) -- lives in this file-scope device array instead of caller buffers, for callers
// that cannot allocate (code under HIP graph capture, tight serving loops). Each device holds its
// own copy for the life of the process; its address is looked up once per device
// (hipGetSymbolAddress) and only that address is handed to the kernels. The counters must start at
// zero: a fill kernel clears them at that set-up, and the in-launch merge leaves them zero after
// every call. Calls that overlap on one device share the array and race.
namespace {

constexpr size_t SCRATCH_BYTES = size_t(64) << 20;          // per device
constexpr size_t SCRATCH_SYNC = 1 << 16;                   // int32 merge counters at the front
constexpr size_t SCRATCH_PART0 = SCRATCH_SYNC * sizeof(int32_t);
static_assert(SCRATCH_PART0 % 256 == 0, "the partials start aligned");

static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

__global__ __launch_bounds__(256) void zero_words(int32_t* p, int n) {
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i < n) p[i] = 0;
}

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[MAX_DEVICES] = {};

// The device address of `scratch` on the current device (set up on the first call there); nullptr
// after a failure, which is then reported through kush_fail.
uint8_t* scratch_on_device(hipStream_t stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) {
        kush_fail(-3, "kush_decode_noalloc: no current device (or device %d beyond %d)", dev, MAX_DEVICES);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            kush_fail(-3, "kush_decode_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                      hipGetErrorString(e));
            return nullptr;
        }
        zero_words<<<dim3((unsigned)((SCRATCH_SYNC + 255) / 256)), dim3(256), 0, stream>>>((int32_t*)ptr,
                                                                                           (int)SCRATCH_SYNC);
        if (kush_check_launch("kush_decode_noalloc (scratch set-up)") != 0) return nullptr;
        g_scratch[dev] = (uint8_t*)ptr;
    }
    return g_scratch[dev];
}

}  // namespace

extern "C" int kush_decode_noalloc(int head_dim, int bits, int group, int dtype, const void* q, void* out,
                                   const void* cache, int64_t block_stride, int64_t head_stride, const void* tail_k,
                                   const int32_t* tail_idx, const int32_t* block_table, const int32_t* seq_lens,
                                   int64_t bt_stride, int32_t hkv, float scale, int32_t n_splits, int32_t n_seqs,
                                   void* stream, int32_t bt_cols, int32_t waves, const int32_t* seq_order,
                                   int32_t rot) {
    float* part_ml = nullptr;
    float* part_o = nullptr;
    int32_t* sync = nullptr;
    if (n_splits > 1 && n_seqs > 0 && hkv > 0 && group > 0) {
        const int64_t rows = (int64_t)n_seqs * hkv * n_splits * group;
        const int64_t counters = (int64_t)n_seqs * hkv * ((group + 15) / 16);
        const int64_t need = (int64_t)SCRATCH_PART0 + rows * (2 + (int64_t)head_dim) * (int64_t)sizeof(float);
        if (counters > (int64_t)SCRATCH_SYNC || need > (int64_t)SCRATCH_BYTES)
            return kush_fail(-2,
                             "kush_decode_noalloc: %d splits of %d sequences x %d kv heads x %d q heads need %lld "
                             "bytes of scratch (%lld merge counters); the maximum is %zu bytes (%zu counters): "
                             "use kush_decode_ex with caller-owned buffers",
                             n_splits, n_seqs, hkv, group, (long long)need, (long long)counters, SCRATCH_BYTES,
                             SCRATCH_SYNC);
        uint8_t* base = scratch_on_device((hipStream_t)stream);
        if (base == nullptr) return -3;
        sync = (int32_t*)base;
        part_ml = (float*)(base + SCRATCH_PART0);
        part_o = part_ml + 2 * rows;
    }
    return decode_impl("kush_decode_noalloc", head_dim, bits, group, dtype, q, out, cache, block_stride, head_stride,
                       tail_k, tail_idx, block_table, seq_lens, bt_stride, bt_cols, hkv, scale, n_splits, part_ml,
                       part_o, sync, waves, seq_order, n_seqs, rot, Append{}, stream);
}
