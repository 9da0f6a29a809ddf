// Streaming floor of the decode: a measurement kernel, not part of the product ABI (it is linked
// into libkushfloor.so, which only bench.py loads). It reads exactly the records a decode step
// reads -- the same block table, the same grid of one workgroup per (sequence, kv head), the same
// waves, LDS ring, buffer-to-LDS DMA and explicit vmcnt waits (issue_page and Ring of
// kush_decode.h) -- and does no attention math: per staged page pair a wave reads one 16-byte chunk
// of each record back from LDS into a running xor, so every byte still has to land before its slot
// is refilled. Its duration is the time the memory system needs to deliver this access pattern with
// this launch shape; the decode's duration above it is what the attention math and the decode's own
// prologue and epilogue cost.
//
// Launch shapes (arguments of kush_floor_stream):
//   mode 0  grid (S, Hkv): the decode's; a workgroup streams every full page of one (sequence, kv head)
//   mode 1  grid (S, z): a workgroup streams the full pages [zi pps, (zi + 1) pps) of one sequence for
//           every kv head, heads fastest, so a page pair is two neighbouring records of one block
//   waves   4 or 8 per workgroup; depth: page pairs each wave holds in its ring (2 = the decode's:
//           one consumed while one is in flight; 3 or 4: more bytes in flight per wave)
// marks (optional, int64 [workgroups][8]): the 100 MHz wall clock at the workgroup's start, when wave 0
// issued its first page DMAs, when wave 0's first pair landed, when every wave's pages were done (after
// the workgroup barrier), and the XCD the workgroup ran on.
#include "kush_decode.h"

using namespace kush;

namespace {

template <int D, int BITS, int NW, int DEPTH>
__global__ __launch_bounds__(NW * WAVE) void floor_kernel(const uint8_t* __restrict__ cache, int64_t bs, int64_t hs,
                                                          const int32_t* __restrict__ block_table,
                                                          const int32_t* __restrict__ seq_lens, int64_t bt_stride,
                                                          int H, int mode, int Z, uint32_t* __restrict__ sums,
                                                          long long* __restrict__ marks) {
    using R = Ring<D, BITS>;
    __shared__ __align__(16) uint8_t ring[DEPTH * 2 * NW * R::SLOT];
    __shared__ __align__(16) int tbl[WIN];
    const long long t_start = wall_clock64();
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    const int s = blockIdx.x;
    const int n = seq_lens[s];
    const int full = n / PAGE;
    // the workgroup's pages [pg0, pg1) and heads: mode 0 one head (blockIdx.y), mode 1 all H heads
    int pg0 = 0, pg1 = full, nh = 1, h0 = blockIdx.y;
    if (mode == 1) {
        const int pps = (full + Z - 1) / Z;
        pg0 = min(full, (int)blockIdx.y * pps);
        pg1 = min(full, pg0 + pps);
        nh = H;
        h0 = 0;
    }
    const int np = pg1 - pg0, nunits = np * nh, pairs = (nunits + 1) / 2;
    const int32_t* bt = block_table + (int64_t)s * bt_stride + pg0;
    for (int i = threadIdx.x; i < np; i += NW * WAVE) tbl[i] = bt[i];
    __builtin_amdgcn_s_waitcnt(0x0F70);            // every compiler load in before the DMAs count in vmcnt
    __syncthreads();

    uint32_t voff[R::DMA];
#pragma unroll
    for (int i = 0; i < R::DMA; ++i) voff[i] = src_chunk<D, BITS>(R::chunk0(i) + lane) * 16u;
    // unit u of the workgroup: page pg0 + u / nh, head h0 + u % nh (wave-uniform)
    const auto issue_unit = [&](uint8_t* dst, int u) {
        const bool valid = u < nunits;
        const int uu = valid ? u : 0;
        const int blk = __builtin_amdgcn_readfirstlane(tbl[uu / nh]);
        const int hh = __builtin_amdgcn_readfirstlane(h0 + uu % nh);
        issue_page<D, BITS>(dst, valid, blk, cache + (int64_t)hh * hs, bs, voff);
    };
    uint8_t* const mine = ring + 2 * w * R::SLOT;                // slot d of this wave: mine + d * 2 NW SLOT
    constexpr int DSTRIDE = 2 * NW * R::SLOT;
    const long long t_issue = wall_clock64();
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        const int p = w + d * NW;
        issue_unit(mine + d * DSTRIDE, 2 * p);
        issue_unit(mine + d * DSTRIDE + R::SLOT, 2 * p + 1);
    }
    uint32_t acc = 0;
    long long t_first = 0;
    for (int i = 0, p = w; p < pairs; ++i, p += NW) {
        KUSH_WAIT_VM((DEPTH - 1) * 2 * R::DMA);
        if (i == 0) t_first = wall_clock64();
        uint8_t* const sl = mine + (i % DEPTH) * DSTRIDE;
        const u4 a = *reinterpret_cast<const u4*>(sl + 16 * lane);
        const u4 b = *reinterpret_cast<const u4*>(sl + R::SLOT + 16 * lane);
        acc ^= a[0] ^ a[1] ^ a[2] ^ a[3] ^ b[0] ^ b[1] ^ b[2] ^ b[3];
        __builtin_amdgcn_s_waitcnt(0xC07F);                      // lgkmcnt(0): the slot's reads are done
        const int nx = p + DEPTH * NW;
        issue_unit(sl, 2 * nx);
        issue_unit(sl + R::SLOT, 2 * nx + 1);
    }
    KUSH_WAIT_VM(0);                                             // the trailing (empty) issues
    const int wg = blockIdx.y * gridDim.x + blockIdx.x;
    sums[(int64_t)wg * NW * WAVE + threadIdx.x] = acc;
    if (marks == nullptr) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long* const r = marks + (int64_t)wg * 8;
        r[0] = t_start;
        r[1] = t_issue;
        r[2] = t_first;
        r[3] = wall_clock64();
        r[4] = __builtin_amdgcn_s_getreg((3 << 11) | 20);        // XCC_ID bits [3:0]
    }
}

// Dynamic chunks (mode 2): the same stream, balanced across the XCDs. Every (sequence, kv head) is cut
// into fixed chunks of CP = 2 NW PW pages, numbered c = (s CPS + k) H + h (k: chunk k of the head's
// CPS). A persistent grid of P workgroups takes chunk blockIdx.x first and then claims chunks from a
// device counter one chunk ahead, so a workgroup on a fast XCD takes more of them; the waves' rings
// run on from one chunk into the next without draining. Wave w streams pairs w, w + NW, .. of each
// chunk (PW per chunk; past a sequence's full pages, empty issues). At pair PW - DEPTH - 1 of each
// chunk, wave 0 publishes the chunk it claimed one chunk earlier in LDS (double-buffered by chunk
// parity), one barrier, every wave loads that chunk's length and block ids (scalar loads through the
// constant address space, which the compiler waits on by lgkmcnt, apart from the DMAs' vmcnt; in by
// the lgkmcnt(0) after the next pair's LDS reads), and wave 0 claims the one after it. The two chunks in hand alternate between two register sets (the
// loop body twice), so no id is copied while its load is in flight. Claim v returns P + v - base: a
// launch makes exactly n_chunks claims (one past the end per workgroup), so the caller passes
// base = launch index x n_chunks and never resets the counter; a claim outside [P, n_chunks) ends the
// workgroup, and no workgroup takes more than n_chunks chunks.
// The claim is a returning vector atomic in asm, outside the compiler's vmcnt accounting (a compiler
// atomic would be waited on with vmcnt(0), draining the ring): it is complete once a DMA issued after
// it has been waited on (vector memory returns in order), which the wait at the top of the next
// chunk's publishing pair guarantees; its register is read only after that wait.
template <int D, int BITS, int NW, int DEPTH, int PW>
__global__ __launch_bounds__(NW * WAVE) void floor_dyn_kernel(const uint8_t* __restrict__ cache, int64_t bs, int64_t hs,
                                                              const int32_t* __restrict__ block_table,
                                                              const int32_t* __restrict__ seq_lens, int64_t bt_stride,
                                                              int H, int CPS, int n_chunks, uint32_t* ctr, uint32_t base,
                                                              uint32_t* __restrict__ sums, long long* __restrict__ marks) {
    static_assert(PW > DEPTH && PW % DEPTH == 0, "a chunk holds whole rounds of the ring and one more pair");
    using R = Ring<D, BITS>;
    using cint = const __attribute__((address_space(4))) int32_t;
    constexpr int CP = 2 * NW * PW, PUB = PW - DEPTH - 1;
    constexpr int DSTRIDE = 2 * NW * R::SLOT;
    __shared__ __align__(16) uint8_t ring[DEPTH * DSTRIDE];
    __shared__ int next_chunk[2];
    const long long t_start = wall_clock64();
    const int lane = threadIdx.x & (WAVE - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
    uint32_t voff[R::DMA];
#pragma unroll
    for (int i = 0; i < R::DMA; ++i) voff[i] = src_chunk<D, BITS>(R::chunk0(i) + lane) * 16u;
    uint8_t* const mine = ring + 2 * w * R::SLOT;

    // the wave's PW pairs of a chunk: the sequence's length, the wave's first page, block ids
    struct Pairs {
        int n, pg0, a[PW], b[PW];
        const uint8_t* head;
    };
    const auto load_pairs = [&](int c, Pairs& p) {
        const int h = c % H, k = (c / H) % CPS, s = c / (H * CPS);
        cint* const bt = (cint*)(block_table + (int64_t)s * bt_stride + k * CP + 2 * w);
        p.head = cache + (int64_t)h * hs;
        p.pg0 = k * CP + 2 * w;
        p.n = ((cint*)seq_lens)[s];
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            p.a[i] = bt[2 * NW * i];
            p.b[i] = bt[2 * NW * i + 1];
        }
    };
    const auto issue_pair = [&](uint8_t* dst, const Pairs& p, int i) {
        const int pg = p.pg0 + 2 * NW * i;                 // page pg is full when (pg + 1) PAGE <= n
        issue_page<D, BITS>(dst, (pg + 1) * PAGE <= p.n, p.a[i], p.head, bs, voff);
        issue_page<D, BITS>(dst + R::SLOT, (pg + 2) * PAGE <= p.n, p.b[i], p.head, bs, voff);
    };
    const auto empty_pair = [&](uint8_t* dst) {
        issue_page<D, BITS>(dst, false, 0, cache, bs, voff);
        issue_page<D, BITS>(dst + R::SLOT, false, 0, cache, bs, voff);
    };
    uint32_t claim = 0;
    const auto claim_next = [&]() {                  // wave 0, lane 0's returning atomic add
        if (w == 0 && lane == 0) {
            const uint32_t one = 1u;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
            asm volatile("global_atomic_add %0, %1, %2, off sc0" : "=v"(claim) : "v"(ctr), "v"(one) : "memory");
#pragma clang diagnostic pop
        }
    };

    const int P = __builtin_amdgcn_readfirstlane((int)gridDim.x);
    int chunks = 0;
    uint32_t acc = 0;
    long long t_first = 0;
    // one chunk: consume its PW pairs, refilling the ring from `cur` and, past its end, from `nxt`
    // (published and loaded at pair PUB); returns whether there is a next chunk
    const auto run_chunk = [&](const Pairs& cur, Pairs& nxt, int parity) -> bool {
        bool more = false;
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            KUSH_WAIT_VM((DEPTH - 1) * 2 * R::DMA);
            if (chunks == 0 && i == 0) t_first = wall_clock64();
            uint8_t* const sl = mine + (i % DEPTH) * DSTRIDE;
            const u4 x = *reinterpret_cast<const u4*>(sl + 16 * lane);
            const u4 y = *reinterpret_cast<const u4*>(sl + R::SLOT + 16 * lane);
            acc ^= x[0] ^ x[1] ^ x[2] ^ x[3] ^ y[0] ^ y[1] ^ y[2] ^ y[3];
            __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): the slot's reads done
            if (i == PUB) {                              // the next chunk: published, then claimed onward
                if (w == 0 && lane == 0) {
                    asm volatile("" : "+v"(claim));      // read only now, after the wait above
                    next_chunk[parity] = (int)(claim - base) + P;
                }
                __syncthreads();
                const int nx = __builtin_amdgcn_readfirstlane(next_chunk[parity]);
                more = __builtin_amdgcn_readfirstlane(nx >= P && nx < n_chunks && chunks + 1 < n_chunks);
                // loaded unconditionally (a valid chunk when there is none next), so no branch joins
                // over the loads and nothing reads them before the next pair's lgkmcnt(0)
                load_pairs(more ? nx : (int)blockIdx.x, nxt);
                if (more) claim_next();
            }
            if (i + DEPTH < PW) issue_pair(sl, cur, i + DEPTH);
            else if (more) issue_pair(sl, nxt, i + DEPTH - PW);
            else empty_pair(sl);
        }
        ++chunks;
        return more;
    };

    Pairs pa, pb;
    load_pairs(blockIdx.x, pa);
    claim_next();
    const long long t_issue = wall_clock64();
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue_pair(mine + d * DSTRIDE, pa, d);
    for (;;) {
        if (!run_chunk(pa, pb, 0)) break;
        if (!run_chunk(pb, pa, 1)) break;
    }
    KUSH_WAIT_VM(0);
    const int wg = blockIdx.x;
    sums[(int64_t)wg * NW * WAVE + threadIdx.x] = acc;
    if (marks == nullptr) return;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long* const r = marks + (int64_t)wg * 8;
        r[0] = t_start;
        r[1] = t_issue;
        r[2] = t_first;
        r[3] = wall_clock64();
        r[4] = __builtin_amdgcn_s_getreg((3 << 11) | 20);        // XCC_ID bits [3:0]
        r[5] = chunks;
    }
}

template <int D, int BITS, int NW, int DEPTH>
constexpr bool floor_fits() {
    return DEPTH * 2 * NW * Ring<D, BITS>::SLOT + 4 * WIN + 8 * NW <= 160 * 1024 && 2 * DEPTH * Ring<D, BITS>::DMA <= 63;
}

template <int D, int BITS, int NW, int DEPTH>
int launch_floor(dim3 grid, hipStream_t st, const void* cache, int64_t bs, int64_t hs, const int32_t* bt,
                 const int32_t* sl, int64_t bt_stride, int H, int mode, int Z, uint32_t* sums, int64_t* marks) {
    if constexpr (floor_fits<D, BITS, NW, DEPTH>()) {
        floor_kernel<D, BITS, NW, DEPTH><<<grid, dim3(NW * WAVE), 0, st>>>(
            (const uint8_t*)cache, bs, hs, bt, sl, bt_stride, H, mode, Z, sums, (long long*)marks);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    } else {
        return -2;
    }
}

template <int D, int BITS>
int by_shape(int waves, int depth, dim3 grid, hipStream_t st, const void* cache, int64_t bs, int64_t hs,
             const int32_t* bt, const int32_t* sl, int64_t bt_stride, int H, int mode, int Z, uint32_t* sums,
             int64_t* marks) {
#define KUSH_FLOOR(NW, DEPTH)                                                                       \
    if (waves == NW && depth == DEPTH)                                                              \
        return launch_floor<D, BITS, NW, DEPTH>(grid, st, cache, bs, hs, bt, sl, bt_stride, H, mode, Z, sums, marks);
    KUSH_FLOOR(4, 2)
    KUSH_FLOOR(4, 3)
    KUSH_FLOOR(4, 4)
    KUSH_FLOOR(8, 2)
#undef KUSH_FLOOR
    return -2;
}

template <int D, int BITS, int NW, int DEPTH, int PW>
int launch_dyn(int P, hipStream_t st, const void* cache, int64_t bs, int64_t hs, const int32_t* bt, const int32_t* sl,
               int64_t bt_stride, int H, int CPS, int n_chunks, uint32_t* ctr, uint32_t base, uint32_t* sums,
               int64_t* marks) {
    if constexpr (floor_fits<D, BITS, NW, DEPTH>()) {
        floor_dyn_kernel<D, BITS, NW, DEPTH, PW><<<dim3(P), dim3(NW * WAVE), 0, st>>>(
            (const uint8_t*)cache, bs, hs, bt, sl, bt_stride, H, CPS, n_chunks, ctr, base, sums, (long long*)marks);
        return hipGetLastError() == hipSuccess ? 0 : -3;
    } else {
        return -2;
    }
}

}  // namespace

// Dynamic chunks of 2 waves pw pages (mode 2 above) on a persistent grid of P workgroups; ctr: one
// uint32 the caller zeroes once, base = (launches so far) x n_chunks, n_chunks = n_seqs hkv
// ceil(max_pages / chunk). Shapes: D 128, bits 4 or 8, waves 4 with depth 2 and pw 4 or 8, waves 8 with
// depth 2 and pw 4; P <= n_chunks and the table's rows hold ceil(max_pages / chunk) chunks. Returns 0,
// -2 for a shape or size it does not take, -3 for a launch error.
extern "C" int kush_floor_dynamic(int head_dim, int bits, const void* cache, int64_t block_stride, int64_t head_stride,
                                  const int32_t* block_table, const int32_t* seq_lens, int64_t bt_stride, int32_t hkv,
                                  int32_t n_seqs, int32_t max_pages, int32_t P, int32_t waves, int32_t depth, int32_t pw,
                                  uint32_t* ctr, uint32_t base, uint32_t* sums, int64_t* marks, void* stream) {
    if (head_dim != 128 || (bits != 4 && bits != 8) || n_seqs <= 0 || hkv <= 0 || P <= 0 || depth != 2) return -2;
    const int CP = 2 * waves * pw;
    const int CPS = (max_pages + CP - 1) / CP;
    const int64_t n_chunks = (int64_t)n_seqs * hkv * CPS;
    if (CPS <= 0 || P > n_chunks || n_chunks >= (1 << 30) || (int64_t)CPS * CP > bt_stride) return -2;
    if (((uintptr_t)cache | (uint64_t)block_stride | (uint64_t)head_stride) & 15) return -2;
    hipStream_t st = (hipStream_t)stream;
    const int nc = (int)n_chunks;
#define KUSH_DYN(NW, PW)                                                                                      \
    if (waves == NW && pw == PW)                                                                              \
        return bits == 4 ? launch_dyn<128, 4, NW, 2, PW>(P, st, cache, block_stride, head_stride, block_table, \
                                                         seq_lens, bt_stride, hkv, CPS, nc, ctr, base, sums, marks) \
                         : launch_dyn<128, 8, NW, 2, PW>(P, st, cache, block_stride, head_stride, block_table, \
                                                         seq_lens, bt_stride, hkv, CPS, nc, ctr, base, sums, marks);
    KUSH_DYN(4, 4)
    KUSH_DYN(4, 8)
    KUSH_DYN(8, 4)
#undef KUSH_DYN
    return -2;
}

// sums: uint32 [workgroups][waves * 64]; marks: int64 [workgroups][8] or null. Returns 0, -2 for a
// shape this library has no kernel for (D 128, bits 4 or 8, waves 4 with depth 2-4, waves 8 with
// depth 2, at most 1,024 pages per workgroup), -3 for a launch error.
extern "C" int kush_floor_stream(int head_dim, int bits, const void* cache, int64_t block_stride, int64_t head_stride,
                                 const int32_t* block_table, const int32_t* seq_lens, int64_t bt_stride, int32_t hkv,
                                 int32_t n_seqs, int32_t max_pages, int32_t mode, int32_t z, int32_t waves,
                                 int32_t depth, uint32_t* sums, int64_t* marks, void* stream) {
    if (head_dim != 128 || (bits != 4 && bits != 8) || n_seqs <= 0 || hkv <= 0 || (mode != 0 && mode != 1))
        return -2;
    const int Z = mode == 1 ? z : 1;
    if (Z <= 0 || (max_pages + Z - 1) / Z > WIN) return -2;
    if (((uintptr_t)cache | (uint64_t)block_stride | (uint64_t)head_stride) & 15) return -2;
    const dim3 grid(n_seqs, mode == 1 ? Z : hkv);
    hipStream_t st = (hipStream_t)stream;
    return bits == 4 ? by_shape<128, 4>(waves, depth, grid, st, cache, block_stride, head_stride, block_table, seq_lens,
                                        bt_stride, hkv, mode, Z, sums, marks)
                     : by_shape<128, 8>(waves, depth, grid, st, cache, block_stride, head_stride, block_table, seq_lens,
                                        bt_stride, hkv, mode, Z, sums, marks);
}
