/*
 * qmm_runtime.cpp -- the C ABI of include/dflash_qmm.h: code-object loading, the work
 * split of the fast kernel, launches, workspace, graph capture.
 *
 * The gfx950 code object built from qmm_kernels.hip is linked into this library with
 * .incbin and loaded with hipModuleLoadData, so the library is one self-contained file.
 */
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>

#include "dflash_qmm.h"
#include "qmm_internal.h"
#include "qmm_params.h"

#ifndef DFQ_HSACO_PATH
#error "DFQ_HSACO_PATH must name the gfx950 code object to embed"
#endif

__asm__(".section .rodata.dfq_hsaco,\"a\",@progbits\n"
        ".p2align 12\n"
        ".globl dfq_hsaco_begin\n"
        ".hidden dfq_hsaco_begin\n"
        "dfq_hsaco_begin:\n"
        ".incbin \"" DFQ_HSACO_PATH "\"\n"
        ".globl dfq_hsaco_end\n"
        ".hidden dfq_hsaco_end\n"
        "dfq_hsaco_end:\n"
        ".byte 0\n"
        ".previous\n");
extern "C" const char dfq_hsaco_begin[];
extern "C" const char dfq_hsaco_end[];

namespace {

thread_local std::string g_last_error;

#ifndef DFQ_WAVES
#define DFQ_WAVES 12                   // must match the kernels' build
#endif
#ifndef DFQ_MIN_KBLOCKS
#define DFQ_MIN_KBLOCKS 1              // k-blocks the planner starts from
#endif
constexpr int kWaves = DFQ_WAVES;
constexpr int kThreads = kWaves * 64;             // qmm_mt8 streaming threads
#ifndef DFQ_PUBLISHERS
#define DFQ_PUBLISHERS 4               // must match the kernels' build
#endif
constexpr int kBlockThreads = kThreads + 64 * DFQ_PUBLISHERS;  // + the publisher waves
/* 16-byte x chunks a staging thread holds for a k-block of kr elements at M rows (0 when no
 * thread layout exists); the kernels take up to DFQ_STAGE_ITEMS(mt). */
static int stage_items(int M, int kr, int gs) {
    const int tpr = DFQ_STAGE_TPR(M, gs);
    return tpr > 0 ? (kr / 8 + tpr - 1) / tpr : 0;
}
/* Whether that x fits the staging of a split of nkb k-blocks.  Past DFQ_STAGE_ITEMS(1) items
 * (the 9..16-row kernels only) the staging costs more than a second k-block saves unless the
 * x is read for enough weights: such a split must be one k-block (up to 12 rows at
 * K = 5120), and is kept only where each range holds at least three tiles' units and one
 * round of workgroups covers the split (checked by the caller).  Measured on MI355X (us,
 * one k-block against two) with two publisher waves: N = 17408, K = 5120 at 10 rows 16.2
 * against 18.4, 11 rows 16.6 against 18.2, 12 rows 16.7 against 18.2; gate|up N = 34816 at
 * 12 rows 27.9 against 31.7; N = 7168 at 12 rows (1.8 tiles a range) 12.2 against 11.45;
 * 16 rows at N = 40000, K = 4096 (two rounds of workgroups) 31.1 against 28.6, N = 80000
 * (four) 58.6 against 49.0.  With four, two k-blocks cost less but still more: N = 17408 at
 * 9 rows 16.0 against 17.0, 10 rows 16.5 against 17.1, 12 rows 16.8 against 17.2 (8-bit
 * 23.5 against 25.2, g128 at 9 rows 14.9 against 17.0); N = 34816 at 9 rows 25.5 against
 * 28.2, at 12 rows 28.1 against 27.9. */
static bool stage_fits(int M, int kr, int gs, int nkb) {
    const int items = stage_items(M, kr, gs);
    if (items < 1) return false;
    if (items <= DFQ_STAGE_ITEMS(1)) return true;
    return M > 8 && nkb == 1 && items <= DFQ_STAGE_ITEMS(2);
}

struct PlanKey {
    int M, N, K, bits, gs;
    bool operator==(const PlanKey& o) const {
        return M == o.M && N == o.N && K == o.K && bits == o.bits && gs == o.gs;
    }
};
struct PlanKeyHash {
    size_t operator()(const PlanKey& k) const {
        uint64_t h = 1469598103934665603ull;
        for (int v : {k.M, k.N, k.K, k.bits, k.gs}) {
            h ^= (uint64_t)(uint32_t)v;
            h *= 1099511628211ull;
        }
        return (size_t)h;
    }
};

}  // namespace

struct dfq_ctx {
    int device = 0;
    int num_cus = 0;
    size_t lds_max = 0;
    hipModule_t module = nullptr;
    hipFunction_t mt8[2][3][2][2] = {};  // [bits 4/8][gs 32/64/128][bf16/f16][chunk 1/8 groups]
    hipFunction_t mt16[2][3][2] = {};    // up to 16 rows, 8-group chunks [bits][gs][bf16/f16]
    hipFunction_t am[2][3][2][2] = {};   // greedy-accept forms, 8-group chunks [..][rows 8/16]
    hipFunction_t pk[2][3][2][2] = {};   // over the packed layout [bits][gs][dt][rows 8/16]
    hipFunction_t pk_am[2][3][2][2] = {};  // greedy-accept forms over the packed layout
    /* 4-bit group 32, 16-group chunks at up to 8 rows [bf16/f16][plain, _am, _pk, _am_pk] */
    hipFunction_t c16[2][4] = {};
    hipFunction_t pack = nullptr;        // MLX arrays -> the packed layout
    hipFunction_t reduce[2] = {};        // second pass of reduce splits [bf16/f16]
    hipFunction_t silu_mul[2] = {};      // SiLU-mul of a fused gate||up output [bf16/f16]
    hipFunction_t argmax_accept[2] = {}; // greedy accept of a verify pass [bf16/f16]
    hipFunction_t qmv[2][3][2][2] = {};  // stock-path GEMV [bits][gs][bf16/f16][rows 1 / <= 4]
    hipFunction_t generic = nullptr;
    hipFunction_t fill = nullptr;
    hipFunction_t read_stream = nullptr; // the plain streaming read (bandwidth reference)
    hipFunction_t read_units = nullptr;  // the fast kernel's own loads with no compute
    hipFunction_t read_units_packed = nullptr;  // the same over the packed layout
    void* scratch = nullptr;             // the fixed scratch of dfq_qmm_noalloc (this device)
    std::mutex mu;
    std::unordered_map<PlanKey, dfq::Plan, PlanKeyHash> plans;
    /* Splits that dfq_qmm_noalloc computed for shapes the cache above does not hold: a table
     * allocated with the context and filled without allocating (the oldest entry goes when
     * it is full), so that a no-allocation caller plans each shape once, not on every call. */
    static constexpr int kFixedPlans = 64;
    PlanKey fixed_key[kFixedPlans] = {};
    dfq::Plan fixed_plan[kFixedPlans];
    int fixed_used = 0;
    int fixed_next = 0;
};

struct dfq_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int device = 0;
};

namespace dfq {

dfq_status fail(dfq_status s, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return s;
}

dfq_status hip_fail(hipError_t e, const char* what) {
    return fail(DFQ_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

/* Makes ctx's device current for the scope and restores the caller's afterwards. */
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

int ctx_device(const dfq_ctx* ctx) { return ctx->device; }

DeviceScope::DeviceScope(const dfq_ctx* ctx) : dev_(ctx_device(ctx)) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != dev_) (void)hipSetDevice(dev_);
}

DeviceScope::~DeviceScope() {
    int cur = -1;
    if (prev_ >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
}

/* Groups of a unit of the packed layout, and of the chunks the 1..8-row kernels prefer: 8
 * (one 16-byte scale load per lane); 16 at 4-bit group 32, whose 8-group chunk holds only
 * 2 KB of codes a unit and pays the per-unit costs twice as often as group 64.  Measured on
 * MI355X, M = 8 (us, 16-group chunks against 8, same box): N = 17408, K = 5120 17.1 against
 * 19.0; one row 16.3 against 18.0; N = 7168 11.9 against 12.9; N = 5120 10.6 against 10.9. */
int chunk_groups(int bits, int gs) { return (bits == 4 && gs == 32) ? 16 : 8; }

int kss_for(int bits, int gs) {
    const int kstep = 512 / bits;
    const int ns = bits == 4 ? (gs == 128 ? 2 : 1) : gs / 32;
    return kstep * ns;
}

/* Workgroup c owns units [c*base + min(c, rem), +base + (c < rem)); same rule as the kernel. */
static int64_t owner_wg(int64_t u, int64_t base, int64_t rem) {
    const int64_t big = rem * (base + 1);
    return u < big ? u / (base + 1) : rem + (u - big) / base;
}

/* Workgroups of k-block range [a, b) that share tile t's units, for a k-block of SS chunks
 * split over G workgroups. */
static int tile_owners(int64_t t, int64_t SS, int64_t G, int64_t T) {
    const int64_t U = T * SS, base = U / G, rem = U % G;
    return (int)(owner_wg(t * SS + SS - 1, base, rem) - owner_wg(t * SS, base, rem) + 1);
}

/* Largest workgroup share (units) for which a narrow N is split into two k-blocks of one tile
 * per workgroup. */
static constexpr int kShortSplitUnits = 24;
/* Fewest tiles a workgroup touches for which its outputs (whole tiles to y, or the parts of a
 * reduce split to their workspace slots) are written at its end rather than as each tile
 * finishes.  Stores from the publisher waves interleave with the weight stream; written at
 * the end they do not, but the end then waits for every wave.  Measured on MI355X at M = 8,
 * K = 5120 (us, at the end against as they finish): the LM head N = 151936 (38 tiles) 83.3
 * against 90.7; gate|up N = 34816 (10) 25.25 against 25.55; N = 17408 (6) 16.54 against
 * 16.37; N = 7168 (3) 11.67 against 11.41.  The 16-row reduce split at N = 17408 (10 tiles
 * in each of two k-blocks): 19.8-20.2 against 20.0-20.8; 12 rows 18.9-19.0 against
 * 19.3-19.6. */
static constexpr int kBurstTiles = 8;
/* Most tiles per workgroup for which two k-blocks take an aligned split rather than stream-K
 * ranges with the second pass.  Measured on MI355X with 9..16 rows (us, aligned against the
 * second pass), the exchange at two values per atomic: N = 5120, K = 5120 (three tiles a
 * workgroup) 11.0 against 12.2; N = 7168 (four) 12.0 against 13.9; N = 17408 (nine)
 * 18.8-19.1 against 19.3-19.7, and 12 rows 18.5 against 19.0; N = 40000, K = 4096 (twenty)
 * 29.6 against 28.8-29.3; N = 60000 (thirty) 42.5 against 38.9-39.3; N = 80000 (forty) 54.2
 * against 48.6-48.8. */
static constexpr int kAlignedMaxTiles = 12;
/* Most tiles a workgroup of a two-k-block aligned split holds at 9..16 rows, where four
 * publisher waves share the exchanges.  Measured on MI355X at K = 4096, 16 rows (us, aligned
 * against the second pass; 4-bit g64 unless stated): N = 40000 (twenty tiles a workgroup)
 * 26.05 against 28.13, 4-bit g32 30.71 against 32.52, 8-bit 39.72 against 39.75; N = 60000
 * (thirty) 37.51 against 38.88 but 4-bit g128 38.29 against 37.49; 13 rows, N = 80000
 * (forty), 4-bit g32: 56.45 against 55.77. */
static constexpr int kAligned16MaxTiles = 24;
/* Most tiles a workgroup of an aligned split of four or more k-blocks (the tree of exchanges)
 * holds at 9..16 rows where the tree needs no more k-blocks than the second pass's split. */
static constexpr int kAlignedRowsMaxTiles = 8;
/* Most k-blocks of an aligned split: from four on, each tile's parts meet over a tree of
 * exchanges (k-blocks - 1 of them, ceil(log2 k-blocks) deep), taken where the launch can place
 * a tile's workgroups on one XCD so that the exchanges run in its L2 (the whole chip,
 * workgroups per k-block a multiple of 8). */
static constexpr int kAlignedMaxKBlocks = 8;
static_assert(kAlignedMaxKBlocks <= 8, "the kernels' exchange tree has three levels");
#ifndef DFQ_LONG_CHAIN
#define DFQ_LONG_CHAIN 1
#endif
/* Smallest ring of partial slots a split shrinks to (beyond the units of one tile, which it
 * must hold to stay free of deadlock) before it takes more workgroups than CUs.  The ring's
 * size measured within noise down to this (N = 17408, K = 5120: 11 rows with 28 slots 16.7
 * against 16.9 us with 43), while the LDS it frees lets more shapes take one k-block and one
 * round of workgroups: 12 rows (14 slots) 16.7 against 18.2 us with two k-blocks, gate|up
 * N = 34816 at 12 rows 27.9 against 31.7. */
#ifndef DFQ_RING_SPARE
#define DFQ_RING_SPARE 4
#endif


bool make_plan(int M, int N, int K, int bits, int gs, int num_cus, size_t lds_max, Plan* pl) {
    const int kss = kss_for(bits, gs);
    if (M < 1 || M > 16 || N < 1 || K < kss || K % kss) return false;
    /* A chunk of 8 groups lets each lane fetch its row's scales with one 16-byte load; up to
     * 8 rows, 4-bit group 32 takes 16 groups (two loads) where K allows. */
    const int gps = kss / gs;
    const int mt = M > 8 ? 2 : 1;
    const int cg = mt == 1 ? chunk_groups(bits, gs) : 8;
    const int ch = (K % (kss * (cg / gps)) == 0)  ? cg / gps
                   : (K % (kss * (8 / gps)) == 0) ? 8 / gps
                                                  : 1;
    /* 9..16 rows: two row tiles per weight tile, built for 8-group chunks only */
    if (mt == 2 && ch == 1) return false;
    const int kch = kss * ch;
    const int chunks = K / kch;
    const int T = (N + 15) / 16;
    /* Fewest k-blocks (at least DFQ_MIN_KBLOCKS) whose largest x slice, plus the per-unit
     * partial slots of the split, fits in LDS.  The chunks spread over the k-blocks with
     * sizes differing by at most one. */
    /* The split into d k-blocks, starting from G0 workgroups per k-block (more when the LDS
     * ring would not fit); false when it does not fit at all. */
    auto split = [&](int d, int64_t G0, Plan* out) -> bool {
        const int ss_max = (chunks + d - 1) / d, ss_min = chunks / d;
        const int kr = ss_max * kch;
        if (!stage_fits(M, kr, gs, d)) return false;
        Plan p{};
        p.kss = kss;
        p.mt = mt;
        p.ch = ch;
        p.T = T;
        p.chunks = chunks;
        p.nkb = d;
        p.kr = kr;
        p.SS = ss_max;
        p.rs = 2 * kr + 16;
        p.xsum_off = ((M + 1) * p.rs + 15) & ~15;
        p.part_off = p.xsum_off + (kr / gs) * 32 * mt;
        /* Partial tiles live in a ring of 512*mt-byte LDS slots over the take order: a range's
         * whole length when it is short, else enough for the units in flight plus a few
         * tiles waiting for their sum (at least the units one tile can have in a range, which
         * keeps the ring free of deadlock), plus a 4-byte generation per slot and a counter
         * per tile.  Where even the smallest ring does not fit beside x and the output blocks,
         * whole rounds of workgroups (2, 3, ... per CU, one at a time) shorten the ranges: a
         * partial last round leaves its few workgroups running alone for a whole range.
         * Measured on MI355X at N = 151936, K = 5120 (us, against growing the workgroups an
         * eighth at a time with the largest ring): 9 rows 91.8 against 125.6, 10 rows 92.9
         * against 130.1, 12 rows 114.0 against 118.9, 16 rows 115.7 against 135.1. */
        const int64_t U = (int64_t)T * ss_max;
        int64_t G = std::min<int64_t>(std::max<int64_t>(1, G0), U);
        size_t need = 0;
        for (int64_t rounds = 2;; G = std::min<int64_t>(U, std::max<int64_t>(1, G0) * rounds++)) {
            const int64_t umax = U / G + ((U % G) ? 1 : 0);
            const int64_t ntl_max = (umax + ss_min - 1) / ss_min + 1;  // tiles a range touches
            /* the largest ring from 4 tiles + 24 units down to one tile + DFQ_RING_SPARE units
             * that fits: a smaller ring before more workgroups than CUs */
            const int64_t ring_hi = std::min<int64_t>(umax, 4 * ss_max + 24);
            const int64_t ring_lo = std::min<int64_t>(ring_hi, ss_max + DFQ_RING_SPARE);
            for (int64_t ring = ring_hi; ring >= ring_lo; --ring) {
                p.umax = (int)umax;
                p.ring = (int)ring;
                p.gen_off = p.part_off + (int)ring * 512 * mt;
                p.cnt_off = p.gen_off + (int)ring * 4;
                /* then each touched tile's finished sum, and 16 per-row 64-bit keys */
                p.tout_off =
                    (int)(((size_t)p.cnt_off + (size_t)(ntl_max + 2) * 4 + 15) & ~(size_t)15);
                p.key_off = p.tout_off + (int)ntl_max * 512 * mt;
                need = (size_t)p.key_off + 16 * 8;
                if (need <= lds_max) break;
            }
            if (need <= lds_max || G == U) break;
        }
        if (need > lds_max) return false;
        if (stage_items(M, kr, gs) > DFQ_STAGE_ITEMS(1) && (p.umax < 3 * ss_max || G > G0))
            return false;
        p.Gkb = (int)G;
        int nslot = 1;
        for (int ss : {ss_min, ss_max})
            for (int64_t t = 0; t < T; ++t) nslot = std::max(nslot, tile_owners(t, ss, G, T));
        p.nslot_kb = nslot;
        /* At most two parts per tile: the pair exchange inside the kernel.  More: plain slot
         * stores and the fixed-order second kernel. */
        p.reduce = d > 1 ? (d > 2 || nslot > 1) : nslot > 2;
        {
            const int64_t umax = p.umax, ntl_max = (umax + ss_min - 1) / ss_min + 1;
            p.burst = ntl_max >= kBurstTiles;
        }
        /* Ask for more than half the CU's LDS so that exactly one workgroup lands per CU. */
        const size_t want = std::max(need, lds_max / 2 + 256);
        p.lds_bytes = (int)std::min(want, lds_max);
        p.lds_need = (int)need;
        p.need_ws = d > 1 || nslot > 1;
        p.ws_bytes = p.need_ws ? (size_t)T * d * nslot * mt * 128 * 4 : 0;
        *out = p;
        return true;
    };
    /* dd = 2 or 3 k-blocks whose workgroups take whole tiles (an "aligned" split of G0
     * workgroups per k-block, at most one per tile): every tile then has one part per
     * k-block, finished by the pair exchange (a chain of two exchanges for three parts), so
     * no second pass is needed, at the price of up to one tile of imbalance between
     * workgroups. */
    auto split_aligned = [&](int dd, int64_t G0, Plan* out) -> bool {
        if (chunks < dd) return false;
        const int ss_max = (chunks + dd - 1) / dd;
        const int kr = ss_max * kch;
        if (!stage_fits(M, kr, gs, dd)) return false;
        int64_t G = std::min<int64_t>(std::max<int64_t>(1, G0), T);
        const int64_t tmax = (T + G - 1) / G;
        /* a multiple of 8 workgroups where that leaves the most tiles a workgroup takes as it
         * is (three k-blocks: 85 -> 80 at N = 5120), so that the launch can place each tile's
         * workgroups on one XCD */
        if ((G & 7) && G > 8 && (T + (G & ~7) - 1) / (G & ~7) == tmax) G &= ~7;
        Plan p{};
        p.kss = kss;
        p.mt = mt;
        p.ch = ch;
        p.T = T;
        p.chunks = chunks;
        p.nkb = dd;
        p.kr = kr;
        p.SS = ss_max;
        p.rs = 2 * kr + 16;
        p.xsum_off = ((M + 1) * p.rs + 15) & ~15;
        p.part_off = p.xsum_off + (kr / gs) * 32 * mt;
        p.umax = (int)(tmax * ss_max);
        p.ring = (int)std::min<int64_t>(p.umax, 4 * ss_max + 24);
        p.gen_off = p.part_off + p.ring * 512 * mt;
        p.cnt_off = p.gen_off + p.ring * 4;
        p.tout_off = (int)(((size_t)p.cnt_off + (size_t)(tmax + 2) * 4 + 15) & ~(size_t)15);
        p.key_off = p.tout_off + (int)tmax * 512 * mt;
        const size_t need = (size_t)p.key_off + 16 * 8;
        if (need > lds_max) return false;
        p.Gkb = (int)G;
        p.nslot_kb = 1;
        p.reduce = false;
        p.aligned = true;
        p.lds_bytes = (int)std::min(std::max(need, lds_max / 2 + 256), lds_max);
        p.lds_need = (int)need;
        p.need_ws = true;
        p.ws_bytes = (size_t)T * dd * mt * 128 * 4;
        *out = p;
        return true;
    };
    for (int d = std::min(DFQ_MIN_KBLOCKS, chunks); d <= chunks; ++d) {
        if (!split(d, num_cus / d, pl)) continue;
        /* Two or three k-blocks of stream-K ranges give tiles three or more parts (second
         * pass); whole tiles per workgroup give one per k-block, finished in the kernel by the
         * pair exchange, at the price of up to one tile of imbalance; taken where its LDS fits
         * (one output block per tile a workgroup holds) and a workgroup holds few enough
         * tiles (with one value per atomic the exchange lost from four tiles on: N = 17408 at
         * 16 rows, 24.4 against 20.7 us). */
        Plan al;
        const int64_t al_max = mt == 2 && d == 2 ? kAligned16MaxTiles : kAlignedMaxTiles;
        if (pl->reduce && (d == 2 || d == 3) && split_aligned(d, num_cus / d, &al) &&
            (T + al.Gkb - 1) / al.Gkb <= al_max) {
            *pl = al;
            return true;
        }
        /* From four k-blocks on, the first aligned split of d .. kAlignedMaxKBlocks k-blocks
         * that fits and whose launch can place each tile's workgroups on one XCD (the parts
         * then meet over a tree of exchanges in its L2): where it holds at most two tiles a
         * workgroup, or where the second pass's split needs more workgroups than the chip has
         * CUs (whole rounds of workgroups) and the aligned one deals every workgroup the same
         * tiles, at most kAlignedMaxTiles of them.  Measured on MI355X (us, against the
         * second pass's split, same box): N = 1024, K = 32768 at 8 rows (two tiles) 12.2
         * against 13.4; 16 rows at N = 5120, K = 17408 (eight k-blocks of ten tiles, against
         * 6 x 47 workgroups with the largest ring) 25.1 against 30.0, but 25.0 against 20.0
         * once the ring's shrinking fits that split in one round of 6 x 42.  Taken elsewhere
         * it lost: 12 rows at that shape (eight tiles, against 5 x 51 workgroups) 22.0
         * against 20.3, 8 rows at N = 5120, K = 32768 (eight tiles) 30.6 against 26.3; 9 rows
         * gained 0.3 us; 56 tiles a workgroup (16 rows, N = 28672, K = 16384, 4-bit g128)
         * 111.8 against 63.9, 68 tiles (11 rows, N = 34816) 134.1 against 76.5.
         * With four publisher waves, 9..16 rows also take it where it needs no more k-blocks
         * than the second pass's split and a workgroup holds at most 8 tiles (us, same
         * comparison, 4-bit g64): N = 5120, K = 17408 at 9 rows 16.86 against 18.15, 10 rows
         * 16.94 against 18.29, 12 rows 18.60 against 19.30, 13 rows 18.33 against 19.83, 15
         * rows 18.57 against 20.17; N = 4096, K = 16384 at 16 rows 16.32 against 18.24;
         * N = 7168, K = 14336 at 10 rows 18.39 against 19.80; g128 at 11 rows 17.37 against
         * 18.72; 8-bit at 12 rows 25.37 against 25.37.  With more k-blocks than the second
         * pass's split it lost: 16 rows at N = 5120 (eight k-blocks of ten tiles against six)
         * 20.76 against 20.52, 4-bit g32 at 10 rows (six against four) 22.05 against 21.31. */
        if (pl->reduce && d >= 4 && DFQ_LONG_CHAIN && num_cus == 256)
            for (int dd = d; dd <= std::min(kAlignedMaxKBlocks, chunks); ++dd) {
                if (!split_aligned(dd, num_cus / dd, &al) || al.Gkb % 8) continue;
                const int64_t tpw = (T + al.Gkb - 1) / al.Gkb;  // most tiles a workgroup
                if (tpw <= 2 || (mt == 2 && dd == d && tpw <= kAlignedRowsMaxTiles) ||
                    ((int64_t)pl->nkb * pl->Gkb > num_cus && T % al.Gkb == 0 &&
                     tpw <= kAlignedMaxTiles)) {
                    *pl = al;
                    return true;
                }
            }

        /* Few tiles (a narrow N): one k-block over every CU spreads each tile over more than
         * two workgroups, which needs the second pass.  Two k-blocks of one tile per
         * workgroup finish every tile with the pair exchange instead, and stage half of x,
         * at the price of fewer CUs; taken while a workgroup's share stays short. */
        Plan alt;
        if (pl->reduce && d == 1 && chunks >= 2 && 2 * T <= num_cus &&
            (chunks + 1) / 2 <= kShortSplitUnits && split(2, T, &alt) && !alt.reduce)
            *pl = alt;
        return true;
    }
    return false;
}

/* The split for a shape, from the context's cache; a shape with none is cached too (T == 0).
 * cache = false (the no-allocation path) looks in the cache, then in the context's fixed
 * table, and stores a split it had to compute in that table, which allocates nothing. */
static bool find_plan(dfq_ctx* ctx, int M, int N, int K, int bits, int gs, Plan* out,
                      bool cache = true) {
    PlanKey key{M, N, K, bits, gs};
    std::lock_guard<std::mutex> lk(ctx->mu);
    auto it = ctx->plans.find(key);
    if (it != ctx->plans.end()) {
        *out = it->second;
        return out->T > 0;
    }
    if (!cache)
        for (int i = 0; i < ctx->fixed_used; ++i)
            if (ctx->fixed_key[i] == key) {
                *out = ctx->fixed_plan[i];
                return out->T > 0;
            }
    Plan p;
    if (!make_plan(M, N, K, bits, gs, ctx->num_cus, ctx->lds_max, &p)) p = Plan{};
    if (cache) {
        ctx->plans.emplace(key, p);
    } else {
        const int slot = ctx->fixed_used < dfq_ctx::kFixedPlans
                             ? ctx->fixed_used++
                             : ctx->fixed_next++ % dfq_ctx::kFixedPlans;
        ctx->fixed_key[slot] = key;
        ctx->fixed_plan[slot] = p;
    }
    *out = p;
    return out->T > 0;
}

static dfq_status get_plan(dfq_ctx* ctx, int M, int N, int K, int bits, int gs, Plan* out,
                           bool cache = true) {
    if (!find_plan(ctx, M, N, K, bits, gs, out, cache))
        return fail(DFQ_ERR_UNSUPPORTED, "no work split for M=%d N=%d K=%d bits=%d gs=%d", M, N,
                    K, bits, gs);
    return DFQ_OK;
}

/* 9..16 rows run in one launch with two row tiles when the shape has such a split, else as
 * two launches of up to 8 rows over the same weights. */
static bool one_pass(dfq_ctx* ctx, int M, int N, int K, int bits, int gs, bool cache = true) {
    Plan p;
    return M <= 8 || find_plan(ctx, M, N, K, bits, gs, &p, cache);
}

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

dfq_status check_fast_args(const dfq_ctx* ctx, int M, int N, int K, int bits, int gs,
                           dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (M < 1 || N < 1 || K < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "M, N, K must be >= 1");
    if (M > 16) return fail(DFQ_ERR_UNSUPPORTED, "fast kernel handles M <= 16 (got %d)", M);
    if (bits != 4 && bits != 8) return fail(DFQ_ERR_UNSUPPORTED, "bits must be 4 or 8");
    if (gs != 32 && gs != 64 && gs != 128)
        return fail(DFQ_ERR_UNSUPPORTED, "group size must be 32, 64 or 128");
    if ((xdt != DFQ_BF16 && xdt != DFQ_F16) || sdt != xdt || ydt != xdt)
        return fail(DFQ_ERR_UNSUPPORTED, "fast kernel needs x, scales and y all bf16 or all fp16");
    const int kss = kss_for(bits, gs);
    if (K % kss) return fail(DFQ_ERR_UNSUPPORTED, "K=%d is not a multiple of %d", K, kss);
    if ((int64_t)N * K * bits / 8 >= (int64_t)1 << 31)
        return fail(DFQ_ERR_UNSUPPORTED, "weights must be smaller than 2 GiB");
    return DFQ_OK;
}

}  // namespace dfq

using namespace dfq;

extern "C" {

const char* dfq_last_error(void) { return g_last_error.c_str(); }

const char* dfq_status_string(dfq_status s) {
    switch (s) {
        case DFQ_OK: return "ok";
        case DFQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case DFQ_ERR_UNSUPPORTED: return "unsupported";
        case DFQ_ERR_WORKSPACE: return "workspace";
        case DFQ_ERR_HIP: return "hip error";
        case DFQ_ERR_NO_DEVICE: return "no device";
        case DFQ_ERR_STATE: return "bad state";
    }
    return "unknown";
}

int dfq_abi_version(void) { return DFQ_ABI_VERSION; }

dfq_status dfq_init(int device, dfq_ctx** out) {
    if (!out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null out");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) return fail(DFQ_ERR_NO_DEVICE, "no HIP device visible");
    if (device < 0 || device >= count)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "device %d out of range (%d devices)", device, count);
    DeviceGuard g(device);
    if (!g.ok) return fail(DFQ_ERR_HIP, "hipSetDevice(%d) failed", device);
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess)
        return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(DFQ_ERR_NO_DEVICE, "device %d is %s, the code object is built for gfx950",
                    device, prop.gcnArchName);
    auto* ctx = new dfq_ctx();
    ctx->device = device;
    ctx->num_cus = prop.multiProcessorCount;
    ctx->lds_max = prop.sharedMemPerBlock;
    if ((e = hipModuleLoadData(&ctx->module, dfq_hsaco_begin)) != hipSuccess) {
        delete ctx;
        return hip_fail(e, "hipModuleLoadData(gfx950 code object)");
    }
    static const int kBits[2] = {4, 8};
    static const int kGs[3] = {32, 64, 128};
    static const char* kDt[2] = {"bf16", "f16"};
    static const char* kCh[2] = {"c1", "c8"};
    for (int b = 0; b < 2; ++b)
        for (int g2 = 0; g2 < 3; ++g2)
            for (int d = 0; d < 2; ++d)
                for (int c = 0; c < 2; ++c) {
                    char name[64];
                    snprintf(name, sizeof name, "dfq_qmm_mt8_b%d_g%d_%s_%s", kBits[b], kGs[g2],
                             kDt[d], kCh[c]);
                    if ((e = hipModuleGetFunction(&ctx->mt8[b][g2][d][c], ctx->module, name)) !=
                        hipSuccess) {
                        (void)hipModuleUnload(ctx->module);
                        delete ctx;
                        return hip_fail(e, name);
                    }
                    snprintf(name, sizeof name, "dfq_qmv_b%d_g%d_%s_m%d", kBits[b], kGs[g2],
                             kDt[d], c == 0 ? 1 : 4);
                    if ((e = hipModuleGetFunction(&ctx->qmv[b][g2][d][c], ctx->module, name)) !=
                        hipSuccess) {
                        (void)hipModuleUnload(ctx->module);
                        delete ctx;
                        return hip_fail(e, name);
                    }
                    if (c == 0) continue;
                    snprintf(name, sizeof name, "dfq_qmm_mt16_b%d_g%d_%s_c8", kBits[b], kGs[g2],
                             kDt[d]);
                    if ((e = hipModuleGetFunction(&ctx->mt16[b][g2][d], ctx->module, name)) !=
                        hipSuccess) {
                        (void)hipModuleUnload(ctx->module);
                        delete ctx;
                        return hip_fail(e, name);
                    }
                    for (int t = 0; t < 2; ++t) {
                        hipFunction_t* dst[3] = {&ctx->am[b][g2][d][t], &ctx->pk[b][g2][d][t],
                                                 &ctx->pk_am[b][g2][d][t]};
                        static const char* kSfx[3] = {"_am", "_pk", "_am_pk"};
                        for (int f = 0; f < 3; ++f) {
                            snprintf(name, sizeof name, "dfq_qmm_mt%d_b%d_g%d_%s_c8%s",
                                     8 * (t + 1), kBits[b], kGs[g2], kDt[d], kSfx[f]);
                            if ((e = hipModuleGetFunction(dst[f], ctx->module, name)) !=
                                hipSuccess) {
                                (void)hipModuleUnload(ctx->module);
                                delete ctx;
                                return hip_fail(e, name);
                            }
                        }
                    }
                }
    for (int d = 0; d < 2; ++d)
        for (int f = 0; f < 4; ++f) {
            static const char* kSfx[4] = {"", "_am", "_pk", "_am_pk"};
            char name[64];
            snprintf(name, sizeof name, "dfq_qmm_mt8_b4_g32_%s_c16%s", kDt[d], kSfx[f]);
            if ((e = hipModuleGetFunction(&ctx->c16[d][f], ctx->module, name)) != hipSuccess) {
                (void)hipModuleUnload(ctx->module);
                delete ctx;
                return hip_fail(e, name);
            }
        }
    if ((e = hipModuleGetFunction(&ctx->generic, ctx->module, "dfq_qmm_generic")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->reduce[0], ctx->module, "dfq_qmm_reduce_bf16")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->reduce[1], ctx->module, "dfq_qmm_reduce_f16")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->silu_mul[0], ctx->module, "dfq_silu_mul_bf16")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->silu_mul[1], ctx->module, "dfq_silu_mul_f16")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->argmax_accept[0], ctx->module, "dfq_argmax_accept_bf16")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->argmax_accept[1], ctx->module, "dfq_argmax_accept_f16")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->fill, ctx->module, "dfq_fill_u32")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->pack, ctx->module, "dfq_pack_weights")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->read_stream, ctx->module, "dfq_read_stream")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->read_units, ctx->module, "dfq_read_units_b4_g64")) != hipSuccess ||
        (e = hipModuleGetFunction(&ctx->read_units_packed, ctx->module,
                                  "dfq_read_units_packed_b4_g64")) != hipSuccess) {
        (void)hipModuleUnload(ctx->module);
        delete ctx;
        return hip_fail(e, "hipModuleGetFunction");
    }
    dfq_status st = scratch_setup(device, &ctx->scratch);
    if (st != DFQ_OK) {
        (void)hipModuleUnload(ctx->module);
        delete ctx;
        return st;
    }
    *out = ctx;
    return DFQ_OK;
}

dfq_status dfq_destroy(dfq_ctx* ctx) {
    if (!ctx) return DFQ_OK;
    {
        DeviceGuard g(ctx->device);
        if (ctx->module) (void)hipModuleUnload(ctx->module);
    }
    delete ctx;
    return DFQ_OK;
}

int dfq_num_cus(const dfq_ctx* ctx) { return ctx ? ctx->num_cus : 0; }

/* ---- memory and streams ----------------------------------------------------------- */

dfq_status dfq_malloc(dfq_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    DeviceGuard g(ctx->device);
    hipError_t e = hipMalloc(out, bytes ? bytes : 1);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipMalloc");
}

dfq_status dfq_free(dfq_ctx* ctx, void* ptr) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!ptr) return DFQ_OK;
    DeviceGuard g(ctx->device);
    hipError_t e = hipFree(ptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipFree");
}

dfq_status dfq_memcpy_h2d(dfq_ctx* ctx, void* dst, const void* src, size_t bytes, void* stream) {
    if (!ctx || (bytes && (!dst || !src))) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    DeviceGuard g(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipMemcpyAsync(H2D)");
}

dfq_status dfq_memcpy_d2h(dfq_ctx* ctx, void* dst, const void* src, size_t bytes, void* stream) {
    if (!ctx || (bytes && (!dst || !src))) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    DeviceGuard g(ctx->device);
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream);
    if (e == hipSuccess) e = hipStreamSynchronize((hipStream_t)stream);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipMemcpyAsync(D2H)");
}

dfq_status dfq_stream_create(dfq_ctx* ctx, void** stream) {
    if (!ctx || !stream) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    DeviceGuard g(ctx->device);
    hipStream_t s = nullptr;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
    *stream = s;
    return DFQ_OK;
}

dfq_status dfq_stream_destroy(dfq_ctx* ctx, void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!stream) return DFQ_OK;
    DeviceGuard g(ctx->device);
    hipError_t e = hipStreamDestroy((hipStream_t)stream);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipStreamDestroy");
}

dfq_status dfq_stream_sync(dfq_ctx* ctx, void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    DeviceGuard g(ctx->device);
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipStreamSynchronize");
}

/* ---- eligibility -------------------------------------------------------------------- */

int dfq_is_eligible(int out_features, int in_features, int bits, int group_size,
                    int mode_affine, int has_biases) {
    if (!mode_affine || !has_biases) return 0;
    if ((bits != 4 && bits != 8) || group_size != DFQ_REQUIRED_GROUP_SIZE) return 0;
    return out_features >= DFQ_MINIMUM_OUTPUT_FEATURES &&
           in_features % DFQ_INPUT_FEATURE_MULTIPLE == 0;
}

int dfq_tiles_for(int rows) { return rows <= DFQ_ROWS_PER_TILE ? 1 : 2; }

int dfq_qmm_supported(const dfq_ctx* ctx, int M, int N, int K, int bits, int gs,
                      dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt) {
    std::string saved = g_last_error;
    dfq_status s = check_fast_args(ctx, M, N, K, bits, gs, xdt, sdt, ydt);
    int ok = s == DFQ_OK;
    if (ok) {
        Plan p;
        ok = make_plan(M, N, K, bits, gs, ctx->num_cus, ctx->lds_max, &p) ||
             (M > 8 && make_plan(8, N, K, bits, gs, ctx->num_cus, ctx->lds_max, &p) &&
              make_plan(M - 8, N, K, bits, gs, ctx->num_cus, ctx->lds_max, &p));
    }
    g_last_error = saved;
    return ok;
}

/* ---- the matmul ----------------------------------------------------------------------- */

/* Workspace of a checked shape: one launch's, or the larger of the two row passes'. */
static dfq_status workspace_need(dfq_ctx* ctx, int M, int N, int K, int bits, int gs,
                                 bool cache, size_t* bytes) {
    dfq_status s;
    Plan p;
    if (one_pass(ctx, M, N, K, bits, gs, cache)) {
        if ((s = get_plan(ctx, M, N, K, bits, gs, &p, cache))) return s;
        *bytes = p.ws_bytes;
        return DFQ_OK;
    }
    if ((s = get_plan(ctx, 8, N, K, bits, gs, &p, cache))) return s;
    size_t need = p.ws_bytes;
    if ((s = get_plan(ctx, M - 8, N, K, bits, gs, &p, cache))) return s;
    *bytes = std::max(need, p.ws_bytes);
    return DFQ_OK;
}

dfq_status dfq_qmm_workspace_bytes(dfq_ctx* ctx, int M, int N, int K, int bits, int gs,
                                   size_t* bytes) {
    if (!bytes) return fail(DFQ_ERR_INVALID_ARGUMENT, "null bytes");
    *bytes = 0;
    dfq_status s = check_fast_args(ctx, M, N, K, bits, gs, DFQ_BF16, DFQ_BF16, DFQ_BF16);
    if (s) return s;
    return workspace_need(ctx, M, N, K, bits, gs, true, bytes);
}

dfq_status dfq_workspace_clear(dfq_ctx* ctx, void* ws, size_t bytes, void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!bytes) return DFQ_OK;
    if (!ws || !aligned(ws, 4) || bytes % 4)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "workspace must be 4-byte aligned and sized");
    DeviceGuard g(ctx->device);
    uint32_t* p = (uint32_t*)ws;
    uint32_t v = 0;
    uint64_t count = bytes / 4;
    void* args[] = {&p, &v, &count};
    unsigned grid = (unsigned)std::min<uint64_t>((count + 255) / 256, 4096);
    hipError_t e = hipModuleLaunchKernel(ctx->fill, grid, 1, 1, 256, 1, 1, 0,
                                         (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_fill_u32");
}

#ifndef DFQ_XCD_PAIR
#define DFQ_XCD_PAIR 1
#endif

/* The kernel argument of one call of a plan (ws: the workspace, NULL when none is needed). */
static QmmParams fill_params(const Plan& pl, const void* x, const uint32_t* w,
                             const void* scales, const void* biases, const void* lbias, void* y,
                             int M, int N, int K, int bits, int gs, void* ws) {
    QmmParams p{};
    p.x = x;
    p.w = w;
    p.scales = scales;
    p.biases = biases;
    p.lbias = lbias;
    p.y = y;
    if (pl.need_ws && ws) p.slots = (float*)ws;
    p.M = M;
    p.N = N;
    p.K = K;
    p.mt = pl.mt;
    p.T = pl.T;
    p.chunks = pl.chunks;
    p.nkb = pl.nkb;
    p.Gkb = pl.Gkb;
    p.nslot_kb = pl.nslot_kb;
    p.reduce = pl.reduce ? 1 : 0;
    p.aligned = pl.aligned ? 1 : 0;
    p.lds_row_stride = pl.rs;
    p.lds_xsum_off = pl.xsum_off;
    p.lds_part_off = pl.part_off;
    p.lds_cnt_off = pl.cnt_off;
    p.lds_gen_off = pl.gen_off;
    p.lds_tout_off = pl.tout_off;
    p.lds_key_off = pl.key_off;
    p.burst = pl.burst ? 1 : 0;
    p.umax = pl.umax;
    p.ring = pl.ring;
    p.w_bytes = (uint32_t)((int64_t)N * K * bits / 8);
    p.s_bytes = (uint32_t)((int64_t)N * (K / gs) * 2);
    return p;
}

/* The greedy-accept block of a fused LM-head launch (see dfq_qmm_argmax_accept). */
struct AcceptArgs {
    uint64_t* keys = nullptr;
    uint32_t* count = nullptr;
    const int32_t* proposals = nullptr;
    int32_t* tokens = nullptr;
    int32_t* accepted = nullptr;
};

static dfq_status launch_mt8(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                             const void* biases, const void* lbias, void* y, int M, int N, int K,
                             int bits, int gs, dfq_dtype dt, void* ws, size_t wsb,
                             hipStream_t stream, int epi = 0, bool cache = true,
                             const AcceptArgs* acc = nullptr, bool packed = false) {
    Plan pl;
    dfq_status s = get_plan(ctx, M, N, K, bits, gs, &pl, cache);
    if (s) return s;
    if (packed && (pl.ch == 1 || K % (chunk_groups(bits, gs) * gs)))
        return fail(DFQ_ERR_UNSUPPORTED,
                    "the packed layout holds chunks of %d groups: K=%d is not a multiple of %d",
                    chunk_groups(bits, gs), K, chunk_groups(bits, gs) * gs);
    if (acc && (pl.reduce || epi || pl.ch == 1))
        return fail(DFQ_ERR_STATE,
                    "greedy-accept mode needs 8-group chunks and a split without a second pass");
    if (pl.need_ws) {
        if (!ws || wsb < pl.ws_bytes)
            return fail(DFQ_ERR_WORKSPACE, "workspace of %zu bytes needed (got %zu)", pl.ws_bytes,
                        ws ? wsb : (size_t)0);
        if (!aligned(ws, 256)) return fail(DFQ_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    }
    QmmParams p = fill_params(pl, x, w, scales, biases, lbias, y, M, N, K, bits, gs, ws);
    p.epi = epi;
    /* On the whole chip (256 CUs: eight XCDs, dealt workgroups round-robin) a tile whose two
     * parts come from workgroups on one XCD is exchanged through that XCD's L2.  Splits whose
     * tiles have one part per k-block at the same range index (aligned, or ranges of the same
     * whole tiles in every k-block), with workgroup counts per k-block that the eight XCDs
     * share evenly, place each tile's workgroups on one XCD. */
    p.xcd8 = (DFQ_XCD_PAIR && ctx->num_cus == 256) ? 1 : 0;
    p.xcd_pair = (p.xcd8 && pl.nkb > 1 && !pl.reduce && (pl.aligned || pl.T % pl.Gkb == 0) &&
                  pl.Gkb % 8 == 0)
                     ? 1
                     : 0;
    if (acc) {
        p.am_keys = acc->keys;
        p.am_count = acc->count;
        p.am_proposals = acc->proposals;
        p.am_tokens = acc->tokens;
        p.am_accepted = acc->accepted;
    }
    const int bi = bits == 4 ? 0 : 1;
    const int gi = gs == 32 ? 0 : gs == 64 ? 1 : 2;
    const int di = dt == DFQ_BF16 ? 0 : 1;
    void* args[] = {&p};
    const int ci = pl.ch > 1 ? 1 : 0;
    const bool c16 = pl.ch * (pl.kss / gs) == 16;  // 4-bit group 32, up to 8 rows
    hipFunction_t fn = c16      ? ctx->c16[di][(acc ? 1 : 0) + (packed ? 2 : 0)]
                       : packed ? (acc ? ctx->pk_am[bi][gi][di][pl.mt - 1]
                                       : ctx->pk[bi][gi][di][pl.mt - 1])
                       : acc        ? ctx->am[bi][gi][di][pl.mt - 1]
                       : pl.mt == 2 ? ctx->mt16[bi][gi][di]
                                    : ctx->mt8[bi][gi][di][ci];
    hipError_t e = hipModuleLaunchKernel(fn, (unsigned)(pl.nkb * pl.Gkb), 1, 1, kBlockThreads, 1,
                                         1, (unsigned)pl.lds_bytes, stream, args, nullptr);
    if (e != hipSuccess) return hip_fail(e, "launch dfq_qmm_mt8");
    if (pl.reduce) {
        e = hipModuleLaunchKernel(ctx->reduce[di], (unsigned)pl.T, 1, 1, 64, 1, 1, 0, stream,
                                  args, nullptr);
        if (e != hipSuccess) return hip_fail(e, "launch dfq_qmm_reduce");
    }
    return DFQ_OK;
}


static dfq_status qmm_any(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const void* lbias, void* y, int M, int N, int K,
                          int bits, int gs, dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt, void* ws,
                          size_t wsb, void* stream, int epi, bool cache = true,
                          bool packed = false);

dfq_status dfq_qmm(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                   const void* biases, const void* lbias, void* y, int M, int N, int K, int bits,
                   int gs, dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt, void* ws, size_t wsb,
                   void* stream) {
    return qmm_any(ctx, x, w, scales, biases, lbias, y, M, N, K, bits, gs, xdt, sdt, ydt, ws, wsb,
                   stream, 0);
}

dfq_status dfq_qmm_noalloc(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, const void* lbias, void* y, int M, int N, int K,
                           int bits, int gs, dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt,
                           void* stream) {
    dfq_status s = check_fast_args(ctx, M, N, K, bits, gs, xdt, sdt, ydt);
    if (s) return s;
    if (!ctx->scratch) return fail(DFQ_ERR_STATE, "the context has no scratch");
    /* the shape's split is looked up, or computed, without storing it: no allocation */
    size_t need = 0;
    if ((s = workspace_need(ctx, M, N, K, bits, gs, false, &need))) return s;
    if (need > DFQ_SCRATCH_MAX_BYTES)
        return fail(DFQ_ERR_WORKSPACE,
                    "M=%d N=%d K=%d needs %zu bytes of workspace; the fixed scratch of "
                    "dfq_qmm_noalloc holds %zu (use dfq_qmm with a workspace)",
                    M, N, K, need, (size_t)DFQ_SCRATCH_MAX_BYTES);
    s = qmm_any(ctx, x, w, scales, biases, lbias, y, M, N, K, bits, gs, xdt, sdt, ydt,
                ctx->scratch, DFQ_SCRATCH_MAX_BYTES, stream, 0, false);
    if (s && need) {
        /* A call of several launches that failed after its first one was queued (the second
         * pass, or the second 8-row pass) can leave partial sums in the scratch, which every
         * later call on this GPU would read as exchange words: clear what the shape uses,
         * behind whatever was queued.  The first error is the one reported. */
        const std::string first = g_last_error;
        DeviceGuard g(ctx->device);
        uint32_t* p = (uint32_t*)ctx->scratch;
        uint32_t v = 0;
        uint64_t count = (need + 3) / 4;
        void* args[] = {&p, &v, &count};
        unsigned grid = (unsigned)std::min<uint64_t>((count + 255) / 256, 4096);
        (void)hipModuleLaunchKernel(ctx->fill, grid, 1, 1, 256, 1, 1, 0, (hipStream_t)stream,
                                    args, nullptr);
        g_last_error = first;
    }
    return s;
}

/* ---- the packed layout -------------------------------------------------------------- */

dfq_status dfq_packed_bytes(int N, int K, int bits, int gs, size_t* bytes) {
    if (!bytes) return fail(DFQ_ERR_INVALID_ARGUMENT, "null bytes");
    *bytes = 0;
    if (N < 1 || K < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "N and K must be >= 1");
    if (bits != 4 && bits != 8) return fail(DFQ_ERR_UNSUPPORTED, "bits must be 4 or 8");
    if (gs != 32 && gs != 64 && gs != 128)
        return fail(DFQ_ERR_UNSUPPORTED, "group size must be 32, 64 or 128");
    const int cg = chunk_groups(bits, gs);
    if (K % (cg * gs))
        return fail(DFQ_ERR_UNSUPPORTED,
                    "the packed layout holds chunks of %d groups: K=%d is not a multiple of %d",
                    cg, K, cg * gs);
    const size_t unit = (size_t)16 * cg * gs * bits / 8 + 512 * (cg / 8);
    *bytes = (size_t)((N + 15) / 16) * (K / (cg * gs)) * unit;
    return DFQ_OK;
}

dfq_status dfq_pack_weights(dfq_ctx* ctx, const uint32_t* w, const void* scales,
                            const void* biases, int N, int K, int bits, int gs, void* packed,
                            void* stream) {
    if (!ctx || !w || !scales || !biases || !packed)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    size_t bytes = 0;
    dfq_status s = dfq_packed_bytes(N, K, bits, gs, &bytes);
    if (s) return s;
    if (!aligned(w, 16) || !aligned(scales, 16) || !aligned(biases, 16) || !aligned(packed, 256))
        return fail(DFQ_ERR_INVALID_ARGUMENT,
                    "w, scales and biases must be 16-byte aligned, packed 256-byte");
    DeviceGuard g(ctx->device);
    uint64_t pieces = bytes / 16;
    void* args[] = {(void*)&w, (void*)&scales, (void*)&biases, &packed, &N, &K, &bits, &gs,
                    &pieces};
    const unsigned grid = (unsigned)std::min<uint64_t>((pieces + 255) / 256, 65536);
    hipError_t e = hipModuleLaunchKernel(ctx->pack, grid, 1, 1, 256, 1, 1, 0,
                                         (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_pack_weights");
}

dfq_status dfq_qmm_packed(dfq_ctx* ctx, const void* x, const void* packed, const void* lbias,
                          void* y, int M, int N, int K, int bits, int gs, dfq_dtype dt, void* ws,
                          size_t wsb, void* stream) {
    return qmm_any(ctx, x, (const uint32_t*)packed, nullptr, nullptr, lbias, y, M, N, K, bits,
                   gs, dt, dt, dt, ws, wsb, stream, 0, true, true);
}

dfq_status dfq_qmm_silu_gate_up_packed(dfq_ctx* ctx, const void* x, const void* packed_gu,
                                       const void* linear_bias_gu, void* h, int M, int H, int K,
                                       int bits, int gs, dfq_dtype dtype, void* ws, size_t wsb,
                                       void* stream) {
    if (H < 8 || H % 8)
        return fail(DFQ_ERR_UNSUPPORTED, "the gate|up epilogue needs H a multiple of 8 (got %d)", H);
    return qmm_any(ctx, x, (const uint32_t*)packed_gu, nullptr, nullptr, linear_bias_gu, h, M,
                   2 * H, K, bits, gs, dtype, dtype, dtype, ws, wsb, stream, 1, true, true);
}

dfq_status dfq_qmm_silu_gate_up(dfq_ctx* ctx, const void* x, const uint32_t* w_gu,
                                const void* scales_gu, const void* biases_gu,
                                const void* linear_bias_gu, void* h, int M, int H, int K,
                                int bits, int gs, dfq_dtype dtype, void* ws, size_t wsb,
                                void* stream) {
    if (H < 8 || H % 8)
        return fail(DFQ_ERR_UNSUPPORTED, "the gate|up epilogue needs H a multiple of 8 (got %d)", H);
    return qmm_any(ctx, x, w_gu, scales_gu, biases_gu, linear_bias_gu, h, M, 2 * H, K, bits, gs,
                   dtype, dtype, dtype, ws, wsb, stream, 1);
}

dfq_status dfq_interleave_gate_up(dfq_ctx* ctx, const void* gate, const void* up, void* out,
                                  int H, size_t row_bytes, void* stream) {
    if (!ctx || !gate || !up || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    if (H < 8 || H % 8 || !row_bytes)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "H must be a positive multiple of 8");
    DeviceGuard g(ctx->device);
    /* blocks of 8 rows: gate rows 8b.. to out rows 16b.., up rows 8b.. to out rows 16b+8.. */
    const size_t blk = 8 * row_bytes;
    hipError_t e = hipMemcpy2DAsync(out, 2 * blk, gate, blk, blk, (size_t)(H / 8),
                                     hipMemcpyDeviceToDevice, (hipStream_t)stream);
    if (e == hipSuccess)
        e = hipMemcpy2DAsync((char*)out + blk, 2 * blk, up, blk, blk, (size_t)(H / 8),
                             hipMemcpyDeviceToDevice, (hipStream_t)stream);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "interleave gate|up");
}

static dfq_status qmm_any(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const void* lbias, void* y, int M, int N, int K,
                          int bits, int gs, dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt, void* ws,
                          size_t wsb, void* stream, int epi, bool cache, bool packed) {
    dfq_status s = check_fast_args(ctx, M, N, K, bits, gs, xdt, sdt, ydt);
    if (s) return s;
    if (!x || !w || (!packed && (!scales || !biases)) || !y)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "null x, w, scales, biases or y");
    if (!aligned(x, 16) || !aligned(w, packed ? 256 : 16) ||
        (!packed && (!aligned(scales, 4) || !aligned(biases, 4))) || !aligned(y, 2) ||
        (lbias && !aligned(lbias, 2)))
        return fail(DFQ_ERR_INVALID_ARGUMENT,
                    "x and w must be 16-byte aligned (a packed weight 256-byte), scales/biases "
                    "4-byte aligned");
    DeviceGuard g(ctx->device);
    const size_t esz = 2;
    if (one_pass(ctx, M, N, K, bits, gs, cache))
        return launch_mt8(ctx, x, w, scales, biases, lbias, y, M, N, K, bits, gs, xdt, ws, wsb,
                          (hipStream_t)stream, epi, cache, nullptr, packed);
    if (packed)
        return fail(DFQ_ERR_UNSUPPORTED,
                    "the packed layout holds chunks of %d groups: K=%d is not a multiple of %d",
                    chunk_groups(bits, gs), K, chunk_groups(bits, gs) * gs);
    /* 9..16 rows with one-super-step chunks: two passes of up to 8 rows over the weights. */
    const size_t ypitch = (size_t)(epi ? N / 2 : N) * esz;
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mc = std::min(8, M - m0);
        s = launch_mt8(ctx, (const char*)x + (size_t)m0 * K * esz, w, scales, biases, lbias,
                       (char*)y + (size_t)m0 * ypitch, mc, N, K, bits, gs, xdt, ws, wsb,
                       (hipStream_t)stream, epi, cache);
        if (s) return s;
    }
    return DFQ_OK;
}

dfq_status dfq_silu_mul(dfq_ctx* ctx, const void* gu, void* h, int M, int N, dfq_dtype dtype,
                        void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!gu || !h) return fail(DFQ_ERR_INVALID_ARGUMENT, "null gu or h");
    if (M < 1 || N < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "M and N must be positive");
    if (dtype != DFQ_BF16 && dtype != DFQ_F16)
        return fail(DFQ_ERR_UNSUPPORTED, "silu_mul takes bf16 or fp16");
    if (!aligned(gu, 2) || !aligned(h, 2))
        return fail(DFQ_ERR_INVALID_ARGUMENT, "gu and h must be 2-byte aligned");
    DeviceGuard g(ctx->device);
    const uint64_t total = (uint64_t)M * N;
    unsigned grid = (unsigned)std::min<uint64_t>((total + 255) / 256, 8192);
    void* args[] = {(void*)&gu, &h, &M, &N};
    hipError_t e = hipModuleLaunchKernel(ctx->silu_mul[dtype == DFQ_BF16 ? 0 : 1], grid, 1, 1,
                                         256, 1, 1, 0, (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_silu_mul");
}

dfq_status dfq_argmax_accept_workspace_bytes(int M, size_t* bytes) {
    if (!bytes) return fail(DFQ_ERR_INVALID_ARGUMENT, "null bytes");
    if (M < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "M must be positive");
    /* one 64-bit key per row, then the arrival counter */
    *bytes = ((size_t)M * 8 + 4 + 255) & ~(size_t)255;
    return DFQ_OK;
}

dfq_status dfq_argmax_accept(dfq_ctx* ctx, const void* logits, int M, int V, dfq_dtype dtype,
                             const int32_t* proposals, int32_t* tokens, int32_t* accepted,
                             void* ws, size_t wsb, void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!logits) return fail(DFQ_ERR_INVALID_ARGUMENT, "null logits");
    if (M < 1 || V < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "M and V must be positive");
    if ((int64_t)V > 0x7fffffff / 2) return fail(DFQ_ERR_UNSUPPORTED, "V too large");
    if (dtype != DFQ_BF16 && dtype != DFQ_F16)
        return fail(DFQ_ERR_UNSUPPORTED, "argmax_accept takes bf16 or fp16 logits");
    size_t need = 0;
    dfq_argmax_accept_workspace_bytes(M, &need);
    if (!ws || wsb < need)
        return fail(DFQ_ERR_WORKSPACE, "workspace of %zu bytes needed (got %zu)", need,
                    ws ? wsb : (size_t)0);
    if (!aligned(ws, 8) || !aligned(logits, 2))
        return fail(DFQ_ERR_INVALID_ARGUMENT, "workspace must be 8-byte aligned");
    DeviceGuard g(ctx->device);
    const int64_t per_row = ((int64_t)V + DFQ_ACCEPT_CHUNK - 1) / DFQ_ACCEPT_CHUNK;
    if ((int64_t)M * per_row > 0x7fffffff) return fail(DFQ_ERR_UNSUPPORTED, "grid too large");
    uint64_t* keys = (uint64_t*)ws;
    uint32_t* counter = (uint32_t*)((char*)ws + (size_t)M * 8);
    void* args[] = {(void*)&logits, &M, &V, (void*)&proposals, &tokens, &accepted, &keys,
                    &counter};
    hipError_t e = hipModuleLaunchKernel(ctx->argmax_accept[dtype == DFQ_BF16 ? 0 : 1],
                                         (unsigned)(M * per_row), 1, 1, 256, 1, 1, 0,
                                         (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_argmax_accept");
}

/* Workspace of dfq_qmm_argmax_accept: the qmm's, then the keys ([16][M] x 8 bytes) and 17
 * arrival counters on 128-byte lines, then, for a split with a second pass, room for the
 * logits. */
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
static constexpr size_t kAcceptCountBytes = 17 * 128;

static dfq_status qmm_accept_layout(dfq_ctx* ctx, int M, int V, int K, int bits, int gs,
                                    bool* fused, size_t* qmm_ws, size_t* total) {
    dfq_status s = check_fast_args(ctx, M, V, K, bits, gs, DFQ_BF16, DFQ_BF16, DFQ_BF16);
    if (s) return s;
    size_t need = 0;
    if ((s = workspace_need(ctx, M, V, K, bits, gs, true, &need))) return s;
    Plan pl;
    *fused = one_pass(ctx, M, V, K, bits, gs) && get_plan(ctx, M, V, K, bits, gs, &pl) == DFQ_OK &&
             !pl.reduce && pl.ch > 1;
    *qmm_ws = align256(need);
    *total = *qmm_ws + align256((size_t)16 * M * 8) + align256(kAcceptCountBytes);
    if (!*fused) *total += align256((size_t)M * V * 2);
    return DFQ_OK;
}

dfq_status dfq_qmm_argmax_accept_workspace_bytes(dfq_ctx* ctx, int M, int V, int K, int bits,
                                                 int gs, size_t* bytes) {
    if (!bytes) return fail(DFQ_ERR_INVALID_ARGUMENT, "null bytes");
    *bytes = 0;
    bool fused;
    size_t qws;
    return qmm_accept_layout(ctx, M, V, K, bits, gs, &fused, &qws, bytes);
}

static dfq_status qmm_argmax_accept(dfq_ctx* ctx, const void* x, const uint32_t* w,
                                    const void* scales, const void* biases, const void* lbias,
                                    void* logits, int M, int V, int K, int bits, int gs,
                                    dfq_dtype dt, const int32_t* proposals, int32_t* tokens,
                                    int32_t* accepted, void* ws, size_t wsb, void* stream,
                                    bool packed) {
    dfq_status s = check_fast_args(ctx, M, V, K, bits, gs, dt, dt, dt);
    if (s) return s;
    if (!x || !w || (!packed && (!scales || !biases)))
        return fail(DFQ_ERR_INVALID_ARGUMENT, "null x, w, scales or biases");
    if (!aligned(x, 16) || !aligned(w, packed ? 256 : 16) ||
        (!packed && (!aligned(scales, 4) || !aligned(biases, 4))) ||
        (logits && !aligned(logits, 2)) || (lbias && !aligned(lbias, 2)))
        return fail(DFQ_ERR_INVALID_ARGUMENT,
                    "x and w must be 16-byte aligned (a packed weight 256-byte), scales/biases "
                    "4-byte aligned");
    bool fused;
    size_t qws, total;
    if ((s = qmm_accept_layout(ctx, M, V, K, bits, gs, &fused, &qws, &total))) return s;
    if (!ws || wsb < total)
        return fail(DFQ_ERR_WORKSPACE, "workspace of %zu bytes needed (got %zu)", total,
                    ws ? wsb : (size_t)0);
    if (!aligned(ws, 256)) return fail(DFQ_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    DeviceGuard g(ctx->device);
    char* base = (char*)ws;
    uint64_t* keys = (uint64_t*)(base + qws);
    uint32_t* count = (uint32_t*)(base + qws + align256((size_t)16 * M * 8));
    if (fused) {
        AcceptArgs acc;
        acc.keys = keys;
        acc.count = count;
        acc.proposals = proposals;
        acc.tokens = tokens;
        acc.accepted = accepted;
        return launch_mt8(ctx, x, w, scales, biases, lbias, logits, M, V, K, bits, gs, dt, ws,
                          qws, (hipStream_t)stream, 0, true, &acc, packed);
    }
    /* a split with a second pass: the logits first (to `logits` or the workspace), then the
     * accept kernel over them, its keys and counter in the accept region */
    void* lg = logits ? logits
                      : (void*)(base + qws + align256((size_t)16 * M * 8) +
                                align256(kAcceptCountBytes));
    if ((s = qmm_any(ctx, x, w, scales, biases, lbias, lg, M, V, K, bits, gs, dt, dt, dt, ws,
                     qws, stream, 0, true, packed)))
        return s;
    return dfq_argmax_accept(ctx, lg, M, V, dt, proposals, tokens, accepted, keys,
                             align256((size_t)16 * M * 8) + align256(kAcceptCountBytes), stream);
}

dfq_status dfq_qmm_argmax_accept(dfq_ctx* ctx, const void* x, const uint32_t* w,
                                 const void* scales, const void* biases, const void* lbias,
                                 void* logits, int M, int V, int K, int bits, int gs,
                                 dfq_dtype dt, const int32_t* proposals, int32_t* tokens,
                                 int32_t* accepted, void* ws, size_t wsb, void* stream) {
    return qmm_argmax_accept(ctx, x, w, scales, biases, lbias, logits, M, V, K, bits, gs, dt,
                             proposals, tokens, accepted, ws, wsb, stream, false);
}

dfq_status dfq_qmm_argmax_accept_packed(dfq_ctx* ctx, const void* x, const void* packed,
                                        const void* lbias, void* logits, int M, int V, int K,
                                        int bits, int gs, dfq_dtype dt, const int32_t* proposals,
                                        int32_t* tokens, int32_t* accepted, void* ws, size_t wsb,
                                        void* stream) {
    return qmm_argmax_accept(ctx, x, (const uint32_t*)packed, nullptr, nullptr, lbias, logits,
                             M, V, K, bits, gs, dt, proposals, tokens, accepted, ws, wsb, stream,
                             true);
}

/* Workgroups and LDS layout of the stock path's GEMV for a shape of at most 4 rows; false
 * where its x (M x K, pre-permuted, and the per-chunk sums) and outputs would not fit in LDS. */
static constexpr int kQmvRows = 4;    // weight rows a wave works on at once (as the kernels)
static constexpr int kQmvWaves = 8;   // waves per workgroup (as the kernels)
static bool qmv_layout(const dfq_ctx* ctx, int M, int N, int K, int bits, QmvParams* p,
                       size_t* lds) {
    const int kpl = 128 / bits;  // k per lane chunk
    if (M < 1 || M > 4 || K % kpl) return false;
    /* one workgroup per CU, each with at least a row group per wave.  Measured on MI355X at
     * one row (us; this form against unit-balanced splits of 1, 2 or 4 rows a unit, 2 to 6
     * units in flight, 8 or 16 waves a CU, the first units issued before the staging):
     * N = 17408, K = 5120: 15.5 against 16.2-20.0; N = 151936: 90.8 against 92-131; N = K =
     * 5120: 8.2 against 8.4-9.6; N = K = 4096 (fp16): 6.3 against 6.1-6.6. */
    const int G = std::max(1, std::min(ctx->num_cus, (N + kQmvRows * kQmvWaves - 1) /
                                                         (kQmvRows * kQmvWaves)));
    const int rows_max = (N + G - 1) / G;
    const size_t xbytes = (size_t)M * K * 2;
    const size_t xsum_off = (xbytes + 15) & ~(size_t)15;
    const size_t cnt_off = xsum_off + (size_t)M * (K / kpl) * 4;
    const size_t out_off = (cnt_off + 16 + 15) & ~(size_t)15;
    const size_t need = out_off + (size_t)M * rows_max * 4;
    if (need > ctx->lds_max) return false;
    p->M = M;
    p->N = N;
    p->K = K;
    p->G = G;
    p->rows_max = rows_max;
    p->lds_xsum_off = (int)xsum_off;
    p->lds_cnt_off = (int)cnt_off;
    p->lds_out_off = (int)out_off;
    *lds = need;
    return true;
}

/* The stock path as MLX takes it for few rows: its GEMV, one launch per 4 rows, for one dtype
 * of x, scales, biases and y (bf16 or fp16), 4- or 8-bit codes, group 32, 64 or 128, K a
 * multiple of one lane's chunk, and x of 4 rows in LDS; DFQ_ERR_UNSUPPORTED otherwise (the
 * per-element path then takes the call). */
static dfq_status qmv_any(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                          const void* biases, const void* lbias, void* y, int M, int N, int K,
                          int bits, int gs, dfq_dtype dt, hipStream_t stream) {
    if ((bits != 4 && bits != 8) || (gs != 32 && gs != 64 && gs != 128) ||
        (dt != DFQ_BF16 && dt != DFQ_F16) || !aligned(x, 16) || !aligned(w, 16) ||
        !aligned(scales, 2) || !aligned(biases, 2) || !aligned(y, 2) ||
        (int64_t)N * K * bits / 8 >= (int64_t)1 << 32)
        return DFQ_ERR_UNSUPPORTED;
    QmvParams p{};
    size_t lds = 0;
    if (!qmv_layout(ctx, std::min(M, 4), N, K, bits, &p, &lds)) return DFQ_ERR_UNSUPPORTED;
    const int bi = bits == 4 ? 0 : 1, gi = gs == 32 ? 0 : gs == 64 ? 1 : 2;
    const int di = dt == DFQ_BF16 ? 0 : 1;
    for (int m0 = 0; m0 < M; m0 += 4) {
        const int mc = std::min(4, M - m0);
        if (!qmv_layout(ctx, mc, N, K, bits, &p, &lds)) return DFQ_ERR_UNSUPPORTED;
        p.x = (const char*)x + (size_t)m0 * K * 2;
        p.w = w;
        p.scales = scales;
        p.biases = biases;
        p.lbias = lbias;
        p.y = (char*)y + (size_t)m0 * N * 2;
        void* args[] = {&p};
        hipError_t e = hipModuleLaunchKernel(ctx->qmv[bi][gi][di][mc == 1 ? 0 : 1],
                                             (unsigned)p.G, 1, 1, kQmvWaves * 64, 1, 1,
                                             (unsigned)lds, stream, args, nullptr);
        if (e != hipSuccess) return hip_fail(e, "launch dfq_qmv");
    }
    return DFQ_OK;
}

dfq_status dfq_qmm_fallback(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                            const void* biases, const void* lbias, void* y, int M, int N, int K,
                            int bits, int gs, dfq_dtype xdt, dfq_dtype sdt, dfq_dtype ydt,
                            void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!x || !w || !scales || !biases || !y)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "null x, w, scales, biases or y");
    if (M < 1 || N < 1 || K < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "M, N, K must be >= 1");
    if (M > 65535) return fail(DFQ_ERR_UNSUPPORTED, "generic path handles M <= 65535");
    if (bits != 2 && bits != 4 && bits != 8)
        return fail(DFQ_ERR_UNSUPPORTED, "generic path handles bits 2, 4, 8 (got %d)", bits);
    if (gs < 32 / bits || gs <= 0 || K % gs || (gs % (32 / bits)))
        return fail(DFQ_ERR_UNSUPPORTED, "group size %d must divide K=%d and hold whole words",
                    gs, K);
    for (dfq_dtype d : {xdt, sdt, ydt})
        if (d != DFQ_BF16 && d != DFQ_F16 && d != DFQ_F32)
            return fail(DFQ_ERR_INVALID_ARGUMENT, "bad dtype");
    if (!aligned(w, 4)) return fail(DFQ_ERR_INVALID_ARGUMENT, "w must be 4-byte aligned");
    DeviceGuard g(ctx->device);
    if (xdt == sdt && sdt == ydt) {
        const dfq_status s = qmv_any(ctx, x, w, scales, biases, lbias, y, M, N, K, bits, gs, xdt,
                                     (hipStream_t)stream);
        if (s != DFQ_ERR_UNSUPPORTED) return s;
    }
    QmmGenericParams p{};
    p.x = x;
    p.w = w;
    p.scales = scales;
    p.biases = biases;
    p.lbias = lbias;
    p.y = y;
    p.M = M;
    p.N = N;
    p.K = K;
    p.bits = bits;
    p.gs = gs;
    p.xdt = xdt;
    p.sdt = sdt;
    p.ydt = ydt;
    void* args[] = {&p};
    hipError_t e = hipModuleLaunchKernel(ctx->generic, (unsigned)N, (unsigned)M, 1, 64, 1, 1, 0,
                                         (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_qmm_generic");
}

/* ---- graphs -------------------------------------------------------------------------- */

dfq_status dfq_graph_begin(dfq_ctx* ctx, void* stream) {
    if (!ctx) return fail(DFQ_ERR_INVALID_ARGUMENT, "null context");
    if (!stream) return fail(DFQ_ERR_INVALID_ARGUMENT, "the default stream cannot be captured");
    DeviceGuard g(ctx->device);
    hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipStreamBeginCapture");
}

dfq_status dfq_graph_end(dfq_ctx* ctx, void* stream, dfq_graph** out) {
    if (!ctx || !out) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    DeviceGuard g(ctx->device);
    hipStreamCaptureStatus st;
    hipError_t e = hipStreamIsCapturing((hipStream_t)stream, &st);
    if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
    if (st != hipStreamCaptureStatusActive) return fail(DFQ_ERR_STATE, "stream is not capturing");
    auto* gr = new dfq_graph();
    gr->device = ctx->device;
    if ((e = hipStreamEndCapture((hipStream_t)stream, &gr->graph)) != hipSuccess) {
        delete gr;
        return hip_fail(e, "hipStreamEndCapture");
    }
    if ((e = hipGraphInstantiate(&gr->exec, gr->graph, nullptr, nullptr, 0)) != hipSuccess) {
        (void)hipGraphDestroy(gr->graph);
        delete gr;
        return hip_fail(e, "hipGraphInstantiate");
    }
    *out = gr;
    return DFQ_OK;
}

dfq_status dfq_graph_launch(dfq_graph* gr, void* stream) {
    if (!gr) return fail(DFQ_ERR_INVALID_ARGUMENT, "null graph");
    DeviceGuard g(gr->device);
    hipError_t e = hipGraphLaunch(gr->exec, (hipStream_t)stream);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "hipGraphLaunch");
}

dfq_status dfq_graph_compose(dfq_ctx* ctx, dfq_graph* const* parts, int n, dfq_graph** out) {
    if (!ctx || !out || (n > 0 && !parts)) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    if (n < 1) return fail(DFQ_ERR_INVALID_ARGUMENT, "no graphs to compose");
    for (int i = 0; i < n; ++i) {
        if (!parts[i] || !parts[i]->graph)
            return fail(DFQ_ERR_INVALID_ARGUMENT, "graph %d is null", i);
        if (parts[i]->device != ctx->device)
            return fail(DFQ_ERR_INVALID_ARGUMENT, "graph %d was captured on device %d, not %d", i,
                        parts[i]->device, ctx->device);
    }
    DeviceGuard g(ctx->device);
    auto* gr = new dfq_graph();
    gr->device = ctx->device;
    hipError_t e = hipGraphCreate(&gr->graph, 0);
    if (e != hipSuccess) {
        delete gr;
        return hip_fail(e, "hipGraphCreate");
    }
    hipGraphNode_t prev = nullptr;
    for (int i = 0; i < n && e == hipSuccess; ++i) {
        hipGraphNode_t node = nullptr;
        e = hipGraphAddChildGraphNode(&node, gr->graph, prev ? &prev : nullptr, prev ? 1 : 0,
                                      parts[i]->graph);
        prev = node;
    }
    if (e == hipSuccess) e = hipGraphInstantiate(&gr->exec, gr->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(gr->graph);
        delete gr;
        return hip_fail(e, "compose graphs");
    }
    *out = gr;
    return DFQ_OK;
}

dfq_status dfq_graph_destroy(dfq_graph* gr) {
    if (!gr) return DFQ_OK;
    DeviceGuard g(gr->device);
    if (gr->exec) (void)hipGraphExecDestroy(gr->exec);
    if (gr->graph) (void)hipGraphDestroy(gr->graph);
    delete gr;
    return DFQ_OK;
}

/* ---- introspection used by tests and the benchmark (not part of the drop-in surface) -- */

/* The fields of a split as the debug calls report them. */
static void plan_fields(const Plan& p, int* out) {
    const int v[15] = {p.T,   p.SS,          p.nkb,           p.Gkb, p.nslot_kb, p.kr,
                       p.lds_bytes, p.need_ws ? 1 : 0, p.ch, p.umax, p.chunks,
                       p.reduce ? 1 : 0, p.ring, p.aligned ? 1 : 0, p.burst ? 1 : 0};
    std::memcpy(out, v, sizeof v);
}

/* Fills the work split the fast kernel uses for a shape: {T, SS, nkb, Gkb, nslot_kb, kr,
 * lds_bytes, need_ws, ch, umax, chunks, reduce, ring, aligned, burst} (SS and kr of the largest
 * k-block). */
dfq_status dfq_debug_plan(dfq_ctx* ctx, int M, int N, int K, int bits, int gs, int* out15) {
    if (!out15) return fail(DFQ_ERR_INVALID_ARGUMENT, "null out");
    Plan p;
    dfq_status s = get_plan(ctx, M, N, K, bits, gs, &p);
    if (s) return s;
    plan_fields(p, out15);
    return DFQ_OK;
}

/* The bandwidth reference: one launch reading `bytes` (a multiple of 4096) from src as a plain
 * streaming read, one workgroup of 8 waves per CU; sink receives 8 * dfq_num_cus words. */
dfq_status dfq_debug_read_stream(dfq_ctx* ctx, const void* src, size_t bytes, uint32_t* sink,
                                 void* stream) {
    if (!ctx || !src || !sink) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    if (!bytes || bytes % 4096 || !aligned(src, 16))
        return fail(DFQ_ERR_INVALID_ARGUMENT, "bytes must be a positive multiple of 4096, src 16-byte aligned");
    DeviceGuard g(ctx->device);
    const void* p = src;
    uint64_t units = bytes / 4096;
    void* args[] = {(void*)&p, &units, &sink};
    hipError_t e = hipModuleLaunchKernel(ctx->read_stream, (unsigned)ctx->num_cus, 1, 1, 512, 1,
                                         1, 0, (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_read_stream");
}

/* The fast kernel's own read of a 4-bit group-64 shape with a one-k-block split: the same
 * workgroup ranges and loads, no compute; sink receives 12 words per workgroup (12 *
 * dfq_num_cus suffices).  w, scales and biases as for dfq_qmm. */
dfq_status dfq_debug_read_units(dfq_ctx* ctx, const uint32_t* w, const void* scales,
                                const void* biases, int M, int N, int K, uint32_t* sink,
                                void* stream) {
    if (!ctx || !w || !scales || !biases || !sink)
        return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    dfq_status s = check_fast_args(ctx, M, N, K, 4, 64, DFQ_BF16, DFQ_BF16, DFQ_BF16);
    if (s) return s;
    Plan pl;
    if ((s = get_plan(ctx, M, N, K, 4, 64, &pl))) return s;
    if (pl.nkb != 1 || pl.ch != 8 / 2 || pl.Gkb > ctx->num_cus)
        return fail(DFQ_ERR_UNSUPPORTED,
                    "the unit read covers one-k-block splits of 8-group chunks over the CUs");
    DeviceGuard g(ctx->device);
    QmmParams p = fill_params(pl, nullptr, w, scales, biases, nullptr, nullptr, M, N, K, 4, 64,
                              nullptr);
    void* args[] = {&p, &sink};
    hipError_t e = hipModuleLaunchKernel(ctx->read_units, (unsigned)pl.Gkb, 1, 1, 768, 1, 1, 0,
                                         (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_read_units");
}

/* The same unit read over a packed weight array: unit (t, c) of the split's 4608 bytes at
 * packed + (t * chunks + c) * 4608, its codes as 4 x 1 KB (instruction j, lane l at j*1024 +
 * l*16) and its scales and biases as 512 bytes; sink receives 12 * dfq_num_cus words. */
dfq_status dfq_debug_read_units_packed(dfq_ctx* ctx, const void* packed, int M, int N, int K,
                                       uint32_t* sink, void* stream) {
    if (!ctx || !packed || !sink) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    dfq_status s = check_fast_args(ctx, M, N, K, 4, 64, DFQ_BF16, DFQ_BF16, DFQ_BF16);
    if (s) return s;
    Plan pl;
    if ((s = get_plan(ctx, M, N, K, 4, 64, &pl))) return s;
    if (pl.nkb != 1 || pl.ch != 8 / 2 || pl.Gkb > ctx->num_cus)
        return fail(DFQ_ERR_UNSUPPORTED,
                    "the unit read covers one-k-block splits of 8-group chunks over the CUs");
    DeviceGuard g(ctx->device);
    QmmParams p = fill_params(pl, nullptr, (const uint32_t*)packed, nullptr, nullptr, nullptr,
                              nullptr, M, N, K, 4, 64, nullptr);
    void* args[] = {&p, &sink};
    hipError_t e = hipModuleLaunchKernel(ctx->read_units_packed, (unsigned)pl.Gkb, 1, 1, 768, 1,
                                         1, 0, (hipStream_t)stream, args, nullptr);
    return e == hipSuccess ? DFQ_OK : hip_fail(e, "launch dfq_read_units_packed");
}

/* Launches of the stock path's GEMV for a shape with x, scales and y all of `dt` and 16-byte
 * aligned arrays: one per 4 rows, or 0 where the per-element path takes the call. */
dfq_status dfq_debug_stock_gemv_launches(dfq_ctx* ctx, int M, int N, int K, int bits, int gs,
                                         dfq_dtype dt, int* launches) {
    if (!ctx || !launches) return fail(DFQ_ERR_INVALID_ARGUMENT, "null argument");
    QmvParams p{};
    size_t lds = 0;
    const bool ok = (bits == 4 || bits == 8) && (gs == 32 || gs == 64 || gs == 128) &&
                    (dt == DFQ_BF16 || dt == DFQ_F16) && M >= 1 &&
                    (int64_t)N * K * bits / 8 < (int64_t)1 << 32 &&
                    qmv_layout(ctx, std::min(M, 4), N, K, bits, &p, &lds);
    *launches = ok ? (M + 3) / 4 : 0;
    return DFQ_OK;
}

/* The same split computed without a device, for a given CU count and LDS limit. */
dfq_status dfq_debug_make_plan(int M, int N, int K, int bits, int gs, int num_cus,
                               size_t lds_max, int* out15) {
    if (!out15) return fail(DFQ_ERR_INVALID_ARGUMENT, "null out");
    Plan p;
    if (!make_plan(M, N, K, bits, gs, num_cus, lds_max, &p))
        return fail(DFQ_ERR_UNSUPPORTED, "no work split");
    plan_fields(p, out15);
    return DFQ_OK;
}

}  // extern "C"
