// K1: persisted-route gather + deterministic counting partition.
//
// Replaces the reference's pair-hash planner
// (complexity_cuda/triton_token_routed.py:172-277, host glue :2205-2318) and
// its CPU/CGGR sort semantics (:69-93, :2320-2351).
//
// Every assignment a = slot*N + t (token t's slot-th route) is one item, so a
// token whose slots name the same expert gets one partition row per slot.
// Items are walked in a fixed order and each expert segment receives its
// items in that order:
//   order 0 (token)      item i = t*k + slot: segment order (token, slot),
//                        the reference's fused GPU partition (which has
//                        distinct experts per token, so (expert, token));
//   order 1 (assignment) item i = a: segment order a, the reference's stable
//                        CPU sort / CGGR.
// Ranks inside a wave come from ballots; the 256-item chunks of a block are
// walked in order with a running per-expert base in LDS; block bases come
// from per-block histograms.  No global atomics: the output is identical on
// every launch.
//
// Work split: at most kMaxSortBlocks blocks.  Up to kMaxSortBlocks * 256
// items every block takes one 256-item chunk (C2: 128 blocks, C5: 256);
// beyond that the chunks per block grow instead of the block count, so each
// block's prefix over the other blocks' histograms stays at most
// kMaxSortBlocks * E reads whatever the token count.
#include "trmoe_common.h"
#include "trmoe_internal.h"

#include <mutex>
#include <string>

namespace trmoe {

constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kMaxSortBlocks = 256;
constexpr int kSingleMaxChunks = 8;   // one block (one launch) up to 2048 items

struct SortArgs {
    const int64_t* ids;
    int n;                  // tokens
    const int64_t* table;   // [k, vocab]
    int64_t vocab;
    int k;
    int E;
    int order;
    int items;              // k * n
    int chunks;             // 256-item chunks per block
    int nblocks;
    int64_t* routes;        // [k, n] or null
    int64_t* sorted;        // [k*n]
    int64_t* inverse;       // [k*n]
    int32_t* offsets;       // [E+1]
    int32_t* counts;        // [E]
    int32_t* block_counts;  // [nblocks, E] (multi-block only)
};

// Expert of item i (-1 past the end) and its assignment index.  Table
// entries outside [0, E) (a contract violation) are clamped so that no write
// leaves the outputs; `routes` keeps the raw table value.
__device__ __forceinline__ int item_expert(const SortArgs& a, int i, int& asg, bool write_routes) {
    if (i >= a.items) {
        asg = 0;
        return -1;
    }
    int s, t;
    if (a.order == 0) {
        t = i / a.k;
        s = i - t * a.k;
    } else {
        s = i / a.n;
        t = i - s * a.n;
    }
    asg = s * a.n + t;
    int64_t id = a.ids[t];
    id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
    const int64_t raw = a.table[(int64_t)s * a.vocab + id];
    if (write_routes && a.routes != nullptr) a.routes[asg] = raw;
    return raw < 0 ? 0 : (raw >= a.E ? a.E - 1 : (int)raw);
}

// Rank of this lane among the lanes of its wave with the same expert, and
// (lane 0 of each wave) the wave's count per expert into wcnt[e].
__device__ __forceinline__ int wave_rank(int ex, int E, int* wcnt) {
    const int lane = threadIdx.x & 63;
    int rank = 0;
    for (int e = 0; e < E; ++e) {
        const uint64_t m = __ballot(ex == e);
        if (lane == 0) wcnt[e] = __popcll(m);
        if (ex == e)
            rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
    }
    return rank;
}

// Launch 1 of the multi-block form: the histogram of each block's items.
__global__ __launch_bounds__(kSortThreads) void k_route_count(SortArgs a) {
    __shared__ int s_cnt[kSortWaves][kMaxExperts];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int base = blockIdx.x * a.chunks * kSortThreads;
    // the wave's counts stay in registers (uniform) until one write per expert
    int cnt[kMaxExperts];
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) cnt[e] = 0;
    for (int c = 0; c < a.chunks; ++c) {
        int asg;
        const int ex = item_expert(a, base + c * kSortThreads + threadIdx.x, asg, true);
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e)
            if (e < a.E) cnt[e] += __popcll(__ballot(ex == e));
    }
    if (lane == 0)
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e) s_cnt[wave][e] = cnt[e];
    __syncthreads();
    if (threadIdx.x < a.E) {
        int s = 0;
        for (int w = 0; w < kSortWaves; ++w) s += s_cnt[w][threadIdx.x];
        a.block_counts[blockIdx.x * a.E + threadIdx.x] = s;
    }
}

// Scatter: this block's base per expert (offsets + earlier blocks' counts),
// then its chunks in order.  SINGLE: one block holds every item and counts
// them itself (items cached in registers between the passes).
template <bool SINGLE>
__global__ __launch_bounds__(kSortThreads) void k_route_scatter(SortArgs a) {
    __shared__ int s_wcnt[kSortWaves][kMaxExperts];
    __shared__ int s_red[kSortWaves][2][kMaxExperts];
    __shared__ int s_run[kMaxExperts];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x;
    const int base = b * a.chunks * kSortThreads;

    int ex_c[SINGLE ? kSingleMaxChunks : 1], asg_c[SINGLE ? kSingleMaxChunks : 1];
    if constexpr (SINGLE) {
        // pass 1: totals over every chunk
        if (lane < kMaxExperts) s_red[wave][1][lane] = 0;
#pragma unroll
        for (int c = 0; c < kSingleMaxChunks; ++c)
            if (c < a.chunks) ex_c[c] = item_expert(a, c * kSortThreads + threadIdx.x, asg_c[c], true);
#pragma unroll
        for (int c = 0; c < kSingleMaxChunks; ++c) {
            if (c >= a.chunks) break;
            for (int e = 0; e < a.E; ++e) {
                const uint64_t m = __ballot(ex_c[c] == e);
                if (lane == 0) s_red[wave][1][e] += __popcll(m);
            }
        }
        if (lane < kMaxExperts) s_red[wave][0][lane] = 0;
    } else {
        // prefix over blocks (nblocks <= 256): the histograms staged in LDS
        // (thread j: block j's row), then thread (part, e) sums expert e's
        // counts over blocks 16 part .. 16 part + 15, all of them and those
        // before this block, and lane e of wave w adds parts 4w .. 4w + 3
        // (LDS sums instead of cross-lane reductions per expert)
        static_assert(kSortThreads == kMaxSortBlocks && kSortThreads % kMaxExperts == 0, "one row per thread");
        constexpr int kParts = kSortThreads / kMaxExperts;
        constexpr int kPerPart = kMaxSortBlocks / kParts;
        __shared__ int s_bc[kMaxSortBlocks][kMaxExperts];
        __shared__ int s_part[kParts][2][kMaxExperts];
        const int j = threadIdx.x;
        int cv[kMaxExperts];
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e) cv[e] = (e < a.E && j < a.nblocks) ? a.block_counts[j * a.E + e] : 0;
        // the first chunk's id -> table lookups go out now, so that their
        // latency overlaps the prefix instead of following it
        ex_c[0] = item_expert(a, base + threadIdx.x, asg_c[0], false);
#pragma unroll
        for (int e = 0; e < kMaxExperts; ++e) s_bc[j][e] = cv[e];
        __syncthreads();
        {
            const int e = threadIdx.x % kMaxExperts, part = threadIdx.x / kMaxExperts;
            int tot = 0, pre = 0;
#pragma unroll
            for (int q = 0; q < kPerPart; ++q) {
                const int jj = part * kPerPart + q;
                const int c = s_bc[jj][e];
                tot += c;
                pre += jj < b ? c : 0;
            }
            s_part[part][0][e] = pre;
            s_part[part][1][e] = tot;
        }
        __syncthreads();
        if (lane < kMaxExperts) {
            int pre = 0, tot = 0;
#pragma unroll
            for (int q = 0; q < kParts / kSortWaves; ++q) {
                pre += s_part[wave * (kParts / kSortWaves) + q][0][lane];
                tot += s_part[wave * (kParts / kSortWaves) + q][1][lane];
            }
            s_red[wave][0][lane] = pre;
            s_red[wave][1][lane] = tot;
        }
    }
    __syncthreads();
    if (wave == 0) {
        // lane e: expert e's totals over the waves, then an exclusive scan
        // of the totals across the lanes (no serial walk over the experts)
        int pre = 0, tot = 0;
        if (lane < a.E)
            for (int w = 0; w < kSortWaves; ++w) {
                pre += s_red[w][0][lane];
                tot += s_red[w][1][lane];
            }
        int incl = tot;
#pragma unroll
        for (int off = 1; off < kMaxExperts; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (lane >= off) incl += v;
        }
        if (lane < a.E) {
            s_run[lane] = incl - tot + pre;
            if (b == 0) {
                a.offsets[lane] = incl - tot;
                a.counts[lane] = tot;
                if (lane == a.E - 1) a.offsets[a.E] = incl;
            }
        }
    }
    __syncthreads();

    // pass 2: chunks in order; s_wcnt turns from wave counts into wave bases
    for (int c = 0; c < a.chunks; ++c) {
        int asg, ex;
        if constexpr (SINGLE) {
            ex = -1;
            asg = 0;
#pragma unroll
            for (int q = 0; q < kSingleMaxChunks; ++q)
                if (q == c) {
                    ex = ex_c[q];
                    asg = asg_c[q];
                }
        } else if (c == 0) {
            ex = ex_c[0];
            asg = asg_c[0];
        } else {
            ex = item_expert(a, base + c * kSortThreads + threadIdx.x, asg, false);
        }
        const int rank = wave_rank(ex, a.E, s_wcnt[wave]);
        __syncthreads();
        if (threadIdx.x < a.E) {
            const int e = threadIdx.x;
            int r = s_run[e];
            for (int w = 0; w < kSortWaves; ++w) {
                const int t = s_wcnt[w][e];
                s_wcnt[w][e] = r;
                r += t;
            }
            s_run[e] = r;
        }
        __syncthreads();
        if (ex >= 0) {
            const int dest = s_wcnt[wave][ex] + rank;
            a.sorted[dest] = asg;
            a.inverse[asg] = dest;
        }
        __syncthreads();
    }
}

// Blocks and 256-item chunks per block of a partition of `items` items.
static void sort_split(int64_t items, int* nblocks, int* chunks) {
    const int64_t total_chunks = (items + kSortThreads - 1) / kSortThreads;
    if (total_chunks <= kSingleMaxChunks) {
        *nblocks = 1;
        *chunks = (int)(total_chunks < 1 ? 1 : total_chunks);
        return;
    }
    const int64_t per = (total_chunks + kMaxSortBlocks - 1) / kMaxSortBlocks;
    *chunks = (int)per;
    *nblocks = (int)((total_chunks + per - 1) / per);
}

int64_t route_sort_blocks(int64_t n, int k, int order) {
    (void)order;
    int nb, ch;
    sort_split(n * k, &nb, &ch);
    return nb;
}

int launch_route_sort(const int64_t* ids, int64_t n, const int64_t* table, int64_t vocab, int k, int E,
                      int order, int64_t* routes, int64_t* sorted, int64_t* inverse, int32_t* offsets,
                      int32_t* counts, void* workspace, size_t workspace_bytes, hipStream_t stream);

// ---------------------------------------------------------------------------
// scratch of the entry point that allocates nothing
// ---------------------------------------------------------------------------
// The per-block histograms of the multi-block partition, at most
// kMaxSortBlocks x kMaxExperts int32 (16 KiB), in a file-scope device array:
// every GPU the library runs on holds its own copy until the process ends.
// In host code `scratch` names only a host-side stand-in, so its device
// address is looked up once per device (with that device current) and only
// that address is passed to kernels.
static __device__ __align__(256) int32_t scratch[kMaxSortBlocks * kMaxExperts];
static_assert(sizeof(scratch) == TRMOE_ROUTE_SORT_NOALLOC_SCRATCH_BYTES, "header and array disagree");

static int noalloc_scratch(void** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void* ptrs[kMaxDevices] = {};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return set_error(TRMOE_ERR_HIP, "route_sort_noalloc: no current HIP device (or more than 64 devices)");
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || p == nullptr) {
            const std::string m = std::string("route_sort_noalloc: hipGetSymbolAddress(scratch): ") +
                                  (err != hipSuccess ? hipGetErrorString(err) : "null address");
            return set_error(TRMOE_ERR_HIP, m.c_str());
        }
        ptrs[dev] = p;
    }
    *out = ptrs[dev];
    return TRMOE_OK;
}

int launch_route_sort_noalloc(const int64_t* ids, int64_t n, const int64_t* table, int64_t vocab, int k, int E,
                              int order, int64_t* routes, int64_t* sorted, int64_t* inverse, int32_t* offsets,
                              int32_t* counts, hipStream_t stream) {
    int nb, ch;
    sort_split(n * k, &nb, &ch);
    const size_t need = nb > 1 ? (size_t)nb * (size_t)E * sizeof(int32_t) : 0;
    if (need > sizeof(scratch)) {
        const std::string m = "route_sort_noalloc: the partition needs " + std::to_string(need) +
                              " bytes of scratch; the static buffer holds " + std::to_string(sizeof(scratch));
        return set_error(TRMOE_ERR_INVALID, m.c_str());
    }
    void* ws = nullptr;
    const int st = noalloc_scratch(&ws);
    if (st) return st;
    return launch_route_sort(ids, n, table, vocab, k, E, order, routes, sorted, inverse, offsets, counts, ws,
                             sizeof(scratch), stream);
}

int launch_route_sort(const int64_t* ids, int64_t n, const int64_t* table, int64_t vocab, int k, int E,
                      int order, int64_t* routes, int64_t* sorted, int64_t* inverse, int32_t* offsets,
                      int32_t* counts, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    SortArgs a{};
    a.ids = ids;
    a.n = (int)n;
    a.table = table;
    a.vocab = vocab;
    a.k = k;
    a.E = E;
    a.order = order;
    a.items = (int)(n * k);
    sort_split(n * k, &a.nblocks, &a.chunks);
    a.routes = routes;
    a.sorted = sorted;
    a.inverse = inverse;
    a.offsets = offsets;
    a.counts = counts;
    a.block_counts = static_cast<int32_t*>(workspace);
    if (a.nblocks == 1) {
        hipLaunchKernelGGL(k_route_scatter<true>, dim3(1), dim3(kSortThreads), 0, stream, a);
        return check_launch("route_scatter(single)");
    }
    if (workspace == nullptr || workspace_bytes < (size_t)a.nblocks * E * sizeof(int32_t))
        return set_error(TRMOE_ERR_INVALID, "route_sort: workspace too small");
    hipLaunchKernelGGL(k_route_count, dim3(a.nblocks), dim3(kSortThreads), 0, stream, a);
    int st = check_launch("route_count");
    if (st) return st;
    hipLaunchKernelGGL(k_route_scatter<false>, dim3(a.nblocks), dim3(kSortThreads), 0, stream, a);
    return check_launch("route_scatter");
}

}  // namespace trmoe
