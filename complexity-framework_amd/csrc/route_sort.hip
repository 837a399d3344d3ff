// K1: persisted-route gather + deterministic counting partition.
//
// Replaces the reference's pair-hash planner
// (complexity_cuda/triton_token_routed.py:172-277, host glue :2205-2318) and
// its CPU/CGGR sort semantics (:69-93, :2320-2351).
//
// Items are walked in a fixed order and each expert segment receives its
// items in that order:
//   order 0 (token)      item = token t, contributing one assignment
//                        a = slot*N + t per selected expert; segment order is
//                        token order (the reference's fused GPU partition);
//   order 1 (assignment) item = assignment a in [0, k*N); segment order is
//                        a (the reference's stable CPU sort / CGGR).
// Ranks come from wavefront ballots plus an LDS prefix over (iteration,
// wave); block prefixes come from per-block histograms, so no global atomics
// are used and the output is identical on every launch.
#include "trmoe_common.h"
#include "trmoe_internal.h"

namespace trmoe {

constexpr int kSortThreads = 256;
constexpr int kSortIters = 4;
constexpr int kSortItemsPerBlock = kSortThreads * kSortIters;
constexpr int kSortWaves = kSortThreads / 64;

struct SortArgs {
    const int64_t* ids;
    int64_t n;
    const int64_t* table;   // [k, vocab]
    int64_t vocab;
    int k;
    int E;
    int order;
    int64_t n_items;
    int64_t* routes;        // [k, n] or null
    int64_t* sorted;        // [k*n]
    int64_t* inverse;       // [k*n]
    int32_t* offsets;       // [E+1]
    int32_t* counts;        // [E]
    int32_t* block_counts;  // [nblocks, E] (multi-block only)
    int nblocks;
};

// Experts of item i: for token items all k slots, for assignment items one.
__device__ __forceinline__ int item_experts(const SortArgs& a, int64_t i, int64_t (&assign)[4], int (&ex)[4]) {
    if (a.order == 0) {
        int64_t id = a.ids[i];
        id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
        for (int s = 0; s < a.k; ++s) {
            ex[s] = (int)a.table[(int64_t)s * a.vocab + id];
            assign[s] = (int64_t)s * a.n + i;
        }
        return a.k;
    }
    int64_t s = i / a.n;
    int64_t t = i - s * a.n;
    int64_t id = a.ids[t];
    id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
    ex[0] = (int)a.table[s * a.vocab + id];
    assign[0] = i;
    return 1;
}

__global__ __launch_bounds__(kSortThreads) void k_route_count(SortArgs a) {
    __shared__ int cnt[kMaxExperts];
    if (threadIdx.x < kMaxExperts) cnt[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * kSortItemsPerBlock;
    for (int j = 0; j < kSortIters; ++j) {
        int64_t i = base + j * kSortThreads + threadIdx.x;
        if (i < a.n_items) {
            int64_t asg[4];
            int ex[4];
            int m = item_experts(a, i, asg, ex);
            for (int s = 0; s < m; ++s)
                if ((unsigned)ex[s] < (unsigned)a.E) atomicAdd(&cnt[ex[s]], 1);
        }
    }
    __syncthreads();
    if (threadIdx.x < a.E) a.block_counts[(int64_t)blockIdx.x * a.E + threadIdx.x] = cnt[threadIdx.x];
}

__device__ __forceinline__ int block_sum(int v, int* red) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    int s = 0;
    for (int w = 0; w < kSortWaves; ++w) s += red[w];
    return s;
}

template <bool SINGLE>
__global__ __launch_bounds__(kSortThreads) void k_route_scatter(SortArgs a) {
    __shared__ int wcnt[kSortIters][kSortWaves][kMaxExperts];
    __shared__ int wbase[kSortIters][kSortWaves][kMaxExperts];
    __shared__ int s_prefix[kMaxExperts];
    __shared__ int s_offset[kMaxExperts + 1];
    __shared__ int red[kSortWaves];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint64_t lt_mask = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
    const int64_t base = (int64_t)blockIdx.x * kSortItemsPerBlock;

    // pass 1: per (iteration, wave, expert) counts from ballots
    for (int j = 0; j < kSortIters; ++j) {
        int64_t i = base + j * kSortThreads + threadIdx.x;
        bool valid = i < a.n_items;
        int64_t asg[4] = {0, 0, 0, 0};
        int ex[4] = {-1, -1, -1, -1};
        int m = valid ? item_experts(a, i, asg, ex) : 0;
        if (valid && a.routes != nullptr) {
            for (int s = 0; s < m; ++s) a.routes[asg[s]] = ex[s];
        }
        for (int e = 0; e < a.E; ++e) {
            bool match = false;
            for (int s = 0; s < m; ++s) match |= (ex[s] == e);
            uint64_t mask = __ballot(match);
            if (lane == 0) wcnt[j][wave][e] = __popcll(mask);
        }
    }
    __syncthreads();

    // block prefix and expert totals
    if (SINGLE) {
        if (threadIdx.x < a.E) {
            int e = threadIdx.x, tot = 0;
            for (int j = 0; j < kSortIters; ++j)
                for (int w = 0; w < kSortWaves; ++w) tot += wcnt[j][w][e];
            s_prefix[e] = 0;
            s_offset[e + 1] = tot;  // temporarily the count
        }
    } else {
        for (int e = 0; e < a.E; ++e) {
            int pre = 0, tot = 0;
            for (int bb = threadIdx.x; bb < a.nblocks; bb += kSortThreads) {
                int c = a.block_counts[(int64_t)bb * a.E + e];
                tot += c;
                if (bb < (int)blockIdx.x) pre += c;
            }
            pre = block_sum(pre, red);
            tot = block_sum(tot, red);
            if (threadIdx.x == 0) {
                s_prefix[e] = pre;
                s_offset[e + 1] = tot;
            }
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        s_offset[0] = 0;
        for (int e = 0; e < a.E; ++e) {
            int c = s_offset[e + 1];
            if (blockIdx.x == 0) a.counts[e] = c;
            s_offset[e + 1] = s_offset[e] + c;
        }
        if (blockIdx.x == 0)
            for (int e = 0; e <= a.E; ++e) a.offsets[e] = s_offset[e];
    }
    if (threadIdx.x < a.E) {
        int e = threadIdx.x, run = 0;
        for (int j = 0; j < kSortIters; ++j)
            for (int w = 0; w < kSortWaves; ++w) {
                wbase[j][w][e] = run;
                run += wcnt[j][w][e];
            }
    }
    __syncthreads();

    // pass 2: scatter
    for (int j = 0; j < kSortIters; ++j) {
        int64_t i = base + j * kSortThreads + threadIdx.x;
        bool valid = i < a.n_items;
        int64_t asg[4] = {0, 0, 0, 0};
        int ex[4] = {-1, -1, -1, -1};
        int m = valid ? item_experts(a, i, asg, ex) : 0;
        for (int e = 0; e < a.E; ++e) {
            int slot = -1;
            for (int s = 0; s < m; ++s)
                if (ex[s] == e) slot = s;
            uint64_t mask = __ballot(slot >= 0);
            if (slot >= 0) {
                int64_t dest = (int64_t)s_offset[e] + s_prefix[e] + wbase[j][wave][e] + __popcll(mask & lt_mask);
                int64_t an = asg[slot];
                a.sorted[dest] = an;
                a.inverse[an] = dest;
            }
        }
    }
}

int64_t route_sort_blocks(int64_t n, int k, int order) {
    int64_t items = (order == 0) ? n : n * k;
    int64_t nb = (items + kSortItemsPerBlock - 1) / kSortItemsPerBlock;
    return nb < 1 ? 1 : nb;
}

int launch_route_sort(const int64_t* ids, int64_t n, const int64_t* table, int64_t vocab, int k, int E,
                      int order, int64_t* routes, int64_t* sorted, int64_t* inverse, int32_t* offsets,
                      int32_t* counts, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    SortArgs a{};
    a.ids = ids;
    a.n = n;
    a.table = table;
    a.vocab = vocab;
    a.k = k;
    a.E = E;
    a.order = order;
    a.n_items = (order == 0) ? n : n * k;
    a.routes = routes;
    a.sorted = sorted;
    a.inverse = inverse;
    a.offsets = offsets;
    a.counts = counts;
    a.nblocks = (int)route_sort_blocks(n, k, order);
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
