/*
 * C restatement of the TR-MoE integer routing -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/ (through ctypes) may load the library built from this file; the
 * shipped HIP library never links it.  It restates, as scalar C over 32-bit
 * unsigned arithmetic, the parts of the reference the GPU must reproduce bit
 * for bit:
 *
 *   oracle_mix32            complexity/tr_hash/routing.py:97-103
 *   oracle_multi_hash_table complexity/tr_hash/routing.py:129-167 (top-k by
 *                           descending score; ties -> lower expert index)
 *   oracle_partition        complexity_cuda/triton_token_routed.py:211-277
 *                           (order 0: expert, then token) and :2320-2351
 *                           (order 1: expert, then assignment index).
 *
 * It is an implementation independent of trmoe_oracle.py (numpy) and of the
 * HIP kernels; the tests require all three to agree.
 */
#include <stdint.h>
#include <string.h>

uint32_t oracle_mix32(uint32_t v) {
    v ^= v >> 16;
    v *= 0x7FEB352Du;
    v ^= v >> 15;
    v *= 0x846CA68Bu;
    v ^= v >> 16;
    return v;
}

/* table: int64[top_k * vocab], row-major [slot][token]. Returns 0 on success. */
int oracle_multi_hash_table(int64_t vocab, int num_experts, int top_k, int64_t layer_index,
                            uint32_t route_seed, int hash_count, int64_t *table) {
    if (num_experts < 1 || num_experts > 64 || top_k < 1 || top_k > num_experts) return 1;
    uint32_t salt = route_seed + (uint32_t)layer_index * 0x9E3779B1u;
    uint32_t expert_salt[8][64];
    uint32_t channel[8];
    for (int h = 0; h < hash_count; ++h) {
        channel[h] = salt + (uint32_t)h * 0x85EBCA77u;
        for (int e = 0; e < num_experts; ++e)
            expert_salt[h][e] = oracle_mix32((uint32_t)e + (channel[h] ^ 0xC2B2AE3Du));
    }
    for (int64_t t = 0; t < vocab; ++t) {
        uint64_t score[64];
        int taken[64];
        for (int e = 0; e < num_experts; ++e) {
            uint64_t s = 0;
            for (int h = 0; h < hash_count; ++h)
                s += oracle_mix32((uint32_t)t ^ expert_salt[h][e] ^ channel[h]);
            score[e] = s;
            taken[e] = 0;
        }
        for (int slot = 0; slot < top_k; ++slot) {
            int best = -1;
            for (int e = 0; e < num_experts; ++e) {
                if (taken[e]) continue;
                if (best < 0 || score[e] > score[best]) best = e;
            }
            taken[best] = 1;
            table[(int64_t)slot * vocab + t] = best;
        }
    }
    return 0;
}

/*
 * routes: int64[top_k * n] (slot-major).  Writes sorted[kn], inverse[kn],
 * offsets[E+1], counts[E].  Two passes: histogram, then a stable placement
 * walk in the order's key sequence.
 */
int oracle_partition(const int64_t *routes, int64_t n, int top_k, int num_experts, int order,
                     int64_t *sorted, int64_t *inverse, int32_t *offsets, int32_t *counts) {
    int64_t kn = n * (int64_t)top_k;
    int64_t cursor[64];
    if (num_experts < 1 || num_experts > 64) return 1;
    memset(counts, 0, sizeof(int32_t) * (size_t)num_experts);
    for (int64_t a = 0; a < kn; ++a) {
        int64_t e = routes[a];
        if (e < 0 || e >= num_experts) return 2;
        counts[e] += 1;
    }
    offsets[0] = 0;
    for (int e = 0; e < num_experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    for (int e = 0; e < num_experts; ++e) cursor[e] = offsets[e];
    if (order == 0) {
        for (int64_t t = 0; t < n; ++t)
            for (int s = 0; s < top_k; ++s) {
                int64_t a = (int64_t)s * n + t;
                int64_t e = routes[a];
                /* the segment of expert e sees tokens in increasing order,
                 * and a token whose slots repeat an expert in slot order */
                sorted[cursor[e]] = a;
                inverse[a] = cursor[e];
                cursor[e] += 1;
            }
    } else if (order == 1) {
        for (int64_t a = 0; a < kn; ++a) {
            int64_t e = routes[a];
            sorted[cursor[e]] = a;
            inverse[a] = cursor[e];
            cursor[e] += 1;
        }
    } else {
        return 3;
    }
    return 0;
}
