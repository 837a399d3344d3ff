// K2/K3/K4: MFMA tile kernels of the TR-MoE layer, plus weight packing.
//
//   k_gate_up_swiglu   shared SwiGLU gate|up GEMM with the SwiGLU epilogue
//                      (engine.py:333-349, first half)
//   k_routed_experts   per-expert gate|up -> SwiGLU -> down over the K1
//                      partition, one workgroup per (expert, 128-row) tile
//                      (triton_token_routed.py:1033-1342)
//   k_down_combine     shared down GEMM; the epilogue gathers each token's k
//                      expert rows through `inverse` and applies the route
//                      weights and branch scales (engine.py:509-531, 578)
//   k_combine          the epilogue alone, for shared_width == 0
//   k_pack             weight re-layout into the K-contiguous packed form
#include "trmoe_common.h"
#include "trmoe_internal.h"
#include "trmoe_gemm.h"
#include "trmoe_tiles.h"
#include "trmoe_pp.h"

#include <stdlib.h>
#include <string.h>

#include <type_traits>

namespace trmoe {

// ---------------------------------------------------------------------------
// packing
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_pack(PackArgs p) {
    const int64_t total = p.groups * p.dst_rows * p.dst_cols;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t col = idx % p.dst_cols;
        const int64_t rowg = idx / p.dst_cols;
        const int64_t row = rowg % p.dst_rows;
        const int64_t g = rowg / p.dst_rows;
        int64_t feat;
        const char* src;
        const float* ssrc;
        if (p.interleave) {
            const int64_t blk = row >> 6, w = row & 63;
            feat = blk * 32 + (w & 31);
            src = (w >= 32) ? (const char*)p.b : (const char*)p.a;
            ssrc = (w >= 32) ? p.sb : p.sa;
        } else {
            feat = row;
            src = (const char*)p.a;
            ssrc = p.sa;
        }
        const bool valid = feat < p.out_features && col < p.in_features;
        const int64_t s = g * p.s_group + feat * p.s_out + col * p.s_in;
        char* d = (char*)p.dst + (g * p.dst_group_stride + row * p.dst_ld + col) * p.elem_bytes;
        if (p.elem_bytes == 1) {
            *(uint8_t*)d = valid ? ((const uint8_t*)src)[s] : 0;
        } else if (p.elem_bytes == 2) {
            *(uint16_t*)d = valid ? ((const uint16_t*)src)[s] : 0;
        } else {
            *(uint32_t*)d = valid ? ((const uint32_t*)src)[s] : 0;
        }
        if (p.dst_scale != nullptr && col == 0) {
            const bool fv = feat < p.out_features;
            p.dst_scale[g * p.dst_scale_group_stride + row] = fv ? ssrc[g * p.scale_group_stride + feat] : 0.0f;
        }
    }
}

int launch_pack(const PackArgs& p, hipStream_t stream) {
    const int64_t total = p.groups * p.dst_rows * p.dst_cols;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(k_pack, dim3((unsigned)blocks), dim3(256), 0, stream, p);
    return check_launch("pack_weight");
}

// ---------------------------------------------------------------------------
// K2: shared gate|up + SwiGLU
// ---------------------------------------------------------------------------
// Gathers the routes of rows [m0, m0 + BM) into s_route for tiles that hold
// expert features (dense-routed strategy).
template <class Shape, bool ROUTED = true>
__device__ __forceinline__ void gate_up_routes(const GateUpArgs& a, int64_t m0, int64_t n0,
                                               int (*s_route)[kMaxTopK]) {
    if constexpr (!ROUTED) return;
    const bool tile_routed = a.ids != nullptr && ((n0 + Shape::BN) >> 1) > a.shared_feats;
    if (tile_routed && threadIdx.x < Shape::BM) {
        const int64_t row = m0 + threadIdx.x;
        int64_t id = row < a.M ? a.ids[row] : 0;
        id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
        for (int j = 0; j < kMaxTopK; ++j)
            s_route[threadIdx.x][j] = (j < a.top_k && row < a.M) ? (int)a.table[(int64_t)j * a.vocab + id] : -1;
    }
}

// SwiGLU epilogue, in two halves: gate_up_epi_tile writes the h values to
// LDS (free after the main loop's last barrier) as a [BM][BN/2] tile with
// rows padded by 16 bytes; after a barrier gate_up_epi_store copies the tile
// out with coalesced 16-byte stores.  gate_up_epilogue runs both; it ends
// with LDS still in use by the copy (callers that reuse LDS barrier first).
// One 32-feature block (gate accumulators acc[tm][2p], up acc[tm][2p + 1])
// of a wave, 32 rows at a time: the rows' LDS data (route weights, RMSNorm
// scales) is read first, then the 16 SwiGLU values per lane are written.  The
// compiler cannot tell the LDS arrays apart, so reads interleaved with the
// writes element by element would each wait for an LDS round trip.
template <class Kind, class Shape, bool RT, bool RS>
__device__ __forceinline__ void gate_up_epi_block(const GateUpArgs& a, const f32x16 (&acc)[Shape::TM][Shape::TN],
                                                  int p, int expert, float sg, float su, int wm0, int fl, char* lds,
                                                  const int (*s_route)[kMaxTopK], const float* s_rscale) {
    using T = typename Kind::T;
    constexpr int kHRowBytes = Shape::BN / 2 * (int)sizeof(T) + 16;
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int tm = 0; tm < Shape::TM; ++tm) {
        float mult[16], rs[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int rl = wm0 + tm * 32 + acc_row(lane, i);
            if constexpr (RT) {   // the token's weight for this block's expert: sum_j w_j [route_j == e]
                const int* rr = s_route[rl];
                float tw = 0.f;
#pragma unroll
                for (int j = 0; j < kMaxTopK; ++j) tw += (rr[j] == expert) ? a.rw[j] : 0.f;
                mult[i] = tw;
            } else {
                mult[i] = a.shared_mult;
            }
            rs[i] = RS ? s_rscale[rl] : 1.0f;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int rl = wm0 + tm * 32 + acc_row(lane, i);
            const float g = acc[tm][2 * p][i] * sg * rs[i];
            const float u = acc[tm][2 * p + 1][i] * su * rs[i];
            const float hv = silu_f(g) * u * mult[i];
            *reinterpret_cast<T*>(lds + rl * kHRowBytes + fl * (int)sizeof(T)) = from_f32<T>(hv);
        }
    }
}

template <class Kind, class Shape, bool ROUTED, bool RS>
__device__ __forceinline__ void gate_up_epi_tile_rs(const GateUpArgs& a, const f32x16 (&acc)[Shape::TM][Shape::TN],
                                                    int64_t n0, char* lds, const int (*s_route)[kMaxTopK],
                                                    const float* s_rscale) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int r = lane & 31;
#pragma unroll
    for (int p = 0; p < Shape::TN / 2; ++p) {
        const int64_t pbase = n0 + wn0 + 64 * p;     // packed row of the gate tile
        const int64_t fblock = pbase >> 1;            // first feature of this 32-feature block
        const int fl = wn0 / 2 + 32 * p + r;          // feature within the tile
        const float sg = a.w_scale ? a.w_scale[pbase + r] : 1.0f;
        const float su = a.w_scale ? a.w_scale[pbase + 32 + r] : 1.0f;
        // expert blocks are multiples of 64 features, so a 32-feature block
        // is wholly shared or wholly one expert's
        if (ROUTED && a.ids != nullptr && fblock >= a.shared_feats) {
            const int expert = (int)((fblock - a.shared_feats) / a.expert_feats);
            gate_up_epi_block<Kind, Shape, ROUTED, RS>(a, acc, p, expert, sg, su, wm0, fl, lds, s_route, s_rscale);
        } else {
            gate_up_epi_block<Kind, Shape, false, RS>(a, acc, p, -1, sg, su, wm0, fl, lds, s_route, s_rscale);
        }
    }
}

template <class Kind, class Shape, bool ROUTED = true>
__device__ __forceinline__ void gate_up_epi_tile(const GateUpArgs& a, const f32x16 (&acc)[Shape::TM][Shape::TN],
                                                 int64_t n0, char* lds, const int (*s_route)[kMaxTopK],
                                                 const float* s_rscale = nullptr) {
    static_assert(Shape::BM * (Shape::BN / 2 * (int)sizeof(typename Kind::T) + 16) <= 160 * 1024,
                  "h tile must fit in LDS");
    if (s_rscale != nullptr)
        gate_up_epi_tile_rs<Kind, Shape, ROUTED, true>(a, acc, n0, lds, s_route, s_rscale);
    else
        gate_up_epi_tile_rs<Kind, Shape, ROUTED, false>(a, acc, n0, lds, s_route, s_rscale);
}

template <class Kind, class Shape>
__device__ __forceinline__ void gate_up_epi_store(const GateUpArgs& a, int64_t m0, int64_t n0, const char* lds) {
    using T = typename Kind::T;
    constexpr int kHRowBytes = Shape::BN / 2 * (int)sizeof(T) + 16;
    constexpr int kChunksPerRow = Shape::BN / 2 * (int)sizeof(T) / 16;
    constexpr int kChunks = Shape::BM * kChunksPerRow;
    char* hbase = static_cast<char*>(a.h) + (n0 >> 1) * (int64_t)sizeof(T);
#pragma unroll 4
    for (int q = threadIdx.x; q < kChunks; q += Shape::NT) {
        const int rl = q / kChunksPerRow, c = q % kChunksPerRow;
        const int64_t row = m0 + rl;
        if (row < a.M)
            *reinterpret_cast<u32x4*>(hbase + row * a.ldh * (int64_t)sizeof(T) + c * 16) =
                *reinterpret_cast<const u32x4*>(lds + rl * kHRowBytes + c * 16);
    }
}

template <class Kind, class Shape, bool ROUTED = true>
__device__ __forceinline__ void gate_up_epilogue(const GateUpArgs& a, f32x16 (&acc)[Shape::TM][Shape::TN],
                                                 int64_t m0, int64_t n0, char* lds,
                                                 const int (*s_route)[kMaxTopK],
                                                 const float* s_rscale = nullptr) {
    gate_up_epi_tile<Kind, Shape, ROUTED>(a, acc, n0, lds, s_route, s_rscale);
    wait_lgkmcnt0();   // LDS tile complete; outstanding global loads (a next tile's operands) keep flying
    lds_barrier();
    gate_up_epi_store<Kind, Shape>(a, m0, n0, lds);
}

// Raw gate|up accumulators to a.gu (the pre-activations the backward reads
// instead of recomputing them), from the accumulator layout with buffer
// stores: cells past the rows or columns get offsets with bit 31 set, past
// any range, and are dropped.
template <class Kind, class Shape>
__device__ __forceinline__ void gate_up_save(const GateUpArgs& a, const f32x16 (&acc)[Shape::TM][Shape::TN],
                                             int64_t m0, int64_t n0, int64_t packed_rows) {
    using T = typename Kind::T;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int mlim = (int)(a.M - m0 < Shape::BM ? a.M - m0 : Shape::BM);
    const int nlim = (int)(packed_rows - n0 < Shape::BN ? packed_rows - n0 : Shape::BN);
    if (mlim <= 0 || nlim <= 0) return;
    const int ld = (int)a.ldgu;
    const auto rsrc = make_rsrc(static_cast<T*>(a.gu) + m0 * a.ldgu + n0,
                                (uint32_t)(((int64_t)(mlim - 1) * ld + nlim) * (int64_t)sizeof(T)));
#pragma unroll
    for (int tn = 0; tn < Shape::TN; ++tn) {
        const int c = wn0 + tn * 32 + (lane & 31);
        const float sc = a.w_scale ? a.w_scale[n0 + c] : 1.0f;
#pragma unroll
        for (int tm = 0; tm < Shape::TM; ++tm)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = wm0 + tm * 32 + acc_row(lane, i);
                const int off = ((r * ld + c) * (int)sizeof(T)) | ((r < mlim && c < nlim) ? 0 : kOutOfRange);
                const float v = acc[tm][tn][i] * sc;
                if constexpr (sizeof(T) == 2)
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<T>(v)), rsrc, off, 0,
                                                          0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rsrc, off, 0, 0);
            }
    }
}

// ROUTED: the tile may hold dense-routed expert features (route gather and
// per-token expert weights compiled in); the shared-feature launches leave
// that code out.  SAVE: also write the raw gate|up outputs to a.gu (training
// forwards), passed the launch's packed row count as gridDim-independent bound.
template <class Kind, bool FP8, class Shape, bool GROUPED = false, bool ROUTED = false, bool SAVE = false>
__global__ __launch_bounds__(Shape::NT) void k_gate_up_swiglu(GateUpArgs a) {
    using T = typename Kind::T;
    extern __shared__ __align__(16) char lds[];
    const int wave = threadIdx.x >> 6;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = a.n_base + (int64_t)blockIdx.y * Shape::BN;

    typename AProvOf<Shape>::type ap;
    if constexpr (GROUPED) {
        __shared__ int s_tile[3];
        grouped_tile<Shape::BM>(a.offsets, a.E, (int)blockIdx.x, s_tile);
        if (s_tile[0] < 0) return;
        const int64_t e = s_tile[0];
        m0 = s_tile[1];
        a.M = s_tile[2];   // rows at or past the segment end are not written
        a.w = static_cast<const char*>(a.w) + e * a.w_expert_stride * (FP8 ? 1 : (int64_t)sizeof(T));
        if (a.w_scale) a.w_scale += e * a.scale_expert_stride;
        if (a.gather != nullptr)
            init_gather_rows(ap, a.x, a.gather, a.gather_mod, m0, a.M - m0, a.ldx * (int64_t)sizeof(T),
                             a.K * (int)sizeof(T));
        else
            init_a<Shape>(ap, a.x, m0, a.M, a.ldx * (int64_t)sizeof(T), a.K * (int)sizeof(T));
    } else {
        init_a<Shape>(ap, a.x, m0, a.M, a.ldx * (int64_t)sizeof(T), a.K * (int)sizeof(T));
    }
    // fused RMSNorm: the row scales of the tile's rows (partition rows read
    // their token's), read back in the epilogue after the main loop's barriers
    __shared__ float s_rscale[Shape::BM];
    if (a.row_scale != nullptr && threadIdx.x < Shape::BM) {
        const int64_t row = m0 + threadIdx.x;
        int64_t tok = row;
        if constexpr (GROUPED) {
            if (a.gather != nullptr && row < a.M) tok = (int64_t)((uint64_t)a.gather[row] % (uint64_t)a.gather_mod);
        }
        s_rscale[threadIdx.x] = row < a.M ? a.row_scale[tok] : 0.0f;
    }
    typename BProvOf<Kind, FP8, Shape>::type bp;
    init_b<Kind, FP8, Shape>(bp, a.w, a.ldw, n0, a.K);

    // Routes of this tile's rows, gathered once while the first stages load;
    // read back in the epilogue after the main loop's barriers.
    __shared__ int s_route[ROUTED ? Shape::BM : 1][kMaxTopK];
    gate_up_routes<Shape, ROUTED>(a, m0, n0, s_route);

    f32x16 acc[Shape::TM][Shape::TN];
    zero_acc<Kind>(acc);
    tile_loop<Kind, Shape>(ap, bp, a.K, lds, wm0, wn0, acc);
    if constexpr (SAVE) gate_up_save<Kind, Shape>(a, acc, m0, n0, a.n_base + (int64_t)gridDim.y * Shape::BN);
    gate_up_epilogue<Kind, Shape, ROUTED>(a, acc, m0, n0, lds, s_route,
                                          a.row_scale != nullptr ? s_rscale : nullptr);
}

// SwiGLU of one finished tile straight from the accumulators of the calling
// wave (no LDS): each lane owns one h feature (its gate column r of the
// wave's 64 packed rows, up column 32 + r) and 16 rows per 32-row block;
// PAIRS: adjacent lanes pair their values into 4-byte stores
// (store_bf16_pairs), else one 2-byte store per value.  Rows at or past M
// fall past the buffer's range and are dropped.
// RS: the gate and up values of each row are also multiplied by
// a.row_scale[row] (the per-token scale of e4m3 activations).
template <int TMW, bool PAIRS = true, bool RS = false>
__device__ __forceinline__ void gate_up_epi_direct(const GateUpArgs& a, const f32x16 (&acc)[TMW][2], int64_t m0,
                                                   int64_t n0, int wm0, int wn0) {
    const int lane = threadIdx.x & 63, r = lane & 31;
    const int64_t pbase = n0 + wn0;   // packed row of the wave's gate block
    // h = silu(g) * u * mult, with the shared multiplier folded into u
    const float sg = a.w_scale ? a.w_scale[pbase + r] : 1.0f;
    const float su = (a.w_scale ? a.w_scale[pbase + 32 + r] : 1.0f) * a.shared_mult;
    const int64_t mlim = a.M - m0 < 64 * TMW ? a.M - m0 : 64 * TMW;
    // the row stride is redefined here so that no offset below is hoisted
    // out of a caller's loop (they would stay live across every stage)
    int ld2 = (int)a.ldh * 2;
    asm volatile("" : "+s"(ld2));
    const auto rsrc = make_rsrc(static_cast<bf16_t*>(a.h) + m0 * a.ldh, (uint32_t)(mlim * ld2));
    const int col = (int)((pbase >> 1) + r);
    if constexpr (PAIRS) {
        const int lb = pair_lane_offset(wm0, col, ld2);
#pragma unroll
        for (int tm = 0; tm < TMW; ++tm) {
            // RS: lane l loads the scale of row wm0 + 32 tm + (l % 32) (clamped
            // into the tile: rows at or past M are not stored), and element i
            // takes its row's, acc_row(lane, i), from that lane
            float rsl = 1.0f;
            if constexpr (RS) {
                const int rrow = wm0 + tm * 32 + r;
                rsl = a.row_scale[m0 + (rrow < mlim ? rrow : mlim - 1)];
            }
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float g = acc[tm][0][i] * sg, u = acc[tm][1][i] * su;
                if constexpr (RS) {
                    const float rs = __shfl(rsl, 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3));
                    g *= rs;
                    u *= rs;
                }
                v[i] = silu_f(g) * u;
            }
            store_bf16_pairs(rsrc, lb + tm * 32 * ld2, ld2, v);
        }
    } else {
        static_assert(!RS, "row scales are applied on the paired-store path");
        // one 2-byte store per value (fewer live registers: the e4m3 kernels
        // keep their loader state out of scratch this way)
        const int lb = (wm0 + 4 * (lane >> 5)) * ld2 + col * 2;
#pragma unroll
        for (int tm = 0; tm < TMW; ++tm)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int off = lb + (tm * 32 + 8 * (i >> 2) + (i & 3)) * ld2;   // row wm0 + tm*32 + acc_row(lane, i)
                const float hv = silu_f(acc[tm][0][i] * sg) * (acc[tm][1][i] * su);
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, from_f32<bf16_t>(hv)), rsrc, off,
                                                      0, 0);
            }
    }
}

// W8A8 h as block-scaled e4m3 (a.hs != nullptr), from transposed
// accumulator blocks (pp_mma_f8<TM, true>): acc[tm][0][i] / acc[tm][1][i]
// are the gate / up outputs of feature f0 + acc_row(lane, i), f0 = the
// wave's first feature, for token wm0 + 32 tm + lane % 32.  So a lane holds
// 16 of the 32 features of its token's block and lane l ^ 32 the other 16.
// h = silu(g) * u with the activations' per-token scale and the weights'
// per-row scales; then per token and block the exponent e: the smallest
// integer with amax <= 448 * 2^e (amax = m * 2^k by frexp, m in [0.5, 1):
// e = k - 9, plus 1 when m > 0.875 = 448 / 2^9), clamped to [-126, 126], and
// 0 for a block without a positive finite maximum (all zeros, or NaN or
// infinite values).  The codes e4m3(h * 2^-e) (round to nearest even,
// clamped to +-448, NaN stays NaN) go to a.h (ldh bytes per row, four
// features per 4-byte store), the E8M0 bytes e + 127 to a.hs (ldhs bytes per
// row, byte feature / 32).
__device__ __forceinline__ int mx_exponent(float amax) {
    if (!(amax > 0.0f) || !__builtin_isfinite(amax)) return 0;
    int k;
    const float m = frexpf(amax, &k);
    const int e = k - 9 + (m > 0.875f ? 1 : 0);
    return e < -126 ? -126 : (e > 126 ? 126 : e);
}

template <int TMW>
__device__ __forceinline__ void gate_up_epi_mx(const GateUpArgs& a, const f32x16 (&acc)[TMW][2], int64_t m0,
                                               int64_t n0, int wm0, int wn0) {
    const int lane = threadIdx.x & 63, r = lane & 31, half = lane >> 5;
    const int64_t pbase = n0 + wn0;   // packed row of the wave's gate block
    const float* ws = a.w_scale + pbase;
    const int64_t mlim = a.M - m0 < 64 * TMW ? a.M - m0 : 64 * TMW;
    int ldq = (int)a.ldh;   // opaque row strides: no offset below is hoisted out of a caller's loop
    asm volatile("" : "+s"(ldq));
    int ldsc = (int)a.ldhs;
    asm volatile("" : "+s"(ldsc));
    const auto rq = make_rsrc(static_cast<uint8_t*>(a.h) + m0 * a.ldh, (uint32_t)(mlim * ldq));
    const auto rs = make_rsrc(static_cast<uint8_t*>(a.hs) + m0 * a.ldhs, (uint32_t)(mlim * ldsc));
    const int f0 = (int)(pbase >> 1);
    const int blk = (int)(pbase >> 6);
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm) {
        const int row = wm0 + tm * 32 + r;   // the lane's token in the tile
        const float rsc = a.row_scale[m0 + (row < mlim ? row : mlim - 1)];
        float v[16];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int fr = 8 * (i >> 2) + 4 * half + (i & 3);   // acc_row(lane, i)
            v[i] = silu_f(acc[tm][0][i] * ws[fr] * rsc) * (acc[tm][1][i] * (ws[32 + fr] * a.shared_mult) * rsc);
            amax = fmaxf(amax, fabsf(v[i]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        const int e = mx_exponent(amax);
        if (half == 0) __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(e + 127), rs, row * ldsc + blk, 0, 0);
        const int rowb = row * ldq + f0 + 4 * half;
#pragma unroll
        for (int b = 0; b < 4; ++b) {   // features f0 + 8 b + 4 half + 0..3
            float q[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float t = ldexpf(v[4 * b + u], -e);
                q[u] = t > 448.0f ? 448.0f : (t < -448.0f ? -448.0f : t);   // NaN stays NaN
            }
            int pk = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
            pk = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], pk, true);
            __builtin_amdgcn_raw_buffer_store_b32((uint32_t)pk, rq, rowb + 8 * b, 0, 0);
        }
    }
}

// gate_up_epi_direct for a tile that may hold dense-routed expert features:
// the calling wave's 32-feature block is wholly shared (gate_up_epi_direct)
// or wholly one expert's, whose h is silu(g) * u times the token's route
// weight for that expert (from s_route, as gate_up_epi_block computes it);
// bf16 pairs straight from the accumulators.
template <int TMW>
__device__ __forceinline__ void gate_up_epi_direct_routed(const GateUpArgs& a, const f32x16 (&acc)[TMW][2],
                                                          int64_t m0, int64_t n0, int wm0, int wn0,
                                                          const int (*s_route)[kMaxTopK]) {
    const int64_t pbase = n0 + wn0;   // packed row of the wave's gate block
    const int64_t fblock = pbase >> 1;
    if (a.ids == nullptr || fblock < a.shared_feats) {
        gate_up_epi_direct<TMW, true>(a, acc, m0, n0, wm0, wn0);
        return;
    }
    const int expert = (int)((fblock - a.shared_feats) / a.expert_feats);
    const int lane = threadIdx.x & 63, r = lane & 31;
    const float sg = a.w_scale ? a.w_scale[pbase + r] : 1.0f;
    const float su = a.w_scale ? a.w_scale[pbase + 32 + r] : 1.0f;
    const int64_t mlim = a.M - m0 < 64 * TMW ? a.M - m0 : 64 * TMW;
    const int ld2 = (int)a.ldh * 2;
    const auto rsrc = make_rsrc(static_cast<bf16_t*>(a.h) + m0 * a.ldh, (uint32_t)(mlim * ld2));
    const int lb = pair_lane_offset(wm0, (int)(fblock + r), ld2);
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int* rr = s_route[wm0 + tm * 32 + acc_row(lane, i)];
            float tw = 0.f;
#pragma unroll
            for (int j = 0; j < kMaxTopK; ++j) tw += (rr[j] == expert) ? a.rw[j] : 0.f;
            v[i] = silu_f(acc[tm][0][i] * sg) * (acc[tm][1][i] * su) * tw;
        }
        store_bf16_pairs(rsrc, lb + tm * 32 * ld2, ld2, v);
    }
}

// gate|up + SwiGLU over bf16 activations and weights, K a multiple of 64.
// ROUTED: the launch covers dense-routed expert columns (route gather and
// per-token expert weights for the tiles that hold them).  TMW = 4: 256-row
// tiles; 2: 128-row tiles (the trailing columns of a launch whose last round
// of 256-row tiles would leave most CUs idle).  SAVE: also write the raw
// gate|up outputs to a.gu (training forward).
template <bool ROUTED, int TMW, bool SAVE = false, bool FP8 = false>
__global__ __launch_bounds__(512, 1) void k_gate_up_pp(GateUpArgs a) {
    using Shape = ShapePP<TMW>;
    using Kind = KindBF16;
    constexpr int BM = Shape::BM;
    extern __shared__ __align__(16) char lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * (BM / 2), wn0 = wig * 64;
    const int64_t m0 = (int64_t)blockIdx.x * BM;
    const int64_t n0 = a.n_base + (int64_t)blockIdx.y * 256;

    // per-row data of the epilogue (read there, after the loop's barriers);
    // gathered before any direct load is issued, so that the loop's load
    // counters only count direct loads
    __shared__ float s_rscale[BM];
    __shared__ int s_route[ROUTED ? BM : 1][kMaxTopK];
    bool gathered = false;
    if (a.row_scale != nullptr) {
        if (threadIdx.x < BM) {
            const int64_t row = m0 + threadIdx.x;
            s_rscale[threadIdx.x] = row < a.M ? a.row_scale[row] : 0.0f;
        }
        gathered = true;
    }
    if constexpr (ROUTED) {
        if (a.ids != nullptr && ((n0 + 256) >> 1) > a.shared_feats) {
            gate_up_routes<Shape, true>(a, m0, n0, s_route);
            gathered = true;
        }
    }
    if (gathered) __syncthreads();

    PPRows<BM> ap;
    std::conditional_t<FP8, PPRows64, PPRows<256>> bp;
    if (group == 1) {
        ap.init(a.x, m0, a.M, a.ldx * (int64_t)sizeof(bf16_t), wig);
    } else {
        if constexpr (FP8)
            bp.init(a.w, n0, n0 + 256, a.ldw, wig);
        else
            bp.init(a.w, n0, n0 + 256, a.ldw * (int64_t)sizeof(bf16_t), wig);
    }
    f32x16 acc[TMW][2];
    zero_acc<Kind>(acc);
    using Lay = std::conditional_t<FP8, PPLayoutF8<TMW>, PPLayoutK<TMW>>;
    // bf16 weights without row scales: each group stores its h rows straight
    // from the accumulators (group 0 while group 1 multiplies the last
    // stage); otherwise, and for the saving 256-row tiles (whose registers
    // would spill), through the LDS tile
    const bool direct = !FP8 && (TMW == 2 || !SAVE) && a.row_scale == nullptr;
    pp_main<TMW, Lay>(ap, bp, a.K / 64, lds, group, wm0, wn0, acc, [&](const f32x16 (&c)[TMW][2]) {
        if (direct) {
            if constexpr (ROUTED)
                gate_up_epi_direct_routed<TMW>(a, c, m0, n0, wm0, wn0, s_route);
            else
                gate_up_epi_direct<TMW, true>(a, c, m0, n0, wm0, wn0);
            return;
        }
        gate_up_epi_tile<Kind, Shape, ROUTED>(a, c, n0, lds, s_route, a.row_scale != nullptr ? s_rscale : nullptr);
    });
    if constexpr (SAVE) gate_up_save<Kind, Shape>(a, acc, m0, n0, a.n_base + (int64_t)gridDim.y * 256);
    if (!direct) gate_up_epi_store<Kind, Shape>(a, m0, n0, lds);
}

// gate_up_save for the persistent kernel: the raw gate|up outputs of the
// calling wave (times the e4m3 scale) to a.gu, offsets built like
// gate_up_epi_direct's so that none is hoisted out of the tile loop.  gu is
// read only by the backward, so it is stored with the non-temporal hint
// (C2 training step, 218 MB of gu: forward + backward 1.116 -> 1.095 ms).
template <int TMW>
__device__ __forceinline__ void gate_up_save_direct(const GateUpArgs& a, const f32x16 (&acc)[TMW][2], int64_t m0,
                                                    int64_t n0, int wm0, int wn0) {
    const int lane = threadIdx.x & 63, r = lane & 31;
    const int64_t mlim = a.M - m0 < 64 * TMW ? a.M - m0 : 64 * TMW;
    int ld2 = (int)a.ldgu * 2;
    asm volatile("" : "+s"(ld2));
    const auto rsrc = make_rsrc(static_cast<bf16_t*>(a.gu) + m0 * a.ldgu, (uint32_t)(mlim * ld2));
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
        const int64_t col = n0 + wn0 + tn * 32 + r;
        const float sc = a.w_scale ? a.w_scale[col] : 1.0f;
        const int lb = pair_lane_offset(wm0, (int)col, ld2);
#pragma unroll
        for (int tm = 0; tm < TMW; ++tm) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = acc[tm][tn][i] * sc;
            store_bf16_pairs<kStoreStream>(rsrc, lb + tm * 32 * ld2, ld2, v);
        }
    }
}

// Persistent gate|up + SwiGLU (shared columns: no routing epilogue, no row
// scales): one workgroup per CU runs tiles blockIdx.x, + gridDim.x, ... of
// the tiles_m x (n_tiles / tiles_m) 256-row tiles as one stream of K stages
// (pp_stream), writing each tile's h from registers while the next tile's
// stages load and multiply.  SAVE: also the raw gate|up outputs (a.gu).
// A8 (with FP8): e4m3 activations too, a.x holding the codes (row stride
// a.ldx bytes) and a.row_scale their per-token scales: 128 K values per
// stage on the e4m3 MFMA (W8A8).  MXH (with A8): transposed accumulator
// blocks, and h leaves as block-scaled e4m3 (gate_up_epi_mx).
template <int TMW, bool SAVE, bool FP8, bool A8 = false, bool MXH = false>
__global__ __launch_bounds__(512, 1) void k_gate_up_pps(GateUpArgs a, int64_t tiles_m, int64_t n_tiles) {
    static_assert(!A8 || (FP8 && !SAVE), "W8A8 is the inference form of the e4m3 weights");
    static_assert(!MXH || A8, "block-scaled h is written by the W8A8 kernel");
    constexpr int BM = 64 * TMW;
    extern __shared__ __align__(16) char lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * (BM / 2), wn0 = wig * 64;
    const int64_t G = gridDim.x;
    const int ntiles = (int)((n_tiles - (int64_t)blockIdx.x + G - 1) / G);
    if (ntiles <= 0) return;
    const bool xcd_rows = (tiles_m & 7) == 0 && (G & 7) == 0;
    auto coords = [&](int i, int64_t& m0, int64_t& n0) {
        uint32_t mt, nt;
        pps_tile((uint32_t)blockIdx.x + (uint32_t)i * (uint32_t)G, (uint32_t)tiles_m, (uint32_t)(n_tiles / tiles_m),
                 xcd_rows, mt, nt);
        m0 = (int64_t)mt * BM;
        n0 = a.n_base + (int64_t)nt * 256;
    };
    const int64_t ldx_b = A8 ? a.ldx : a.ldx * (int64_t)sizeof(bf16_t);
    const int64_t ldw_b = FP8 ? a.ldw : a.ldw * (int64_t)sizeof(bf16_t);

    PPRows<BM> ap;
    std::conditional_t<FP8 && !A8, PPRows64, PPRows<256>> bp;
    int64_t m0, n0;
    coords(0, m0, n0);
    if (group == 1) {
        ap.init(a.x, m0, a.M, ldx_b, wig);
    } else {
        if constexpr (FP8)
            bp.init(a.w, n0, n0 + 256, ldw_b, wig);
        else
            bp.init(a.w, n0, n0 + 256, ldw_b, wig);
    }
    f32x16 acc[TMW][2];
    zero_acc<KindBF16>(acc);
    using Lay = std::conditional_t<A8, PPLayoutK8<TMW, true>,
                                   std::conditional_t<FP8, PPLayoutF8<TMW, true>, PPLayoutK<TMW, true>>>;
    pp_stream<TMW, Lay, MXH>(
        ap, bp, A8 ? a.K / 128 : a.K / 64, ntiles, lds, group, wm0, wn0, acc,
        [&](int i) {   // i >= ntiles: no rows (the refills past the last stage load zeros)
            int64_t tm0, tn0;
            coords(i, tm0, tn0);
            ap.retarget(a.x, tm0, i < ntiles ? a.M : tm0, ldx_b);
        },
        [&](int i) {
            int64_t tm0, tn0;
            coords(i, tm0, tn0);
            bp.retarget(a.w, tn0, i < ntiles ? tn0 + 256 : tn0, ldw_b);
        },
        [&](int i, const f32x16 (&c)[TMW][2]) {
            int64_t tm0, tn0;
            coords(i, tm0, tn0);
            if constexpr (SAVE) gate_up_save_direct<TMW>(a, c, tm0, tn0, wm0, wn0);
            if constexpr (MXH)
                gate_up_epi_mx<TMW>(a, c, tm0, tn0, wm0, wn0);
            else if constexpr (A8)
                gate_up_epi_direct<TMW, true, true>(a, c, tm0, tn0, wm0, wn0);
            else
                gate_up_epi_direct<TMW, !FP8>(a, c, tm0, tn0, wm0, wn0);
        });
}

// ---------------------------------------------------------------------------
// K4: shared down + weighted un-permute + combine
// ---------------------------------------------------------------------------
template <class Kind, bool FP8, class Shape, bool GROUPED = false>
__global__ __launch_bounds__(Shape::NT) void k_down_combine(DownArgs a) {
    using T = typename Kind::T;
    extern __shared__ __align__(16) char lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = (int64_t)blockIdx.y * Shape::BN;

    if constexpr (GROUPED) {
        __shared__ int s_tile[3];
        grouped_tile<Shape::BM>(a.offsets, a.E, (int)blockIdx.x, s_tile);
        if (s_tile[0] < 0) return;
        const int64_t e = s_tile[0];
        m0 = s_tile[1];
        a.M = s_tile[2];
        a.w = static_cast<const char*>(a.w) + e * a.w_expert_stride * (FP8 ? 1 : (int64_t)sizeof(T));
        if (a.w_scale) a.w_scale += e * a.scale_expert_stride;
    }
    typename AProvOf<Shape>::type ap;
    init_a<Shape>(ap, a.h, m0, a.M, a.ldh * (int64_t)sizeof(T), a.K * (int)sizeof(T));
    typename BProvOf<Kind, FP8, Shape>::type bp;
    init_b<Kind, FP8, Shape>(bp, a.w, a.ldw, n0, a.K);

    // y row of each (tile row, slot), clamped so that a malformed route table
    // cannot become a wild read; gathered while the first stages load.
    __shared__ int s_yrow[Shape::BM][kMaxTopK];
    if (a.y != nullptr && threadIdx.x < Shape::BM) {
        const int64_t row = m0 + threadIdx.x;
        const int64_t last = (int64_t)a.top_k * a.M - 1;
        for (int j = 0; j < kMaxTopK; ++j) {
            int64_t v = (j < a.top_k && row < a.M) ? a.inverse[(int64_t)j * a.M + row] : 0;
            s_yrow[threadIdx.x][j] = (int)(v < 0 ? 0 : (v > last ? last : v));
        }
    }

    f32x16 acc[Shape::TM][Shape::TN];
    zero_acc<Kind>(acc);
    tile_loop<Kind, Shape>(ap, bp, a.K, lds, wm0, wn0, acc);

    const int r = lane & 31;
    float cscale[Shape::TN];
#pragma unroll
    for (int tn = 0; tn < Shape::TN; ++tn) {
        const int64_t col = n0 + wn0 + tn * 32 + r;
        cscale[tn] = a.shared_scale * ((a.w_scale && col < a.N) ? a.w_scale[col] : 1.0f);
    }
    const T* y = static_cast<const T*>(a.y);
    const T* res = static_cast<const T*>(a.residual);
    T* out = static_cast<T*>(a.out);
    if constexpr (sizeof(T) == 2) {
        // bf16: the scaled shared term goes to LDS as a [BM][BN] tile (rows
        // padded by 16 bytes); the routed gather, residual and store then run
        // over 16-byte chunks of 8 columns.
        constexpr int kORowBytes = Shape::BN * 2 + 16;
#pragma unroll
        for (int tm = 0; tm < Shape::TM; ++tm)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int rl = wm0 + tm * 32 + acc_row(lane, i);
#pragma unroll
                for (int tn = 0; tn < Shape::TN; ++tn)
                    *reinterpret_cast<T*>(lds + rl * kORowBytes + (wn0 + tn * 32 + r) * 2) =
                        from_f32<T>(acc[tm][tn][i] * cscale[tn]);
            }
        __syncthreads();
        constexpr int kChunksPerRow = Shape::BN / 8;
        for (int q = threadIdx.x; q < Shape::BM * kChunksPerRow; q += Shape::NT) {
            const int rl = q / kChunksPerRow, c = q % kChunksPerRow;
            const int64_t row = m0 + rl;
            const int64_t col = n0 + c * 8;
            if (row >= a.M || col >= a.N) continue;
            const u32x4 sv = *reinterpret_cast<const u32x4*>(lds + rl * kORowBytes + c * 16);
            const bf16x8 sb = __builtin_bit_cast(bf16x8, sv);
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (float)sb[e];
            if (a.vec_ok && col + 8 <= a.N) {
                if (y != nullptr) {
                    float acc_r[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                    for (int j = 0; j < a.top_k; ++j) {
                        const bf16x8 yv = __builtin_bit_cast(
                            bf16x8, *reinterpret_cast<const u32x4*>(y + (int64_t)s_yrow[rl][j] * a.ldy + col));
#pragma unroll
                        for (int e = 0; e < 8; ++e) acc_r[e] += a.rw[j] * (float)yv[e];
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] += a.routed_scale * acc_r[e];
                }
                if (res != nullptr) {
                    const bf16x8 rv = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(res + row * a.ldr + col));
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] += (float)rv[e];
                }
                bf16x8 ov;
#pragma unroll
                for (int e = 0; e < 8; ++e) ov[e] = (bf16_t)v[e];
                *reinterpret_cast<u32x4*>(out + row * a.ldo + col) = __builtin_bit_cast(u32x4, ov);
            } else {
                for (int e = 0; e < 8 && col + e < a.N; ++e) {
                    float x = v[e];
                    if (y != nullptr) {
                        float sacc = 0.f;
                        for (int j = 0; j < a.top_k; ++j)
                            sacc += a.rw[j] * to_f32(y[(int64_t)s_yrow[rl][j] * a.ldy + col + e]);
                        x += a.routed_scale * sacc;
                    }
                    if (res != nullptr) x += to_f32(res[row * a.ldr + col + e]);
                    out[row * a.ldo + col + e] = from_f32<T>(x);
                }
            }
        }
    } else {
        // f32: the tile would not fit in LDS; combine straight from registers
#pragma unroll
        for (int tm = 0; tm < Shape::TM; ++tm) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int rl = wm0 + tm * 32 + acc_row(lane, i);
                const int64_t row = m0 + rl;
                if (row >= a.M) continue;
#pragma unroll
                for (int tn = 0; tn < Shape::TN; ++tn) {
                    const int64_t col = n0 + wn0 + tn * 32 + r;
                    if (col >= a.N) continue;
                    float v = acc[tm][tn][i] * cscale[tn];
                    if (y != nullptr) {
                        float sacc = 0.f;
                        for (int j = 0; j < a.top_k; ++j)
                            sacc += a.rw[j] * to_f32(y[(int64_t)s_yrow[rl][j] * a.ldy + col]);
                        v += a.routed_scale * sacc;
                    }
                    if (res != nullptr) v += to_f32(res[row * a.ldr + col]);
                    out[row * a.ldo + col] = from_f32<T>(v);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// K3: routed experts (gate|up -> SwiGLU -> down) over the partition
// ---------------------------------------------------------------------------
// Tile t of the launch maps to expert e and rows [row0, row0 + 128) of its
// segment; tiles past the last segment exit.  Phase 1 streams the gathered
// token rows against 64-feature chunks of the expert's packed gate|up rows and
// leaves h (128 rows x F_pad features) in LDS in the operand layout; phase 2
// streams the expert's packed down rows in 128-column chunks against it.
template <class Kind, bool FP8, class Shape>
__global__ __launch_bounds__(Shape::NT) void k_routed_experts(RoutedArgs a) {
    using T = typename Kind::T;
    constexpr int SE = Kind::kStageElems;
    constexpr int EPC = Kind::kPerChunk;
    extern __shared__ __align__(16) char lds[];
    char* hs = lds + Shape::kLdsBytes;
    const int hs_stage_bytes = Shape::BM * kRowBytes;

    // tile -> (expert, row range)
    __shared__ int s_tile[3];
    if (threadIdx.x == 0) {
        int acc_tiles = 0, e_sel = -1, row0 = 0, row1 = 0;
        for (int e = 0; e < a.E; ++e) {
            const int b = a.offsets[e], c = a.offsets[e + 1] - b;
            const int nt = (c + Shape::BM - 1) / Shape::BM;
            if ((int)blockIdx.x < acc_tiles + nt) {
                e_sel = e;
                row0 = b + ((int)blockIdx.x - acc_tiles) * Shape::BM;
                row1 = min(row0 + Shape::BM, b + c);
                break;
            }
            acc_tiles += nt;
        }
        s_tile[0] = e_sel;
        s_tile[1] = row0;
        s_tile[2] = row1;
    }
    __syncthreads();
    const int e = s_tile[0];
    if (e < 0) return;
    const int64_t row0 = s_tile[1];
    const int rows = s_tile[2] - s_tile[1];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int r = lane & 31;

    const int64_t gu_rows = 2 * (int64_t)a.F_pad;
    const char* wgu = static_cast<const char*>(a.wgu) + (int64_t)e * gu_rows * a.wgu_ld * a.w_elem_bytes;
    const float* sgu = a.sgu ? a.sgu + (int64_t)e * gu_rows : nullptr;
    const char* wd = static_cast<const char*>(a.wd) + (int64_t)e * a.H_pad * a.wd_ld * a.w_elem_bytes;
    const float* sd = a.sd ? a.sd + (int64_t)e * a.H_pad : nullptr;

    // ---- phase 1: h = silu(x Wg) * (x Wu) into LDS
    const int nchunks = a.F_pad / 64;
    for (int fc = 0; fc < nchunks; ++fc) {
        BufRows<Shape::BM, Shape::NT> ap;
        ap.rsrc = make_rsrc(a.x, (uint32_t)(a.n_tokens * a.ldx * (int64_t)sizeof(T)));
        ap.kbytes = a.K * (int)sizeof(T);
#pragma unroll
        for (int j = 0; j < BufRows<Shape::BM, Shape::NT>::kChunks; ++j) {
            const int row = (threadIdx.x >> 3) + (Shape::NT / 8) * j;
            if (row < rows) {
                const int64_t t = (int64_t)((uint64_t)a.sorted[row0 + row] % (uint64_t)a.n_tokens);
                ap.row_off[j] = (int)(t * a.ldx * (int64_t)sizeof(T));
            } else {
                ap.row_off[j] = kOutOfRange;
            }
        }
        typename BProvSel<Kind, FP8, Shape::BN, Shape::NT>::type bp;
        init_bprov<Kind, FP8, Shape::BN, Shape::NT>(bp, wgu, a.wgu_ld, (int64_t)fc * 128, a.K);
        f32x16 acc[Shape::TM][Shape::TN];
        zero_acc<Kind>(acc);
        tile_loop<Kind, Shape>(ap, bp, a.K, lds, wm0, wn0, acc);

        const int prow = fc * 128 + wn0;          // packed row of this wave's gate tile
        const int feat = (prow >> 1) + r;          // feature index in [0, F_pad)
        const float sg = sgu ? sgu[prow + r] : 1.0f;
        const float su = sgu ? sgu[prow + 32 + r] : 1.0f;
        const int st = feat / SE, el = feat % SE;
        char* hcol = hs + st * hs_stage_bytes;
#pragma unroll
        for (int tm = 0; tm < Shape::TM; ++tm) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = wm0 + tm * 32 + acc_row(lane, i);
                const float g = acc[tm][0][i] * sg;
                const float u = acc[tm][1][i] * su;
                T* dst = reinterpret_cast<T*>(hcol + lds_byte(row, el / EPC)) + (el % EPC);
                *dst = from_f32<T>(silu_f(g) * u);
            }
        }
    }

    // ---- phase 2: y = h Wd, 128 output columns at a time
    const int ncol = (a.H + Shape::BN - 1) / Shape::BN;
    T* y = static_cast<T*>(a.y);
    for (int oc = 0; oc < ncol; ++oc) {
        typename BProvSel<Kind, FP8, Shape::BN, Shape::NT>::type bp;
        init_bprov<Kind, FP8, Shape::BN, Shape::NT>(bp, wd, a.wd_ld, (int64_t)oc * Shape::BN, a.W);
        f32x16 acc[Shape::TM][Shape::TN];
        zero_acc<Kind>(acc);
        tile_loop_lds_a<Kind, Shape>(hs, hs_stage_bytes, bp, a.W, lds, wm0, wn0, acc);
#pragma unroll
        for (int tn = 0; tn < Shape::TN; ++tn) {
            const int64_t col = (int64_t)oc * Shape::BN + wn0 + tn * 32 + r;
            if (col >= a.H) continue;
            const float cs = sd ? sd[col] : 1.0f;
#pragma unroll
            for (int tm = 0; tm < Shape::TM; ++tm) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = wm0 + tm * 32 + acc_row(lane, i);
                    if (row < rows) y[(row0 + row) * a.ldy + col] = from_f32<T>(acc[tm][tn][i] * cs);
                }
            }
        }
    }
}

// Row tile rt (256 rows) of a K1 partition: expert e and partition rows
// [r0, r1); e = -1 past the last tile.  A uniform walk over the E segments.
__device__ __forceinline__ void pps_grouped_rows(const int32_t* offsets, int E, int rt, int& e, int& r0, int& r1) {
    int acc_tiles = 0;
    e = -1;
    r0 = r1 = 0;
    for (int q = 0; q < E; ++q) {
        const int b = offsets[q], c = offsets[q + 1] - b;
        const int nt = (c + 255) >> 8;
        if (rt < acc_tiles + nt) {
            e = q;
            r0 = b + (rt - acc_tiles) * 256;
            r1 = r0 + 256 < b + c ? r0 + 256 : b + c;
            return;
        }
        acc_tiles += nt;
    }
}

// Expert-grouped down (K3's second GEMM) as a persistent ping-pong stream:
// y[r, :] = (h[r, :] We^T) * scale_e for the partition rows r of expert e's
// segment, over (row tile, column tile) pairs of 256 x 256.  The row tiles
// are padded to a multiple of 8 and tile t is row tile (t % 8) + 8 q, column
// tile j - q n_ct with j = t / 8, q = j / n_ct: the column tiles of a row
// tile run on one XCD (workgroups go to XCD t % 8), next to each other, so
// its h rows are read once into that XCD's L2.  Padding tiles load nothing
// and store nothing.  K (the expert width) is a multiple of 64.  STREAM: the
// y rows are stored with the non-temporal hint (y is read only by the shared
// down, after the shared gate|up; see launch_down_grouped_pps).
template <bool FP8, bool STREAM>
__global__ __launch_bounds__(512, 1) void k_down_grouped_pps(DownArgs a) {
    extern __shared__ __align__(16) char lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * 128, wn0 = wig * 64;
    int n_rt = 0;
    for (int q = 0; q < a.E; ++q) n_rt += (a.offsets[q + 1] - a.offsets[q] + 255) >> 8;
    const int n_ct = (a.N + 255) >> 8;
    const int n_tiles = ((n_rt + 7) & ~7) * n_ct;
    const int G = (int)gridDim.x;
    const int ntiles = (n_tiles - (int)blockIdx.x + G - 1) / G;
    if (ntiles <= 0) return;
    auto tile = [&](int i, int& e, int& r0, int& r1, int& n0) {
        const uint32_t t = blockIdx.x + (uint32_t)i * (uint32_t)G;
        const uint32_t j = t >> 3, q = j / (uint32_t)n_ct;
        n0 = (int)(j - q * (uint32_t)n_ct) * 256;
        pps_grouped_rows(a.offsets, a.E, (int)((t & 7) + 8 * q), e, r0, r1);
        if (i >= ntiles) e = -1;   // past the workgroup's tiles: nothing
    };
    const int64_t ldh_b = a.ldh * 2;
    const int64_t ldw_b = FP8 ? a.ldw : a.ldw * 2;
    const int64_t wstride_b = a.w_expert_stride * (FP8 ? 1 : 2);
    auto point_a = [&](auto& ap, int i, bool first) {
        int e, r0, r1, n0;
        tile(i, e, r0, r1, n0);
        if (first)
            ap.init(a.h, r0, e >= 0 ? r1 : r0, ldh_b, wig);
        else
            ap.retarget(a.h, r0, e >= 0 ? r1 : r0, ldh_b);
    };
    auto point_b = [&](auto& bp, int i, bool first) {
        int e, r0, r1, n0;
        tile(i, e, r0, r1, n0);
        const char* w = static_cast<const char*>(a.w) + (int64_t)(e < 0 ? 0 : e) * wstride_b;
        if (first)
            bp.init(w, n0, e >= 0 ? a.N : n0, ldw_b, wig);
        else
            bp.retarget(w, n0, e >= 0 ? a.N : n0, ldw_b);
    };
    PPRows<256> ap;
    std::conditional_t<FP8, PPRows64, PPRows<256>> bp;
    if (group == 1)
        point_a(ap, 0, true);
    else
        point_b(bp, 0, true);
    f32x16 acc[4][2];
    zero_acc<KindBF16>(acc);
    using Lay = std::conditional_t<FP8, PPLayoutF8<4, true>, PPLayoutK<4, true>>;
    pp_stream<4, Lay>(
        ap, bp, a.K / 64, ntiles, lds, group, wm0, wn0, acc, [&](int i) { point_a(ap, i, false); },
        [&](int i) { point_b(bp, i, false); },
        [&](int i, const f32x16 (&c)[4][2]) {
            int e, r0, r1, n0;
            tile(i, e, r0, r1, n0);
            if (e < 0) return;
            int ld2 = (int)a.ldo * 2;
            asm volatile("" : "+s"(ld2));   // keeps the offsets below out of the caller's loop
            const auto rsrc = make_rsrc(static_cast<bf16_t*>(a.out) + (int64_t)r0 * a.ldo, (uint32_t)((r1 - r0) * ld2));
            const int r = threadIdx.x & 31;
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const int col = n0 + wn0 + tn * 32 + r;
                const float cs = a.shared_scale *
                                 ((a.w_scale != nullptr && col < a.N) ? a.w_scale[e * a.scale_expert_stride + col] : 1.0f);
                const int lb = pair_lane_offset(wm0, col, ld2) | (col < a.N ? 0 : kOutOfRange);
#pragma unroll
                for (int tm = 0; tm < 4; ++tm) {
                    float v[16];
#pragma unroll
                    for (int q = 0; q < 16; ++q) v[q] = c[tm][tn][q] * cs;
                    store_bf16_pairs<STREAM ? kStoreStream : 0>(rsrc, lb + tm * 32 * ld2, ld2, v);
                }
            }
        });
}

// Expert-grouped gate|up + SwiGLU (K3's first GEMM) as a persistent
// ping-pong stream: h[r, :] = SwiGLU(x[gather[r] % gather_mod] We_gu^T) for
// the partition rows r of expert e's segment, over (row tile, packed column
// tile) pairs of 256 x 256 in the order of k_down_grouped_pps.  When group 1
// moves to a new tile each of its lanes loads one tile row's gather index
// and keeps that row's byte offset in LDS (s_goff); rows past the segment
// and padding tiles load zeros, and their h rows are not written.  The
// packed gate|up rows per expert are a multiple of 256; no row scales.
template <bool FP8>
__global__ __launch_bounds__(512, 1) void k_gate_up_grouped_pps(GateUpArgs a) {
    extern __shared__ __align__(16) char lds[];
    __shared__ int s_goff[256];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * 128, wn0 = wig * 64;
    int n_rt = 0;
    for (int q = 0; q < a.E; ++q) n_rt += (a.offsets[q + 1] - a.offsets[q] + 255) >> 8;
    const int n_ct = (int)(a.w_expert_stride / a.ldw) >> 8;   // packed rows per expert / 256
    const int n_tiles = ((n_rt + 7) & ~7) * n_ct;
    const int G = (int)gridDim.x;
    const int ntiles = (n_tiles - (int)blockIdx.x + G - 1) / G;
    if (ntiles <= 0) return;
    auto tile = [&](int i, int& e, int& r0, int& r1, int& n0) {
        const uint32_t t = blockIdx.x + (uint32_t)i * (uint32_t)G;
        const uint32_t j = t >> 3, q = j / (uint32_t)n_ct;
        n0 = (int)(j - q * (uint32_t)n_ct) * 256;
        pps_grouped_rows(a.offsets, a.E, (int)((t & 7) + 8 * q), e, r0, r1);
        if (i >= ntiles) e = -1;
    };
    const int64_t ldx_b = a.ldx * 2;
    const int64_t ldw_b = FP8 ? a.ldw : a.ldw * 2;
    const int64_t wstride_b = a.w_expert_stride * (FP8 ? 1 : 2);
    // group 1: the x byte offsets of tile i's rows into s_goff (one row per lane)
    auto gather_rows = [&](int i) {
        int e, r0, r1, n0;
        tile(i, e, r0, r1, n0);
        const int r = (int)threadIdx.x - 256;
        int off = kOutOfRange;
        if (e >= 0 && r0 + r < r1) {
            const int64_t v = a.gather[r0 + r];
            const int64_t t = (int64_t)((uint64_t)v % (uint64_t)a.gather_mod);
            off = (int)(t * ldx_b);
        }
        s_goff[r] = off;
    };
    auto point_b = [&](auto& bp, int i, bool first) {
        int e, r0, r1, n0;
        tile(i, e, r0, r1, n0);
        const char* w = static_cast<const char*>(a.w) + (int64_t)(e < 0 ? 0 : e) * wstride_b;
        if (first)
            bp.init(w, n0, e >= 0 ? n0 + 256 : n0, ldw_b, wig);
        else
            bp.retarget(w, n0, e >= 0 ? n0 + 256 : n0, ldw_b);
    };
    PPGather ap;
    std::conditional_t<FP8, PPRows64, PPRows<256>> bp;
    if (group == 1) {
        ap.init(a.x, a.gather_mod * ldx_b, s_goff, wig);
        gather_rows(0);
    } else {
        point_b(bp, 0, true);
    }
    f32x16 acc[4][2];
    zero_acc<KindBF16>(acc);
    using Lay = std::conditional_t<FP8, PPLayoutF8<4, true>, PPLayoutK<4, true>>;
    pp_stream<4, Lay>(
        ap, bp, a.K / 64, ntiles, lds, group, wm0, wn0, acc, [&](int i) { gather_rows(i); },
        [&](int i) { point_b(bp, i, false); },
        [&](int i, const f32x16 (&c)[4][2]) {
            int e, r0, r1, n0;
            tile(i, e, r0, r1, n0);
            if (e < 0) return;
            GateUpArgs t = a;
            t.M = r1;
            if (t.w_scale) t.w_scale += (int64_t)e * a.scale_expert_stride;
            gate_up_epi_direct<4, !FP8>(t, c, r0, n0, wm0, wn0);
        });
}

// ---------------------------------------------------------------------------
// k_combine: routed un-permute without a shared branch
// ---------------------------------------------------------------------------
template <class T>
__global__ __launch_bounds__(256) void k_combine(CombineArgs a) {
    const int64_t total = a.M * a.N;
    const T* y = static_cast<const T*>(a.y);
    const T* res = static_cast<const T*>(a.residual);
    T* out = static_cast<T*>(a.out);
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = idx / a.N, col = idx - row * a.N;
        float s = 0.f;
        for (int j = 0; j < a.top_k; ++j) {
            int64_t r = a.inverse[(int64_t)j * a.M + row];
            r = r < 0 ? 0 : (r >= a.top_k * a.M ? a.top_k * a.M - 1 : r);
            s += a.rw[j] * to_f32(y[r * a.ldy + col]);
        }
        float v = a.routed_scale * s;
        if (res != nullptr) v += to_f32(res[row * a.ldr + col]);
        out[row * a.ldo + col] = from_f32<T>(v);
    }
}

// Tile of a 1-D down launch over tiles_m x tiles_n 256 x 256 tiles.
// Workgroups go to the 8 XCDs round-robin (id % 8).  With tiles_m a multiple
// of 8, XCD x takes row tiles x, x + 8, ..., each with every column tile in
// consecutive ids, so a round reads each row panel of h into one L2 once
// and all its column tiles use it there (C5: 128 x 8 tiles, 4 rounds; in
// row-fastest order each h panel came back in all four rounds from HBM, 369 MB
// of h being more than the 256 MB Infinity Cache).  Other shapes: row tiles
// fastest.
__device__ __forceinline__ void down_tile(uint32_t id, uint32_t tiles_m, uint32_t tiles_n, uint32_t& mt,
                                          uint32_t& nt) {
    if ((tiles_m & 7) == 0) {
        const uint32_t x = id & 7, j = id >> 3;
        nt = j % tiles_n;
        mt = x + 8 * (j / tiles_n);
    } else {
        mt = id % tiles_m;
        nt = id / tiles_m;
    }
}

// LDS stages of k_down_pp: three with e4m3 weights and bf16 h (48 KiB each;
// C5's h does not fit the Infinity Cache, and its HBM reads need the longer
// lead), else two.
template <bool FP8, bool A8>
constexpr int kDownPPStages = (FP8 && !A8) ? 3 : 2;

// K4 on the ping-pong main loop (bf16 activations; bf16 or, FP8, e4m3
// weights expanded at the fragment read; K a multiple of 64): 256x256 tiles
// over the hidden columns; weight rows past the hidden size load as zero (the
// last tile of H = 896 multiplies 128 of them).  Epilogue: each
// group writes shared_scale * column scale * acc for its rows to LDS as bf16
// (the tile kernel's rounding), then every thread adds the route-weighted y
// rows and the residual over 16-byte chunks and stores.  A8 (with FP8): h
// holds block-scaled e4m3 codes (a.h, ldh bytes per row; a.hs the E8M0
// scales), multiplied on the e4m3 MFMA with the scales in its operand, 128 K
// values per stage.
template <bool FP8, bool A8 = false>
__global__ __launch_bounds__(512, 1) void k_down_pp(DownArgs a) {
    static_assert(!A8 || FP8, "block-scaled h goes with e4m3 weights");
    constexpr int BM = 256, BN = 256;
    using T = bf16_t;
    extern __shared__ __align__(16) char lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * (BM / 2), wn0 = wig * 64;
    const int lane = threadIdx.x & 63;
    uint32_t mt, nt;
    down_tile(blockIdx.x, (uint32_t)((a.M + BM - 1) / BM), (uint32_t)((a.N + BN - 1) / BN), mt, nt);
    const int64_t m0 = (int64_t)mt * BM;
    const int64_t n0 = (int64_t)nt * BN;

    // y row of each (tile row, slot), clamped so that a malformed inverse
    // cannot become a wild read; gathered before any direct load is issued
    __shared__ int s_yrow[BM][kMaxTopK];
    if (a.y != nullptr) {
        if (threadIdx.x < BM) {
            const int64_t row = m0 + threadIdx.x;
            const int64_t last = (int64_t)a.top_k * a.M - 1;
            for (int j = 0; j < kMaxTopK; ++j) {
                int64_t v = (j < a.top_k && row < a.M) ? a.inverse[(int64_t)j * a.M + row] : 0;
                s_yrow[threadIdx.x][j] = (int)(v < 0 ? 0 : (v > last ? last : v));
            }
        }
        __syncthreads();
    }

    PPRows<BM> ap;
    std::conditional_t<FP8 && !A8, PPRows64, PPRows<256>> bp;
    if (group == 1) {
        ap.init(a.h, m0, a.M, A8 ? a.ldh : a.ldh * (int64_t)sizeof(T), wig);
    } else {   // rows past N load as zero
        if constexpr (FP8)
            bp.init(a.w, n0, a.N, a.ldw, wig);
        else
            bp.init(a.w, n0, a.N, a.ldw * (int64_t)sizeof(T), wig);
    }
    f32x16 acc[4][2];
    zero_acc<KindBF16>(acc);
    constexpr int kORowBytes = BN * 2 + 16;
    using Lay = std::conditional_t<A8, PPLayoutK8<4, true>, std::conditional_t<FP8, PPLayoutF8<4>, PPLayoutK<4>>>;
    std::conditional_t<A8, PPBlockScales, PPNoScales> sc;
    if constexpr (A8) sc.init(a.hs, a.ldhs, m0, a.M, wm0);
    // nothing to add to the product (no routed rows, no residual): each
    // group stores its rows straight from the accumulators as bf16 pairs
    // (group 0 while group 1 multiplies the last stage), with no LDS tile
    // and no copy-out pass
    const bool direct = a.y == nullptr && a.residual == nullptr && a.vec_ok;
    pp_main<4, Lay, kDownPPStages<FP8, A8>>(ap, bp, A8 ? a.K / 128 : a.K / 64, lds, group, wm0, wn0, acc,
                                             [&](const f32x16 (&c)[4][2]) {
        const int r = lane & 31;
        float cs[2];
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int64_t col = n0 + wn0 + tn * 32 + r;
            cs[tn] = a.shared_scale * ((a.w_scale != nullptr && col < a.N) ? a.w_scale[col] : 1.0f);
        }
        if (direct) {
            const int ld2 = (int)a.ldo * 2;
            const int64_t mlim = a.M - m0 < BM ? a.M - m0 : BM;
            const auto rsrc = make_rsrc(static_cast<T*>(a.out) + m0 * a.ldo, (uint32_t)(mlim * ld2));
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const int64_t col = n0 + wn0 + tn * 32 + r;
                const int lb = pair_lane_offset(wm0, (int)col, ld2) | (col < a.N ? 0 : kOutOfRange);
#pragma unroll
                for (int tm = 0; tm < 4; ++tm) {
                    float v[16];
#pragma unroll
                    for (int q = 0; q < 16; ++q) v[q] = c[tm][tn][q] * cs[tn];
                    store_bf16_pairs(rsrc, lb + tm * 32 * ld2, ld2, v);
                }
            }
            return;
        }
#pragma unroll
        for (int tm = 0; tm < 4; ++tm)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int rl = wm0 + tm * 32 + acc_row(lane, i);
#pragma unroll
                for (int tn = 0; tn < 2; ++tn)
                    *reinterpret_cast<T*>(lds + rl * kORowBytes + (wn0 + tn * 32 + r) * 2) =
                        from_f32<T>(c[tm][tn][i] * cs[tn]);
            }
    }, sc);
    if (direct) return;

    const T* y = static_cast<const T*>(a.y);
    const T* res = static_cast<const T*>(a.residual);
    T* out = static_cast<T*>(a.out);
    constexpr int kChunksPerRow = BN / 8;
    for (int q = threadIdx.x; q < BM * kChunksPerRow; q += 512) {
        const int rl = q / kChunksPerRow, c = q % kChunksPerRow;
        const int64_t row = m0 + rl;
        const int64_t col = n0 + c * 8;
        if (row >= a.M || col >= a.N) continue;
        const bf16x8 sb = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lds + rl * kORowBytes + c * 16));
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)sb[e];
        if (a.vec_ok && col + 8 <= a.N) {
            if (y != nullptr) {
                float acc_r[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                for (int j = 0; j < a.top_k; ++j) {
                    const bf16x8 yv = __builtin_bit_cast(
                        bf16x8, *reinterpret_cast<const u32x4*>(y + (int64_t)s_yrow[rl][j] * a.ldy + col));
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc_r[e] += a.rw[j] * (float)yv[e];
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += a.routed_scale * acc_r[e];
            }
            if (res != nullptr) {
                const bf16x8 rv = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(res + row * a.ldr + col));
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] += (float)rv[e];
            }
            bf16x8 ov;
#pragma unroll
            for (int e = 0; e < 8; ++e) ov[e] = (bf16_t)v[e];
            *reinterpret_cast<u32x4*>(out + row * a.ldo + col) = __builtin_bit_cast(u32x4, ov);
        } else {
            for (int e = 0; e < 8 && col + e < a.N; ++e) {
                float x = v[e];
                if (y != nullptr) {
                    float sacc = 0.f;
                    for (int j = 0; j < a.top_k; ++j)
                        sacc += a.rw[j] * to_f32(y[(int64_t)s_yrow[rl][j] * a.ldy + col + e]);
                    x += a.routed_scale * sacc;
                }
                if (res != nullptr) x += to_f32(res[row * a.ldr + col + e]);
                out[row * a.ldo + col + e] = from_f32<T>(x);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <class F>
static int ensure_lds(F* fn, int bytes) {
    return set_kernel_lds(reinterpret_cast<const void*>(fn), bytes);
}

// Tile choice: 256x256 workgroup tiles (8 waves of 128x64) halve the L2->CU
// traffic per MFMA relative to 128x128 and are used whenever they still give
// at least two workgroups per CU; the down GEMM uses 256x224 when the hidden
// size is a multiple of 224 (896 = 4 x 224: one full wave of 256 tiles with
// no padded columns).  bf16/f32 operands take the direct buffer->LDS loads
// (PGR 4); e4m3 weights the register-staged loop that expands them.
constexpr int64_t kBigTileMinBlocks = 512;
// The ping-pong gate|up keeps its 256x256 tiles down to half a wave of
// workgroups: its two 4-wave groups hide the loads that an underfilled grid of
// the plain 256x256 loop cannot (bf16 layer, 2048 tokens: gate|up 43.6 ->
// 34.7 us at 128 tiles; the down keeps kBigTileMinBlocks, where a lower bound
// made 8192 tokens slower).
constexpr int64_t kPPGateUpMinBlocks = 128;

static int device_cus() { return current_device_cus(); }

template <class Kind, bool FP8, class Shape>
static int launch_gate_up_shape(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    dim3 grid((unsigned)((a.M + Shape::BM - 1) / Shape::BM), (unsigned)((packed_rows - a.n_base) / Shape::BN));
    constexpr int kEpi = Shape::BM * (Shape::BN / 2 * (int)sizeof(typename Kind::T) + 16);
    constexpr int kLds = kEpi > Shape::kLdsBytes ? kEpi : Shape::kLdsBytes;
    int st = ensure_lds(k_gate_up_swiglu<Kind, FP8, Shape>, kLds);
    if (st) return st;
    hipLaunchKernelGGL((k_gate_up_swiglu<Kind, FP8, Shape>), grid, dim3(Shape::NT), kLds, stream, a);
    return check_launch("shared_gate_up");
}

// 256x256 tiles, but when the last round of tiles would leave at least half
// of the CUs idle, the trailing column tiles run as a second launch of
// 256x128 tiles: twice the workgroups for the same work (at C2, 1664 tiles =
// 6 full rounds + 128 tiles becomes 1536 + 256 half-width tiles).
template <class Kind>
static int launch_gate_up_dma_balanced(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    const int64_t tiles_m = (a.M + 255) / 256;
    const int64_t cols = (packed_rows - a.n_base) / 256;
    const int64_t cus = device_cus();
    int64_t tail_cols = 0;
    // smallest number of trailing columns whose removal leaves whole rounds
    for (int64_t k = 1; k < cols; ++k)
        if ((tiles_m * (cols - k)) % cus == 0 && tiles_m * k * 2 <= cus) {
            tail_cols = k;
            break;
        }
    if (tail_cols == 0) return launch_gate_up_shape<Kind, false, ShapeBigDma>(a, packed_rows, stream);
    const int64_t split = a.n_base + (cols - tail_cols) * 256;
    int st = launch_gate_up_shape<Kind, false, ShapeBigDma>(a, split, stream);
    if (st) return st;
    GateUpArgs t = a;
    t.n_base = split;
    return launch_gate_up_shape<Kind, false, ShapeTallDma>(t, packed_rows, stream);
}

template <class Kind, bool FP8>
static int launch_gate_up_kind(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    const int64_t big_blocks = ((a.M + 255) / 256) * (packed_rows / 256);
    if (packed_rows % 256 == 0 && big_blocks >= kBigTileMinBlocks) {
        if constexpr (FP8)
            return launch_gate_up_shape<Kind, FP8, ShapeBigF8Dma>(a, packed_rows, stream);
        else
            return launch_gate_up_dma_balanced<Kind>(a, packed_rows, stream);
    }
    // fewer 128x128 tiles than CUs: 64x128 (bf16 at 512 tokens: the op 36.5 -> 27.6 us)
    if (packed_rows % 128 == 0 && ((a.M + 127) / 128) * (packed_rows / 128) < device_cus())
        return launch_gate_up_shape<Kind, FP8, SmallShape<FP8, 128>>(a, packed_rows, stream);
    return launch_gate_up_shape<Kind, FP8, ShapeMain>(a, packed_rows, stream);
}

// Expert columns of a dense-routed gate|up, [a.n_base, packed_rows), in
// 256x128 tiles with the routing code compiled in.
template <class Kind, bool FP8, class Shape>
static int launch_gate_up_routed_cols_shape(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    dim3 grid((unsigned)((a.M + Shape::BM - 1) / Shape::BM), (unsigned)((packed_rows - a.n_base) / Shape::BN));
    constexpr int kEpi = Shape::BM * (Shape::BN / 2 * (int)sizeof(typename Kind::T) + 16);
    constexpr int kLds = kEpi > Shape::kLdsBytes ? kEpi : Shape::kLdsBytes;
    auto kern = k_gate_up_swiglu<Kind, FP8, Shape, false, true>;
    int st = ensure_lds(kern, kLds);
    if (st) return st;
    hipLaunchKernelGGL(kern, grid, dim3(Shape::NT), kLds, stream, a);
    return check_launch("dense_routed_gate_up");
}

template <class Kind, bool FP8>
static int launch_gate_up_routed_cols(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    {
        // fewer 128x256 tiles than CUs: 64x128 (C1's 512 expert columns at 2048
        // tokens: 32 -> 128 workgroups, the op 300 -> 217 us)
        const int64_t cols = packed_rows - a.n_base;
        if (cols % 128 == 0 && ((a.M + 127) / 128) * (cols / 256) < device_cus())
            return launch_gate_up_routed_cols_shape<Kind, FP8, SmallShape<FP8, 128>>(a, packed_rows, stream);
    }
    if (!FP8 && (packed_rows - a.n_base) % 256 == 0)
        return launch_gate_up_routed_cols_shape<Kind, FP8, std::conditional_t<FP8, ShapeMain, ShapeTallDma>>(
            a, packed_rows, stream);
    return launch_gate_up_routed_cols_shape<Kind, FP8, std::conditional_t<FP8, ShapeMain, ShapeGroupNarrowDma>>(
        a, packed_rows, stream);
}

// Training forwards (a.gu set): the direct-load tiles with the raw gate|up
// store, 256x256 where the packed rows allow it, else 256x128 (2 W rows of
// 64-feature blocks always do); dense-routed expert columns with the routing
// epilogue.  Every M takes the tile kernels (the decode-shape kernels have
// no save).
template <class Kind, class Shape, bool ROUTED>
static int launch_gate_up_save_shape(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    dim3 grid((unsigned)((a.M + Shape::BM - 1) / Shape::BM), (unsigned)((packed_rows - a.n_base) / Shape::BN));
    constexpr int kEpi = Shape::BM * (Shape::BN / 2 * (int)sizeof(typename Kind::T) + 16);
    constexpr int kLds = kEpi > Shape::kLdsBytes ? kEpi : Shape::kLdsBytes;
    auto kern = k_gate_up_swiglu<Kind, false, Shape, false, ROUTED, true>;
    int st = ensure_lds(kern, kLds);
    if (st) return st;
    if (grid.x == 0 || grid.y == 0) return TRMOE_OK;
    hipLaunchKernelGGL(kern, grid, dim3(Shape::NT), kLds, stream, a);
    return check_launch("gate_up (saving pre-activations)");
}

template <class Kind, bool ROUTED>
static int launch_gate_up_save_kind(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if ((packed_rows - a.n_base) % 256 == 0) return launch_gate_up_save_shape<Kind, ShapeBigDma, ROUTED>(a, packed_rows, stream);
    return launch_gate_up_save_shape<Kind, ShapeGroupNarrowDma, ROUTED>(a, packed_rows, stream);
}

static int launch_gate_up_save(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (act != wdt || (act != TRMOE_BF16 && act != TRMOE_F32))
        return set_error(TRMOE_ERR_UNSUPPORTED, "gate_up: saving pre-activations needs bf16/f32 weights");
    if (packed_rows % 128 != 0) return set_error(TRMOE_ERR_INVALID, "gate_up: packed rows not a multiple of 128");
    const bool bf = act == TRMOE_BF16;
    if (a.ids != nullptr) {
        const int64_t shared_rows = 2 * a.shared_feats;
        if (shared_rows > 0) {
            GateUpArgs sh = a;
            sh.ids = nullptr;
            const int st = bf ? launch_gate_up_save_kind<KindBF16, false>(sh, shared_rows, stream)
                              : launch_gate_up_save_kind<KindF32, false>(sh, shared_rows, stream);
            if (st) return st;
        }
        GateUpArgs ex = a;
        ex.n_base = shared_rows;
        return bf ? launch_gate_up_save_kind<KindBF16, true>(ex, packed_rows, stream)
                  : launch_gate_up_save_kind<KindF32, true>(ex, packed_rows, stream);
    }
    return bf ? launch_gate_up_save_kind<KindBF16, false>(a, packed_rows, stream)
              : launch_gate_up_save_kind<KindF32, false>(a, packed_rows, stream);
}

// One wave per token: the sum of squares of its row (16-byte loads, an
// element tail for hidden % (16 / sizeof(T)) != 0), reduced across the wave.
template <class T>
__global__ __launch_bounds__(256) void k_rms_row_scale(const T* x, int64_t n, int hidden, int64_t ldx, float eps,
                                                       float* out) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + wave;
    if (row >= n) return;
    constexpr int kV = 16 / (int)sizeof(T);
    const T* xr = x + row * ldx;
    float s = 0.f;
    const int full = hidden / kV * kV;
    for (int k = lane * kV; k < full; k += 64 * kV) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(xr + k);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (sizeof(T) == 2) {
                const float lo = __builtin_bit_cast(float, v[j] << 16);
                const float hi = __builtin_bit_cast(float, v[j] & 0xffff0000u);
                s += lo * lo;
                s += hi * hi;
            } else {
                const float f = __builtin_bit_cast(float, (uint32_t)v[j]);
                s += f * f;
            }
        }
    }
    for (int k = full + lane; k < hidden; k += 64) {
        const float f = to_f32(xr[k]);
        s += f * f;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) out[row] = rsqrtf(s / (float)hidden + eps);
}

int launch_rms_row_scale(int act, const void* x, int64_t n, int64_t hidden, int64_t ldx, float eps, float* row_scale,
                         hipStream_t stream) {
    if (n <= 0) return TRMOE_OK;
    const dim3 grid((unsigned)((n + 3) / 4));
    if (act == TRMOE_BF16)
        hipLaunchKernelGGL(k_rms_row_scale<bf16_t>, grid, dim3(256), 0, stream, static_cast<const bf16_t*>(x), n,
                           (int)hidden, ldx, eps, row_scale);
    else if (act == TRMOE_F32)
        hipLaunchKernelGGL(k_rms_row_scale<float>, grid, dim3(256), 0, stream, static_cast<const float*>(x), n,
                           (int)hidden, ldx, eps, row_scale);
    else
        return set_error(TRMOE_ERR_UNSUPPORTED, "rms_row_scale: bf16 or f32 activations");
    return check_launch("rms_row_scale");
}

// bf16 prefill-sized gate|up (shared or dense-routed, every column tile in
// one launch) on the ping-pong tiles: 256x256 tiles over whole 64-element K
// stages, at least kPPGateUpMinBlocks tiles.
static bool pp_eligible(int act, int wdt, const GateUpArgs& a, int64_t packed_rows) {
    const int64_t cols = packed_rows - a.n_base;
    const bool types = act == TRMOE_BF16 && (wdt == TRMOE_BF16 || (wdt == TRMOE_FP8_E4M3 && a.gu == nullptr));
    return types && a.K > 0 && a.K % 64 == 0 && cols > 0 && cols % 256 == 0 &&
           ((a.M + 255) / 256) * (cols / 256) >= kPPGateUpMinBlocks;
}

template <bool ROUTED, int TMW, bool SAVE, bool FP8>
static int launch_gate_up_pp_shape(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    constexpr int BM = ShapePP<TMW>::BM;
    const dim3 grid((unsigned)((a.M + BM - 1) / BM), (unsigned)((packed_rows - a.n_base) / 256));
    using Lay = std::conditional_t<FP8, PPLayoutF8<TMW>, PPLayoutK<TMW>>;
    constexpr int kEpi = BM * (128 * 2 + 16);                // the SwiGLU tile, over the stages
    constexpr int kLds = 2 * Lay::kStage > kEpi ? 2 * Lay::kStage : kEpi;
    auto kern = k_gate_up_pp<ROUTED, TMW, SAVE, FP8>;
    const int st = ensure_lds(kern, kLds);
    if (st) return st;
    if (grid.x == 0 || grid.y == 0) return TRMOE_OK;
    hipLaunchKernelGGL(kern, grid, dim3(512), kLds, stream, a);
    return check_launch(ROUTED ? "dense_routed_gate_up" : "shared_gate_up");
}

// Persistent 256-row tiles over packed rows [a.n_base, packed_rows): one
// workgroup per CU (fewer when there are fewer tiles).
template <bool SAVE, bool FP8>
static int launch_gate_up_pps(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    const int64_t tiles_m = (a.M + 255) / 256;
    const int64_t n_tiles = tiles_m * ((packed_rows - a.n_base) / 256);
    const int64_t cus = device_cus();
    const int64_t grid = n_tiles < cus ? n_tiles : cus;
    using Lay = std::conditional_t<FP8, PPLayoutF8<4>, PPLayoutK<4>>;
    constexpr int kLds = 2 * Lay::kStage;
    auto kern = k_gate_up_pps<4, SAVE, FP8>;
    const int st = ensure_lds(kern, kLds);
    if (st) return st;
    if (grid <= 0) return TRMOE_OK;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(512), kLds, stream, a, tiles_m, n_tiles);
    return check_launch("shared_gate_up");
}

// W8A8 shared gate|up: every tile on the persistent stream (a last round
// that leaves CUs idle is not split off: there is no e4m3-activation tile
// kernel).  The caller checks K % 128 == 0 and whole 256-row column tiles.
int launch_gate_up_a8(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    const int64_t tiles_m = (a.M + 255) / 256;
    const int64_t n_tiles = tiles_m * ((packed_rows - a.n_base) / 256);
    const int64_t cus = device_cus();
    const int64_t grid = n_tiles < cus ? n_tiles : cus;
    constexpr int kLds = 2 * PPLayoutK8<4>::kStage;
    auto kern = a.hs != nullptr ? k_gate_up_pps<4, false, true, true, true> : k_gate_up_pps<4, false, true, true>;
    const int st = ensure_lds(kern, kLds);
    if (st) return st;
    if (grid <= 0) return TRMOE_OK;
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(512), kLds, stream, a, tiles_m, n_tiles);
    return check_launch("shared_gate_up_a8");
}

// 256-row tiles; when their last round would leave at least half of the CUs
// idle, the fewest trailing columns whose removal leaves whole rounds run as
// a second launch of 128-row tiles (C2: 64 x 24 tiles, then 128 x 2 half
// tiles: seven rounds become six and a round of half tiles).  Launches whose
// first columns hold no expert features leave the routing code out.
template <bool ROUTED, bool SAVE, bool FP8 = false>
static int launch_gate_up_pp(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    const int64_t tiles_m = (a.M + 255) / 256;
    const int64_t cols = (packed_rows - a.n_base) / 256;
    const int64_t cus = device_cus();
    int64_t tail = 0;
    if ((tiles_m * cols) % cus != 0)
        for (int64_t k = 1; k < cols; ++k)
            if ((tiles_m * (cols - k)) % cus == 0 && tiles_m * k * 2 <= cus) {
                tail = k;
                break;
            }
    const int64_t split = a.n_base + (cols - tail) * 256;
    const bool head_routed = ROUTED && a.ids != nullptr && split > 2 * a.shared_feats;
    int st = head_routed            ? launch_gate_up_pp_shape<ROUTED, 4, SAVE, FP8>(a, split, stream)
             : a.row_scale != nullptr ? launch_gate_up_pp_shape<false, 4, SAVE, FP8>(a, split, stream)
                                      : launch_gate_up_pps<SAVE, FP8>(a, split, stream);
    if (st || tail == 0) return st;
    GateUpArgs t = a;
    t.n_base = split;
    return launch_gate_up_pp_shape<ROUTED, 2, SAVE, FP8>(t, packed_rows, stream);
}

int launch_gate_up(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (a.gu != nullptr) {
        if (pp_eligible(act, wdt, a, packed_rows))
            return a.ids != nullptr ? launch_gate_up_pp<true, true>(a, packed_rows, stream)
                                    : launch_gate_up_pp<false, true>(a, packed_rows, stream);
        return launch_gate_up_save(act, wdt, a, packed_rows, stream);
    }
    if (a.M <= kSkinnyMaxTokens && packed_rows % 64 == 0)
        return launch_gate_up_skinny(act, wdt, a, packed_rows, stream);
    if (a.row_scale == nullptr && a.rms_eps > 0.0f)
        return set_error(TRMOE_ERR_INVALID, "gate_up: in-kernel RMSNorm scales need the decode kernels (n <= 128)");
    if (pp_eligible(act, wdt, a, packed_rows)) {
        if (wdt == TRMOE_FP8_E4M3)
            return a.ids != nullptr ? launch_gate_up_pp<true, false, true>(a, packed_rows, stream)
                                    : launch_gate_up_pp<false, false, true>(a, packed_rows, stream);
        return a.ids != nullptr ? launch_gate_up_pp<true, false>(a, packed_rows, stream)
                                : launch_gate_up_pp<false, false>(a, packed_rows, stream);
    }
    if (a.ids != nullptr) {
        // dense-routed: the shared columns as a plain gate|up launch, then the
        // expert columns with the routing epilogue
        const int64_t shared_rows = 2 * a.shared_feats;
        if (shared_rows > 0) {
            GateUpArgs sh = a;
            sh.ids = nullptr;
            const int st = launch_gate_up(act, wdt, sh, shared_rows, stream);
            if (st) return st;
        }
        GateUpArgs ex = a;
        ex.n_base = shared_rows;
        if (act == TRMOE_F32 && wdt == TRMOE_F32) return launch_gate_up_routed_cols<KindF32, false>(ex, packed_rows, stream);
        if (act == TRMOE_BF16 && wdt == TRMOE_BF16)
            return launch_gate_up_routed_cols<KindBF16, false>(ex, packed_rows, stream);
        if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3)
            return launch_gate_up_routed_cols<KindBF16, true>(ex, packed_rows, stream);
        return set_error(TRMOE_ERR_UNSUPPORTED, "dense_routed_gate_up: unsupported dtype pair");
    }
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return launch_gate_up_kind<KindF32, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return launch_gate_up_kind<KindBF16, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return launch_gate_up_kind<KindBF16, true>(a, packed_rows, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_gate_up: unsupported dtype pair");
}

template <class Kind, bool FP8, class Shape>
static int launch_down_shape(const DownArgs& a, hipStream_t stream) {
    dim3 grid((unsigned)((a.M + Shape::BM - 1) / Shape::BM), (unsigned)((a.N + Shape::BN - 1) / Shape::BN));
    constexpr int kEpi = sizeof(typename Kind::T) == 2 ? Shape::BM * (Shape::BN * 2 + 16) : 0;
    constexpr int kLds = kEpi > Shape::kLdsBytes ? kEpi : Shape::kLdsBytes;
    int st = ensure_lds(k_down_combine<Kind, FP8, Shape>, kLds);
    if (st) return st;
    hipLaunchKernelGGL((k_down_combine<Kind, FP8, Shape>), grid, dim3(Shape::NT), kLds, stream, a);
    return check_launch("shared_down_combine");
}

// bf16 down GEMMs with at least a full round of 256x256 tiles run on the
// ping-pong main loop.
template <bool FP8, bool A8 = false>
static int launch_down_pp(const DownArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)(((a.M + 255) / 256) * ((a.N + 255) / 256)));
    using Lay = std::conditional_t<A8, PPLayoutK8<4, true>, std::conditional_t<FP8, PPLayoutF8<4>, PPLayoutK<4>>>;
    constexpr int kEpi = 256 * (256 * 2 + 16);   // the bf16 output tile, over the stages
    constexpr int kBufs = kDownPPStages<FP8, A8> * Lay::kStage;
    constexpr int kLds = kEpi > kBufs ? kEpi : kBufs;
    const int st = ensure_lds(k_down_pp<FP8, A8>, kLds);
    if (st) return st;
    hipLaunchKernelGGL((k_down_pp<FP8, A8>), grid, dim3(512), kLds, stream, a);
    return check_launch(A8 ? "shared_down_combine_a8" : "shared_down_combine");
}

int launch_down_combine_a8(const DownArgs& a, hipStream_t stream) {
    if (a.M <= 0) return TRMOE_OK;
    return launch_down_pp<true, true>(a, stream);
}

// The packed down weights have round_up(N, 256) rows, so every tile choice
// below reads only packed rows.
template <class Kind, bool FP8>
static int launch_down_kind(const DownArgs& a, hipStream_t stream) {
    const int64_t mt = (a.M + 255) / 256;
    if constexpr (std::is_same_v<Kind, KindBF16>) {
        if (a.K > 0 && a.K % 64 == 0 && mt * ((a.N + 255) / 256) >= 256) return launch_down_pp<FP8>(a, stream);
    }
    const bool fits224 = a.N % ShapeDown224::BN == 0;
    if constexpr (FP8) {
        if (a.N % 256 == 0 && mt * (a.N / 256) >= 256) return launch_down_shape<Kind, FP8, ShapeBigF8Dma>(a, stream);
    }
    const bool big = (fits224 && mt * (a.N / ShapeDown224::BN) >= 256) || mt * ((a.N + 255) / 256) >= kBigTileMinBlocks;
    // fewer 128x128 tiles than CUs: 64x64 tiles (C1, 2048 x 896 f32: 112 -> 448
    // workgroups, 237 -> 124 us; bf16 at 512 / 2048 tokens: 40 -> 19, 41 -> 24 us)
    if (!big && ((a.M + 127) / 128) * ((a.N + 127) / 128) < device_cus())
        return launch_down_shape<Kind, FP8, SmallShape<FP8, 64>>(a, stream);
    if (!big) return launch_down_shape<Kind, FP8, ShapeMain>(a, stream);
    if constexpr (FP8) {
        if (fits224) return launch_down_shape<Kind, FP8, ShapeDown224>(a, stream);
        return launch_down_shape<Kind, FP8, ShapeBig>(a, stream);
    } else {
        if (fits224) return launch_down_shape<Kind, FP8, ShapeDown224Dma>(a, stream);
        return launch_down_shape<Kind, FP8, ShapeBigDma>(a, stream);
    }
}

int launch_down_combine(int act, int wdt, const DownArgs& a, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return launch_down_kind<KindF32, false>(a, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return launch_down_kind<KindBF16, false>(a, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return launch_down_kind<KindBF16, true>(a, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_down_combine: unsupported dtype pair");
}

// ---------------------------------------------------------------------------
// expert-grouped launches (two-pass routed experts)
// ---------------------------------------------------------------------------

template <class Kind, bool FP8, class Shape>
static int launch_gate_up_grouped_shape(const GateUpArgs& a, int64_t assignments, int64_t packed_rows,
                                        hipStream_t stream) {
    const int64_t tiles_m = (assignments + Shape::BM - 1) / Shape::BM + a.E;   // each segment adds <= 1 partial tile
    dim3 grid((unsigned)tiles_m, (unsigned)(packed_rows / Shape::BN));
    constexpr int kEpi = Shape::BM * (Shape::BN / 2 * (int)sizeof(typename Kind::T) + 16);
    constexpr int kLds = kEpi > Shape::kLdsBytes ? kEpi : Shape::kLdsBytes;
    int st = ensure_lds(k_gate_up_swiglu<Kind, FP8, Shape, true>, kLds);
    if (st) return st;
    hipLaunchKernelGGL((k_gate_up_swiglu<Kind, FP8, Shape, true>), grid, dim3(Shape::NT), kLds, stream, a);
    return check_launch("routed_experts (gate|up)");
}

// Persistent expert-grouped gate|up: one workgroup per CU (bf16 activations,
// K a multiple of 64, packed rows per expert a multiple of 256, gathered
// rows, no row scales).
template <bool FP8>
static int launch_gate_up_grouped_pps(const GateUpArgs& a, hipStream_t stream) {
    using Lay = std::conditional_t<FP8, PPLayoutF8<4, true>, PPLayoutK<4, true>>;
    constexpr int kLds = 2 * Lay::kStage;
    const int st = ensure_lds(k_gate_up_grouped_pps<FP8>, kLds);
    if (st) return st;
    hipLaunchKernelGGL(k_gate_up_grouped_pps<FP8>, dim3((unsigned)device_cus()), dim3(512), kLds, stream, a);
    return check_launch("routed_experts (gate|up)");
}

template <class Kind, bool FP8>
static int gate_up_grouped_kind(const GateUpArgs& a, int64_t assignments, int64_t packed_rows, hipStream_t stream) {
    if constexpr (std::is_same_v<Kind, KindBF16>) {
        if (a.K > 0 && a.K % 64 == 0 && packed_rows % 256 == 0 && a.gather != nullptr && a.row_scale == nullptr &&
            a.rms_eps == 0.0f && a.gu == nullptr && a.w_expert_stride == packed_rows * a.ldw)
            return launch_gate_up_grouped_pps<FP8>(a, stream);
    }
    const bool wide = packed_rows % 256 == 0;
    {
        // fewer tiles of the shapes below than CUs: 64x128 (C2 grouped, 4 x 64
        // experts: 132 -> 516 workgroups, routed experts 47.5 -> 44.6 us)
        const int64_t bn = wide ? 256 : 128;
        const int64_t bm = FP8 ? (wide ? 256 : 128) : 256;
        if (packed_rows % 128 == 0 && ((assignments + bm - 1) / bm + a.E) * (packed_rows / bn) < device_cus())
            return launch_gate_up_grouped_shape<Kind, FP8, SmallShape<FP8, 128>>(a, assignments, packed_rows, stream);
    }
    if constexpr (FP8) {
        if (wide) return launch_gate_up_grouped_shape<Kind, FP8, ShapeBigF8Dma>(a, assignments, packed_rows, stream);
        return launch_gate_up_grouped_shape<Kind, FP8, ShapeMain>(a, assignments, packed_rows, stream);
    } else {
        if (wide) return launch_gate_up_grouped_shape<Kind, FP8, ShapeBigDma>(a, assignments, packed_rows, stream);
        return launch_gate_up_grouped_shape<Kind, FP8, ShapeGroupNarrowDma>(a, assignments, packed_rows, stream);
    }
}

int launch_gate_up_grouped(int act, int wdt, const GateUpArgs& a, int64_t assignments, int64_t packed_rows,
                           hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return gate_up_grouped_kind<KindF32, false>(a, assignments, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16)
        return gate_up_grouped_kind<KindBF16, false>(a, assignments, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3)
        return gate_up_grouped_kind<KindBF16, true>(a, assignments, packed_rows, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "routed_experts: unsupported dtype pair");
}

template <class Kind, bool FP8, class Shape>
static int launch_down_grouped_shape(const DownArgs& a, int64_t assignments, hipStream_t stream) {
    const int64_t tiles_m = (assignments + Shape::BM - 1) / Shape::BM + a.E;
    dim3 grid((unsigned)tiles_m, (unsigned)((a.N + Shape::BN - 1) / Shape::BN));
    constexpr int kEpi = sizeof(typename Kind::T) == 2 ? Shape::BM * (Shape::BN * 2 + 16) : 0;
    constexpr int kLds = kEpi > Shape::kLdsBytes ? kEpi : Shape::kLdsBytes;
    int st = ensure_lds(k_down_combine<Kind, FP8, Shape, true>, kLds);
    if (st) return st;
    hipLaunchKernelGGL((k_down_combine<Kind, FP8, Shape, true>), grid, dim3(Shape::NT), kLds, stream, a);
    return check_launch("routed_experts (down)");
}

// Persistent expert-grouped down: one workgroup per CU (K a multiple of 64,
// bf16 activations, every shape; column and row tails are masked).  A y of
// at least half the 256 MB Infinity Cache does not stay cached until the
// shared down reads it, so its rows are streamed (C5, 268 MB: routed experts
// 333 -> 295 us; C2's grouped strategy, 58 MB: the layer 307 -> 311 us with
// the hint, so it keeps the default policy).  The hint on the h of either
// gate|up was no faster at C5, and slower for the grouped one.
template <bool FP8>
static int launch_down_grouped_pps(const DownArgs& a, int64_t assignments, hipStream_t stream) {
    using Lay = std::conditional_t<FP8, PPLayoutF8<4, true>, PPLayoutK<4, true>>;
    constexpr int kLds = 2 * Lay::kStage;
    const bool stream_y = assignments * a.N * 2 >= (int64_t{128} << 20);
    auto kern = stream_y ? k_down_grouped_pps<FP8, true> : k_down_grouped_pps<FP8, false>;
    const int st = ensure_lds(kern, kLds);
    if (st) return st;
    hipLaunchKernelGGL(kern, dim3((unsigned)device_cus()), dim3(512), kLds, stream, a);
    return check_launch("routed_experts (down)");
}

template <class Kind, bool FP8>
static int down_grouped_kind(const DownArgs& a, int64_t assignments, hipStream_t stream) {
    if constexpr (std::is_same_v<Kind, KindBF16>) {
        if (a.K > 0 && a.K % 64 == 0 && a.y == nullptr && a.residual == nullptr)
            return launch_down_grouped_pps<FP8>(a, assignments, stream);
    }
    const bool fits224 = a.N % ShapeDown224::BN == 0;
    if constexpr (FP8) {
        if (a.N % 256 == 0) return launch_down_grouped_shape<Kind, FP8, ShapeBigF8Dma>(a, assignments, stream);
        if (fits224) return launch_down_grouped_shape<Kind, FP8, ShapeDown224>(a, assignments, stream);
        return launch_down_grouped_shape<Kind, FP8, ShapeBig>(a, assignments, stream);
    } else {
        if (fits224) return launch_down_grouped_shape<Kind, FP8, ShapeDown224Dma>(a, assignments, stream);
        return launch_down_grouped_shape<Kind, FP8, ShapeBigDma>(a, assignments, stream);
    }
}

int launch_down_grouped(int act, int wdt, const DownArgs& a, int64_t assignments, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return down_grouped_kind<KindF32, false>(a, assignments, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return down_grouped_kind<KindBF16, false>(a, assignments, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return down_grouped_kind<KindBF16, true>(a, assignments, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "routed_experts: unsupported dtype pair");
}

// 64-row tiles halve the LDS-resident h for wide fp32 experts.
using ShapeRoutedSmall = TileShape<64, 128, 2, 2>;

template <class Shape>
static int routed_lds_bytes_for(int act, int64_t f_pad) {
    const int64_t per_row = (act == TRMOE_F32) ? 4 * f_pad : 2 * f_pad;
    return Shape::kLdsBytes + (int)(Shape::BM * per_row);
}

constexpr int kMaxLdsBytes = 160 * 1024;

int routed_lds_bytes(int act, int64_t f_pad) {
    const int big = routed_lds_bytes_for<ShapeMain>(act, f_pad);
    return big <= kMaxLdsBytes ? big : routed_lds_bytes_for<ShapeRoutedSmall>(act, f_pad);
}

template <class Kind, bool FP8, class Shape>
static int launch_routed_shape(int act, const RoutedArgs& a, int64_t assignments, hipStream_t stream) {
    const int lds = routed_lds_bytes_for<Shape>(act, a.F_pad);
    // tiles of all segments <= ceil(assignments / BM) + one partial tile per expert
    const int64_t max_tiles = (assignments + Shape::BM - 1) / Shape::BM + a.E;
    int st = ensure_lds(k_routed_experts<Kind, FP8, Shape>, lds);
    if (st) return st;
    hipLaunchKernelGGL((k_routed_experts<Kind, FP8, Shape>), dim3((unsigned)max_tiles), dim3(Shape::NT), lds,
                       stream, a);
    return check_launch("routed_experts");
}

template <class Kind, bool FP8>
static int launch_routed_kind(int act, const RoutedArgs& a, int64_t assignments, hipStream_t stream) {
    if (routed_lds_bytes_for<ShapeMain>(act, a.F_pad) <= kMaxLdsBytes)
        return launch_routed_shape<Kind, FP8, ShapeMain>(act, a, assignments, stream);
    return launch_routed_shape<Kind, FP8, ShapeRoutedSmall>(act, a, assignments, stream);
}

int launch_routed(int act, int wdt, const RoutedArgs& a, int64_t assignments, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return launch_routed_kind<KindF32, false>(act, a, assignments, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return launch_routed_kind<KindBF16, false>(act, a, assignments, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3)
        return launch_routed_kind<KindBF16, true>(act, a, assignments, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "routed_experts: unsupported dtype pair");
}

int launch_combine(int act, const CombineArgs& a, hipStream_t stream) {
    const int64_t total = a.M * a.N;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    if (act == TRMOE_F32) {
        hipLaunchKernelGGL(k_combine<float>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(k_combine<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    }
    return check_launch("combine");
}

}  // namespace trmoe
