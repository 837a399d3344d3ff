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
// B operand selection: same kind as A, or e4m3 expanded to bf16
// ---------------------------------------------------------------------------
template <class Kind, bool FP8, int ROWS>
struct BProvSel {
    using type = BufRows<ROWS>;
};
template <class Kind, int ROWS>
struct BProvSel<Kind, true, ROWS> {
    using type = BufRowsFP8<ROWS>;
};

// Packed weight rows [row0, row0 + ROWS) of a [rows, ld] packed tensor
// (every such row exists: packing pads rows to the tile multiple).
template <class Kind, bool FP8, int ROWS>
__device__ __forceinline__ void init_bprov(typename BProvSel<Kind, FP8, ROWS>::type& bp, const void* base,
                                           int64_t ld, int64_t row0, int K) {
    const int64_t elem = FP8 ? 1 : (int64_t)sizeof(typename Kind::T);
    init_dense_rows(bp, base, row0, row0 + ROWS, ld * elem, (int)(K * elem));
}

using ShapeMain = TileShape<128, 128, 2>;
using ShapeBig = TileShape<256, 256, 2>;
using ShapeDown224 = TileShape<256, 224, 4>;

// ---------------------------------------------------------------------------
// K2: shared gate|up + SwiGLU
// ---------------------------------------------------------------------------
template <class Kind, bool FP8, class Shape>
__global__ __launch_bounds__(kThreads) void k_gate_up_swiglu(GateUpArgs a) {
    using T = typename Kind::T;
    extern __shared__ __align__(16) char lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = (int64_t)blockIdx.y * Shape::BN;

    BufRows<Shape::BM> ap;
    init_dense_rows(ap, a.x, m0, a.M, a.ldx * (int64_t)sizeof(T), a.K * (int)sizeof(T));
    typename BProvSel<Kind, FP8, Shape::BN>::type bp;
    init_bprov<Kind, FP8, Shape::BN>(bp, a.w, a.ldw, n0, a.K);

    // Routes of this tile's rows, gathered once while the first stages load
    // (tiles holding expert features only); read back in the epilogue after
    // the main loop's barriers.
    __shared__ int s_route[Shape::BM][kMaxTopK];
    const bool tile_routed = a.ids != nullptr && ((n0 + Shape::BN) >> 1) > a.shared_feats;
    if (tile_routed && threadIdx.x < Shape::BM) {
        const int64_t row = m0 + threadIdx.x;
        int64_t id = row < a.M ? a.ids[row] : 0;
        id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
        for (int j = 0; j < kMaxTopK; ++j)
            s_route[threadIdx.x][j] = (j < a.top_k && row < a.M) ? (int)a.table[(int64_t)j * a.vocab + id] : -1;
    }

    f32x16 acc[Shape::TM][Shape::TN];
    zero_acc<Kind>(acc);
    tile_loop<Kind, Shape>(ap, bp, a.K, lds, wm0, wn0, acc);

    const int r = lane & 31;
#pragma unroll
    for (int p = 0; p < Shape::TN / 2; ++p) {
        const int64_t pbase = n0 + wn0 + 64 * p;     // packed row of the gate tile
        const int64_t fblock = pbase >> 1;            // first feature of this 32-feature block
        const int64_t feat = fblock + r;
        const float sg = a.w_scale ? a.w_scale[pbase + r] : 1.0f;
        const float su = a.w_scale ? a.w_scale[pbase + 32 + r] : 1.0f;
        // expert blocks are multiples of 64 features, so a 32-feature block
        // is wholly shared or wholly one expert's
        const bool routed = a.ids != nullptr && fblock >= a.shared_feats;
        const int64_t expert = routed ? (fblock - a.shared_feats) / a.expert_feats : -1;
        const float mult = routed ? 1.0f : a.shared_mult;
#pragma unroll
        for (int tm = 0; tm < Shape::TM; ++tm) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int64_t row = m0 + wm0 + tm * 32 + acc_row(lane, i);
                if (row < a.M) {
                    const float g = acc[tm][2 * p][i] * sg;
                    const float u = acc[tm][2 * p + 1][i] * su;
                    float hv = silu_f(g) * u * mult;
                    if (routed) {
                        const int* rr = s_route[wm0 + tm * 32 + acc_row(lane, i)];
                        float tw = 0.f;
#pragma unroll
                        for (int j = 0; j < kMaxTopK; ++j) tw += (rr[j] == expert) ? a.rw[j] : 0.f;
                        hv *= tw;
                    }
                    static_cast<T*>(a.h)[row * a.ldh + feat] = from_f32<T>(hv);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// K4: shared down + weighted un-permute + combine
// ---------------------------------------------------------------------------
template <class Kind, bool FP8, class Shape>
__global__ __launch_bounds__(kThreads) void k_down_combine(DownArgs a) {
    using T = typename Kind::T;
    extern __shared__ __align__(16) char lds[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = (int64_t)blockIdx.y * Shape::BN;

    BufRows<Shape::BM> ap;
    init_dense_rows(ap, a.h, m0, a.M, a.ldh * (int64_t)sizeof(T), a.K * (int)sizeof(T));
    typename BProvSel<Kind, FP8, Shape::BN>::type bp;
    init_bprov<Kind, FP8, Shape::BN>(bp, a.w, a.ldw, n0, a.K);

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
#pragma unroll
    for (int tm = 0; tm < Shape::TM; ++tm) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int64_t row = m0 + wm0 + tm * 32 + acc_row(lane, i);
            if (row >= a.M) continue;
            int64_t yrow[kMaxTopK];
            if (y != nullptr) {
                const int* yr = s_yrow[wm0 + tm * 32 + acc_row(lane, i)];
                for (int j = 0; j < a.top_k; ++j) yrow[j] = (int64_t)yr[j] * a.ldy;
            }
#pragma unroll
            for (int tn = 0; tn < Shape::TN; ++tn) {
                const int64_t col = n0 + wn0 + tn * 32 + r;
                if (col >= a.N) continue;
                float v = acc[tm][tn][i] * cscale[tn];
                if (y != nullptr) {
                    float s = 0.f;
                    for (int j = 0; j < a.top_k; ++j) s += a.rw[j] * to_f32(y[yrow[j] + col]);
                    v += a.routed_scale * s;
                }
                if (res != nullptr) v += to_f32(res[row * a.ldr + col]);
                out[row * a.ldo + col] = from_f32<T>(v);
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
__global__ __launch_bounds__(kThreads) void k_routed_experts(RoutedArgs a) {
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
        BufRows<Shape::BM> ap;
        ap.rsrc = make_rsrc(a.x, (uint32_t)(a.n_tokens * a.ldx * (int64_t)sizeof(T)));
        ap.kbytes = a.K * (int)sizeof(T);
#pragma unroll
        for (int j = 0; j < BufRows<Shape::BM>::kChunks; ++j) {
            const int row = (threadIdx.x >> 3) + 32 * j;
            if (row < rows) {
                const int64_t t = (int64_t)((uint64_t)a.sorted[row0 + row] % (uint64_t)a.n_tokens);
                ap.row_off[j] = (int)(t * a.ldx * (int64_t)sizeof(T));
            } else {
                ap.row_off[j] = kOutOfRange;
            }
        }
        typename BProvSel<Kind, FP8, Shape::BN>::type bp;
        init_bprov<Kind, FP8, Shape::BN>(bp, wgu, a.wgu_ld, (int64_t)fc * 128, a.K);
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
        typename BProvSel<Kind, FP8, Shape::BN>::type bp;
        init_bprov<Kind, FP8, Shape::BN>(bp, wd, a.wd_ld, (int64_t)oc * Shape::BN, a.W);
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

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <class F>
static int ensure_lds(F* fn, int bytes) {
    if (bytes <= 65536) return TRMOE_OK;
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess) return set_error(TRMOE_ERR_HIP, hipGetErrorString(err));
    return TRMOE_OK;
}

// Tile choice: 256x256 workgroup tiles (128x128 per wave) halve the L2->CU
// traffic per MFMA relative to 128x128 and are used whenever they still give
// at least two workgroups per CU; the down GEMM uses 256x224 when the hidden
// size is a multiple of 224 (896 = 4 x 224: one full wave of 256 tiles with
// no padded columns).
constexpr int64_t kBigTileMinBlocks = 512;

// TRMOE_GEMM_TILE=small|big forces one tile family (tuning sweeps); unset = auto.
static int tile_override() {
    static int v = [] {
        const char* e = getenv("TRMOE_GEMM_TILE");
        if (e == nullptr) return 0;
        if (strcmp(e, "small") == 0) return 1;
        if (strcmp(e, "big") == 0) return 2;
        return 0;
    }();
    return v;
}

template <class Kind, bool FP8, class Shape>
static int launch_gate_up_shape(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    dim3 grid((unsigned)((a.M + Shape::BM - 1) / Shape::BM), (unsigned)(packed_rows / Shape::BN));
    int st = ensure_lds(k_gate_up_swiglu<Kind, FP8, Shape>, Shape::kLdsBytes);
    if (st) return st;
    hipLaunchKernelGGL((k_gate_up_swiglu<Kind, FP8, Shape>), grid, dim3(kThreads), Shape::kLdsBytes, stream, a);
    return check_launch("shared_gate_up");
}

template <class Kind, bool FP8>
static int launch_gate_up_kind(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    const int64_t big_blocks = ((a.M + ShapeBig::BM - 1) / ShapeBig::BM) * (packed_rows / ShapeBig::BN);
    const int ov = tile_override();
    if (packed_rows % ShapeBig::BN == 0 && (ov == 2 || (ov == 0 && big_blocks >= kBigTileMinBlocks)))
        return launch_gate_up_shape<Kind, FP8, ShapeBig>(a, packed_rows, stream);
    return launch_gate_up_shape<Kind, FP8, ShapeMain>(a, packed_rows, stream);
}

int launch_gate_up(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return launch_gate_up_kind<KindF32, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return launch_gate_up_kind<KindBF16, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return launch_gate_up_kind<KindBF16, true>(a, packed_rows, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_gate_up: unsupported dtype pair");
}

template <class Kind, bool FP8, class Shape>
static int launch_down_shape(const DownArgs& a, hipStream_t stream) {
    dim3 grid((unsigned)((a.M + Shape::BM - 1) / Shape::BM), (unsigned)((a.N + Shape::BN - 1) / Shape::BN));
    int st = ensure_lds(k_down_combine<Kind, FP8, Shape>, Shape::kLdsBytes);
    if (st) return st;
    hipLaunchKernelGGL((k_down_combine<Kind, FP8, Shape>), grid, dim3(kThreads), Shape::kLdsBytes, stream, a);
    return check_launch("shared_down_combine");
}

// The packed down weights have round_up(N, 256) rows, so every tile choice
// below reads only packed rows.
template <class Kind, bool FP8>
static int launch_down_kind(const DownArgs& a, hipStream_t stream) {
    const int64_t mt = (a.M + 255) / 256;
    const int ov = tile_override();
    if (ov == 1) return launch_down_shape<Kind, FP8, ShapeMain>(a, stream);
    if (a.N % ShapeDown224::BN == 0 && (ov == 2 || mt * (a.N / ShapeDown224::BN) >= 256))
        return launch_down_shape<Kind, FP8, ShapeDown224>(a, stream);
    if (ov == 2 || mt * ((a.N + 255) / 256) >= kBigTileMinBlocks) return launch_down_shape<Kind, FP8, ShapeBig>(a, stream);
    return launch_down_shape<Kind, FP8, ShapeMain>(a, stream);
}

int launch_down_combine(int act, int wdt, const DownArgs& a, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return launch_down_kind<KindF32, false>(a, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return launch_down_kind<KindBF16, false>(a, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return launch_down_kind<KindBF16, true>(a, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_down_combine: unsupported dtype pair");
}

// 64-row tiles halve the LDS-resident h for wide fp32 experts.
using ShapeRoutedSmall = TileShape<64, 128, 2>;

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
    hipLaunchKernelGGL((k_routed_experts<Kind, FP8, Shape>), dim3((unsigned)max_tiles), dim3(kThreads), lds,
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
