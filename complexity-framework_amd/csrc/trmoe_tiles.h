// Tile operand providers, tile shapes and expert-grouped tile helpers shared
// by the forward GEMMs (trmoe_gemm.hip) and the backward (trmoe_backward.hip).
#pragma once

#include "trmoe_common.h"
#include "trmoe_gemm.h"

#include <type_traits>

namespace trmoe {

// ---------------------------------------------------------------------------
// B operand selection: same kind as A, or e4m3 expanded to bf16
// ---------------------------------------------------------------------------
template <class Kind, bool FP8, int ROWS, int NT>
struct BProvSel {
    using type = BufRows<ROWS, NT>;
};
template <class Kind, int ROWS, int NT>
struct BProvSel<Kind, true, ROWS, NT> {
    using type = BufRowsFP8<ROWS, NT>;
};

// Packed weight rows [row0, row0 + ROWS) of a [rows, ld] packed tensor
// (every such row exists: packing pads rows to the tile multiple).
template <class Kind, bool FP8, int ROWS, int NT>
__device__ __forceinline__ void init_bprov(typename BProvSel<Kind, FP8, ROWS, NT>::type& bp, const void* base,
                                           int64_t ld, int64_t row0, int K) {
    const int64_t elem = FP8 ? 1 : (int64_t)sizeof(typename Kind::T);
    init_dense_rows(bp, base, row0, row0 + ROWS, ld * elem, (int)(K * elem));
}

// Operand providers of a tile shape: direct buffer->LDS loads for PGR 4,
// register-staged loads otherwise (and always for e4m3 weights, which are
// expanded to bf16 on the way into LDS).
template <class Shape, int ROWS>
using DmaProv = DmaRows<ROWS, Shape::NT>;
template <class Shape>
struct AProvOf {
    using type = std::conditional_t<(Shape::PGR >= 4), DmaProv<Shape, Shape::BM>, BufRows<Shape::BM, Shape::NT>>;
};
template <class Kind, bool FP8, class Shape>
struct BProvOf {
    static_assert(!(FP8 && Shape::PGR == 4), "e4m3 weights: register path or PGR 6");
    static_assert(!(!FP8 && Shape::PGR == 6), "PGR 6 is the e4m3 weight layout");
    // PGR 6: e4m3 rows of 64 bytes per K stage, the 64-byte-row DMA layout
    using type = std::conditional_t<
        Shape::PGR == 6, DmaRows64<Shape::BN, Shape::NT>,
        std::conditional_t<(Shape::PGR >= 4), DmaProv<Shape, Shape::BN>,
                           typename BProvSel<Kind, FP8, Shape::BN, Shape::NT>::type>>;
};
template <class Shape>
__device__ __forceinline__ void init_a(typename AProvOf<Shape>::type& ap, const void* base, int64_t row0,
                                       int64_t rows_total, int64_t ld_bytes, int kbytes) {
    if constexpr (Shape::PGR >= 4)
        ap.init(base, row0, rows_total, ld_bytes, kbytes);
    else
        init_dense_rows(ap, base, row0, rows_total, ld_bytes, kbytes);
}
template <class Kind, bool FP8, class Shape>
__device__ __forceinline__ void init_b(typename BProvOf<Kind, FP8, Shape>::type& bp, const void* base, int64_t ld,
                                       int64_t row0, int K) {
    if constexpr (Shape::PGR >= 4) {
        const int64_t elem = FP8 ? 1 : (int64_t)sizeof(typename Kind::T);
        bp.init(base, row0, row0 + Shape::BN, ld * elem, (int)(K * elem));
    } else {
        init_bprov<Kind, FP8, Shape::BN, Shape::NT>(bp, base, ld, row0, K);
    }
}

using ShapeMain = TileShape<128, 128, 2, 2>;
using ShapeBig = TileShape<256, 256, 2, 4>;        // 8 waves of 128x64, 2 waves per SIMD
using ShapeDown224 = TileShape<256, 224, 4, 1>;
using ShapeBigDma = TileShape<256, 256, 2, 4, 4>;    // 8 waves, direct buffer->LDS operand loads
using ShapeDown224Dma = TileShape<256, 224, 4, 1, 4>;
using ShapeBigF8Dma = TileShape<256, 256, 2, 4, 6>;  // e4m3 weights loaded straight into LDS
using ShapeGroupNarrowDma = TileShape<256, 128, 4, 2, 4>;   // 256x128 direct-load tiles
using ShapeTallDma = TileShape<128, 256, 1, 4, 4>;          // 128x256: 4 waves of 128x64
// Launches whose larger tiles would leave CUs idle: 64 x BN tiles of 4 waves,
// 32x32 each for the down (BN 64), 32x64 for gate|up columns (BN 128: the
// SwiGLU epilogue needs 64 packed columns, 32 gate + 32 up, per wave);
// direct loads, or the register path that expands e4m3 weights.
template <bool FP8, int BN>
using SmallShape = std::conditional_t<FP8, TileShape<64, BN, 2, 2>, TileShape<64, BN, 2, 2, 4>>;

// ---------------------------------------------------------------------------
// expert-grouped tiles
// ---------------------------------------------------------------------------
// Tile `tile` of the partition (row tiles of BM rows, expert by expert) ->
// (expert, first row, end row); expert -1 past the last tile.  Segments
// shorter than a tile cost one partial tile, so Zipf-skewed experts only pay
// for their own rows.
template <int BM>
__device__ __forceinline__ void grouped_tile(const int32_t* offsets, int E, int tile, int (&s_tile)[3]) {
    if (threadIdx.x == 0) {
        int acc_tiles = 0, e_sel = -1, r0 = 0, r1 = 0;
        for (int e = 0; e < E; ++e) {
            const int b = offsets[e], c = offsets[e + 1] - b;
            const int nt = (c + BM - 1) / BM;
            if (tile < acc_tiles + nt) {
                e_sel = e;
                r0 = b + (tile - acc_tiles) * BM;
                r1 = r0 + BM < b + c ? r0 + BM : b + c;
                break;
            }
            acc_tiles += nt;
        }
        s_tile[0] = e_sel;
        s_tile[1] = r0;
        s_tile[2] = r1;
    }
    __syncthreads();
}

// Gathered A rows for the direct-load providers: row r of the tile is
// a[gather[row0 + r] % mod] (rows at or past nrows load zero).
template <class Prov>
__device__ __forceinline__ void init_gather_rows(Prov& p, const void* base, const int64_t* gather, int64_t mod,
                                                 int64_t row0, int64_t nrows, int64_t ld_bytes, int kbytes) {
    p.rsrc = make_rsrc(base, (uint32_t)(mod * ld_bytes));
    p.kbytes = kbytes;
    if constexpr (requires_wave_field<Prov>::value) {
        p.wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int lane = threadIdx.x & 63;
        constexpr int kRowsPerInstr = Prov::kRowsPerInstr;
#pragma unroll
        for (int j = 0; j < Prov::kInstr; ++j) {
            const int r = (p.wave * Prov::kInstr + j) * kRowsPerInstr + lane / (64 / kRowsPerInstr);
            p.koff[j] = Prov::chunk_of(lane, r) * 16;
            if (r < nrows) {
                const int64_t t = (int64_t)((uint64_t)gather[row0 + r] % (uint64_t)mod);
                p.off[j] = (int)(t * ld_bytes) + p.koff[j];
            } else {
                p.off[j] = kOutOfRange;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < Prov::kChunks; ++j) {
            const int r = (threadIdx.x >> 3) + (Prov::kThreadsPerBlock / 8) * j;
            if (r < nrows) {
                const int64_t t = (int64_t)((uint64_t)gather[row0 + r] % (uint64_t)mod);
                p.row_off[j] = (int)(t * ld_bytes);
            } else {
                p.row_off[j] = kOutOfRange;
            }
        }
    }
}

}  // namespace trmoe
