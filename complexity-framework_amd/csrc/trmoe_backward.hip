// Backward of the TR-MoE layer (bf16 / f32 weights).
//
//   k_swiglu_bwd    per (256-row tile, 128 features): g|u = x Wgu^T
//                   (recomputed, not saved by the forward), dh = dout W_down,
//                   then dg, du and hm = m*silu(g)*u in one epilogue.  The
//                   dense and grouped forms follow the forward's strategies:
//                   grouped rows are partition rows read through `gather`,
//                   the way the reference's HashCGGRGroupedGEMM reads tokens
//                   (triton_token_routed.py:1669-1745).
//   k_wgrad         weight gradients as token-reduction GEMMs over expert
//                   segments without padding, split over tokens
//                   (cggr_grad_w / hash_cggr_grad_w,
//                   triton_token_routed.py:751-1028); operands are stored
//                   with the reduction index as rows, so both are transposed
//                   in registers on their way into the usual LDS layout.
//   k_wgrad_reduce  sums the split partials in split order (deterministic).
//
// The data gradient dx = [dg|du] Wgu (plus, for routed rows, the sum of a
// token's partition rows through `inverse`) runs on the forward's down/combine
// kernels with transposed packed weights (trmoe_abi.hip).
#include "trmoe_common.h"
#include "trmoe_internal.h"
#include "trmoe_gemm.h"
#include "trmoe_tiles.h"
#include "trmoe_pp.h"
#include "trmoe_map.h"

#include <stdlib.h>

#include <type_traits>

namespace trmoe {

// ---------------------------------------------------------------------------
// transposing operand provider
// ---------------------------------------------------------------------------
// Operand held as a row-major matrix whose ROWS are the reduction index:
// element (k, m) at row k, column m.  Each thread loads KB rows (KB = K
// values per 16-byte LDS chunk: 8 bf16, 4 f32) of MB = kChunks consecutive
// columns, and writes MB chunks, each the KB K values of one column, into
// the [column][K] swizzled layout the MFMA stage reads.  Rows are
// [t_base, t_end) of the matrix (direct), or the byte offsets of a table in
// LDS (gathered rows, kOutOfRange past the segment).
template <class Kind, int ROWS, int NT, bool GATHER>
struct BufRowsT {
    using T = typename Kind::T;
    static constexpr int KB = Kind::kPerChunk;
    static constexpr int kChunks = ROWS * 8 / NT;
    static constexpr int MB = kChunks;
    static constexpr int kGroups = ROWS / MB;
    static constexpr int kThreadsPerBlock = NT;
    static constexpr int kRowLoadBytes = MB * (int)sizeof(T);
    static_assert(kGroups * 8 == NT, "one (column group, K chunk) pair per thread");
    static_assert(kRowLoadBytes == 8 || kRowLoadBytes == 16 || kRowLoadBytes == 32, "row loads of 8-32 bytes");
    static_assert(kRowLoadBytes != 8 || KB == 8, "8-byte row loads are bf16");
    using Reg = u32x4;
    __amdgpu_buffer_rsrc_t rsrc;
    int col_off;        // byte offset of the thread's first column, kOutOfRange past the last
    int kc;             // K chunk of the stage this thread fills
    int ld;             // bytes per row (the host keeps the matrix below 2^31 bytes)
    int base;           // byte offset of the segment's first row (direct rows)
    int len;            // rows in the segment
    const int* table;

    __device__ __forceinline__ void init(const void* base_ptr, int64_t rows_total, int64_t ld_bytes, int64_t col0,
                                         int64_t ncols) {
        rsrc = make_rsrc(base_ptr, (uint32_t)(rows_total * ld_bytes));
        const int mg = threadIdx.x % kGroups;
        kc = threadIdx.x / kGroups;
        const int64_t c = col0 + (int64_t)mg * MB;
        col_off = c < ncols ? (int)(c * (int64_t)sizeof(T)) : kOutOfRange;
        ld = (int)ld_bytes;
        base = 0;
        len = 0;
        table = nullptr;
    }
    __device__ __forceinline__ void segment(int64_t t0, int n, const int* tab) {
        base = (int)(t0 * (int64_t)ld);
        len = n;
        table = tab;
    }
    __device__ __forceinline__ int offset(int lk) const {
        int o;
        if constexpr (GATHER)
            o = table[lk];
        else
            o = lk < len ? base + lk * ld : kOutOfRange;
        return (o < 0 || col_off < 0) ? kOutOfRange : o + col_off;
    }
    __device__ __forceinline__ void prefetch(int kt, Reg (&reg)[kChunks]) const {
        const int lk0 = kt * Kind::kStageElems + kc * KB;
        if constexpr (kRowLoadBytes == 8) {
#pragma unroll
            for (int k = 0; k < KB; k += 2) {
                const u32x2 lo = buffer_load8(rsrc, offset(lk0 + k));
                const u32x2 hi = buffer_load8(rsrc, offset(lk0 + k + 1));
                reg[k >> 1] = u32x4{lo[0], lo[1], hi[0], hi[1]};
            }
        } else if constexpr (kRowLoadBytes == 16) {
            static_assert(KB == kChunks, "one register per row");
#pragma unroll
            for (int k = 0; k < KB; ++k) reg[k] = buffer_load16(rsrc, offset(lk0 + k));
        } else {
            static_assert(2 * KB == kChunks, "two registers per row");
#pragma unroll
            for (int k = 0; k < KB; ++k) {
                const int o = offset(lk0 + k);
                reg[2 * k] = buffer_load16(rsrc, o);
                reg[2 * k + 1] = buffer_load16(rsrc, o < 0 ? kOutOfRange : o + 16);
            }
        }
    }
    // the dword of loaded row k that holds column j (bf16: two columns per dword)
    // (if constexpr: the other layout's subscripts would leave the vector)
    __device__ __forceinline__ uint32_t row_dword(const Reg (&reg)[kChunks], int k, int j) const {
        if constexpr (kRowLoadBytes == 8)
            return reg[k >> 1][(k & 1) * 2 + (j >> 1)];
        else
            return reg[k][j >> 1];
    }
    // element (row k, column j) of an f32 block
    __device__ __forceinline__ uint32_t elem(const Reg (&reg)[kChunks], int k, int j) const {
        if constexpr (kRowLoadBytes == 16)
            return reg[k][j];
        else
            return reg[2 * k + (j >> 2)][j & 3];
    }
    __device__ __forceinline__ void commit_one(char* stage, const Reg (&reg)[kChunks], int j) const {
        u32x4 v;
        if constexpr (sizeof(T) == 2) {
            // dword d = (element (2d, j), element (2d+1, j)): one byte permute
            // of the two rows' dwords holding column j
            const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
            for (int d = 0; d < 4; ++d)
                v[d] = __builtin_amdgcn_perm(row_dword(reg, 2 * d + 1, j), row_dword(reg, 2 * d, j), sel);
        } else {
#pragma unroll
            for (int d = 0; d < 4; ++d) v[d] = elem(reg, d, j);
        }
        const int mg = threadIdx.x % kGroups;
        *reinterpret_cast<u32x4*>(stage + lds_byte(mg * MB + j, kc)) = v;
    }
    __device__ __forceinline__ void commit(char* stage, const Reg (&reg)[kChunks]) const {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) commit_one(stage, reg, j);
    }
};

// bf16 operand with K as rows, loaded straight into LDS: a K stage is 64
// rows of COLS = 256 columns (512 bytes), 16-byte chunk c of row k stored at
// chunk c ^ ((k & 3) << 2), so that the transposing fragment reads below hit
// 64 distinct banks.  One wave instruction fills two rows.
template <int NT, bool GATHER>
struct DmaRowsT {
    static constexpr int kRowB = 512;
    static constexpr int kInstr = 64 * kRowB / 1024 / (NT / 64);   // per wave per stage
    static_assert(kInstr >= 1 && kInstr % 2 == 0, "whole row pairs per wave");
    __amdgpu_buffer_rsrc_t rsrc;
    int coloff[2];   // lane's source column bytes for rows with (row & 2) == 0 / 2, kOutOfRange past M
    int h;           // row of the pair this lane fills
    int wave;
    int base, len, ld;
    const int* table;

    __device__ __forceinline__ void init(const void* base_ptr, int64_t rows_total, int64_t ld_bytes, int64_t col0,
                                         int64_t ncols) {
        rsrc = make_rsrc(base_ptr, (uint32_t)(rows_total * ld_bytes));
        const int lane = threadIdx.x & 63;
        wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        h = lane >> 5;
        const int pc = lane & 31;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int c = pc ^ ((2 * p + h) << 2);
            const int64_t col = col0 + 8 * c;
            coloff[p] = col < ncols ? (int)(col * 2) : kOutOfRange;
        }
        ld = (int)ld_bytes;
        base = 0;
        len = 0;
        table = nullptr;
    }
    __device__ __forceinline__ void segment(int64_t t0, int n, const int* tab) {
        base = (int)(t0 * (int64_t)ld);
        len = n;
        table = tab;
    }
    __device__ __forceinline__ void issue(int kt, char* stage) const {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
            const int q = wave * kInstr + j;          // row pair of the stage
            const int lk = kt * 64 + 2 * q + h;
            int ro;
            if constexpr (GATHER)
                ro = table[lk];
            else
                ro = lk < len ? base + lk * ld : kOutOfRange;
            const int co = coloff[j & 1];             // (row & 3) = 2 (j & 1) + h
            const int o = (ro < 0 || co < 0) ? kOutOfRange : ro + co;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(stage + q * 1024), 16, o, 0, 0, 0);
        }
    }
};


// One 64-K stage of MFMAs from two DmaRowsT stages ([k][256] each).  For
// K group g, lane l needs K values 16g + 8(l/32) + 0..7 of column l % 32 of
// each 32-column block: two transposing reads whose 16 source lanes address
// rows +((l & 15) >> 2) and 8-byte column blocks (l & 3).
template <int TM, int TN>
__device__ __forceinline__ void mma_stage_tr(const char* As, const char* Bs, int wm0, int wn0,
                                             f32x16 (&acc)[TM][TN]) {
    const int lane = threadIdx.x & 63;
    const int j = (lane & 15) >> 2;
    const int h = lane >> 5;
    const int cw = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int wb = 8 * (lane & 1);
    const int swz = j << 2;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        u32x4 a[TM], b[TN];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int rowb = (16 * g + 8 * h + 4 * r + j) * 512;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const u32x2 v = ds_read_tr16(As + rowb + ((((wm0 + 32 * tm) >> 3) + cw) ^ swz) * 16 + wb);
                a[tm][2 * r] = v[0];
                a[tm][2 * r + 1] = v[1];
            }
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) {
                const u32x2 v = ds_read_tr16(Bs + rowb + ((((wn0 + 32 * tn) >> 3) + cw) ^ swz) * 16 + wb);
                b[tn][2 * r] = v[0];
                b[tn][2 * r + 1] = v[1];
            }
        }
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) mfma_group(KindBF16{}, a[tm], b[tn], acc[tm][tn]);
    }
}

// ---------------------------------------------------------------------------
// SwiGLU backward
// ---------------------------------------------------------------------------
using ShapeBwdGU = TileShape<256, 256, 2, 4, 4>;   // packed gate|up columns of 128 features
using ShapeBwdDH = TileShape<256, 128, 2, 4, 4>;   // the same 128 features of dh

// Epilogue of the saved-g|u bf16 SwiGLU backward without LDS: lanes pair up
// (DPP swap of one dh value, as in store_bf16_pairs) so that each lane owns
// two adjacent features of one row, read as 4-byte pairs from the saved
// gate|up rows; dg, du (packed gate|up column order) and hm leave as 4-byte
// pairs.  acc[.][tn] holds the wave's 32 features from wf0.  Rows past the
// tile's end fall past the buffers' ranges; features past F get
// out-of-range offsets.
template <bool ROUTED, int TN = 1>
__device__ __forceinline__ void swiglu_bwd_pairs(const SwigluBwdArgs& a, const f32x16 (&acc)[4][TN], int tn,
                                                 int64_t m0, int64_t m_end, int64_t f0, int wm0, int wf0,
                                                 const int (*s_route)[kMaxTopK]) {
    const int lane = threadIdx.x & 63;
    const bool odd = lane & 1;
    const int64_t fb = (f0 + wf0 + (lane & 31)) & ~(int64_t)1;   // first feature of the lane's pair
    const int pc2 = (int)(64 * (fb >> 5) + (fb & 31)) * 2;       // its packed gate column, in bytes
    const int rows = (int)(m_end - m0 < 256 ? m_end - m0 : 256);
    // row strides redefined here, so that no offset below is hoisted out of
    // a persistent caller's loop (they would stay live across every stage)
    int ldg2 = (int)a.ldgu * 2, ldd2 = (int)a.lddgu * 2, ldh2 = (int)a.ldhm * 2;
    asm volatile("" : "+s"(ldg2), "+s"(ldd2), "+s"(ldh2));
    const auto rg = make_rsrc(static_cast<const bf16_t*>(a.gu) + m0 * a.ldgu, (uint32_t)(rows * ldg2));
    const auto rd = make_rsrc(static_cast<bf16_t*>(a.dgu) + m0 * a.lddgu, (uint32_t)(rows * ldd2));
    const auto rh = make_rsrc(a.hm != nullptr ? static_cast<bf16_t*>(a.hm) + m0 * a.ldhm : a.dgu,
                              a.hm != nullptr ? (uint32_t)(rows * ldh2) : 0u);
    const int bad = fb < a.F ? 0 : kOutOfRange;
    // a 32-feature block is wholly shared or wholly one expert's
    const bool routed = ROUTED && f0 + wf0 >= a.shared_feats;
    const int expert = routed ? (int)((f0 + wf0 - a.shared_feats) / a.expert_feats) : -1;
    const int row_lane = wm0 + 4 * (lane >> 5) + (lane & 1);   // the pair's row for i = 0, 1
    // lane offsets of row_lane; rows below add uniform multiples of the strides
    // (opaque, so that no row - row_lane multiple is folded back into a
    // per-row product the compiler would hoist and keep live)
    int lg = row_lane * ldg2 + pc2, ld = row_lane * ldd2 + pc2, lh = row_lane * ldh2 + (int)fb * 2;
    asm volatile("" : "+v"(lg), "+v"(ld), "+v"(lh));
    uint32_t gv[2][8], uv[2][8];
    auto load = [&](int tm, int buf) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int off = (lg + (tm * 32 + 8 * (p >> 1) + 2 * (p & 1)) * ldg2) | bad;
            gv[buf][p] = __builtin_amdgcn_raw_buffer_load_b32(rg, off, 0, 0);
            uv[buf][p] = __builtin_amdgcn_raw_buffer_load_b32(rg, off + 64, 0, 0);
        }
    };
    load(0, 0);
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
        if (tm + 1 < 4) load(tm + 1, (tm + 1) & 1);
        const int buf = tm & 1;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const int dr = tm * 32 + 8 * (p >> 1) + 2 * (p & 1);   // row - row_lane
            const int rl = row_lane + dr;
            const float v0 = acc[tm][tn][2 * p], v1 = acc[tm][tn][2 * p + 1];
            const float other = dpp_swap_pairs(odd ? v0 : v1);
            const float dh[2] = {odd ? other : v0, odd ? v1 : other};   // features fb, fb + 1 of row rl
            float mult = a.shared_mult;
            if constexpr (ROUTED) {
                if (routed) {
                    float tw = 0.f;
#pragma unroll
                    for (int j = 0; j < kMaxTopK; ++j) tw += (s_route[rl][j] == expert) ? a.rw[j] : 0.f;
                    mult = tw;
                }
            }
            const bf16x2 g2 = __builtin_bit_cast(bf16x2, (uint32_t)gv[buf][p]);
            const bf16x2 u2 = __builtin_bit_cast(bf16x2, (uint32_t)uv[buf][p]);
            float dg[2], du[2], hv[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const float g = (float)g2[q], u = (float)u2[q];
                const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
                const float sg = __builtin_amdgcn_rcpf(1.0f + e);   // sigmoid(g)
                const float sl = g * sg;                            // silu(g)
                const float dm = dh[q] * mult;
                dg[q] = dm * u * (sg + sl * (1.0f - sg));           // silu'(g) = s + g s (1 - s)
                du[q] = dm * sl;
                // the forward epilogue's expression order, so hm is its h
                hv[q] = (routed ? sl * u : sl * u * a.shared_mult);
                if (routed) hv[q] *= mult;
            }
            const int od = (ld + dr * ldd2) | bad;
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, bf16x2{(bf16_t)dg[0], (bf16_t)dg[1]}),
                                                  rd, od, 0, 0);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, bf16x2{(bf16_t)du[0], (bf16_t)du[1]}),
                                                  rd, od + 64, 0, 0);
            if (a.hm != nullptr)
                __builtin_amdgcn_raw_buffer_store_b32(
                    __builtin_bit_cast(uint32_t, bf16x2{(bf16_t)hv[0], (bf16_t)hv[1]}), rh,
                    (lh + dr * ldh2) | bad, 0, 0);
        }
    }
}

// SAVED: g|u come from a.gu (written by the forward) instead of a
// recomputing tile loop.
template <class Kind, bool GROUPED, bool ROUTED, bool SAVED = false>
__global__ __launch_bounds__(512) void k_swiglu_bwd(SwigluBwdArgs a) {
    using T = typename Kind::T;
    using SG = ShapeBwdGU;
    using SD = ShapeBwdDH;
    static_assert(SG::BM == SD::BM && SG::WAVES_M == SD::WAVES_M && SG::WAVES_N == SD::WAVES_N &&
                      SG::WN == 2 * SD::WN && SD::TN == 1 && SG::TN == 2,
                  "a wave holds gate, up and dh of the same 32 features");
    extern __shared__ __align__(16) char lds[];
    constexpr int64_t kElem = (int64_t)sizeof(T);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / SG::WAVES_N) * SG::WM;
    const int wn0 = (wave % SG::WAVES_N) * SG::WN;   // packed gate|up column within the tile
    const int wf0 = (wave % SD::WAVES_N) * SD::WN;   // feature within the tile (= wn0 / 2)
    int64_t m0 = (int64_t)blockIdx.x * SG::BM;
    int64_t m_end = a.M;
    const int64_t f0 = a.f_base + (int64_t)blockIdx.y * SD::BN;
    const char* wgu = static_cast<const char*>(a.wgu);
    const char* wdt = static_cast<const char*>(a.wdt);

    typename AProvOf<SG>::type ax, ad;
    if constexpr (GROUPED) {
        __shared__ int s_tile[3];
        grouped_tile<SG::BM>(a.offsets, a.E, (int)blockIdx.x, s_tile);
        if (s_tile[0] < 0) return;
        const int64_t e = s_tile[0];
        m0 = s_tile[1];
        m_end = s_tile[2];
        wgu += e * a.wgu_expert_stride * kElem;
        wdt += e * a.wdt_expert_stride * kElem;
        init_gather_rows(ax, a.x, a.gather, a.gather_mod, m0, m_end - m0, a.ldx * kElem, a.K * (int)kElem);
        init_gather_rows(ad, a.dout, a.gather, a.gather_mod, m0, m_end - m0, a.ldd * kElem, a.K * (int)kElem);
    } else {
        init_a<SG>(ax, a.x, m0, a.M, a.ldx * kElem, a.K * (int)kElem);
        init_a<SD>(ad, a.dout, m0, a.M, a.ldd * kElem, a.K * (int)kElem);
    }
    typename BProvOf<Kind, false, SG>::type bgu;
    typename BProvOf<Kind, false, SD>::type bdt;
    bgu.init(wgu, 2 * f0, 2 * a.F, a.ldwgu * kElem, a.K * (int)kElem);
    bdt.init(wdt, f0, a.F, a.ldwdt * kElem, a.K * (int)kElem);

    __shared__ int s_route[ROUTED ? SG::BM : 1][kMaxTopK];
    if constexpr (ROUTED) {
        if (threadIdx.x < SG::BM && f0 + SD::BN > a.shared_feats) {
            const int64_t row = m0 + threadIdx.x;
            int64_t id = row < a.M ? a.ids[row] : 0;
            id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
            for (int j = 0; j < kMaxTopK; ++j)
                s_route[threadIdx.x][j] =
                    (j < a.top_k && row < a.M) ? (int)a.table[(int64_t)j * a.vocab + id] : -1;
        }
    }

    f32x16 acc_gu[SAVED ? 1 : SG::TM][SAVED ? 1 : SG::TN];
    if constexpr (!SAVED) {
        zero_acc<Kind>(acc_gu);
        tile_loop<Kind, SG>(ax, bgu, a.K, lds, wm0, wn0, acc_gu);
    }
    f32x16 acc_dh[SD::TM][SD::TN];
    zero_acc<Kind>(acc_dh);
    tile_loop<Kind, SD>(ad, bdt, a.K, lds, wm0, wf0, acc_dh);
    if constexpr (SAVED && sizeof(T) == 2 && !GROUPED) {
        swiglu_bwd_pairs<ROUTED>(a, acc_dh, 0, m0, m_end, f0, wm0, wf0, s_route);
        return;
    }
    // bf16 saved g|u: the tile's 256 rows x 256 packed columns (128 KiB)
    // staged in LDS (free after the loop) with direct loads, as four 64-column
    // stages, then read back in the accumulator layout
    constexpr bool kStaged = SAVED && sizeof(T) == 2;
    if constexpr (kStaged) {
        typename AProvOf<SG>::type gp;
        const int64_t cols = 2 * (a.F - f0) < 256 ? 2 * (a.F - f0) : 256;
        gp.init(static_cast<const T*>(a.gu) + 2 * f0, m0, m_end, a.ldgu * kElem, (int)(cols * kElem));
#pragma unroll
        for (int kt = 0; kt < 4; ++kt) gp.issue(kt, lds + kt * SG::BM * kRowBytes);
        wait_vmcnt<0>();
        __syncthreads();
    }

    const int64_t f = f0 + wf0 + (lane & 31);
    // bf16: dg|du go through LDS (the staging layout of the saved g|u, in
    // place) and leave as 16-byte stores; f32 stores them directly
    constexpr bool kLdsOut = sizeof(T) == 2;
    if (!kLdsOut && f >= a.F) return;
    const bool fvalid = f < a.F;
    // expert blocks are multiples of 64 features: a 32-feature wave block is
    // wholly shared or one expert's
    const bool routed = ROUTED && f0 + wf0 >= a.shared_feats;
    const int64_t expert = routed ? (f0 + wf0 - a.shared_feats) / a.expert_feats : -1;
    const float mult0 = routed ? 1.0f : a.shared_mult;
    T* dgu = static_cast<T*>(a.dgu);
    T* hm = static_cast<T*>(a.hm);
    // with g|u staged (no recompute accumulators live), hm also waits in
    // registers and leaves through LDS after dg|du
    constexpr bool kHmLds = kStaged;
    T hreg[kHmLds ? SG::TM : 1][kHmLds ? 16 : 1];
    const int64_t pc = 64 * (f >> 5) + (f & 31);   // packed gate column
    const int pcl = (int)(pc - 2 * f0);             // ... within the tile
    char* const gst = lds + (pcl >> 6) * SG::BM * kRowBytes;   // its 64-column LDS stage
    const int cb = (pcl & 63) * 2;                              // byte within a 128-byte stage row
#pragma unroll
    for (int tm = 0; tm < SG::TM; ++tm) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int rl = wm0 + tm * 32 + acc_row(lane, i);
            const int64_t row = m0 + rl;
            const bool valid = fvalid && row < m_end;
            if (!kLdsOut && !valid) continue;
            float g = 0.f, u = 0.f;
            if constexpr (kStaged) {
                g = to_f32(*reinterpret_cast<const T*>(gst + lds_byte(rl, cb >> 4) + (cb & 15)));
                u = to_f32(*reinterpret_cast<const T*>(gst + lds_byte(rl, (cb + 64) >> 4) + (cb & 15)));
            } else if constexpr (SAVED) {
                if (valid) {
                    const T* gr = static_cast<const T*>(a.gu) + row * a.ldgu + pc;
                    g = to_f32(gr[0]);
                    u = to_f32(gr[32]);
                }
            } else {
                g = acc_gu[tm][0][i];
                u = acc_gu[tm][1][i];
            }
            const float dh = acc_dh[tm][0][i];
            float mult = mult0;
            if constexpr (ROUTED) {
                if (routed) {
                    float tw = 0.f;
#pragma unroll
                    for (int j = 0; j < kMaxTopK; ++j) tw += (s_route[rl][j] == expert) ? a.rw[j] : 0.f;
                    mult = tw;
                }
            }
            if constexpr (GROUPED) {
                if (valid) {
                    const int64_t slot = (int64_t)((uint64_t)a.gather[row] / (uint64_t)a.gather_mod);
                    mult = a.rw[slot < kMaxTopK ? slot : kMaxTopK - 1];
                }
            }
            const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
            const float s = __builtin_amdgcn_rcpf(1.0f + e);   // sigmoid(g)
            const float sl = silu_f(g);
            const float dm = dh * mult;
            const float dgv = dm * u * (s + sl * (1.0f - s));   // silu'(g) = s + g s (1 - s)
            const float duv = dm * sl;
            if constexpr (kLdsOut) {
                *reinterpret_cast<T*>(gst + lds_byte(rl, cb >> 4) + (cb & 15)) = from_f32<T>(dgv);
                *reinterpret_cast<T*>(gst + lds_byte(rl, (cb + 64) >> 4) + (cb & 15)) = from_f32<T>(duv);
            } else {
                dgu[row * a.lddgu + pc] = from_f32<T>(dgv);
                dgu[row * a.lddgu + pc + 32] = from_f32<T>(duv);
            }
            // same expression order as the forward epilogue, so hm is the
            // forward's h for the shared and dense-routed forms
            float hv = sl * u * mult0;
            if (ROUTED && routed) hv *= mult;
            if (GROUPED) hv = sl * u * mult;
            if constexpr (kHmLds) hreg[tm][i] = from_f32<T>(hv);
            else if (hm != nullptr && valid) hm[row * a.ldhm + f] = from_f32<T>(hv);
        }
    }
    if constexpr (kLdsOut) {
        // copy the dg|du tile out: 256 rows x 4 stages x 8 chunks of 16 bytes
        wait_lgkmcnt0();
        __syncthreads();
        const int64_t cols = 2 * (a.F - f0) < 256 ? 2 * (a.F - f0) : 256;
        for (int q = threadIdx.x; q < SG::BM * 32; q += SG::NT) {
            const int kt = q / (SG::BM * 8), r = (q / 8) % SG::BM, c = q % 8;
            const int col = kt * 64 + c * 8;
            if (m0 + r < m_end && col < cols)
                *reinterpret_cast<u32x4*>(dgu + (m0 + r) * a.lddgu + 2 * f0 + col) =
                    *reinterpret_cast<const u32x4*>(lds + kt * SG::BM * kRowBytes + lds_byte(r, c));
        }
    }
    if constexpr (kHmLds) {
        if (hm == nullptr) return;
        // hm: 256 rows x 128 features as two 64-feature stages
        __syncthreads();
        const int fl = wf0 + (lane & 31);
        char* const hst = lds + (fl >> 6) * SG::BM * kRowBytes;
        const int hb = (fl & 63) * 2;
#pragma unroll
        for (int tm = 0; tm < SG::TM; ++tm)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                *reinterpret_cast<T*>(hst + lds_byte(wm0 + tm * 32 + acc_row(lane, i), hb >> 4) + (hb & 15)) =
                    hreg[tm][i];
        wait_lgkmcnt0();
        __syncthreads();
        const int64_t hcols = a.F - f0 < SD::BN ? a.F - f0 : SD::BN;
        for (int q = threadIdx.x; q < SG::BM * 16; q += SG::NT) {
            const int kt = q / (SG::BM * 8), r = (q / 8) % SG::BM, c = q % 8;
            const int col = kt * 64 + c * 8;
            if (m0 + r < m_end && col < hcols)
                *reinterpret_cast<u32x4*>(hm + (m0 + r) * a.ldhm + f0 + col) =
                    *reinterpret_cast<const u32x4*>(lds + kt * SG::BM * kRowBytes + lds_byte(r, c));
        }
    }
}


// Persistent form of the saved-g|u bf16 SwiGLU backward for shared features
// (no route multipliers): dh = dout . W_down^T as 256-row x 256-feature tiles
// on the ping-pong stream (pp_stream, one workgroup per CU), each finished
// tile's epilogue (swiglu_bwd_pairs, twice: the wave's two 32-feature
// blocks) straight from the accumulators while the other group multiplies.
// Tiles cover features [0, 256 * n_tiles / tiles_m); features at or past F
// load zero weights and store nothing.
__global__ __launch_bounds__(512, 1) void k_swiglu_bwd_pps(SwigluBwdArgs a, int64_t tiles_m, int64_t n_tiles) {
    extern __shared__ __align__(16) char lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * 128, wn0 = wig * 64;
    const int64_t G = gridDim.x;
    const int ntiles = (int)((n_tiles - (int64_t)blockIdx.x + G - 1) / G);
    if (ntiles <= 0) return;
    const bool xcd_rows = (tiles_m & 7) == 0 && (G & 7) == 0;
    auto coords = [&](int i, int64_t& m0, int64_t& f0) {
        uint32_t mt, nt;
        pps_tile((uint32_t)blockIdx.x + (uint32_t)i * (uint32_t)G, (uint32_t)tiles_m, (uint32_t)(n_tiles / tiles_m),
                 xcd_rows, mt, nt);
        m0 = (int64_t)mt * 256;
        f0 = (int64_t)nt * 256;
    };
    const int64_t ldd_b = a.ldd * (int64_t)sizeof(bf16_t);
    const int64_t ldw_b = a.ldwdt * (int64_t)sizeof(bf16_t);

    PPRows<256> ap, bp;
    int64_t m0, f0;
    coords(0, m0, f0);
    if (group == 1)
        ap.init(a.dout, m0, a.M, ldd_b, wig);
    else
        bp.init(a.wdt, f0, a.F, ldw_b, wig);
    f32x16 acc[4][2];
    zero_acc<KindBF16>(acc);
    pp_stream<4, PPLayoutK<4, true>>(
        ap, bp, a.K / 64, ntiles, lds, group, wm0, wn0, acc,
        [&](int i) {   // i >= ntiles: no rows (the refills past the last stage load zeros)
            int64_t tm0, tf0;
            coords(i, tm0, tf0);
            ap.retarget(a.dout, tm0, i < ntiles ? a.M : tm0, ldd_b);
        },
        [&](int i) {
            int64_t tm0, tf0;
            coords(i, tm0, tf0);
            bp.retarget(a.wdt, tf0, i < ntiles ? a.F : tf0, ldw_b);
        },
        [&](int i, const f32x16 (&c)[4][2]) {
            int64_t tm0, tf0;
            coords(i, tm0, tf0);
            swiglu_bwd_pairs<false, 2>(a, c, 0, tm0, a.M, tf0, wm0, wn0, nullptr);
            swiglu_bwd_pairs<false, 2>(a, c, 1, tm0, a.M, tf0, wm0, wn0 + 32, nullptr);
        });
}
// ---------------------------------------------------------------------------
// weight gradients
// ---------------------------------------------------------------------------
using ShapeWgrad = TileShape<256, 256, 2, 2, 1>;   // 4 waves of 128x128 (accumulators in AGPRs)
constexpr int kWgradSeg = 2048;   // most rows of one split when an operand is gathered

// Stores a wave's accumulators through a buffer descriptor: bf16 (BF16) or
// f32 cells at (r * ld + c); cells outside [0, mlim) x [0, nlim) get an
// offset with bit 31 set, past any range, and are dropped by the hardware.
template <class Shape, bool BF16>
__device__ __forceinline__ void wgrad_store(const f32x16 (&acc)[Shape::TM][Shape::TN], __amdgpu_buffer_rsrc_t rsrc,
                                            int wm0, int wn0, int col, int lane, int ld, int mlim, int nlim) {
    constexpr int kEsz = BF16 ? 2 : 4;
#pragma unroll
    for (int tm = 0; tm < Shape::TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < Shape::TN; ++tn) {
            const int c = wn0 + tn * 32 + col;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = wm0 + tm * 32 + acc_row(lane, i);
                const int off = ((r * ld + c) * kEsz) | ((r < mlim && c < nlim) ? 0 : kOutOfRange);
                // the element is copied to a scalar first: a bit cast of the
                // vector element expression itself reads element 0
                const float v = acc[tm][tn][i];
                if constexpr (BF16)
                    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (bf16_t)v), rsrc, off, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), rsrc, off, 0, 0);
            }
        }
}

template <class Kind, class Shape, bool GA, bool GB>
__global__ __launch_bounds__(Shape::NT) void k_wgrad(WgradArgs a) {
    using T = typename Kind::T;
    extern __shared__ __align__(16) char lds[];
    constexpr int kTable = kWgradSeg + Kind::kStageElems;   // the loop prefetches one stage past the end
    __shared__ int s_ta[GA ? kTable : 1];
    __shared__ int s_tb[GB ? kTable : 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = (int64_t)blockIdx.y * Shape::BN;
    const int e = (int)blockIdx.z / a.splits, sp = (int)blockIdx.z % a.splits;
    const int64_t seg0 = a.offsets ? a.offsets[e] : 0;
    const int64_t seg1 = a.offsets ? a.offsets[e + 1] : a.T;
    const int64_t per = ((seg1 - seg0 + a.splits - 1) / a.splits + Kind::kStageElems - 1) / Kind::kStageElems *
                        Kind::kStageElems;
    const int64_t t0 = seg0 + sp * per;
    const int64_t t1 = t0 + per < seg1 ? t0 + per : seg1;

    BufRowsT<Kind, Shape::BM, Shape::NT, GA> ap;
    BufRowsT<Kind, Shape::BN, Shape::NT, GB> bp;
    ap.init(a.a, a.a_rows, a.lda * (int64_t)sizeof(T), m0, a.M);
    bp.init(a.b, a.b_rows, a.ldb * (int64_t)sizeof(T), n0, a.N);

    // Gathered operands: the byte offsets of the rows are staged in LDS,
    // kWgradSeg rows at a time.
    f32x16 acc[Shape::TM][Shape::TN];
    zero_acc<Kind>(acc);
    for (int64_t s0 = t0; s0 < t1; s0 += kWgradSeg) {
        const int len = (int)(t1 - s0 < kWgradSeg ? t1 - s0 : kWgradSeg);
        if constexpr (GA || GB) {
            // partition values are below 2^31 (the host checks top_k * tokens)
            const uint32_t mod = (uint32_t)a.gather_mod;
            const int lda_b = (int)(a.lda * (int64_t)sizeof(T)), ldb_b = (int)(a.ldb * (int64_t)sizeof(T));
            for (int i = threadIdx.x; i < kTable; i += Shape::NT) {
                if constexpr (GA)
                    s_ta[i] = i < len ? (int)((uint32_t)a.a_gather[s0 + i] % mod) * lda_b : kOutOfRange;
                if constexpr (GB)
                    s_tb[i] = i < len ? (int)((uint32_t)a.b_gather[s0 + i] % mod) * ldb_b : kOutOfRange;
            }
            __syncthreads();
        }
        ap.segment(s0, len, s_ta);
        bp.segment(s0, len, s_tb);
        tile_loop_pgr1<Kind, Shape>(ap, bp, len, lds, wm0, wn0, acc);
        // tile_loop_pgr1 ends on a barrier: the tables may be refilled
    }

    // Branch-free stores: buffer stores at an offset past the descriptor's
    // range are dropped, so cells outside the output take kOutOfRange.
    const bool direct = a.splits == 1;
    const int64_t obase_el = direct ? (int64_t)e * a.out_expert_stride + m0 * a.ldo + n0
                                    : ((int64_t)e * a.splits + sp) * a.M * a.N + m0 * a.N + n0;
    const int ld = (int)(direct ? a.ldo : a.N);
    const int mlim = (int)(a.M - m0 < Shape::BM ? a.M - m0 : Shape::BM);
    const int nlim = (int)(a.N - n0 < Shape::BN ? a.N - n0 : Shape::BN);
    const int esz = direct ? (int)sizeof(T) : 4;
    void* obase = direct ? static_cast<void*>(static_cast<T*>(a.out) + obase_el)
                         : static_cast<void*>(a.partial + obase_el);
    const auto orsrc = make_rsrc(obase, (uint32_t)(((int64_t)(mlim - 1) * ld + nlim) * esz));
    const int col = lane & 31;
    if (direct && sizeof(T) == 2)
        wgrad_store<Shape, true>(acc, orsrc, wm0, wn0, col, lane, ld, mlim, nlim);
    else
        wgrad_store<Shape, false>(acc, orsrc, wm0, wn0, col, lane, ld, mlim, nlim);
}

// bf16 weight gradients with both operands loaded straight into LDS and
// transposed at the fragment read (ds_read_b64_tr_b16); same arguments,
// segments, splits and epilogue as k_wgrad.
using ShapeWgradTr = TileShape<256, 256, 2, 4, 4>;   // 8 waves of 128x64

template <bool GA, bool GB>
__global__ __launch_bounds__(ShapeWgradTr::NT) void k_wgrad_tr(WgradArgs a) {
    using Shape = ShapeWgradTr;
    using T = bf16_t;
    extern __shared__ __align__(16) char lds[];
    constexpr int kTable = kWgradSeg + 128;   // the loop issues up to two stages ahead
    __shared__ int s_ta[GA ? kTable : 1];
    __shared__ int s_tb[GB ? kTable : 1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm0 = (wave / Shape::WAVES_N) * Shape::WM;
    const int wn0 = (wave % Shape::WAVES_N) * Shape::WN;
    const int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = (int64_t)blockIdx.y * Shape::BN;
    const int e = (int)blockIdx.z / a.splits, sp = (int)blockIdx.z % a.splits;
    const int64_t seg0 = a.offsets ? a.offsets[e] : 0;
    const int64_t seg1 = a.offsets ? a.offsets[e + 1] : a.T;
    const int64_t per = ((seg1 - seg0 + a.splits - 1) / a.splits + 63) / 64 * 64;
    const int64_t t0 = seg0 + sp * per;
    const int64_t t1 = t0 + per < seg1 ? t0 + per : seg1;

    DmaRowsT<Shape::NT, GA> ap;
    DmaRowsT<Shape::NT, GB> bp;
    ap.init(a.a, a.a_rows, a.lda * 2, m0, a.M);
    bp.init(a.b, a.b_rows, a.ldb * 2, n0, a.N);
    constexpr int kABytes = Shape::BM * kRowBytes;   // 64 rows x 512 bytes
    constexpr int kPer = 2 * DmaRowsT<Shape::NT, GA>::kInstr;

    f32x16 acc[Shape::TM][Shape::TN];
    zero_acc<KindBF16>(acc);
    for (int64_t s0 = t0; s0 < t1; s0 += kWgradSeg) {
        const int len = (int)(t1 - s0 < kWgradSeg ? t1 - s0 : kWgradSeg);
        if constexpr (GA || GB) {
            const uint32_t mod = (uint32_t)a.gather_mod;
            const int lda_b = (int)(a.lda * 2), ldb_b = (int)(a.ldb * 2);
            for (int i = threadIdx.x; i < kTable; i += Shape::NT) {
                if constexpr (GA)
                    s_ta[i] = i < len ? (int)((uint32_t)a.a_gather[s0 + i] % mod) * lda_b : kOutOfRange;
                if constexpr (GB)
                    s_tb[i] = i < len ? (int)((uint32_t)a.b_gather[s0 + i] % mod) * ldb_b : kOutOfRange;
            }
            __syncthreads();
        }
        ap.segment(s0, len, s_ta);
        bp.segment(s0, len, s_tb);
        const int nk = (len + 63) / 64;
        ap.issue(0, lds);
        bp.issue(0, lds + kABytes);
        if (nk > 1) {
            ap.issue(1, lds + Shape::kStageBytes);
            bp.issue(1, lds + Shape::kStageBytes + kABytes);
        }
        for (int kt = 0; kt < nk; ++kt) {
            char* st = lds + (kt & 1) * Shape::kStageBytes;
            if (kt + 1 < nk)
                wait_vmcnt<kPer>();
            else
                wait_vmcnt<0>();
            lds_barrier();
            mma_stage_tr<Shape::TM, Shape::TN>(st, st + kABytes, wm0, wn0, acc);
            if (kt + 2 < nk) {
                wait_lgkmcnt0();
                lds_barrier();
                ap.issue(kt + 2, st);
                bp.issue(kt + 2, st + kABytes);
            }
        }
        __syncthreads();   // stages and tables free for the next segment
    }

    const bool direct = a.splits == 1;
    const int64_t obase_el = direct ? (int64_t)e * a.out_expert_stride + m0 * a.ldo + n0
                                    : ((int64_t)e * a.splits + sp) * a.M * a.N + m0 * a.N + n0;
    const int ld = (int)(direct ? a.ldo : a.N);
    const int mlim = (int)(a.M - m0 < Shape::BM ? a.M - m0 : Shape::BM);
    const int nlim = (int)(a.N - n0 < Shape::BN ? a.N - n0 : Shape::BN);
    void* obase = direct ? static_cast<void*>(static_cast<T*>(a.out) + obase_el)
                         : static_cast<void*>(a.partial + obase_el);
    const auto orsrc = make_rsrc(obase, (uint32_t)(((int64_t)(mlim - 1) * ld + nlim) * (direct ? 2 : 4)));
    const int col = lane & 31;
    if (direct)
        wgrad_store<Shape, true>(acc, orsrc, wm0, wn0, col, lane, ld, mlim, nlim);
    else
        wgrad_store<Shape, false>(acc, orsrc, wm0, wn0, col, lane, ld, mlim, nlim);
}

// bf16 weight gradients of token-major operands without gathered rows, on
// the ping-pong main loop: each group loads one operand straight into LDS
// (PPRowsT) and every wave transposes at the fragment read; the workgroup's
// whole token range (its split) in one pass.  Same arguments, splits and
// epilogue as k_wgrad_tr.
__global__ __launch_bounds__(512, 1) void k_wgrad_pp(WgradArgs a) {
    using Shape = ShapeWgradTr;   // 256 x 256: waves 2 x 4 of 128 x 64, the ping-pong groups' layout
    extern __shared__ __align__(16) char lds[];
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int group = wave >> 2, wig = wave & 3;
    const int wm0 = group * Shape::WM, wn0 = wig * Shape::WN;
    const int64_t m0 = (int64_t)blockIdx.x * Shape::BM;
    const int64_t n0 = (int64_t)blockIdx.y * Shape::BN;
    const int e = (int)blockIdx.z / a.splits, sp = (int)blockIdx.z % a.splits;
    const int64_t seg0 = a.offsets ? a.offsets[e] : 0;
    const int64_t seg1 = a.offsets ? a.offsets[e + 1] : a.T;
    const int64_t per = ((seg1 - seg0 + a.splits - 1) / a.splits + 63) / 64 * 64;
    const int64_t t0 = seg0 + sp * per;
    const int64_t t1 = t0 + per < seg1 ? t0 + per : seg1;
    const int len = t1 > t0 ? (int)(t1 - t0) : 0;

    PPRowsT ap, bp;
    if (group == 1) {
        ap.init(a.a, a.a_rows, a.lda * 2, m0, a.M, wig);
        ap.segment(t0, len);
    } else {
        bp.init(a.b, a.b_rows, a.ldb * 2, n0, a.N, wig);
        bp.segment(t0, len);
    }
    f32x16 acc[Shape::TM][Shape::TN];
    zero_acc<KindBF16>(acc);
    const int nk = (len + 63) / 64;
    if (nk > 0) pp_main<4, PPLayoutT>(ap, bp, nk, lds, group, wm0, wn0, acc, [](const f32x16 (&)[4][2]) {});

    const bool direct = a.partial == nullptr;   // else an fp32 partial for the reduction (which may map it)
    const int64_t obase_el = direct ? (int64_t)e * a.out_expert_stride + m0 * a.ldo + n0
                                    : ((int64_t)e * a.splits + sp) * a.M * a.N + m0 * a.N + n0;
    const int ld = (int)(direct ? a.ldo : a.N);
    const int mlim = (int)(a.M - m0 < Shape::BM ? a.M - m0 : Shape::BM);
    const int nlim = (int)(a.N - n0 < Shape::BN ? a.N - n0 : Shape::BN);
    void* obase = direct ? static_cast<void*>(static_cast<bf16_t*>(a.out) + obase_el)
                         : static_cast<void*>(a.partial + obase_el);
    const auto orsrc = make_rsrc(obase, (uint32_t)(((int64_t)(mlim - 1) * ld + nlim) * (direct ? 2 : 4)));
    const int col = lane & 31;
    if (direct)
        wgrad_store<Shape, true>(acc, orsrc, wm0, wn0, col, lane, ld, mlim, nlim);
    else
        wgrad_store<Shape, false>(acc, orsrc, wm0, wn0, col, lane, ld, mlim, nlim);
}

template <class T>
__global__ __launch_bounds__(256) void k_wgrad_reduce(WgradArgs a) {
    // four consecutive columns per thread (N is a multiple of 8): 16-byte
    // loads of each split's partial, summed in split order per element
    const int64_t mn = a.M * a.N;
    const int64_t q4 = a.N >> 2;
    const int64_t total = (int64_t)a.E * a.M * q4;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = idx / q4;   // e * M + m
        const int64_t n = (idx - row * q4) * 4;
        const int64_t e = row / a.M, m = row - e * a.M;
        const float* p = a.partial + e * a.splits * mn + m * a.N + n;
        float s[4] = {0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < a.splits; ++sp) {
            const float4 v = *reinterpret_cast<const float4*>(p + sp * mn);
            s[0] += v.x;
            s[1] += v.y;
            s[2] += v.z;
            s[3] += v.w;
        }
        T* out = static_cast<T*>(a.out);
        if (a.map_mode == 1) {
            const int64_t o = a.map_off[m];
            const int64_t st = a.map_stride[m];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t d = mapped_dest(o, n + c, st, a.out_elems);
                if (d >= 0) out[d] = from_f32<T>(s[c]);
            }
        } else if (a.map_mode == 2) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t d = mapped_dest(a.map_off[n + c], m, a.map_stride[n + c], a.out_elems);
                if (d >= 0) out[d] = from_f32<T>(s[c]);
            }
        } else {
            const int64_t dst = e * a.out_expert_stride + m * a.ldo + n;
#pragma unroll
            for (int c = 0; c < 4; ++c) out[dst + c] = from_f32<T>(s[c]);
        }
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <class F>
static int bwd_lds(F* fn, int bytes) {
    return set_kernel_lds(reinterpret_cast<const void*>(fn), bytes);
}

template <class Kind, bool GROUPED, bool ROUTED, bool SAVED = false>
static int swiglu_bwd_kind(const SwigluBwdArgs& a, int64_t assignments, hipStream_t stream) {
    auto kern = k_swiglu_bwd<Kind, GROUPED, ROUTED, SAVED>;
    constexpr int kLds = ShapeBwdGU::kLdsBytes;
    int st = bwd_lds(kern, kLds);
    if (st) return st;
    const int64_t tiles_m =
        GROUPED ? (assignments + ShapeBwdGU::BM - 1) / ShapeBwdGU::BM + a.E : (a.M + ShapeBwdGU::BM - 1) / ShapeBwdGU::BM;
    const int64_t tiles_f = (a.F - a.f_base + ShapeBwdDH::BN - 1) / ShapeBwdDH::BN;
    if (tiles_m <= 0 || tiles_f <= 0) return TRMOE_OK;
    hipLaunchKernelGGL(kern, dim3((unsigned)tiles_m, (unsigned)tiles_f), dim3(512), kLds, stream, a);
    return check_launch("swiglu_backward");
}

static int bwd_device_cus() { return current_device_cus(); }

// The persistent launch: 256-feature tiles over features [0, feats).
static int launch_swiglu_bwd_pps(const SwigluBwdArgs& a, int64_t feats, hipStream_t stream) {
    const int64_t tiles_m = (a.M + 255) / 256;
    const int64_t n_tiles = tiles_m * ((feats + 255) / 256);
    const int64_t cus = bwd_device_cus();
    const int64_t grid = n_tiles < cus ? n_tiles : cus;
    constexpr int kLds = 2 * PPLayoutK<4, true>::kStage;
    int st = bwd_lds(k_swiglu_bwd_pps, kLds);
    if (st) return st;
    if (grid <= 0) return TRMOE_OK;
    hipLaunchKernelGGL(k_swiglu_bwd_pps, dim3((unsigned)grid), dim3(512), kLds, stream, a, tiles_m, n_tiles);
    return check_launch("swiglu_backward");
}

int launch_swiglu_bwd(int act, const SwigluBwdArgs& a, int64_t assignments, hipStream_t stream) {
    const bool grouped = a.offsets != nullptr, routed = a.ids != nullptr;
    if (a.gu != nullptr) {
        // saved pre-activations (shared and dense-routed forms)
        if (grouped) return set_error(TRMOE_ERR_UNSUPPORTED, "swiglu_backward: saved gate|up for grouped rows");
        if (act == TRMOE_BF16) {
            // features without route multipliers (whole 256-feature tiles of
            // them when routed) on the persistent stream when that fills at
            // least a round of CUs; the rest on the tile kernel
            const int64_t feats = routed ? (a.shared_feats < a.F ? a.shared_feats : a.F) / 256 * 256 : a.F;
            const int64_t tiles = ((a.M + 255) / 256) * ((feats + 255) / 256);
            if (a.f_base == 0 && a.K % 64 == 0 && feats > 0 && tiles >= bwd_device_cus()) {
                const int st = launch_swiglu_bwd_pps(a, feats, stream);
                if (st || feats >= a.F) return st;
                SwigluBwdArgs t = a;
                t.f_base = feats;
                return routed ? swiglu_bwd_kind<KindBF16, false, true, true>(t, assignments, stream)
                              : swiglu_bwd_kind<KindBF16, false, false, true>(t, assignments, stream);
            }
            return routed ? swiglu_bwd_kind<KindBF16, false, true, true>(a, assignments, stream)
                          : swiglu_bwd_kind<KindBF16, false, false, true>(a, assignments, stream);
        }
        return routed ? swiglu_bwd_kind<KindF32, false, true, true>(a, assignments, stream)
                      : swiglu_bwd_kind<KindF32, false, false, true>(a, assignments, stream);
    }
    if (act == TRMOE_BF16) {
        if (grouped) return swiglu_bwd_kind<KindBF16, true, false>(a, assignments, stream);
        if (routed) return swiglu_bwd_kind<KindBF16, false, true>(a, assignments, stream);
        return swiglu_bwd_kind<KindBF16, false, false>(a, assignments, stream);
    }
    if (grouped) return swiglu_bwd_kind<KindF32, true, false>(a, assignments, stream);
    if (routed) return swiglu_bwd_kind<KindF32, false, true>(a, assignments, stream);
    return swiglu_bwd_kind<KindF32, false, false>(a, assignments, stream);
}


// Split count: a workgroup holds a CU (128 KiB of LDS), so the launch runs
// in ceil(tiles * s / CUs) rounds of rows/s rows each; every split adds an
// fp32 partial of M*N*E values written and read back by the reduction
// (about M*N*E * 6e-5 row-steps of a tile at the measured rates).  Picks
// the s (at most 32, at least 256 rows per split) with the smallest sum.
int wgrad_splits(int64_t M, int64_t N, int E, int64_t rows_per_segment) {
    const int64_t tiles = ((M + ShapeWgrad::BM - 1) / ShapeWgrad::BM) * ((N + ShapeWgrad::BN - 1) / ShapeWgrad::BN) * E;
    const int64_t cus = bwd_device_cus();
    const double per_split = (double)M * (double)N * (double)E * 6e-5;
    int best = 1;
    double best_cost = 1e300;
    for (int s = 1; s <= 32; ++s) {
        if (s > 1 && rows_per_segment / s < 256) break;
        const int64_t rounds = (tiles * s + cus - 1) / cus;
        const double cost = (double)rounds * (double)((rows_per_segment + s - 1) / s) + (s > 1 ? s * per_split : 0.0);
        if (cost < best_cost) {
            best_cost = cost;
            best = s;
        }
    }
    return best;
}

template <class Kind, bool GA, bool GB>
static int wgrad_kind(const WgradArgs& a, hipStream_t stream) {
    auto kern = k_wgrad<Kind, ShapeWgrad, GA, GB>;
    constexpr int kLds = ShapeWgrad::kLdsBytes;
    int st = bwd_lds(kern, kLds);
    if (st) return st;
    const dim3 grid((unsigned)((a.M + ShapeWgrad::BM - 1) / ShapeWgrad::BM),
                    (unsigned)((a.N + ShapeWgrad::BN - 1) / ShapeWgrad::BN), (unsigned)(a.E * a.splits));
    hipLaunchKernelGGL(kern, grid, dim3(ShapeWgrad::NT), kLds, stream, a);
    st = check_launch("weight_grad");
    if (st || a.splits == 1) return st;
    int64_t blocks = ((int64_t)a.E * a.M * (a.N / 4) + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_wgrad_reduce<typename Kind::T>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return check_launch("weight_grad (reduce)");
}

template <bool GA, bool GB>
static int wgrad_tr(const WgradArgs& a, hipStream_t stream) {
    auto kern = k_wgrad_tr<GA, GB>;
    constexpr int kLds = ShapeWgradTr::kLdsBytes;
    int st = bwd_lds(kern, kLds);
    if (st) return st;
    const dim3 grid((unsigned)((a.M + ShapeWgradTr::BM - 1) / ShapeWgradTr::BM),
                    (unsigned)((a.N + ShapeWgradTr::BN - 1) / ShapeWgradTr::BN), (unsigned)(a.E * a.splits));
    hipLaunchKernelGGL(kern, grid, dim3(ShapeWgradTr::NT), kLds, stream, a);
    st = check_launch("weight_grad");
    if (st || a.splits == 1) return st;
    int64_t blocks = ((int64_t)a.E * a.M * (a.N / 4) + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_wgrad_reduce<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return check_launch("weight_grad (reduce)");
}

static int wgrad_pp(const WgradArgs& a, hipStream_t stream) {
    constexpr int kLds = 2 * PPLayoutT::kStage;
    int st = bwd_lds(k_wgrad_pp, kLds);
    if (st) return st;
    const dim3 grid((unsigned)((a.M + ShapeWgradTr::BM - 1) / ShapeWgradTr::BM),
                    (unsigned)((a.N + ShapeWgradTr::BN - 1) / ShapeWgradTr::BN), (unsigned)(a.E * a.splits));
    hipLaunchKernelGGL(k_wgrad_pp, grid, dim3(512), kLds, stream, a);
    st = check_launch("weight_grad");
    if (st || a.partial == nullptr) return st;
    int64_t blocks = ((int64_t)a.E * a.M * (a.N / 4) + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    hipLaunchKernelGGL(k_wgrad_reduce<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, stream, a);
    return check_launch("weight_grad (reduce)");
}

// bf16: direct loads + transposing fragment reads (on the ping-pong loop
// without gathered rows); f32: the register-transposing kernel.
int launch_wgrad(int act, const WgradArgs& a, hipStream_t stream) {
    const bool ga = a.a_gather != nullptr, gb = a.b_gather != nullptr;
    if (act == TRMOE_BF16 && !ga && !gb) return wgrad_pp(a, stream);
    if (act == TRMOE_BF16) {
        if (ga) return gb ? wgrad_tr<true, true>(a, stream) : wgrad_tr<true, false>(a, stream);
        return gb ? wgrad_tr<false, true>(a, stream) : wgrad_tr<false, false>(a, stream);
    }
    if (ga) return gb ? wgrad_kind<KindF32, true, true>(a, stream) : wgrad_kind<KindF32, true, false>(a, stream);
    return gb ? wgrad_kind<KindF32, false, true>(a, stream) : wgrad_kind<KindF32, false, false>(a, stream);
}

}  // namespace trmoe
