// Shared device machinery of the TR-MoE HIP kernels (gfx950 / CDNA4).
//
// Tile GEMM building blocks for C[m, n] = sum_k A[m, k] * B[n, k]: both
// operands are K-contiguous ("NT"), which is the layout the MFMA operand
// registers want.  Activations are A; weights are B, pre-packed by
// trmoe_pack_weight() into [rows, cols] with rows padded to the tile width and
// cols padded to a multiple of 8 elements (zero filled).
//
// LDS holds one K stage of a tile as rows of 128 bytes (64 bf16 or 32 f32).
// The 16-byte chunk c of row r is stored at chunk c ^ swz(r) with
// swz(r) = (r ^ (r >> 3)) & 7, so the 32 rows one MFMA operand read touches
// spread over every bank for both 32- and 64-bank LDS organisations.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trmoe {

typedef __bf16 bf16_t;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kRowBytes = 128;   // LDS bytes per tile row per K stage
constexpr int kThreads = 256;    // every tile kernel runs 4 waves of 64

__device__ __forceinline__ int lds_swz(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int lds_byte(int r, int c) {
    return r * kRowBytes + ((c ^ lds_swz(r)) << 4);
}

// ---------------------------------------------------------------------------
// element kinds
// ---------------------------------------------------------------------------
struct KindBF16 {
    using T = bf16_t;
    static constexpr int kPerChunk = 8;       // elements per 16-byte chunk
    static constexpr int kStageElems = 64;    // K elements per LDS stage
};
struct KindF32 {
    using T = float;
    static constexpr int kPerChunk = 4;
    static constexpr int kStageElems = 32;
};

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) { return (float)v; }
template <class T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) { return (bf16_t)v; }

// One 32-byte K group of an MFMA step: every lane supplies the 16-byte chunk
// at K offset 16*(lane/32) bytes of the group for its row (A) / column (B).
// Both operands use the same K mapping, so the dot product is exact for any
// within-group K order the instruction uses internally.
__device__ __forceinline__ void mfma_group(KindBF16, u32x4 a, u32x4 b, f32x16& acc) {
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
}
__device__ __forceinline__ void mfma_group(KindF32, u32x4 a, u32x4 b, f32x16& acc) {
    f32x4 fa = __builtin_bit_cast(f32x4, a);
    f32x4 fb = __builtin_bit_cast(f32x4, b);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[0], fb[0], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[1], fb[1], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[2], fb[2], acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[3], fb[3], acc, 0, 0, 0);
}

// Accumulator element i of a 32x32 MFMA tile held by `lane`.
__device__ __forceinline__ int acc_row(int lane, int i) {
    return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}
__device__ __forceinline__ int acc_col(int lane) { return lane & 31; }

// ---------------------------------------------------------------------------
// global chunk loads
// ---------------------------------------------------------------------------
// 16 bytes of K elements [k, k + kPerChunk) of one row; zero beyond K.
template <class Kind>
__device__ __forceinline__ u32x4 load_chunk(const typename Kind::T* row, int k, int K, bool vec_ok) {
    using T = typename Kind::T;
    if (row == nullptr || k >= K) return u32x4{0, 0, 0, 0};
    if (vec_ok && k + Kind::kPerChunk <= K) {
        return *reinterpret_cast<const u32x4*>(row + k);
    }
    union { u32x4 v; T e[Kind::kPerChunk]; } u;
    u.v = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < Kind::kPerChunk; ++i)
        if (k + i < K) u.e[i] = row[k + i];
    return u.v;
}

// 8 OCP e4m3 weights -> 8 bf16 (exact: every e4m3 value is a bf16 value).
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(u32x2 q) {
    bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, false);
    bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[0], 1.0f, true);
    bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, false);
    bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(q[1], 1.0f, true);
    return u32x4{__builtin_bit_cast(uint32_t, p0), __builtin_bit_cast(uint32_t, p1),
                 __builtin_bit_cast(uint32_t, p2), __builtin_bit_cast(uint32_t, p3)};
}

// ---------------------------------------------------------------------------
// operand providers for the tile main loop
// ---------------------------------------------------------------------------
// Each provider owns ROWS rows of one operand tile.  A thread handles
// ROWS*8/256 chunks: chunk q = tid + 256*j sits at row q/8, chunk q%8.

// Activation rows from global memory (dense or gathered), staged through LDS.
template <class Kind, int ROWS>
struct GlobalRows {
    using T = typename Kind::T;
    static constexpr int kChunks = ROWS * 8 / kThreads;
    const T* rowp[kChunks];
    u32x4 reg[kChunks];
    int K;
    bool vec_ok;

    __device__ void prefetch(int kt) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            int q = threadIdx.x + kThreads * j;
            int c = q & 7;
            reg[j] = load_chunk<Kind>(rowp[j], kt * Kind::kStageElems + c * Kind::kPerChunk, K, vec_ok);
        }
    }
    __device__ void commit(char* stage) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            int q = threadIdx.x + kThreads * j;
            *reinterpret_cast<u32x4*>(stage + lds_byte(q >> 3, q & 7)) = reg[j];
        }
    }
};

// Packed weight rows [rows, ld] (bf16 or f32), no row guard (rows are padded).
template <class Kind, int ROWS>
struct PackedRows {
    using T = typename Kind::T;
    static constexpr int kChunks = ROWS * 8 / kThreads;
    const T* base;     // first row of the tile
    int64_t ld;        // elements per packed row
    u32x4 reg[kChunks];
    int K;

    __device__ void prefetch(int kt) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            int q = threadIdx.x + kThreads * j;
            int r = q >> 3, c = q & 7;
            int k = kt * Kind::kStageElems + c * Kind::kPerChunk;
            reg[j] = (k < K) ? *reinterpret_cast<const u32x4*>(base + r * ld + k) : u32x4{0, 0, 0, 0};
        }
    }
    __device__ void commit(char* stage) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            int q = threadIdx.x + kThreads * j;
            *reinterpret_cast<u32x4*>(stage + lds_byte(q >> 3, q & 7)) = reg[j];
        }
    }
};

// Packed e4m3 weight rows [rows, ld bytes]; expanded to bf16 on the way to LDS.
template <int ROWS>
struct PackedRowsFP8 {
    static constexpr int kChunks = ROWS * 8 / kThreads;
    const uint8_t* base;
    int64_t ld;
    u32x2 reg[kChunks];
    int K;

    __device__ void prefetch(int kt) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            int q = threadIdx.x + kThreads * j;
            int r = q >> 3, c = q & 7;
            int k = kt * 64 + c * 8;
            reg[j] = (k < K) ? *reinterpret_cast<const u32x2*>(base + r * ld + k) : u32x2{0, 0};
        }
    }
    __device__ void commit(char* stage) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            int q = threadIdx.x + kThreads * j;
            *reinterpret_cast<u32x4*>(stage + lds_byte(q >> 3, q & 7)) = fp8x8_to_bf16x8(reg[j]);
        }
    }
};

// ---------------------------------------------------------------------------
// the tile main loop
// ---------------------------------------------------------------------------
// Block tile BM x BN, 4 waves as WAVES_M x WAVES_N, each wave TM x TN MFMA
// tiles of 32x32.  Two LDS stages; one barrier per K stage.  `lds` holds
// 2 * (BM + BN) * 128 bytes.
template <int BM_, int BN_, int WAVES_M_>
struct TileShape {
    static constexpr int BM = BM_;
    static constexpr int BN = BN_;
    static constexpr int WAVES_M = WAVES_M_;
    static constexpr int WAVES_N = 4 / WAVES_M;
    static constexpr int WM = BM / WAVES_M;
    static constexpr int WN = BN / WAVES_N;
    static constexpr int TM = WM / 32;
    static constexpr int TN = WN / 32;
    static constexpr int kStageBytes = (BM + BN) * kRowBytes;
    static constexpr int kLdsBytes = 2 * kStageBytes;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
};

template <class Kind, int TM, int TN>
__device__ __forceinline__ void mma_stage(const char* As, const char* Bs, int wm0, int wn0,
                                          f32x16 (&acc)[TM][TN]) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        u32x4 a[TM], b[TN];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
            a[tm] = *reinterpret_cast<const u32x4*>(As + lds_byte(wm0 + tm * 32 + r, 2 * g + h));
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
            b[tn] = *reinterpret_cast<const u32x4*>(Bs + lds_byte(wn0 + tn * 32 + r, 2 * g + h));
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) mfma_group(Kind{}, a[tm], b[tn], acc[tm][tn]);
    }
}

template <class Kind, int TM, int TN>
__device__ __forceinline__ void zero_acc(f32x16 (&acc)[TM][TN]) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[tm][tn][i] = 0.f;
}

// A and B both streamed from global through the two LDS stages.
template <class Kind, class Shape, class AProv, class BProv>
__device__ __forceinline__ void tile_loop(AProv& ap, BProv& bp, int K, char* lds, int wm0, int wn0,
                                          f32x16 (&acc)[Shape::TM][Shape::TN]) {
    const int nk = (K + Kind::kStageElems - 1) / Kind::kStageElems;
    char* stage0 = lds;
    char* stage1 = lds + Shape::kStageBytes;
    constexpr int kABytes = Shape::BM * kRowBytes;
    ap.prefetch(0);
    bp.prefetch(0);
    ap.commit(stage0);
    bp.commit(stage0 + kABytes);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        char* cur = (kt & 1) ? stage1 : stage0;
        char* nxt = (kt & 1) ? stage0 : stage1;
        const bool more = kt + 1 < nk;
        if (more) {
            ap.prefetch(kt + 1);
            bp.prefetch(kt + 1);
        }
        mma_stage<Kind, Shape::TM, Shape::TN>(cur, cur + kABytes, wm0, wn0, acc);
        if (more) {
            ap.commit(nxt);
            bp.commit(nxt + kABytes);
        }
        __syncthreads();
    }
}

// A resident in LDS (one 128-byte-row stage per K stage, BM rows each), B
// streamed.  `bstage` holds 2 * BN * 128 bytes.
template <class Kind, class Shape, class BProv>
__device__ __forceinline__ void tile_loop_lds_a(const char* a_lds, int a_stage_bytes, BProv& bp, int K,
                                                char* bstage, int wm0, int wn0,
                                                f32x16 (&acc)[Shape::TM][Shape::TN]) {
    const int nk = (K + Kind::kStageElems - 1) / Kind::kStageElems;
    constexpr int kBBytes = Shape::BN * kRowBytes;
    bp.prefetch(0);
    bp.commit(bstage);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        char* cur = bstage + (kt & 1) * kBBytes;
        char* nxt = bstage + ((kt + 1) & 1) * kBBytes;
        const bool more = kt + 1 < nk;
        if (more) bp.prefetch(kt + 1);
        mma_stage<Kind, Shape::TM, Shape::TN>(a_lds + kt * a_stage_bytes, cur, wm0, wn0, acc);
        if (more) bp.commit(nxt);
        __syncthreads();
    }
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + __expf(-g)); }

}  // namespace trmoe
