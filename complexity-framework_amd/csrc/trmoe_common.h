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

#include <type_traits>

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
// 64-byte rows (four 16-byte chunks, swizzled by (r >> 1) & 3: every 8-lane
// phase of a ds_read_b128 lands on distinct bank groups).
constexpr int kRow64 = 64;
__device__ __forceinline__ int lds_swz64(int r) { return (r >> 1) & 3; }
__device__ __forceinline__ int lds_byte64(int r, int c) { return r * kRow64 + ((c ^ lds_swz64(r)) << 4); }

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

// Row of accumulator element i of a 32x32 MFMA tile held by `lane` (its
// column is lane % 32).
__device__ __forceinline__ int acc_row(int lane, int i) {
    return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}

// ---------------------------------------------------------------------------
// buffer loads
// ---------------------------------------------------------------------------
// Operands are read with raw buffer loads: a load whose byte offset is at or
// past the descriptor's range returns zero, so absent rows and the K tail
// need no branches.  kOutOfRange is an offset no range reaches (ranges are
// kept below 2^31 bytes by the host).
constexpr int kOutOfRange = (int)0x80000000u;
constexpr int kBufferFlags = 0x00020000;   // gfx9 raw buffer, 32-bit dword data

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}

__device__ __forceinline__ u32x4 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, int offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, offset, 0, 0));
}

__device__ __forceinline__ u32x2 buffer_load8(__amdgpu_buffer_rsrc_t rsrc, int offset) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, offset, 0, 0));
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
// A provider owns ROWS rows of one operand tile.  Thread t handles the
// ROWS*8/256 chunks q = t + 256*j: row q/8, 16-byte chunk t%8 of the row's
// 128-byte K stage.  prefetch(kt) issues the buffer loads of stage kt into
// registers, commit() writes them to an LDS stage in the swizzled layout.
//
// Row requirements (checked by the host): rows start 16-byte aligned and the
// elements between K and the next multiple of 8 are zero (or K % 8 == 0), so
// whole 16-byte chunks can be loaded.

// 16-byte-chunk operand (bf16 or f32 elements in memory and in LDS).
template <int ROWS, int NT>
struct BufRows {
    static constexpr int kChunks = ROWS * 8 / NT;
    static constexpr int kThreadsPerBlock = NT;
    using Reg = u32x4;
    __amdgpu_buffer_rsrc_t rsrc;
    int row_off[kChunks];   // byte offset of the row, kOutOfRange when absent
    int kbytes;             // bytes of K per row; chunks at or past it load zero

    __device__ void prefetch(int kt, Reg (&reg)[kChunks]) const {
        const int kb = kt * kRowBytes + (threadIdx.x & 7) * 16;
        const bool in_k = kb < kbytes;
#pragma unroll
        for (int j = 0; j < kChunks; ++j) reg[j] = buffer_load16(rsrc, in_k ? row_off[j] + kb : kOutOfRange);
    }
    __device__ void commit(char* stage, const Reg (&reg)[kChunks]) const {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) commit_one(stage, reg, j);
    }
    __device__ __forceinline__ void commit_one(char* stage, const Reg (&reg)[kChunks], int j) const {
        const int q = threadIdx.x + NT * j;
        *reinterpret_cast<u32x4*>(stage + lds_byte(q >> 3, q & 7)) = reg[j];
    }
};

// e4m3 operand: 8-byte chunks in memory (64 K values per stage), expanded to
// 16-byte bf16 chunks in LDS.
template <int ROWS, int NT>
struct BufRowsFP8 {
    static constexpr int kChunks = ROWS * 8 / NT;
    static constexpr int kThreadsPerBlock = NT;
    using Reg = u32x2;
    __amdgpu_buffer_rsrc_t rsrc;
    int row_off[kChunks];
    int kbytes;

    __device__ void prefetch(int kt, Reg (&reg)[kChunks]) const {
        const int kb = kt * 64 + (threadIdx.x & 7) * 8;
        const bool in_k = kb < kbytes;
#pragma unroll
        for (int j = 0; j < kChunks; ++j) reg[j] = buffer_load8(rsrc, in_k ? row_off[j] + kb : kOutOfRange);
    }
    __device__ void commit(char* stage, const Reg (&reg)[kChunks]) const {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) commit_one(stage, reg, j);
    }
    __device__ __forceinline__ void commit_one(char* stage, const Reg (&reg)[kChunks], int j) const {
        const int q = threadIdx.x + NT * j;
        *reinterpret_cast<u32x4*>(stage + lds_byte(q >> 3, q & 7)) = fp8x8_to_bf16x8(reg[j]);
    }
};

// Dense rows [row0, row0 + ROWS) of a row-major matrix with `rows_total`
// rows of `ld_bytes` bytes; rows past the end load zero.
template <class Prov>
__device__ __forceinline__ void init_dense_rows(Prov& p, const void* base, int64_t row0, int64_t rows_total,
                                                int64_t ld_bytes, int kbytes) {
    constexpr int NT = Prov::kThreadsPerBlock;
    constexpr int ROWS = Prov::kChunks * NT / 8;
    const int64_t avail = rows_total - row0;
    const int64_t nrows = avail < ROWS ? avail : ROWS;
    p.rsrc = make_rsrc(static_cast<const char*>(base) + row0 * ld_bytes, (uint32_t)(nrows * ld_bytes));
    p.kbytes = kbytes;
#pragma unroll
    for (int j = 0; j < Prov::kChunks; ++j) {
        const int r = (threadIdx.x >> 3) + (NT / 8) * j;
        p.row_off[j] = (r < nrows) ? (int)(r * ld_bytes) : kOutOfRange;
    }
}

// ---------------------------------------------------------------------------
// the tile main loop
// ---------------------------------------------------------------------------
// Block tile BM x BN, 4 waves as WAVES_M x WAVES_N, each wave TM x TN MFMA
// tiles of 32x32.  Two LDS stages; one barrier per K stage.  `lds` holds
// 2 * (BM + BN) * 128 bytes.
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_, int PGR_ = 1>
struct TileShape {
    // 1: register-staged loads, one stage ahead (tile_loop_pgr1);
    // 4: direct buffer->LDS loads (tile_loop_dma, bf16/f32 operands only);
    static constexpr int PGR = PGR_;
    static constexpr int BM = BM_;
    static constexpr int BN = BN_;
    static constexpr int WAVES_M = WAVES_M_;
    static constexpr int WAVES_N = WAVES_N_;
    static constexpr int NT = 64 * WAVES_M * WAVES_N;   // threads per workgroup
    static constexpr int WM = BM / WAVES_M;
    static constexpr int WN = BN / WAVES_N;
    static constexpr int TM = WM / 32;
    static constexpr int TN = WN / 32;
    // 6: direct loads, bf16 A rows of 128 bytes + e4m3 B rows of 64 bytes per
    //    64-element K stage, expanded to bf16 at the fragment read
    static constexpr int kStages = 2;
    static constexpr int kStageBytes = PGR == 6 ? BM * kRowBytes + BN * 64 : (BM + BN) * kRowBytes;
    static constexpr int kLdsBytes = kStages * kStageBytes;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert((BM * 8) % NT == 0 && (BN * 8) % NT == 0, "tile rows must split evenly over threads");
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

// One 64-element K stage with e4m3 B rows of 64 bytes (lds_byte64 layout):
// lane (r, h) of group g reads the 8 bytes of K elements 16g + 8h .. +7 and
// expands them to bf16 (exact) for the MFMA.
template <int TM, int TN>
__device__ __forceinline__ void mma_stage_f8(const char* As, const char* Bs, int wm0, int wn0,
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
            b[tn] = fp8x8_to_bf16x8(*reinterpret_cast<const u32x2*>(Bs + lds_byte64(wn0 + tn * 32 + r, g) + 8 * h));
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < TN; ++tn) mfma_group(KindBF16{}, a[tm], b[tn], acc[tm][tn]);
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

// A and B both streamed from global through two LDS stages.  Each K stage
// is one basic block: the loads of stage kt+1 are issued before the MFMAs of
// stage kt and written to the other LDS stage after them (past the last
// stage they read zeros and land in a stage nobody reads), then one barrier.
template <class Kind, class Shape, class AProv, class BProv>
__device__ __forceinline__ void tile_loop_pgr1(const AProv& ap, const BProv& bp, int K, char* lds, int wm0,
                                               int wn0, f32x16 (&acc)[Shape::TM][Shape::TN]) {
    const int nk = (K + Kind::kStageElems - 1) / Kind::kStageElems;
    constexpr int kABytes = Shape::BM * kRowBytes;
    typename AProv::Reg ra[AProv::kChunks];
    typename BProv::Reg rb[BProv::kChunks];
    ap.prefetch(0, ra);
    bp.prefetch(0, rb);
    ap.commit(lds, ra);
    bp.commit(lds + kABytes, rb);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        char* cur = lds + (kt & 1) * Shape::kStageBytes;
        char* nxt = lds + ((kt + 1) & 1) * Shape::kStageBytes;
        ap.prefetch(kt + 1, ra);
        bp.prefetch(kt + 1, rb);
        // keep the loads at the top of the stage: left alone, the scheduler
        // sinks them next to the LDS writes and exposes their whole latency
        __builtin_amdgcn_sched_barrier(0);
        mma_stage<Kind, Shape::TM, Shape::TN>(cur, cur + kABytes, wm0, wn0, acc);
        __builtin_amdgcn_sched_barrier(0);
        ap.commit(nxt, ra);
        bp.commit(nxt + kABytes, rb);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// direct buffer -> LDS operand loads
// ---------------------------------------------------------------------------
// `buffer_load_dwordx4 ... lds` writes each lane's 16 bytes to LDS at
// M0 + 16 * lane, without passing through VGPRs (out-of-range offsets write
// zeros, like ordinary buffer loads).  One wave instruction therefore fills
// 8 consecutive 128-byte tile rows; the swizzle is applied on the global
// side: the lane that owns LDS slot s of row r fetches K chunk s ^ swz(r),
// so the stage ends up in the layout lds_byte() describes.
//
// Waits are explicit: vmcnt counts these loads, and a workgroup barrier
// after the wait makes every wave's rows visible.

#define TRMOE_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt on vmcnt only (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4)); }

// Workgroup barrier that orders the compiler's memory operations around it
// without the vmcnt(0) drain of __syncthreads().
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int ROWS, int NT>
struct DmaRows {
    static constexpr int kInstr = ROWS * 8 / NT;   // wave instructions per thread per stage
    static constexpr int kWaves = NT / 64;
    static constexpr int kRowsPerInstr = 8;
    // K chunk the lane fetches for LDS row r (its slot is lane & 7)
    static __device__ __forceinline__ int chunk_of(int lane, int r) { return (lane & 7) ^ lds_swz(r); }
    static_assert(ROWS % (8 * kWaves) == 0, "each wave fills whole 8-row groups");
    __amdgpu_buffer_rsrc_t rsrc;
    int off[kInstr];    // lane's byte offset in the row for K stage 0, kOutOfRange when absent
    int koff[kInstr];   // byte offset of the lane's chunk within a K stage
    int kbytes;
    int wave;           // wave index, uniform

    // rows [row0, row0 + ROWS) of a matrix with rows_total rows of ld_bytes
    __device__ __forceinline__ void init(const void* base, int64_t row0, int64_t rows_total, int64_t ld_bytes,
                                         int kbytes_) {
        const int64_t avail = rows_total - row0;
        const int64_t nrows = avail < ROWS ? avail : ROWS;
        rsrc = make_rsrc(static_cast<const char*>(base) + row0 * ld_bytes, (uint32_t)(nrows * ld_bytes));
        kbytes = kbytes_;
        wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
            const int r = (wave * kInstr + j) * 8 + (lane >> 3);
            koff[j] = chunk_of(lane, r) * 16;
            off[j] = r < nrows ? (int)(r * ld_bytes) + koff[j] : kOutOfRange;
        }
    }
    __device__ __forceinline__ void issue(int kt, char* stage) const {
        const int kb = kt * kRowBytes;
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
            const int o = (kb + koff[j] < kbytes) ? off[j] + kb : kOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(stage + (wave * kInstr + j) * 8 * kRowBytes),
                                                    16, o, 0, 0, 0);
        }
    }
};

// The K loop over two LDS stages filled by DmaRows, stages 0 and 1 already
// requested (and, of all vector memory operations issued so far, stage 1's
// are the most recent): stage kt+2 is requested as soon as every wave has
// read stage kt, so each load has one stage of MFMA work to land.
template <class Kind, class Shape, class AP, class BP>
__device__ __forceinline__ void dma_mainloop(const AP& ap, const BP& bp, int nk, char* lds, int wm0, int wn0,
                                             f32x16 (&acc)[Shape::TM][Shape::TN]) {
    constexpr int kABytes = Shape::BM * kRowBytes;
    constexpr int kPer = AP::kInstr + BP::kInstr;
    for (int kt = 0; kt < nk; ++kt) {
        char* st = lds + (kt & 1) * Shape::kStageBytes;
        if (kt + 1 < nk)
            wait_vmcnt<kPer>();
        else
            wait_vmcnt<0>();
        lds_barrier();
        if constexpr (Shape::PGR == 6)
            mma_stage_f8<Shape::TM, Shape::TN>(st, st + kABytes, wm0, wn0, acc);
        else
            mma_stage<Kind, Shape::TM, Shape::TN>(st, st + kABytes, wm0, wn0, acc);
        if (kt + 2 < nk) {
            wait_lgkmcnt0();   // this wave's reads of the stage are complete
            lds_barrier();     // ... and every other wave's
            ap.issue(kt + 2, st);
            bp.issue(kt + 2, st + kABytes);
        }
    }
}

// ---- 64-byte rows (e4m3 weights: 64 K values per stage) --------------------
// Rows hold four 16-byte chunks swizzled by (r >> 1) & 3, which keeps every
// 8-lane phase of a ds_read_b128 on distinct bank groups.

template <int ROWS, int NT>
struct DmaRows64 {
    static constexpr int kInstr = ROWS * 4 / NT;   // each wave instruction fills 16 rows
    static constexpr int kWaves = NT / 64;
    static constexpr int kRowsPerInstr = 16;
    static __device__ __forceinline__ int chunk_of(int lane, int r) { return (lane & 3) ^ lds_swz64(r); }
    static_assert(ROWS % (16 * kWaves) == 0, "each wave fills whole 16-row groups");
    __amdgpu_buffer_rsrc_t rsrc;
    int off[kInstr];
    int koff[kInstr];
    int kbytes;
    int wave;

    __device__ __forceinline__ void init(const void* base, int64_t row0, int64_t rows_total, int64_t ld_bytes,
                                         int kbytes_) {
        const int64_t avail = rows_total - row0;
        const int64_t nrows = avail < ROWS ? avail : ROWS;
        rsrc = make_rsrc(static_cast<const char*>(base) + row0 * ld_bytes, (uint32_t)(nrows * ld_bytes));
        kbytes = kbytes_;
        wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
        const int lane = threadIdx.x & 63;
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
            const int r = (wave * kInstr + j) * 16 + (lane >> 2);
            koff[j] = chunk_of(lane, r) * 16;
            off[j] = r < nrows ? (int)(r * ld_bytes) + koff[j] : kOutOfRange;
        }
    }
    __device__ __forceinline__ void issue(int kt, char* stage) const {
        const int kb = kt * kRow64;
#pragma unroll
        for (int j = 0; j < kInstr; ++j) {
            const int o = (kb + koff[j] < kbytes) ? off[j] + kb : kOutOfRange;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(stage + (wave * kInstr + j) * 16 * kRow64),
                                                    16, o, 0, 0, 0);
        }
    }
};

// Direct-load providers (a `wave` field and per-lane offsets) versus the
// register-staged ones (`row_off`).
template <class P>
struct requires_wave_field : std::false_type {};
template <int R, int N>
struct requires_wave_field<DmaRows<R, N>> : std::true_type {};
template <int R, int N>
struct requires_wave_field<DmaRows64<R, N>> : std::true_type {};

// Whole tile: request stages 0 and 1, run the K loop, end with a full
// barrier (callers reuse LDS in their epilogues).
template <class Kind, class Shape, class AP, class BP>
__device__ __forceinline__ void tile_loop_dma(const AP& ap, const BP& bp, int K, char* lds, int wm0, int wn0,
                                              f32x16 (&acc)[Shape::TM][Shape::TN]) {
    const int nk = (K + Kind::kStageElems - 1) / Kind::kStageElems;
    constexpr int kABytes = Shape::BM * kRowBytes;
    ap.issue(0, lds);
    bp.issue(0, lds + kABytes);
    if (nk > 1) {
        ap.issue(1, lds + Shape::kStageBytes);
        bp.issue(1, lds + Shape::kStageBytes + kABytes);
    }
    dma_mainloop<Kind, Shape>(ap, bp, nk, lds, wm0, wn0, acc);
    __syncthreads();
}

template <class Kind, class Shape, class AProv, class BProv>
__device__ __forceinline__ void tile_loop(const AProv& ap, const BProv& bp, int K, char* lds, int wm0, int wn0,
                                          f32x16 (&acc)[Shape::TM][Shape::TN]) {
    if constexpr (Shape::PGR == 4 || Shape::PGR == 6)
        tile_loop_dma<Kind, Shape>(ap, bp, K, lds, wm0, wn0, acc);
    else
        tile_loop_pgr1<Kind, Shape>(ap, bp, K, lds, wm0, wn0, acc);
}

// A resident in LDS (one 128-byte-row stage per K stage, BM rows each), B
// streamed.  `bstage` holds 2 * BN * 128 bytes.
template <class Kind, class Shape, class BProv>
__device__ __forceinline__ void tile_loop_lds_a(const char* a_lds, int a_stage_bytes, const BProv& bp, int K,
                                                char* bstage, int wm0, int wn0,
                                                f32x16 (&acc)[Shape::TM][Shape::TN]) {
    const int nk = (K + Kind::kStageElems - 1) / Kind::kStageElems;
    constexpr int kBBytes = Shape::BN * kRowBytes;
    typename BProv::Reg rb[BProv::kChunks];
    bp.prefetch(0, rb);
    bp.commit(bstage, rb);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        char* cur = bstage + (kt & 1) * kBBytes;
        char* nxt = bstage + ((kt + 1) & 1) * kBBytes;
        const bool more = kt + 1 < nk;
        if (more) bp.prefetch(kt + 1, rb);
        __builtin_amdgcn_sched_barrier(0);
        mma_stage<Kind, Shape::TM, Shape::TN>(a_lds + kt * a_stage_bytes, cur, wm0, wn0, acc);
        __builtin_amdgcn_sched_barrier(0);
        if (more) bp.commit(nxt, rb);
        __syncthreads();
    }
}

// silu(g) = g / (1 + e^-g) with the hardware exp2 and reciprocal (about
// 1 ulp each); for g < -126/log2(e) the exponential overflows to +inf and
// the reciprocal returns 0, the correct limit.
__device__ __forceinline__ float silu_f(float g) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace trmoe
