// Ping-pong main loop of the bf16 prefill GEMMs (gate|up, down, weight
// gradients): loaders, stage layouts, fragment reads and the loop itself.
#pragma once

#include "trmoe_common.h"

namespace trmoe {

// ---------------------------------------------------------------------------
// ping-pong main loop
// ---------------------------------------------------------------------------
// 256x256 tiles, 8 waves of 128x64, two LDS stages of 64-element K (A rows
// then B rows, 128-byte swizzled rows, filled by direct buffer->LDS loads).
// The two waves of each SIMD alternate roles every phase: while one
// multiplies a whole K stage from registers, the other reads its next
// stage's fragments from LDS, so the matrix pipe runs one wave's MFMAs at a
// time and the LDS reads and load issue of the other hide under them.
//
// Group 0 = waves 0..3 (tile rows 0..127), group 1 = waves 4..7 (rows
// 128..255, one phase behind).  With a barrier closing every phase:
//   phase 2t    group 0 reads stage t, then issues B(t+1) [weights] into
//               the other buffer; group 1 multiplies stage t-1 and, between
//               its MFMAs, issues A(t+1) [activations] into that buffer
//   phase 2t+1  group 0 multiplies stage t, then waits for its B(t+1);
//               group 1 reads stage t, then waits for its A(t+1)
// so every stage is complete (each issuing group waited for its own loads)
// one barrier before its first reader, and a buffer is refilled only after
// every wave of both groups has read it and passed a barrier: a group's
// waves read a stage in the same phase, so a load issued by one of them in
// that phase could overwrite rows that another has not read yet.  In the
// phase after its last multiply group 0 writes its half of the epilogue tile
// to LDS while group 1 multiplies.

// One operand's direct loads by one group of 4 waves: ROWS rows x 128 bytes
// per stage, ROWS / 32 wave instructions (8 rows each) per wave.
template <int ROWS>
struct PPRows {
    static constexpr int kInstr = ROWS / 32;
    __amdgpu_buffer_rsrc_t rsrc;
    int row0;        // lane's first row: ROWS / 4 * wave_in_group + lane / 8
    int row_bytes;   // row stride in bytes
    int nrows;       // rows present; rows at or past it load zero
    int c0;          // (lane % 8) ^ (lane / 8), the lane's part of the K chunk
    int wig;

    __device__ __forceinline__ void init(const void* base, int64_t first_row, int64_t rows_total, int64_t ld_bytes,
                                         int wave_in_group) {
        const int64_t avail = rows_total - first_row;
        nrows = (int)(avail < 0 ? 0 : (avail < ROWS ? avail : ROWS));   // the descriptor's range: never negative
        rsrc = make_rsrc(static_cast<const char*>(base) + first_row * ld_bytes, (uint32_t)(nrows * ld_bytes));
        const int lane = threadIdx.x & 63;
        wig = wave_in_group;
        row0 = ROWS / 4 * wave_in_group + (lane >> 3);
        row_bytes = (int)ld_bytes;
        c0 = ((lane & 7) ^ (lane >> 3)) & 7;
    }
    // the same loader over another row block of the operand (the lane's
    // position in the stage does not change)
    __device__ __forceinline__ void retarget(const void* base, int64_t first_row, int64_t rows_total,
                                             int64_t ld_bytes) {
        const int64_t avail = rows_total - first_row;
        nrows = (int)(avail < 0 ? 0 : (avail < ROWS ? avail : ROWS));   // the descriptor's range: never negative
        rsrc = make_rsrc(static_cast<const char*>(base) + first_row * ld_bytes, (uint32_t)(nrows * ld_bytes));
    }
    // stage kt (bytes [128 kt, 128 kt + 128) of every row) into `dst` (the
    // operand's part of an LDS stage).  LDS slot (lane % 8) of row r holds K
    // chunk slot ^ swz(r); the rows of instruction j have r / 8 = kInstr *
    // wave_in_group + j, so swz(r) = (lane / 8) ^ (kInstr * wave_in_group + j).
    // A row at or past nrows starts at or past the descriptor's range
    // (nrows * row_bytes), so it loads zeros without a select; the stage's K
    // offset goes in the scalar offset.
    __device__ __forceinline__ void issue_one(int j, int kt, char* dst) const {
        const int r = row0 + 8 * j;
        const int chunk = (c0 ^ (kInstr * wig + j)) & 7;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(dst + (kInstr * wig + j) * 8 * kRowBytes), 16,
                                                r * row_bytes + (chunk << 4), kt * kRowBytes, 0, 0);
    }
    __device__ __forceinline__ void issue(int kt, char* dst) const {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) issue_one(j, kt, dst);
    }
};

// Gathered activation rows for group 1's loads: 256 tile rows, tile row r
// read from byte offset goff[r] of the whole operand (kOutOfRange: zeros).
// goff lives in LDS; the lanes of wave_in_group w load and own rows
// 64 w .. 64 w + 63, so a wave only reads offsets it wrote itself.
struct PPGather {
    static constexpr int kInstr = 8;
    __amdgpu_buffer_rsrc_t rsrc;
    const int* goff;
    int row0;   // 64 wave_in_group + lane / 8
    int c0;     // (lane % 8) ^ (lane / 8)
    int wig;

    __device__ __forceinline__ void init(const void* base, int64_t bytes, const int* goff_lds, int wave_in_group) {
        rsrc = make_rsrc(base, (uint32_t)bytes);
        goff = goff_lds;
        const int lane = threadIdx.x & 63;
        wig = wave_in_group;
        row0 = 64 * wave_in_group + (lane >> 3);
        c0 = ((lane & 7) ^ (lane >> 3)) & 7;
    }
    // an absent row's kOutOfRange (2^31) stays past the operand's range with
    // its chunk added; the stage's K offset is the scalar offset
    __device__ __forceinline__ void issue_one(int j, int kt, char* dst) const {
        const int chunk = (c0 ^ (kInstr * wig + j)) & 7;
        const int g = goff[row0 + 8 * j];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(dst + (kInstr * wig + j) * 8 * kRowBytes), 16,
                                                g + (chunk << 4), kt * kRowBytes, 0, 0);
    }
    __device__ __forceinline__ void issue(int kt, char* dst) const {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) issue_one(j, kt, dst);
    }
};

template <bool V>
struct BoolC {
    static constexpr bool value = V;
};

// Phase boundary: no instruction (MFMAs included) moves across it.
__device__ __forceinline__ void pp_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
}

// The wave's fragments of one K stage: A rows wm0 + 32 tm + r (A block of
// a_rows rows first in the stage), B rows wn0 + 32 tn + r, 16-byte chunk
// 2 g + h of the 128-byte row.
//
// Addresses: for a row 32 t + r of a block starting at a multiple of 64 rows,
// lds_swz(row) = lds_swz(r) ^ 4 (t & 1), so every fragment address is one of
// eight per-lane patterns (K group g, parity of t) plus a uniform offset.
// The patterns are redefined at each call: kept live across a caller's loop
// they and their hoisted sums would take registers the loop needs.  The
// persistent loop (pp_stream), whose tile loop would otherwise spill, reads
// this way (PAT); pp_main's kernels keep one address per fragment, which
// measured a few percent faster there.
__device__ __forceinline__ void pp_patterns(int (&pat)[4][2]) {
    const int lane = threadIdx.x & 63;
    const int r = lane & 31, h = lane >> 5;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            pat[g][p] = r * kRowBytes + (((2 * g + h) ^ lds_swz(r) ^ (4 * p)) << 4);
            asm volatile("" : "+v"(pat[g][p]));
        }
}

template <int TM, bool PAT = false>
__device__ __forceinline__ void pp_read(const char* st, int a_rows, int wm0, int wn0, u32x4 (&fa)[4][TM],
                                        u32x4 (&fb)[4][2]) {
    if constexpr (PAT) {
        int pat[4][2];
        pp_patterns(pat);
        const char* As = st + wm0 * kRowBytes;
        const char* Bs = st + (a_rows + wn0) * kRowBytes;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                fa[g][tm] = *reinterpret_cast<const u32x4*>(As + tm * 32 * kRowBytes + pat[g][tm & 1]);
#pragma unroll
            for (int tn = 0; tn < 2; ++tn)
                fb[g][tn] = *reinterpret_cast<const u32x4*>(Bs + tn * 32 * kRowBytes + pat[g][tn & 1]);
        }
    } else {
        const int lane = threadIdx.x & 63;
        const int r = lane & 31, h = lane >> 5;
        const char* As = st;
        const char* Bs = st + a_rows * kRowBytes;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                fa[g][tm] = *reinterpret_cast<const u32x4*>(As + lds_byte(wm0 + tm * 32 + r, 2 * g + h));
#pragma unroll
            for (int tn = 0; tn < 2; ++tn)
                fb[g][tn] = *reinterpret_cast<const u32x4*>(Bs + lds_byte(wn0 + tn * 32 + r, 2 * g + h));
        }
    }
}

template <int TM>
__device__ __forceinline__ void pp_mma(const u32x4 (&fa)[4][TM], const u32x4 (&fb)[4][2], f32x16 (&acc)[TM][2]) {
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) mfma_group(KindBF16{}, fa[g][tm], fb[g][tn], acc[tm][tn]);
}

// pp_mma with the loads of one stage of an operand issued between the MFMAs
// (one every 8 TM / kInstr MFMAs), so that their issue hides under the
// matrix pipe instead of delaying the phase's first MFMA.
template <int TM, class LD>
__device__ __forceinline__ void pp_mma_load(const u32x4 (&fa)[4][TM], const u32x4 (&fb)[4][2], f32x16 (&acc)[TM][2],
                                            const LD& ld, int kt, char* dst) {
    constexpr int kMfma = 8 * TM;
    constexpr int kEvery = kMfma / LD::kInstr;
    static_assert(kEvery >= 1 && kMfma % LD::kInstr == 0, "loads must spread evenly over the MFMAs");
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const int i = (g * TM + tm) * 2 + tn;
                mfma_group(KindBF16{}, fa[g][tm], fb[g][tn], acc[tm][tn]);
                if (i % kEvery == 0) ld.issue_one(i / kEvery, kt, dst);
            }
    // keep that order through scheduling: one MFMA, one load, the rest of its MFMAs
#pragma unroll
    for (int j = 0; j < LD::kInstr; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);            // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);            // VMEM read
        __builtin_amdgcn_sched_group_barrier(0x008, kEvery - 1, 0);   // MFMA
    }
}

// e4m3 x e4m3 stages (W8A8): a 128-byte stage row holds 128 K values, two
// v_mfma_scale_f32_32x32x64_f8f6f4 steps (unit scales).  That MFMA takes 32
// bytes of K per lane (row lane % 32, the two lane halves disjoint K); any
// assignment of the stage's bytes to (lane half, operand register) works as
// long as A and B use the same one.  K step q takes the 16-byte chunks that
// the bf16 reads give K groups 2q and 2q + 1 (chunks 4q + h and 4q + 2 + h of
// lane half h), read straight into the two halves of one 8-register operand.
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x8 lds_pair(const char* p0, const char* p1) {
    const i32x4 lo = *reinterpret_cast<const i32x4*>(p0);
    const i32x4 hi = *reinterpret_cast<const i32x4*>(p1);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int TM, bool PAT = false>
__device__ __forceinline__ void pp_read_f8(const char* st, int a_rows, int wm0, int wn0, i32x8 (&fa)[2][TM],
                                           i32x8 (&fb)[2][2]) {
    if constexpr (PAT) {
        int pat[4][2];
        pp_patterns(pat);
        const char* As = st + wm0 * kRowBytes;
        const char* Bs = st + (a_rows + wn0) * kRowBytes;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                fa[q][tm] = lds_pair(As + tm * 32 * kRowBytes + pat[2 * q][tm & 1],
                                     As + tm * 32 * kRowBytes + pat[2 * q + 1][tm & 1]);
#pragma unroll
            for (int tn = 0; tn < 2; ++tn)
                fb[q][tn] = lds_pair(Bs + tn * 32 * kRowBytes + pat[2 * q][tn & 1],
                                     Bs + tn * 32 * kRowBytes + pat[2 * q + 1][tn & 1]);
        }
    } else {
        const int lane = threadIdx.x & 63;
        const int r = lane & 31, h = lane >> 5;
        const char* As = st;
        const char* Bs = st + a_rows * kRowBytes;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
#pragma unroll
            for (int tm = 0; tm < TM; ++tm)
                fa[q][tm] = lds_pair(As + lds_byte(wm0 + tm * 32 + r, 4 * q + h),
                                     As + lds_byte(wm0 + tm * 32 + r, 4 * q + 2 + h));
#pragma unroll
            for (int tn = 0; tn < 2; ++tn)
                fb[q][tn] = lds_pair(Bs + lds_byte(wn0 + tn * 32 + r, 4 * q + h),
                                     Bs + lds_byte(wn0 + tn * 32 + r, 4 * q + 2 + h));
        }
    }
}

__device__ __forceinline__ void mfma_f8(const i32x8& a, const i32x8& b, f32x16& acc) {
    // formats 0 / 0: e4m3 operands; scales 127: 2^0 in E8M0
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, 0, 127, 0, 127);
}

// TR: transposed accumulator blocks, B times A: block (tm, tn) holds row
// 32 tn + acc_row(lane, i) of B's rows against A's row 32 tm + lane % 32.
template <int TM, bool TR = false>
__device__ __forceinline__ void pp_mma_f8(const i32x8 (&fa)[2][TM], const i32x8 (&fb)[2][2],
                                          f32x16 (&acc)[TM][2]) {
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                if constexpr (TR)
                    mfma_f8(fb[q][tn], fa[q][tm], acc[tm][tn]);
                else
                    mfma_f8(fa[q][tm], fb[q][tn], acc[tm][tn]);
            }
}

// pp_mma_f8 with one stage of an operand's loads spread over its MFMAs (as
// pp_mma_load does for bf16).
template <int TM, class LD, bool TR = false>
__device__ __forceinline__ void pp_mma_load_f8(const i32x8 (&fa)[2][TM], const i32x8 (&fb)[2][2],
                                               f32x16 (&acc)[TM][2], const LD& ld, int kt, char* dst) {
    constexpr int kMfma = 4 * TM;
    constexpr int kEvery = kMfma / LD::kInstr;
    static_assert(kEvery >= 1 && kMfma % LD::kInstr == 0, "loads must spread evenly over the MFMAs");
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const int i = (q * TM + tm) * 2 + tn;
                if constexpr (TR)
                    mfma_f8(fb[q][tn], fa[q][tm], acc[tm][tn]);
                else
                    mfma_f8(fa[q][tm], fb[q][tn], acc[tm][tn]);
                if (i % kEvery == 0) ld.issue_one(i / kEvery, kt, dst);
            }
#pragma unroll
    for (int j = 0; j < LD::kInstr; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);            // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);            // VMEM read
        __builtin_amdgcn_sched_group_barrier(0x008, kEvery - 1, 0);   // MFMA
    }
}

// Block-scaled A (W8A8 with e4m3 h): the A operand's E8M0 scales, one per
// row and 32 K values, in the MFMA's scale operand.  A K step's 64 K values
// are two blocks: bytes [0, 32) of the step (registers 0-3 of both lane
// halves) take the scale of lane half 0 (the row's lane l), bytes [32, 64)
// (registers 4-7) that of lane half 1 (lane l + 32); the operand's byte
// OPSEL holds it.  B's scale is 2^0.  sa[tm]: the row's four block scales
// of the stage shifted right by 8 (lane / 32), so that byte 0 is the lane
// half's block of step 0 and byte 2 its block of step 1.
template <int OPSEL>
__device__ __forceinline__ void mfma_f8s(const i32x8& a, const i32x8& b, f32x16& acc, uint32_t sa) {
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, acc, 0, 0, OPSEL, (int)sa, 0, 127);
}

template <int TM>
__device__ __forceinline__ void pp_mma_f8s(const i32x8 (&fa)[2][TM], const i32x8 (&fb)[2][2], f32x16 (&acc)[TM][2],
                                           const uint32_t (&sa)[TM]) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) mfma_f8s<0>(fa[0][tm], fb[0][tn], acc[tm][tn], sa[tm]);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) mfma_f8s<2>(fa[1][tm], fb[1][tn], acc[tm][tn], sa[tm]);
}

// pp_mma_f8s with one stage of an operand's loads spread over its MFMAs.
template <int TM, class LD>
__device__ __forceinline__ void pp_mma_load_f8s(const i32x8 (&fa)[2][TM], const i32x8 (&fb)[2][2],
                                                f32x16 (&acc)[TM][2], const uint32_t (&sa)[TM], const LD& ld, int kt,
                                                char* dst) {
    constexpr int kMfma = 4 * TM;
    constexpr int kEvery = kMfma / LD::kInstr;
    static_assert(kEvery >= 1 && kMfma % LD::kInstr == 0, "loads must spread evenly over the MFMAs");
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int i = tm * 2 + tn;
            mfma_f8s<0>(fa[0][tm], fb[0][tn], acc[tm][tn], sa[tm]);
            if (i % kEvery == 0) ld.issue_one(i / kEvery, kt, dst);
        }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn) {
            const int i = 2 * TM + tm * 2 + tn;
            mfma_f8s<2>(fa[1][tm], fb[1][tn], acc[tm][tn], sa[tm]);
            if (i % kEvery == 0) ld.issue_one(i / kEvery, kt, dst);
        }
#pragma unroll
    for (int j = 0; j < LD::kInstr; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);            // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);            // VMEM read
        __builtin_amdgcn_sched_group_barrier(0x008, kEvery - 1, 0);   // MFMA
    }
}

// Scale sources of pp_main: none (unit scales), or the E8M0 block scales of
// the wave's A rows (a byte array of ldhs bytes per row, 4 bytes per 128-K
// stage): the dword of stage t of rows wm0 + 32 tm + lane % 32 of the tile.
// Rows past the descriptor's range (rows_total) read 0, a scale of 2^-127
// on rows whose codes load as zero.
struct PPNoScales {
    static constexpr bool kOn = false;
    template <int TM>
    __device__ __forceinline__ void load(int, uint32_t (&)[TM]) const {}
};

struct PPBlockScales {
    static constexpr bool kOn = true;
    __amdgpu_buffer_rsrc_t rsrc;
    int off;      // byte offset of the lane's row for tm = 0
    int step;     // 32 rows
    int shift;    // 8 (lane / 32)
    __device__ __forceinline__ void init(const void* hs, int64_t ldhs, int64_t first_row, int64_t rows_total,
                                         int wm0) {
        const int64_t avail = rows_total - first_row;
        const int64_t nrows = avail < 0 ? 0 : (avail < 256 ? avail : 256);
        rsrc = make_rsrc(static_cast<const char*>(hs) + first_row * ldhs, (uint32_t)(nrows * ldhs));
        const int lane = threadIdx.x & 63;
        off = (wm0 + (lane & 31)) * (int)ldhs;
        step = 32 * (int)ldhs;
        shift = 8 * (lane >> 5);
    }
    template <int TM>
    __device__ __forceinline__ void load(int t, uint32_t (&dst)[TM]) const {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) dst[tm] = __builtin_amdgcn_raw_buffer_load_b32(rsrc, off + tm * step, 4 * t, 0);
    }
    template <int TM>
    __device__ __forceinline__ void take(const uint32_t (&src)[TM], uint32_t (&dst)[TM]) const {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm) dst[tm] = src[tm] >> shift;
    }
};

// Layouts whose stages hold e4m3 A and B (kF8Mma) multiply with pp_mma_f8.
template <class L, class = void>
struct F8Mma : std::false_type {};
template <class L>
struct F8Mma<L, std::void_t<decltype(L::kF8Mma)>> : std::integral_constant<bool, L::kF8Mma> {};

// Tile of the ping-pong kernel: 64 * TMW rows x 256 packed columns, waves
// 2 x 4 of 32 * TMW rows x 64 columns (the epilogue's layout).
template <int TMW>
using ShapePP = TileShape<64 * TMW, 256, 2, 4, 4>;

// Stage layouts of the ping-pong loop.  PPLayoutK: operands with K along
// their rows (activations x, packed weights): A rows then B rows of 128
// bytes.  PPLayoutT: operands with K across rows (the weight gradients'
// token-major operands): 64 K rows of 256 A columns, then of 256 B columns.
template <int TMW, bool PAT = false>
struct PPLayoutK {
    static constexpr int kBOff = 64 * TMW * kRowBytes;
    static constexpr int kStage = (64 * TMW + 256) * kRowBytes;
    __device__ __forceinline__ static void read(const char* st, int wm0, int wn0, u32x4 (&fa)[4][TMW],
                                                u32x4 (&fb)[4][2]) {
        pp_read<TMW, PAT>(st, 64 * TMW, wm0, wn0, fa, fb);
    }
};

// e4m3 activations and e4m3 weights (W8A8): the bytes of PPLayoutK, 128 K
// values per stage row, multiplied by pp_mma_f8.
template <int TMW, bool PAT = false>
struct PPLayoutK8 {
    static constexpr bool kF8Mma = true;
    static constexpr int kBOff = 64 * TMW * kRowBytes;
    static constexpr int kStage = (64 * TMW + 256) * kRowBytes;
    __device__ __forceinline__ static void read(const char* st, int wm0, int wn0, i32x8 (&fa)[2][TMW],
                                                i32x8 (&fb)[2][2]) {
        pp_read_f8<TMW, PAT>(st, 64 * TMW, wm0, wn0, fa, fb);
    }
};

// The e4m3 weight operand loaded by one group of 4 waves: 256 rows of 64
// bytes (64 K values) per stage, 16 rows per wave instruction, chunk c of
// row r stored at chunk c ^ lds_swz64(r) (the lds_byte64 layout); rows at or
// past rows_total and K bytes at or past kbytes load zero.
struct PPRows64 {
    static constexpr int kInstr = 4;   // 16 instructions of 16 rows per stage over 4 waves
    __amdgpu_buffer_rsrc_t rsrc;
    int row;      // lane's row for instruction 0: 64 wave_in_group + lane / 4 (instruction j adds 16 j)
    int koff;     // lane's byte in the row: chunk (lane % 4) ^ lds_swz64(row), the same for every j
    int nrows;    // rows present
    int ld;       // row stride in bytes
    int wig;

    // K (bytes per row) is a multiple of 64 for every caller, so a stage
    // never reaches past a row's K bytes and only rows need a range check.
    __device__ __forceinline__ void init(const void* base, int64_t row0, int64_t rows_total, int64_t ld_bytes,
                                         int wave_in_group) {
        wig = wave_in_group;
        const int lane = threadIdx.x & 63;
        row = wig * kInstr * 16 + (lane >> 2);
        koff = ((lane & 3) ^ lds_swz64(row)) * 16;   // lds_swz64(row + 16 j) == lds_swz64(row)
        retarget(base, row0, rows_total, ld_bytes);
    }
    __device__ __forceinline__ void retarget(const void* base, int64_t row0, int64_t rows_total, int64_t ld_bytes) {
        const int64_t avail = rows_total - row0;
        nrows = (int)(avail < 0 ? 0 : (avail < 256 ? avail : 256));   // the descriptor's range: never negative
        ld = (int)ld_bytes;
        rsrc = make_rsrc(static_cast<const char*>(base) + row0 * ld_bytes, (uint32_t)(nrows * ld_bytes));
    }
    // A row at or past nrows starts at or past the descriptor's range, so it
    // loads zeros without a select; the stage's K offset is the scalar offset.
    __device__ __forceinline__ void issue_one(int j, int kt, char* dst) const {
        const int r = row + 16 * j;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(dst + (wig * kInstr + j) * 16 * kRow64), 16,
                                                r * ld + koff, kt * kRow64, 0, 0);
    }
    __device__ __forceinline__ void issue(int kt, char* dst) const {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) issue_one(j, kt, dst);
    }
};

// bf16 activation rows of 128 bytes, then e4m3 weight rows of 64 bytes; the
// weight fragments are expanded to bf16 at the read (exact).
template <int TMW, bool PAT = false>
struct PPLayoutF8 {
    static constexpr int kBOff = 64 * TMW * kRowBytes;
    static constexpr int kStage = 64 * TMW * kRowBytes + 256 * kRow64;
    __device__ __forceinline__ static void read(const char* st, int wm0, int wn0, u32x4 (&fa)[4][TMW],
                                                u32x4 (&fb)[4][2]) {
        const int lane = threadIdx.x & 63;
        const int r = lane & 31, h = lane >> 5;
        const char* Bs = st + kBOff;
        if constexpr (PAT) {
            int pat[4][2];
            pp_patterns(pat);
            // weight rows 32 tn + r (wn0 a multiple of 64): lds_swz64
            // depends on r only, so four per-lane patterns (K group g) cover them
            int pb[4];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                pb[g] = r * kRow64 + ((g ^ lds_swz64(r)) << 4) + 8 * h;
                asm volatile("" : "+v"(pb[g]));
            }
            const char* As = st + wm0 * kRowBytes;
            const char* Bw = Bs + wn0 * kRow64;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int tm = 0; tm < TMW; ++tm)
                    fa[g][tm] = *reinterpret_cast<const u32x4*>(As + tm * 32 * kRowBytes + pat[g][tm & 1]);
#pragma unroll
                for (int tn = 0; tn < 2; ++tn)
                    fb[g][tn] = fp8x8_to_bf16x8(*reinterpret_cast<const u32x2*>(Bw + tn * 32 * kRow64 + pb[g]));
            }
        } else {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
#pragma unroll
                for (int tm = 0; tm < TMW; ++tm)
                    fa[g][tm] = *reinterpret_cast<const u32x4*>(st + lds_byte(wm0 + tm * 32 + r, 2 * g + h));
#pragma unroll
                for (int tn = 0; tn < 2; ++tn)
                    fb[g][tn] = fp8x8_to_bf16x8(
                        *reinterpret_cast<const u32x2*>(Bs + lds_byte64(wn0 + tn * 32 + r, g) + 8 * h));
            }
        }
    }
};

typedef short trmoe_v4s __attribute__((ext_vector_type(4)));

// 8 bytes of a transposing LDS read: lane i of each 16-lane group receives
// element i of the 4 rows addressed by lanes 4j + i/4 (j = 0..3).
__device__ __forceinline__ u32x2 ds_read_tr16(const char* p) {
    const trmoe_v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) trmoe_v4s*)(p));
    return __builtin_bit_cast(u32x2, v);
}

// One token-major operand (K across rows) loaded by one group of 4 waves: a
// stage is 64 K rows of 256 columns (512 bytes), 16-byte chunk c of row k
// stored at chunk c ^ ((k & 3) << 2), so that the transposing fragment reads
// of pp_read_tr hit 64 distinct banks.  A wave instruction fills the two rows
// of a pair (lanes 0..31 the even row, 32..63 the odd one); rows at or past
// the segment's length and columns at or past ncols load zero.
struct PPRowsT {
    static constexpr int kInstr = 8;   // 32 row pairs per stage over 4 waves
    __amdgpu_buffer_rsrc_t rsrc;
    int coloff[2];   // the lane's source column bytes for rows with (row & 2) == 0 / 2
    int h;           // row of the pair this lane fills
    int wig;
    int base, len, ld;

    __device__ __forceinline__ void init(const void* base_ptr, int64_t rows_total, int64_t ld_bytes, int64_t col0,
                                         int64_t ncols, int wave_in_group) {
        rsrc = make_rsrc(base_ptr, (uint32_t)(rows_total * ld_bytes));
        const int lane = threadIdx.x & 63;
        wig = wave_in_group;
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
    }
    // rows [t0, t0 + n) of the operand are the K range (the caller keeps
    // (t0 + n) * ld below 2^31)
    __device__ __forceinline__ void segment(int64_t t0, int n) {
        base = (int)(t0 * (int64_t)ld);
        len = n;
    }
    __device__ __forceinline__ void issue_one(int j, int kt, char* dst) const {
        const int q = wig * kInstr + j;       // row pair of the stage; (q & 1) == (j & 1)
        const int lk = kt * 64 + 2 * q + h;
        const int ro = lk < len ? base + lk * ld : kOutOfRange;
        const int co = coloff[j & 1];         // (row & 3) = 2 (j & 1) + h
        const int o = (ro < 0 || co < 0) ? kOutOfRange : ro + co;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, TRMOE_LDS_PTR(dst + q * 1024), 16, o, 0, 0, 0);
    }
    __device__ __forceinline__ void issue(int kt, char* dst) const {
#pragma unroll
        for (int j = 0; j < kInstr; ++j) issue_one(j, kt, dst);
    }
};

// The wave's fragments of one K stage from two PPRowsT stages ([64][256]
// each): for K group g, lane l needs K values 16 g + 8 (l / 32) + 0..7 of
// column l % 32 of each 32-column block, two transposing reads whose 16
// source lanes address rows +((l & 15) >> 2) and 8-byte column blocks l & 3.
template <int TM>
__device__ __forceinline__ void pp_read_tr(const char* As, const char* Bs, int wm0, int wn0, u32x4 (&fa)[4][TM],
                                           u32x4 (&fb)[4][2]) {
    const int lane = threadIdx.x & 63;
    const int j = (lane & 15) >> 2;
    const int h = lane >> 5;
    const int cw = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
    const int wb = 8 * (lane & 1);
    const int swz = j << 2;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int rowb = (16 * g + 8 * h + 4 * r + j) * 512;
#pragma unroll
            for (int tm = 0; tm < TM; ++tm) {
                const u32x2 v = ds_read_tr16(As + rowb + ((((wm0 + 32 * tm) >> 3) + cw) ^ swz) * 16 + wb);
                fa[g][tm][2 * r] = v[0];
                fa[g][tm][2 * r + 1] = v[1];
            }
#pragma unroll
            for (int tn = 0; tn < 2; ++tn) {
                const u32x2 v = ds_read_tr16(Bs + rowb + ((((wn0 + 32 * tn) >> 3) + cw) ^ swz) * 16 + wb);
                fb[g][tn][2 * r] = v[0];
                fb[g][tn][2 * r + 1] = v[1];
            }
        }
}

struct PPLayoutT {
    static constexpr int kBOff = 64 * 512;
    static constexpr int kStage = 2 * 64 * 512;
    __device__ __forceinline__ static void read(const char* st, int wm0, int wn0, u32x4 (&fa)[4][4],
                                                u32x4 (&fb)[4][2]) {
        pp_read_tr<4>(st, st + kBOff, wm0, wn0, fa, fb);
    }
};

// The ping-pong main loop over nk K stages of two groups' direct loads (A:
// 64 TMW rows by group 1 through ap, B: 256 rows by group 0 through bp) into
// the stages at lds (layout Lay), accumulating each wave's 32 TMW x 64 block
// (rows wm0.., columns wn0..).
// rows_out(acc) writes the calling group's rows of the epilogue tile to LDS:
// group 0 in the phase after its last multiply, while group 1 multiplies the
// last stage, and group 1 after it.  Every wave leaves after a barrier that
// follows both groups' rows_out, so the tile can be read right away.
// Each group raises its waves' priority (s_setprio 1) for its MFMA phase:
// a SIMD holds one wave of each group, and the one feeding the matrix pipe
// then issues ahead of the one reading LDS and issuing loads (C2 layer
// 268 -> 263 us, C5 2141 -> 2123 us; results unchanged).
// e4m3 layouts (kF8Mma) multiply with pp_mma_f8, or with sc's block scales
// (SC::kOn, pp_mma_f8s): each wave loads the scale dwords of stage t + 1
// while it multiplies stage t (group 0 with its B refill, group 1 after the
// phase barrier), and they land by the wait that ends that phase.
//
// NB = 3 (stages that fit three times in LDS: e4m3 weights, 48 KiB): stage
// t lives in buffer t % 3 and each group requests its operand three stages
// ahead, A(t + 3) between group 1's MFMAs of stage t and B(t + 2) after
// group 0's reads of stage t (buffer (t + 2) % 3 held stage t - 1, read by
// both groups before the barrier that opened the phase).  A load then has
// about three phases to land instead of one and a half; each wait leaves the
// newest stage's loads in flight (vmcnt counts in issue order).
template <int TMW, class Lay, int NB = 2, class LA, class LB, class RowsOut, class SC = PPNoScales>
__device__ __forceinline__ void pp_main(const LA& ap, const LB& bp, int nk, char* lds, int group, int wm0, int wn0,
                                        f32x16 (&acc)[TMW][2], RowsOut&& rows_out, const SC& sc = SC{}) {
    constexpr int kStage = Lay::kStage;
    constexpr int kBOff = Lay::kBOff;
    static_assert(NB == 2 || NB == 3, "two or three LDS stages");
    // one scalar buffer offset per stage (kept opaque, so that t % 3 is not
    // strength-reduced into per-fragment vector arithmetic)
    auto buf = [&](int t) -> char* {
        if constexpr (NB == 2)
            return lds + (t & 1) * kStage;
        else
            return lds + __builtin_amdgcn_readfirstlane((t % 3) * kStage);
    };
    char* st0 = lds;
    char* st1 = lds + kStage;
    constexpr int kAI = LA::kInstr, kBI = LB::kInstr;
    constexpr bool kF8 = F8Mma<Lay>::value;
    static_assert(kF8 || !SC::kOn, "block scales are for e4m3 stages");
    static_assert(NB == 2 || !SC::kOn, "block scales take two stages");

    std::conditional_t<kF8, i32x8[2][TMW], u32x4[4][TMW]> fa;
    std::conditional_t<kF8, i32x8[2][2], u32x4[4][2]> fb;
    uint32_t sa[TMW] = {}, sn[TMW] = {};   // block scales of the stage multiplied next / of the one after
    auto mma = [&]() {
        if constexpr (SC::kOn)
            pp_mma_f8s<TMW>(fa, fb, acc, sa);
        else if constexpr (kF8)
            pp_mma_f8<TMW>(fa, fb, acc);
        else
            pp_mma<TMW>(fa, fb, acc);
    };

    // prologue: stages 0 and 1 requested, stage 0 landed everywhere (and
    // the scales of stage 0, requested before them)
    if constexpr (SC::kOn) sc.template load<TMW>(0, sn);
    if constexpr (NB == 3) {
        // stages 0..2 requested, stage 0 landed
        const int pre = nk < 3 ? nk : 3;
        for (int s = 0; s < pre; ++s) {
            if (group == 1)
                ap.issue(s, buf(s));
            else
                bp.issue(s, buf(s) + kBOff);
        }
        if (pre == 3) {
            if (group == 1)
                wait_vmcnt<2 * kAI>();
            else
                wait_vmcnt<2 * kBI>();
        } else if (pre == 2) {
            if (group == 1)
                wait_vmcnt<kAI>();
            else
                wait_vmcnt<kBI>();
        } else {
            wait_vmcnt<0>();
        }
    } else if (group == 1) {
        ap.issue(0, st0);
        if (nk > 1) {
            ap.issue(1, st1);
            wait_vmcnt<kAI>();
        } else {
            wait_vmcnt<0>();
        }
    } else {
        bp.issue(0, st0 + kBOff);
        if (nk > 1) {
            bp.issue(1, st1 + kBOff);
            wait_vmcnt<kBI>();
        } else {
            wait_vmcnt<0>();
        }
    }
    if constexpr (SC::kOn) sc.take(sn, sa);
    pp_barrier();

    if (group == 0) {
        for (int t = 0; t < nk; ++t) {
            const char* st = buf(t);
            Lay::read(st, wm0, wn0, fa, fb);
            wait_lgkmcnt0();
            // B(t+NB-1) goes out after this wave's reads: LDS reads issued
            // behind a wave's own buffer->LDS loads wait for those loads
            __builtin_amdgcn_sched_barrier(0);
            if (t >= 1 && t + NB - 1 < nk) bp.issue(t + NB - 1, buf(t + NB - 1) + kBOff);
            if constexpr (SC::kOn)
                if (t + 1 < nk) sc.template load<TMW>(t + 1, sn);
            pp_barrier();
            __builtin_amdgcn_s_setprio(1);
            mma();
            __builtin_amdgcn_s_setprio(0);
            __builtin_amdgcn_sched_barrier(0);   // B(t+1) is waited for after the MFMAs, not among them
            if constexpr (NB == 3) {
                if (t + 2 < nk)
                    wait_vmcnt<kBI>();   // B(t+2) may stay in flight
                else
                    wait_vmcnt<0>();
            } else {
                wait_vmcnt<0>();
            }
            if constexpr (SC::kOn) sc.take(sn, sa);
            pp_barrier();
        }
        // phase 2nk: group 1 multiplies the last stage, group 0 writes its
        // rows of the epilogue tile (every stage has been read)
        rows_out(acc);
        wait_lgkmcnt0();
        pp_barrier();
        pp_barrier();   // phase 2nk+1: group 1's rows
    } else {
        pp_barrier();   // phase 0: group 0 reads stage 0
        // iteration t: read stage t; multiply it, refilling its buffer with
        // A(t+2) while t + 2 < nk (two loops rather than a branch around the
        // MFMAs, which would give each branch its own accumulator registers)
        auto step = [&](int t, auto load) {
            const char* st = buf(t);
            Lay::read(st, wm0, wn0, fa, fb);
            wait_lgkmcnt0();
            // A(t+1), issued at the start of the previous phase (NB = 3: two
            // phases earlier, A(t+2) staying in flight), has landed
            if constexpr (NB == 3) {
                if (t + 2 < nk)
                    wait_vmcnt<kAI>();
                else
                    wait_vmcnt<0>();
            } else {
                wait_vmcnt<0>();
            }
            if constexpr (SC::kOn)
                if (t >= 1) sc.take(sn, sa);   // stage t's scales, requested in the previous phase
            pp_barrier();
            if constexpr (SC::kOn)
                if (t + 1 < nk) sc.template load<TMW>(t + 1, sn);
            // Both groups are done with stage t only now: the other waves of
            // this group read it in the phase that just ended, so A(t+2)
            // cannot be issued into it before this barrier.
            __builtin_amdgcn_s_setprio(1);
            if constexpr (decltype(load)::value) {
                if constexpr (SC::kOn)
                    pp_mma_load_f8s<TMW>(fa, fb, acc, sa, ap, t + 2, (t & 1) ? st1 : st0);
                else if constexpr (kF8)
                    pp_mma_load_f8<TMW>(fa, fb, acc, ap, t + NB, buf(t));
                else
                    pp_mma_load<TMW>(fa, fb, acc, ap, t + NB, buf(t));
            } else {
                mma();
            }
            __builtin_amdgcn_s_setprio(0);
            pp_barrier();
        };
        int t = 0;
        for (; t + NB < nk; ++t) step(t, BoolC<true>{});
        for (; t < nk; ++t) step(t, BoolC<false>{});
        rows_out(acc);
        wait_lgkmcnt0();
        pp_barrier();
    }
}

// Accumulators set to a zero that is redefined at each use, so that no
// zero block is hoisted out of a caller's loop.
template <int TM, int TN>
__device__ __forceinline__ void zero_acc_opaque(f32x16 (&acc)[TM][TN]) {
    float z = 0.0f;
    asm volatile("" : "+v"(z));
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[tm][tn][i] = z;
}

// Stores of one 32x32 accumulator block held as bf16 pairs: lane l owns
// column c = l % 32 and rows acc_row(l, i); rows i, i + 1 (i even) are
// consecutive, so adjacent lanes swap one value (DPP quad_perm 1,0,3,2) and
// each lane writes 4 bytes: the even lane columns c, c + 1 of row i, the odd
// lane columns c - 1, c of row i + 1.  v[i] is the value of row i; `lb` the
// lane's byte offset of its pair (its row for i = 0, plus 1 for odd lanes,
// times the row stride, plus 2 (c & ~1)); rows advance by ld2 bytes.
// Offsets at or past the buffer's range are dropped.  POLICY is the buffer
// store's cache-policy operand: 0, or kStoreStream (the nt bit, a
// non-temporal hint) for outputs that no kernel reads soon.
constexpr int kStoreStream = 2;

__device__ __forceinline__ float dpp_swap_pairs(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
}

__device__ __forceinline__ int pair_lane_offset(int row0, int col, int ld2) {
    const int lane = threadIdx.x & 63;
    return (row0 + 4 * (lane >> 5) + (lane & 1)) * ld2 + (col & ~1) * 2;
}

template <int POLICY = 0>
__device__ __forceinline__ void store_bf16_pairs(__amdgpu_buffer_rsrc_t rsrc, int lb, int ld2, const float (&v)[16]) {
    const bool odd = threadIdx.x & 1;
#pragma unroll
    for (int p = 0; p < 8; ++p) {
        const float v0 = v[2 * p], v1 = v[2 * p + 1];
        const float other = dpp_swap_pairs(odd ? v0 : v1);
        const bf16x2 pr = odd ? bf16x2{(bf16_t)other, (bf16_t)v1} : bf16x2{(bf16_t)v0, (bf16_t)other};
        const int off = lb + (8 * (p >> 1) + 2 * (p & 1)) * ld2;   // row acc_row(lane, 2 p) - acc_row(lane, 0)
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, pr), rsrc, off, 0, POLICY);
    }
}

// Tile i of a persistent launch over tiles_m x tiles_n tiles -> (row tile,
// column tile).  Workgroups are dispatched to the 8 XCDs round-robin, so tile
// i runs on XCD i % 8.  With xcd_rows, XCD x owns the row tiles
// [x mpx, x mpx + mpx), mpx = tiles_m / 8, in groups of bm (4 when mpx
// allows), so that the 32 workgroups of an XCD that run together hold
// bm row panels x 32 / bm column panels (4 x 8), which read each K slice of
// 12 panels per round instead of 18 for 16 x 2.  The column tiles are walked
// in bands of 32 / bm; within a band the row groups alternate fastest, so
// consecutive rounds of an XCD keep their weight panels and change only the
// activation panels (C2 gate|up: 178 -> 175 us).  Other shapes walk row
// tiles first.
__device__ __forceinline__ void pps_tile(uint32_t i, uint32_t tiles_m, uint32_t tiles_n, bool xcd_rows,
                                         uint32_t& mt, uint32_t& nt) {
    if (xcd_rows) {
        const uint32_t mpx = tiles_m >> 3, j = i >> 3;
        const uint32_t bm = (mpx & 3) == 0 ? 4 : ((mpx & 1) == 0 ? 2 : 1);
        const uint32_t ng = mpx / bm, cb = 32 / bm;
        const uint32_t rest = j / bm;                          // (row group, column) pair in walk order
        const uint32_t band = rest / (cb * ng), in = rest - band * cb * ng;
        const uint32_t wb = tiles_n - band * cb < cb ? tiles_n - band * cb : cb;   // the last band may be narrower
        const uint32_t mg = in / wb;
        nt = band * cb + (in - mg * wb);
        mt = (i & 7) * mpx + mg * bm + (j - rest * bm);
    } else {
        nt = i / tiles_m;
        mt = i - nt * tiles_m;
    }
}

// Persistent form of pp_main.  The workgroup's ntiles tiles (nk K stages
// each) run as one stream of stages s = nk * i + kt through the same two LDS
// buffers, phase schedule and refill rules, so the next tile's first stages
// are requested while the current one is still being multiplied and no
// barrier-bound prologue or LDS-staged epilogue sits between tiles.  Each
// group writes a finished tile straight from its accumulators (epi(i, acc),
// global stores only, no LDS) at the start of its read phase of the next
// tile's first stage, before the reads, while the other group multiplies;
// the last tile's epilogue runs as in pp_main.  retarget_a(i) / retarget_b(i)
// point the A / B loader at tile i, each called by the group that issues
// that operand before its first load of tile i (the caller has pointed both
// at tile 0); for i == ntiles the loader must load nothing (zeros): group 1
// issues its refills unconditionally, so the last two stages request two
// stages past the end into buffers nobody reads again.  TR (e4m3 stages):
// transposed accumulator blocks (pp_mma_f8<TM, true>).  The MFMA phases run
// at raised wave priority, as in pp_main.
template <int TMW, class Lay, bool TR = false, class LA, class LB, class RA, class RB, class Epi>
__device__ __forceinline__ void pp_stream(LA& ap, LB& bp, int nk, int ntiles, char* lds, int group, int wm0,
                                          int wn0, f32x16 (&acc)[TMW][2], RA&& retarget_a, RB&& retarget_b,
                                          Epi&& epi) {
    constexpr int kStage = Lay::kStage;
    constexpr int kBOff = Lay::kBOff;
    char* st0 = lds;
    char* st1 = lds + kStage;
    constexpr int kAI = LA::kInstr, kBI = LB::kInstr;
    const int S = nk * ntiles;

    // fragments of one stage: 16-byte chunks per K group, or 32-byte e4m3
    // operands per K step
    constexpr bool kF8 = F8Mma<Lay>::value;
    std::conditional_t<kF8, i32x8[2][TMW], u32x4[4][TMW]> fa;
    std::conditional_t<kF8, i32x8[2][2], u32x4[4][2]> fb;

    // The issuing group's next load: stage `ld_kt` of tile `ld_tile`,
    // advanced by counting (no division in the loop); the loader is pointed
    // at a new tile when the count wraps.
    int ld_kt = 0, ld_tile = 0;
    auto advance = [&](auto&& retarget) {
        if (++ld_kt == nk) {
            ld_kt = 0;
            retarget(++ld_tile);
        }
    };

    // prologue: stages 0 and 1 requested, stage 0 landed everywhere
    if (group == 1) {
        ap.issue(0, st0);
        advance(retarget_a);
        ap.issue(ld_kt, st1);
        advance(retarget_a);   // next: stage 2
        wait_vmcnt<kAI>();
    } else {
        bp.issue(0, st0 + kBOff);
        if (S > 1) {
            advance(retarget_b);
            bp.issue(ld_kt, st1 + kBOff);
            wait_vmcnt<kBI>();
        } else {
            wait_vmcnt<0>();
        }
        advance(retarget_b);   // next: stage 2
    }
    pp_barrier();

    if (group == 0) {
        int s = 0;
        for (int i = 0; i < ntiles; ++i) {
            if (i > 0) {
                // the previous tile's epilogue, before this stage's reads (its
                // accumulators and the fragments are never live together),
                // while group 1 multiplies that tile's last stage
                epi(i - 1, acc);
                zero_acc_opaque(acc);
                __builtin_amdgcn_sched_barrier(0);
            }
            for (int kt = 0; kt < nk; ++kt, ++s) {
                const char* st = (s & 1) ? st1 : st0;
                Lay::read(st, wm0, wn0, fa, fb);
                wait_lgkmcnt0();
                // B(s+1) goes out after this wave's reads: LDS reads issued
                // behind a wave's own buffer->LDS loads wait for those loads
                __builtin_amdgcn_sched_barrier(0);
                if (s >= 1 && s + 1 < S) {
                    bp.issue(ld_kt, ((s + 1) & 1 ? st1 : st0) + kBOff);
                    advance(retarget_b);
                }
                pp_barrier();
                __builtin_amdgcn_s_setprio(1);
                if constexpr (kF8)
                    pp_mma_f8<TMW, TR>(fa, fb, acc);
                else
                    pp_mma<TMW>(fa, fb, acc);
                __builtin_amdgcn_s_setprio(0);
                __builtin_amdgcn_sched_barrier(0);   // B(s+1) and the epilogue's stores waited for after the MFMAs
                wait_vmcnt<0>();
                pp_barrier();
            }
        }
        // phase 2S: group 1 multiplies the last stage, group 0 writes its rows
        epi(ntiles - 1, acc);
        pp_barrier();
        pp_barrier();   // phase 2S+1: group 1's rows
    } else {
        pp_barrier();   // phase 0: group 0 reads stage 0
        int s = 0;
        for (int i = 0; i < ntiles; ++i) {
            if (i > 0) {   // group 0 multiplies this tile's first stage
                epi(i - 1, acc);
                zero_acc_opaque(acc);
                __builtin_amdgcn_sched_barrier(0);
            }
            // stage s: read it; multiply it, refilling its buffer with A(s+2)
            for (int kt = 0; kt < nk; ++kt, ++s) {
                const char* st = (s & 1) ? st1 : st0;
                Lay::read(st, wm0, wn0, fa, fb);
                wait_lgkmcnt0();
                wait_vmcnt<0>();   // A(s+1), issued in the previous phase, has landed (and the epilogue's stores)
                const int kt2 = ld_kt;
                pp_barrier();
                __builtin_amdgcn_s_setprio(1);
                if constexpr (kF8)
                    pp_mma_load_f8<TMW, LA, TR>(fa, fb, acc, ap, kt2, (s & 1) ? st1 : st0);
                else
                    pp_mma_load<TMW>(fa, fb, acc, ap, kt2, (s & 1) ? st1 : st0);
                __builtin_amdgcn_s_setprio(0);
                __builtin_amdgcn_sched_barrier(0);
                advance(retarget_a);   // the loader's registers are read at issue, so it may move now
                pp_barrier();
            }
        }
        epi(ntiles - 1, acc);
        wait_vmcnt<0>();   // the two loads past the end land before the workgroup's LDS is released
        pp_barrier();
    }
}

}  // namespace trmoe
