// Decode-shape (few tokens) variants of K2 and K4.
//
// With M <= 128 tokens the layer is weight-streaming: every weight byte is
// used M times, far below the MFMA/HBM balance point (~300 FLOP/B for bf16),
// so the kernels are organised to keep as many weight loads in flight as the
// CUs allow and to touch each weight byte once:
//
//   k_gate_up_skinny   one workgroup per 16 output features (16 gate + 16 up
//                      packed rows) and all M tokens; the waves split K, copy
//                      their K spans of the operands into LDS with direct
//                      loads (staged_k_loop), and reduce through LDS before
//                      the SwiGLU epilogue (same epilogue contract as
//                      k_gate_up_swiglu, including the dense-routed scaling)
//   k_down_skinny      split-K: workgroup (8, 16 or 32 output columns, K chunk)
//                      writes an fp32 partial [split][M][N] to the caller's
//                      workspace
//   k_down_reduce      sums the partials in split order (deterministic),
//                      applies the row scales, the routed un-permute and the
//                      residual, and stores the output
#include "trmoe_common.h"
#include "trmoe_internal.h"
#include "trmoe_gemm.h"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>

namespace trmoe {

namespace {

// 16x16 MFMA tiles: a K group is 64 bytes of an activation row; lane l
// supplies row l & 15 and the 16-byte chunk l >> 4 of the group (one
// instruction touches 16 rows x 64 contiguous bytes of each operand).
// Output element i of lane l is row 4 * (l >> 4) + i, column l & 15.
__device__ __forceinline__ void mfma16(KindBF16, u32x4 a, u32x4 b, f32x4& acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                  0, 0, 0);
}
__device__ __forceinline__ void mfma16(KindF32, u32x4 a, u32x4 b, f32x4& acc) {
    const f32x4 fa = __builtin_bit_cast(f32x4, a);
    const f32x4 fb = __builtin_bit_cast(f32x4, b);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[i], fb[i], acc, 0, 0, 0);
}

// Weight fragment of one K group for the lane's row: 16 bytes of bf16/f32,
// or 8 bytes of e4m3 (half as many bytes as the activation group) expanded
// to bf16.
template <class Kind, bool FP8>
struct WFrag {
    using Reg = u32x4;
    static __device__ __forceinline__ Reg load(__amdgpu_buffer_rsrc_t r, int row_off, int g, int q, int kb_a) {
        const int o = 64 * g + 16 * q;
        return buffer_load16(r, o < kb_a ? row_off + o : kOutOfRange);
    }
    static __device__ __forceinline__ u32x4 expand(Reg v) { return v; }
};
template <class Kind>
struct WFrag<Kind, true> {
    using Reg = u32x2;
    static __device__ __forceinline__ Reg load(__amdgpu_buffer_rsrc_t r, int row_off, int g, int q, int kb_a) {
        return buffer_load8(r, 64 * g + 16 * q < kb_a ? row_off + 32 * g + 8 * q : kOutOfRange);
    }
    static __device__ __forceinline__ u32x4 expand(Reg v) { return fp8x8_to_bf16x8(v); }
};

// One direct buffer -> LDS load of 16 bytes per lane (lane l's bytes land at
// lds + 16 l).  A plain function: the host pass of hipcc rejects a second
// use of a function template specialization that calls the builtin itself.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* lds, int off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, TRMOE_LDS_PTR(lds), 16, off, 0, 0, 0);
}

// The K loop of the decode kernels, operands staged through LDS.  The
// accumulators are 16x16x32 MFMA tiles: acc[tm][u] += A(rows tm*16..+15) .
// W(rows of block u)^T.  A 16x16x32 operand load straight into registers
// takes 16 rows x 64 bytes, so each instruction touches 16 cache lines
// in every 16-lane quarter, and that -- not bytes -- is what limits the
// loop (the activations are read by every workgroup).  Here each wave
// copies its own K spans (128 bytes) of all MT*16 activation rows, and with
// SW also of its 16*NU weight rows, into its LDS region with direct loads
// (8 rows x 128 bytes per instruction, lds_byte() layout) and reads the MFMA
// fragments back from LDS; without SW the weight fragments come straight
// into registers (16 rows x 64 bytes per instruction).  Weight block u is the 16 rows from
// row w_row0[u] of the weight descriptor (whose byte offsets, with SW off,
// are w_off[u] for the lane's row); with BR = 8 only its first 8 rows are
// staged and the other 8 output columns of the block are to be ignored.
// FRAG (with SW off): the descriptor is a fragment-major copy whose block 0
// is row 0, and weight fragments are 1 KiB contiguous loads.  Spans [s0, s1) in batches of SB;
// `region` holds SB * (MT + (SW ? NU : 0)) * 16 rows of 128 bytes.
// Sum of squares of the activation elements in one 16-byte chunk.
__device__ __forceinline__ float chunk_sumsq(KindBF16, u32x4 v) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float lo = __builtin_bit_cast(float, v[j] << 16);
        const float hi = __builtin_bit_cast(float, v[j] & 0xffff0000u);
        s += lo * lo;
        s += hi * hi;
    }
    return s;
}
__device__ __forceinline__ float chunk_sumsq(KindF32, u32x4 v) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float f = __builtin_bit_cast(float, (uint32_t)v[j]);
        s += f * f;
    }
    return s;
}

template <int MT>
constexpr int ssq_rows() { return (MT * 16 + 63) / 64; }

template <class Kind, bool FP8, int MT, int NU, int SB, bool SW, int BR = 16, bool FRAG = false>
__device__ __forceinline__ void staged_k_loop(__amdgpu_buffer_rsrc_t ar, int a_rows, int lda_b, char* region,
                                              __amdgpu_buffer_rsrc_t wr, const int (&w_row0)[NU], int ldw_b,
                                              const int (&w_off)[NU], int s0, int s1, int kb_a,
                                              f32x4 (&acc)[MT][NU], bool ssq_on = false,
                                              float* ssq = nullptr, int w_half = -1) {
    static_assert(!(SW && FP8), "e4m3 weight rows are 64 bytes per span: not staged");
    using WF = WFrag<Kind, FP8>;
    constexpr int kRowsA = MT * 16;
    constexpr int kRows = kRowsA + (SW ? NU * 16 : 0);
    const int lane = threadIdx.x & 63;
    const int q = lane >> 4;
    // fragment-major weights, w_half >= 0: the tile uses rows 8 w_half ..
    // 8 w_half + 7 of each 16-row block, so the lanes holding the other half
    // (row lane % 16) load nothing (zeros: their products are never stored)
    const bool w_live = w_half < 0 || ((lane & 15) >> 3) == w_half;
    int xo[MT * 2];   // the lane's row offset + chunk for each 8-row copy instruction
#pragma unroll
    for (int j = 0; j < MT * 2; ++j) {
        const int row = j * 8 + (lane >> 3);
        xo[j] = row < a_rows ? row * lda_b + 16 * ((lane & 7) ^ lds_swz(row)) : kOutOfRange;
    }
    static_assert(BR == 8 || BR == 16, "weight blocks of 8 or 16 rows");
    constexpr int kWI = BR / 8;   // copy instructions per weight block
    int wo[SW ? NU * kWI : 1];
    if constexpr (SW) {
#pragma unroll
        for (int j = 0; j < NU * kWI; ++j) {
            const int lr = (j / kWI) * 16 + (j % kWI) * 8 + (lane >> 3);   // row within the staged weight rows
            wo[j] = (w_row0[j / kWI] + (j % kWI) * 8 + (lane >> 3)) * ldw_b + 16 * ((lane & 7) ^ lds_swz(kRowsA + lr));
        }
    }
    for (int sb = s0; sb < s1; sb += SB) {
        typename WF::Reg wv[SW ? 1 : SB][2][NU];
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const int sp = sb + j;
            if (sp < s1) {
                char* st = region + j * kRows * kRowBytes;
#pragma unroll
                for (int i = 0; i < MT * 2; ++i) {
                    const int o = 128 * sp + 16 * ((lane & 7) ^ lds_swz(i * 8 + (lane >> 3)));
                    dma16(ar, st + i * 8 * kRowBytes, o < kb_a ? xo[i] + 128 * sp : kOutOfRange);
                }
                if constexpr (SW) {
#pragma unroll
                    for (int i = 0; i < NU * kWI; ++i) {
                        const int r0 = kRowsA + (i / kWI) * 16 + (i % kWI) * 8;   // first LDS row of the copy
                        const int o = 128 * sp + 16 * ((lane & 7) ^ lds_swz(r0 + (lane >> 3)));
                        dma16(wr, st + r0 * kRowBytes, o < kb_a ? wo[i] + 128 * sp : kOutOfRange);
                    }
                } else {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
#pragma unroll
                        for (int u = 0; u < NU; ++u) {
                            const int gg = 2 * sp + h;
                            if constexpr (FRAG) {
                                // fragment-major weights: block w_row0[u] / 16, group gg is
                                // 1 KiB, and lane l's 16 bytes sit at 16 l
                                const int G = (kb_a + 63) / 64;
                                wv[j][h][u] = buffer_load16(
                                    wr, (64 * gg < kb_a && w_live) ? ((w_row0[u] >> 4) * G + gg) * 1024 + 16 * lane
                                                                   : kOutOfRange);
                            } else {
                                wv[j][h][u] = WF::load(wr, w_off[u], gg, q, kb_a);
                            }
                        }
                }
            }
        }
        wait_vmcnt<0>();
        asm volatile("" ::: "memory");
        if (ssq_on) {
            // fused RMSNorm: the lane's activation rows (lane, lane + 64) summed
            // over this batch's spans, straight from the staged copies
#pragma unroll
            for (int j = 0; j < SB; ++j) {
                if (sb + j < s1) {
                    const char* st = region + j * kRows * kRowBytes;
#pragma unroll
                    for (int rr = 0; rr < ssq_rows<MT>(); ++rr) {
                        const int row = lane + 64 * rr;
                        if (row < kRowsA) {
#pragma unroll
                            for (int c = 0; c < 8; ++c)
                                ssq[rr] += chunk_sumsq(Kind{}, *reinterpret_cast<const u32x4*>(st + lds_byte(row, c)));
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            if (sb + j < s1) {
                const char* st = region + j * kRows * kRowBytes;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    u32x4 av[MT];
#pragma unroll
                    for (int tm = 0; tm < MT; ++tm)
                        av[tm] = *reinterpret_cast<const u32x4*>(st + lds_byte(tm * 16 + (lane & 15), 4 * h + q));
#pragma unroll
                    for (int u = 0; u < NU; ++u) {
                        u32x4 b;
                        if constexpr (SW)
                            b = *reinterpret_cast<const u32x4*>(st + lds_byte(kRowsA + u * 16 + (lane & 15), 4 * h + q));
                        else
                            b = WF::expand(wv[j][h][u]);
#pragma unroll
                        for (int tm = 0; tm < MT; ++tm) mfma16(Kind{}, av[tm], b, acc[tm][u]);
                    }
                }
            }
        }
        // this wave's LDS reads of the batch are consumed before the next
        // batch's copies are issued
        wait_lgkmcnt0();
        asm volatile("" ::: "memory");
    }
}

// red[wave][e][lane] with e = (tm*NU+u)*4+i.
template <int MT, int NU>
__device__ __forceinline__ void skinny_stash(float* red, const f32x4 (&acc)[MT][NU]) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int tm = 0; tm < MT; ++tm)
#pragma unroll
        for (int u = 0; u < NU; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) red[((wave * MT * NU + tm * NU + u) * 4 + i) * 64 + lane] = acc[tm][u][i];
}

template <int MT, int NU, int NW>
__device__ __forceinline__ float skinny_sum(const float* red, int tm, int u, int i, int lane) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) s += red[((w * MT * NU + tm * NU + u) * 4 + i) * 64 + lane];
    return s;
}

template <int MT, int NU>
__device__ __forceinline__ void zero_acc16(f32x4 (&acc)[MT][NU]) {
#pragma unroll
    for (int tm = 0; tm < MT; ++tm)
#pragma unroll
        for (int u = 0; u < NU; ++u) acc[tm][u] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// The down epilogue for one output element: row scale, shared scale, the
// route-weighted y rows of the token, the residual.
template <class T>
__device__ __forceinline__ void down_finish(const DownArgs& a, int64_t row, int64_t col, float s) {
    float v = s * a.shared_scale * (a.w_scale ? a.w_scale[col] : 1.0f);
    if (a.y != nullptr) {
        const T* y = static_cast<const T*>(a.y);
        const int64_t last = (int64_t)a.top_k * a.M - 1;
        float racc = 0.f;
        for (int j = 0; j < a.top_k; ++j) {
            int64_t yr = a.inverse[(int64_t)j * a.M + row];
            yr = yr < 0 ? 0 : (yr > last ? last : yr);
            racc += a.rw[j] * to_f32(y[yr * a.ldy + col]);
        }
        v += a.routed_scale * racc;
    }
    if (a.residual != nullptr) v += to_f32(static_cast<const T*>(a.residual)[row * a.ldr + col]);
    static_cast<T*>(a.out)[row * a.ldo + col] = from_f32<T>(v);
}

}  // namespace

// One workgroup per 16 output features (32 packed rows: 16 gate rows and the
// matching 16 up rows of a 64-row packed group) and all M tokens.
// Spans (128 bytes of K) per batch of staged_k_loop with ROWS staged rows
// per span: as many as fit 144 KiB of LDS over the workgroup's waves, at
// most 8.  Weights are staged too (SW) when both operands fit two spans.
template <int ROWS, int NW>
constexpr int staged_batch() {
    constexpr int per = 147456 / (NW * ROWS * kRowBytes);
    return per < 1 ? 1 : (per > 8 ? 8 : per);
}
template <int ROWS, int NW>
constexpr int staged_lds_bytes() { return NW * staged_batch<ROWS, NW>() * ROWS * kRowBytes; }
template <bool FP8, int MT, int NU, int NW>
constexpr bool stage_weights() { return !FP8 && staged_batch<(MT + NU) * 16, NW>() >= 2; }
template <bool FP8, int MT, int NU, int NW>
constexpr int staged_rows() { return (MT + (stage_weights<FP8, MT, NU, NW>() ? NU : 0)) * 16; }
template <int MT, int NW>
constexpr int rms_slots() { return NW * MT * 16; }

template <class Kind, bool FP8, int MT, int NW, bool FRAG = false>
__global__ __launch_bounds__(64 * NW) void k_gate_up_skinny(GateUpArgs a) {
    using T = typename Kind::T;
    constexpr int NT = 64 * NW;
    constexpr int kWB = FP8 ? 1 : (int)sizeof(T);
    extern __shared__ __align__(16) float red[];
    __shared__ int s_route[MT * 16][kMaxTopK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int64_t f0 = (int64_t)blockIdx.x * 16;                   // first output feature
    const int64_t pg = (f0 >> 5) * 64 + (f0 & 31);                 // its gate row in the packed weight
    // descriptors first: built ahead of the divergent route gather they stay
    // in scalar registers
    const int kb_a = a.K * (int)sizeof(T);
    const auto ar = make_rsrc(a.x, (uint32_t)(a.M * a.ldx * (int64_t)sizeof(T)));
    // fragment-major weights: the 16-row blocks pg / 16 .. + 2 (gate, -, up)
    const int frag_g = (kb_a + 63) / 64;
    const auto wr = FRAG ? make_rsrc(static_cast<const char*>(a.w_frag) + (pg >> 4) * (int64_t)frag_g * 1024,
                                     (uint32_t)(3 * frag_g * 1024))
                         : make_rsrc(static_cast<const char*>(a.w) + pg * a.ldw * kWB, (uint32_t)(48 * a.ldw * kWB));

    const bool routed = a.ids != nullptr && f0 >= a.shared_feats;
    // the route gather (two dependent loads) runs on the last waves, which
    // have the fewest K spans
    if (routed && threadIdx.x >= NT - MT * 16) {
        const int64_t row = threadIdx.x - (NT - MT * 16);
        int64_t id = row < a.M ? a.ids[row] : 0;
        id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
        for (int j = 0; j < kMaxTopK; ++j)
            s_route[row][j] = (j < a.top_k && row < a.M) ? (int)a.table[(int64_t)j * a.vocab + id] : -1;
    }
    int w_off[2];
    w_off[0] = (int)(r * a.ldw * kWB);          // gate row pg + r
    w_off[1] = (int)((32 + r) * a.ldw * kWB);   // up row pg + 32 + r

    constexpr bool SW = !FRAG && stage_weights<FP8, MT, 2, NW>();
    constexpr int kRows = (MT + (SW ? 2 : 0)) * 16;
    constexpr int SB = staged_batch<kRows, NW>();
    const int w_row0[2] = {0, 32};
    const int spans = (kb_a + 127) / 128;
    const int per_wave = (spans + NW - 1) / NW;
    const int s0 = wave * per_wave;
    const int s1 = s0 + per_wave < spans ? s0 + per_wave : spans;
    f32x4 acc[MT][2];
    zero_acc16<MT, 2>(acc);
    char* region = reinterpret_cast<char*>(red) + wave * SB * kRows * kRowBytes;
    // fused RMSNorm: per-token scales given (row_scale) or computed here from
    // the staged activations (the sum over the waves' K spans)
    const bool rms_in = a.row_scale == nullptr && a.rms_eps > 0.0f;
    const bool rms = rms_in || a.row_scale != nullptr;
    float ssq[ssq_rows<MT>()] = {};
    staged_k_loop<Kind, FP8, MT, 2, SB, SW, 16, FRAG>(ar, (int)a.M, (int)(a.ldx * (int64_t)sizeof(T)), region, wr,
                                                      w_row0, (int)(a.ldw * kWB), w_off, s0, s1, kb_a, acc, rms_in,
                                                      ssq);
    __shared__ float s_ssq[rms_slots<MT, NW>()];
    __shared__ float s_rs[MT * 16];
    if (rms_in) {
#pragma unroll
        for (int rr = 0; rr < ssq_rows<MT>(); ++rr) {
            const int row = (threadIdx.x & 63) + 64 * rr;
            if (row < MT * 16) s_ssq[wave * MT * 16 + row] = ssq[rr];
        }
    }
    __syncthreads();   // every wave is done with its staging region
    if (rms && threadIdx.x < MT * 16) {
        float rs;
        if (rms_in) {
            float t = 0.f;
            for (int w = 0; w < NW; ++w) t += s_ssq[w * MT * 16 + threadIdx.x];
            rs = rsqrtf(t / (float)a.K + a.rms_eps);
        } else {
            rs = (int64_t)threadIdx.x < a.M ? a.row_scale[threadIdx.x] : 0.0f;
        }
        s_rs[threadIdx.x] = rs;
    }
    skinny_stash<MT, 2>(red, acc);
    __syncthreads();

    const int64_t expert = routed ? (f0 - a.shared_feats) / a.expert_feats : -1;
    const float mult = routed ? 1.0f : a.shared_mult;
    T* h = static_cast<T*>(a.h);
    for (int qi = threadIdx.x; qi < MT * 4 * 64; qi += NT) {
        const int l = qi & 63, i = (qi >> 6) & 3, tm = qi >> 8;
        const int row = tm * 16 + 4 * (l >> 4) + i;
        if (row >= a.M) continue;
        const int fl = l & 15;
        const float sg = a.w_scale ? a.w_scale[pg + fl] : 1.0f;
        const float su = a.w_scale ? a.w_scale[pg + 32 + fl] : 1.0f;
        const float rs = rms ? s_rs[row] : 1.0f;
        const float g = skinny_sum<MT, 2, NW>(red, tm, 0, i, l) * sg * rs;
        const float u = skinny_sum<MT, 2, NW>(red, tm, 1, i, l) * su * rs;
        float hv = silu_f(g) * u * mult;
        if (routed) {
            float tw = 0.f;
#pragma unroll
            for (int j = 0; j < kMaxTopK; ++j) tw += (s_route[row][j] == expert) ? a.rw[j] : 0.f;
            hv *= tw;
        }
        h[row * a.ldh + f0 + fl] = from_f32<T>(hv);
    }
}

// Workgroup L of the down's 1-D grid -> (column tile, K split).  Workgroups
// go to the 8 XCDs round-robin; with 2, 4 or 8 splits (and whole rounds)
// XCD x takes split x % S only, so each XCD's L2 fetches one K range of h
// instead of all of it.
__device__ __forceinline__ void down_tile_split(int L, int ncol, int S, int& ct, int& sp) {
    if (S > 1 && 8 % S == 0 && (ncol * S) % 8 == 0 && ncol % (8 / S) == 0) {
        const int x = L & 7, j = L >> 3;
        sp = x % S;
        ct = j * (8 / S) + x / S;
    } else {
        ct = L % ncol;
        sp = L / ncol;
    }
}

// Split-K partial of the down GEMM: block (COLS-column tile, K split) writes
// part[(split * M + row) * N + col] for its rows and columns; with a single
// split it finishes the output itself.  COLS = 8 uses half of a 16-row
// weight block (twice the workgroups for the same columns).
template <class Kind, bool FP8, int MT, int COLS, int NW, bool FRAG = false>
__global__ __launch_bounds__(64 * NW) void k_down_skinny(DownArgs a, float* part, int spans_per_split, int ncol,
                                                        int splits) {
    using T = typename Kind::T;
    constexpr int NT = 64 * NW;
    constexpr int kWB = FP8 ? 1 : (int)sizeof(T);
    constexpr int NU = (COLS + 15) / 16;
    constexpr int kCols = COLS;
    extern __shared__ __align__(16) float red[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15;
    int ct, split;
    down_tile_split((int)blockIdx.x, ncol, splits, ct, split);
    const int64_t n0 = (int64_t)ct * kCols;

    const int kb_a = a.K * (int)sizeof(T);
    const auto ar = make_rsrc(a.h, (uint32_t)(a.M * a.ldh * (int64_t)sizeof(T)));
    // fragment-major weights start at the 16-row block holding n0; an 8-column
    // tile at n0 % 16 == 8 uses lanes 8..15 of its block
    const int frag_g = (kb_a + 63) / 64;
    const int64_t cbase = FRAG ? (n0 & ~(int64_t)15) : n0;
    const auto wr = FRAG ? make_rsrc(static_cast<const char*>(a.w_frag) + (cbase >> 4) * (int64_t)frag_g * 1024,
                                     (uint32_t)(NU * frag_g * 1024))
                         : make_rsrc(static_cast<const char*>(a.w) + n0 * a.ldw * kWB, (uint32_t)(kCols * a.ldw * kWB));
    int w_off[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) w_off[u] = (int)((u * 16 + r) * a.ldw * kWB);

    constexpr bool SW = !FRAG && stage_weights<FP8, MT, NU, NW>();
    constexpr int kRows = (MT + (SW ? NU : 0)) * 16;
    constexpr int SB = staged_batch<kRows, NW>();
    int w_row0[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) w_row0[u] = u * 16;
    const int spans = (kb_a + 127) / 128;
    const int p0 = split * spans_per_split;
    const int p1 = p0 + spans_per_split < spans ? p0 + spans_per_split : spans;
    const int per_wave = (p1 - p0 + NW - 1) / NW;
    const int s0 = p0 + wave * per_wave;
    const int s1 = s0 + per_wave < p1 ? s0 + per_wave : p1;
    f32x4 acc[MT][NU];
    zero_acc16<MT, NU>(acc);
    char* region = reinterpret_cast<char*>(red) + wave * SB * kRows * kRowBytes;
    staged_k_loop<Kind, FP8, MT, NU, SB, SW, (COLS < 16 ? 8 : 16), FRAG>(
        ar, (int)a.M, (int)(a.ldh * (int64_t)sizeof(T)), region, wr, w_row0, (int)(a.ldw * kWB), w_off, s0, s1, kb_a,
        acc, false, nullptr, (FRAG && COLS < 16) ? (int)((n0 >> 3) & 1) : -1);
    __syncthreads();   // every wave is done with its staging region
    skinny_stash<MT, NU>(red, acc);
    __syncthreads();

    const bool single = splits == 1;
    float* dst = part + (int64_t)split * a.M * a.N;
    for (int qi = threadIdx.x; qi < MT * NU * 4 * 64; qi += NT) {
        const int l = qi & 63, i = (qi >> 6) & 3, u = (qi >> 8) % NU, tm = (qi >> 8) / NU;
        const int row = tm * 16 + 4 * (l >> 4) + i;
        const int64_t col = cbase + u * 16 + (l & 15);
        if (row >= a.M || col < n0 || col >= n0 + kCols || col >= a.N) continue;
        const float v = skinny_sum<MT, NU, NW>(red, tm, u, i, l);
        if (single)
            down_finish<T>(a, row, col, v);
        else
            dst[row * (int64_t)a.N + col] = v;
    }
}

// Sums the partials in split order (deterministic), applies the row scales,
// the routed un-permute and the residual, and stores the output.  A
// separate launch: the kernel boundary publishes the partials of every XCD
// (a device-scope release inside k_down_skinny would write back the whole
// L2 of each XCD per workgroup, which costs far more than the launch).
template <class T, int V>
__global__ __launch_bounds__(256) void k_down_reduce(DownArgs a, const float* part, int splits) {
    // V consecutive columns per thread (16-byte partial loads when V = 4);
    // the launcher keeps M * N below 2^31, so every index fits an int
    const int nv = (int)a.N / V;
    const int idx = (int)blockIdx.x * 256 + (int)threadIdx.x;
    if (idx >= (int)a.M * nv) return;
    const int row = idx / nv, c0 = (idx - row * nv) * V;
    const int plane = (int)a.M * (int)a.N;
    const float* p = part + row * (int)a.N + c0;
    using VT = typename std::conditional<V == 4, f32x4, float>::type;
    VT acc{};
    int sp = 0;
    for (; sp + 2 <= splits; sp += 2) {   // two partials in flight; the sum keeps split order
        const VT v0 = *reinterpret_cast<const VT*>(p + sp * plane);
        const VT v1 = *reinterpret_cast<const VT*>(p + (sp + 1) * plane);
        acc += v0;
        acc += v1;
    }
    for (; sp < splits; ++sp) acc += *reinterpret_cast<const VT*>(p + sp * plane);
    if constexpr (V == 4) {
#pragma unroll
        for (int j = 0; j < 4; ++j) down_finish<T>(a, row, c0 + j, acc[j]);
    } else {
        down_finish<T>(a, row, c0, acc);
    }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

namespace {

template <class F>
int set_lds(F* fn, int bytes) {
    return set_kernel_lds(reinterpret_cast<const void*>(fn), bytes);
}

constexpr int red_bytes(int mt, int nu, int nw) { return nw * mt * nu * 4 * 64 * 4; }

// Staged rows per span: the activations, plus the weight rows when they are
// staged (never with fragment-major weights).
template <bool FP8, int MT, int NU, int NW, bool FRAG>
constexpr int skinny_rows() { return FRAG ? MT * 16 : staged_rows<FP8, MT, NU, NW>(); }

template <class Kind, bool FP8, int MT, int NW, bool FRAG>
int gate_up_skinny_mt(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    auto kern = k_gate_up_skinny<Kind, FP8, MT, NW, FRAG>;
    constexpr int kLds = std::max(red_bytes(MT, 2, NW), staged_lds_bytes<skinny_rows<FP8, MT, 2, NW, FRAG>(), NW>());
    int st = set_lds(kern, kLds);
    if (st) return st;
    hipLaunchKernelGGL(kern, dim3((unsigned)(packed_rows / 32)), dim3(64 * NW), kLds, stream, a);
    return check_launch("shared_gate_up (skinny)");
}

template <class Kind, bool FP8, bool FRAG>
int gate_up_skinny_frag(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (a.M <= 16) return gate_up_skinny_mt<Kind, FP8, 1, 8, FRAG>(a, packed_rows, stream);
    if (a.M <= 32) return gate_up_skinny_mt<Kind, FP8, 2, 8, FRAG>(a, packed_rows, stream);
    if (a.M <= 64) return gate_up_skinny_mt<Kind, FP8, 4, 8, FRAG>(a, packed_rows, stream);
    return gate_up_skinny_mt<Kind, FP8, 8, 4, FRAG>(a, packed_rows, stream);
}

template <class Kind, bool FP8>
int gate_up_skinny_kind(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if constexpr (!FP8) {
        if (a.w_frag != nullptr) return gate_up_skinny_frag<Kind, FP8, true>(a, packed_rows, stream);
    }
    return gate_up_skinny_frag<Kind, FP8, false>(a, packed_rows, stream);
}

// K spans (128 bytes of K) per split: the whole K (no reduction launch) up
// to 8 tokens; about 16 spans (2 KiB of K: four splits at K = 3328) up to 64
// tokens and 8 above, spread evenly over the splits.
int down_spans_per_split(int64_t M, int spans) {
    int target = M <= 8 ? spans : (M <= 64 ? 16 : 8);
    if (target > spans) target = spans;
    if (target < 1) target = 1;
    const int splits = (spans + target - 1) / target;
    return (spans + splits - 1) / splits;
}

template <class Kind, bool FP8, int MT, int COLS, int NW, bool FRAG>
int down_skinny_mt(const DownArgs& a, float* part, int sps, int splits, hipStream_t stream) {
    constexpr int NU = (COLS + 15) / 16;
    auto kern = k_down_skinny<Kind, FP8, MT, COLS, NW, FRAG>;
    constexpr int kLds = std::max(red_bytes(MT, NU, NW), staged_lds_bytes<skinny_rows<FP8, MT, NU, NW, FRAG>(), NW>());
    int st = set_lds(kern, kLds);
    if (st) return st;
    const int ncol = (int)((a.N + COLS - 1) / COLS);
    hipLaunchKernelGGL(kern, dim3((unsigned)(ncol * splits)), dim3(64 * NW), kLds, stream, a, part, sps, ncol, splits);
    st = check_launch("shared_down_combine (skinny)");
    if (st || splits == 1) return st;
    const bool vec = a.N % 4 == 0 && (reinterpret_cast<uintptr_t>(part) & 15) == 0;
    auto red = vec ? k_down_reduce<typename Kind::T, 4> : k_down_reduce<typename Kind::T, 1>;
    const int64_t total = a.M * (int64_t)(vec ? a.N / 4 : a.N);
    hipLaunchKernelGGL(red, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, a, (const float*)part, splits);
    return check_launch("shared_down_combine (skinny reduce)");
}

// Column tile: 8 columns up to 16 tokens (the whole K in one workgroup, so
// twice the workgroups), 16 up to 64 tokens, 32 above (half the re-reads of
// the activations).
int down_cols(int64_t M) { return M <= 16 ? 8 : (M <= 64 ? 16 : 32); }

template <class Kind, bool FP8, int COLS, bool FRAG>
int down_skinny_cols(const DownArgs& a, float* part, int sps, int splits, hipStream_t stream) {
    if (a.M <= 16) return down_skinny_mt<Kind, FP8, 1, COLS, 8, FRAG>(a, part, sps, splits, stream);
    if (a.M <= 32) return down_skinny_mt<Kind, FP8, 2, COLS, 8, FRAG>(a, part, sps, splits, stream);
    if (a.M <= 64) return down_skinny_mt<Kind, FP8, 4, COLS, 8, FRAG>(a, part, sps, splits, stream);
    return down_skinny_mt<Kind, FP8, 8, COLS, 4, FRAG>(a, part, sps, splits, stream);
}

template <class Kind, bool FP8, bool FRAG>
int down_skinny_frag(const DownArgs& a, float* part, int sps, int splits, hipStream_t stream) {
    const int cols = down_cols(a.M);
    if (cols == 8) return down_skinny_cols<Kind, FP8, 8, FRAG>(a, part, sps, splits, stream);
    if (cols == 16) return down_skinny_cols<Kind, FP8, 16, FRAG>(a, part, sps, splits, stream);
    return down_skinny_cols<Kind, FP8, 32, FRAG>(a, part, sps, splits, stream);
}

template <class Kind, bool FP8>
int down_skinny_kind(const DownArgs& a, float* part, int sps, int splits, hipStream_t stream) {
    if constexpr (!FP8) {
        if (a.w_frag != nullptr) return down_skinny_frag<Kind, FP8, true>(a, part, sps, splits, stream);
    }
    return down_skinny_frag<Kind, FP8, false>(a, part, sps, splits, stream);
}

}  // namespace

// One 16-byte chunk per thread: destination chunk d of block (b, g) is
// lane l = d % 64 of that block's 1 KiB, i.e. row 16 b + (l & 15), K bytes
// 64 g + 16 (l >> 4); chunks at or past kbytes are zero.
__global__ __launch_bounds__(256) void k_pack_fragments(const char* src, int64_t rows, int64_t kbytes,
                                                        int64_t ld_bytes, char* dst, int64_t groups) {
    const int64_t total = rows / 16 * groups * 64;
    for (int64_t d = (int64_t)blockIdx.x * 256 + threadIdx.x; d < total; d += (int64_t)gridDim.x * 256) {
        const int64_t blk = d / (groups * 64), rem = d % (groups * 64);
        const int64_t g = rem / 64;
        const int l = (int)(rem % 64);
        const int64_t row = blk * 16 + (l & 15), kb = g * 64 + 16 * (l >> 4);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (kb < kbytes) v = *reinterpret_cast<const u32x4*>(src + row * ld_bytes + kb);
        *reinterpret_cast<u32x4*>(dst + d * 16) = v;
    }
}

int launch_pack_fragments(const void* src, int64_t rows, int64_t kbytes, int64_t ld_bytes, void* dst,
                          hipStream_t stream) {
    const int64_t groups = (kbytes + 63) / 64;
    const int64_t total = rows / 16 * groups * 64;
    if (total <= 0) return TRMOE_OK;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_pack_fragments, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const char*>(src),
                       rows, kbytes, ld_bytes, static_cast<char*>(dst), groups);
    return check_launch("pack_fragments");
}

// Streaming floor of the decode kernels: one pass over a byte range with
// 16-byte loads, eight in flight per thread before any is used; each
// workgroup XOR-folds what it read into sink[blockIdx.x], so no load is dead.
__global__ __launch_bounds__(256) void k_stream_read(const u32x4* __restrict__ src, int64_t n16,
                                                     uint32_t* __restrict__ sink) {
    __shared__ uint32_t s_fold[4];
    const int64_t stride = (int64_t)gridDim.x * 256;
    uint32_t fold = 0;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += 8 * stride) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t j = i + u * stride;
            v[u] = j < n16 ? src[j] : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) fold ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) fold ^= (uint32_t)__shfl_xor((int)fold, off);
    if ((threadIdx.x & 63) == 0) s_fold[threadIdx.x >> 6] = fold;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = s_fold[0] ^ s_fold[1] ^ s_fold[2] ^ s_fold[3];
}

int launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int blocks, hipStream_t stream) {
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)blocks), dim3(256), 0, stream,
                       static_cast<const u32x4*>(src), bytes / 16, sink);
    return check_launch("stream_read");
}

int launch_gate_up_skinny(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return gate_up_skinny_kind<KindF32, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return gate_up_skinny_kind<KindBF16, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return gate_up_skinny_kind<KindBF16, true>(a, packed_rows, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_gate_up: unsupported dtype pair");
}

size_t down_skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, int act) {
    if (M < 1 || M > kSkinnyMaxTokens) return 0;
    const int eb = act == TRMOE_F32 ? 4 : 2;
    const int spans = (int)((K * eb + 127) / 128);
    const int64_t splits = (spans + down_spans_per_split(M, spans) - 1) / down_spans_per_split(M, spans);
    return (size_t)(splits * M * N * (int64_t)sizeof(float));
}

int launch_down_skinny(int act, int wdt, const DownArgs& a, void* workspace, hipStream_t stream) {
    if (a.M * (int64_t)a.N >= ((int64_t)1 << 31))
        return set_error(TRMOE_ERR_UNSUPPORTED, "shared_down_combine: decode path needs tokens * hidden < 2^31");
    const int eb = act == TRMOE_F32 ? 4 : 2;
    const int spans = (int)(((int64_t)a.K * eb + 127) / 128);
    const int sps = down_spans_per_split(a.M, spans);
    const int splits = (spans + sps - 1) / sps;
    float* part = static_cast<float*>(workspace);
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return down_skinny_kind<KindF32, false>(a, part, sps, splits, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return down_skinny_kind<KindBF16, false>(a, part, sps, splits, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3)
        return down_skinny_kind<KindBF16, true>(a, part, sps, splits, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_down_combine: unsupported dtype pair");
}

}  // namespace trmoe
