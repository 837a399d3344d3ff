// Decode-shape (few tokens) variants of K2 and K4.
//
// With M <= 128 tokens the layer is weight-streaming: every weight byte is
// used M times, far below the MFMA/HBM balance point (~300 FLOP/B for bf16),
// so the kernels are organised to keep as many weight loads in flight as the
// CUs allow and to touch each weight byte once:
//
//   k_gate_up_skinny   one workgroup per 16 output features (16 gate + 16 up
//                      packed rows) and all M tokens; the waves split K, each
//                      loading its operands straight into 16x16 MFMA
//                      registers (no LDS staging), and reduce through LDS
//                      before the SwiGLU epilogue (same epilogue contract as
//                      k_gate_up_swiglu, including the dense-routed scaling)
//   k_down_skinny      split-K: workgroup (32 output columns, K chunk)
//                      writes an fp32 partial [split][M][N] to the caller's
//                      workspace
//   k_down_reduce      sums the partials in split order (deterministic),
//                      applies the row scales, the routed un-permute and the
//                      residual, and stores the output
#include "trmoe_common.h"
#include "trmoe_internal.h"
#include "trmoe_gemm.h"

#include <stdlib.h>

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

// acc[tm][u] += A(rows tm*16..+15) . W(rows u*16..+15)^T over the K groups
// [g0, g1) of this wave, loading GB groups at a time.  a_off[tm] / w_off[u]
// are the byte offsets of the lane's row in each operand (kOutOfRange for
// absent rows); kb_a is the byte length of K in an activation row.
template <class Kind, bool FP8, int MT, int NU, int GB>
__device__ __forceinline__ void skinny_k_loop(__amdgpu_buffer_rsrc_t ar, const int (&a_off)[MT],
                                              __amdgpu_buffer_rsrc_t wr, const int (&w_off)[NU], int g0, int g1,
                                              int kb_a, f32x4 (&acc)[MT][NU]) {
    using WF = WFrag<Kind, FP8>;
    const int q = (threadIdx.x & 63) >> 4;
    for (int gb = g0; gb < g1; gb += GB) {
        u32x4 av[GB][MT];
        typename WF::Reg wv[GB][NU];
#pragma unroll
        for (int j = 0; j < GB; ++j) {
            const int g = gb + j;
            const bool ok = g < g1;
            const int ao = 64 * g + 16 * q;
#pragma unroll
            for (int tm = 0; tm < MT; ++tm)
                av[j][tm] = buffer_load16(ar, (ok && ao < kb_a) ? a_off[tm] + ao : kOutOfRange);
#pragma unroll
            for (int u = 0; u < NU; ++u) wv[j][u] = WF::load(wr, ok ? w_off[u] : kOutOfRange, g, q, kb_a);
        }
        // every load of the batch is in flight before the first MFMA waits
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < GB; ++j)
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const u32x4 b = WF::expand(wv[j][u]);
#pragma unroll
                for (int tm = 0; tm < MT; ++tm) mfma16(Kind{}, av[j][tm], b, acc[tm][u]);
            }
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
template <class Kind, bool FP8, int MT, int NW, int GB>
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
    const auto wr = make_rsrc(static_cast<const char*>(a.w) + pg * a.ldw * kWB, (uint32_t)(48 * a.ldw * kWB));

    const bool routed = a.ids != nullptr && f0 >= a.shared_feats;
    if (routed && threadIdx.x < MT * 16) {
        const int64_t row = threadIdx.x;
        int64_t id = row < a.M ? a.ids[row] : 0;
        id = id < 0 ? 0 : (id >= a.vocab ? a.vocab - 1 : id);
        for (int j = 0; j < kMaxTopK; ++j)
            s_route[row][j] = (j < a.top_k && row < a.M) ? (int)a.table[(int64_t)j * a.vocab + id] : -1;
    }
    int a_off[MT], w_off[2];
#pragma unroll
    for (int tm = 0; tm < MT; ++tm) {
        const int row = tm * 16 + r;
        a_off[tm] = row < a.M ? (int)(row * a.ldx * (int64_t)sizeof(T)) : kOutOfRange;
    }
    w_off[0] = (int)(r * a.ldw * kWB);          // gate row pg + r
    w_off[1] = (int)((32 + r) * a.ldw * kWB);   // up row pg + 32 + r

    const int groups = (kb_a + 63) / 64;
    const int per_wave = (groups + NW - 1) / NW;
    const int g0 = wave * per_wave;
    const int g1 = g0 + per_wave < groups ? g0 + per_wave : groups;
    f32x4 acc[MT][2];
    zero_acc16<MT, 2>(acc);
    skinny_k_loop<Kind, FP8, MT, 2, GB>(ar, a_off, wr, w_off, g0, g1, kb_a, acc);
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
        const float g = skinny_sum<MT, 2, NW>(red, tm, 0, i, l) * sg;
        const float u = skinny_sum<MT, 2, NW>(red, tm, 1, i, l) * su;
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

// Split-K partial of the down GEMM: block (x = 16*NU-column tile, y = K
// split) writes part[(split * M + row) * N + col] for its rows and columns;
// with a single split it finishes the output itself.
template <class Kind, bool FP8, int MT, int NU, int NW, int GB>
__global__ __launch_bounds__(64 * NW) void k_down_skinny(DownArgs a, float* part, int groups_per_split) {
    using T = typename Kind::T;
    constexpr int NT = 64 * NW;
    constexpr int kWB = FP8 ? 1 : (int)sizeof(T);
    constexpr int kCols = 16 * NU;
    extern __shared__ __align__(16) float red[];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane & 15;
    const int64_t n0 = (int64_t)blockIdx.x * kCols;
    const int split = blockIdx.y;

    const int kb_a = a.K * (int)sizeof(T);
    const auto ar = make_rsrc(a.h, (uint32_t)(a.M * a.ldh * (int64_t)sizeof(T)));
    const auto wr = make_rsrc(static_cast<const char*>(a.w) + n0 * a.ldw * kWB, (uint32_t)(kCols * a.ldw * kWB));
    int a_off[MT], w_off[NU];
#pragma unroll
    for (int tm = 0; tm < MT; ++tm) {
        const int row = tm * 16 + r;
        a_off[tm] = row < a.M ? (int)(row * a.ldh * (int64_t)sizeof(T)) : kOutOfRange;
    }
#pragma unroll
    for (int u = 0; u < NU; ++u) w_off[u] = (int)((u * 16 + r) * a.ldw * kWB);

    const int groups = (kb_a + 63) / 64;
    const int s0 = split * groups_per_split;
    const int s1 = s0 + groups_per_split < groups ? s0 + groups_per_split : groups;
    const int per_wave = (s1 - s0 + NW - 1) / NW;
    const int g0 = s0 + wave * per_wave;
    const int g1 = g0 + per_wave < s1 ? g0 + per_wave : s1;
    f32x4 acc[MT][NU];
    zero_acc16<MT, NU>(acc);
    skinny_k_loop<Kind, FP8, MT, NU, GB>(ar, a_off, wr, w_off, g0, g1, kb_a, acc);
    skinny_stash<MT, NU>(red, acc);
    __syncthreads();

    const bool single = gridDim.y == 1;
    float* dst = part + (int64_t)split * a.M * a.N;
    for (int qi = threadIdx.x; qi < MT * NU * 4 * 64; qi += NT) {
        const int l = qi & 63, i = (qi >> 6) & 3, u = (qi >> 8) % NU, tm = (qi >> 8) / NU;
        const int row = tm * 16 + 4 * (l >> 4) + i;
        const int64_t col = n0 + u * 16 + (l & 15);
        if (row >= a.M || col >= a.N) continue;
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
template <class T>
__global__ __launch_bounds__(256) void k_down_reduce(DownArgs a, const float* part, int splits) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= a.M * (int64_t)a.N) return;
    const int64_t row = idx / a.N, col = idx % a.N;
    const int64_t plane = a.M * (int64_t)a.N;
    float s = 0.f;
    for (int sp = 0; sp < splits; ++sp) s += part[sp * plane + idx];
    down_finish<T>(a, row, col, s);
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

template <class Kind, bool FP8, int MT, int NW, int GB>
int gate_up_skinny_mt(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    auto kern = k_gate_up_skinny<Kind, FP8, MT, NW, GB>;
    constexpr int kLds = red_bytes(MT, 2, NW);
    int st = set_lds(kern, kLds);
    if (st) return st;
    hipLaunchKernelGGL(kern, dim3((unsigned)(packed_rows / 32)), dim3(64 * NW), kLds, stream, a);
    return check_launch("shared_gate_up (skinny)");
}

template <class Kind, bool FP8>
int gate_up_skinny_kind(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (a.M <= 16) return gate_up_skinny_mt<Kind, FP8, 1, 8, 8>(a, packed_rows, stream);
    if (a.M <= 32) return gate_up_skinny_mt<Kind, FP8, 2, 8, 8>(a, packed_rows, stream);
    if (a.M <= 64) return gate_up_skinny_mt<Kind, FP8, 4, 8, 4>(a, packed_rows, stream);
    return gate_up_skinny_mt<Kind, FP8, 8, 4, 2>(a, packed_rows, stream);
}

// K groups (64 bytes of K) per split: the whole K (no reduction launch) up
// to 8 tokens; then 32 groups (2 KiB of K: four splits at K = 3328) up to 64
// tokens and 16 above -- the measured optimum of a sweep over 8..56 groups
// and 16/32-column tiles at C3's shapes.  At least two groups per wave.
int down_groups_per_split(int64_t M, int groups, int nw) {
    int gps = M <= 8 ? groups : (M <= 64 ? 32 : 16);
    if (gps < 2 * nw) gps = 2 * nw;
    const char* e = getenv("TRMOE_SKINNY_GPS");
    if (e != nullptr && atoi(e) > 0) gps = atoi(e);
    gps = (gps + nw - 1) / nw * nw;
    if (gps > groups) gps = (groups + nw - 1) / nw * nw;
    return gps;
}

int down_nw(int64_t M) { return M <= 64 ? 8 : 4; }

template <class Kind, bool FP8, int MT, int NU, int NW, int GB>
int down_skinny_mt(const DownArgs& a, float* part, int gps, int splits, hipStream_t stream) {
    auto kern = k_down_skinny<Kind, FP8, MT, NU, NW, GB>;
    constexpr int kLds = red_bytes(MT, NU, NW);
    int st = set_lds(kern, kLds);
    if (st) return st;
    hipLaunchKernelGGL(kern, dim3((unsigned)((a.N + 16 * NU - 1) / (16 * NU)), (unsigned)splits), dim3(64 * NW), kLds,
                       stream, a, part, gps);
    st = check_launch("shared_down_combine (skinny)");
    if (st || splits == 1) return st;
    const int64_t total = a.M * (int64_t)a.N;
    hipLaunchKernelGGL(k_down_reduce<typename Kind::T>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       a, (const float*)part, splits);
    return check_launch("shared_down_combine (skinny reduce)");
}

// Column tile: 16 columns (twice the workgroups) up to 64 tokens, 32 above
// (half the re-reads of the activations).  TRMOE_SKINNY_NU=1/2 forces.
int down_nu(int64_t M) {
    const char* e = getenv("TRMOE_SKINNY_NU");
    if (e != nullptr && (atoi(e) == 1 || atoi(e) == 2)) return atoi(e);
    return M <= 64 ? 1 : 2;
}

template <class Kind, bool FP8, int NU>
int down_skinny_nu(const DownArgs& a, float* part, int gps, int splits, hipStream_t stream) {
    if (a.M <= 16) return down_skinny_mt<Kind, FP8, 1, NU, 8, 8>(a, part, gps, splits, stream);
    if (a.M <= 32) return down_skinny_mt<Kind, FP8, 2, NU, 8, 8>(a, part, gps, splits, stream);
    if (a.M <= 64) return down_skinny_mt<Kind, FP8, 4, NU, 8, 4>(a, part, gps, splits, stream);
    return down_skinny_mt<Kind, FP8, 8, NU, 4, 2>(a, part, gps, splits, stream);
}

template <class Kind, bool FP8>
int down_skinny_kind(const DownArgs& a, float* part, int gps, int splits, hipStream_t stream) {
    if (down_nu(a.M) == 1) return down_skinny_nu<Kind, FP8, 1>(a, part, gps, splits, stream);
    return down_skinny_nu<Kind, FP8, 2>(a, part, gps, splits, stream);
}

}  // namespace

int launch_gate_up_skinny(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream) {
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return gate_up_skinny_kind<KindF32, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return gate_up_skinny_kind<KindBF16, false>(a, packed_rows, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3) return gate_up_skinny_kind<KindBF16, true>(a, packed_rows, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_gate_up: unsupported dtype pair");
}

size_t down_skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, int act) {
    if (M < 1 || M > kSkinnyMaxTokens) return 0;
    const int eb = act == TRMOE_F32 ? 4 : 2;
    const int groups = (int)((K * eb + 63) / 64);
    const int gps = down_groups_per_split(M, groups, down_nw(M));
    const int64_t splits = (groups + gps - 1) / gps;
    return (size_t)(splits * M * N * (int64_t)sizeof(float));
}

int launch_down_skinny(int act, int wdt, const DownArgs& a, void* workspace, hipStream_t stream) {
    const int eb = act == TRMOE_F32 ? 4 : 2;
    const int groups = (int)(((int64_t)a.K * eb + 63) / 64);
    const int gps = down_groups_per_split(a.M, groups, down_nw(a.M));
    const int splits = (groups + gps - 1) / gps;
    float* part = static_cast<float*>(workspace);
    if (act == TRMOE_F32 && wdt == TRMOE_F32) return down_skinny_kind<KindF32, false>(a, part, gps, splits, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_BF16) return down_skinny_kind<KindBF16, false>(a, part, gps, splits, stream);
    if (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3)
        return down_skinny_kind<KindBF16, true>(a, part, gps, splits, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "shared_down_combine: unsupported dtype pair");
}

}  // namespace trmoe
