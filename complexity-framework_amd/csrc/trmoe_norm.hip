// Row-wise kernels over token rows: the block MLP's RMSNorm (training and
// fp8 layers) and the per-token e4m3 quantizer of the W8A8 gate|up.
//
//   k_rmsnorm_fwd   one wave per token row: r = 1 / sqrt(mean(x^2) + eps) in
//                   fp32, y = T(x * r) * w (the rounding of the "llama"
//                   casting of liger-kernel's RMSNorm, which the reference
//                   calls on CUDA, complexity/core/normalization/norms.py:
//                   46-55), r saved for the backward.
//   k_rmsnorm_bwd   one wave per row, rows strided over a fixed grid:
//                   m = dy * w, dx = r m - (r^3 / H) (m . x) x (plus an
//                   optional residual gradient), and each workgroup's
//                   fp32 sum of dy * T(x * r) over its rows (the weight
//                   gradient's partial).
//   k_rmsnorm_dw    sums the partials in workgroup order (deterministic).
//   k_quantize_rows one wave per row: scale = amax / 448 (1 for a zero row,
//                   or one holding a NaN) and codes e4m3(clamp(x / scale)),
//                   the oracle's quantize_e4m3 over each row, bit for bit.
//
// HBM-bound: a row is read once into registers (16-byte loads, chunk c of a
// row on lane c % 64), so hidden sizes up to 64 * kMaxChunks chunks per row.
#include "trmoe_common.h"
#include "trmoe_internal.h"
#include "trmoe_gemm.h"

namespace trmoe {

namespace {

constexpr int kNormWaves = 4;
constexpr int kMaxChunks = 8;           // 16-byte chunks per lane
constexpr int kDwGroups = 1024;         // most workgroups (weight partials) of the backward

// Element e of a 16-byte chunk as fp32 (8 bf16 or 4 f32).
template <class T>
__device__ __forceinline__ float chunk_elem(const u32x4& v, int e) {
    if constexpr (sizeof(T) == 2) {
        const uint32_t u = v[e >> 1];
        return __builtin_bit_cast(float, (e & 1) ? (u & 0xffff0000u) : (u << 16));
    } else {
        return __builtin_bit_cast(float, (uint32_t)v[e]);
    }
}

// Packs kV fp32 values into a 16-byte chunk of T (round to nearest even).
template <class T>
__device__ __forceinline__ u32x4 pack_chunk(const float (&f)[16 / sizeof(T)]) {
    u32x4 out;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x2 p = {(bf16_t)f[2 * j], (bf16_t)f[2 * j + 1]};
            out[j] = __builtin_bit_cast(uint32_t, p);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = __builtin_bit_cast(uint32_t, (float)f[j]);
    }
    return out;
}

__device__ __forceinline__ float wave_sum(float s) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    return s;
}

template <class T>
__device__ __forceinline__ float round_to(float v) {
    return to_f32(from_f32<T>(v));
}

template <class T, int MC>
__global__ __launch_bounds__(64 * kNormWaves) void k_rmsnorm_fwd(const T* __restrict__ x, int64_t n, int hidden,
                                                                  int64_t ldx, const T* __restrict__ w, float eps,
                                                                  T* __restrict__ y, int64_t ldy,
                                                                  float* __restrict__ rs) {
    constexpr int kV = 16 / (int)sizeof(T);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kNormWaves + wave;
    if (row >= n) return;
    const int nch = hidden / kV;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * ldx);
    const u32x4* wr = reinterpret_cast<const u32x4*>(w);
    u32x4 xv[MC], wv[MC];
#pragma unroll
    for (int j = 0; j < MC; ++j) {
        const int c = lane + 64 * j;
        xv[j] = c < nch ? xr[c] : u32x4{0u, 0u, 0u, 0u};
        wv[j] = c < nch ? wr[c] : u32x4{0u, 0u, 0u, 0u};
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < MC; ++j)
#pragma unroll
        for (int e = 0; e < kV; ++e) {
            const float f = chunk_elem<T>(xv[j], e);
            s += f * f;
        }
    s = wave_sum(s);
    const float r = rsqrtf(s / (float)hidden + eps);
    u32x4* yr = reinterpret_cast<u32x4*>(y + row * ldy);
#pragma unroll
    for (int j = 0; j < MC; ++j) {
        const int c = lane + 64 * j;
        if (c >= nch) continue;
        float f[kV];
#pragma unroll
        for (int e = 0; e < kV; ++e) f[e] = round_to<T>(chunk_elem<T>(xv[j], e) * r) * chunk_elem<T>(wv[j], e);
        yr[c] = pack_chunk<T>(f);
    }
    if (lane == 0) rs[row] = r;
}

template <class T, int MC>
__global__ __launch_bounds__(64 * kNormWaves) void k_rmsnorm_bwd(const T* __restrict__ x, int64_t ldx,
                                                                  const T* __restrict__ w,
                                                                  const float* __restrict__ rs,
                                                                  const T* __restrict__ dy, int64_t lddy,
                                                                  const T* dres, int64_t lddres, int64_t n,
                                                                  int hidden, T* dx, int64_t lddx,
                                                                  float* __restrict__ part) {
    // dres and dx may be one buffer: each element is read, then written, by
    // the same lane
    constexpr int kV = 16 / (int)sizeof(T);
    extern __shared__ float s_dw[];                  // [kNormWaves][hidden]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nch = hidden / kV;
    const float inv_h = 1.0f / (float)hidden;
    const u32x4* wr = reinterpret_cast<const u32x4*>(w);
    u32x4 wv[MC];
    float acc[MC][kV];
#pragma unroll
    for (int j = 0; j < MC; ++j) {
        const int c = lane + 64 * j;
        wv[j] = c < nch ? wr[c] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < kV; ++e) acc[j][e] = 0.f;
    }
    for (int64_t row = (int64_t)blockIdx.x * kNormWaves + wave; row < n; row += (int64_t)gridDim.x * kNormWaves) {
        const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * ldx);
        const u32x4* gr = reinterpret_cast<const u32x4*>(dy + row * lddy);
        u32x4 xv[MC], gv[MC], rv[MC];
#pragma unroll
        for (int j = 0; j < MC; ++j) {
            const int c = lane + 64 * j;
            const bool in = c < nch;
            xv[j] = in ? xr[c] : u32x4{0u, 0u, 0u, 0u};
            gv[j] = in ? gr[c] : u32x4{0u, 0u, 0u, 0u};
            rv[j] = (in && dres != nullptr) ? reinterpret_cast<const u32x4*>(dres + row * lddres)[c]
                                            : u32x4{0u, 0u, 0u, 0u};
        }
        const float r = rs[row];
        float s = 0.f;
#pragma unroll
        for (int j = 0; j < MC; ++j)
#pragma unroll
            for (int e = 0; e < kV; ++e)
                s += chunk_elem<T>(gv[j], e) * chunk_elem<T>(wv[j], e) * chunk_elem<T>(xv[j], e);
        s = wave_sum(s);
        const float coef = r * r * r * s * inv_h;
        u32x4* dr = reinterpret_cast<u32x4*>(dx + row * lddx);
#pragma unroll
        for (int j = 0; j < MC; ++j) {
            const int c = lane + 64 * j;
            if (c >= nch) continue;
            float f[kV];
#pragma unroll
            for (int e = 0; e < kV; ++e) {
                const float xe = chunk_elem<T>(xv[j], e), ge = chunk_elem<T>(gv[j], e);
                f[e] = r * (ge * chunk_elem<T>(wv[j], e)) - coef * xe + chunk_elem<T>(rv[j], e);
                acc[j][e] += ge * round_to<T>(xe * r);
            }
            dr[c] = pack_chunk<T>(f);
        }
    }
    // the workgroup's partial: its waves' sums added in wave order
#pragma unroll
    for (int j = 0; j < MC; ++j) {
        const int c = lane + 64 * j;
        if (c >= nch) continue;
#pragma unroll
        for (int e = 0; e < kV; ++e) s_dw[wave * hidden + c * kV + e] = acc[j][e];
    }
    __syncthreads();
    float* dst = part + (int64_t)blockIdx.x * hidden;
    for (int k = threadIdx.x; k < hidden; k += 64 * kNormWaves) {
        float t = s_dw[k];
#pragma unroll
        for (int v = 1; v < kNormWaves; ++v) t += s_dw[v * hidden + k];
        dst[k] = t;
    }
}

// dw[k] = sum over workgroups b (in order) of part[b][k]: 32 columns (whole
// 128-byte lines) x 32 strided groups of partials per workgroup (a group
// sums every 32nd partial, eight loads in flight), the groups then added in
// order.  Latency-bound: the chain per thread is what sets the time.
template <class T>
__global__ __launch_bounds__(1024) void k_rmsnorm_dw(const float* __restrict__ part, int groups, int hidden,
                                                      T* __restrict__ dw) {
    __shared__ float s[32][33];
    const int c = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int col = (int)blockIdx.x * 32 + c;
    float t = 0.f;
    if (col < hidden) {
        int b = g;
        for (; b + 224 < groups; b += 256) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(b + 32 * u) * hidden + col];
#pragma unroll
            for (int u = 0; u < 8; ++u) t += v[u];
        }
        for (; b < groups; b += 32) t += part[(int64_t)b * hidden + col];
    }
    s[g][c] = t;
    __syncthreads();
    if (g == 0 && col < hidden) {
        float u = s[0][c];
#pragma unroll
        for (int v = 1; v < 32; ++v) u += s[v][c];
        dw[col] = from_f32<T>(u);
    }
}

template <class T, int MC>
__global__ __launch_bounds__(64 * kNormWaves) void k_quantize_rows(const T* __restrict__ x, int64_t n, int k,
                                                                    int64_t ldx, uint8_t* __restrict__ q,
                                                                    int64_t ldq, float* __restrict__ scale) {
    constexpr int kV = 16 / (int)sizeof(T);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * kNormWaves + wave;
    if (row >= n) return;
    const int nch = k / kV;
    const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * ldx);
    u32x4 xv[MC];
#pragma unroll
    for (int j = 0; j < MC; ++j) {
        const int c = lane + 64 * j;
        xv[j] = c < nch ? xr[c] : u32x4{0u, 0u, 0u, 0u};
    }
    float amax = 0.f;
    bool nan = false;
#pragma unroll
    for (int j = 0; j < MC; ++j)
#pragma unroll
        for (int e = 0; e < kV; ++e) {
            const float f = chunk_elem<T>(xv[j], e);
            nan |= f != f;
            amax = fmaxf(amax, fabsf(f));
        }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    nan = __ballot(nan) != 0;
    // a row holding a NaN has a NaN amax, which is not > 0: scale 1
    const float sc = (!nan && amax > 0.f) ? amax / 448.0f : 1.0f;
    uint8_t* qr = q + row * ldq;
#pragma unroll
    for (int j = 0; j < MC; ++j) {
        const int c = lane + 64 * j;
        if (c >= nch) continue;
        // four codes per word: v_cvt_pk_fp8_f32 (OCP e4m3, round to nearest
        // even -- torch's conversion, matched bit for bit over every bf16
        // value by the GPU tests) of the correctly rounded quotients
        uint32_t w[kV / 4];
#pragma unroll
        for (int t = 0; t < kV / 4; ++t) {
            float v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float f = chunk_elem<T>(xv[j], 4 * t + u) / sc;
                v[u] = f > 448.0f ? 448.0f : (f < -448.0f ? -448.0f : f);   // NaN stays NaN
            }
            int packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[0], v[1], 0, false);
            packed = __builtin_amdgcn_cvt_pk_fp8_f32(v[2], v[3], packed, true);
            w[t] = (uint32_t)packed;
        }
        if constexpr (kV == 8)
            *reinterpret_cast<u32x2*>(qr + c * kV) = u32x2{w[0], w[1]};
        else
            *reinterpret_cast<uint32_t*>(qr + c * kV) = w[0];
    }
    if (lane == 0) scale[row] = sc;
}

template <class T, int MC>
int quant_mc(const void* x, int64_t n, int64_t k, int64_t ldx, void* q, int64_t ldq, float* scale,
             hipStream_t stream) {
    const dim3 grid((unsigned)((n + kNormWaves - 1) / kNormWaves));
    hipLaunchKernelGGL((k_quantize_rows<T, MC>), grid, dim3(64 * kNormWaves), 0, stream, static_cast<const T*>(x), n,
                       (int)k, ldx, static_cast<uint8_t*>(q), ldq, scale);
    return check_launch("quantize_rows_e4m3");
}

template <class T>
int quant_kind(const void* x, int64_t n, int64_t k, int64_t ldx, void* q, int64_t ldq, float* scale,
               hipStream_t stream);

template <class T>
int chunks_per_lane(int64_t hidden) {
    constexpr int kV = 16 / (int)sizeof(T);
    const int64_t per = (hidden / kV + 63) / 64;
    return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 0;
}

template <class T, int MC>
int fwd_mc(const T* x, int64_t n, int64_t hidden, int64_t ldx, const T* w, float eps, T* y, int64_t ldy, float* rs,
           hipStream_t stream) {
    const dim3 grid((unsigned)((n + kNormWaves - 1) / kNormWaves));
    hipLaunchKernelGGL((k_rmsnorm_fwd<T, MC>), grid, dim3(64 * kNormWaves), 0, stream, x, n, (int)hidden, ldx, w, eps,
                       y, ldy, rs);
    return check_launch("rmsnorm_forward");
}

template <class T>
int fwd_kind(const void* x, int64_t n, int64_t hidden, int64_t ldx, const void* w, float eps, void* y, int64_t ldy,
             float* rs, hipStream_t stream) {
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    T* yp = static_cast<T*>(y);
    switch (chunks_per_lane<T>(hidden)) {
    case 1: return fwd_mc<T, 1>(xp, n, hidden, ldx, wp, eps, yp, ldy, rs, stream);
    case 2: return fwd_mc<T, 2>(xp, n, hidden, ldx, wp, eps, yp, ldy, rs, stream);
    case 4: return fwd_mc<T, 4>(xp, n, hidden, ldx, wp, eps, yp, ldy, rs, stream);
    case 8: return fwd_mc<T, 8>(xp, n, hidden, ldx, wp, eps, yp, ldy, rs, stream);
    default: return set_error(TRMOE_ERR_UNSUPPORTED, "rmsnorm: hidden too large for one row per wave");
    }
}

template <class T, int MC>
int bwd_mc(const T* x, int64_t ldx, const T* w, const float* rs, const T* dy, int64_t lddy, const T* dres,
           int64_t lddres, int64_t n, int64_t hidden, T* dx, int64_t lddx, T* dw, float* part, hipStream_t stream) {
    const int groups = rmsnorm_groups(n);
    const int lds = kNormWaves * (int)hidden * (int)sizeof(float);
    int st = set_kernel_lds(reinterpret_cast<const void*>(k_rmsnorm_bwd<T, MC>), lds);
    if (st) return st;
    hipLaunchKernelGGL((k_rmsnorm_bwd<T, MC>), dim3((unsigned)groups), dim3(64 * kNormWaves), lds, stream, x, ldx, w,
                       rs, dy, lddy, dres, lddres, n, (int)hidden, dx, lddx, part);
    st = check_launch("rmsnorm_backward");
    if (st) return st;
    hipLaunchKernelGGL((k_rmsnorm_dw<T>), dim3((unsigned)((hidden + 31) / 32)), dim3(1024), 0, stream,
                       (const float*)part, groups, (int)hidden, dw);
    return check_launch("rmsnorm_backward (weight gradient)");
}

template <class T>
int bwd_kind(const void* x, int64_t ldx, const void* w, const float* rs, const void* dy, int64_t lddy,
             const void* dres, int64_t lddres, int64_t n, int64_t hidden, void* dx, int64_t lddx, void* dw,
             float* part, hipStream_t stream) {
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    const T* gp = static_cast<const T*>(dy);
    const T* rp = static_cast<const T*>(dres);
    T* dxp = static_cast<T*>(dx);
    T* dwp = static_cast<T*>(dw);
    switch (chunks_per_lane<T>(hidden)) {
    case 1: return bwd_mc<T, 1>(xp, ldx, wp, rs, gp, lddy, rp, lddres, n, hidden, dxp, lddx, dwp, part, stream);
    case 2: return bwd_mc<T, 2>(xp, ldx, wp, rs, gp, lddy, rp, lddres, n, hidden, dxp, lddx, dwp, part, stream);
    case 4: return bwd_mc<T, 4>(xp, ldx, wp, rs, gp, lddy, rp, lddres, n, hidden, dxp, lddx, dwp, part, stream);
    case 8: return bwd_mc<T, 8>(xp, ldx, wp, rs, gp, lddy, rp, lddres, n, hidden, dxp, lddx, dwp, part, stream);
    default: return set_error(TRMOE_ERR_UNSUPPORTED, "rmsnorm: hidden too large for one row per wave");
    }
}

template <class T>
int quant_kind(const void* x, int64_t n, int64_t k, int64_t ldx, void* q, int64_t ldq, float* scale,
               hipStream_t stream) {
    switch (chunks_per_lane<T>(k)) {
    case 1: return quant_mc<T, 1>(x, n, k, ldx, q, ldq, scale, stream);
    case 2: return quant_mc<T, 2>(x, n, k, ldx, q, ldq, scale, stream);
    case 4: return quant_mc<T, 4>(x, n, k, ldx, q, ldq, scale, stream);
    case 8: return quant_mc<T, 8>(x, n, k, ldx, q, ldq, scale, stream);
    default: return set_error(TRMOE_ERR_UNSUPPORTED, "quantize_rows_e4m3: row too long for one row per wave");
    }
}

}  // namespace

int launch_quantize_rows_e4m3(int act, const void* x, int64_t n, int64_t k, int64_t ldx, void* q, int64_t ldq,
                              float* scale, hipStream_t stream) {
    if (n <= 0) return TRMOE_OK;
    if (act == TRMOE_BF16) return quant_kind<bf16_t>(x, n, k, ldx, q, ldq, scale, stream);
    if (act == TRMOE_F32) return quant_kind<float>(x, n, k, ldx, q, ldq, scale, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "quantize_rows_e4m3: bf16 or f32 activations");
}

int rmsnorm_groups(int64_t n) {
    const int64_t g = (n + kNormWaves - 1) / kNormWaves;
    return (int)(g < kDwGroups ? (g < 1 ? 1 : g) : kDwGroups);
}

int64_t rmsnorm_max_hidden(int act) {
    return (int64_t)64 * kMaxChunks * (act == TRMOE_BF16 ? 8 : 4);
}

int launch_rmsnorm_forward(int act, const void* x, int64_t n, int64_t hidden, int64_t ldx, const void* w, float eps,
                           void* y, int64_t ldy, float* rs, hipStream_t stream) {
    if (n <= 0) return TRMOE_OK;
    if (act == TRMOE_BF16) return fwd_kind<bf16_t>(x, n, hidden, ldx, w, eps, y, ldy, rs, stream);
    if (act == TRMOE_F32) return fwd_kind<float>(x, n, hidden, ldx, w, eps, y, ldy, rs, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "rmsnorm_forward: bf16 or f32 activations");
}

int launch_rmsnorm_backward(int act, const void* x, int64_t ldx, const void* w, const float* rs, const void* dy,
                            int64_t lddy, const void* dres, int64_t lddres, int64_t n, int64_t hidden, void* dx,
                            int64_t lddx, void* dw, float* part, hipStream_t stream) {
    if (act == TRMOE_BF16)
        return bwd_kind<bf16_t>(x, ldx, w, rs, dy, lddy, dres, lddres, n, hidden, dx, lddx, dw, part, stream);
    if (act == TRMOE_F32)
        return bwd_kind<float>(x, ldx, w, rs, dy, lddy, dres, lddres, n, hidden, dx, lddx, dw, part, stream);
    return set_error(TRMOE_ERR_UNSUPPORTED, "rmsnorm_backward: bf16 or f32 activations");
}

}  // namespace trmoe
