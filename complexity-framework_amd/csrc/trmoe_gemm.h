// Kernel argument blocks and launchers of the TR-MoE tile kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trmoe {

struct PackArgs {
    const void* a;
    const void* b;
    const float* sa;
    const float* sb;
    int64_t groups, out_features, in_features;
    int64_t s_group, s_out, s_in;
    int64_t scale_group_stride;
    void* dst;
    float* dst_scale;
    int64_t dst_rows, dst_cols;      // packed rows / cols written per group
    int64_t dst_ld;                  // elements between packed rows
    int64_t dst_group_stride;        // elements between groups
    int64_t dst_scale_group_stride;  // floats between groups of dst_scale
    int interleave;
    int elem_bytes;
};

struct GateUpArgs {
    const void* x;
    int64_t ldx;
    int64_t M;
    int K;
    const void* w;
    int64_t ldw;
    const float* w_scale;
    void* h;
    int64_t ldh;
    // Dense-routed epilogue: packed features at or past `shared_feats` belong
    // to expert (f - shared_feats) / expert_feats and are scaled by the
    // token's route weight for that expert (0 when not routed); shared
    // features are scaled by shared_mult.  ids == nullptr: no routed block.
    float shared_mult;
    int64_t shared_feats;
    int64_t expert_feats;
    const int64_t* ids;
    const int64_t* table;   // [top_k, vocab]
    int64_t vocab;
    int top_k;
    float rw[4];            // per-slot route weight times the routed scale
    int64_t n_base;         // first packed row of blockIdx.y == 0 (tail launches)
    // Saved pre-activations for the backward (null: not written): gu[row,
    // packed column] = the raw gate / up GEMM outputs (times the e4m3 scale),
    // in the packed column order of the weights.
    void* gu;
    int64_t ldgu;
    // Fused RMSNorm (the weights hold W * norm_weight per input column): the
    // gate and up accumulators of token t are multiplied by row_scale[t]
    // before the SwiGLU.  row_scale == nullptr and rms_eps > 0: the decode
    // kernels compute 1 / sqrt(mean(x_t^2) + rms_eps) themselves.
    const float* row_scale;
    float rms_eps;
    // Fragment-major copy of w (trmoe_pack_fragments) for the decode kernels,
    // or null: bf16/f32 weights, K groups of 64 bytes per 16-row block.
    const void* w_frag;
    // Expert-grouped mode (offsets != nullptr): blockIdx.x walks the
    // (expert, row tile) pairs of a K1 partition; A rows are
    // a[gather[r] % gather_mod] (contiguous partition rows r when gather is
    // null); the weights and their scales advance by w_expert_stride
    // elements and scale_expert_stride floats per expert; output rows are
    // partition rows.
    const int32_t* offsets;
    int E;
    const int64_t* gather;
    int64_t gather_mod;
    int64_t w_expert_stride;
    int64_t scale_expert_stride;
    // Block-scaled e4m3 h (W8A8 with launch_gate_up_a8 only; null: h is
    // bf16): h holds e4m3 codes (row stride ldh bytes) and hs one E8M0
    // exponent per token and 32 features (row stride ldhs bytes).
    void* hs;
    int64_t ldhs;
};

struct DownArgs {
    const void* h;
    int64_t ldh;
    int64_t M;
    int K;
    const void* w;
    int64_t ldw;
    const float* w_scale;
    int N;
    const void* y;
    int64_t ldy;
    const int64_t* inverse;
    int top_k;
    float rw[4];
    float shared_scale;
    float routed_scale;
    const void* residual;
    int64_t ldr;
    void* out;
    int64_t ldo;
    int vec_ok;             // y / residual / out rows 16-byte aligned (vector epilogue)
    const void* w_frag;     // fragment-major copy of w for the decode kernels, or null
    // Expert-grouped mode (offsets != nullptr): blockIdx.x walks the
    // (expert, row tile) pairs of a K1 partition; A rows are
    // a[gather[r] % gather_mod] (contiguous partition rows r when gather is
    // null); the weights and their scales advance by w_expert_stride
    // elements and scale_expert_stride floats per expert; output rows are
    // partition rows.
    const int32_t* offsets;
    int E;
    const int64_t* gather;
    int64_t gather_mod;
    int64_t w_expert_stride;
    int64_t scale_expert_stride;
    // Block-scaled e4m3 h (launch_down_combine_a8 only): h holds e4m3 codes
    // (row stride ldh bytes), hs one E8M0 exponent per token and 32 K values
    // (row stride ldhs bytes, a multiple of 4).
    const void* hs;
    int64_t ldhs;
};

struct RoutedArgs {
    const void* x;
    int64_t ldx;
    int64_t n_tokens;
    int K;                 // hidden
    const int64_t* sorted;
    const int32_t* offsets;
    int E;
    const void* wgu;       // [E, 2*F_pad, wgu_ld]
    int64_t wgu_ld;
    const float* sgu;      // [E, 2*F_pad] or null
    const void* wd;        // [E, H_pad, wd_ld]
    int64_t wd_ld;
    const float* sd;       // [E, H_pad] or null
    int w_elem_bytes;
    int F_pad;             // expert width rounded up to 64
    int W;                 // expert width (down K)
    int H;                 // output columns
    int H_pad;             // packed down rows per expert: H rounded up to 256
    void* y;
    int64_t ldy;
};

struct CombineArgs {
    int64_t M, N;
    const void* y;
    int64_t ldy;
    const int64_t* inverse;
    int top_k;
    float rw[4];
    float routed_scale;
    const void* residual;
    int64_t ldr;
    void* out;
    int64_t ldo;
};

// Token counts at or below this run the decode-shape kernels (trmoe_skinny.hip).
constexpr int64_t kSkinnyMaxTokens = 128;

// Backward of the SwiGLU block: per (row, feature), with g|u recomputed
// from x and dh = dout . W_down^T:
//   dg = dh*m*u*silu'(g), du = dh*m*silu(g), hm = m*silu(g)*u
// where m is the feature's multiplier (shared_mult for shared features; the
// token's route weight times the routed scale for dense-routed expert
// features; rw[slot of the partition row] in grouped mode).  dg|du are
// written in the packed gate|up column order (32 gate then 32 up columns per
// 32-feature block), hm in feature order.
struct SwigluBwdArgs {
    const void* x;
    int64_t ldx;
    const void* dout;
    int64_t ldd;
    int64_t M;               // output rows (tokens, or partition rows when grouped)
    int64_t x_rows;          // rows of x and dout (buffer range)
    int K;                   // hidden
    const void* wgu;         // packed gate|up rows [2F, K]
    int64_t ldwgu;
    const void* wdt;         // W_down^T rows [F, K]
    int64_t ldwdt;
    const void* gu;          // saved gate|up pre-activations [M, 2F] (null: recomputed from x)
    int64_t ldgu;
    int64_t F;               // features (per expert when grouped)
    int64_t f_base;          // first feature of the launch (the features below it run elsewhere)
    void* dgu;
    int64_t lddgu;
    void* hm;                // may be null
    int64_t ldhm;
    float shared_mult;
    int64_t shared_feats;    // dense-routed: features at or past it are experts'
    int64_t expert_feats;
    const int64_t* ids;      // dense-routed routes (null: no routed features)
    const int64_t* table;
    int64_t vocab;
    int top_k;
    float rw[4];             // per-slot route weight times the routed scale
    const int32_t* offsets;  // grouped mode
    int E;
    const int64_t* gather;
    int64_t gather_mod;
    int64_t wgu_expert_stride;   // elements
    int64_t wdt_expert_stride;
};

// Token-reduction GEMM: out[e][m][n] = sum over rows t of segment e of
// A[ra(t)][m] * B[rb(t)][n], ra(t) = a_gather ? a_gather[t] % gather_mod : t
// (same for B).  Segment e is [offsets[e], offsets[e+1]) or [0, T) without
// offsets.  Each segment is split over `splits` workgroups whose fp32
// partials are summed in split order by a second launch.
struct WgradArgs {
    const void* a;
    int64_t lda;
    int64_t a_rows;
    const void* b;
    int64_t ldb;
    int64_t b_rows;
    const int64_t* a_gather;
    const int64_t* b_gather;
    int64_t gather_mod;
    int64_t M, N;
    int64_t T;
    const int32_t* offsets;
    int E;
    int splits;
    void* out;
    int64_t ldo;
    int64_t out_expert_stride;   // elements
    float* partial;              // [E][splits][M][N] when splits > 1
    // Destination map of the summed tile (E == 1, through the reduction):
    // 0 none (out[m * ldo + n]); 1 rows: out[map_off[m] + n * map_stride[m]];
    // 2 columns: out[map_off[n] + m * map_stride[n]]; negative offsets skip,
    // and so do destinations outside [0, out_elems).
    int map_mode;
    const int64_t* map_off;
    const int64_t* map_stride;
    int64_t out_elems;
};

int launch_pack(const PackArgs& p, hipStream_t stream);
int launch_gate_up_skinny(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream);
size_t down_skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, int act);
int launch_stream_read(const void* src, int64_t bytes, uint32_t* sink, int blocks, hipStream_t stream);
int launch_down_skinny(int act, int wdt, const DownArgs& a, void* workspace, hipStream_t stream);
int launch_gate_up(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream);
// Fragment-major copy of a packed [rows, ld] weight (rows % 16 == 0):
// block (r / 16, K group g of 64 bytes) is 1 KiB at (r/16 * G + g) * 1024,
// laid out [16-byte chunk q][row r % 16][16 bytes], zeros past kbytes.
int launch_pack_fragments(const void* src, int64_t rows, int64_t kbytes, int64_t ld_bytes, void* dst,
                          hipStream_t stream);
// row_scale[t] = 1 / sqrt(mean_k x[t, k]^2 + eps) in fp32 for t < n.
// W8A8 shared gate|up (persistent stream, e4m3 MFMA): a.x e4m3 codes with row
// stride a.ldx bytes, a.row_scale their per-token scales, a.w e4m3 packed
// weights with a.w_scale; needs a.K % 128 == 0 and whole 256-row column tiles.
int launch_gate_up_a8(const GateUpArgs& a, int64_t packed_rows, hipStream_t stream);
// K4 on block-scaled e4m3 h and e4m3 weights (the e4m3 MFMA with one E8M0
// scale per 32 K values of each row of h); K a multiple of 128.
int launch_down_combine_a8(const DownArgs& a, hipStream_t stream);
int launch_rms_row_scale(int act, const void* x, int64_t n, int64_t hidden, int64_t ldx, float eps, float* row_scale,
                         hipStream_t stream);
// RMSNorm with its backward (trmoe_norm.hip): y = T(x * r) * w with r saved;
// dx = r (dy w) - (r^3 / H) ((dy w) . x) x (+ dres); dw from one fp32 partial
// per backward workgroup (rmsnorm_groups(n) of them) summed in order.
int rmsnorm_groups(int64_t n);
// Per-row e4m3 codes and scales (scale = amax / 448) of x[n, k] (trmoe_norm.hip).
int launch_quantize_rows_e4m3(int act, const void* x, int64_t n, int64_t k, int64_t ldx, void* q, int64_t ldq,
                              float* scale, hipStream_t stream);
int64_t rmsnorm_max_hidden(int act);
int launch_rmsnorm_forward(int act, const void* x, int64_t n, int64_t hidden, int64_t ldx, const void* w, float eps,
                           void* y, int64_t ldy, float* rs, hipStream_t stream);
int launch_rmsnorm_backward(int act, const void* x, int64_t ldx, const void* w, const float* rs, const void* dy,
                            int64_t lddy, const void* dres, int64_t lddres, int64_t n, int64_t hidden, void* dx,
                            int64_t lddx, void* dw, float* part, hipStream_t stream);
int launch_down_combine(int act, int wdt, const DownArgs& a, hipStream_t stream);
int routed_lds_bytes(int act, int64_t f_pad);
int launch_routed(int act, int wdt, const RoutedArgs& a, int64_t assignments, hipStream_t stream);
// Grouped gate|up (a.offsets set) over `assignments` partition rows.
int launch_gate_up_grouped(int act, int wdt, const GateUpArgs& a, int64_t assignments, int64_t packed_rows,
                           hipStream_t stream);
// Grouped down (a.offsets set): out rows = partition rows, no combine.
int launch_down_grouped(int act, int wdt, const DownArgs& a, int64_t assignments, hipStream_t stream);
// Backward (trmoe_backward.hip).  Grouped swiglu_bwd walks `assignments`
// partition rows; wgrad_splits picks the split count for a workspace of
// `workspace_bytes` (0: as many as the heuristic wants).
int launch_swiglu_bwd(int act, const SwigluBwdArgs& a, int64_t assignments, hipStream_t stream);
int wgrad_splits(int64_t M, int64_t N, int E, int64_t rows_per_segment);
int launch_wgrad(int act, const WgradArgs& a, hipStream_t stream);
int launch_combine(int act, const CombineArgs& a, hipStream_t stream);

}  // namespace trmoe
