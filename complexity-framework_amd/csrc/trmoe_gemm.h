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

int launch_pack(const PackArgs& p, hipStream_t stream);
int launch_gate_up_skinny(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream);
size_t down_skinny_workspace_bytes(int64_t M, int64_t N, int64_t K, int act);
int launch_down_skinny(int act, int wdt, const DownArgs& a, void* workspace, hipStream_t stream);
int launch_gate_up(int act, int wdt, const GateUpArgs& a, int64_t packed_rows, hipStream_t stream);
int launch_down_combine(int act, int wdt, const DownArgs& a, hipStream_t stream);
int routed_lds_bytes(int act, int64_t f_pad);
int launch_routed(int act, int wdt, const RoutedArgs& a, int64_t assignments, hipStream_t stream);
// Grouped gate|up (a.offsets set) over `assignments` partition rows.
int launch_gate_up_grouped(int act, int wdt, const GateUpArgs& a, int64_t assignments, int64_t packed_rows,
                           hipStream_t stream);
// Grouped down (a.offsets set): out rows = partition rows, no combine.
int launch_down_grouped(int act, int wdt, const DownArgs& a, int64_t assignments, hipStream_t stream);
int launch_combine(int act, const CombineArgs& a, hipStream_t stream);

}  // namespace trmoe
