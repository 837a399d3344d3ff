/*
 * trmoe.h -- C ABI of the MI355X (gfx950) TR-MoE feed-forward kernels.
 *
 * One layer of the reference's TRHashEngine forward
 * (complexity/tr_hash/engine.py:534-579) is
 *
 *     out = shared_scale * shared_swiglu(x) + routed_scale * routed(x, ids)
 *
 * and this library computes it with four kernel families:
 *
 *   K1 trmoe_route_sort          route gather + counting partition
 *   K2 trmoe_shared_gate_up      shared SwiGLU gate|up GEMM, SwiGLU epilogue
 *   K3 trmoe_routed_experts      grouped expert MLP over the partition
 *   K4 trmoe_shared_down_combine shared down GEMM with the weighted
 *                                un-permute of K3's rows fused in its epilogue
 *      trmoe_combine             the same un-permute when shared_width == 0
 *
 * Conventions (every entry point):
 *   - device pointers are plain, caller-owned and stay valid until the work
 *     queued on `stream` (a hipStream_t, NULL = default stream) completes;
 *   - the library never allocates or frees device memory; scratch is passed
 *     in (see *_workspace_bytes);
 *   - work is enqueued asynchronously on `stream`; no call synchronises;
 *   - kernels launch on the calling thread's current HIP device: `stream`
 *     and every pointer must belong to that device (make it current with
 *     hipSetDevice first);
 *   - the return value is a trmoe_status; on failure trmoe_last_error()
 *     returns a message that stays valid until the calling thread's next
 *     call into the library;
 *   - tensors are row-major with the element strides given (ld*);
 *   - activation rows (x, h) start 16-byte aligned, their stride is a multiple
 *     of 16 bytes, and when hidden*elem is not a multiple of 16 the elements
 *     up to the next multiple of 16 bytes are zero: the kernels read whole
 *     16-byte chunks through buffer loads (out-of-range chunks read as zero).
 *
 * Weights are consumed in a packed layout produced on the device by
 * trmoe_pack_weight() (see trmoe_pack_dims()).
 */
#ifndef TRMOE_H
#define TRMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRMOE_ABI_VERSION 1

enum trmoe_status {
    TRMOE_OK = 0,
    TRMOE_ERR_INVALID = 1,      /* bad argument (shape, pointer, enum)   */
    TRMOE_ERR_UNSUPPORTED = 2,  /* valid but not implemented here         */
    TRMOE_ERR_HIP = 3           /* a HIP runtime call or launch failed    */
};

enum trmoe_dtype {
    TRMOE_F32 = 0,
    TRMOE_BF16 = 1,
    TRMOE_FP8_E4M3 = 2          /* OCP float8_e4m3fn, weights only        */
};

enum trmoe_order {
    /* segment order (expert, token): the reference's fused GPU partition,
     * complexity_cuda/triton_token_routed.py:211-277 */
    TRMOE_ORDER_TOKEN = 0,
    /* segment order (expert, slot*N + token): the reference's stable CPU
     * sort, triton_token_routed.py:2320-2351 (and CGGR, :69-93) */
    TRMOE_ORDER_ASSIGNMENT = 1
};

enum trmoe_pack_kind {
    /* two [out, in] sources interleaved in groups of 32 output rows
     * (gate rows 0..31, up rows 0..31, gate rows 32..63, ...) so that one
     * GEMM tile holds gate and up of the same features */
    TRMOE_PACK_GATE_UP = 0,
    /* one [out, in] source */
    TRMOE_PACK_PLAIN = 1
};

/* Library ABI version (TRMOE_ABI_VERSION it was built with). */
int trmoe_abi_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* trmoe_last_error(void);

/* 1 if the current HIP device is a gfx950 the kernels were built for. */
int trmoe_device_supported(void);

/*
 * Packed weight geometry.  For `kind` GATE_UP, `out_features` is the width of
 * each of the two sources (shared or expert width) and the packed tensor has
 * *rows = 2 * round_up(out_features, row_align / 2) rows; for PLAIN,
 * *rows = round_up(out_features, row_align).  *cols = round_up(in_features, 8).
 * row_align must be a positive multiple of 64.
 */
int trmoe_pack_dims(int kind, int64_t out_features, int64_t in_features, int64_t row_align,
                    int64_t* rows, int64_t* cols);

/*
 * Pack `groups` weight matrices (one per expert; 1 for shared weights) into
 * dst[groups][rows][cols] (dtype `dtype`, rows/cols from trmoe_pack_dims).
 * Source element (g, o, i) is read at src[g*s_group + o*s_out + i*s_in]
 * (element strides), which covers nn.Linear weights [out, in]
 * (s_out=in, s_in=1) and the reference's expert tensors [E, in, out]
 * (s_out=1, s_in=out) without a host transpose.  src_b is the up source for
 * GATE_UP (NULL for PLAIN).  For TRMOE_FP8_E4M3, src_* hold e4m3 codes and
 * scale_a/scale_b hold per-output-channel float scales at
 * scale[g*scale_group_stride + o]; dst_scale[groups][rows] receives them in
 * packed row order.  For other dtypes the scale pointers must be NULL.
 * dst_ld / dst_group_stride / dst_scale_group_stride (elements; 0 = dense
 * defaults cols / rows*dst_ld / rows) let a group land inside a larger
 * packed tensor, as the dense-routed layout below requires.
 * Reference tensors: engine.py:127-163 (expert_gate/up [E,H,W], expert_down
 * [E,W,H], shared_* nn.Linear).
 */
int trmoe_pack_weight(int kind, int dtype, const void* src_a, const void* src_b, int64_t groups,
                      int64_t out_features, int64_t in_features, int64_t s_group, int64_t s_out,
                      int64_t s_in, const float* scale_a, const float* scale_b,
                      int64_t scale_group_stride, int64_t row_align, void* dst, int64_t dst_ld,
                      int64_t dst_group_stride, float* dst_scale, int64_t dst_scale_group_stride,
                      void* stream);

/*
 * K1 -- replaces sort_pair_hash_by_expert (triton_token_routed.py:2205-2351)
 * and the route gather TRHashEngine._routes (engine.py:316-318).
 *
 * token_ids int64[n] are clamped to [0, vocab-1]; route_table int64[k, vocab]
 * is the (active) persisted table.  Assignment a = slot*n + t.  Outputs:
 *   routes         int64[k, n]   (may be NULL) routes[s, t] = table[s, id_t]
 *   sorted_indices int64[k*n]    assignment at each partition position
 *   inverse        int64[k*n]    inverse[sorted_indices[r]] = r
 *   expert_offsets int32[E+1]    segment starts, offsets[E] = k*n
 *   expert_counts  int32[E]
 * 1 <= num_experts <= 16, top_k in {1, 2, 4}, top_k <= num_experts, entries of
 * the table in [0, num_experts) (entries outside are clamped into it, so no
 * write leaves the outputs).  A token's slots may name one expert twice:
 * every assignment has its own partition row, and the token order breaks
 * (expert, token) ties by slot.  workspace: per-block histograms,
 * trmoe_route_sort_workspace_bytes() (at most 256 blocks x num_experts int32;
 * 0 when one block takes every assignment).
 */
size_t trmoe_route_sort_workspace_bytes(int64_t n_tokens, int top_k, int num_experts, int order);
int trmoe_route_sort(const int64_t* token_ids, int64_t n_tokens, const int64_t* route_table,
                     int64_t vocab_size, int top_k, int num_experts, int order, int64_t* routes,
                     int64_t* sorted_indices, int64_t* inverse, int32_t* expert_offsets,
                     int32_t* expert_counts, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * K1 without a workspace argument.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, validation and results as trmoe_route_sort, bit for bit; the
 * caller still passes the inputs and outputs.  The per-block histograms of
 * the multi-block partition live in a file-scope device array of
 * TRMOE_ROUTE_SORT_NOALLOC_SCRATCH_BYTES (256 blocks x 16 experts of int32),
 * one copy per GPU held until the process ends; a partition that would need
 * more is rejected with TRMOE_ERR_INVALID (the block split never asks for
 * more).  The call allocates and frees nothing; its first call on a device
 * looks up that device's copy of the array.  Every call on one GPU shares
 * that GPU's array, which keeps the last call's contents (nothing in it must
 * start at zero): calls ordered on one stream are safe, calls that overlap
 * on one GPU (unordered streams) race.
 */
#define TRMOE_ROUTE_SORT_NOALLOC_SCRATCH_BYTES 16384
int trmoe_route_sort_noalloc(const int64_t* token_ids, int64_t n_tokens, const int64_t* route_table,
                             int64_t vocab_size, int top_k, int num_experts, int order, int64_t* routes,
                             int64_t* sorted_indices, int64_t* inverse, int32_t* expert_offsets,
                             int32_t* expert_counts, void* stream);

/*
 * K2 -- shared SwiGLU first half; replaces the two nn.Linear calls and
 * _silu_mul of TRHashEngine._shared (engine.py:333-349).
 *
 * x[n, hidden] (act_dtype, row stride ldx) times the GATE_UP-packed
 * [shared_gate; shared_up] weights (w_dtype, pack row_align 256):
 *     h[t, f] = silu(x_t . Wg_f) * (x_t . Wu_f)      f < round_up(S, 128)
 * h is act_dtype with row stride ldh >= round_up(S, 128); the padding columns
 * are written as zero.  (act, w) dtypes: (F32, F32), (BF16, BF16),
 * (BF16, FP8_E4M3) with w_scale = the packed scales.
 */
int trmoe_shared_gate_up(int act_dtype, int w_dtype, const void* x, int64_t n_tokens,
                         int64_t hidden, int64_t ldx, const void* w_packed, const float* w_scale,
                         int64_t shared_width, void* h, int64_t ldh, void* stream);

/*
 * K2+K3 fused, "dense-routed" strategy (for expert widths small against the
 * shared width).  The packed gate|up weights hold the shared features
 * (round_up(S, 128)) followed by every expert's features (round_up(W, 64)
 * each), all GATE_UP-interleaved over round_up(hidden, 8) columns, with
 * 2 * trmoe_dense_routed_features() rows.  For token t and feature f:
 *     shared f:           h[t, f] = shared_scale * silu(g) * u
 *     expert e, slot j:   h[t, f] = routed_scale * sum_j w_j [route_j(t) == e] * silu(g) * u
 * so that one trmoe_shared_down_combine() over h with the matching packed
 * down weights (shared_down.weight columns, then each expert's down^T) and
 * shared_scale = 1, no y, is the whole layer: the masked dense expert loop
 * of the reference's universal path (engine.py:66-104) inside the shared
 * GEMMs.  Routes are gathered from route_table[k, vocab] with clamped ids.
 */
int64_t trmoe_dense_routed_features(int64_t shared_width, int num_experts, int64_t expert_width);
int trmoe_dense_routed_gate_up(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                               int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                               int num_experts, int64_t expert_width, const int64_t* token_ids,
                               const int64_t* route_table, int64_t vocab_size, int top_k,
                               const float* route_weights, float shared_scale, float routed_scale, void* h,
                               int64_t ldh, void* stream);

/*
 * K3 -- routed experts; replaces hash_cggr_grouped_gemm (gate, up),
 * fused_swiglu and cggr_grouped_gemm (down) of the reference's fused path
 * (triton_token_routed.py:1033-1342, engine.py:485-507).
 *
 * For every partition position r of expert e (expert_offsets from K1):
 *     t = sorted_indices[r] mod n_tokens
 *     y[r, :] = (silu(x_t . Wg_e) * (x_t . Wu_e)) . Wd_e
 * w_gate_up: GATE_UP-packed expert gate/up, groups = E, row_align 128;
 * w_down: PLAIN-packed transposed expert down ([E, hidden, width] view of the
 * reference's [E, width, hidden]), row_align 256.  y is act_dtype [k*n, ldy].
 * `num_experts` is the active expert count; `expert_width` the active width.
 *
 * workspace: device scratch of trmoe_routed_experts_workspace_bytes() bytes.
 * With it the experts run as two grouped GEMMs (gate|up + SwiGLU into the
 * workspace, then down), each tiled over 256-row tiles of every expert
 * segment; with NULL (or fewer bytes) one fused kernel keeps each tile's
 * SwiGLU output in LDS instead.  Both give the same results to rounding.
 */
size_t trmoe_routed_experts_workspace_bytes(int act_dtype, int64_t n_assignments, int64_t expert_width);
int trmoe_routed_experts(int act_dtype, int w_dtype, const void* x, int64_t n_tokens,
                         int64_t hidden, int64_t ldx, const int64_t* sorted_indices,
                         const int32_t* expert_offsets, int num_experts, int top_k,
                         const void* w_gate_up, const float* s_gate_up, const void* w_down,
                         const float* s_down, int64_t expert_width, void* y, int64_t ldy,
                         void* workspace, size_t workspace_bytes, void* stream);

/*
 * K4 -- shared down GEMM + weighted un-permute + combine; replaces
 * shared_down, pair_hash_reduce / pair_hash_weighted_reduce
 * (triton_token_routed.py:280-330, 376-435) and the final
 * `shared_scale*shared + routed_scale*routed` (engine.py:578).
 *
 *     out[t, c] = shared_scale * (h_t . Wd_c)
 *               + routed_scale * sum_j route_weights[j] * y[inverse[j*n + t], c]
 *               (+ residual[t, c] when residual != NULL)
 * h: K2's output (act_dtype, [n, ldh], K = round_up(S, 128));
 * w_down: PLAIN-packed shared_down.weight [hidden, S] (row_align 256).
 * y/inverse may be NULL (no routed term).  route_weights: top_k host floats.
 *
 * workspace: device scratch of trmoe_shared_down_combine_workspace_bytes()
 * bytes (may be NULL when that is 0).  Decode-sized calls (n_tokens <= 128)
 * split K across workgroups, write fp32 partials there and sum them in split
 * order in a second launch, so results do not depend on scheduling.  With a
 * smaller workspace the call runs the tile kernel instead.  Calls that share
 * a workspace must be ordered on one stream.
 */
size_t trmoe_shared_down_combine_workspace_bytes(int act_dtype, int64_t n_tokens, int64_t shared_width,
                                                 int64_t hidden);
int trmoe_shared_down_combine(int act_dtype, int w_dtype, const void* h, int64_t n_tokens,
                              int64_t shared_width, int64_t ldh, const void* w_down,
                              const float* w_scale, int64_t hidden, const void* y, int64_t ldy,
                              const int64_t* inverse, int top_k, const float* route_weights,
                              float shared_scale, float routed_scale, const void* residual,
                              int64_t ldr, void* out, int64_t ldo, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * K4 without a shared branch (shared_width == 0, engine.py:335):
 *     out[t, c] = routed_scale * sum_j route_weights[j] * y[inverse[j*n+t], c]
 *                 (+ residual[t, c])
 */
int trmoe_combine(int act_dtype, int64_t n_tokens, int64_t hidden, const void* y, int64_t ldy,
                  const int64_t* inverse, int top_k, const float* route_weights,
                  float routed_scale, const void* residual, int64_t ldr, void* out, int64_t ldo,
                  void* stream);

/* ---------------------------------------------------------------------------
 * Block MLP with the post-attention RMSNorm fused (F2; replaces, in
 * complexity/models/block.py:271-278, `post_attention_layernorm` (RMSNorm,
 * complexity/core/normalization/norms.py:46-55) feeding the MLP, as
 * fused_rmsnorm_gate_up does in complexity_cuda/fused_mlp.py:362-428).
 *
 *     rmsnorm(x)_t = x_t * r_t * norm_weight,   r_t = 1 / sqrt(mean_k x_t,k^2 + eps)
 *
 * norm_weight scales input channels, so it is folded into the gate/up
 * weights once (pack W * norm_weight[None, :], expert weights along their
 * input axis) and r_t multiplies token t's gate and up accumulators before
 * the SwiGLU.  The *_rms entry points are the ones above with that scale:
 *   row_scale != NULL: r from trmoe_rms_row_scale (fp32 [n_tokens]);
 *   row_scale == NULL: eps > 0 and n_tokens <= 128 -- the decode kernels sum
 *   the squares of the activation rows they stage anyway (no extra launch).
 * The residual add is trmoe_shared_down_combine's `residual` (x itself).
 * ------------------------------------------------------------------------- */
int trmoe_rms_row_scale(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx, float eps,
                        float* row_scale, void* stream);
int trmoe_shared_gate_up_rms(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                             int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                             const float* row_scale, float eps, void* h, int64_t ldh, void* stream);
int trmoe_dense_routed_gate_up_rms(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                                   int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                                   int num_experts, int64_t expert_width, const int64_t* token_ids,
                                   const int64_t* route_table, int64_t vocab_size, int top_k,
                                   const float* route_weights, float shared_scale, float routed_scale,
                                   const float* row_scale, float eps, void* h, int64_t ldh, void* stream);
/* ---------------------------------------------------------------------------
 * RMSNorm for training (and for the fp8 layers, whose packs cannot take the
 * norm weight).  Replaces RMSNorm.forward (complexity/core/normalization/
 * norms.py:46-55), which on CUDA calls liger-kernel's RMSNorm
 * (LigerRMSNormFunction.apply(x, weight, eps, 0.0, "llama", False);
 * pyproject.toml pins liger-kernel>=0.5.0), with its autograd backward:
 *
 *   r_t = 1 / sqrt(mean_k x_t,k^2 + eps)       (fp32, saved to row_scale)
 *   y_t,k = T(x_t,k * r_t) * w_k               (rounded to T twice, "llama")
 *   dx_t,k = r_t m_t,k - (r_t^3 / hidden) (sum_j m_t,j x_t,j) x_t,k [+ dres_t,k],
 *            m = dy * w
 *   dw_k = sum_t dy_t,k * T(x_t,k * r_t)       (fp32 partials summed in a
 *                                               fixed order: deterministic)
 *
 * act_dtype f32 or bf16 for x, weight, y, dy, dres, dx and dweight alike;
 * rows 16-byte aligned, strides multiples of 16 bytes, hidden a multiple of
 * 16 bytes of elements and at most 4096 (bf16) / 2048 (f32).  dres (NULL:
 * none) is added to dx and may be dx itself (same stride).  workspace: device
 * scratch of trmoe_rmsnorm_backward_workspace_bytes() bytes.
 * ------------------------------------------------------------------------- */
int trmoe_rmsnorm_forward(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                          const void* weight, float eps, void* y, int64_t ldy, float* row_scale, void* stream);
size_t trmoe_rmsnorm_backward_workspace_bytes(int act_dtype, int64_t n_tokens, int64_t hidden);
int trmoe_rmsnorm_backward(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                           const void* weight, const float* row_scale, const void* dy, int64_t lddy,
                           const void* dres, int64_t lddres, void* dx, int64_t lddx, void* dweight,
                           void* workspace, size_t workspace_bytes, void* stream);
/* ---------------------------------------------------------------------------
 * W8A8 shared gate|up: e4m3 activations with per-token scales on the e4m3
 * MFMA.  No counterpart in the reference, which has no fp8 path: this is the
 * e4m3-activation form of trmoe_shared_gate_up (the shared_gate/shared_up
 * linears and silu*mul, complexity/tr_hash/engine.py:333-349) for layers
 * whose weights are e4m3 already (trmoe_pack_weight with TRMOE_FP8_E4M3).
 *
 * trmoe_quantize_rows_e4m3: for each row t of x (f32 or bf16, k a multiple
 *   of 16 bytes of elements, at most 4096 bf16 / 2048 f32)
 *     scale_t = amax_k |x_t,k| / 448   (1 when that is 0, or the row holds a NaN)
 *     q_t,k   = e4m3(clamp(x_t,k / scale_t, -448, 448)), round to nearest even
 *   -- the weights' per-output-channel quantizer applied to token rows.
 * trmoe_shared_gate_up_a8: h (bf16) = silu(g) * u with
 *     [g | u]_t,c = scale_t * w_scale_c * sum_k q_t,k * W8_c,k
 *   hidden a multiple of 128; x_q rows 16-byte aligned (ldxq bytes apart, a
 *   multiple of 16); h as for trmoe_shared_gate_up.
 * ------------------------------------------------------------------------- */
int trmoe_quantize_rows_e4m3(int act_dtype, const void* x, int64_t n_rows, int64_t k, int64_t ldx, void* q,
                             int64_t ldq, float* scale, void* stream);
int trmoe_shared_gate_up_a8(const void* x_q, const float* x_scale, int64_t n_tokens, int64_t hidden, int64_t ldxq,
                            const void* w_packed, const float* w_scale, int64_t shared_width, void* h, int64_t ldh,
                            void* stream);
/* ---------------------------------------------------------------------------
 * W8A8 shared down on block-scaled e4m3 h.  No counterpart in the reference
 * (no fp8 path there): the e4m3-activation forms of trmoe_shared_gate_up's h
 * and of trmoe_shared_down_combine (shared_down and the combine,
 * complexity/tr_hash/engine.py:333-349, 578), for layers with e4m3 weights.
 *
 * trmoe_shared_gate_up_a8_mx: h as in trmoe_shared_gate_up_a8 (in fp32),
 *   written as e4m3 codes with one power-of-two scale per token and block of
 *   32 features, b = f / 32:
 *     e_t,b  = the smallest integer with max_{f in b} |h_t,f| <= 448 * 2^e,
 *              clamped to [-126, 126]; 0 when that maximum is 0 or not
 *              finite
 *     h_q    = e4m3(h * 2^-e), round to nearest even, clamped to +-448
 *     h_scale[t * ldhs + b] = e + 127 (E8M0)
 *   h_q: [n, ldhq] bytes, ldhq a multiple of 16 and >= round_up(S, 128),
 *   16-byte aligned; the padding features are written as code 0, scale 127.
 *   h_scale: [n, ldhs] bytes, ldhs a multiple of 4 and >= round_up(S, 128)/32.
 * trmoe_shared_down_combine_a8: trmoe_shared_down_combine (bf16 y, residual
 *   and out) with h = h_q * 2^(h_scale - 127) per block, on the e4m3 MFMA
 *   with the block scales in its operand: S a multiple of 128, w_down the
 *   PLAIN-packed e4m3 shared_down.weight with its per-row scales w_scale.
 * ------------------------------------------------------------------------- */
int trmoe_shared_gate_up_a8_mx(const void* x_q, const float* x_scale, int64_t n_tokens, int64_t hidden, int64_t ldxq,
                               const void* w_packed, const float* w_scale, int64_t shared_width, void* h_q,
                               int64_t ldhq, void* h_scale, int64_t ldhs, void* stream);
int trmoe_shared_down_combine_a8(const void* h_q, const void* h_scale, int64_t n_tokens, int64_t shared_width,
                                 int64_t ldhq, int64_t ldhs, const void* w_down, const float* w_scale, int64_t hidden,
                                 const void* y, int64_t ldy, const int64_t* inverse, int top_k,
                                 const float* route_weights, float shared_scale, float routed_scale,
                                 const void* residual, int64_t ldr, void* out, int64_t ldo, void* stream);
/* row_scale required; the workspace of trmoe_routed_experts_workspace_bytes() too. */
int trmoe_routed_experts_rms(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                             int64_t ldx, const int64_t* sorted_indices, const int32_t* expert_offsets,
                             int num_experts, int top_k, const void* w_gate_up, const float* s_gate_up,
                             const void* w_down, const float* s_down, int64_t expert_width, const float* row_scale,
                             void* y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Fragment-major weights for decode-sized calls (no reference counterpart:
 * a second layout of the same packed weights).
 *
 * A 16x16x32 MFMA operand is 16 rows x 64 bytes.  trmoe_pack_fragments
 * copies a packed [rows, ld] weight (rows % 16 == 0; bf16/f32) so that each
 * such fragment is 1 KiB contiguous:
 *     dst[((r / 16) * G + k / 64) * 1024 + ((k % 64) / 16) * 256 + (r % 16) * 16 + k % 16]
 *         = byte k of packed row r,      G = ceil(cols * elem / 64)
 * with zeros past cols.  The decode kernels (n_tokens <= 128) then load
 * weights with whole-line 1 KiB reads instead of 16 rows x 64 bytes.  cols
 * must be the K of the calls that use it: `hidden` for gate|up packs,
 * `shared_width` (the value passed to trmoe_shared_down_combine_ex) for down
 * packs.  The copy doubles the weight memory of the layers that keep it.
 * ------------------------------------------------------------------------- */
size_t trmoe_fragment_bytes(int dtype, int64_t rows, int64_t cols);
int trmoe_pack_fragments(int dtype, const void* packed, int64_t rows, int64_t cols, int64_t ld, void* dst,
                         void* stream);

/*
 * Optional extras of the *_ex entry points (all-zero = the plain call):
 *   row_scale / rms_eps: the fused RMSNorm scales of the *_rms entry points
 *                        (gate|up calls only);
 *   w_frag / w_frag_cols: a trmoe_pack_fragments copy of the call's packed
 *                        weights and the cols it was packed with (checked
 *                        against the call's K); used when n_tokens <= 128.
 */
typedef struct trmoe_call_extras {
    const float* row_scale;
    float rms_eps;
    const void* w_frag;
    int64_t w_frag_cols;
} trmoe_call_extras;

int trmoe_shared_gate_up_ex(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                            int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width, void* h,
                            int64_t ldh, const trmoe_call_extras* extras, void* stream);
int trmoe_dense_routed_gate_up_ex(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                                  int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                                  int num_experts, int64_t expert_width, const int64_t* token_ids,
                                  const int64_t* route_table, int64_t vocab_size, int top_k,
                                  const float* route_weights, float shared_scale, float routed_scale, void* h,
                                  int64_t ldh, const trmoe_call_extras* extras, void* stream);
int trmoe_shared_down_combine_ex(int act_dtype, int w_dtype, const void* h, int64_t n_tokens, int64_t shared_width,
                                 int64_t ldh, const void* w_down, const float* w_scale, int64_t hidden, const void* y,
                                 int64_t ldy, const int64_t* inverse, int top_k, const float* route_weights,
                                 float shared_scale, float routed_scale, const void* residual, int64_t ldr, void* out,
                                 int64_t ldo, void* workspace, size_t workspace_bytes,
                                 const trmoe_call_extras* extras, void* stream);

/* ---------------------------------------------------------------------------
 * Backward (bf16 / f32 weights; fp8 weights are inference-only).
 *
 * Together these keep the HIP path differentiable: they replace the autograd
 * of the shared linears and silu*mul (engine.py:333-349) and of the routed
 * branch -- grad-x of HashCGGRGroupedGEMM / CGGRGroupedGEMM through the
 * inverse permutation, PairHashReduce's expand and the unpadded grad-W
 * kernels (triton_token_routed.py:1616-1833, 751-1028).
 * ------------------------------------------------------------------------- */

/*
 * SwiGLU backward.  For every row r and feature f (gate|up either saved by
 * the forward, see gu below, or recomputed from x):
 *     g, u = x_r . Wg_f, x_r . Wu_f          w_gate_up: the forward's GATE_UP pack
 *     dh   = dout_r . Wd[:, f]               w_down_t: W_down^T, PLAIN-packed [F, hidden]
 *     dgu[r, 64*(f/32) + f%32]      = dh * m * u * silu'(g)
 *     dgu[r, 64*(f/32) + 32 + f%32] = dh * m * silu(g)
 *     hm[r, f]                      = m * silu(g) * u      (hm may be NULL)
 * so dgu is the gradient of the gate|up GEMM output in the packed column
 * order and hm the forward's (scaled) SwiGLU output.  dgu/hm are act_dtype;
 * their rows (and gu's) are 16-byte aligned with a stride that is a multiple
 * of 16 bytes, like the activation rows.
 *
 * gu (shared and dense-routed forms; NULL = recompute g|u from x): the raw
 * gate|up outputs the *_gate_up_save forward wrote, [n, ldgu] in the packed
 * column order; the backward then runs one GEMM (dh) instead of three.
 *
 * shared:        rows = tokens, F = round_up(shared_width, 128), m = shared_scale;
 *                w_down_t from shared_down.weight [hidden, S] (out = S rows)
 * dense-routed:  the layout of trmoe_dense_routed_gate_up, F =
 *                trmoe_dense_routed_features(); m as in its forward
 *                (routed_scale * sum_j w_j [route_j(t) == e] on expert e's features);
 *                w_down_t: the dense packed down weight transposed [F, hidden]
 * routed:        rows = K1 partition rows r of expert e; x/dout rows are
 *                sorted_indices[r] mod n_tokens; F = round_up(expert_width, 64)
 *                per expert: w_gate_up the expert GATE_UP pack (row_align 128),
 *                w_down_t the expert down [E, W, hidden] PLAIN-packed per expert
 *                with row_align 64; m = routed_scale * route_weights[sorted_indices[r] / n_tokens]
 */
int trmoe_shared_swiglu_backward(int act_dtype, const void* x, const void* dout, int64_t n_tokens, int64_t hidden,
                                 int64_t ldx, int64_t ldd, const void* w_gate_up, const void* w_down_t,
                                 int64_t shared_width, float shared_scale, const void* gu, int64_t ldgu, void* dgu,
                                 int64_t lddgu, void* hm, int64_t ldhm, void* stream);
int trmoe_dense_routed_swiglu_backward(int act_dtype, const void* x, const void* dout, int64_t n_tokens,
                                       int64_t hidden, int64_t ldx, int64_t ldd, const void* w_gate_up,
                                       const void* w_down_t, int64_t shared_width, int num_experts,
                                       int64_t expert_width, const int64_t* token_ids, const int64_t* route_table,
                                       int64_t vocab_size, int top_k, const float* route_weights,
                                       float shared_scale, float routed_scale, const void* gu, int64_t ldgu,
                                       void* dgu, int64_t lddgu, void* hm, int64_t ldhm, void* stream);
int trmoe_routed_swiglu_backward(int act_dtype, const void* x, const void* dout, int64_t n_tokens, int64_t hidden,
                                 int64_t ldx, int64_t ldd, const int64_t* sorted_indices,
                                 const int32_t* expert_offsets, int num_experts, int top_k, const void* w_gate_up,
                                 const void* w_down_t, int64_t expert_width, const float* route_weights,
                                 float routed_scale, void* dgu, int64_t lddgu, void* hm, int64_t ldhm,
                                 void* stream);

/*
 * Training forwards: trmoe_shared_gate_up / trmoe_dense_routed_gate_up with
 * bf16/f32 weights that also write the raw gate|up GEMM outputs (the
 * pre-activations) to gu [n, ldgu] in the packed column order, ldgu >= twice
 * the feature count; the backward reads them instead of recomputing (the
 * reference's autograd saves the same tensors: the gate and up nn.Linear
 * outputs, engine.py:333-349).  Any n takes the tile kernels.
 */
int trmoe_shared_gate_up_save(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                              const void* w_packed, int64_t shared_width, void* h, int64_t ldh, void* gu,
                              int64_t ldgu, void* stream);
int trmoe_dense_routed_gate_up_save(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                                    const void* w_packed, int64_t shared_width, int num_experts,
                                    int64_t expert_width, const int64_t* token_ids, const int64_t* route_table,
                                    int64_t vocab_size, int top_k, const float* route_weights, float shared_scale,
                                    float routed_scale, void* h, int64_t ldh, void* gu, int64_t ldgu,
                                    void* stream);

/*
 * Weight gradients as token-reduction GEMMs; replaces cggr_grad_w /
 * hash_cggr_grad_w (triton_token_routed.py:751-1028: per expert, no padding,
 * split over tokens) and the grad-W of the shared linears.  For segment e
 * ([expert_offsets[e], expert_offsets[e+1]), or [0, n_rows) when
 * num_segments == 1 and expert_offsets is NULL):
 *     out[e][i, j] = sum over rows t of the segment of a[ra(t), i] * b[rb(t), j]
 * with ra(t) = a_gather ? a_gather[t] mod gather_mod : t (rb likewise), so an
 * operand is read through K1's sorted_indices without a gathered copy.
 * m, n, lda, ldb: multiples of 8; out is act_dtype [m, ldo] per segment,
 * out_expert_stride elements apart.  With a workspace of
 * trmoe_weight_grad_workspace_bytes() each segment is split over several
 * workgroups whose fp32 partials are summed in split order (results do not
 * depend on scheduling); without it one workgroup reduces each tile.
 */
size_t trmoe_weight_grad_workspace_bytes(int act_dtype, int64_t m, int64_t n, int num_segments, int64_t n_rows);
int trmoe_weight_grad(int act_dtype, const void* a, int64_t lda, int64_t a_rows, const void* b, int64_t ldb,
                      int64_t b_rows, const int64_t* a_gather, const int64_t* b_gather, int64_t gather_mod,
                      int64_t m, int64_t n, int64_t n_rows, const int32_t* expert_offsets, int num_segments,
                      void* out, int64_t ldo, int64_t out_expert_stride, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * The same token-reduction GEMM (bf16, one segment, no gathered rows) with
 * its result written straight into the parameters' own layouts, so that no
 * strided copy of the gradient follows it: the grad-W that the reference's
 * autograd hands to AccumulateGrad for the shared linears and the expert
 * tensors (engine.py:333-349, triton_token_routed.py:751-1028), which here
 * arrive as one packed [m, n] product.  The summed fp32 tile goes to
 *     map_mode 1 (rows):    out[map_off[i] + j * map_stride[i]]
 *     map_mode 2 (columns): out[map_off[j] + i * map_stride[j]]
 * in act_dtype elements; a negative map_off skips the row (column), and a
 * destination outside [0, out_elems) is not written (out holds out_elems
 * elements).  The workspace (trmoe_weight_grad_mapped_workspace_bytes) is
 * required.
 */
size_t trmoe_weight_grad_mapped_workspace_bytes(int act_dtype, int64_t m, int64_t n, int64_t n_rows);
int trmoe_weight_grad_mapped(int act_dtype, const void* a, int64_t lda, int64_t a_rows, const void* b, int64_t ldb,
                             int64_t b_rows, int64_t m, int64_t n, int64_t n_rows, int map_mode,
                             const int64_t* map_off, const int64_t* map_stride, void* out, int64_t out_elems,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Grouped plain GEMM over a K1 partition: y[r, :] = h[r, :] . W_e^T for the
 * rows r of expert e, with w PLAIN-packed per expert [E, round_up(out, 256),
 * round_up(k, 8)].  The backward uses it for the data gradient of the routed
 * rows, [dg|du]_r . [Wg_e; Wu_e] (the grad-x half of
 * HashCGGRGroupedGEMM.backward, triton_token_routed.py:1703-1726); the
 * per-token sum over a token's rows is then trmoe_shared_down_combine's /
 * trmoe_combine's un-permute with unit weights.
 */
int trmoe_grouped_linear(int act_dtype, const void* h, int64_t ldh, int64_t n_rows, int64_t k,
                         const int32_t* expert_offsets, int num_experts, const void* w, int64_t out_features,
                         void* y, int64_t ldy, void* stream);

/*
 * Measurement aid with no counterpart in the reference: one kernel launch that
 * reads bytes [src, src + bytes) once with 16-byte loads over sink_words
 * workgroups and writes the XOR of the 32-bit words each workgroup read to
 * sink[workgroup] (the XOR of all sink words is the XOR of the range).  It
 * times the single-launch streaming floor that the decode kernels' weight
 * bytes are compared with.  bytes: a positive multiple of 16, src 16-byte
 * aligned; 1 <= sink_words <= 65535.
 */
int trmoe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int sink_words, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRMOE_H */
