// extern "C" entry points of libtrmoe: argument validation on the host, then
// one launch (or two for the multi-block partition) on the caller's stream.
// Every shape a kernel's grid and indexing assume is checked here first.
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>
#include <set>
#include <string>
#include <utility>

#include "trmoe_common.h"
#include "trmoe_gemm.h"
#include "trmoe_internal.h"

namespace trmoe {

static thread_local std::string g_last_error;

int set_error(int status, const char* msg) {
    g_last_error = msg ? msg : "";
    return status;
}

int set_kernel_lds(const void* kernel, int bytes) {
    if (bytes <= 65536) return TRMOE_OK;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair(kernel, dev);
    if (done.count(key)) return TRMOE_OK;
    hipError_t err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess) return set_error(TRMOE_ERR_HIP, hipGetErrorString(err));
    done.insert(key);
    return TRMOE_OK;
}

int current_device_cus() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cache[kMaxDevices];   // 0 = not yet read
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    const bool cached = dev >= 0 && dev < kMaxDevices;
    if (cached) {
        const int v = cache[dev].load(std::memory_order_relaxed);
        if (v > 0) return v;
    }
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    if (cached) cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

int check_launch(const char* what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        std::string m = std::string(what) + ": " + hipGetErrorString(err);
        return set_error(TRMOE_ERR_HIP, m.c_str());
    }
    return TRMOE_OK;
}

static inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
static inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
static inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int elem_bytes(int dtype) {
    switch (dtype) {
        case TRMOE_F32: return 4;
        case TRMOE_BF16: return 2;
        case TRMOE_FP8_E4M3: return 1;
        default: return 0;
    }
}

// Activation rows are read as whole 16-byte chunks through buffer loads whose
// ranges stay below 2^31 bytes.
static bool rows_ok(const void* p, int64_t ld, int elem) {
    return aligned16(p) && (ld * elem) % 16 == 0 && ld * elem < ((int64_t)1 << 23);
}

static bool valid_pair(int act, int wdt) {
    return (act == TRMOE_F32 && wdt == TRMOE_F32) || (act == TRMOE_BF16 && wdt == TRMOE_BF16) ||
           (act == TRMOE_BF16 && wdt == TRMOE_FP8_E4M3);
}

#define TRMOE_REQUIRE(cond, msg)                                  \
    do {                                                          \
        if (!(cond)) return set_error(TRMOE_ERR_INVALID, (msg));  \
    } while (0)

}  // namespace trmoe

using namespace trmoe;

extern "C" {

int trmoe_abi_version(void) { return TRMOE_ABI_VERSION; }

const char* trmoe_last_error(void) { return g_last_error.c_str(); }

int trmoe_device_supported(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int trmoe_pack_dims(int kind, int64_t out_features, int64_t in_features, int64_t row_align,
                    int64_t* rows, int64_t* cols) {
    TRMOE_REQUIRE(kind == TRMOE_PACK_GATE_UP || kind == TRMOE_PACK_PLAIN, "pack_dims: bad kind");
    TRMOE_REQUIRE(out_features > 0 && in_features > 0, "pack_dims: dimensions must be positive");
    TRMOE_REQUIRE(row_align > 0 && row_align % 64 == 0, "pack_dims: row_align must be a positive multiple of 64");
    TRMOE_REQUIRE(rows != nullptr && cols != nullptr, "pack_dims: null output");
    *rows = (kind == TRMOE_PACK_GATE_UP) ? 2 * round_up(out_features, row_align / 2)
                                         : round_up(out_features, row_align);
    *cols = round_up(in_features, 8);
    return TRMOE_OK;
}

int trmoe_pack_weight(int kind, int dtype, const void* src_a, const void* src_b, int64_t groups,
                      int64_t out_features, int64_t in_features, int64_t s_group, int64_t s_out,
                      int64_t s_in, const float* scale_a, const float* scale_b,
                      int64_t scale_group_stride, int64_t row_align, void* dst, int64_t dst_ld,
                      int64_t dst_group_stride, float* dst_scale, int64_t dst_scale_group_stride,
                      void* stream) {
    int64_t rows = 0, cols = 0;
    int st = trmoe_pack_dims(kind, out_features, in_features, row_align, &rows, &cols);
    if (st) return st;
    TRMOE_REQUIRE(elem_bytes(dtype) > 0, "pack_weight: bad dtype");
    TRMOE_REQUIRE(groups > 0, "pack_weight: groups must be positive");
    TRMOE_REQUIRE(src_a != nullptr && dst != nullptr, "pack_weight: null pointer");
    TRMOE_REQUIRE(kind == TRMOE_PACK_PLAIN || src_b != nullptr, "pack_weight: GATE_UP needs src_b");
    if (dtype == TRMOE_FP8_E4M3) {
        TRMOE_REQUIRE(scale_a != nullptr && dst_scale != nullptr, "pack_weight: fp8 needs scales");
        TRMOE_REQUIRE(kind == TRMOE_PACK_PLAIN || scale_b != nullptr, "pack_weight: fp8 GATE_UP needs scale_b");
    } else {
        TRMOE_REQUIRE(scale_a == nullptr && scale_b == nullptr && dst_scale == nullptr,
                      "pack_weight: scales are only for fp8 weights");
    }
    PackArgs p{};
    p.a = src_a;
    p.b = (kind == TRMOE_PACK_GATE_UP) ? src_b : src_a;
    p.sa = scale_a;
    p.sb = (kind == TRMOE_PACK_GATE_UP) ? scale_b : scale_a;
    p.groups = groups;
    p.out_features = out_features;
    p.in_features = in_features;
    p.s_group = s_group;
    p.s_out = s_out;
    p.s_in = s_in;
    p.scale_group_stride = scale_group_stride;
    p.dst = dst;
    p.dst_scale = dst_scale;
    p.dst_rows = rows;
    p.dst_cols = cols;
    p.dst_ld = dst_ld ? dst_ld : cols;
    p.dst_group_stride = dst_group_stride ? dst_group_stride : rows * p.dst_ld;
    p.dst_scale_group_stride = dst_scale_group_stride ? dst_scale_group_stride : rows;
    TRMOE_REQUIRE(p.dst_ld >= cols, "pack_weight: dst_ld smaller than the packed columns");
    p.interleave = (kind == TRMOE_PACK_GATE_UP);
    p.elem_bytes = elem_bytes(dtype);
    return launch_pack(p, as_stream(stream));
}

size_t trmoe_route_sort_workspace_bytes(int64_t n_tokens, int top_k, int num_experts, int order) {
    if (n_tokens < 0 || top_k < 1 || num_experts < 1) return 0;
    int64_t nb = route_sort_blocks(n_tokens, top_k, order);
    return nb <= 1 ? 0 : (size_t)nb * (size_t)num_experts * sizeof(int32_t);
}

int trmoe_route_sort(const int64_t* token_ids, int64_t n_tokens, const int64_t* route_table,
                     int64_t vocab_size, int top_k, int num_experts, int order, int64_t* routes,
                     int64_t* sorted_indices, int64_t* inverse, int32_t* expert_offsets,
                     int32_t* expert_counts, void* workspace, size_t workspace_bytes,
                     void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0, "route_sort: n_tokens must be non-negative");
    TRMOE_REQUIRE(top_k == 1 || top_k == 2 || top_k == 4, "route_sort: top_k must be 1, 2 or 4");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "route_sort: num_experts must be in [1, 16]");
    TRMOE_REQUIRE(top_k <= num_experts, "route_sort: top_k cannot exceed num_experts");
    TRMOE_REQUIRE(vocab_size > 0, "route_sort: vocab_size must be positive");
    TRMOE_REQUIRE(order == TRMOE_ORDER_TOKEN || order == TRMOE_ORDER_ASSIGNMENT, "route_sort: bad order");
    TRMOE_REQUIRE(route_table != nullptr && expert_offsets != nullptr && expert_counts != nullptr,
                  "route_sort: null pointer");
    TRMOE_REQUIRE(n_tokens == 0 || (token_ids != nullptr && sorted_indices != nullptr && inverse != nullptr),
                  "route_sort: null pointer");
    TRMOE_REQUIRE(n_tokens * top_k < (int64_t)1 << 31, "route_sort: too many assignments");
    return launch_route_sort(token_ids, n_tokens, route_table, vocab_size, top_k, num_experts, order,
                             routes, sorted_indices, inverse, expert_offsets, expert_counts, workspace,
                             workspace_bytes, as_stream(stream));
}

int trmoe_route_sort_noalloc(const int64_t* token_ids, int64_t n_tokens, const int64_t* route_table,
                             int64_t vocab_size, int top_k, int num_experts, int order, int64_t* routes,
                             int64_t* sorted_indices, int64_t* inverse, int32_t* expert_offsets,
                             int32_t* expert_counts, void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0, "route_sort_noalloc: n_tokens must be non-negative");
    TRMOE_REQUIRE(top_k == 1 || top_k == 2 || top_k == 4, "route_sort_noalloc: top_k must be 1, 2 or 4");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts,
                  "route_sort_noalloc: num_experts must be in [1, 16]");
    TRMOE_REQUIRE(top_k <= num_experts, "route_sort_noalloc: top_k cannot exceed num_experts");
    TRMOE_REQUIRE(vocab_size > 0, "route_sort_noalloc: vocab_size must be positive");
    TRMOE_REQUIRE(order == TRMOE_ORDER_TOKEN || order == TRMOE_ORDER_ASSIGNMENT, "route_sort_noalloc: bad order");
    TRMOE_REQUIRE(route_table != nullptr && expert_offsets != nullptr && expert_counts != nullptr,
                  "route_sort_noalloc: null pointer");
    TRMOE_REQUIRE(n_tokens == 0 || (token_ids != nullptr && sorted_indices != nullptr && inverse != nullptr),
                  "route_sort_noalloc: null pointer");
    TRMOE_REQUIRE(n_tokens * top_k < (int64_t)1 << 31, "route_sort_noalloc: too many assignments");
    return launch_route_sort_noalloc(token_ids, n_tokens, route_table, vocab_size, top_k, num_experts, order,
                                     routes, sorted_indices, inverse, expert_offsets, expert_counts,
                                     as_stream(stream));
}

// Fused RMSNorm scales of the *_rms entry points: a row_scale array, or
// (row_scale null) eps > 0 for scales computed by the decode kernels.
static int rms_args_ok(const char* who, const float* row_scale, float eps, int64_t n_tokens) {
    if (row_scale != nullptr) return TRMOE_OK;
    if (!(eps > 0.0f)) {
        std::string m = std::string(who) + ": row_scale null needs eps > 0";
        return set_error(TRMOE_ERR_INVALID, m.c_str());
    }
    if (n_tokens > kSkinnyMaxTokens) {
        std::string m = std::string(who) + ": in-kernel RMSNorm scales need n_tokens <= 128 (else trmoe_rms_row_scale)";
        return set_error(TRMOE_ERR_INVALID, m.c_str());
    }
    return TRMOE_OK;
}

static int shared_gate_up_impl(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                               int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                               void* h, int64_t ldh, void* gu, int64_t ldgu, void* stream,
                               const float* row_scale = nullptr, float rms_eps = 0.0f,
                               const void* w_frag = nullptr) {
    TRMOE_REQUIRE(valid_pair(act_dtype, w_dtype), "shared_gate_up: unsupported dtype pair");
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && shared_width > 0, "shared_gate_up: bad dimensions");
    TRMOE_REQUIRE(ldx >= hidden, "shared_gate_up: ldx < hidden");
    TRMOE_REQUIRE(ldh >= round_up(shared_width, 128), "shared_gate_up: ldh < round_up(shared_width, 128)");
    TRMOE_REQUIRE(hidden < (int64_t)1 << 30, "shared_gate_up: hidden too large");
    TRMOE_REQUIRE((w_dtype == TRMOE_FP8_E4M3) == (w_scale != nullptr), "shared_gate_up: w_scale iff fp8");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x && w_packed && h, "shared_gate_up: null pointer");
    TRMOE_REQUIRE(aligned16(w_packed), "shared_gate_up: packed weights must be 16-byte aligned");
    TRMOE_REQUIRE(rows_ok(x, ldx, elem_bytes(act_dtype)),
                  "shared_gate_up: x rows must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    TRMOE_REQUIRE(aligned16(h) && (ldh * elem_bytes(act_dtype)) % 16 == 0,
                  "shared_gate_up: h must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    GateUpArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.M = n_tokens;
    a.K = (int)hidden;
    a.w = w_packed;
    a.ldw = round_up(hidden, 8);
    a.w_scale = w_scale;
    a.h = h;
    a.ldh = ldh;
    a.shared_mult = 1.0f;
    a.shared_feats = 0;
    a.expert_feats = 1;
    a.ids = nullptr;
    a.table = nullptr;
    a.vocab = 1;
    a.top_k = 0;
    for (int j = 0; j < 4; ++j) a.rw[j] = 0.f;
    a.gu = gu;
    a.ldgu = ldgu;
    a.row_scale = row_scale;
    a.rms_eps = rms_eps;
    a.w_frag = w_frag;
    return launch_gate_up(act_dtype, w_dtype, a, 2 * round_up(shared_width, 128), as_stream(stream));
}

int trmoe_rms_row_scale(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx, float eps,
                        float* row_scale, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "rms_row_scale: bf16 or f32 activations");
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && hidden < (int64_t)1 << 30, "rms_row_scale: bad dimensions");
    TRMOE_REQUIRE(ldx >= hidden, "rms_row_scale: ldx < hidden");
    TRMOE_REQUIRE(eps >= 0.0f, "rms_row_scale: eps must be non-negative");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x && row_scale, "rms_row_scale: null pointer");
    TRMOE_REQUIRE(rows_ok(x, ldx, elem_bytes(act_dtype)),
                  "rms_row_scale: x rows must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    return launch_rms_row_scale(act_dtype, x, n_tokens, hidden, ldx, eps, row_scale, as_stream(stream));
}

int trmoe_quantize_rows_e4m3(int act_dtype, const void* x, int64_t n_rows, int64_t k, int64_t ldx, void* q,
                             int64_t ldq, float* scale, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "quantize_rows_e4m3: bf16 or f32 rows");
    TRMOE_REQUIRE(n_rows >= 0, "quantize_rows_e4m3: n_rows < 0");
    TRMOE_REQUIRE(k > 0 && (k * elem_bytes(act_dtype)) % 16 == 0 && k <= rmsnorm_max_hidden(act_dtype),
                  "quantize_rows_e4m3: k must be a positive multiple of 16 bytes of elements, at most 4096 bf16 "
                  "or 2048 f32");
    TRMOE_REQUIRE(ldx >= k && ldq >= k, "quantize_rows_e4m3: row stride < k");
    if (n_rows == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x && q && scale, "quantize_rows_e4m3: null pointer");
    TRMOE_REQUIRE(rows_ok(x, ldx, elem_bytes(act_dtype)) && rows_ok(q, ldq, 1),
                  "quantize_rows_e4m3: x and q must be 16-byte aligned with row strides that are multiples of 16 "
                  "bytes");
    return launch_quantize_rows_e4m3(act_dtype, x, n_rows, k, ldx, q, ldq, scale, as_stream(stream));
}

int trmoe_shared_gate_up_a8(const void* x_q, const float* x_scale, int64_t n_tokens, int64_t hidden, int64_t ldxq,
                            const void* w_packed, const float* w_scale, int64_t shared_width, void* h, int64_t ldh,
                            void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && shared_width > 0, "shared_gate_up_a8: bad dimensions");
    TRMOE_REQUIRE(hidden % 128 == 0 && hidden < (int64_t)1 << 30, "shared_gate_up_a8: hidden must be a multiple of 128");
    TRMOE_REQUIRE(ldxq >= hidden, "shared_gate_up_a8: ldxq < hidden");
    TRMOE_REQUIRE(ldh >= round_up(shared_width, 128), "shared_gate_up_a8: ldh < round_up(shared_width, 128)");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x_q && x_scale && w_packed && w_scale && h, "shared_gate_up_a8: null pointer");
    TRMOE_REQUIRE(aligned16(w_packed), "shared_gate_up_a8: packed weights must be 16-byte aligned");
    TRMOE_REQUIRE(rows_ok(x_q, ldxq, 1),
                  "shared_gate_up_a8: x_q rows must be 16-byte aligned with a row stride that is a multiple of 16 "
                  "bytes");
    TRMOE_REQUIRE(aligned16(h) && (ldh * 2) % 16 == 0,
                  "shared_gate_up_a8: h must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    GateUpArgs a{};
    a.x = x_q;
    a.ldx = ldxq;
    a.M = n_tokens;
    a.K = (int)hidden;
    a.w = w_packed;
    a.ldw = hidden;
    a.w_scale = w_scale;
    a.h = h;
    a.ldh = ldh;
    a.shared_mult = 1.0f;
    a.shared_feats = 0;
    a.expert_feats = 1;
    a.vocab = 1;
    a.row_scale = x_scale;
    return launch_gate_up_a8(a, 2 * round_up(shared_width, 128), as_stream(stream));
}

int trmoe_shared_gate_up_a8_mx(const void* x_q, const float* x_scale, int64_t n_tokens, int64_t hidden, int64_t ldxq,
                               const void* w_packed, const float* w_scale, int64_t shared_width, void* h_q,
                               int64_t ldhq, void* h_scale, int64_t ldhs, void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && shared_width > 0, "shared_gate_up_a8_mx: bad dimensions");
    TRMOE_REQUIRE(hidden % 128 == 0 && hidden < (int64_t)1 << 30,
                  "shared_gate_up_a8_mx: hidden must be a multiple of 128");
    TRMOE_REQUIRE(ldxq >= hidden, "shared_gate_up_a8_mx: ldxq < hidden");
    const int64_t f_pad = round_up(shared_width, 128);
    // a 256-row tile's bytes stay below 2^31 (32-bit buffer offsets)
    TRMOE_REQUIRE(ldhq >= f_pad && ldhq % 16 == 0 && ldhq < (int64_t)1 << 23,
                  "shared_gate_up_a8_mx: ldhq must be a multiple of 16, at least round_up(shared_width, 128)");
    TRMOE_REQUIRE(ldhs >= f_pad / 32 && ldhs % 4 == 0 && ldhs < (int64_t)1 << 23,
                  "shared_gate_up_a8_mx: ldhs must be a multiple of 4, at least round_up(shared_width, 128) / 32");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(n_tokens * ldhq < (int64_t)1 << 40, "shared_gate_up_a8_mx: h_q too large");
    TRMOE_REQUIRE(x_q && x_scale && w_packed && w_scale && h_q && h_scale, "shared_gate_up_a8_mx: null pointer");
    TRMOE_REQUIRE(aligned16(w_packed), "shared_gate_up_a8_mx: packed weights must be 16-byte aligned");
    TRMOE_REQUIRE(rows_ok(x_q, ldxq, 1),
                  "shared_gate_up_a8_mx: x_q rows must be 16-byte aligned with a row stride that is a multiple of 16 "
                  "bytes");
    TRMOE_REQUIRE(aligned16(h_q) && reinterpret_cast<uintptr_t>(h_scale) % 4 == 0,
                  "shared_gate_up_a8_mx: h_q must be 16-byte and h_scale 4-byte aligned");
    GateUpArgs a{};
    a.x = x_q;
    a.ldx = ldxq;
    a.M = n_tokens;
    a.K = (int)hidden;
    a.w = w_packed;
    a.ldw = hidden;
    a.w_scale = w_scale;
    a.h = h_q;
    a.ldh = ldhq;
    a.hs = h_scale;
    a.ldhs = ldhs;
    a.shared_mult = 1.0f;
    a.shared_feats = 0;
    a.expert_feats = 1;
    a.vocab = 1;
    a.row_scale = x_scale;
    return launch_gate_up_a8(a, 2 * f_pad, as_stream(stream));
}

static bool rmsnorm_hidden_ok(int act_dtype, int64_t hidden) {
    return hidden > 0 && (hidden * elem_bytes(act_dtype)) % 16 == 0 && hidden <= rmsnorm_max_hidden(act_dtype);
}

int trmoe_rmsnorm_forward(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                          const void* weight, float eps, void* y, int64_t ldy, float* row_scale, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "rmsnorm_forward: bf16 or f32 activations");
    TRMOE_REQUIRE(n_tokens >= 0, "rmsnorm_forward: n_tokens < 0");
    TRMOE_REQUIRE(rmsnorm_hidden_ok(act_dtype, hidden),
                  "rmsnorm_forward: hidden must be a positive multiple of 16 bytes of elements, at most 4096 bf16 "
                  "or 2048 f32");
    TRMOE_REQUIRE(ldx >= hidden && ldy >= hidden, "rmsnorm_forward: row stride < hidden");
    TRMOE_REQUIRE(eps >= 0.0f, "rmsnorm_forward: eps must be non-negative");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x && weight && y && row_scale, "rmsnorm_forward: null pointer");
    const int eb = elem_bytes(act_dtype);
    TRMOE_REQUIRE(rows_ok(x, ldx, eb) && rows_ok(y, ldy, eb) && aligned16(weight),
                  "rmsnorm_forward: x, y and weight must be 16-byte aligned with row strides that are multiples of "
                  "16 bytes");
    return launch_rmsnorm_forward(act_dtype, x, n_tokens, hidden, ldx, weight, eps, y, ldy, row_scale,
                                  as_stream(stream));
}

size_t trmoe_rmsnorm_backward_workspace_bytes(int act_dtype, int64_t n_tokens, int64_t hidden) {
    if ((act_dtype != TRMOE_F32 && act_dtype != TRMOE_BF16) || n_tokens < 0 || !rmsnorm_hidden_ok(act_dtype, hidden))
        return 0;
    return (size_t)rmsnorm_groups(n_tokens) * (size_t)hidden * sizeof(float);
}

int trmoe_rmsnorm_backward(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                           const void* weight, const float* row_scale, const void* dy, int64_t lddy,
                           const void* dres, int64_t lddres, void* dx, int64_t lddx, void* dweight,
                           void* workspace, size_t workspace_bytes, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "rmsnorm_backward: bf16 or f32 activations");
    TRMOE_REQUIRE(n_tokens >= 0, "rmsnorm_backward: n_tokens < 0");
    TRMOE_REQUIRE(rmsnorm_hidden_ok(act_dtype, hidden),
                  "rmsnorm_backward: hidden must be a positive multiple of 16 bytes of elements, at most 4096 bf16 "
                  "or 2048 f32");
    TRMOE_REQUIRE(ldx >= hidden && lddy >= hidden && lddx >= hidden && (dres == nullptr || lddres >= hidden),
                  "rmsnorm_backward: row stride < hidden");
    TRMOE_REQUIRE(dres == nullptr || dres != dx || lddres == lddx,
                  "rmsnorm_backward: dres in place of dx needs the same row stride");
    TRMOE_REQUIRE(weight && dweight && workspace, "rmsnorm_backward: null pointer");
    TRMOE_REQUIRE(workspace_bytes >= trmoe_rmsnorm_backward_workspace_bytes(act_dtype, n_tokens, hidden),
                  "rmsnorm_backward: workspace smaller than trmoe_rmsnorm_backward_workspace_bytes()");
    const int eb = elem_bytes(act_dtype);
    if (n_tokens > 0) {
        TRMOE_REQUIRE(x && row_scale && dy && dx, "rmsnorm_backward: null pointer");
        TRMOE_REQUIRE(rows_ok(x, ldx, eb) && rows_ok(dy, lddy, eb) && rows_ok(dx, lddx, eb) &&
                          (dres == nullptr || rows_ok(dres, lddres, eb)),
                      "rmsnorm_backward: x, dy, dres and dx must be 16-byte aligned with row strides that are "
                      "multiples of 16 bytes");
    }
    TRMOE_REQUIRE(aligned16(weight), "rmsnorm_backward: weight must be 16-byte aligned");
    return launch_rmsnorm_backward(act_dtype, x, ldx, weight, row_scale, dy, lddy, dres, lddres, n_tokens, hidden,
                                   dx, lddx, dweight, static_cast<float*>(workspace), as_stream(stream));
}

int trmoe_shared_gate_up_rms(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                             int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                             const float* row_scale, float eps, void* h, int64_t ldh, void* stream) {
    const int st = rms_args_ok("shared_gate_up_rms", row_scale, eps, n_tokens);
    if (st) return st;
    return shared_gate_up_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, w_packed, w_scale, shared_width, h,
                               ldh, nullptr, 0, stream, row_scale, row_scale ? 0.0f : eps);
}

int trmoe_shared_gate_up(int act_dtype, int w_dtype, const void* x, int64_t n_tokens,
                         int64_t hidden, int64_t ldx, const void* w_packed, const float* w_scale,
                         int64_t shared_width, void* h, int64_t ldh, void* stream) {
    return shared_gate_up_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, w_packed, w_scale, shared_width, h,
                               ldh, nullptr, 0, stream);
}

int trmoe_shared_gate_up_save(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                              const void* w_packed, int64_t shared_width, void* h, int64_t ldh, void* gu,
                              int64_t ldgu, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "shared_gate_up_save: bf16 or f32 weights");
    TRMOE_REQUIRE(n_tokens == 0 || gu != nullptr, "shared_gate_up_save: null gu");
    TRMOE_REQUIRE(shared_width > 0 && ldgu >= 2 * round_up(shared_width, 128),
                  "shared_gate_up_save: ldgu < 2 * round_up(shared_width, 128)");
    return shared_gate_up_impl(act_dtype, act_dtype, x, n_tokens, hidden, ldx, w_packed, nullptr, shared_width, h,
                               ldh, gu, ldgu, stream);
}

int64_t trmoe_dense_routed_features(int64_t shared_width, int num_experts, int64_t expert_width) {
    if (shared_width < 0 || num_experts < 1 || expert_width < 1) return -1;
    return round_up(round_up(shared_width, 128) + num_experts * round_up(expert_width, 64), 128);
}

static int dense_routed_gate_up_impl(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                                     int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                                     int num_experts, int64_t expert_width, const int64_t* token_ids,
                                     const int64_t* route_table, int64_t vocab_size, int top_k,
                                     const float* route_weights, float shared_scale, float routed_scale, void* h,
                                     int64_t ldh, void* gu, int64_t ldgu, void* stream,
                                     const float* row_scale = nullptr, float rms_eps = 0.0f,
                                     const void* w_frag = nullptr) {
    TRMOE_REQUIRE(valid_pair(act_dtype, w_dtype), "dense_routed_gate_up: unsupported dtype pair");
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && shared_width >= 0 && expert_width > 0,
                  "dense_routed_gate_up: bad dimensions");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "dense_routed_gate_up: num_experts must be in [1, 16]");
    TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= num_experts, "dense_routed_gate_up: bad top_k");
    TRMOE_REQUIRE(vocab_size > 0, "dense_routed_gate_up: vocab_size must be positive");
    const int64_t feats = trmoe_dense_routed_features(shared_width, num_experts, expert_width);
    TRMOE_REQUIRE(ldx >= hidden, "dense_routed_gate_up: ldx < hidden");
    TRMOE_REQUIRE(ldh >= feats, "dense_routed_gate_up: ldh < trmoe_dense_routed_features()");
    TRMOE_REQUIRE(hidden < (int64_t)1 << 30, "dense_routed_gate_up: hidden too large");
    TRMOE_REQUIRE((w_dtype == TRMOE_FP8_E4M3) == (w_scale != nullptr), "dense_routed_gate_up: w_scale iff fp8");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x && w_packed && h && token_ids && route_table && route_weights,
                  "dense_routed_gate_up: null pointer");
    TRMOE_REQUIRE(aligned16(w_packed), "dense_routed_gate_up: packed weights must be 16-byte aligned");
    TRMOE_REQUIRE(rows_ok(x, ldx, elem_bytes(act_dtype)),
                  "dense_routed_gate_up: x rows must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    TRMOE_REQUIRE(aligned16(h) && (ldh * elem_bytes(act_dtype)) % 16 == 0,
                  "dense_routed_gate_up: h must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    GateUpArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.M = n_tokens;
    a.K = (int)hidden;
    a.w = w_packed;
    a.ldw = round_up(hidden, 8);
    a.w_scale = w_scale;
    a.h = h;
    a.ldh = ldh;
    a.shared_mult = shared_scale;
    a.shared_feats = round_up(shared_width, 128);
    a.expert_feats = round_up(expert_width, 64);
    a.ids = token_ids;
    a.table = route_table;
    a.vocab = vocab_size;
    a.top_k = top_k;
    for (int j = 0; j < 4; ++j) a.rw[j] = j < top_k ? routed_scale * route_weights[j] : 0.f;
    a.gu = gu;
    a.ldgu = ldgu;
    a.row_scale = row_scale;
    a.rms_eps = rms_eps;
    a.w_frag = w_frag;
    return launch_gate_up(act_dtype, w_dtype, a, 2 * feats, as_stream(stream));
}

int trmoe_dense_routed_gate_up_rms(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                                   int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                                   int num_experts, int64_t expert_width, const int64_t* token_ids,
                                   const int64_t* route_table, int64_t vocab_size, int top_k,
                                   const float* route_weights, float shared_scale, float routed_scale,
                                   const float* row_scale, float eps, void* h, int64_t ldh, void* stream) {
    const int st = rms_args_ok("dense_routed_gate_up_rms", row_scale, eps, n_tokens);
    if (st) return st;
    return dense_routed_gate_up_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, w_packed, w_scale, shared_width,
                                     num_experts, expert_width, token_ids, route_table, vocab_size, top_k,
                                     route_weights, shared_scale, routed_scale, h, ldh, nullptr, 0, stream,
                                     row_scale, row_scale ? 0.0f : eps);
}

int trmoe_dense_routed_gate_up(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                               int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                               int num_experts, int64_t expert_width, const int64_t* token_ids,
                               const int64_t* route_table, int64_t vocab_size, int top_k,
                               const float* route_weights, float shared_scale, float routed_scale, void* h,
                               int64_t ldh, void* stream) {
    return dense_routed_gate_up_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, w_packed, w_scale, shared_width,
                                     num_experts, expert_width, token_ids, route_table, vocab_size, top_k,
                                     route_weights, shared_scale, routed_scale, h, ldh, nullptr, 0, stream);
}

int trmoe_dense_routed_gate_up_save(int act_dtype, const void* x, int64_t n_tokens, int64_t hidden, int64_t ldx,
                                    const void* w_packed, int64_t shared_width, int num_experts,
                                    int64_t expert_width, const int64_t* token_ids, const int64_t* route_table,
                                    int64_t vocab_size, int top_k, const float* route_weights, float shared_scale,
                                    float routed_scale, void* h, int64_t ldh, void* gu, int64_t ldgu,
                                    void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16,
                  "dense_routed_gate_up_save: bf16 or f32 weights");
    TRMOE_REQUIRE(n_tokens == 0 || gu != nullptr, "dense_routed_gate_up_save: null gu");
    TRMOE_REQUIRE(ldgu >= 2 * trmoe_dense_routed_features(shared_width, num_experts, expert_width),
                  "dense_routed_gate_up_save: ldgu < 2 * trmoe_dense_routed_features()");
    return dense_routed_gate_up_impl(act_dtype, act_dtype, x, n_tokens, hidden, ldx, w_packed, nullptr,
                                     shared_width, num_experts, expert_width, token_ids, route_table, vocab_size,
                                     top_k, route_weights, shared_scale, routed_scale, h, ldh, gu, ldgu, stream);
}

static int routed_experts_impl(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                               int64_t ldx, const int64_t* sorted_indices, const int32_t* expert_offsets,
                               int num_experts, int top_k, const void* w_gate_up, const float* s_gate_up,
                               const void* w_down, const float* s_down, int64_t expert_width, void* y, int64_t ldy,
                               void* workspace, size_t workspace_bytes, void* stream, const float* row_scale) {
    TRMOE_REQUIRE(valid_pair(act_dtype, w_dtype), "routed_experts: unsupported dtype pair");
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && expert_width > 0, "routed_experts: bad dimensions");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "routed_experts: num_experts must be in [1, 16]");
    TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= num_experts, "routed_experts: bad top_k");
    TRMOE_REQUIRE(ldx >= hidden && ldy >= hidden, "routed_experts: bad leading dimension");
    TRMOE_REQUIRE(hidden < (int64_t)1 << 30, "routed_experts: hidden too large");
    TRMOE_REQUIRE((w_dtype == TRMOE_FP8_E4M3) == (s_gate_up != nullptr && s_down != nullptr),
                  "routed_experts: scales iff fp8");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(x && sorted_indices && expert_offsets && w_gate_up && w_down && y, "routed_experts: null pointer");
    TRMOE_REQUIRE(aligned16(w_gate_up) && aligned16(w_down), "routed_experts: packed weights must be 16-byte aligned");
    const int64_t f_pad = round_up(expert_width, 64);
    if (routed_lds_bytes(act_dtype, f_pad) > 160 * 1024)
        return set_error(TRMOE_ERR_UNSUPPORTED, "routed_experts: expert_width too large for the LDS-resident tile");
    TRMOE_REQUIRE(rows_ok(x, ldx, elem_bytes(act_dtype)),
                  "routed_experts: x rows must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    if (n_tokens * ldx * elem_bytes(act_dtype) >= ((int64_t)1 << 31))
        return set_error(TRMOE_ERR_UNSUPPORTED, "routed_experts: x must be smaller than 2 GiB");
    RoutedArgs a{};
    a.x = x;
    a.ldx = ldx;
    a.n_tokens = n_tokens;
    a.K = (int)hidden;
    a.sorted = sorted_indices;
    a.offsets = expert_offsets;
    a.E = num_experts;
    a.wgu = w_gate_up;
    a.wgu_ld = round_up(hidden, 8);
    a.sgu = s_gate_up;
    a.wd = w_down;
    a.wd_ld = round_up(expert_width, 8);
    a.sd = s_down;
    a.w_elem_bytes = elem_bytes(w_dtype);
    a.F_pad = (int)f_pad;
    a.W = (int)expert_width;
    a.H = (int)hidden;
    a.H_pad = (int)round_up(hidden, 256);  // packed down rows per expert
    a.y = y;
    a.ldy = ldy;
    const int64_t assignments = n_tokens * top_k;
    const size_t need = trmoe_routed_experts_workspace_bytes(act_dtype, assignments, expert_width);
    if (workspace == nullptr || workspace_bytes < need) {
        if (row_scale != nullptr)
            return set_error(TRMOE_ERR_INVALID, "routed_experts_rms: needs trmoe_routed_experts_workspace_bytes()");
        return launch_routed(act_dtype, w_dtype, a, assignments, as_stream(stream));
    }
    TRMOE_REQUIRE(aligned16(workspace), "routed_experts: workspace must be 16-byte aligned");
    TRMOE_REQUIRE(aligned16(y) && (ldy * elem_bytes(act_dtype)) % 16 == 0,
                  "routed_experts: y must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    // gate|up + SwiGLU: partition rows gathered from x -> h[assignments, F_pad]
    GateUpArgs g{};
    g.x = x;
    g.ldx = ldx;
    g.M = assignments;
    g.K = (int)hidden;
    g.w = w_gate_up;
    g.ldw = a.wgu_ld;
    g.w_scale = s_gate_up;
    g.h = workspace;
    g.ldh = f_pad;
    g.shared_mult = 1.0f;
    g.shared_feats = 0;
    g.expert_feats = 1;
    g.offsets = expert_offsets;
    g.E = num_experts;
    g.gather = sorted_indices;
    g.gather_mod = n_tokens;
    g.w_expert_stride = 2 * f_pad * a.wgu_ld;
    g.scale_expert_stride = 2 * f_pad;
    g.row_scale = row_scale;
    int st = launch_gate_up_grouped(act_dtype, w_dtype, g, assignments, 2 * f_pad, as_stream(stream));
    if (st) return st;
    // down: h rows (partition order) -> y rows
    DownArgs d{};
    d.h = workspace;
    d.ldh = f_pad;
    d.M = assignments;
    d.K = (int)expert_width;
    d.w = w_down;
    d.ldw = a.wd_ld;
    d.w_scale = s_down;
    d.N = (int)hidden;
    d.shared_scale = 1.0f;
    d.routed_scale = 0.0f;
    d.out = y;
    d.ldo = ldy;
    d.vec_ok = 1;
    d.offsets = expert_offsets;
    d.E = num_experts;
    d.w_expert_stride = a.H_pad * a.wd_ld;
    d.scale_expert_stride = a.H_pad;
    return launch_down_grouped(act_dtype, w_dtype, d, assignments, as_stream(stream));
}

int trmoe_routed_experts(int act_dtype, int w_dtype, const void* x, int64_t n_tokens,
                         int64_t hidden, int64_t ldx, const int64_t* sorted_indices,
                         const int32_t* expert_offsets, int num_experts, int top_k,
                         const void* w_gate_up, const float* s_gate_up, const void* w_down,
                         const float* s_down, int64_t expert_width, void* y, int64_t ldy,
                         void* workspace, size_t workspace_bytes, void* stream) {
    return routed_experts_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, sorted_indices, expert_offsets,
                               num_experts, top_k, w_gate_up, s_gate_up, w_down, s_down, expert_width, y, ldy,
                               workspace, workspace_bytes, stream, nullptr);
}

int trmoe_routed_experts_rms(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                             int64_t ldx, const int64_t* sorted_indices, const int32_t* expert_offsets,
                             int num_experts, int top_k, const void* w_gate_up, const float* s_gate_up,
                             const void* w_down, const float* s_down, int64_t expert_width, const float* row_scale,
                             void* y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream) {
    TRMOE_REQUIRE(n_tokens == 0 || row_scale != nullptr, "routed_experts_rms: null row_scale");
    return routed_experts_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, sorted_indices, expert_offsets,
                               num_experts, top_k, w_gate_up, s_gate_up, w_down, s_down, expert_width, y, ldy,
                               workspace, workspace_bytes, stream, row_scale);
}

size_t trmoe_routed_experts_workspace_bytes(int act_dtype, int64_t n_assignments, int64_t expert_width) {
    if ((act_dtype != TRMOE_F32 && act_dtype != TRMOE_BF16) || n_assignments < 1 || expert_width < 1) return 0;
    return (size_t)(n_assignments * round_up(expert_width, 64) * elem_bytes(act_dtype));
}

static int shared_down_combine_impl(int act_dtype, int w_dtype, const void* h, int64_t n_tokens,
                                    int64_t shared_width, int64_t ldh, const void* w_down, const float* w_scale,
                                    int64_t hidden, const void* y, int64_t ldy, const int64_t* inverse, int top_k,
                                    const float* route_weights, float shared_scale, float routed_scale,
                                    const void* residual, int64_t ldr, void* out, int64_t ldo, void* workspace,
                                    size_t workspace_bytes, void* stream, const void* w_frag) {
    TRMOE_REQUIRE(valid_pair(act_dtype, w_dtype), "shared_down_combine: unsupported dtype pair");
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && shared_width > 0, "shared_down_combine: bad dimensions");
    TRMOE_REQUIRE(ldh >= shared_width && ldo >= hidden, "shared_down_combine: bad leading dimension");
    TRMOE_REQUIRE(shared_width < (int64_t)1 << 30, "shared_down_combine: shared_width too large");
    TRMOE_REQUIRE((w_dtype == TRMOE_FP8_E4M3) == (w_scale != nullptr), "shared_down_combine: w_scale iff fp8");
    TRMOE_REQUIRE((y == nullptr) == (inverse == nullptr), "shared_down_combine: y and inverse go together");
    if (y != nullptr) {
        TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, "shared_down_combine: bad top_k");
        TRMOE_REQUIRE(route_weights != nullptr, "shared_down_combine: null route_weights");
        TRMOE_REQUIRE(ldy >= hidden, "shared_down_combine: ldy < hidden");
    }
    TRMOE_REQUIRE(residual == nullptr || ldr >= hidden, "shared_down_combine: ldr < hidden");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(h && w_down && out, "shared_down_combine: null pointer");
    TRMOE_REQUIRE(aligned16(w_down), "shared_down_combine: packed weights must be 16-byte aligned");
    TRMOE_REQUIRE(rows_ok(h, ldh, elem_bytes(act_dtype)),
                  "shared_down_combine: h rows must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    DownArgs a{};
    a.h = h;
    a.ldh = ldh;
    a.M = n_tokens;
    a.K = (int)shared_width;
    a.w = w_down;
    a.ldw = round_up(shared_width, 8);
    a.w_scale = w_scale;
    a.N = (int)hidden;
    a.y = y;
    a.ldy = ldy;
    a.inverse = inverse;
    a.top_k = (y != nullptr) ? top_k : 0;
    for (int j = 0; j < 4; ++j) a.rw[j] = (y != nullptr && j < top_k) ? route_weights[j] : 0.f;
    a.shared_scale = shared_scale;
    a.routed_scale = routed_scale;
    a.residual = residual;
    a.ldr = ldr;
    a.out = out;
    a.ldo = ldo;
    {
        const int eb = elem_bytes(act_dtype);
        a.vec_ok = aligned16(out) && (ldo * eb) % 16 == 0 && (y == nullptr || (aligned16(y) && (ldy * eb) % 16 == 0)) &&
                   (residual == nullptr || (aligned16(residual) && (ldr * eb) % 16 == 0));
    }
    a.w_frag = w_frag;
    const size_t need = down_skinny_workspace_bytes(n_tokens, hidden, shared_width, act_dtype);
    if (need > 0 && workspace != nullptr && workspace_bytes >= need) {
        TRMOE_REQUIRE(aligned16(workspace), "shared_down_combine: workspace must be 16-byte aligned");
        return launch_down_skinny(act_dtype, w_dtype, a, workspace, as_stream(stream));
    }
    return launch_down_combine(act_dtype, w_dtype, a, as_stream(stream));
}

int trmoe_shared_down_combine(int act_dtype, int w_dtype, const void* h, int64_t n_tokens,
                              int64_t shared_width, int64_t ldh, const void* w_down,
                              const float* w_scale, int64_t hidden, const void* y, int64_t ldy,
                              const int64_t* inverse, int top_k, const float* route_weights,
                              float shared_scale, float routed_scale, const void* residual,
                              int64_t ldr, void* out, int64_t ldo, void* workspace,
                              size_t workspace_bytes, void* stream) {
    return shared_down_combine_impl(act_dtype, w_dtype, h, n_tokens, shared_width, ldh, w_down, w_scale, hidden, y,
                                    ldy, inverse, top_k, route_weights, shared_scale, routed_scale, residual, ldr,
                                    out, ldo, workspace, workspace_bytes, stream, nullptr);
}

int trmoe_shared_down_combine_a8(const void* h_q, const void* h_scale, int64_t n_tokens, int64_t shared_width,
                                 int64_t ldhq, int64_t ldhs, const void* w_down, const float* w_scale, int64_t hidden,
                                 const void* y, int64_t ldy, const int64_t* inverse, int top_k,
                                 const float* route_weights, float shared_scale, float routed_scale,
                                 const void* residual, int64_t ldr, void* out, int64_t ldo, void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0 && hidden < (int64_t)1 << 30, "shared_down_combine_a8: bad dimensions");
    TRMOE_REQUIRE(shared_width > 0 && shared_width % 128 == 0 && shared_width < (int64_t)1 << 30,
                  "shared_down_combine_a8: shared_width must be a positive multiple of 128");
    // a 256-row tile's bytes stay below 2^31 (32-bit buffer offsets)
    TRMOE_REQUIRE(ldhq >= shared_width && ldhq % 16 == 0 && ldhq < (int64_t)1 << 23,
                  "shared_down_combine_a8: ldhq must be a multiple of 16, at least shared_width");
    TRMOE_REQUIRE(ldhs >= shared_width / 32 && ldhs % 4 == 0 && ldhs < (int64_t)1 << 23,
                  "shared_down_combine_a8: ldhs must be a multiple of 4, at least shared_width / 32");
    TRMOE_REQUIRE(ldo >= hidden, "shared_down_combine_a8: ldo < hidden");
    TRMOE_REQUIRE((y == nullptr) == (inverse == nullptr), "shared_down_combine_a8: y and inverse go together");
    if (y != nullptr) {
        TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, "shared_down_combine_a8: bad top_k");
        TRMOE_REQUIRE(route_weights != nullptr, "shared_down_combine_a8: null route_weights");
        TRMOE_REQUIRE(ldy >= hidden, "shared_down_combine_a8: ldy < hidden");
    }
    TRMOE_REQUIRE(residual == nullptr || ldr >= hidden, "shared_down_combine_a8: ldr < hidden");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(n_tokens * ldhq < (int64_t)1 << 40, "shared_down_combine_a8: h_q too large");
    TRMOE_REQUIRE(h_q && h_scale && w_down && w_scale && out, "shared_down_combine_a8: null pointer");
    TRMOE_REQUIRE(aligned16(w_down) && aligned16(h_q) && reinterpret_cast<uintptr_t>(h_scale) % 4 == 0,
                  "shared_down_combine_a8: w_down and h_q must be 16-byte, h_scale 4-byte aligned");
    DownArgs a{};
    a.h = h_q;
    a.ldh = ldhq;
    a.hs = h_scale;
    a.ldhs = ldhs;
    a.M = n_tokens;
    a.K = (int)shared_width;
    a.w = w_down;
    a.ldw = round_up(shared_width, 8);
    a.w_scale = w_scale;
    a.N = (int)hidden;
    a.y = y;
    a.ldy = ldy;
    a.inverse = inverse;
    a.top_k = (y != nullptr) ? top_k : 0;
    for (int j = 0; j < 4; ++j) a.rw[j] = (y != nullptr && j < top_k) ? route_weights[j] : 0.f;
    a.shared_scale = shared_scale;
    a.routed_scale = routed_scale;
    a.residual = residual;
    a.ldr = ldr;
    a.out = out;
    a.ldo = ldo;
    a.vec_ok = aligned16(out) && (ldo * 2) % 16 == 0 && (y == nullptr || (aligned16(y) && (ldy * 2) % 16 == 0)) &&
               (residual == nullptr || (aligned16(residual) && (ldr * 2) % 16 == 0));
    return launch_down_combine_a8(a, as_stream(stream));
}

size_t trmoe_fragment_bytes(int dtype, int64_t rows, int64_t cols) {
    const int eb = elem_bytes(dtype);
    if ((dtype != TRMOE_F32 && dtype != TRMOE_BF16) || rows <= 0 || rows % 16 != 0 || cols <= 0) return 0;
    return (size_t)(rows / 16) * (size_t)((cols * eb + 63) / 64) * 1024;
}

int trmoe_pack_fragments(int dtype, const void* packed, int64_t rows, int64_t cols, int64_t ld, void* dst,
                         void* stream) {
    TRMOE_REQUIRE(dtype == TRMOE_F32 || dtype == TRMOE_BF16, "pack_fragments: bf16 or f32 weights");
    TRMOE_REQUIRE(rows > 0 && rows % 16 == 0 && cols > 0 && ld >= round_up(cols, 8),
                  "pack_fragments: rows must be a positive multiple of 16, ld >= round_up(cols, 8)");
    TRMOE_REQUIRE(packed && dst, "pack_fragments: null pointer");
    TRMOE_REQUIRE(aligned16(packed) && aligned16(dst), "pack_fragments: buffers must be 16-byte aligned");
    TRMOE_REQUIRE(rows * ld * elem_bytes(dtype) < ((int64_t)1 << 40), "pack_fragments: too large");
    return launch_pack_fragments(packed, rows, cols * elem_bytes(dtype), ld * elem_bytes(dtype), dst,
                                 as_stream(stream));
}

// Extras of the *_ex entry points: validated against the call they ride on.
static int extras_ok(const char* who, const trmoe_call_extras* ex, int act_dtype, int w_dtype, int64_t k,
                     int64_t n_tokens, bool rms_allowed) {
    if (ex == nullptr) return TRMOE_OK;
    if (ex->w_frag != nullptr) {
        if (w_dtype != act_dtype || (act_dtype != TRMOE_F32 && act_dtype != TRMOE_BF16)) {
            std::string m = std::string(who) + ": w_frag needs bf16 or f32 weights";
            return set_error(TRMOE_ERR_INVALID, m.c_str());
        }
        if (!aligned16(ex->w_frag) || ex->w_frag_cols != k) {
            std::string m = std::string(who) + ": w_frag must be 16-byte aligned and packed with cols = " +
                            std::to_string(k);
            return set_error(TRMOE_ERR_INVALID, m.c_str());
        }
    }
    if (!rms_allowed && (ex->row_scale != nullptr || ex->rms_eps != 0.0f)) {
        std::string m = std::string(who) + ": no RMSNorm scales on this call";
        return set_error(TRMOE_ERR_INVALID, m.c_str());
    }
    if (ex->row_scale != nullptr || ex->rms_eps > 0.0f) return rms_args_ok(who, ex->row_scale, ex->rms_eps, n_tokens);
    return TRMOE_OK;
}

int trmoe_shared_gate_up_ex(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                            int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width, void* h,
                            int64_t ldh, const trmoe_call_extras* extras, void* stream) {
    const int st = extras_ok("shared_gate_up_ex", extras, act_dtype, w_dtype, hidden, n_tokens, true);
    if (st) return st;
    const trmoe_call_extras e = extras ? *extras : trmoe_call_extras{};
    return shared_gate_up_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, w_packed, w_scale, shared_width, h,
                               ldh, nullptr, 0, stream, e.row_scale, e.row_scale ? 0.0f : e.rms_eps, e.w_frag);
}

int trmoe_dense_routed_gate_up_ex(int act_dtype, int w_dtype, const void* x, int64_t n_tokens, int64_t hidden,
                                  int64_t ldx, const void* w_packed, const float* w_scale, int64_t shared_width,
                                  int num_experts, int64_t expert_width, const int64_t* token_ids,
                                  const int64_t* route_table, int64_t vocab_size, int top_k,
                                  const float* route_weights, float shared_scale, float routed_scale, void* h,
                                  int64_t ldh, const trmoe_call_extras* extras, void* stream) {
    const int st = extras_ok("dense_routed_gate_up_ex", extras, act_dtype, w_dtype, hidden, n_tokens, true);
    if (st) return st;
    const trmoe_call_extras e = extras ? *extras : trmoe_call_extras{};
    return dense_routed_gate_up_impl(act_dtype, w_dtype, x, n_tokens, hidden, ldx, w_packed, w_scale, shared_width,
                                     num_experts, expert_width, token_ids, route_table, vocab_size, top_k,
                                     route_weights, shared_scale, routed_scale, h, ldh, nullptr, 0, stream,
                                     e.row_scale, e.row_scale ? 0.0f : e.rms_eps, e.w_frag);
}

int trmoe_shared_down_combine_ex(int act_dtype, int w_dtype, const void* h, int64_t n_tokens, int64_t shared_width,
                                 int64_t ldh, const void* w_down, const float* w_scale, int64_t hidden, const void* y,
                                 int64_t ldy, const int64_t* inverse, int top_k, const float* route_weights,
                                 float shared_scale, float routed_scale, const void* residual, int64_t ldr, void* out,
                                 int64_t ldo, void* workspace, size_t workspace_bytes,
                                 const trmoe_call_extras* extras, void* stream) {
    const int st = extras_ok("shared_down_combine_ex", extras, act_dtype, w_dtype, shared_width, n_tokens, false);
    if (st) return st;
    return shared_down_combine_impl(act_dtype, w_dtype, h, n_tokens, shared_width, ldh, w_down, w_scale, hidden, y,
                                    ldy, inverse, top_k, route_weights, shared_scale, routed_scale, residual, ldr,
                                    out, ldo, workspace, workspace_bytes, stream, extras ? extras->w_frag : nullptr);
}

size_t trmoe_shared_down_combine_workspace_bytes(int act_dtype, int64_t n_tokens, int64_t shared_width,
                                                 int64_t hidden) {
    if (act_dtype != TRMOE_F32 && act_dtype != TRMOE_BF16) return 0;
    if (n_tokens < 1 || shared_width < 1 || hidden < 1) return 0;
    return down_skinny_workspace_bytes(n_tokens, hidden, shared_width, act_dtype);
}

int trmoe_combine(int act_dtype, int64_t n_tokens, int64_t hidden, const void* y, int64_t ldy,
                  const int64_t* inverse, int top_k, const float* route_weights,
                  float routed_scale, const void* residual, int64_t ldr, void* out, int64_t ldo,
                  void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "combine: bad dtype");
    TRMOE_REQUIRE(n_tokens >= 0 && hidden > 0, "combine: bad dimensions");
    TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK, "combine: bad top_k");
    TRMOE_REQUIRE(ldy >= hidden && ldo >= hidden && (residual == nullptr || ldr >= hidden),
                  "combine: bad leading dimension");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(y && inverse && route_weights && out, "combine: null pointer");
    CombineArgs a{};
    a.M = n_tokens;
    a.N = hidden;
    a.y = y;
    a.ldy = ldy;
    a.inverse = inverse;
    a.top_k = top_k;
    for (int j = 0; j < 4; ++j) a.rw[j] = j < top_k ? route_weights[j] : 0.f;
    a.routed_scale = routed_scale;
    a.residual = residual;
    a.ldr = ldr;
    a.out = out;
    a.ldo = ldo;
    return launch_combine(act_dtype, a, as_stream(stream));
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
static int swiglu_bwd_common(const char* who, int act_dtype, const void* x, const void* dout, int64_t rows,
                             int64_t hidden, int64_t ldx, int64_t ldd, const void* w_gate_up,
                             const void* w_down_t, void* dgu, int64_t lddgu, void* hm, int64_t ldhm,
                             int64_t features, int64_t x_rows) {
    (void)rows;
    if (act_dtype != TRMOE_F32 && act_dtype != TRMOE_BF16)
        return set_error(TRMOE_ERR_UNSUPPORTED, "swiglu_backward: bf16 or f32 only (fp8 weights are inference-only)");
    if (hidden <= 0 || hidden >= ((int64_t)1 << 30)) return set_error(TRMOE_ERR_INVALID, "swiglu_backward: bad hidden");
    if (ldx < hidden || ldd < hidden) return set_error(TRMOE_ERR_INVALID, "swiglu_backward: bad leading dimension");
    if (lddgu < 2 * features || (hm != nullptr && ldhm < features))
        return set_error(TRMOE_ERR_INVALID, "swiglu_backward: dgu/hm row stride too small");
    if (!(x && dout && w_gate_up && w_down_t && dgu)) return set_error(TRMOE_ERR_INVALID, "swiglu_backward: null pointer");
    const int eb = elem_bytes(act_dtype);
    if (!aligned16(w_gate_up) || !aligned16(w_down_t))
        return set_error(TRMOE_ERR_INVALID, "swiglu_backward: packed weights must be 16-byte aligned");
    if (!rows_ok(x, ldx, eb) || !rows_ok(dout, ldd, eb) || !rows_ok(dgu, lddgu, eb) ||
        (hm != nullptr && !rows_ok(hm, ldhm, eb)))
        return set_error(TRMOE_ERR_INVALID, "swiglu_backward: x/dout/dgu/hm rows must be 16-byte aligned with a "
                                            "stride that is a multiple of 16 bytes");
    if (x_rows * ldx * eb >= ((int64_t)1 << 31) || x_rows * ldd * eb >= ((int64_t)1 << 31))
        return set_error(TRMOE_ERR_UNSUPPORTED, "swiglu_backward: x and dout must be smaller than 2 GiB");
    (void)who;
    return TRMOE_OK;
}

static void swiglu_bwd_fill(SwigluBwdArgs& a, const void* x, const void* dout, int64_t hidden, int64_t ldx,
                            int64_t ldd, const void* w_gate_up, const void* w_down_t, int64_t features, void* dgu,
                            int64_t lddgu, void* hm, int64_t ldhm) {
    a.x = x;
    a.ldx = ldx;
    a.dout = dout;
    a.ldd = ldd;
    a.K = (int)hidden;
    a.wgu = w_gate_up;
    a.ldwgu = round_up(hidden, 8);
    a.wdt = w_down_t;
    a.ldwdt = round_up(hidden, 8);
    a.F = features;
    a.dgu = dgu;
    a.lddgu = lddgu;
    a.hm = hm;
    a.ldhm = ldhm;
    a.expert_feats = 1;
}

int trmoe_shared_swiglu_backward(int act_dtype, const void* x, const void* dout, int64_t n_tokens, int64_t hidden,
                                 int64_t ldx, int64_t ldd, const void* w_gate_up, const void* w_down_t,
                                 int64_t shared_width, float shared_scale, const void* gu, int64_t ldgu, void* dgu,
                                 int64_t lddgu, void* hm, int64_t ldhm, void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0 && shared_width > 0, "shared_swiglu_backward: bad dimensions");
    if (n_tokens == 0) return TRMOE_OK;
    const int64_t F = round_up(shared_width, 128);
    int st = swiglu_bwd_common("shared_swiglu_backward", act_dtype, x, dout, n_tokens, hidden, ldx, ldd, w_gate_up,
                               w_down_t, dgu, lddgu, hm, ldhm, F, n_tokens);
    if (st) return st;
    SwigluBwdArgs a{};
    swiglu_bwd_fill(a, x, dout, hidden, ldx, ldd, w_gate_up, w_down_t, F, dgu, lddgu, hm, ldhm);
    a.M = n_tokens;
    a.x_rows = n_tokens;
    a.shared_mult = shared_scale;
    TRMOE_REQUIRE(gu == nullptr || ldgu >= 2 * F, "shared_swiglu_backward: ldgu < 2 * round_up(S, 128)");
    TRMOE_REQUIRE(gu == nullptr || rows_ok(gu, ldgu, elem_bytes(act_dtype)), "shared_swiglu_backward: gu rows must be 16-byte aligned");
    a.gu = gu;
    a.ldgu = ldgu;
    return launch_swiglu_bwd(act_dtype, a, 0, as_stream(stream));
}

int trmoe_dense_routed_swiglu_backward(int act_dtype, const void* x, const void* dout, int64_t n_tokens,
                                       int64_t hidden, int64_t ldx, int64_t ldd, const void* w_gate_up,
                                       const void* w_down_t, int64_t shared_width, int num_experts,
                                       int64_t expert_width, const int64_t* token_ids, const int64_t* route_table,
                                       int64_t vocab_size, int top_k, const float* route_weights,
                                       float shared_scale, float routed_scale, const void* gu, int64_t ldgu,
                                       void* dgu, int64_t lddgu, void* hm, int64_t ldhm, void* stream) {
    const int64_t F = trmoe_dense_routed_features(shared_width, num_experts, expert_width);
    TRMOE_REQUIRE(F > 0 && n_tokens >= 0, "dense_routed_swiglu_backward: bad dimensions");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "dense_routed_swiglu_backward: bad num_experts");
    TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= num_experts, "dense_routed_swiglu_backward: bad top_k");
    TRMOE_REQUIRE(vocab_size > 0, "dense_routed_swiglu_backward: bad vocab_size");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(token_ids && route_table && route_weights, "dense_routed_swiglu_backward: null pointer");
    int st = swiglu_bwd_common("dense_routed_swiglu_backward", act_dtype, x, dout, n_tokens, hidden, ldx, ldd,
                               w_gate_up, w_down_t, dgu, lddgu, hm, ldhm, F, n_tokens);
    if (st) return st;
    SwigluBwdArgs a{};
    swiglu_bwd_fill(a, x, dout, hidden, ldx, ldd, w_gate_up, w_down_t, F, dgu, lddgu, hm, ldhm);
    a.M = n_tokens;
    a.x_rows = n_tokens;
    a.shared_mult = shared_scale;
    a.shared_feats = shared_width > 0 ? round_up(shared_width, 128) : 0;
    a.expert_feats = round_up(expert_width, 64);
    a.ids = token_ids;
    a.table = route_table;
    a.vocab = vocab_size;
    a.top_k = top_k;
    for (int j = 0; j < 4; ++j) a.rw[j] = j < top_k ? route_weights[j] * routed_scale : 0.f;
    TRMOE_REQUIRE(gu == nullptr || ldgu >= 2 * F, "dense_routed_swiglu_backward: ldgu < 2 * features");
    TRMOE_REQUIRE(gu == nullptr || rows_ok(gu, ldgu, elem_bytes(act_dtype)), "dense_routed_swiglu_backward: gu rows must be 16-byte aligned");
    a.gu = gu;
    a.ldgu = ldgu;
    return launch_swiglu_bwd(act_dtype, a, 0, as_stream(stream));
}

int trmoe_routed_swiglu_backward(int act_dtype, const void* x, const void* dout, int64_t n_tokens, int64_t hidden,
                                 int64_t ldx, int64_t ldd, const int64_t* sorted_indices,
                                 const int32_t* expert_offsets, int num_experts, int top_k, const void* w_gate_up,
                                 const void* w_down_t, int64_t expert_width, const float* route_weights,
                                 float routed_scale, void* dgu, int64_t lddgu, void* hm, int64_t ldhm,
                                 void* stream) {
    TRMOE_REQUIRE(n_tokens >= 0 && expert_width > 0, "routed_swiglu_backward: bad dimensions");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "routed_swiglu_backward: bad num_experts");
    TRMOE_REQUIRE(top_k >= 1 && top_k <= kMaxTopK && top_k <= num_experts, "routed_swiglu_backward: bad top_k");
    TRMOE_REQUIRE(n_tokens * top_k < ((int64_t)1 << 31), "routed_swiglu_backward: too many assignments");
    if (n_tokens == 0) return TRMOE_OK;
    TRMOE_REQUIRE(sorted_indices && expert_offsets && route_weights, "routed_swiglu_backward: null pointer");
    const int64_t F = round_up(expert_width, 64);
    int st = swiglu_bwd_common("routed_swiglu_backward", act_dtype, x, dout, n_tokens * top_k, hidden, ldx, ldd,
                               w_gate_up, w_down_t, dgu, lddgu, hm, ldhm, F, n_tokens);
    if (st) return st;
    SwigluBwdArgs a{};
    swiglu_bwd_fill(a, x, dout, hidden, ldx, ldd, w_gate_up, w_down_t, F, dgu, lddgu, hm, ldhm);
    a.M = n_tokens * top_k;
    a.x_rows = n_tokens;
    a.offsets = expert_offsets;
    a.E = num_experts;
    a.gather = sorted_indices;
    a.gather_mod = n_tokens;
    a.top_k = top_k;
    for (int j = 0; j < 4; ++j) a.rw[j] = j < top_k ? route_weights[j] * routed_scale : 0.f;
    a.wgu_expert_stride = 2 * F * a.ldwgu;
    a.wdt_expert_stride = F * a.ldwdt;
    return launch_swiglu_bwd(act_dtype, a, n_tokens * top_k, as_stream(stream));
}

size_t trmoe_weight_grad_workspace_bytes(int act_dtype, int64_t m, int64_t n, int num_segments, int64_t n_rows) {
    if ((act_dtype != TRMOE_F32 && act_dtype != TRMOE_BF16) || m <= 0 || n <= 0 || num_segments < 1 || n_rows < 0)
        return 0;
    const int splits = wgrad_splits(m, n, num_segments, n_rows / num_segments);
    return splits > 1 ? (size_t)splits * num_segments * m * n * sizeof(float) : 0;
}

int trmoe_weight_grad(int act_dtype, const void* a, int64_t lda, int64_t a_rows, const void* b, int64_t ldb,
                      int64_t b_rows, const int64_t* a_gather, const int64_t* b_gather, int64_t gather_mod,
                      int64_t m, int64_t n, int64_t n_rows, const int32_t* expert_offsets, int num_segments,
                      void* out, int64_t ldo, int64_t out_expert_stride, void* workspace, size_t workspace_bytes,
                      void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "weight_grad: bf16 or f32 only");
    TRMOE_REQUIRE(m > 0 && n > 0 && n_rows >= 0 && num_segments >= 1, "weight_grad: bad dimensions");
    TRMOE_REQUIRE(m % 8 == 0 && n % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0,
                  "weight_grad: m, n, lda and ldb must be multiples of 8");
    TRMOE_REQUIRE(lda >= m && ldb >= n && ldo >= n, "weight_grad: bad leading dimension");
    TRMOE_REQUIRE(num_segments == 1 || expert_offsets != nullptr, "weight_grad: segments need expert_offsets");
    TRMOE_REQUIRE(num_segments == 1 || out_expert_stride >= m * ldo, "weight_grad: out_expert_stride too small");
    TRMOE_REQUIRE((a_gather == nullptr && b_gather == nullptr) || gather_mod > 0, "weight_grad: gather_mod");
    TRMOE_REQUIRE(a && b && out, "weight_grad: null pointer");
    const int eb = elem_bytes(act_dtype);
    TRMOE_REQUIRE(aligned16(a) && aligned16(b), "weight_grad: operands must be 16-byte aligned");
    if (a_rows * lda * eb >= ((int64_t)1 << 31) || b_rows * ldb * eb >= ((int64_t)1 << 31))
        return set_error(TRMOE_ERR_UNSUPPORTED, "weight_grad: operands must be smaller than 2 GiB");
    TRMOE_REQUIRE(a_gather == nullptr || gather_mod <= a_rows, "weight_grad: gather_mod > a_rows");
    TRMOE_REQUIRE(b_gather == nullptr || gather_mod <= b_rows, "weight_grad: gather_mod > b_rows");
    TRMOE_REQUIRE(a_gather != nullptr || a_rows >= n_rows, "weight_grad: a_rows < n_rows");
    TRMOE_REQUIRE(b_gather != nullptr || b_rows >= n_rows, "weight_grad: b_rows < n_rows");
    TRMOE_REQUIRE(n_rows < ((int64_t)1 << 31), "weight_grad: too many rows");
    WgradArgs w{};
    w.a = a;
    w.lda = lda;
    w.a_rows = a_rows;
    w.b = b;
    w.ldb = ldb;
    w.b_rows = b_rows;
    w.a_gather = a_gather;
    w.b_gather = b_gather;
    w.gather_mod = gather_mod > 0 ? gather_mod : 1;
    w.M = m;
    w.N = n;
    w.T = n_rows;
    w.offsets = num_segments > 1 || expert_offsets != nullptr ? expert_offsets : nullptr;
    w.E = num_segments;
    w.out = out;
    w.ldo = ldo;
    w.out_expert_stride = out_expert_stride;
    const size_t need = trmoe_weight_grad_workspace_bytes(act_dtype, m, n, num_segments, n_rows);
    if (need > 0 && workspace != nullptr && workspace_bytes >= need) {
        TRMOE_REQUIRE(aligned16(workspace), "weight_grad: workspace must be 16-byte aligned");
        w.splits = wgrad_splits(m, n, num_segments, n_rows / num_segments);
        w.partial = static_cast<float*>(workspace);
    } else {
        w.splits = 1;
        w.partial = nullptr;
    }
    return launch_wgrad(act_dtype, w, as_stream(stream));
}

size_t trmoe_weight_grad_mapped_workspace_bytes(int act_dtype, int64_t m, int64_t n, int64_t n_rows) {
    if (act_dtype != TRMOE_BF16 || m <= 0 || n <= 0 || n_rows < 0) return 0;
    const int splits = wgrad_splits(m, n, 1, n_rows);
    return (size_t)splits * m * n * sizeof(float);
}

int trmoe_weight_grad_mapped(int act_dtype, const void* a, int64_t lda, int64_t a_rows, const void* b, int64_t ldb,
                             int64_t b_rows, int64_t m, int64_t n, int64_t n_rows, int map_mode,
                             const int64_t* map_off, const int64_t* map_stride, void* out, int64_t out_elems,
                             void* workspace, size_t workspace_bytes, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_BF16, "weight_grad_mapped: bf16 only");
    TRMOE_REQUIRE(m > 0 && n > 0 && n_rows >= 0, "weight_grad_mapped: bad dimensions");
    TRMOE_REQUIRE(m % 8 == 0 && n % 8 == 0 && lda % 8 == 0 && ldb % 8 == 0,
                  "weight_grad_mapped: m, n, lda and ldb must be multiples of 8");
    TRMOE_REQUIRE(lda >= m && ldb >= n, "weight_grad_mapped: bad leading dimension");
    TRMOE_REQUIRE(map_mode == 1 || map_mode == 2, "weight_grad_mapped: map_mode must be 1 (rows) or 2 (columns)");
    TRMOE_REQUIRE(a && b && out && map_off && map_stride && workspace, "weight_grad_mapped: null pointer");
    TRMOE_REQUIRE(out_elems > 0, "weight_grad_mapped: out_elems must be positive");
    TRMOE_REQUIRE(aligned16(a) && aligned16(b) && aligned16(workspace),
                  "weight_grad_mapped: operands and workspace must be 16-byte aligned");
    if (a_rows * lda * 2 >= ((int64_t)1 << 31) || b_rows * ldb * 2 >= ((int64_t)1 << 31))
        return set_error(TRMOE_ERR_UNSUPPORTED, "weight_grad_mapped: operands must be smaller than 2 GiB");
    TRMOE_REQUIRE(a_rows >= n_rows && b_rows >= n_rows && n_rows < ((int64_t)1 << 31),
                  "weight_grad_mapped: operands have fewer than n_rows rows");
    const size_t need = trmoe_weight_grad_mapped_workspace_bytes(act_dtype, m, n, n_rows);
    TRMOE_REQUIRE(workspace_bytes >= need, "weight_grad_mapped: workspace too small");
    WgradArgs w{};
    w.a = a;
    w.lda = lda;
    w.a_rows = a_rows;
    w.b = b;
    w.ldb = ldb;
    w.b_rows = b_rows;
    w.gather_mod = 1;
    w.M = m;
    w.N = n;
    w.T = n_rows;
    w.E = 1;
    w.out = out;
    w.ldo = n;
    w.out_expert_stride = m * n;
    w.splits = wgrad_splits(m, n, 1, n_rows);
    w.partial = static_cast<float*>(workspace);
    w.map_mode = map_mode;
    w.map_off = map_off;
    w.map_stride = map_stride;
    w.out_elems = out_elems;
    return launch_wgrad(act_dtype, w, as_stream(stream));
}

int trmoe_grouped_linear(int act_dtype, const void* h, int64_t ldh, int64_t n_rows, int64_t k,
                         const int32_t* expert_offsets, int num_experts, const void* w, int64_t out_features,
                         void* y, int64_t ldy, void* stream) {
    TRMOE_REQUIRE(act_dtype == TRMOE_F32 || act_dtype == TRMOE_BF16, "grouped_linear: bf16 or f32 only");
    TRMOE_REQUIRE(n_rows >= 0 && k > 0 && out_features > 0, "grouped_linear: bad dimensions");
    TRMOE_REQUIRE(num_experts >= 1 && num_experts <= kMaxExperts, "grouped_linear: bad num_experts");
    TRMOE_REQUIRE(ldh >= k && ldy >= out_features, "grouped_linear: bad leading dimension");
    TRMOE_REQUIRE(k < ((int64_t)1 << 30) && out_features < ((int64_t)1 << 30), "grouped_linear: too large");
    if (n_rows == 0) return TRMOE_OK;
    TRMOE_REQUIRE(h && expert_offsets && w && y, "grouped_linear: null pointer");
    const int eb = elem_bytes(act_dtype);
    TRMOE_REQUIRE(aligned16(w), "grouped_linear: packed weights must be 16-byte aligned");
    TRMOE_REQUIRE(rows_ok(h, ldh, eb), "grouped_linear: h rows must be 16-byte aligned");
    TRMOE_REQUIRE(aligned16(y) && (ldy * eb) % 16 == 0,
                  "grouped_linear: y must be 16-byte aligned with a row stride that is a multiple of 16 bytes");
    if (n_rows * ldh * eb >= ((int64_t)1 << 31))
        return set_error(TRMOE_ERR_UNSUPPORTED, "grouped_linear: h must be smaller than 2 GiB");
    DownArgs d{};
    d.h = h;
    d.ldh = ldh;
    d.M = n_rows;
    d.K = (int)k;
    d.w = w;
    d.ldw = round_up(k, 8);
    d.N = (int)out_features;
    d.shared_scale = 1.0f;
    d.routed_scale = 0.0f;
    d.out = y;
    d.ldo = ldy;
    d.vec_ok = 1;
    d.offsets = expert_offsets;
    d.E = num_experts;
    d.w_expert_stride = round_up(out_features, 256) * d.ldw;
    return launch_down_grouped(act_dtype, act_dtype, d, n_rows, as_stream(stream));
}

int trmoe_stream_read(const void* src, int64_t bytes, uint32_t* sink, int sink_words, void* stream) {
    TRMOE_REQUIRE(src != nullptr && sink != nullptr, "stream_read: null pointer");
    TRMOE_REQUIRE(bytes > 0 && bytes % 16 == 0 && aligned16(src),
                  "stream_read: bytes must be a positive multiple of 16 and src 16-byte aligned");
    TRMOE_REQUIRE(sink_words >= 1 && sink_words <= 65535, "stream_read: sink_words must be in [1, 65535]");
    return launch_stream_read(src, bytes, sink, sink_words, as_stream(stream));
}

}  // extern "C"
