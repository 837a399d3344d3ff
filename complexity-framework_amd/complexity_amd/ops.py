"""Torch-tensor wrappers over the C ABI of libtrmoe (include/trmoe.h).

Every function here launches HIP kernels on the current stream of the
tensors' device and returns freshly allocated outputs (torch's caching
allocator); inputs are never modified.  The layer-level entry points and the
packers make the tensors' GPU current for the call (the library launches on
the current device); the per-kernel wrappers they chain expect it current
already.  There is no fallback: if the library is missing or a call fails, an
exception is raised.
"""

from __future__ import annotations

import ctypes
import functools
from dataclasses import dataclass, field
from typing import Optional, Sequence, Tuple

import torch

from . import _native as N

ORDER_TOKEN = N.ORDER_TOKEN
ORDER_ASSIGNMENT = N.ORDER_ASSIGNMENT

# Padding the packed layouts use (must match the kernel tiles).
SHARED_GATE_UP_ALIGN = 256   # rows = 2 * round_up(S, 128)
SKINNY_MAX_TOKENS = 128      # token counts the decode-shape kernels take
EXPERT_GATE_UP_ALIGN = 128   # rows = 2 * round_up(W, 64)
DOWN_ALIGN = 256             # rows = round_up(H, 256)

_DTYPES = {torch.float32: N.F32, torch.bfloat16: N.BF16, torch.float8_e4m3fn: N.FP8_E4M3}


def _round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise NotImplementedError(f"TR-MoE HIP kernels do not support {dtype}") from None


def _p(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(t: torch.Tensor):
    """torch's current stream on t's device, as the hipStream_t handle."""
    if _RAW_STREAM is not None:
        return ctypes.c_void_p(_RAW_STREAM(t.device.index))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _lib():
    return N.load()


def _on_tensor_device(fn):
    """Runs fn with the first tensor argument's GPU as torch's (and so HIP's)
    current device: the library launches on the current device, and a tensor
    on another GPU would otherwise get kernels of the wrong one."""
    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        for a in args:
            if isinstance(a, torch.Tensor):
                dev = a.device
                if dev.type == "cuda" and dev.index is not None and dev.index != torch.cuda.current_device():
                    with torch.cuda.device(dev):
                        return fn(*args, **kwargs)
                break
        return fn(*args, **kwargs)
    return wrapper


def rows16(x: torch.Tensor) -> torch.Tensor:
    """x[n, k] laid out as the kernels read activations: 16-byte-aligned rows,
    a row stride that is a multiple of 16 bytes, and zeros between k and the
    next multiple of 16 bytes (the kernels load whole 16-byte chunks).
    Returns x itself when it already qualifies, else a zero-padded copy."""
    elem = x.element_size()
    n, k = x.shape
    if (x.stride(1) == 1 and x.data_ptr() % 16 == 0 and (x.stride(0) * elem) % 16 == 0
            and (k * elem) % 16 == 0):
        return x
    ld = _round_up(k * elem, 16) // elem
    padded = torch.zeros(n, ld, dtype=x.dtype, device=x.device)
    padded[:, :k] = x
    return padded[:, :k]


def _require_cuda(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("TR-MoE HIP ops need tensors on a ROCm device")


# ---------------------------------------------------------------------------
# K1
# ---------------------------------------------------------------------------

@_on_tensor_device
def route_sort(token_ids: torch.Tensor, route_table: torch.Tensor, num_experts: int,
               order: int = ORDER_TOKEN, return_routes: bool = False):
    """(sorted int64[kN], inverse int64[kN], offsets int32[E+1], counts int32[E][, routes int64[k,N]])."""
    lib = _lib()
    _require_cuda(token_ids, route_table)
    ids = token_ids.reshape(-1)
    if ids.dtype != torch.int64:
        ids = ids.to(torch.int64)
    ids = ids.contiguous()
    table = route_table.contiguous()
    if table.dtype != torch.int64 or table.ndim != 2:
        raise ValueError("route_table must be int64 [top_k, vocab]")
    k, vocab = table.shape
    n = ids.numel()
    dev = ids.device
    sorted_idx = torch.empty(k * n, dtype=torch.int64, device=dev)
    inverse = torch.empty(k * n, dtype=torch.int64, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    routes = torch.empty(k, n, dtype=torch.int64, device=dev) if return_routes else None
    ws_bytes = lib.trmoe_route_sort_workspace_bytes(n, k, num_experts, order)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    st = lib.trmoe_route_sort(_p(ids), n, _p(table), vocab, k, num_experts, order, _p(routes),
                              _p(sorted_idx), _p(inverse), _p(offsets), _p(counts), _p(ws), ws_bytes,
                              _stream(ids))
    N.check(st, "trmoe_route_sort")
    if return_routes:
        return sorted_idx, inverse, offsets, counts, routes
    return sorted_idx, inverse, offsets, counts


# ---------------------------------------------------------------------------
# packing
# ---------------------------------------------------------------------------

def pack_dims(kind: int, out_features: int, in_features: int, row_align: int) -> Tuple[int, int]:
    lib = _lib()
    rows, cols = ctypes.c_int64(), ctypes.c_int64()
    N.check(lib.trmoe_pack_dims(kind, out_features, in_features, row_align, ctypes.byref(rows),
                                ctypes.byref(cols)), "trmoe_pack_dims")
    return rows.value, cols.value


def _pack(kind: int, a: torch.Tensor, b: Optional[torch.Tensor], groups: int, out_f: int, in_f: int,
          strides: Tuple[int, int, int], row_align: int, scale_a=None, scale_b=None,
          into: Optional[torch.Tensor] = None, dst_ld: int = 0, dst_group_stride: int = 0):
    """Scales are [groups, out_f] (or [out_f] for one group); made contiguous here.

    ``into`` (a view whose data pointer is the first packed element) writes
    the groups into a larger packed tensor with the given element strides."""
    lib = _lib()
    _require_cuda(a, b)
    rows, cols = pack_dims(kind, out_f, in_f, row_align)
    dst = torch.empty(groups, rows, cols, dtype=a.dtype, device=a.device) if into is None else into
    dst_scale = None
    scale_stride = 0
    if scale_a is not None:
        dst_scale = torch.empty(groups, rows, dtype=torch.float32, device=a.device)
        scale_a = scale_a.float().contiguous().reshape(groups, out_f)
        scale_b = scale_b.float().contiguous().reshape(groups, out_f) if scale_b is not None else None
        scale_stride = out_f
    st = lib.trmoe_pack_weight(kind, dtype_code(a.dtype), _p(a), _p(b), groups, out_f, in_f,
                               strides[0], strides[1], strides[2], _p(scale_a), _p(scale_b),
                               scale_stride, row_align, _p(dst), dst_ld, dst_group_stride, _p(dst_scale), 0,
                               _stream(a))
    N.check(st, "trmoe_pack_weight")
    return dst, dst_scale


@_on_tensor_device
def pack_linear_gate_up(w_gate: torch.Tensor, w_up: torch.Tensor, scale_gate=None, scale_up=None):
    """nn.Linear weights [S, H] (gate, up) -> packed [2*round_up(S,128), round_up(H,8)]."""
    S, H = w_gate.shape
    if w_up.shape != w_gate.shape or w_up.stride() != w_gate.stride():
        raise ValueError("gate and up weights must have the same shape and strides")
    dst, sc = _pack(N.PACK_GATE_UP, w_gate, w_up, 1, S, H, (0, w_gate.stride(0), w_gate.stride(1)),
                    SHARED_GATE_UP_ALIGN, scale_gate, scale_up)
    return dst[0], (sc[0] if sc is not None else None)


@_on_tensor_device
def pack_linear_down(w_down: torch.Tensor, scale=None):
    """nn.Linear weight [H, S] -> packed [round_up(H,256), round_up(S,8)]."""
    H, S = w_down.shape
    dst, sc = _pack(N.PACK_PLAIN, w_down, None, 1, H, S, (0, w_down.stride(0), w_down.stride(1)),
                    DOWN_ALIGN, scale, None)
    return dst[0], (sc[0] if sc is not None else None)


@_on_tensor_device
def pack_expert_gate_up(gate: torch.Tensor, up: torch.Tensor, scale_gate=None, scale_up=None):
    """Expert tensors [E, H, W] (any strides, e.g. an active-capacity slice)
    -> packed [E, 2*round_up(W,64), round_up(H,8)]; scales [E, W] (stride given)."""
    E, H, W = gate.shape
    if up.shape != gate.shape or up.stride() != gate.stride():
        raise ValueError("gate and up expert weights must have the same shape and strides")
    return _pack(N.PACK_GATE_UP, gate, up, E, W, H, (gate.stride(0), gate.stride(2), gate.stride(1)),
                 EXPERT_GATE_UP_ALIGN, scale_gate, scale_up)


@_on_tensor_device
def pack_expert_down(down: torch.Tensor, scale=None):
    """Expert down [E, W, H] -> packed [E, round_up(H,256), round_up(W,8)]; scale [E, H]."""
    E, W, H = down.shape
    return _pack(N.PACK_PLAIN, down, None, E, H, W, (down.stride(0), down.stride(2), down.stride(1)),
                 DOWN_ALIGN, scale, None)


def dense_routed_features(shared_width: int, num_experts: int, expert_width: int) -> int:
    return int(_lib().trmoe_dense_routed_features(shared_width, num_experts, expert_width))


@_on_tensor_device
def pack_dense_routed(shared_gate, shared_up, shared_down, gate, up, down):
    """Fused weights of the dense-routed strategy (bf16 / f32 only).

    gate|up: shared features then each expert's, GATE_UP-interleaved,
    [2F, round_up(H, 8)]; down: [round_up(H, 256), F] with shared_down.weight
    in columns [0, S) and expert e's down^T at column round_up(S,128) +
    e*round_up(W,64).  F = dense_routed_features(S, E, W); gaps are zero.
    Expert tensors may be active-capacity slices [E', H, W'] / [E', W', H]."""
    E, H, W = gate.shape
    S = 0 if shared_gate is None else shared_gate.shape[0]
    F = dense_routed_features(S, E, W)
    s_pad, w_pad = _round_up(S, 128), _round_up(W, 64)
    cols = _round_up(H, 8)
    dev, dt = gate.device, gate.dtype
    gu = torch.zeros(2 * F, cols, dtype=dt, device=dev)
    dd = torch.zeros(_round_up(H, DOWN_ALIGN), F, dtype=dt, device=dev)
    if S:
        if shared_up.stride() != shared_gate.stride():
            raise ValueError("shared gate and up weights must have the same strides")
        _pack(N.PACK_GATE_UP, shared_gate, shared_up, 1, S, H, (0, shared_gate.stride(0), shared_gate.stride(1)),
              SHARED_GATE_UP_ALIGN, into=gu, dst_ld=cols)
        _pack(N.PACK_PLAIN, shared_down, None, 1, H, S, (0, shared_down.stride(0), shared_down.stride(1)),
              DOWN_ALIGN, into=dd, dst_ld=F)
    if up.stride() != gate.stride():
        raise ValueError("gate and up expert weights must have the same strides")
    _pack(N.PACK_GATE_UP, gate, up, E, W, H, (gate.stride(0), gate.stride(2), gate.stride(1)),
          EXPERT_GATE_UP_ALIGN, into=gu[2 * s_pad:], dst_ld=cols, dst_group_stride=2 * w_pad * cols)
    _pack(N.PACK_PLAIN, down, None, E, H, W, (down.stride(0), down.stride(2), down.stride(1)),
          DOWN_ALIGN, into=dd[:, s_pad:], dst_ld=F, dst_group_stride=w_pad)
    return gu, dd, F


def dense_routed_gate_up(x: torch.Tensor, w_packed: torch.Tensor, shared_width: int, num_experts: int,
                         expert_width: int, token_ids: torch.Tensor, route_table: torch.Tensor,
                         route_weights: Sequence[float], shared_scale: float, routed_scale: float,
                         save: bool = False, row_scale: Optional[torch.Tensor] = None, rms_eps: float = 0.0,
                         w_frag=None):
    """h_ext[N, F]: shared SwiGLU features and route-weighted expert features.
    save: also return the raw gate|up outputs gu[N, 2F] (packed column order).
    row_scale / rms_eps: fused RMSNorm; w_frag: (pack_fragments copy, cols) for
    decode sizes (trmoe_dense_routed_gate_up_ex)."""
    lib = _lib()
    _require_cuda(x, w_packed, token_ids, route_table)
    x = rows16(x)
    n, hidden = x.shape
    F = dense_routed_features(shared_width, num_experts, expert_width)
    ids = token_ids.reshape(-1)
    ids = (ids if ids.dtype == torch.int64 else ids.to(torch.int64)).contiguous()
    table = route_table.contiguous()
    h = torch.empty(n, F, dtype=x.dtype, device=x.device)
    rw = _weights_arg(route_weights)
    if save:
        gu = torch.empty(n, 2 * F, dtype=x.dtype, device=x.device)
        st = lib.trmoe_dense_routed_gate_up_save(dtype_code(x.dtype), _p(x), n, hidden, x.stride(0), _p(w_packed),
                                                 shared_width, num_experts, expert_width, _p(ids), _p(table),
                                                 table.shape[1], table.shape[0], ctypes.cast(rw, ctypes.c_void_p),
                                                 float(shared_scale), float(routed_scale), _p(h), F, _p(gu), 2 * F,
                                                 _stream(x))
        N.check(st, "trmoe_dense_routed_gate_up_save")
        return h, gu
    if row_scale is not None or rms_eps > 0.0 or w_frag is not None:
        ex, _keep = _extras(row_scale, rms_eps, w_frag)
        st = lib.trmoe_dense_routed_gate_up_ex(dtype_code(x.dtype), dtype_code(w_packed.dtype), _p(x), n, hidden,
                                               x.stride(0), _p(w_packed), None, shared_width, num_experts,
                                               expert_width, _p(ids), _p(table), table.shape[1], table.shape[0],
                                               ctypes.cast(rw, ctypes.c_void_p), float(shared_scale),
                                               float(routed_scale), _p(h), F, ex, _stream(x))
        N.check(st, "trmoe_dense_routed_gate_up_ex")
        return h
    st = lib.trmoe_dense_routed_gate_up(dtype_code(x.dtype), dtype_code(w_packed.dtype), _p(x), n, hidden,
                                        x.stride(0), _p(w_packed), None, shared_width, num_experts, expert_width,
                                        _p(ids), _p(table), table.shape[1], table.shape[0],
                                        ctypes.cast(rw, ctypes.c_void_p), float(shared_scale),
                                        float(routed_scale), _p(h), F, _stream(x))
    N.check(st, "trmoe_dense_routed_gate_up")
    return h


# ---------------------------------------------------------------------------
# compute
# ---------------------------------------------------------------------------

def shared_gate_up(x: torch.Tensor, w_packed: torch.Tensor, w_scale: Optional[torch.Tensor],
                   shared_width: int, save: bool = False, row_scale: Optional[torch.Tensor] = None,
                   rms_eps: float = 0.0, w_frag=None):
    """h[N, round_up(S,128)] = silu(x Wg^T) * (x Wu^T).  save: also return the
    raw gate|up outputs gu[N, 2 round_up(S,128)] (bf16/f32 weights).
    row_scale / rms_eps: fused RMSNorm; w_frag: (pack_fragments copy, cols)
    for decode sizes (trmoe_shared_gate_up_ex)."""
    lib = _lib()
    _require_cuda(x, w_packed)
    x = rows16(x)
    n, hidden = x.shape
    ldh = _round_up(shared_width, 128)
    h = torch.empty(n, ldh, dtype=x.dtype, device=x.device)
    if save:
        gu = torch.empty(n, 2 * ldh, dtype=x.dtype, device=x.device)
        st = lib.trmoe_shared_gate_up_save(dtype_code(x.dtype), _p(x), n, hidden, x.stride(0), _p(w_packed),
                                           shared_width, _p(h), ldh, _p(gu), 2 * ldh, _stream(x))
        N.check(st, "trmoe_shared_gate_up_save")
        return h, gu
    if row_scale is not None or rms_eps > 0.0 or w_frag is not None:
        ex, _keep = _extras(row_scale, rms_eps, w_frag)
        st = lib.trmoe_shared_gate_up_ex(dtype_code(x.dtype), dtype_code(w_packed.dtype), _p(x), n, hidden,
                                         x.stride(0), _p(w_packed), _p(w_scale), shared_width, _p(h), ldh, ex,
                                         _stream(x))
        N.check(st, "trmoe_shared_gate_up_ex")
        return h
    st = lib.trmoe_shared_gate_up(dtype_code(x.dtype), dtype_code(w_packed.dtype), _p(x), n, hidden,
                                  x.stride(0), _p(w_packed), _p(w_scale), shared_width, _p(h), ldh,
                                  _stream(x))
    N.check(st, "trmoe_shared_gate_up")
    return h


@_on_tensor_device
def quantize_rows_e4m3(x: torch.Tensor):
    """(q float8_e4m3fn [N, K], scale fp32 [N]): each row of x quantized as
    the engine quantizes weight rows (scale = amax / 448, 1 for a zero row;
    q = e4m3(clamp(x / scale, +-448)), ties to even)."""
    lib = _lib()
    _require_cuda(x)
    if x.dtype not in RMSNORM_MAX_HIDDEN:
        raise ValueError(f"quantize_rows_e4m3: bf16 or f32 rows, not {x.dtype}")
    x = _rows(x)
    n, k = x.shape
    ldq = _round_up(k, 16)
    q = torch.empty(n, ldq, dtype=torch.float8_e4m3fn, device=x.device)[:, :k]
    scale = torch.empty(n, dtype=torch.float32, device=x.device)
    st = lib.trmoe_quantize_rows_e4m3(dtype_code(x.dtype), _p(x), n, k, x.stride(0), _p(q), ldq, _p(scale),
                                      _stream(x))
    N.check(st, "trmoe_quantize_rows_e4m3")
    return q, scale


@_on_tensor_device
def shared_gate_up_a8(xq: torch.Tensor, x_scale: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                      shared_width: int) -> torch.Tensor:
    """W8A8 shared gate|up: h[N, round_up(S,128)] bf16 = silu(g) * u with
    [g|u] = (x_scale * xq) (w_scale * W8)^T on the e4m3 MFMA; xq, x_scale from
    quantize_rows_e4m3, w_packed / w_scale the layer's e4m3 pack."""
    lib = _lib()
    _require_cuda(xq, w_packed)
    if xq.dtype != torch.float8_e4m3fn or w_packed.dtype != torch.float8_e4m3fn:
        raise ValueError("shared_gate_up_a8: e4m3 activations and weights")
    n, hidden = xq.shape
    ldh = _round_up(shared_width, 128)
    h = torch.empty(n, ldh, dtype=torch.bfloat16, device=xq.device)
    st = lib.trmoe_shared_gate_up_a8(_p(xq), _p(x_scale.contiguous()), n, hidden, xq.stride(0), _p(w_packed),
                                     _p(w_scale), shared_width, _p(h), ldh, _stream(xq))
    N.check(st, "trmoe_shared_gate_up_a8")
    return h


@_on_tensor_device
def shared_gate_up_a8_mx(xq: torch.Tensor, x_scale: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                         shared_width: int):
    """W8A8 shared gate|up with h left as block-scaled e4m3: (h_q, h_scale)
    with h_q [N, round_up(S,128)] e4m3 codes and h_scale [N, round_up(S,128)
    / 32] uint8 E8M0 exponents, h = h_q * 2^(h_scale - 127) per block of 32
    features (trmoe_shared_gate_up_a8_mx: the smallest power of two that
    brings the block's maximum to 448 or below)."""
    lib = _lib()
    _require_cuda(xq, w_packed)
    if xq.dtype != torch.float8_e4m3fn or w_packed.dtype != torch.float8_e4m3fn:
        raise ValueError("shared_gate_up_a8_mx: e4m3 activations and weights")
    n, hidden = xq.shape
    f_pad = _round_up(shared_width, 128)
    h_q = torch.empty(n, f_pad, dtype=torch.float8_e4m3fn, device=xq.device)
    h_s = torch.empty(n, f_pad // 32, dtype=torch.uint8, device=xq.device)
    st = lib.trmoe_shared_gate_up_a8_mx(_p(xq), _p(x_scale.contiguous()), n, hidden, xq.stride(0), _p(w_packed),
                                        _p(w_scale), shared_width, _p(h_q), f_pad, _p(h_s), f_pad // 32, _stream(xq))
    N.check(st, "trmoe_shared_gate_up_a8_mx")
    return h_q, h_s


@_on_tensor_device
def shared_down_combine_a8(h_q: torch.Tensor, h_scale: torch.Tensor, shared_width: int, w_down: torch.Tensor,
                           w_scale: torch.Tensor, hidden: int, y: Optional[torch.Tensor],
                           inverse: Optional[torch.Tensor], top_k: int, route_weights: Sequence[float],
                           shared_scale: float, routed_scale: float,
                           residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    """shared_down_combine on block-scaled e4m3 h (shared_gate_up_a8_mx's
    outputs) and the layer's e4m3 down pack: bf16 out [N, hidden]; S a
    multiple of 128."""
    lib = _lib()
    _require_cuda(h_q, h_scale, w_down, y, inverse, residual)
    if h_q.dtype != torch.float8_e4m3fn or w_down.dtype != torch.float8_e4m3fn or h_scale.dtype != torch.uint8:
        raise ValueError("shared_down_combine_a8: e4m3 h and weights, uint8 scales")
    n = h_q.shape[0]
    out = torch.empty(n, hidden, dtype=torch.bfloat16, device=h_q.device)
    rw = _weights_arg(route_weights)
    st = lib.trmoe_shared_down_combine_a8(
        _p(h_q), _p(h_scale), n, shared_width, h_q.stride(0), h_scale.stride(0), _p(w_down), _p(w_scale), hidden,
        _p(y), hidden, _p(inverse), top_k, ctypes.cast(rw, ctypes.c_void_p), float(shared_scale),
        float(routed_scale), _p(residual), residual.stride(0) if residual is not None else 0, _p(out), hidden,
        _stream(h_q))
    N.check(st, "trmoe_shared_down_combine_a8")
    return out


def routed_experts(x: torch.Tensor, sorted_idx: torch.Tensor, offsets: torch.Tensor, num_experts: int,
                   top_k: int, w_gate_up: torch.Tensor, s_gate_up, w_down: torch.Tensor, s_down,
                   expert_width: int, two_pass: bool = True,
                   row_scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y[k*N, H] in partition order.  two_pass: grouped gate|up and down
    GEMMs through a workspace (the default when y rows are 16-byte aligned);
    False: the fused per-tile kernel.  row_scale: fused RMSNorm scales
    (trmoe_routed_experts_rms, two-pass only)."""
    lib = _lib()
    _require_cuda(x, sorted_idx, offsets, w_gate_up, w_down)
    x = rows16(x)
    n, hidden = x.shape
    y = torch.empty(top_k * n, hidden, dtype=x.dtype, device=x.device)
    ws, ws_bytes = None, 0
    if two_pass and (hidden * x.element_size()) % 16 == 0:
        ws_bytes = lib.trmoe_routed_experts_workspace_bytes(dtype_code(x.dtype), top_k * n, expert_width)
        if ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    if row_scale is not None:
        st = lib.trmoe_routed_experts_rms(dtype_code(x.dtype), dtype_code(w_gate_up.dtype), _p(x), n, hidden,
                                          x.stride(0), _p(sorted_idx), _p(offsets), num_experts, top_k,
                                          _p(w_gate_up), _p(s_gate_up), _p(w_down), _p(s_down), expert_width,
                                          _p(row_scale), _p(y), hidden, _p(ws), ws_bytes, _stream(x))
        N.check(st, "trmoe_routed_experts_rms")
        return y
    st = lib.trmoe_routed_experts(dtype_code(x.dtype), dtype_code(w_gate_up.dtype), _p(x), n, hidden,
                                  x.stride(0), _p(sorted_idx), _p(offsets), num_experts, top_k,
                                  _p(w_gate_up), _p(s_gate_up), _p(w_down), _p(s_down), expert_width,
                                  _p(y), hidden, _p(ws), ws_bytes, _stream(x))
    N.check(st, "trmoe_routed_experts")
    return y


@_on_tensor_device
def rms_row_scale(x: torch.Tensor, eps: float) -> torch.Tensor:
    """r[N] fp32 = 1 / sqrt(mean_k x[t, k]^2 + eps): the per-token factor of
    RMSNorm (complexity/core/normalization/norms.py:53-54)."""
    lib = _lib()
    _require_cuda(x)
    x = rows16(x)
    n, hidden = x.shape
    r = torch.empty(n, dtype=torch.float32, device=x.device)
    st = lib.trmoe_rms_row_scale(dtype_code(x.dtype), _p(x), n, hidden, x.stride(0), float(eps), _p(r), _stream(x))
    N.check(st, "trmoe_rms_row_scale")
    return r


# Largest hidden size of the RMSNorm kernels (one row per wave, in registers).
RMSNORM_MAX_HIDDEN = {torch.bfloat16: 4096, torch.float32: 2048}


def rmsnorm_unsupported(x: torch.Tensor, weight: torch.Tensor) -> Optional[str]:
    """Why trmoe_rmsnorm_* cannot take (x, weight) (None when it can)."""
    if x.dtype not in RMSNORM_MAX_HIDDEN:
        return f"RMSNorm kernels take bf16 or f32 activations, not {x.dtype}"
    if weight.dtype != x.dtype:
        return f"RMSNorm kernels need the norm weight in the activation dtype ({weight.dtype} vs {x.dtype})"
    hidden = x.shape[-1]
    if (hidden * x.element_size()) % 16 or hidden > RMSNORM_MAX_HIDDEN[x.dtype]:
        return (f"RMSNorm kernels need hidden to be a multiple of 16 bytes of elements and at most "
                f"{RMSNORM_MAX_HIDDEN[x.dtype]} ({hidden})")
    return None


def _rows(x: torch.Tensor) -> torch.Tensor:
    """x[n, k] with unit column stride, 16-byte aligned rows and a row stride
    that is a multiple of 16 bytes (k * elem is one already)."""
    if x.stride(1) == 1 and x.data_ptr() % 16 == 0 and (x.stride(0) * x.element_size()) % 16 == 0:
        return x
    return x.contiguous() if x.data_ptr() % 16 == 0 else x.clone(memory_format=torch.contiguous_format)


def _vec16(w: torch.Tensor) -> torch.Tensor:
    w = w.contiguous()
    return w if w.data_ptr() % 16 == 0 else w.clone()


@_on_tensor_device
def rmsnorm_forward(x: torch.Tensor, weight: torch.Tensor, eps: float):
    """(y, r): y = T(x * r) * weight with r[N] fp32 = 1 / sqrt(mean(x^2) + eps),
    the reference's RMSNorm (complexity/core/normalization/norms.py:46-55, the
    liger-kernel "llama" casting it calls on CUDA); r is what the backward
    needs."""
    lib = _lib()
    _require_cuda(x)
    reason = rmsnorm_unsupported(x, weight)
    if reason:
        raise ValueError(reason)
    x = _rows(x)
    weight = _vec16(weight)
    n, hidden = x.shape
    y = torch.empty(n, hidden, dtype=x.dtype, device=x.device)
    r = torch.empty(n, dtype=torch.float32, device=x.device)
    st = lib.trmoe_rmsnorm_forward(dtype_code(x.dtype), _p(x), n, hidden, x.stride(0), _p(weight), float(eps),
                                   _p(y), hidden, _p(r), _stream(x))
    N.check(st, "trmoe_rmsnorm_forward")
    return y, r


@_on_tensor_device
def rmsnorm_backward(x: torch.Tensor, weight: torch.Tensor, r: torch.Tensor, dy: torch.Tensor,
                     dres: Optional[torch.Tensor] = None):
    """(dx, dweight) of rmsnorm_forward for the output gradient dy; dres, when
    given, is added to dx (the residual branch's gradient of the same x)."""
    lib = _lib()
    _require_cuda(x)
    reason = rmsnorm_unsupported(x, weight)
    if reason:
        raise ValueError(reason)
    x, dy = _rows(x), _rows(dy.to(x.dtype))
    dres = None if dres is None else _rows(dres.to(x.dtype))
    weight = _vec16(weight)
    r = r.contiguous()
    n, hidden = x.shape
    code = dtype_code(x.dtype)
    dx = torch.empty(n, hidden, dtype=x.dtype, device=x.device)
    dw = torch.empty(hidden, dtype=x.dtype, device=x.device)
    ws_bytes = lib.trmoe_rmsnorm_backward_workspace_bytes(code, n, hidden)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    st = lib.trmoe_rmsnorm_backward(code, _p(x), n, hidden, x.stride(0), _p(weight), _p(r), _p(dy), dy.stride(0),
                                    _p(dres), dres.stride(0) if dres is not None else 0, _p(dx), hidden, _p(dw),
                                    _p(ws), ws_bytes, _stream(x))
    N.check(st, "trmoe_rmsnorm_backward")
    return dx, dw


def _extras(row_scale: Optional[torch.Tensor] = None, rms_eps: float = 0.0, w_frag=None):
    """trmoe_call_extras for the *_ex calls; w_frag = (fragment copy, cols)."""
    e = N.CallExtras()
    e.row_scale = _p(row_scale)
    e.rms_eps = float(rms_eps)
    if w_frag is not None:
        e.w_frag = _p(w_frag[0])
        e.w_frag_cols = int(w_frag[1])
    return ctypes.byref(e), e


@_on_tensor_device
def pack_fragments(w_packed: torch.Tensor, cols: int) -> tuple:
    """(fragment-major copy of a packed bf16/f32 weight, cols) for the decode
    kernels (trmoe_pack_fragments); cols is the K of the calls that use it."""
    lib = _lib()
    _require_cuda(w_packed)
    rows, ld = w_packed.shape
    nbytes = lib.trmoe_fragment_bytes(dtype_code(w_packed.dtype), rows, cols)
    if nbytes == 0:
        raise ValueError("pack_fragments: bf16/f32 weights with rows % 16 == 0")
    dst = torch.empty(nbytes, dtype=torch.uint8, device=w_packed.device)
    st = lib.trmoe_pack_fragments(dtype_code(w_packed.dtype), _p(w_packed), rows, cols, ld, _p(dst),
                                  _stream(w_packed))
    N.check(st, "trmoe_pack_fragments")
    return dst, int(cols)


def _weights_arg(route_weights: Sequence[float]):
    arr = (ctypes.c_float * 4)(*[float(w) for w in list(route_weights)[:4]])
    return arr


# Scratch of the decode-sized down GEMM (split-K partials): one cached buffer
# per (device, stream), so that calls on one stream (which are ordered) share
# it and no call allocates after the first.  Inside a `workspace_scope` the
# scope's own buffer is used instead: a captured graph bakes the buffer's
# address into its launches, so every graph owns one (two graphs replayed on
# different streams then never share partials).
_DOWN_WS: dict = {}
_WS_SCOPE: list = []


class workspace_scope:
    """Context in which the down GEMM's split-K scratch comes from this object
    (grown on demand) rather than the per-stream cache.  Keep the object alive
    as long as anything recorded inside the scope (a graph) may run."""

    def __init__(self):
        self.buffer: Optional[torch.Tensor] = None

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        if self.buffer is None or self.buffer.device != device or self.buffer.numel() < nbytes:
            self.buffer = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        return self.buffer

    def __enter__(self):
        _WS_SCOPE.append(self)
        return self

    def __exit__(self, *exc):
        _WS_SCOPE.remove(self)


def _down_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    if _WS_SCOPE:
        return _WS_SCOPE[-1].get(device, nbytes)
    key = (device.index, _RAW_STREAM(device.index) if _RAW_STREAM is not None
           else torch.cuda.current_stream(device).cuda_stream)
    ws = _DOWN_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _DOWN_WS[key] = ws
    return ws


def shared_down_combine(h: torch.Tensor, shared_width: int, w_down: torch.Tensor, w_scale, hidden: int,
                        y: Optional[torch.Tensor], inverse: Optional[torch.Tensor], top_k: int,
                        route_weights: Sequence[float], shared_scale: float, routed_scale: float,
                        residual: Optional[torch.Tensor] = None, w_frag=None) -> torch.Tensor:
    """out = shared_scale * h Wd^T + routed_scale * combine(y) (+ residual);
    w_frag: (pack_fragments copy of w_down, shared_width) for decode sizes."""
    lib = _lib()
    _require_cuda(h, w_down, y, inverse, residual)
    n = h.shape[0]
    out = torch.empty(n, hidden, dtype=h.dtype, device=h.device)
    rw = _weights_arg(route_weights)
    ws_bytes = lib.trmoe_shared_down_combine_workspace_bytes(dtype_code(h.dtype), n, shared_width, hidden)
    ws = _down_workspace(h.device, ws_bytes) if ws_bytes else None
    if w_frag is not None:
        ex, _keep = _extras(w_frag=w_frag)
        st = lib.trmoe_shared_down_combine_ex(
            dtype_code(h.dtype), dtype_code(w_down.dtype), _p(h), n, shared_width, h.stride(0), _p(w_down),
            _p(w_scale), hidden, _p(y), hidden, _p(inverse), top_k, ctypes.cast(rw, ctypes.c_void_p),
            float(shared_scale), float(routed_scale), _p(residual),
            residual.stride(0) if residual is not None else 0, _p(out), hidden, _p(ws), ws_bytes, ex, _stream(h))
        N.check(st, "trmoe_shared_down_combine_ex")
        return out
    st = lib.trmoe_shared_down_combine(
        dtype_code(h.dtype), dtype_code(w_down.dtype), _p(h), n, shared_width, h.stride(0), _p(w_down),
        _p(w_scale), hidden, _p(y), hidden, _p(inverse), top_k, ctypes.cast(rw, ctypes.c_void_p),
        float(shared_scale), float(routed_scale), _p(residual),
        residual.stride(0) if residual is not None else 0, _p(out), hidden, _p(ws), ws_bytes, _stream(h))
    N.check(st, "trmoe_shared_down_combine")
    return out


def stream_read(src: torch.Tensor, sink: torch.Tensor) -> None:
    """One launch that reads src's bytes once (trmoe_stream_read): the
    single-launch streaming floor the decode kernels are compared with.
    sink: int32 [G], G workgroups; word g receives the XOR of the 32-bit words
    workgroup g read."""
    lib = _lib()
    _require_cuda(src, sink)
    if not src.is_contiguous() or sink.dtype != torch.int32:
        raise ValueError("stream_read: contiguous src and an int32 sink")
    nbytes = src.numel() * src.element_size()
    st = lib.trmoe_stream_read(_p(src), nbytes, _p(sink), sink.numel(), _stream(src))
    N.check(st, "trmoe_stream_read")


def combine(y: torch.Tensor, inverse: torch.Tensor, n_tokens: int, top_k: int,
            route_weights: Sequence[float], routed_scale: float,
            residual: Optional[torch.Tensor] = None) -> torch.Tensor:
    lib = _lib()
    _require_cuda(y, inverse, residual)
    hidden = y.shape[1]
    out = torch.empty(n_tokens, hidden, dtype=y.dtype, device=y.device)
    rw = _weights_arg(route_weights)
    st = lib.trmoe_combine(dtype_code(y.dtype), n_tokens, hidden, _p(y), hidden, _p(inverse), top_k,
                           ctypes.cast(rw, ctypes.c_void_p), float(routed_scale), _p(residual),
                           residual.stride(0) if residual is not None else 0, _p(out), hidden, _stream(y))
    N.check(st, "trmoe_combine")
    return out


# ---------------------------------------------------------------------------
# whole layer
# ---------------------------------------------------------------------------

STRATEGY_GROUPED = "grouped"
STRATEGY_DENSE = "dense"


def choose_strategy(shared_width: int, num_experts: int, expert_width: int, top_k: int, fp8: bool) -> str:
    """Dense-routed when computing every expert for every token costs at most
    8% more MFMA work than the routed experts' own share (and the weights are
    not e4m3: the fused down rows would mix per-block scales)."""
    if fp8:
        return STRATEGY_GROUPED
    extra = (num_experts - top_k) * expert_width
    useful = shared_width + top_k * expert_width
    return STRATEGY_DENSE if extra <= 0.08 * useful else STRATEGY_GROUPED


@dataclass
class PackedLayer:
    """Weights of one layer in kernel layout (built by TRHashEngine)."""

    act_dtype: torch.dtype
    num_experts: int
    expert_width: int
    strategy: str = STRATEGY_GROUPED
    expert_gate_up: Optional[torch.Tensor] = None
    expert_gate_up_scale: Optional[torch.Tensor] = None
    expert_down: Optional[torch.Tensor] = None
    expert_down_scale: Optional[torch.Tensor] = None
    shared_width: int = 0
    shared_gate_up: Optional[torch.Tensor] = None
    shared_gate_up_scale: Optional[torch.Tensor] = None
    shared_down: Optional[torch.Tensor] = None
    shared_down_scale: Optional[torch.Tensor] = None
    dense_gate_up: Optional[torch.Tensor] = None     # dense-routed fused weights
    dense_down: Optional[torch.Tensor] = None
    dense_features: int = 0
    # fragment-major copies for decode-sized calls, built on first use:
    # name -> (copy, cols)
    frag: dict = field(default_factory=dict)

    @property
    def fp8(self) -> bool:
        """True when any packed weight holds e4m3 codes (inference-only)."""
        for name in ("expert_gate_up", "expert_down", "shared_gate_up", "shared_down", "dense_gate_up", "dense_down"):
            t = getattr(self, name)
            if t is not None and t.dtype == torch.float8_e4m3fn:
                return True
        return False

    def fragments(self, name: str, cols: int):
        """pack_fragments of the bf16/f32 weight `name` (None for fp8)."""
        if self.act_dtype not in (torch.bfloat16, torch.float32):
            return None
        w = getattr(self, name)
        if w is None or w.dtype != self.act_dtype:
            return None
        got = self.frag.get(name)
        if got is None:
            got = pack_fragments(w, cols)
            self.frag[name] = got
        return got


def fp8_activation_mode(mode):
    """The W8A8 switch: False, True (the shared gate|up and down on e4m3
    activations) or "gate_up" (the shared gate|up only)."""
    if mode is False or mode is True or mode == "gate_up":
        return mode
    raise ValueError(f"fp8_activations: False, True or 'gate_up', not {mode!r}")


@_on_tensor_device
def layer_forward(x: torch.Tensor, token_ids: torch.Tensor, route_table: torch.Tensor, packed: PackedLayer,
                  route_weights: Sequence[float], shared_scale: float, routed_scale: float,
                  order: int = ORDER_TOKEN, residual: Optional[torch.Tensor] = None, save: bool = False,
                  norm_eps: Optional[float] = None, act_fp8=False):
    """out[N, H] = shared_scale*shared(x) + routed_scale*routed(x) (+ residual).

    grouped: K1 partition, K3 grouped experts, K2 shared gate|up, K4 down with
    the un-permute in its epilogue.  dense: fused gate|up over shared and
    expert features with route-weighted expert outputs, then one down GEMM.
    norm_eps: the layer runs on rmsnorm(x) (the packs must hold the gate/up
    weights times the norm weight); the per-token scales come from the decode
    kernels themselves up to 128 tokens (dense strategy), else from
    rms_row_scale.  save: returns (out, gu, h): the raw gate|up outputs and,
    for the dense strategy, the down GEMM's input h (else None), which the
    backward reuses.  act_fp8 (e4m3 packs, grouped strategy, above decode
    sizes, hidden a multiple of 128): True or "gate_up": the shared gate|up
    runs W8A8 on x quantized per token (quantize_rows_e4m3,
    shared_gate_up_a8); True with S a multiple of 128: its h leaves as
    block-scaled e4m3 and the shared down runs W8A8 too
    (shared_gate_up_a8_mx, shared_down_combine_a8)."""
    n, hidden = x.shape
    top_k = route_table.shape[0]
    act_fp8 = fp8_activation_mode(act_fp8)
    if save and packed.fp8:
        raise ValueError("layer_forward: e4m3 weights are inference-only (no saved pre-activations, no backward)")
    if n == 0:
        out = torch.empty(0, hidden, dtype=x.dtype, device=x.device)
        return (out, None, None) if save else out
    x = rows16(x)
    gu = None
    rscale, eps_in = None, 0.0
    if norm_eps is not None:
        if save:
            raise ValueError("layer_forward: the fused RMSNorm is inference-only")
        if packed.strategy == STRATEGY_DENSE and n <= SKINNY_MAX_TOKENS:
            eps_in = float(norm_eps)
        else:
            rscale = rms_row_scale(x, norm_eps)
    # decode sizes read the weights through their fragment-major copies
    decode = n <= SKINNY_MAX_TOKENS and not save
    if packed.strategy == STRATEGY_DENSE:
        h = dense_routed_gate_up(x, packed.dense_gate_up, packed.shared_width, packed.num_experts,
                                 packed.expert_width, token_ids, route_table, route_weights, shared_scale,
                                 routed_scale, save=save, row_scale=rscale, rms_eps=eps_in,
                                 w_frag=packed.fragments("dense_gate_up", hidden) if decode else None)
        if save:
            h, gu = h
        out = shared_down_combine(h, packed.dense_features, packed.dense_down, None, hidden, None, None,
                                  top_k, route_weights, 1.0, 1.0, residual,
                                  w_frag=packed.fragments("dense_down", packed.dense_features) if decode else None)
        return (out, gu, h) if save else out
    sorted_idx, inverse, offsets, _ = route_sort(token_ids, route_table, packed.num_experts, order)
    y = routed_experts(x, sorted_idx, offsets, packed.num_experts, top_k, packed.expert_gate_up,
                       packed.expert_gate_up_scale, packed.expert_down, packed.expert_down_scale,
                       packed.expert_width, row_scale=rscale)
    if packed.shared_width > 0:
        if (act_fp8 and packed.shared_gate_up.dtype == torch.float8_e4m3fn and rscale is None and not decode
                and hidden % 128 == 0 and hidden <= RMSNORM_MAX_HIDDEN.get(x.dtype, 0)):
            xq, xs = quantize_rows_e4m3(x)
            if act_fp8 is True and packed.shared_width % 128 == 0:
                # h stays e4m3 (one power-of-two scale per 32 features) into the down
                h_q, h_s = shared_gate_up_a8_mx(xq, xs, packed.shared_gate_up, packed.shared_gate_up_scale,
                                                packed.shared_width)
                return shared_down_combine_a8(h_q, h_s, packed.shared_width, packed.shared_down,
                                              packed.shared_down_scale, hidden, y, inverse, top_k, route_weights,
                                              shared_scale, routed_scale, residual)
            h = shared_gate_up_a8(xq, xs, packed.shared_gate_up, packed.shared_gate_up_scale, packed.shared_width)
        else:
            h = shared_gate_up(x, packed.shared_gate_up, packed.shared_gate_up_scale, packed.shared_width,
                               save=save, row_scale=rscale,
                               w_frag=packed.fragments("shared_gate_up", hidden) if decode else None)
        if save:
            h, gu = h
        out = shared_down_combine(h, packed.shared_width, packed.shared_down, packed.shared_down_scale,
                                  hidden, y, inverse, top_k, route_weights, shared_scale, routed_scale,
                                  residual,
                                  w_frag=packed.fragments("shared_down", packed.shared_width) if decode else None)
    else:
        out = combine(y, inverse, n, top_k, route_weights, routed_scale, residual)
    return (out, gu, None) if save else out


# ---------------------------------------------------------------------------
# backward (bf16 / f32 weights)
# ---------------------------------------------------------------------------

@_on_tensor_device
def pack_linear_down_t(w_down: torch.Tensor) -> torch.Tensor:
    """shared_down.weight [H, S] -> W_down^T packed [round_up(S,128), round_up(H,8)]."""
    H, S = w_down.shape
    dst, _ = _pack(N.PACK_PLAIN, w_down, None, 1, S, H, (0, w_down.stride(1), w_down.stride(0)), 128)
    return dst[0]


@_on_tensor_device
def pack_expert_down_t(down: torch.Tensor) -> torch.Tensor:
    """Expert down [E, W, H] -> [E, round_up(W,64), round_up(H,8)] (rows = features)."""
    E, W, H = down.shape
    dst, _ = _pack(N.PACK_PLAIN, down, None, E, W, H, (down.stride(0), down.stride(1), down.stride(2)), 64)
    return dst


@_on_tensor_device
def pack_dense_down_t(dense_down: torch.Tensor, features: int, hidden: int) -> torch.Tensor:
    """The dense-routed packed down [round_up(H,256), F] -> [F, round_up(H,8)]."""
    dst, _ = _pack(N.PACK_PLAIN, dense_down, None, 1, features, hidden, (0, 1, dense_down.stride(0)), 64)
    return dst[0]


@_on_tensor_device
def pack_gate_up_t(gate_up_packed: torch.Tensor, hidden: int) -> torch.Tensor:
    """A GATE_UP pack [G, 2F, ld] (or [2F, ld]) -> its transpose [G, round_up(H,256), 2F]:
    the down-style weight of the data gradient [dg|du] . [Wg; Wu]."""
    single = gate_up_packed.dim() == 2
    p = gate_up_packed.unsqueeze(0) if single else gate_up_packed
    G, rows, ld = p.shape
    dst, _ = _pack(N.PACK_PLAIN, p, None, G, hidden, rows, (p.stride(0), 1, ld), DOWN_ALIGN)
    return dst[0] if single else dst


def shared_swiglu_backward(x: torch.Tensor, dout: torch.Tensor, w_gate_up: torch.Tensor, w_down_t: torch.Tensor,
                           shared_width: int, shared_scale: float, gu: Optional[torch.Tensor] = None):
    """(dgu[N, 2F], hm[N, F]) of the shared SwiGLU, F = round_up(S, 128); gu:
    the forward's saved gate|up outputs (None: recomputed from x)."""
    lib = _lib()
    _require_cuda(x, dout, w_gate_up, w_down_t)
    n, hidden = x.shape
    F_ = _round_up(shared_width, 128)
    dgu = torch.empty(n, 2 * F_, dtype=x.dtype, device=x.device)
    hm = torch.empty(n, F_, dtype=x.dtype, device=x.device)
    st = lib.trmoe_shared_swiglu_backward(dtype_code(x.dtype), _p(x), _p(dout), n, hidden, x.stride(0),
                                          dout.stride(0), _p(w_gate_up), _p(w_down_t), shared_width,
                                          float(shared_scale), _p(gu), 0 if gu is None else gu.stride(0), _p(dgu),
                                          2 * F_, _p(hm), F_, _stream(x))
    N.check(st, "trmoe_shared_swiglu_backward")
    return dgu, hm


def dense_routed_swiglu_backward(x, dout, w_gate_up, w_down_t, shared_width, num_experts, expert_width,
                                 token_ids, route_table, route_weights, shared_scale, routed_scale, gu=None,
                                 want_hm: bool = True):
    """(dgu[N, 2F], hm[N, F]) over the dense-routed features; hm is None
    (not computed) without want_hm."""
    lib = _lib()
    _require_cuda(x, dout, w_gate_up, w_down_t, token_ids, route_table)
    n, hidden = x.shape
    F_ = dense_routed_features(shared_width, num_experts, expert_width)
    ids = token_ids.reshape(-1)
    ids = (ids if ids.dtype == torch.int64 else ids.to(torch.int64)).contiguous()
    table = route_table.contiguous()
    dgu = torch.empty(n, 2 * F_, dtype=x.dtype, device=x.device)
    hm = torch.empty(n, F_, dtype=x.dtype, device=x.device) if want_hm else None
    rw = _weights_arg(route_weights)
    st = lib.trmoe_dense_routed_swiglu_backward(dtype_code(x.dtype), _p(x), _p(dout), n, hidden, x.stride(0),
                                                dout.stride(0), _p(w_gate_up), _p(w_down_t), shared_width,
                                                num_experts, expert_width, _p(ids), _p(table), table.shape[1],
                                                table.shape[0], ctypes.cast(rw, ctypes.c_void_p),
                                                float(shared_scale), float(routed_scale), _p(gu),
                                                0 if gu is None else gu.stride(0), _p(dgu), 2 * F_, _p(hm), F_,
                                                _stream(x))
    N.check(st, "trmoe_dense_routed_swiglu_backward")
    return dgu, hm


def routed_swiglu_backward(x, dout, sorted_idx, offsets, num_experts, top_k, w_gate_up, w_down_t, expert_width,
                           route_weights, routed_scale):
    """(dgu[kN, 2Wp], hm[kN, Wp]) in partition order, Wp = round_up(W, 64)."""
    lib = _lib()
    _require_cuda(x, dout, sorted_idx, offsets, w_gate_up, w_down_t)
    n, hidden = x.shape
    wp = _round_up(expert_width, 64)
    rows = top_k * n
    dgu = torch.empty(rows, 2 * wp, dtype=x.dtype, device=x.device)
    hm = torch.empty(rows, wp, dtype=x.dtype, device=x.device)
    rw = _weights_arg(route_weights)
    st = lib.trmoe_routed_swiglu_backward(dtype_code(x.dtype), _p(x), _p(dout), n, hidden, x.stride(0),
                                          dout.stride(0), _p(sorted_idx), _p(offsets), num_experts, top_k,
                                          _p(w_gate_up), _p(w_down_t), expert_width,
                                          ctypes.cast(rw, ctypes.c_void_p), float(routed_scale), _p(dgu), 2 * wp,
                                          _p(hm), wp, _stream(x))
    N.check(st, "trmoe_routed_swiglu_backward")
    return dgu, hm


def weight_grad(a: torch.Tensor, b: torch.Tensor, m: int, n: int, n_rows: int, a_gather=None, b_gather=None,
                gather_mod: int = 0, offsets=None, segments: int = 1) -> torch.Tensor:
    """out[e][i, j] = sum over rows t of segment e of a[ra(t), i] * b[rb(t), j] -> [segments, m, n]."""
    lib = _lib()
    _require_cuda(a, b)
    code = dtype_code(a.dtype)
    out = torch.empty(segments, m, n, dtype=a.dtype, device=a.device)
    ws_bytes = lib.trmoe_weight_grad_workspace_bytes(code, m, n, segments, n_rows)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=a.device) if ws_bytes else None
    st = lib.trmoe_weight_grad(code, _p(a), a.stride(0), a.shape[0], _p(b), b.stride(0), b.shape[0], _p(a_gather),
                               _p(b_gather), gather_mod, m, n, n_rows, _p(offsets), segments, _p(out), n, m * n,
                               _p(ws), ws_bytes, _stream(a))
    N.check(st, "trmoe_weight_grad")
    return out


def weight_grad_mapped(a: torch.Tensor, b: torch.Tensor, m: int, n: int, n_rows: int, mode: int,
                       map_off: torch.Tensor, map_stride: torch.Tensor, out: torch.Tensor) -> None:
    """sum_t a[t, i] * b[t, j] over rows t < n_rows written into `out` (flat,
    bf16) at map_off[i] + j * map_stride[i] (mode 1) or map_off[j] + i *
    map_stride[j] (mode 2); negative offsets, and destinations outside
    `out`, are skipped."""
    lib = _lib()
    _require_cuda(a, b, map_off, map_stride, out)
    ws_bytes = lib.trmoe_weight_grad_mapped_workspace_bytes(dtype_code(a.dtype), m, n, n_rows)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=a.device)
    st = lib.trmoe_weight_grad_mapped(dtype_code(a.dtype), _p(a), a.stride(0), a.shape[0], _p(b), b.stride(0),
                                      b.shape[0], m, n, n_rows, mode, _p(map_off), _p(map_stride), _p(out), out.numel(),
                                      _p(ws), ws_bytes, _stream(a))
    N.check(st, "trmoe_weight_grad_mapped")


# Destination maps of the dense strategy's two weight gradients into one flat
# buffer holding the six parameter gradients contiguously: shared_gate,
# shared_up [S, H], shared_down [H, S], expert_gate, expert_up [E, H, W],
# expert_down [E, W, H].  Cached per shape and device.
_DENSE_GRAD_MAPS: dict = {}


def _dense_grad_maps(S: int, E: int, W: int, hidden: int, device):
    key = (S, E, W, hidden, str(device))
    hit = _DENSE_GRAD_MAPS.get(key)
    if hit is not None:
        return hit
    s_pad, w_pad = _round_up(S, 128), _round_up(W, 64)
    F_ = s_pad + E * w_pad
    sh, ew = S * hidden, E * W * hidden
    o_gate, o_up, o_sd = 0, sh, 2 * sh
    o_eg, o_eu, o_ed = 3 * sh, 3 * sh + ew, 3 * sh + 2 * ew
    # dWgu rows: packed gate|up row p of feature f = 32 (p // 64) + p % 32
    p = torch.arange(2 * F_, dtype=torch.int64)
    f = 32 * (p // 64) + p % 32
    up = (p // 32) % 2 == 1
    fe = f - s_pad
    e, j = fe.div(w_pad, rounding_mode="floor"), fe % w_pad
    shared, expert = f < S, (f >= s_pad) & (j < W)
    roff = torch.full_like(p, -1)
    rstride = torch.ones_like(p)
    roff[shared] = torch.where(up, o_up, o_gate)[shared] + f[shared] * hidden
    roff[expert] = torch.where(up, o_eu, o_eg)[expert] + e[expert] * hidden * W + j[expert]
    rstride[expert] = W
    # dWd columns: feature f of the down weight [H, F]
    c = torch.arange(F_, dtype=torch.int64)
    ce, cj = (c - s_pad).div(w_pad, rounding_mode="floor"), (c - s_pad) % w_pad
    cshared, cexpert = c < S, (c >= s_pad) & (cj < W)
    coff = torch.full_like(c, -1)
    cstride = torch.ones_like(c)
    coff[cshared] = o_sd + c[cshared]
    cstride[cshared] = S
    coff[cexpert] = o_ed + ce[cexpert] * W * hidden + cj[cexpert] * hidden
    maps = (roff.to(device), rstride.to(device), coff.to(device), cstride.to(device),
            (o_gate, o_up, o_sd, o_eg, o_eu, o_ed, 3 * sh + 3 * ew))
    _DENSE_GRAD_MAPS[key] = maps
    return maps


def grouped_linear(h: torch.Tensor, k: int, offsets: torch.Tensor, num_experts: int, w_packed: torch.Tensor,
                   out_features: int) -> torch.Tensor:
    """y[r] = h[r, :k] . W_e^T over a partition, W PLAIN-packed per expert."""
    lib = _lib()
    _require_cuda(h, offsets, w_packed)
    y = torch.empty(h.shape[0], out_features, dtype=h.dtype, device=h.device)
    st = lib.trmoe_grouped_linear(dtype_code(h.dtype), _p(h), h.stride(0), h.shape[0], k, _p(offsets), num_experts,
                                  _p(w_packed), out_features, _p(y), out_features, _stream(h))
    N.check(st, "trmoe_grouped_linear")
    return y


@dataclass
class BackwardPacks:
    """Transposed weight packs the backward reads (built from a PackedLayer)."""

    dense_down_t: Optional[torch.Tensor] = None
    dense_gate_up_t: Optional[torch.Tensor] = None
    shared_down_t: Optional[torch.Tensor] = None
    shared_gate_up_t: Optional[torch.Tensor] = None
    expert_down_t: Optional[torch.Tensor] = None
    expert_gate_up_t: Optional[torch.Tensor] = None


def backward_packs(packed: PackedLayer, hidden: int, shared_down=None, expert_down=None) -> BackwardPacks:
    """shared_down: shared_down.weight [H, S]; expert_down: the active [E, W, H] slice."""
    bp = BackwardPacks()
    if packed.strategy == STRATEGY_DENSE:
        bp.dense_down_t = pack_dense_down_t(packed.dense_down, packed.dense_features, hidden)
        bp.dense_gate_up_t = pack_gate_up_t(packed.dense_gate_up, hidden)
        return bp
    if packed.shared_width > 0:
        bp.shared_down_t = pack_linear_down_t(shared_down)
        bp.shared_gate_up_t = pack_gate_up_t(packed.shared_gate_up, hidden)
    bp.expert_down_t = pack_expert_down_t(expert_down)
    bp.expert_gate_up_t = pack_gate_up_t(packed.expert_gate_up, hidden)
    return bp


# Second stream of the backward: the weight-gradient GEMMs of the gate|up
# weights run beside the data gradient and the down weights' gradient (they
# only share read-only inputs), so the launches fill the CUs the others leave
# idle.  Default priority, one per device.
_SIDE: dict = {}


def _side_stream(device: torch.device):
    st = _SIDE.get(device.index)
    if st is None:
        st = torch.cuda.Stream(device=device)
        _SIDE[device.index] = st
    return st


class _OnSide:
    """Runs a block on the side stream after the current stream's work so far;
    inputs are marked as used there, outputs as used on the current stream."""

    def __init__(self, device, inputs):
        self.side = _side_stream(device)
        self.inputs = inputs
        self.outputs = []

    def __enter__(self):
        if self.side is None:
            return self
        self.cur = torch.cuda.current_stream(self.side.device)
        self.side.wait_stream(self.cur)
        for t in self.inputs:
            t.record_stream(self.side)
        self.ctx = torch.cuda.stream(self.side)
        self.ctx.__enter__()
        return self

    def __exit__(self, *exc):
        if self.side is not None:
            self.ctx.__exit__(*exc)

    def join(self):
        """Make the current stream wait for the side stream's block."""
        if self.side is None:
            return
        self.cur.wait_stream(self.side)
        for t in self.outputs:
            t.record_stream(self.cur)


def _gate_up_rows(g: torch.Tensor, features: int):
    """Packed gate|up rows [2F, H] -> (gate rows [F, H], up rows [F, H]) views."""
    v = g.view(features // 32, 2, 32, g.shape[-1])
    return v[:, 0].reshape(features, -1), v[:, 1].reshape(features, -1)


@_on_tensor_device
def layer_backward(dout: torch.Tensor, x: torch.Tensor, token_ids: torch.Tensor, route_table: torch.Tensor,
                   packed: PackedLayer, bwd: BackwardPacks, route_weights: Sequence[float], shared_scale: float,
                   routed_scale: float, order: int = ORDER_TOKEN, need_dx: bool = True, need_dw: bool = True,
                   saved_gu: Optional[torch.Tensor] = None, saved_h: Optional[torch.Tensor] = None):
    """Gradients of layer_forward: (dx[N, H] or None, grads) with grads a dict of
    shared_gate/shared_up [S, H], shared_down [H, S], expert_gate/expert_up
    [E, H, W], expert_down [E, W, H] (active sizes; None when not needed).
    saved_gu / saved_h: what layer_forward(save=True) returned (the dense
    strategy's down weight gradient then reads the forward's h)."""
    n, hidden = x.shape
    top_k = route_table.shape[0]
    E, W, S = packed.num_experts, packed.expert_width, packed.shared_width
    grads = dict.fromkeys(("shared_gate", "shared_up", "shared_down", "expert_gate", "expert_up", "expert_down"))
    if n == 0:
        return (torch.zeros_like(x) if need_dx else None), grads
    x = rows16(x)
    dout = rows16(dout.contiguous())
    s_pad, w_pad = _round_up(S, 128), _round_up(W, 64)
    if packed.strategy == STRATEGY_DENSE:
        F_ = packed.dense_features
        # bf16: both weight gradients go straight into one flat buffer in the
        # parameters' layouts (their views are the gradients, no copies)
        mapped = need_dw and x.dtype == torch.bfloat16
        if mapped:
            roff, rstride, coff, cstride, offs = _dense_grad_maps(S, E, W, hidden, x.device)
            flat = torch.empty(offs[-1], dtype=x.dtype, device=x.device)
        dgu, hm = dense_routed_swiglu_backward(x, dout, packed.dense_gate_up, bwd.dense_down_t, S, E, W, token_ids,
                                               route_table, route_weights, shared_scale, routed_scale, gu=saved_gu,
                                               want_hm=need_dw and saved_h is None)
        if saved_h is not None:
            hm = saved_h
        # the gate|up weight gradient (side stream) overlaps dx and dWd
        side = _OnSide(x.device, (dgu, x))
        if need_dw:
            with side:
                if mapped:
                    weight_grad_mapped(dgu, x, 2 * F_, hidden, n, 1, roff, rstride, flat)
                    side.outputs.append(flat)
                else:
                    dwgu = weight_grad(dgu, x, 2 * F_, hidden, n)[0]     # [2F, H]
                    side.outputs.append(dwgu)
        dx = None
        if need_dx:
            dx = shared_down_combine(dgu, 2 * F_, bwd.dense_gate_up_t, None, hidden, None, None, top_k,
                                     (1.0,) * top_k, 1.0, 1.0)
        if mapped:
            weight_grad_mapped(dout, hm, hidden, F_, n, 2, coff, cstride, flat)
            side.join()
            o_gate, o_up, o_sd, o_eg, o_eu, o_ed, _ = offs
            sh, ew = S * hidden, E * W * hidden
            if S:
                grads["shared_gate"] = flat[o_gate:o_gate + sh].view(S, hidden)
                grads["shared_up"] = flat[o_up:o_up + sh].view(S, hidden)
                grads["shared_down"] = flat[o_sd:o_sd + sh].view(hidden, S)
            grads["expert_gate"] = flat[o_eg:o_eg + ew].view(E, hidden, W)
            grads["expert_up"] = flat[o_eu:o_eu + ew].view(E, hidden, W)
            grads["expert_down"] = flat[o_ed:o_ed + ew].view(E, W, hidden)
            return dx, grads
        if need_dw:
            dwd = weight_grad(dout, hm, hidden, F_, n)[0]            # [H, F]
            side.join()
            g_rows, u_rows = _gate_up_rows(dwgu, F_)
            if S:
                grads["shared_gate"], grads["shared_up"] = g_rows[:S], u_rows[:S]
                grads["shared_down"] = dwd[:, :S]
            eg = g_rows[s_pad:].view(E, w_pad, hidden)[:, :W]
            eu = u_rows[s_pad:].view(E, w_pad, hidden)[:, :W]
            grads["expert_gate"] = eg.transpose(1, 2)
            grads["expert_up"] = eu.transpose(1, 2)
            grads["expert_down"] = dwd[:, s_pad:].reshape(hidden, E, w_pad)[:, :, :W].permute(1, 2, 0)
        return dx, grads

    sorted_idx, inverse, offsets, _ = route_sort(token_ids, route_table, E, order)
    dgu_r, hm_r = routed_swiglu_backward(x, dout, sorted_idx, offsets, E, top_k, packed.expert_gate_up,
                                         bwd.expert_down_t, W, route_weights, routed_scale)
    dgu_s = hm_s = None
    if S > 0:
        dgu_s, hm_s = shared_swiglu_backward(x, dout, packed.shared_gate_up, bwd.shared_down_t, S, shared_scale,
                                             gu=saved_gu)
    rows = top_k * n
    # the gate|up weight gradients (side stream) overlap dx and the down ones
    side = _OnSide(x.device, tuple(t for t in (dgu_s, x, dgu_r, sorted_idx, offsets) if t is not None))
    if need_dw:
        with side:
            if S > 0:
                dwgu_s = weight_grad(dgu_s, x, 2 * s_pad, hidden, n)[0]          # [2S_pad, H]
                side.outputs.append(dwgu_s)
            dwgu_e = weight_grad(x, dgu_r, hidden, 2 * w_pad, rows, a_gather=sorted_idx, gather_mod=n,
                                 offsets=offsets, segments=E)                     # [E, H, 2W_pad]
            side.outputs.append(dwgu_e)
    dx = None
    if need_dx:
        dxa = grouped_linear(dgu_r, 2 * w_pad, offsets, E, bwd.expert_gate_up_t, hidden)
        ones = (1.0,) * top_k
        if S > 0:
            dx = shared_down_combine(dgu_s, 2 * s_pad, bwd.shared_gate_up_t, None, hidden, dxa, inverse, top_k, ones,
                                     1.0, 1.0)
        else:
            dx = combine(dxa, inverse, n, top_k, ones, 1.0)
    if need_dw:
        if S > 0:
            dwd_s = weight_grad(dout, hm_s, hidden, s_pad, n)[0]                 # [H, S_pad]
        dwd_e = weight_grad(hm_r, dout, w_pad, hidden, rows, b_gather=sorted_idx, gather_mod=n, offsets=offsets,
                            segments=E)                                           # [E, W_pad, H]
        side.join()
        if S > 0:
            g_rows, u_rows = _gate_up_rows(dwgu_s, s_pad)
            grads["shared_gate"], grads["shared_up"] = g_rows[:S], u_rows[:S]
            grads["shared_down"] = dwd_s[:, :S]
        v = dwgu_e.view(E, hidden, w_pad // 32, 2, 32)
        grads["expert_gate"] = v[:, :, :, 0].reshape(E, hidden, w_pad)[:, :, :W]
        grads["expert_up"] = v[:, :, :, 1].reshape(E, hidden, w_pad)[:, :, :W]
        grads["expert_down"] = dwd_e[:, :W]
    return dx, grads
