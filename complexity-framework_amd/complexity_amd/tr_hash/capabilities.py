"""Backend resolution with explicit reasons (behaviour of complexity/tr_hash/capabilities.py).

The reference resolves AUTO/PYTORCH/CGGR/FUSED_CUDA/CUDA_GRAPH
(capabilities.py:68-175).  This build has no Triton kernels; its native
backend is HIP (gfx950).  On a ROCm device, AUTO, CGGR and FUSED_CUDA requests
are served by the HIP kernels: CGGR requests keep the reference CGGR
partition order (expert, assignment), fused requests the fused order
(expert, token).  Nothing is chosen silently: every fallback carries a reason
in ``BackendDecision.reasons`` and a missing HIP library on a GPU raises.
"""

from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from .config import TRHashBackend, TRHashEngineConfig, TRHashPhase, TRHashPrecision

PARTITION_TOKEN = "token"
PARTITION_ASSIGNMENT = "assignment"


@dataclass(frozen=True)
class BackendDecision:
    requested: TRHashBackend
    selected: TRHashBackend
    reasons: Tuple[str, ...]
    graph_safe: bool
    quantized: bool
    partition: str = PARTITION_TOKEN


def _hip_available() -> bool:
    from .. import _native

    return _native.available()


def _hip_load_error() -> str:
    from .. import _native

    return _native.load_error() or "unknown"


def _custom_cggr_available() -> bool:
    """This build ships no Triton CGGR kernels (the HIP backend replaces them)."""
    return False


def _fused_cuda_available() -> bool:
    """This build ships no Triton fused kernels (the HIP backend replaces them)."""
    return False


def supports_fused_cuda(config: TRHashEngineConfig) -> bool:
    """Shapes the reference's hash-native fused path covers (capabilities.py:62-65)."""
    return config.top_k == 2 and 2 <= config.num_experts <= 8


def supports_hip(config: TRHashEngineConfig) -> bool:
    """Shapes the HIP kernels cover: every supported expert count and top-k."""
    return config.num_experts <= 16 and config.top_k in (1, 2, 4)


_NO_HIP_BACKWARD = "HIP backward needs bf16/f32 weights (not e4m3 copies) and hidden_size % 8 == 0"


def supports_hip_backward(config: TRHashEngineConfig, quantized_weights: bool = False) -> bool:
    """Differentiable HIP calls: bf16/f32 weights (e4m3 copies are
    inference-only, whether the config asks for fp8 or the engine was
    quantised with ``quantize_fp8_()``) and a hidden size that is a multiple
    of 8 (the weight-gradient GEMMs read 16-byte column chunks)."""
    return (config.precision is not TRHashPrecision.FP8 and not quantized_weights
            and config.hidden_size % 8 == 0)


def _allow_fallback() -> bool:
    return os.environ.get("TRMOE_ALLOW_PYTORCH_FALLBACK", "0") not in ("", "0", "false", "False")


def _decision(requested, selected, reasons=(), *, graph_safe=False, quantized=False, partition=PARTITION_TOKEN):
    return BackendDecision(
        requested=requested,
        selected=selected,
        reasons=tuple(reasons),
        graph_safe=graph_safe,
        quantized=quantized,
        partition=partition,
    )


def select_backend(
    config: TRHashEngineConfig,
    *,
    device_type: str,
    cggr_available: Optional[bool] = None,
    fused_cuda_available: Optional[bool] = None,
    hip_available: Optional[bool] = None,
    autograd: bool = False,
    quantized_weights: bool = False,
) -> BackendDecision:
    """Resolve the backend for one forward.

    ``autograd`` is True when the forward must be differentiable.  The HIP
    backend has a backward for bf16/f32 weights (``supports_hip_backward``);
    other differentiable calls resolve to PYTORCH with a reason (or raise when
    HIP was requested explicitly).  ``quantized_weights`` is True when the
    engine computes from e4m3 copies whatever its config precision says.
    """

    if cggr_available is None:
        cggr_available = _custom_cggr_available()
    if fused_cuda_available is None:
        fused_cuda_available = _fused_cuda_available()
    if hip_available is None:
        hip_available = _hip_available() if device_type == "cuda" else False

    if config.precision is TRHashPrecision.INT8:
        raise NotImplementedError(
            "int8 is reserved by the TR-Hash API but requires the phase-2 quantized grouped-GEMM kernel"
        )
    quantized = config.precision is TRHashPrecision.FP8
    requested = config.backend
    partition = PARTITION_ASSIGNMENT if (requested is TRHashBackend.CGGR or not supports_fused_cuda(config)) else PARTITION_TOKEN

    if requested is TRHashBackend.PYTORCH:
        return _decision(requested, TRHashBackend.PYTORCH, quantized=quantized)

    if requested is TRHashBackend.CUDA_GRAPH:
        if device_type != "cuda":
            raise RuntimeError("CUDA Graph backend requires a CUDA device")
        if config.phase is not TRHashPhase.INFERENCE:
            raise RuntimeError("CUDA Graph backend is inference-only")
        return _decision(requested, TRHashBackend.CUDA_GRAPH, graph_safe=True, quantized=quantized, partition=partition)

    if requested is TRHashBackend.HIP:
        if device_type != "cuda":
            raise RuntimeError("HIP backend requires a ROCm (cuda) device")
        if not hip_available:
            raise RuntimeError(f"HIP backend requested but the TR-MoE library is unavailable: {_hip_load_error()}")
        if not supports_hip(config):
            raise RuntimeError("HIP backend supports top_k in {1, 2, 4} and at most 16 experts")
        if autograd and not supports_hip_backward(config, quantized_weights):
            raise RuntimeError(
                "HIP backward needs bf16/f32 weights (not e4m3 copies) and hidden_size % 8 == 0; run under "
                "torch.no_grad() or select pytorch"
            )
        return _decision(requested, TRHashBackend.HIP, quantized=quantized, partition=partition)

    if requested is TRHashBackend.FUSED_CUDA:
        if device_type != "cuda":
            raise RuntimeError("fused CUDA backend requires a CUDA device")
        if not supports_fused_cuda(config):
            raise RuntimeError("fused CUDA backend requires top_k=2 and two to eight experts")
        if fused_cuda_available and not hip_available:
            return _decision(requested, TRHashBackend.FUSED_CUDA, quantized=quantized)
        if not hip_available:
            raise RuntimeError(
                "fused CUDA backend requested but neither Triton kernels nor the HIP library are available: "
                + _hip_load_error()
            )
        if autograd and not supports_hip_backward(config, quantized_weights):
            return _decision(requested, TRHashBackend.PYTORCH, [_NO_HIP_BACKWARD], quantized=quantized)
        return _decision(requested, TRHashBackend.HIP, ["fused_cuda served by HIP kernels"], quantized=quantized)

    if requested is TRHashBackend.CGGR:
        if device_type != "cuda":
            raise RuntimeError("CGGR backend requires a CUDA device")
        if cggr_available and not hip_available:
            return _decision(requested, TRHashBackend.CGGR, quantized=quantized, partition=PARTITION_ASSIGNMENT)
        if not hip_available:
            raise RuntimeError("CGGR backend requested but Triton CGGR and the HIP library are unavailable")
        if autograd and not supports_hip_backward(config, quantized_weights):
            return _decision(requested, TRHashBackend.PYTORCH, [_NO_HIP_BACKWARD], quantized=quantized)
        return _decision(requested, TRHashBackend.HIP, ["cggr served by HIP kernels"], quantized=quantized,
                         partition=PARTITION_ASSIGNMENT)

    # AUTO
    reasons = []
    if device_type != "cuda":
        reasons.append("CGGR requires CUDA")
        return _decision(requested, TRHashBackend.PYTORCH, reasons, quantized=quantized)
    if hip_available and supports_hip(config):
        if autograd and not supports_hip_backward(config, quantized_weights):
            return _decision(requested, TRHashBackend.PYTORCH, [_NO_HIP_BACKWARD], quantized=quantized)
        return _decision(requested, TRHashBackend.HIP, quantized=quantized, partition=partition)
    if fused_cuda_available and supports_fused_cuda(config):
        return _decision(requested, TRHashBackend.FUSED_CUDA, quantized=quantized)
    if cggr_available:
        return _decision(requested, TRHashBackend.CGGR, quantized=quantized, partition=PARTITION_ASSIGNMENT)
    if not hip_available:
        if not _allow_fallback():
            raise RuntimeError(
                "TR-MoE HIP library unavailable on a GPU device ("
                + _hip_load_error()
                + "); build it with `python -m complexity_amd.build_native`, request backend='pytorch', "
                "or set TRMOE_ALLOW_PYTORCH_FALLBACK=1"
            )
        reasons.append("HIP library unavailable: " + _hip_load_error())
    else:
        reasons.append("shape not supported by the HIP kernels")
    return _decision(requested, TRHashBackend.PYTORCH, reasons, quantized=quantized)


def precision_to_torch_dtype(precision: TRHashPrecision) -> torch.dtype:
    mapping = {
        TRHashPrecision.FP32: torch.float32,
        TRHashPrecision.BF16: torch.bfloat16,
        TRHashPrecision.FP16: torch.float16,
        TRHashPrecision.FP8: torch.bfloat16,  # fp8 weights, bf16 activations
    }
    try:
        return mapping[precision]
    except KeyError as exc:
        raise NotImplementedError(f"{precision.value} needs the quantized TR-Hash backend") from exc
