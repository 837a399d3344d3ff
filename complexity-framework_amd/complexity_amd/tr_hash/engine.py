"""TR-Hash SwiGLU engine with a native HIP backend (mirror of complexity/tr_hash/engine.py).

Module surface kept identical to the reference (engine.py:107-716): the
``route_table`` / ``fused_route_codes`` / ``fused_expert_pairs`` buffers,
``expert_{gate,up,down}`` parameters, ``shared_{gate,up,down}`` linears,
``set_active_capacity``, ``load_route_table``, ``capability_summary`` (same
21 keys), ``last_backend`` and the graph-bucket path, so state dicts and call
sites move over unchanged.

Backends:

* ``PYTORCH`` -- the universal definition (engine.py:66-104, 333-349, 578),
  used for CPU tensors (and for differentiable fp8 calls);
* ``HIP`` -- the gfx950 kernels of ``libtrmoe`` (route partition, shared
  SwiGLU GEMM, grouped routed experts, down GEMM with the un-permute and
  combine in its epilogue); differentiable for bf16/f32 weights through one
  autograd Function whose backward also runs HIP kernels (``hip_autograd``);
* ``CUDA_GRAPH`` -- HIP (or PYTORCH) captured per static bucket.

``precision=fp8`` keeps e4m3 copies of every weight with per-output-channel
scales (``*_fp8`` / ``*_scale`` buffers, saved in the state dict); both
backends then compute with the dequantised values q * scale.
"""

from __future__ import annotations

import logging
import os
from dataclasses import replace
from typing import Callable, Dict, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops
from .buckets import GraphBucketPlanner
from .hip_autograd import RMSNormResidualFunction, _LayerPlan, hip_layer_autograd
from .capabilities import (
    PARTITION_ASSIGNMENT,
    BackendDecision,
    select_backend,
    supports_fused_cuda,
)
from .config import SUPPORTED_EXPERT_COUNTS, GraphBucket, TRHashBackend, TRHashEngineConfig, TRHashPhase, TRHashPrecision
from .routing import build_route_table, compile_top2_pair_metadata
from . import weights

logger = logging.getLogger(__name__)

E4M3_MAX = 448.0
_FP8_WEIGHTS = ("expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up", "shared_down")


def _silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return F.silu(gate) * up


def reference_topk_swiglu(
    flat_x: torch.Tensor,
    routes: torch.Tensor,
    gate_weights: torch.Tensor,
    up_weights: torch.Tensor,
    down_weights: torch.Tensor,
    route_weights: torch.Tensor,
    *,
    activation: Callable[[torch.Tensor, torch.Tensor], torch.Tensor] = _silu_mul,
    intermediate_transform: Optional[Callable[[torch.Tensor, int], torch.Tensor]] = None,
) -> torch.Tensor:
    """Universal routed formula: masked dense loop over experts (engine.py:66-104).

    For each expert e the tokens routed to it (token weight tw = sum of the
    route weights of the slots that selected e) run the expert SwiGLU; the
    result scaled by tw is accumulated in expert order in ``flat_x.dtype``.
    """
    if flat_x.ndim != 2:
        raise ValueError("flat_x must be [tokens, hidden]")
    if routes.ndim != 2 or routes.size(1) != flat_x.size(0):
        raise ValueError("routes must be [top_k, tokens]")
    if route_weights.shape != routes.shape:
        raise ValueError("route_weights must match routes")
    if gate_weights.shape != up_weights.shape:
        raise ValueError("gate and up expert weights must have the same shape")
    if gate_weights.ndim != 3 or down_weights.ndim != 3:
        raise ValueError("expert weights must be rank-3 tensors")
    if gate_weights.size(0) != down_weights.size(0):
        raise ValueError("expert weight tensors must have the same expert count")
    total = torch.zeros_like(flat_x)
    for e in range(gate_weights.size(0)):
        tw = (routes.eq(e).to(flat_x.dtype) * route_weights).sum(dim=0)
        xe = flat_x * tw.ne(0).to(flat_x.dtype).unsqueeze(-1)
        inner = activation(xe @ gate_weights[e], xe @ up_weights[e])
        if intermediate_transform is not None:
            inner = intermediate_transform(inner, e)
        total = total + (inner @ down_weights[e]).to(total.dtype) * tw.unsqueeze(-1)
    return total


def _quantize_e4m3(weight: torch.Tensor):
    """Per-output-channel e4m3: scale = amax/448 over dim 1 (the reduction axis).

    Computed on the host so the stored codes do not depend on the device's
    division and conversion rounding (checkpoints are reproducible).
    """
    w = weight.detach().float().cpu()
    amax = w.abs().amax(dim=1, keepdim=True)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (w / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, scale.squeeze(1).contiguous()


class TRHashEngine(nn.Module):
    """Shared SwiGLU plus deterministic top-k token-ID experts."""

    def __init__(self, config: TRHashEngineConfig):
        super().__init__()
        self.config = config
        self.register_buffer("route_table", build_route_table(config))
        self.register_buffer(
            "_route_weights", torch.tensor(config.route_weights, dtype=torch.float32), persistent=False
        )
        codes, pairs = self._compile_fused_metadata(self.route_table)
        self.register_buffer("fused_route_codes", codes)
        self.register_buffer("fused_expert_pairs", pairs)

        E, H, W = config.num_experts, config.hidden_size, config.expert_width
        self.expert_gate = nn.Parameter(torch.empty(E, H, W))
        self.expert_up = nn.Parameter(torch.empty(E, H, W))
        self.expert_down = nn.Parameter(torch.empty(E, W, H))
        if config.shared_width:
            self.shared_gate = nn.Linear(H, config.shared_width, bias=False)
            self.shared_up = nn.Linear(H, config.shared_width, bias=False)
            self.shared_down = nn.Linear(config.shared_width, H, bias=False)
        else:
            self.shared_gate = None
            self.shared_up = None
            self.shared_down = None
        self.reset_parameters()

        self.last_backend: Optional[BackendDecision] = None
        self.last_norm: Optional[str] = None
        # W8A8: with e4m3 weights (quantize_fp8_), also quantize activations
        # to e4m3 so the shared GEMMs run on the e4m3 MFMA (prefill sizes,
        # grouped strategy).  True: each token's x (per-token scale) into the
        # shared gate|up, and its h as e4m3 with a power-of-two scale per 32
        # features into the shared down (shared width a multiple of 128, else
        # the down keeps bf16 h); "gate_up": the gate|up only.  Off by
        # default: the reference has no fp8 path and keeps activations in the
        # compute dtype.
        self.fp8_activations = False
        self._graph_pool: Dict[GraphBucket, "_CapturedTRHashGraph"] = {}
        self._bucket_planner = GraphBucketPlanner(config.graph_buckets) if config.graph_buckets else None
        self._active_num_experts = config.num_experts
        self._active_expert_width = config.expert_width
        self._active_route_table = self.route_table
        self._fused_shared_gate_up_weight: Optional[torch.Tensor] = None
        self._packed_key = None
        self._packed_norm = None   # (key, pack) with a block RMSNorm weight folded in
        self._bwd_packed = None
        self._decision_cache: Dict[tuple, BackendDecision] = {}
        self._packed: Optional[ops.PackedLayer] = None
        self._fp8 = False
        # HIP routed-expert strategy: "grouped" (route partition + grouped
        # expert GEMMs + un-permute in the down epilogue), "dense" (every
        # expert folded into the shared GEMMs, masked by route weights) or
        # "auto" (dense when it adds at most 8% MFMA work).
        self.routed_strategy = "auto"
        if config.precision is TRHashPrecision.FP8:
            self.quantize_fp8_()

    # ------------------------------------------------------------------ plumbing
    def _apply(self, fn, recurse: bool = True):
        # _active_route_table is a plain attribute (an alias of route_table or
        # a rebuilt reduced table), so move it with the module explicitly.
        aliased = self._active_route_table is self.route_table
        super()._apply(fn, recurse=recurse)
        self._active_route_table = self.route_table if aliased else fn(self._active_route_table)
        if self._fused_shared_gate_up_weight is not None:
            self._fused_shared_gate_up_weight = fn(self._fused_shared_gate_up_weight)
        self._packed_key = None
        self._packed = None
        self._packed_norm = None
        # captured graphs hold the old tensors' addresses
        self._graph_pool.clear()
        return self

    @property
    def active_num_experts(self) -> int:
        return self._active_num_experts

    @property
    def active_expert_width(self) -> int:
        return self._active_expert_width

    def set_active_capacity(self, *, num_experts: Optional[int] = None, expert_width: Optional[int] = None) -> None:
        """Use a prefix sub-network (engine.py:214-261); routing is rebuilt for it."""
        if num_experts is not None:
            if num_experts not in SUPPORTED_EXPERT_COUNTS:
                raise ValueError(f"num_experts must be one of {SUPPORTED_EXPERT_COUNTS}, got {num_experts}")
            if num_experts > self.config.num_experts:
                raise ValueError(
                    f"active num_experts ({num_experts}) cannot exceed the allocated capacity "
                    f"({self.config.num_experts})"
                )
            if num_experts == self.config.num_experts:
                self._active_route_table = self.route_table
            else:
                reduced = replace(self.config, num_experts=num_experts)
                self._active_route_table = build_route_table(reduced).to(device=self.route_table.device)
            self._active_num_experts = num_experts
        if expert_width is not None:
            if not 0 < expert_width <= self.config.expert_width:
                raise ValueError(
                    f"active expert_width must be in (0, {self.config.expert_width}], got {expert_width}"
                )
            self._active_expert_width = expert_width
        if num_experts is not None or expert_width is not None:
            self._graph_pool.clear()
            self._packed_key = None
            self._packed = None
            self._packed_norm = None

    def _compile_fused_metadata(self, route_table: torch.Tensor):
        if supports_fused_cuda(self.config):
            return compile_top2_pair_metadata(route_table, num_experts=self.config.num_experts)
        return torch.empty(0, dtype=torch.uint8), torch.empty((0, 2), dtype=torch.int32)

    def load_route_table(self, route_table: torch.Tensor) -> None:
        """Install an external [top_k, vocab] table (engine.py:276-306)."""
        if tuple(route_table.shape) != tuple(self.route_table.shape):
            raise ValueError(
                f"route_table shape {tuple(route_table.shape)} does not match "
                f"the engine's {tuple(self.route_table.shape)} ([top_k, vocab_size])"
            )
        if int(route_table.min()) < 0 or int(route_table.max()) >= self.config.num_experts:
            raise ValueError("route_table contains an out-of-range expert index")
        self.route_table.copy_(route_table.to(device=self.route_table.device))
        codes, pairs = self._compile_fused_metadata(self.route_table)
        self.fused_route_codes = codes.to(device=self.fused_route_codes.device)
        self.fused_expert_pairs = pairs.to(device=self.fused_expert_pairs.device)
        if self._active_num_experts == self.config.num_experts:
            self._active_route_table = self.route_table
        else:
            reduced = replace(self.config, num_experts=self._active_num_experts)
            self._active_route_table = build_route_table(reduced).to(device=self.route_table.device)
        self._graph_pool.clear()

    def reset_parameters(self) -> None:
        std = self.config.initializer_range
        for p in (self.expert_gate, self.expert_up, self.expert_down):
            nn.init.normal_(p, mean=0.0, std=std)
        for m in (self.shared_gate, self.shared_up, self.shared_down):
            if m is not None:
                nn.init.normal_(m.weight, mean=0.0, std=std)

    # ------------------------------------------------------------------ fp8
    def quantize_fp8_(self) -> None:
        """(Re)build the e4m3 weight copies and per-output-channel scales from
        the current parameters; forwards then use q * scale."""
        masters = weights.materialize(self)
        for name in _FP8_WEIGHTS:
            w = masters[name]
            if w is None:
                continue
            q, s = _quantize_e4m3(w)
            for suffix, t in (("_fp8", q), ("_scale", s)):
                key = name + suffix
                if key in self._buffers:
                    self._buffers[key] = t.to(device=w.device)
                else:
                    self.register_buffer(key, t.to(device=w.device))
        self._fp8 = True
        self._packed_key = None
        self._packed = None
        self._packed_norm = None
        self._decision_cache.clear()
        self._graph_pool.clear()

    def _dequantized(self, name: str, dtype: torch.dtype) -> torch.Tensor:
        q = getattr(self, name + "_fp8")
        s = getattr(self, name + "_scale")
        return (q.float() * s.unsqueeze(1)).to(dtype)

    # ------------------------------------------------------------------ pytorch backend
    def _routes(self, token_ids: torch.Tensor) -> torch.Tensor:
        clamped = token_ids.clamp(0, self.config.vocab_size - 1)
        return self._active_route_table[:, clamped]

    def _expert_tensors(self, dtype: Optional[torch.dtype] = None):
        if self._fp8:
            dt = dtype or torch.bfloat16
            return tuple(self._dequantized(n, dt) for n in ("expert_gate", "expert_up", "expert_down"))
        return self.expert_gate, self.expert_up, self.expert_down

    def _active_expert_weights(self, dtype: Optional[torch.dtype] = None):
        """(gate, up, down) truncated to the active capacity (engine.py:320-331)."""
        gate, up, down = self._expert_tensors(dtype)
        E, W = self._active_num_experts, self._active_expert_width
        if E == self.config.num_experts and W == self.config.expert_width:
            return gate, up, down
        return (
            gate[:E, :, :W].contiguous(),
            up[:E, :, :W].contiguous(),
            down[:E, :W, :].contiguous(),
        )

    def _shared(self, flat_x: torch.Tensor) -> torch.Tensor:
        if self.shared_gate is None:
            return torch.zeros_like(flat_x)
        if self._fp8:
            dt = flat_x.dtype
            g = F.linear(flat_x, self._dequantized("shared_gate", dt))
            u = F.linear(flat_x, self._dequantized("shared_up", dt))
            return F.linear(_silu_mul(g, u), self._dequantized("shared_down", dt))
        fused = self._fused_shared_gate_up_weight
        gate_lora = getattr(self.shared_gate, "is_lora_adapter", False)
        up_lora = getattr(self.shared_up, "is_lora_adapter", False)
        if fused is not None and gate_lora and up_lora:
            width = int(self.shared_gate.base.out_features)
            base_g, base_u = F.linear(flat_x, fused).split([width, width], dim=-1)
            gate = base_g + self.shared_gate.lora_residual(flat_x)
            up = base_u + self.shared_up.lora_residual(flat_x)
        else:
            gate = self.shared_gate(flat_x)
            up = self.shared_up(flat_x)
        return self.shared_down(_silu_mul(gate, up))

    def refresh_fused_shared_lora_weight(self) -> bool:
        gate_lora = getattr(self.shared_gate, "is_lora_adapter", False)
        up_lora = getattr(self.shared_up, "is_lora_adapter", False)
        if not (gate_lora and up_lora):
            self._fused_shared_gate_up_weight = None
            return False
        self._fused_shared_gate_up_weight = torch.cat(
            [self.shared_gate.base.weight, self.shared_up.base.weight], dim=0
        ).detach()
        return True

    def _reference_routed(self, flat_x: torch.Tensor, routes: torch.Tensor) -> torch.Tensor:
        rw = self._route_weights.to(dtype=flat_x.dtype)[:, None].expand_as(routes)
        gate, up, down = self._active_expert_weights(flat_x.dtype)
        return reference_topk_swiglu(flat_x, routes, gate, up, down, rw)

    # ------------------------------------------------------------------ hip backend
    def _hip_act_dtype(self) -> torch.dtype:
        if self._fp8:
            return torch.bfloat16
        dt = weights.stored_dtype(self, "expert_gate")
        if dt not in (torch.float32, torch.bfloat16):
            raise NotImplementedError(f"HIP kernels support float32/bfloat16/fp8 weights, got {dt}")
        return dt

    def _hip_packed(self, norm_weight: Optional[torch.Tensor] = None,
                    current: Optional[dict] = None) -> ops.PackedLayer:
        """Weights in kernel layout, rebuilt when what a weight would
        materialise to or the active capacity changes.

        The key never materialises a weight: ordinary tensors are keyed on
        storage pointer and in-place version, a parametrized weight (the
        reference's expert LoRA, lora.py:93-215) on every tensor of its
        parametrization, a shared LoRA adapter on its base and factors.  A
        parametrization in training mode is not cached.  current: the weights
        this call already materialised (weights.materialize), used when the
        pack has to be rebuilt; otherwise they are materialised here, once.

        norm_weight: a block's RMSNorm weight folded into the gate/up weights
        (their input axis), for forward_norm_residual; cached apart from the
        plain pack."""
        E, W = self._active_num_experts, self._active_expert_width
        strategy = self.routed_strategy
        if strategy == "auto":
            strategy = ops.choose_strategy(self.config.shared_width, E, W, self.config.top_k, self._fp8)
        if strategy == ops.STRATEGY_DENSE and self._fp8:
            raise NotImplementedError("the dense-routed strategy needs bf16/f32 weights")
        if norm_weight is not None and self._fp8:
            raise NotImplementedError("the fused RMSNorm folds its weight into bf16/f32 gate/up weights")
        if self._fp8:
            names = [n for n in _FP8_WEIGHTS if hasattr(self, n + "_fp8")]
            wkey = tuple(weights._tkey(getattr(self, n + sfx)) for n in names for sfx in ("_fp8", "_scale"))
        else:
            wkey = weights.weights_key(self)
        key = None
        if wkey is not None:
            key = (
                wkey,
                E,
                W,
                strategy,
                None if norm_weight is None else (norm_weight.data_ptr(), norm_weight._version, norm_weight.dtype),
            )
        if norm_weight is not None:
            cached = self._packed_norm
            if key is not None and cached is not None and cached[0] == key:
                return cached[1]
        elif key is not None and self._packed is not None and self._packed_key == key:
            return self._packed
        if current is None and not self._fp8:
            current = weights.materialize(self)
        packed = self._build_packed(E, W, strategy, norm_weight, current)
        if norm_weight is not None:
            self._packed_norm = (key, packed)
        else:
            self._packed, self._packed_key = packed, key
        return packed

    def _build_packed(self, E: int, W: int, strategy: str, norm_weight: Optional[torch.Tensor],
                      cw: Optional[dict]) -> ops.PackedLayer:
        """cw: name -> weight as materialised for this call (None for e4m3 packs)."""

        def fold(w: torch.Tensor, shape) -> torch.Tensor:
            # W * norm_weight along the input axis, rounded once to w's dtype
            if norm_weight is None:
                return w
            return (w.float() * norm_weight.float().reshape(shape)).to(w.dtype)

        with torch.no_grad():
            if strategy == ops.STRATEGY_DENSE:
                shared = (None, None, None)
                if self.shared_gate is not None:
                    shared = (cw["shared_gate"], cw["shared_up"], cw["shared_down"])
                if shared[0] is not None:
                    shared = (fold(shared[0], (1, -1)), fold(shared[1], (1, -1)), shared[2])
                gu, dd, feats = ops.pack_dense_routed(
                    *shared, fold(cw["expert_gate"][:E, :, :W], (1, -1, 1)), fold(cw["expert_up"][:E, :, :W], (1, -1, 1)),
                    cw["expert_down"][:E, :W, :]
                )
                packed = ops.PackedLayer(
                    act_dtype=self._hip_act_dtype(),
                    num_experts=E,
                    expert_width=W,
                    strategy=strategy,
                    shared_width=self.config.shared_width,
                    dense_gate_up=gu,
                    dense_down=dd,
                    dense_features=feats,
                )
                return packed
            if self._fp8:
                gq, gs = self.expert_gate_fp8[:E, :, :W], self.expert_gate_scale[:E, :W]
                uq, us = self.expert_up_fp8[:E, :, :W], self.expert_up_scale[:E, :W]
                dq, ds = self.expert_down_fp8[:E, :W, :], self.expert_down_scale[:E]
                egu, egu_s = ops.pack_expert_gate_up(gq, uq, gs, us)
                ed, ed_s = ops.pack_expert_down(dq, ds)
            else:
                egu, egu_s = ops.pack_expert_gate_up(fold(cw["expert_gate"][:E, :, :W], (1, -1, 1)),
                                                     fold(cw["expert_up"][:E, :, :W], (1, -1, 1)))
                ed, ed_s = ops.pack_expert_down(cw["expert_down"][:E, :W, :])
            packed = ops.PackedLayer(
                act_dtype=self._hip_act_dtype(),
                num_experts=E,
                expert_width=W,
                strategy=ops.STRATEGY_GROUPED,
                expert_gate_up=egu,
                expert_gate_up_scale=egu_s,
                expert_down=ed,
                expert_down_scale=ed_s,
            )
            if self.shared_gate is not None:
                packed.shared_width = self.config.shared_width
                if self._fp8:
                    sgu, sgu_s = ops.pack_linear_gate_up(
                        self.shared_gate_fp8, self.shared_up_fp8, self.shared_gate_scale, self.shared_up_scale
                    )
                    sd, sd_s = ops.pack_linear_down(self.shared_down_fp8, self.shared_down_scale)
                else:
                    sgu, sgu_s = ops.pack_linear_gate_up(fold(cw["shared_gate"], (1, -1)),
                                                         fold(cw["shared_up"], (1, -1)))
                    sd, sd_s = ops.pack_linear_down(cw["shared_down"])
                packed.shared_gate_up, packed.shared_gate_up_scale = sgu, sgu_s
                packed.shared_down, packed.shared_down_scale = sd, sd_s
        return packed

    def _hip_forward(self, flat_x: torch.Tensor, flat_ids: torch.Tensor, decision: BackendDecision,
                     residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        grad = torch.is_grad_enabled() and (
            flat_x.requires_grad
            or (residual is not None and residual.requires_grad)
            or weights.any_requires_grad(self)
        )
        # a differentiable call materialises each weight once: the same tensors
        # feed the pack (when it is rebuilt), the autograd inputs and the
        # backward packs (the reference fetches each expert tensor once,
        # engine.py:461-464)
        current = weights.materialize(self) if grad else None
        packed = self._hip_packed(current=current)
        x = flat_x if flat_x.dtype == packed.act_dtype else flat_x.to(packed.act_dtype)
        x = x.contiguous()
        order = ops.ORDER_ASSIGNMENT if decision.partition == PARTITION_ASSIGNMENT else ops.ORDER_TOKEN
        res = None
        if residual is not None:
            res = residual.reshape(-1, residual.size(-1))
            res = (res if res.dtype == packed.act_dtype else res.to(packed.act_dtype)).contiguous()
        if grad:
            params = tuple(current[n] for n in weights.WEIGHT_NAMES)
            plan = _LayerPlan(
                packed,
                lambda: self._hip_backward_packs(packed, current),
                flat_ids,
                self._active_route_table,
                self.config.route_weights,
                self.config.shared_output_scale,
                self.config.routed_output_scale,
                order,
                (self._active_num_experts, self._active_expert_width),
            )
            out = hip_layer_autograd(plan, x, res, params)
        else:
            out = ops.layer_forward(
                x,
                flat_ids,
                self._active_route_table,
                packed,
                self.config.route_weights,
                self.config.shared_output_scale,
                self.config.routed_output_scale,
                order=order,
                residual=res,
                act_fp8=ops.fp8_activation_mode(self.fp8_activations) if self._fp8 else False,
            )
        return out if out.dtype == flat_x.dtype else out.to(flat_x.dtype)

    def _hip_backward_packs(self, packed: ops.PackedLayer, current: dict) -> ops.BackwardPacks:
        """Transposed weight packs of the backward, cached with the forward pack.
        current: the weights the forward materialised (weights.materialize)."""
        if self._bwd_packed is not None and self._bwd_packed[0] is packed:
            return self._bwd_packed[1]
        E, W = self._active_num_experts, self._active_expert_width
        with torch.no_grad():
            bp = ops.backward_packs(
                packed,
                self.config.hidden_size,
                current["shared_down"],
                current["expert_down"][:E, :W, :],
            )
        self._bwd_packed = (packed, bp)
        return bp

    # ------------------------------------------------------------------ forward
    def _forward_eager(self, hidden_states: torch.Tensor, token_ids: torch.Tensor, backend,
                       decision: Optional[BackendDecision] = None) -> torch.Tensor:
        if hidden_states.ndim != 3:
            raise ValueError("hidden_states must be [batch, sequence, hidden]")
        if token_ids.shape != hidden_states.shape[:2]:
            raise ValueError("token_ids must match hidden batch/sequence dimensions")
        if hidden_states.size(-1) != self.config.hidden_size:
            raise ValueError(f"expected hidden size {self.config.hidden_size}, got {hidden_states.size(-1)}")
        batch, sequence, hidden = hidden_states.shape
        reduced = (
            self._active_num_experts != self.config.num_experts
            or self._active_expert_width != self.config.expert_width
        )
        if reduced and backend is TRHashBackend.FUSED_CUDA:
            raise RuntimeError(
                "FUSED_CUDA requires the full allocated capacity: its precompiled pair metadata is tied to "
                "config.num_experts. Use TRHashBackend.PYTORCH or CGGR while active capacity is reduced "
                f"(active={self._active_num_experts}/{self.config.num_experts} experts, "
                f"{self._active_expert_width}/{self.config.expert_width} width)."
            )
        flat_x = hidden_states.reshape(-1, hidden)
        if backend is TRHashBackend.HIP:
            if decision is None:
                decision = BackendDecision(TRHashBackend.HIP, TRHashBackend.HIP, (), False, self._fp8)
            out = self._hip_forward(flat_x, token_ids.reshape(-1), decision)
            return out.view(batch, sequence, hidden)
        if backend in (TRHashBackend.FUSED_CUDA, TRHashBackend.CGGR):
            raise RuntimeError(f"{backend.value} Triton kernels are not part of this build")
        shared = self._shared(flat_x)
        routes = self._routes(token_ids).reshape(self.config.top_k, -1)
        routed = self._reference_routed(flat_x, routes)
        out = self.config.shared_output_scale * shared + self.config.routed_output_scale * routed
        return out.view(batch, sequence, hidden)

    def _needs_autograd(self, hidden_states: torch.Tensor) -> bool:
        if not torch.is_grad_enabled():
            return False
        return hidden_states.requires_grad or any(p.requires_grad for p in self.parameters())

    def _decide(self, hidden_states: torch.Tensor) -> BackendDecision:
        # the decision depends on the frozen config, the device type, whether
        # the call is differentiable, the shared modules and their adapters'
        # dropout state; cached on those
        mods = self._modules
        shared = tuple(mods.get(n) for n in weights.SHARED_NAMES)
        key = (hidden_states.device.type, self._needs_autograd(hidden_states), id(self.config),
               tuple(id(m) for m in shared),
               tuple(m is not None and getattr(m, "is_lora_adapter", False) and weights.lora_dropout_active(m)
                     for m in shared),
               self._fp8)
        cached = self._decision_cache.get(key)
        if cached is not None:
            return cached
        decision = select_backend(
            self.config,
            device_type=hidden_states.device.type,
            autograd=key[1],
            quantized_weights=self._fp8,
        )
        reason = weights.shared_adapter_blocker(self) if decision.selected is TRHashBackend.HIP else None
        if reason is not None:
            # A LoRALinear on a shared linear adds a low-rank residual before
            # the SwiGLU (engine.py:337-345).  The HIP kernels serve it by its
            # merged weight; active LoRA dropout (or an adapter of unknown
            # form) has no merged weight, so the layer runs on the universal
            # path.
            if decision.requested is TRHashBackend.HIP:
                raise RuntimeError("HIP backend: " + reason)
            decision = replace(decision, selected=TRHashBackend.PYTORCH, reasons=decision.reasons + (reason,))
        if len(self._decision_cache) > 16:
            self._decision_cache.clear()
        self._decision_cache[key] = decision
        return decision

    def forward(self, hidden_states: torch.Tensor, token_ids: torch.Tensor) -> torch.Tensor:
        decision = self._decide(hidden_states)
        self.last_backend = decision
        if decision.selected is TRHashBackend.CUDA_GRAPH:
            return self._forward_cuda_graph(hidden_states, token_ids)
        return self._forward_eager(hidden_states, token_ids, decision.selected, decision)

    def forward_with_residual(self, hidden_states: torch.Tensor, token_ids: torch.Tensor,
                              residual: torch.Tensor) -> torch.Tensor:
        """``residual + forward(hidden_states, token_ids)``; on the HIP backend
        the add runs in the down-projection epilogue (block.py:270-278)."""
        decision = self._decide(hidden_states)
        self.last_backend = decision
        if decision.selected is TRHashBackend.HIP and hidden_states.ndim == 3:
            b, t, h = hidden_states.shape
            if token_ids.shape != hidden_states.shape[:2]:
                raise ValueError("token_ids must match hidden batch/sequence dimensions")
            out = self._hip_forward(hidden_states.reshape(-1, h), token_ids.reshape(-1), decision, residual)
            return out.view(b, t, h)
        return residual + self.forward(hidden_states, token_ids)

    def forward_norm_residual(self, hidden_states: torch.Tensor, token_ids: torch.Tensor,
                              norm_weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
        """``hidden + forward(rmsnorm(hidden), token_ids)``: the MLP half of a
        block (block.py:271-278) with its post-attention RMSNorm
        (norms.py:46-55) fused.  On the HIP backend, outside autograd and with
        bf16/f32 weights, the norm weight is folded into the packed gate/up
        weights, each token's 1/rms scales its gate and up accumulators (the
        decode kernels compute it from the activations they already stage),
        and the residual add runs in the down epilogue.  Under autograd, or
        with fp8 weights, the norm runs on the RMSNorm kernels
        (``RMSNormResidualFunction``: differentiable in hidden and
        norm_weight, with the residual's gradient added inside the norm's
        backward kernel) and then forward_with_residual.  Otherwise (another backend, or a dtype or
        hidden size the kernels do not take) it runs as the reference writes
        it.  ``last_norm`` records which: "fused", "rmsnorm" or "torch"."""
        if norm_weight.shape != (hidden_states.shape[-1],):
            raise ValueError("norm_weight must have shape (hidden_size,)")
        decision = self._decide(hidden_states)
        self.last_backend = decision
        grad = torch.is_grad_enabled() and (
            hidden_states.requires_grad
            or norm_weight.requires_grad
            or weights.any_requires_grad(self)
        )
        hip = decision.selected is TRHashBackend.HIP and hidden_states.ndim == 3 and eps > 0.0
        if hip and (grad or self._fp8) and ops.rmsnorm_unsupported(hidden_states, norm_weight) is None:
            b, t, h = hidden_states.shape
            flat = hidden_states.reshape(-1, h)
            self.last_norm = "rmsnorm"
            if grad:
                # the residual's gradient joins dx inside the norm's backward
                normed, res = RMSNormResidualFunction.apply(flat, norm_weight, float(eps))
                return self.forward_with_residual(normed.view(b, t, h), token_ids, res.view(b, t, h))
            normed, _ = ops.rmsnorm_forward(flat, norm_weight, float(eps))
            return self.forward_with_residual(normed.view(b, t, h), token_ids, hidden_states)
        if hip and not grad and not self._fp8:
            b, t, h = hidden_states.shape
            if token_ids.shape != hidden_states.shape[:2]:
                raise ValueError("token_ids must match hidden batch/sequence dimensions")
            packed = self._hip_packed(norm_weight)
            flat = hidden_states.reshape(-1, h)
            x = (flat if flat.dtype == packed.act_dtype else flat.to(packed.act_dtype)).contiguous()
            order = ops.ORDER_ASSIGNMENT if decision.partition == PARTITION_ASSIGNMENT else ops.ORDER_TOKEN
            out = ops.layer_forward(
                x,
                token_ids.reshape(-1),
                self._active_route_table,
                packed,
                self.config.route_weights,
                self.config.shared_output_scale,
                self.config.routed_output_scale,
                order=order,
                residual=x,
                norm_eps=float(eps),
            )
            out = out if out.dtype == hidden_states.dtype else out.to(hidden_states.dtype)
            self.last_norm = "fused"
            return out.view(b, t, h)
        variance = hidden_states.pow(2).mean(-1, keepdim=True)
        normed = norm_weight * (hidden_states * torch.rsqrt(variance + eps))
        self.last_norm = "torch"
        return self.forward_with_residual(normed, token_ids, hidden_states)

    def _forward_cuda_graph(self, hidden_states: torch.Tensor, token_ids: torch.Tensor) -> torch.Tensor:
        if self.training or torch.is_grad_enabled():
            raise RuntimeError("CUDA Graph TR-Hash requires eval mode and torch.no_grad()")
        if hidden_states.device.type != "cuda":
            raise RuntimeError("CUDA Graph TR-Hash requires CUDA tensors")
        if self._bucket_planner is None:
            raise RuntimeError("CUDA Graph backend has no configured buckets")
        batch, sequence, _ = hidden_states.shape
        bucket = self._bucket_planner.select(batch, sequence)
        runner = self._graph_pool.get(bucket)
        if runner is None:
            runner = _CapturedTRHashGraph(self, bucket, hidden_states)
            self._graph_pool[bucket] = runner
        return runner.replay(hidden_states, token_ids)

    def capability_summary(self, device_type: str = "cpu") -> dict:
        """Stable, serializable metadata (engine.py:616-655; same 21 keys)."""
        decision = select_backend(self.config, device_type=device_type)
        return {
            "experts": self.config.num_experts,
            "top_k": self.config.top_k,
            "shared_width": self.config.shared_width,
            "expert_width": self.config.expert_width,
            "stored_width": self.config.stored_mlp_width,
            "active_width": self.config.active_mlp_width,
            "active_width_fraction": self.config.active_width_fraction,
            "active_num_experts": self._active_num_experts,
            "active_expert_width": self._active_expert_width,
            "is_reduced_capacity": (
                self._active_num_experts != self.config.num_experts
                or self._active_expert_width != self.config.expert_width
            ),
            "attention": self.config.attention_backbone.value,
            "routing": self.config.routing_strategy.value,
            "phase": self.config.phase.value,
            "precision": self.config.precision.value,
            "world_size": self.config.world_size,
            "parallelism": "replicated_ddp" if self.config.world_size > 1 else "single_device",
            "requested_backend": decision.requested.value,
            "selected_backend": decision.selected.value,
            "backend_reasons": list(decision.reasons),
            "fused_cuda_eligible": supports_fused_cuda(self.config),
            "cuda_graph_buckets": [[b.batch_size, b.sequence_length] for b in self.config.graph_buckets],
        }


class _CapturedTRHashGraph:
    """One lazily captured static-shape inference graph (engine.py:658-716).

    The captured body is the HIP backend (its kernels record no memset nodes
    and allocate nothing outside torch's graph pool).  Without the library
    the capture raises, unless TRMOE_ALLOW_PYTORCH_FALLBACK=1 asks for the
    PYTORCH definition explicitly.

    The reference's graph reads the live parameters.  Here the kernels read
    the engine's packed copies, so the runner keeps the pack it captured
    (and its split-K scratch) alive and captures again at replay when the
    engine's current pack is another one: after load_state_dict, an in-place
    weight update or a change of routing strategy.  The same holds for the
    engine's fp8_activations switch, which picks other kernels.
    """

    def __init__(self, engine: TRHashEngine, bucket: GraphBucket, sample: torch.Tensor):
        if engine.config.phase is not TRHashPhase.INFERENCE:
            raise RuntimeError("only inference graphs can be captured")
        from .. import _native

        self.engine = engine
        self.bucket = bucket
        if _native.available():
            self.inner = TRHashBackend.HIP
        elif capabilities_allow_fallback():
            self.inner = TRHashBackend.PYTORCH
        else:
            raise RuntimeError(f"CUDA_GRAPH needs the HIP library: {_native.load_error()}")
        shape = (bucket.batch_size, bucket.sequence_length, engine.config.hidden_size)
        self.hidden = torch.zeros(shape, dtype=sample.dtype, device=sample.device)
        self.token_ids = torch.zeros(bucket.batch_size, bucket.sequence_length, dtype=torch.long,
                                     device=sample.device)
        self._capture()

    def _current_pack(self):
        return self.engine._hip_packed() if self.inner is TRHashBackend.HIP else None

    def _capture(self) -> None:
        engine = self.engine
        self.graph = None
        self.output = None
        self.packed = self._current_pack()
        self.act_fp8 = engine.fp8_activations
        self.scratch = ops.workspace_scope()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with self.scratch, torch.cuda.stream(stream):
            for _ in range(3):
                self.output = engine._forward_eager(self.hidden, self.token_ids, self.inner)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with self.scratch, torch.cuda.graph(graph):
            self.output = engine._forward_eager(self.hidden, self.token_ids, self.inner)
        self.graph = graph

    def replay(self, hidden_states: torch.Tensor, token_ids: torch.Tensor) -> torch.Tensor:
        batch, sequence, _ = hidden_states.shape
        if self.inner is TRHashBackend.HIP and (self._current_pack() is not self.packed
                                                or self.engine.fp8_activations != self.act_fp8):
            self._capture()
        self.hidden.zero_()
        self.token_ids.zero_()
        self.hidden[:batch, :sequence].copy_(hidden_states)
        self.token_ids[:batch, :sequence].copy_(token_ids)
        self.graph.replay()
        return self.output[:batch, :sequence].clone()
