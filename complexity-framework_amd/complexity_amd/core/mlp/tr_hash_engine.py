"""MLP adapter that runs TRHashEngine as a block's feed-forward.

Mirror of complexity/core/mlp/tr_hash_engine.py:25-158: same registry names
(``tr_hash_engine``, ``tr_hash_moe``), same config mapping, same runtime
controls.  Backend policy (``_backend``): ``use_custom_kernels=False`` forces
the PYTORCH definition, ``"hip"`` forces the gfx950 kernels, ``use_cggr=True``
requests CGGR (served here by the HIP kernels with the CGGR partition order),
anything else is AUTO (HIP on a ROCm device).
"""

from __future__ import annotations

from dataclasses import replace

from ...tr_hash import (
    AttentionBackbone,
    TRHashBackend,
    TRHashEngine,
    TRHashEngineConfig,
    TRHashPhase,
    TRHashPrecision,
    TRHashStrategy,
)
from ..registry import register_mlp
from .base import MLPBase, MLPConfig


def _route_weights(top_k: int, primary_weight):
    if top_k == 1:
        return (1.0,)
    primary = 1.0 / top_k if primary_weight is None else float(primary_weight)
    primary = min(1.0, max(0.0, primary))
    rest = (1.0 - primary) / (top_k - 1)
    return (primary,) + (rest,) * (top_k - 1)


_STRATEGY_ALIASES = {
    "modulo": TRHashStrategy.MODULO_CYCLIC,
    "modulo_cyclic": TRHashStrategy.MODULO_CYCLIC,
    "token_id_balanced_hash": TRHashStrategy.BALANCED_HASH,
    "token_id_multi_hash": TRHashStrategy.MULTI_HASH,
    "token_id_hierarchical_hash": TRHashStrategy.HIERARCHICAL_HASH,
}


def _strategy(value: str) -> TRHashStrategy:
    try:
        return _STRATEGY_ALIASES[str(value).lower()]
    except KeyError:
        raise ValueError(
            "tr_hash_engine supports modulo_cyclic, token_id_balanced_hash, token_id_multi_hash, "
            f"or token_id_hierarchical_hash; got {value!r}"
        ) from None


def _norm(policy):
    return policy.strip().lower() if isinstance(policy, str) else policy


def _backend(config: MLPConfig) -> TRHashBackend:
    kernels, cggr = _norm(config.use_custom_kernels), _norm(config.use_cggr)
    if kernels in {False, "false"}:
        return TRHashBackend.PYTORCH
    if kernels == "hip":
        return TRHashBackend.HIP
    if cggr in {True, "true"}:
        return TRHashBackend.CGGR
    return TRHashBackend.AUTO


@register_mlp("tr_hash_engine")
@register_mlp("tr_hash_moe")
class TRHashEngineMLP(MLPBase):
    """Shared SwiGLU plus fixed token-ID experts executed by TRHashEngine."""

    def __init__(self, config: MLPConfig, *, precision: TRHashPrecision = TRHashPrecision.BF16):
        super().__init__(config)
        if config.intermediate_size % config.num_experts:
            raise ValueError("TR-Hash routed width must be divisible by num_experts")
        if config.shared_expert:
            shared = config.shared_intermediate_size
            shared_width = int(shared if shared is not None else config.intermediate_size)
        else:
            shared_width = 0
        self.top_k = int(config.top_k)
        if self.top_k == 1:
            self._primary_weight = 1.0
        else:
            pw = config.top_k_primary_weight
            self._primary_weight = float(1.0 / self.top_k if pw is None else pw)
        self.engine = TRHashEngine(
            TRHashEngineConfig(
                hidden_size=config.hidden_size,
                vocab_size=config.vocab_size,
                num_experts=config.num_experts,
                top_k=self.top_k,
                shared_width=shared_width,
                expert_width=config.intermediate_size // config.num_experts,
                initializer_range=float(config.initializer_range),
                routing_strategy=_strategy(config.routing_strategy),
                layer_index=int(config.layer_idx),
                route_hash_count=int(config.route_hash_count),
                route_weights=_route_weights(self.top_k, config.top_k_primary_weight),
                shared_output_scale=float(config.shared_output_scale),
                routed_output_scale=float(config.routed_output_scale),
                attention_backbone=AttentionBackbone.GQA,
                phase=TRHashPhase.TRAINING,
                precision=precision,
                backend=_backend(config),
            )
        )
        if config.active_num_experts is not None or config.active_expert_width is not None:
            self.engine.set_active_capacity(
                num_experts=config.active_num_experts,
                expert_width=config.active_expert_width,
            )

    def forward(self, hidden_states, token_ids=None, **kwargs):
        if token_ids is None:
            raise ValueError("tr_hash_engine requires token_ids")
        return self.engine(hidden_states, token_ids)

    def forward_with_residual(self, hidden_states, residual, token_ids=None):
        """``residual + forward(hidden_states)`` (block.py:278), the add fused
        into the down projection on the HIP backend."""
        if token_ids is None:
            raise ValueError("tr_hash_engine requires token_ids")
        return self.engine.forward_with_residual(hidden_states, token_ids, residual)

    def forward_norm_residual(self, hidden_states, norm, token_ids=None):
        """``hidden + forward(norm(hidden))`` for the block's RMSNorm module
        ``norm`` (weight, eps; block.py:271-278), fused on the HIP backend."""
        if token_ids is None:
            raise ValueError("tr_hash_engine requires token_ids")
        return self.engine.forward_norm_residual(hidden_states, token_ids, norm.weight, norm.eps)

    def set_top_k_primary_weight(self, weight: float) -> None:
        if self.top_k == 1:
            self._primary_weight = 1.0
            return
        self._primary_weight = min(1.0, max(0.0, float(weight)))
        self.engine.config = replace(
            self.engine.config, route_weights=_route_weights(self.top_k, self._primary_weight)
        )

    def set_active_experts(self, num_experts: int) -> None:
        self.engine.set_active_capacity(num_experts=num_experts)

    def set_active_expert_width(self, width: int) -> None:
        self.engine.set_active_capacity(expert_width=width)

    def training_control_capabilities(self) -> frozenset:
        return frozenset({"topk_primary_weight", "active_num_experts", "active_expert_width"})

    def training_telemetry(self) -> dict:
        return {
            "topk_w": float(self._primary_weight),
            "active_num_experts": float(self.engine.active_num_experts),
            "active_expert_width": float(self.engine.active_expert_width),
        }

    def capability_summary(self, device_type: str = "cpu") -> dict:
        return self.engine.capability_summary(device_type)
