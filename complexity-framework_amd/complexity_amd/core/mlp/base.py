"""MLP plug-in base and config (the parts of complexity/core/mlp/base.py this path reads).

``MLPConfig`` keeps the reference's field names and defaults (base.py:16-73)
so that a block can hand the same config object to either implementation;
fields that only other MLP families use are accepted and ignored here.
"""

from __future__ import annotations

from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

_STRATEGIES = {
    "modulo",
    "modulo_cyclic",
    "modulo_balanced_secondary",
    "modulo_frequency_balanced_secondary",
    "token_id_balanced_hash",
    "token_id_pair_coverage_hash",
    "token_id_multi_hash",
    "token_id_hierarchical_hash",
}
_REMOVED = {"zipf", "round_robin", "random", "lsh_hidden"}


@dataclass
class MLPConfig:
    hidden_size: int
    intermediate_size: int
    hidden_act: str = "silu"
    bias: bool = False
    num_experts: int = 1
    expert_initialization: str = "gpt_normal"
    initializer_range: float = 0.02
    vocab_size: int = 100000
    hash_routing: str = ""
    routing_strategy: str = "modulo_cyclic"
    route_hash_count: int = 2
    token_frequencies: Optional[torch.Tensor] = None
    lsh_routing: bool = False
    lsh_bits: int = 0
    lsh_from_layer: int = 0
    lsh_threshold_mode: str = "zero"
    shared_expert: bool = True
    shared_intermediate_size: Optional[int] = None
    shared_expert_chunk_tokens: int = 0
    use_shared_routed_gates: bool = False
    shared_gate_init: float = 1.0
    routed_gate_init: float = 1.0
    shared_output_scale: float = 1.0
    routed_output_scale: float = 1.0
    top_k: int = 1
    top_k_primary_weight: Optional[float] = None  # None -> 1/top_k
    learn_hash_pair_gates: bool = False
    hash_pair_gate_init: float = 0.5
    learn_hash_channel_modulation: bool = False
    hash_channel_scale_init: float = 0.0
    layer_idx: int = 0
    static_expert_capacity: bool = False
    collect_moe_telemetry: bool = False
    active_num_experts: Optional[int] = None
    active_expert_width: Optional[int] = None
    use_custom_kernels: object = "auto"  # "auto", True, False, or "hip"
    use_cggr: object = "auto"
    lexical_object_rank: int = 16
    lexical_object_gate_init: float = 0.1
    micro_num_experts: int = 4
    micro_expert_width: int = 16
    micro_expert_gate_init: float = 0.1

    def __post_init__(self):
        for name in ("hidden_size", "intermediate_size", "num_experts", "vocab_size", "top_k"):
            if getattr(self, name) <= 0:
                raise ValueError(f"{name} must be positive")
        if self.initializer_range <= 0.0:
            raise ValueError("initializer_range must be positive")
        if self.expert_initialization not in {"gpt_normal", "legacy_kaiming"}:
            raise ValueError("expert_initialization must be 'gpt_normal' or 'legacy_kaiming'")
        if self.top_k > self.num_experts:
            raise ValueError("top_k cannot exceed num_experts")
        if self.top_k_primary_weight is not None and not 0.0 <= self.top_k_primary_weight <= 1.0:
            raise ValueError("top_k_primary_weight must be in [0, 1]")
        if self.routing_strategy in _REMOVED:
            raise ValueError(
                f"routing_strategy={self.routing_strategy!r} was removed: routing is deterministic "
                "token-ID / hash-table only"
            )
        if self.routing_strategy not in _STRATEGIES:
            raise ValueError(f"routing_strategy must be one of {sorted(_STRATEGIES)}")
        if not 2 <= self.route_hash_count <= 8:
            raise ValueError("route_hash_count must be between 2 and 8")
        for name in ("use_cggr",):
            value = getattr(self, name)
            if isinstance(value, str) and value.strip().lower() not in {"auto", "true", "false"}:
                raise ValueError(f"{name} must be one of 'auto', 'true', 'false', True, or False")
        if isinstance(self.use_custom_kernels, str) and self.use_custom_kernels.strip().lower() not in {
            "auto", "true", "false", "hip"
        }:
            raise ValueError("use_custom_kernels must be one of 'auto', 'true', 'false', 'hip', True, or False")
        if self.shared_intermediate_size is not None and self.shared_intermediate_size <= 0:
            raise ValueError("shared_intermediate_size must be positive when set")
        if self.shared_output_scale < 0.0:
            raise ValueError("shared_output_scale must be non-negative")
        if self.routed_output_scale < 0.0:
            raise ValueError("routed_output_scale must be non-negative")
        if self.active_num_experts is not None:
            if self.active_num_experts <= 0:
                raise ValueError("active_num_experts must be positive")
            if self.active_num_experts > self.num_experts:
                raise ValueError(
                    "active_num_experts cannot exceed num_experts "
                    f"({self.active_num_experts} > {self.num_experts})"
                )
        if self.active_expert_width is not None:
            if self.active_expert_width <= 0:
                raise ValueError("active_expert_width must be positive")
            limit = self.intermediate_size // self.num_experts
            if self.active_expert_width > limit:
                raise ValueError(
                    "active_expert_width cannot exceed intermediate_size // "
                    f"num_experts ({self.active_expert_width} > {limit})"
                )


class MLPBase(nn.Module, ABC):
    """Feed-forward plug-in interface: forward(hidden_states, token_ids=None, **kwargs)."""

    def __init__(self, config: MLPConfig):
        super().__init__()
        self.config = config
        self.hidden_size = config.hidden_size
        self.intermediate_size = config.intermediate_size

    def training_control_capabilities(self) -> frozenset:
        return frozenset()

    def training_telemetry(self) -> dict:
        return {}

    @abstractmethod
    def forward(self, hidden_states: torch.Tensor, token_ids: Optional[torch.Tensor] = None, **kwargs):
        """[batch, seq, hidden] -> [batch, seq, hidden]."""

    @staticmethod
    def get_activation(name: str):
        table = {
            "silu": F.silu,
            "swish": F.silu,
            "gelu": F.gelu,
            "relu": F.relu,
            "gelu_new": lambda x: F.gelu(x, approximate="tanh"),
        }
        if name not in table:
            raise ValueError(f"Unknown activation: {name}. Choose from {list(table)}")
        return table[name]
