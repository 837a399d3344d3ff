"""Seeded synthetic workloads of the measured TR-MoE configurations.

Shapes follow the benchmark configurations of this path: one TR-MoE layer at
the 200M dimensions (hidden 896, shared SwiGLU 3072, 4 experts x 64, top-2
multi-hash routing over a 32000 vocab) in fp32 (C1), bf16 prefill (C2) and
bf16 decode (C3; C4's 16-layer decode at 8 tokens), and the scaled fp8 layer
(C5).  Seeds: token ids from
generator ``seed``, x ~ N(0,1) from ``seed+1``, weights ~ N(0, 0.02) from
``seed+2`` drawn in parameter order (expert_gate, expert_up, expert_down,
shared_gate, shared_up, shared_down), all on the CPU so every device and the
CPU oracle see identical values.
"""

from __future__ import annotations

from dataclasses import dataclass, replace
from typing import Dict, Optional

import torch


@dataclass(frozen=True)
class LayerWorkload:
    name: str
    batch: int
    seq: int
    hidden: int = 896
    shared: int = 3072
    experts: int = 4
    width: int = 64
    top_k: int = 2
    vocab: int = 32000
    dtype: str = "bf16"         # activation/weight dtype: fp32 | bf16 | fp8 (weights)
    ids: str = "zipf"           # zipf | uniform
    zipf_s: float = 1.1
    layer_index: int = 0
    active_experts: Optional[int] = None
    active_width: Optional[int] = None

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def flops(self) -> float:
        """Algorithmic FLOPs: 6 N H (S + k W_active)."""
        w = self.active_width or self.width
        return 6.0 * self.tokens * self.hidden * (self.shared + self.top_k * w)


C1 = LayerWorkload("c1_fp32_2048", 4, 512, dtype="fp32", ids="uniform")
C2 = LayerWorkload("c2_bf16_prefill_16384", 8, 2048)
C3 = LayerWorkload("c3_bf16_decode_64", 64, 1)
# C4's MLP layers in greedy decode: 8 sequences, one token each, 16 layers
# with route tables of layer_index 0..15 (bench.py builds one engine per layer)
C4_DECODE = LayerWorkload("c4_bf16_decode_8", 8, 1)
C5 = LayerWorkload("c5_fp8_32768", 16, 2048, hidden=2048, shared=5632, experts=16, width=256, dtype="fp8")
C5_ACTIVE = replace(C5, name="c5_fp8_32768_active_8x128", active_experts=8, active_width=128)

WORKLOADS = {w.name: w for w in (C1, C2, C3, C4_DECODE, C5, C5_ACTIVE)}


def zipf_ids(n: int, vocab: int, s: float, generator: torch.Generator) -> torch.Tensor:
    """Truncated Zipf: P(rank r) ~ r^-s for r = 1..vocab, id = r - 1."""
    ranks = torch.arange(1, vocab + 1, dtype=torch.float64)
    p = ranks.pow(-s)
    p = p / p.sum()
    return torch.multinomial(p, n, replacement=True, generator=generator).to(torch.int64)


def make_token_ids(w: LayerWorkload, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    if w.ids == "uniform":
        ids = torch.randint(0, w.vocab, (w.tokens,), generator=g, dtype=torch.int64)
    else:
        ids = zipf_ids(w.tokens, w.vocab, w.zipf_s, g)
    return ids.view(w.batch, w.seq)


def make_hidden(w: LayerWorkload, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randn(w.batch, w.seq, w.hidden, generator=g, dtype=torch.float32)


def make_weights(w: LayerWorkload, seed: int = 0, std: float = 0.02) -> Dict[str, torch.Tensor]:
    """fp32 master weights in the engine's parameter layouts."""
    g = torch.Generator().manual_seed(seed + 2)
    E, H, W, S = w.experts, w.hidden, w.width, w.shared

    def normal(*shape):
        return torch.randn(*shape, generator=g, dtype=torch.float32) * std

    out = {
        "expert_gate": normal(E, H, W),
        "expert_up": normal(E, H, W),
        "expert_down": normal(E, W, H),
    }
    if S:
        out["shared_gate.weight"] = normal(S, H)
        out["shared_up.weight"] = normal(S, H)
        out["shared_down.weight"] = normal(H, S)
    return out


def engine_config(w: LayerWorkload, backend: str = "auto", **overrides):
    from .tr_hash import TRHashEngineConfig

    precision = {"fp32": "fp32", "bf16": "bf16", "fp8": "fp8"}[w.dtype]
    kwargs = dict(
        hidden_size=w.hidden,
        vocab_size=w.vocab,
        num_experts=w.experts,
        top_k=w.top_k,
        shared_width=w.shared,
        expert_width=w.width,
        routing_strategy="token_id_multi_hash",
        layer_index=w.layer_index,
        route_hash_count=2,
        precision=precision,
        phase="inference",
        backend=backend,
    )
    kwargs.update(overrides)
    return TRHashEngineConfig(**kwargs)


def build_engine(w: LayerWorkload, device, backend: str = "auto", seed: int = 0, **overrides):
    """TRHashEngine with the workload's weights loaded (fp8: quantised from them)."""
    from .tr_hash import TRHashEngine

    engine = TRHashEngine(engine_config(w, backend, **overrides))
    weights = make_weights(w, seed)
    with torch.no_grad():
        for name, value in weights.items():
            mod, _, attr = name.rpartition(".")
            target = getattr(engine, mod) if mod else engine
            getattr(target, attr).copy_(value)
    param_dtype = torch.float32 if w.dtype == "fp32" else torch.bfloat16
    engine = engine.to(device=device, dtype=param_dtype)
    if w.dtype == "fp8":
        engine.quantize_fp8_()
    if w.active_experts is not None or w.active_width is not None:
        engine.set_active_capacity(num_experts=w.active_experts, expert_width=w.active_width)
    return engine.eval()
