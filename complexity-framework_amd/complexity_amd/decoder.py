"""TR-GQA decoder around the TR-MoE layer: the harness of the 200M model.

The decoder is the reference's TR-GQA stack (ComplexityModel with
``attention_type="gqa"``, ``mlp_type="tr_hash_engine"``) at the released 200M
shape: 16 blocks of

    h = h + o_proj(SDPA(RoPE(qk_norm(q)), RoPE(qk_norm(k)), v))    block.py:205-268
    h = h + mlp(post_attention_layernorm(h), token_ids)             block.py:270-278

with RMSNorm (norms.py:46-55), fused KQV projection and GQA of 14 query over
2 key/value heads of width 64 (gqa.py:88-165, 169-218, SDPA at :229-266),
rotary embeddings over the absolute position (rotary.py:17-80, 239-295), a
final RMSNorm and the LM head tied to the embedding (builder.py:377-519).
The MLP half of every block is ``TRHashEngine.forward_norm_residual`` with
the route table of its layer index, i.e. the HIP kernels with the block's
RMSNorm and residual add fused in.

The reference's ``generate`` raises (builder.py:525-550), so the greedy loop
here is this build's own: ``prefill`` runs the prompt and fills a static KV
cache, ``decode_step`` appends one token per sequence, and ``generate``
replays a HIP-graph capture of the decode step (the position is a device
counter, so one capture serves every step).

Decode attention over the static cache: for one new token, GQA is the 14
query heads viewed as 2 groups of 7 rows, one group per key/value head
(head h uses key/value head h // 7, as ``repeat_interleave`` pairs them), so
SDPA runs on [B, 2, 7, 64] queries against the cache without copying it;
positions past the current one are masked.  The mask rules out the flash
kernel; SDPA's memory-efficient kernel takes it, and the math kernel is
never allowed (it would route bf16 batched products through a transposed
operand).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .tr_hash import TRHashEngine, TRHashEngineConfig

try:   # torch >= 2.3
    from torch.nn.attention import SDPBackend, sdpa_kernel
except ImportError:  # pragma: no cover - the image ships torch 2.10
    SDPBackend = None
    sdpa_kernel = None


@dataclass(frozen=True)
class TRGQAConfig:
    """The released TR-HASH MoE 200M shape (docs/tr-hash-200m-release.md)."""

    vocab_size: int = 32000
    hidden_size: int = 896
    num_layers: int = 16
    num_heads: int = 14
    num_kv_heads: int = 2
    head_dim: int = 64
    shared_width: int = 3072
    num_experts: int = 4
    expert_width: int = 64
    top_k: int = 2
    route_hash_count: int = 2
    route_weights: tuple = (0.5, 0.5)
    shared_output_scale: float = 1.0
    routed_output_scale: float = 2.0
    norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    max_position_embeddings: int = 2048
    initializer_range: float = 0.02

    @property
    def kv_groups(self) -> int:
        return self.num_heads // self.num_kv_heads


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight in the input dtype (norms.py:47-56)."""

    def __init__(self, size: int, eps: float):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(size))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        variance = x.pow(2).mean(-1, keepdim=True)
        return self.weight * (x * torch.rsqrt(variance + self.eps))


def _rotate_half(x: torch.Tensor) -> torch.Tensor:
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def rope_tables(head_dim: int, positions: int, theta: float):
    """cos/sin [positions, head_dim] in fp32 (rotary.py:41-56: emb = [freqs, freqs])."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(positions, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


class GQAttention(nn.Module):
    """Grouped-query attention with QK RMSNorm and RoPE (gqa.py:43-165)."""

    def __init__(self, cfg: TRGQAConfig):
        super().__init__()
        self.cfg = cfg
        H, D = cfg.hidden_size, cfg.head_dim
        self.k_proj = nn.Linear(H, cfg.num_kv_heads * D, bias=False)
        self.q_proj = nn.Linear(H, cfg.num_heads * D, bias=False)
        self.v_proj = nn.Linear(H, cfg.num_kv_heads * D, bias=False)
        self.o_proj = nn.Linear(cfg.num_heads * D, H, bias=False)
        self.q_norm = RMSNorm(D, 1e-6)
        self.k_norm = RMSNorm(D, 1e-6)
        self.scale = 1.0 / math.sqrt(D)
        self._kqv: Optional[torch.Tensor] = None
        self._kqv_key = None

    def kqv_weight(self) -> torch.Tensor:
        """[k; q; v] rows of one fused projection (gqa.py:211-218), cached on
        the three weights' storage and version."""
        ws = (self.k_proj.weight, self.q_proj.weight, self.v_proj.weight)
        key = tuple((w.data_ptr(), w._version) for w in ws)
        if self._kqv is None or self._kqv_key != key:
            with torch.no_grad():
                self._kqv = torch.cat(ws, dim=0)
            self._kqv_key = key
        return self._kqv

    def project(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor):
        """q [B, 14, T, D], k/v [B, 2, T, D] after QK norm and RoPE; cos/sin
        [T, D] (or [B, T, D]) in x's dtype."""
        B, T, _ = x.shape
        cfg = self.cfg
        kqv = F.linear(x, self.kqv_weight())
        kd, qd = cfg.num_kv_heads * cfg.head_dim, cfg.num_heads * cfg.head_dim
        k, q, v = kqv.split([kd, qd, kd], dim=-1)
        q = q.view(B, T, cfg.num_heads, cfg.head_dim).transpose(1, 2)
        k = k.view(B, T, cfg.num_kv_heads, cfg.head_dim).transpose(1, 2)
        v = v.view(B, T, cfg.num_kv_heads, cfg.head_dim).transpose(1, 2)
        q, k = self.q_norm(q), self.k_norm(k)
        if cos.dim() == 2:
            cos, sin = cos[None, None], sin[None, None]
        else:
            cos, sin = cos[:, None], sin[:, None]
        q = q * cos + _rotate_half(q) * sin
        k = k * cos + _rotate_half(k) * sin
        return q, k, v

    def prefill_attention(self, q, k, v) -> torch.Tensor:
        """Causal SDPA over the prompt, key/value heads repeated (gqa.py:150-152, 229-266)."""
        g = self.cfg.kv_groups
        k = k.repeat_interleave(g, dim=1)
        v = v.repeat_interleave(g, dim=1)
        return _sdpa(q, k, v, None, causal=True, scale=self.scale)

    def decode_attention(self, q, k_cache, v_cache, mask) -> torch.Tensor:
        """One new token per sequence: q [B, 14, 1, D] as [B, 2, 7, D] against
        the static cache [B, 2, L, D] with the position mask [1, 1, 1, L]."""
        B = q.shape[0]
        cfg = self.cfg
        qg = q.reshape(B, cfg.num_kv_heads, cfg.kv_groups, cfg.head_dim)
        out = _sdpa(qg, k_cache, v_cache, mask, causal=False, scale=self.scale)
        return out.reshape(B, cfg.num_heads, 1, cfg.head_dim)

    def output(self, attn: torch.Tensor) -> torch.Tensor:
        B, _, T, _ = attn.shape
        return self.o_proj(attn.transpose(1, 2).reshape(B, T, -1))


def _sdpa(q, k, v, mask, *, causal: bool, scale: float) -> torch.Tensor:
    """SDPA on the flash / memory-efficient kernels for reduced precision (the
    math kernel raises instead of running); any kernel for fp32."""
    if q.dtype == torch.float32 or sdpa_kernel is None:
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal, scale=scale)
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, is_causal=causal, scale=scale)


class TRGQABlock(nn.Module):
    def __init__(self, cfg: TRGQAConfig, layer_index: int, backend: str):
        super().__init__()
        self.input_layernorm = RMSNorm(cfg.hidden_size, cfg.norm_eps)
        self.self_attn = GQAttention(cfg)
        self.post_attention_layernorm = RMSNorm(cfg.hidden_size, cfg.norm_eps)
        self.mlp = TRHashEngine(TRHashEngineConfig(
            hidden_size=cfg.hidden_size, vocab_size=cfg.vocab_size, num_experts=cfg.num_experts,
            top_k=cfg.top_k, shared_width=cfg.shared_width, expert_width=cfg.expert_width,
            initializer_range=cfg.initializer_range, routing_strategy="token_id_multi_hash",
            layer_index=layer_index, route_hash_count=cfg.route_hash_count, route_weights=cfg.route_weights,
            shared_output_scale=cfg.shared_output_scale, routed_output_scale=cfg.routed_output_scale,
            attention_backbone="gqa", phase="inference", precision="bf16", backend=backend))
        self.layer_index = layer_index


# Replaces a block's MLP half (tests compare against a decoder whose MLPs run
# another definition): (layer index, h [B, T, H], token ids [B, T], block)
# -> h + mlp(post_attention_layernorm(h)).
MLPFn = Callable[[int, torch.Tensor, torch.Tensor, TRGQABlock], torch.Tensor]


class TRGQADecoder(nn.Module):
    """16-layer TR-GQA decoder with a static KV cache and a greedy loop."""

    def __init__(self, cfg: TRGQAConfig = TRGQAConfig(), backend: str = "auto", mlp_fn: Optional[MLPFn] = None):
        super().__init__()
        self.cfg = cfg
        self.embed_tokens = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(TRGQABlock(cfg, i, backend) for i in range(cfg.num_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.norm_eps)
        self.mlp_fn = mlp_fn
        self.k_cache: List[torch.Tensor] = []
        self.v_cache: List[torch.Tensor] = []
        self.cache_len = 0
        self._pos: Optional[torch.Tensor] = None   # device int64 [1]: next decode position
        self._rope = None
        self._graph = None

    # ------------------------------------------------------------------ weights
    @torch.no_grad()
    def init_weights(self, seed: int = 0) -> "TRGQADecoder":
        """Seeded GPT-style init (builder.py:177-232): N(0, 0.02) for linears,
        expert tensors and the embedding; o_proj and the MLP down projections
        N(0, 0.02 / sqrt(2 * layers)); norm weights one.  Drawn on the CPU in
        parameter order, so every device and dtype sees the same values."""
        g = torch.Generator().manual_seed(seed)
        std = self.cfg.initializer_range
        residual_std = std / math.sqrt(2 * self.cfg.num_layers)
        for name, p in self.named_parameters():
            if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
                p.fill_(1.0)
                continue
            s = residual_std if (name.endswith("o_proj.weight") or name.endswith("expert_down")
                                 or name.endswith("shared_down.weight")) else std
            p.copy_((torch.randn(p.shape, generator=g, dtype=torch.float32) * s).to(p.dtype))
        return self

    # ------------------------------------------------------------------ pieces
    def _mlp(self, block: TRGQABlock, h: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
        if self.mlp_fn is not None:
            return self.mlp_fn(block.layer_index, h, ids, block)
        norm = block.post_attention_layernorm
        return block.mlp.forward_norm_residual(h, ids, norm.weight, norm.eps)

    def _rope_tables(self, positions: int, device, dtype):
        if self._rope is None or self._rope[0].shape[0] < positions or self._rope[0].device != device \
                or self._rope[0].dtype != dtype:
            n = max(positions, self.cfg.max_position_embeddings)
            cos, sin = rope_tables(self.cfg.head_dim, n, self.cfg.rope_theta)
            self._rope = (cos.to(device=device, dtype=dtype), sin.to(device=device, dtype=dtype))
        return self._rope

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        return F.linear(self.norm(h), self.embed_tokens.weight)

    # ------------------------------------------------------------------ prompt
    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, max_new_tokens: int = 0, return_logits: bool = True,
                timings: Optional[Dict[str, list]] = None):
        """Runs the prompt [B, T], allocates the static KV cache for
        T + max_new_tokens positions and fills its first T; returns the logits
        [B, T, V] (or the last hidden state when return_logits is False).
        timings: lists of (start, end) CUDA events per layer under "attention"
        and "mlp"."""
        B, T = input_ids.shape
        cfg = self.cfg
        dev = input_ids.device
        dt = self.embed_tokens.weight.dtype
        # static cache rounded to 64 positions (the masked decode kernel wants
        # an aligned mask row; positions past the current one are masked)
        L = (T + max_new_tokens + 63) // 64 * 64
        self.k_cache = [torch.zeros(B, cfg.num_kv_heads, L, cfg.head_dim, device=dev, dtype=dt)
                        for _ in self.layers]
        self.v_cache = [torch.zeros_like(c) for c in self.k_cache]
        self.cache_len = T
        self._graph = None
        cos, sin = self._rope_tables(L, dev, dt)
        cos, sin = cos[:T], sin[:T]
        h = self.embed_tokens(input_ids)
        for i, block in enumerate(self.layers):
            ev = _events(timings, "attention")
            x = block.input_layernorm(h)
            q, k, v = block.self_attn.project(x, cos, sin)
            self.k_cache[i][:, :, :T].copy_(k)
            self.v_cache[i][:, :, :T].copy_(v)
            h = h + block.self_attn.output(block.self_attn.prefill_attention(q, k, v))
            _end(ev)
            ev = _events(timings, "mlp")
            h = self._mlp(block, h, input_ids)
            _end(ev)
        self._pos = torch.full((1,), T, dtype=torch.int64, device=dev)
        return self.logits(h) if return_logits else h

    # ------------------------------------------------------------------ decode
    def _decode_body(self, ids: torch.Tensor) -> torch.Tensor:
        """One token per sequence at device position self._pos (ids [B]);
        returns logits [B, V].  Graph-capturable: no host reads."""
        cfg = self.cfg
        B = ids.shape[0]
        L = self.k_cache[0].shape[2]
        dt = self.embed_tokens.weight.dtype
        cos_t, sin_t = self._rope_tables(L, ids.device, dt)
        pos = self._pos
        cos = cos_t.index_select(0, pos)           # [1, D]
        sin = sin_t.index_select(0, pos)
        span = torch.arange(L, device=ids.device)
        mask = torch.where(span <= pos, 0.0, -1e9).to(dt).view(1, 1, 1, L)
        tok = ids.view(B, 1)
        h = self.embed_tokens(tok)
        for i, block in enumerate(self.layers):
            x = block.input_layernorm(h)
            q, k, v = block.self_attn.project(x, cos, sin)
            self.k_cache[i].index_copy_(2, pos, k)
            self.v_cache[i].index_copy_(2, pos, v)
            attn = block.self_attn.decode_attention(q, self.k_cache[i], self.v_cache[i], mask)
            h = h + block.self_attn.output(attn)
            h = self._mlp(block, h, tok)
        return self.logits(h).view(B, -1)

    @torch.no_grad()
    def decode_step(self, ids: torch.Tensor) -> torch.Tensor:
        """Eager decode of one token per sequence; advances the position."""
        if self.cache_len >= self.k_cache[0].shape[2]:
            raise RuntimeError("KV cache full: prefill with a larger max_new_tokens")
        out = self._decode_body(ids)
        self._pos.add_(1)
        self.cache_len += 1
        return out

    @torch.no_grad()
    def capture_decode(self, batch: int):
        """Captures one greedy decode step in a HIP graph: static ids in,
        argmax ids out (written back as the next step's input), position
        advanced on the device.  Warm-up runs happen on a copy of the cache
        state and are undone."""
        dev = self.embed_tokens.weight.device
        self._g_ids = torch.zeros(batch, dtype=torch.int64, device=dev)
        self._g_logits = None
        saved_pos = self._pos.clone()
        saved = [(k.clone(), v.clone()) for k, v in zip(self.k_cache, self.v_cache)]
        # the graph owns the scratch its launches were recorded with
        self._g_scratch = ops.workspace_scope()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with self._g_scratch, torch.cuda.stream(stream):
            for _ in range(2):   # builds every lazy pack before capture
                self._graph_step()
                self._pos.copy_(saved_pos)
        torch.cuda.current_stream().wait_stream(stream)
        graph = torch.cuda.CUDAGraph()
        with self._g_scratch, torch.cuda.graph(graph):
            self._graph_step()
        self._pos.copy_(saved_pos)
        for (k, v), (k0, v0) in zip(zip(self.k_cache, self.v_cache), saved):
            k.copy_(k0)
            v.copy_(v0)
        self._graph = graph
        return graph

    def _graph_step(self):
        logits = self._decode_body(self._g_ids)
        self._g_logits = logits
        self._g_ids.copy_(logits.argmax(dim=-1))
        self._pos.add_(1)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, steps: int, use_graph: bool = True) -> torch.Tensor:
        """Greedy continuation of the prompt [B, T]: the prompt's next token
        then `steps` decode steps of one token per sequence -> [B, steps + 1]."""
        h = self.prefill(input_ids, steps + 1, return_logits=False)
        first = self.logits(h[:, -1:]).argmax(dim=-1).view(-1)
        return self.continue_greedy(first, steps, use_graph)

    @torch.no_grad()
    def continue_greedy(self, first: torch.Tensor, steps: int, use_graph: bool = True) -> torch.Tensor:
        """`steps` greedy decode steps after prefill, starting from the token
        `first` [B]; returns [B, steps + 1] (first included)."""
        B = first.shape[0]
        out = torch.empty(B, steps + 1, dtype=torch.int64, device=first.device)
        out[:, 0] = first
        if self.cache_len + steps > self.k_cache[0].shape[2]:
            raise RuntimeError("KV cache too small: prefill with a larger max_new_tokens")
        if use_graph:
            if self._graph is None:
                self.capture_decode(B)
            self._g_ids.copy_(first)
            for s in range(1, steps + 1):
                self._graph.replay()
                out[:, s] = self._g_ids
            self.cache_len += steps
            return out
        ids = first
        for s in range(1, steps + 1):
            ids = self.decode_step(ids).argmax(dim=-1)
            out[:, s] = ids
        return out


def _events(timings, key):
    if timings is None:
        return None
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    timings.setdefault(key, []).append((s, e))
    return e


def _end(ev):
    if ev is not None:
        ev.record()
