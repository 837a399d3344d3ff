"""Deterministic token-ID route tables (behaviour of complexity/tr_hash/routing.py).

Tables are built once on the host, as in the reference, and persisted as the
``route_table`` buffer ``int64[top_k, vocab]``; the GPU only gathers from
them.  The arithmetic (32-bit masked hashes, salts, strides, seeded
permutations) must match the reference bit for bit, because trained expert
weights are paired with the exact table they were trained against; golden
digests written by the reference pin every strategy here.
"""

from __future__ import annotations

from dataclasses import replace
from itertools import combinations

import torch

from .config import TRHashEngineConfig, TRHashStrategy

_U32 = 0xFFFFFFFF
_GOLDEN = 0x9E3779B1       # per-layer salt multiplier
_CHANNEL = 0x85EBCA77      # per-hash-channel salt step / stride salt
_EXPERT = 0xC2B2AE3D       # expert salt


def mix32(values: torch.Tensor) -> torch.Tensor:
    """Wellons' lowbias32 on int64 tensors holding 32-bit values (routing.py:97-103)."""
    v = values & _U32
    for shift, mult in ((16, 0x7FEB352D), (15, 0x846CA68B)):
        v = ((v ^ (v >> shift)) * mult) & _U32
    return (v ^ (v >> 16)) & _U32


def _salt(config: TRHashEngineConfig) -> int:
    return (int(config.route_seed) + int(config.layer_index) * _GOLDEN) & _U32


def _seeded_randperm(n: int, seed: int) -> torch.Tensor:
    gen = torch.Generator(device="cpu").manual_seed(int(seed))
    return torch.randperm(n, generator=gen, device="cpu")


def _layer_permutation(num_experts: int, layer_index: int, seed: int) -> torch.Tensor:
    return _seeded_randperm(num_experts, int(seed) + 104729 * int(layer_index))


def _multi_hash(config: TRHashEngineConfig) -> torch.Tensor:
    """Rendezvous voting: top-k of the summed per-channel scores (routing.py:129-167)."""
    token = torch.arange(config.vocab_size, dtype=torch.int64).view(-1, 1)
    expert = torch.arange(config.num_experts, dtype=torch.int64).view(1, -1)
    salt = _salt(config)
    channels = [(salt + h * _CHANNEL) & _U32 for h in range(config.route_hash_count)]
    score = sum(mix32(token ^ mix32(expert + (c ^ _EXPERT)) ^ c) for c in channels)
    return score.topk(config.top_k, dim=1, largest=True, sorted=True).indices.t().contiguous()


def _affine_hash(config: TRHashEngineConfig) -> torch.Tensor:
    """base + slot * odd_stride (mod E) (routing.py:106-126)."""
    token = torch.arange(config.vocab_size, dtype=torch.int64)
    salt = _salt(config)
    base = mix32(token ^ salt) % config.num_experts
    stride = (mix32(token + (salt ^ _CHANNEL)) | 1) % config.num_experts
    slots = torch.arange(config.top_k, dtype=torch.int64).view(-1, 1)
    return (base.view(1, -1) + slots * stride.view(1, -1)) % config.num_experts


def _modulo_cyclic(config: TRHashEngineConfig) -> torch.Tensor:
    """Permuted token % E, then consecutive experts (routing.py:81-94)."""
    perm = _layer_permutation(config.num_experts, config.layer_index, config.route_seed ^ 0xC0DE)
    primary = perm[torch.arange(config.vocab_size) % config.num_experts]
    slots = torch.arange(config.top_k, dtype=torch.int64).view(-1, 1)
    return (primary.view(1, -1) + slots) % config.num_experts


def _balanced_hash(config: TRHashEngineConfig) -> torch.Tensor:
    """Collision-free tuples with exact per-slot balance (routing.py:17-78)."""
    E, V, k = config.num_experts, config.vocab_size, config.top_k
    if E == 1:
        return torch.zeros(k, V, dtype=torch.int64)
    order = _seeded_randperm(V, int(config.route_seed) + 104729 * int(config.layer_index))
    rank = torch.arange(V, dtype=torch.int64)
    block, position = rank // E, rank % E
    odd = torch.arange(1, E, 2, dtype=torch.int64)
    pick = mix32(block + int(config.route_seed) + int(config.layer_index) * _GOLDEN) % odd.numel()
    stride = odd[pick]
    perm = _layer_permutation(E, config.layer_index, config.route_seed ^ 0x5EC0D)
    slots = torch.arange(k, dtype=torch.int64).view(-1, 1)
    ranked = perm[(position.view(1, -1) + slots * stride.view(1, -1)) % E]
    table = torch.empty(k, V, dtype=torch.int64)
    table[:, order] = ranked
    return table


def expand_route_table_hierarchically(
    routes: torch.Tensor,
    *,
    source_num_experts: int,
    target_num_experts: int,
    layer_index: int,
    route_seed: int = 0x71D5A17,
) -> torch.Tensor:
    """Split each source expert e into clones e + c*source (routing.py:170-210)."""
    if routes.ndim != 2:
        raise ValueError("routes must be shaped [top_k, vocab_size]")
    if source_num_experts < 1:
        raise ValueError("source_num_experts must be positive")
    if target_num_experts <= source_num_experts:
        raise ValueError("target_num_experts must exceed source_num_experts")
    if target_num_experts % source_num_experts:
        raise ValueError("target_num_experts must be a multiple of source_num_experts")
    parents = routes.detach().to(device="cpu", dtype=torch.int64)
    if parents.numel() and (int(parents.min()) < 0 or int(parents.max()) >= source_num_experts):
        raise ValueError("routes contain an invalid source expert index")
    clones = target_num_experts // source_num_experts
    token = torch.arange(parents.size(1), dtype=torch.int64).view(1, -1)
    slot = torch.arange(parents.size(0), dtype=torch.int64).view(-1, 1)
    salt = (int(route_seed) + int(layer_index) * _GOLDEN) & _U32
    clone = mix32(token ^ (parents * _CHANNEL) ^ (slot * _EXPERT) ^ salt) % clones
    return parents + clone * source_num_experts


def _hierarchical_hash(config: TRHashEngineConfig) -> torch.Tensor:
    if config.num_experts < 4 or config.num_experts % 2:
        raise ValueError("hierarchical hash requires an even expert count of at least four")
    parents = config.num_experts // 2
    if config.top_k > parents:
        raise ValueError("top_k cannot exceed the hierarchical parent expert count")
    base = _balanced_hash(replace(config, num_experts=parents, routing_strategy=TRHashStrategy.BALANCED_HASH))
    return expand_route_table_hierarchically(
        base,
        source_num_experts=parents,
        target_num_experts=config.num_experts,
        layer_index=config.layer_index,
        route_seed=config.route_seed,
    )


_BUILDERS = {
    TRHashStrategy.MULTI_HASH: _multi_hash,
    TRHashStrategy.AFFINE_HASH: _affine_hash,
    TRHashStrategy.BALANCED_HASH: _balanced_hash,
    TRHashStrategy.MODULO_CYCLIC: _modulo_cyclic,
    TRHashStrategy.HIERARCHICAL_HASH: _hierarchical_hash,
}


def build_route_table(config: TRHashEngineConfig) -> torch.Tensor:
    """CPU ``int64[top_k, vocab_size]`` table, validated (routing.py:235-259)."""
    try:
        builder = _BUILDERS[config.routing_strategy]
    except KeyError:  # pragma: no cover - the enum makes this unreachable
        raise ValueError(f"unsupported TR-Hash strategy: {config.routing_strategy}")
    routes = builder(config).to(torch.int64).contiguous()
    if tuple(routes.shape) != (config.top_k, config.vocab_size):
        raise RuntimeError("route builder returned an invalid shape")
    if int(routes.min()) < 0 or int(routes.max()) >= config.num_experts:
        raise RuntimeError("route builder returned an invalid expert index")
    if config.top_k > 1:
        ordered = routes.sort(dim=0).values
        if bool((ordered[1:] == ordered[:-1]).any()):
            raise RuntimeError("route builder selected one expert twice")
    return routes


def _pair_masks(pair_count: int):
    return (0x7, 0x8) if pair_count <= 8 else (0x1F, 0x20)


def compile_top2_pair_metadata(routes: torch.Tensor, *, num_experts: int):
    """uint8 pair code per token + lexicographic pair list (routing.py:262-311)."""
    if routes.ndim != 2 or routes.size(0) != 2:
        raise ValueError("routes must be shaped [2, vocab_size]")
    if not 2 <= num_experts <= 8:
        raise ValueError("compact pair metadata supports two to eight experts")
    r = routes.detach().to(device="cpu", dtype=torch.int64)
    if r.numel() and (int(r.min()) < 0 or int(r.max()) >= num_experts):
        raise ValueError("routes contain an invalid expert index")
    pairs = torch.tensor(list(combinations(range(num_experts), 2)), dtype=torch.int32)
    if pairs.size(0) > 32:
        raise ValueError("compact pair encoding supports at most 32 pairs")
    lo, hi = torch.minimum(r[0], r[1]), torch.maximum(r[0], r[1])
    if bool((lo == hi).any()):
        raise ValueError("top-2 pair routes must select two distinct experts")
    # index of (lo, hi) among lexicographic pairs of range(E)
    pair_index = lo * num_experts - lo * (lo + 1) // 2 + (hi - lo - 1)
    _, swap_bit = _pair_masks(int(pairs.size(0)))
    swapped = (r[0] == hi).to(torch.int64)
    return (pair_index | (swapped * swap_bit)).to(torch.uint8), pairs


def decode_top2_pair_metadata(route_codes: torch.Tensor, expert_pairs: torch.Tensor) -> torch.Tensor:
    """Inverse of compile_top2_pair_metadata (routing.py:314-338)."""
    if route_codes.ndim != 1 or route_codes.dtype != torch.uint8:
        raise ValueError("route_codes must be a one-dimensional uint8 tensor")
    if expert_pairs.ndim != 2 or expert_pairs.size(1) != 2:
        raise ValueError("expert_pairs must be shaped [pair_count, 2]")
    codes = route_codes.to(torch.int64)
    pair_mask, swap_mask = _pair_masks(int(expert_pairs.size(0)))
    idx = codes & pair_mask
    if idx.numel() and int(idx.max()) >= expert_pairs.size(0):
        raise ValueError("route_codes reference an unavailable expert pair")
    chosen = expert_pairs[idx].to(torch.int64)
    swap = (codes & swap_mask) != 0
    first = torch.where(swap, chosen[:, 1], chosen[:, 0])
    second = torch.where(swap, chosen[:, 0], chosen[:, 1])
    return torch.stack((first, second))
