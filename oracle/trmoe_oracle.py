"""CPU oracle for the TR-MoE feed-forward hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The shipped package (``complexity_amd``) never
imports anything under ``oracle/``.

It restates, independently of the product code, the algorithm of the
reference's universal PyTorch dispatch for ``TRHashEngine``:

* integer routing (``complexity/tr_hash/routing.py``) in numpy uint64
  arithmetic masked to 32 bits (a C restatement of the multi-hash table and
  the counting partition lives in ``route_oracle.c``);
* the two permutation orders of the expert partition
  (``complexity_cuda/triton_token_routed.py``);
* the floating-point layer (``complexity/tr_hash/engine.py``) with torch CPU
  fp32/bf16 ops, both as the reference's masked dense per-expert loop and as
  the token-by-token loop of the reference's own test.

Pinning (what checks each function beyond retyping it):

* ``mix32`` -- round trip through the published inverse of Wellons'
  "lowbias32" (constants 0x43021123 / 0x1d69e2a5), which fails if any forward
  constant or shift is wrong; plus golden tables written by the reference.
* route tables -- golden fixtures written by the reference's
  ``build_route_table`` (``tests/golden/make_reference_vectors.py``) and the
  invariants of ``tests/test_tr_hash_engine.py:51-110,159-180``; the C
  restatement must agree bit for bit.
* pair metadata -- golden fixtures + decode(encode(r)) == r.
* counting partition -- brute force over every assignment on small inputs
  (sort by the named key) + permutation/inverse/histogram invariants.
* layer forward -- the masked-dense loop against the token-by-token loop
  (two different formulations, as the reference's own test does), shared
  SwiGLU against an explicit per-token loop, and the f32 path against f64.
* layer backward -- ``engine_backward`` (autograd of ``engine_forward``)
  against central finite differences in f64 (``torch.autograd.gradcheck``);
  the closed-form ``swiglu_backward`` against that autograd.
* ``rms_norm`` -- torch's own ``F.rms_norm`` (an independent implementation)
  and the closed form of a constant row (every element becomes sign * weight);
  its autograd against central differences.
* ``engine_forward_w8a8`` -- equal to ``engine_forward`` on activations that
  quantize exactly (e4m3 grid values whose row maximum is 448 * 2^j), equal
  to it when the layer has no shared branch, and within e4m3's relative error
  of it otherwise.
* ``block_exponents_e4m3`` / ``quantize_blocks_e4m3`` -- the exponent rule
  against a brute-force search for the smallest e with amax <= 448 * 2^e in
  float64, over random and boundary maxima (448 * 2^j and its float32
  neighbours, zero, non-finite, the clamps); every block's largest code in
  [224, 448]; exactly representable blocks round-trip unchanged.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

MASK32 = 0xFFFFFFFF
DEFAULT_ROUTE_SEED = 0x71D5A17

ORDER_TOKEN = 0        # (expert, token): the reference's fused GPU partition
ORDER_ASSIGNMENT = 1   # (expert, slot*N + token): CPU fallback / CGGR sort


# ---------------------------------------------------------------------------
# integer routing
# ---------------------------------------------------------------------------

def mix32(values) -> np.ndarray:
    """32-bit avalanche hash (routing.py:97-103, Wellons' lowbias32).

    Operates on uint64 arrays holding 32-bit values; every product is below
    2**63 so uint64 arithmetic is exact before masking.
    """
    v = np.asarray(values, dtype=np.uint64) & np.uint64(MASK32)
    v = (v ^ (v >> np.uint64(16))) & np.uint64(MASK32)
    v = (v * np.uint64(0x7FEB352D)) & np.uint64(MASK32)
    v = (v ^ (v >> np.uint64(15))) & np.uint64(MASK32)
    v = (v * np.uint64(0x846CA68B)) & np.uint64(MASK32)
    return (v ^ (v >> np.uint64(16))) & np.uint64(MASK32)


def mix32_inverse(values) -> np.ndarray:
    """Published inverse of lowbias32 (independent constants); test helper."""
    v = np.asarray(values, dtype=np.uint64) & np.uint64(MASK32)
    v = (v ^ (v >> np.uint64(16))) & np.uint64(MASK32)
    v = (v * np.uint64(0x43021123)) & np.uint64(MASK32)
    v = (v ^ (v >> np.uint64(15)) ^ (v >> np.uint64(30))) & np.uint64(MASK32)
    v = (v * np.uint64(0x1D69E2A5)) & np.uint64(MASK32)
    return (v ^ (v >> np.uint64(16))) & np.uint64(MASK32)


def layer_salt(route_seed: int, layer_index: int) -> int:
    """routing.py:114, :156-158."""
    return (int(route_seed) + int(layer_index) * 0x9E3779B1) & MASK32


def multi_hash_scores(vocab_size: int, num_experts: int, layer_index: int,
                      route_seed: int = DEFAULT_ROUTE_SEED,
                      hash_count: int = 2) -> np.ndarray:
    """Rendezvous scores ``[V, E]`` of routing.py:129-166 (uint64, unmasked sum)."""
    tokens = np.arange(vocab_size, dtype=np.uint64)[:, None]
    experts = np.arange(num_experts, dtype=np.uint64)[None, :]
    salt = layer_salt(route_seed, layer_index)
    scores = np.zeros((vocab_size, num_experts), dtype=np.uint64)
    for h in range(hash_count):
        channel = (salt + h * 0x85EBCA77) & MASK32
        expert_salt = mix32(experts + np.uint64(channel ^ 0xC2B2AE3D))
        scores += mix32(tokens ^ expert_salt ^ np.uint64(channel))
    return scores


def multi_hash_table(vocab_size: int, num_experts: int, top_k: int,
                     layer_index: int, route_seed: int = DEFAULT_ROUTE_SEED,
                     hash_count: int = 2) -> np.ndarray:
    """``[k, V]`` int64 table: top-k experts by descending score (routing.py:167).

    Ties (none occur at the shapes this build is measured on) are broken
    toward the lower expert index.
    """
    scores = multi_hash_scores(vocab_size, num_experts, layer_index, route_seed, hash_count)
    # stable argsort of the negated order: descending score, ascending expert
    order = np.argsort(-scores.astype(np.float64), axis=1, kind="stable")
    # float64 keeps 2**33 distinct integers exactly, so the order is exact
    return order[:, :top_k].T.astype(np.int64).copy()


def affine_hash_table(vocab_size: int, num_experts: int, top_k: int,
                      layer_index: int, route_seed: int = DEFAULT_ROUTE_SEED) -> np.ndarray:
    """routing.py:106-126: base + r * odd_stride (mod E)."""
    tokens = np.arange(vocab_size, dtype=np.uint64)
    salt = layer_salt(route_seed, layer_index)
    base = mix32(tokens ^ np.uint64(salt)) % np.uint64(num_experts)
    stride = (mix32(tokens + np.uint64(salt ^ 0x85EBCA77)) | np.uint64(1)) % np.uint64(num_experts)
    rows = [(base + np.uint64(r) * stride) % np.uint64(num_experts) for r in range(top_k)]
    return np.stack(rows).astype(np.int64)


def _randperm(n: int, seed: int) -> np.ndarray:
    # routing.py:12-14 / :33-40 draw from torch's CPU generator; the oracle
    # calls the same generator (this is the RNG stream, not arithmetic).
    gen = torch.Generator(device="cpu").manual_seed(int(seed))
    return torch.randperm(n, generator=gen, device="cpu").numpy().astype(np.int64)


def modulo_cyclic_table(vocab_size: int, num_experts: int, top_k: int,
                        layer_index: int, route_seed: int = DEFAULT_ROUTE_SEED) -> np.ndarray:
    """routing.py:81-94."""
    perm = _randperm(num_experts, (route_seed ^ 0xC0DE) + 104729 * layer_index)
    primary = perm[np.arange(vocab_size) % num_experts]
    return np.stack([(primary + r) % num_experts for r in range(top_k)]).astype(np.int64)


def balanced_hash_table(vocab_size: int, num_experts: int, top_k: int,
                        layer_index: int, route_seed: int = DEFAULT_ROUTE_SEED) -> np.ndarray:
    """routing.py:17-78: per rank-block odd stride over a permuted expert set."""
    if num_experts == 1:
        return np.zeros((top_k, vocab_size), dtype=np.int64)
    token_order = _randperm(vocab_size, route_seed + 104729 * layer_index)
    rank = np.arange(vocab_size, dtype=np.int64)
    group = rank // num_experts
    position = rank % num_experts
    odd = np.arange(1, num_experts, 2, dtype=np.int64)
    sidx = mix32((group + route_seed + layer_index * 0x9E3779B1).astype(np.uint64)
                 & np.uint64(0xFFFFFFFFFFFFFFFF)).astype(np.int64) % odd.size
    stride = odd[sidx]
    perm = _randperm(num_experts, (route_seed ^ 0x5EC0D) + 104729 * layer_index)
    ranked = np.stack([perm[(position + r * stride) % num_experts] for r in range(top_k)])
    table = np.empty((top_k, vocab_size), dtype=np.int64)
    table[:, token_order] = ranked
    return table


def hierarchical_expand(routes: np.ndarray, source: int, target: int,
                        layer_index: int, route_seed: int = DEFAULT_ROUTE_SEED) -> np.ndarray:
    """routing.py:170-210: expert e -> e + clone * source."""
    clones = target // source
    tokens = np.arange(routes.shape[1], dtype=np.uint64)[None, :]
    slots = np.arange(routes.shape[0], dtype=np.uint64)[:, None]
    parents = routes.astype(np.uint64)
    salt = layer_salt(route_seed, layer_index)
    key = tokens ^ ((parents * np.uint64(0x85EBCA77)) & np.uint64(0xFFFFFFFFFFFFFFFF)) \
        ^ (slots * np.uint64(0xC2B2AE3D)) ^ np.uint64(salt)
    clone_ids = mix32(key).astype(np.int64) % clones
    return routes.astype(np.int64) + clone_ids * source


def hierarchical_hash_table(vocab_size: int, num_experts: int, top_k: int,
                            layer_index: int, route_seed: int = DEFAULT_ROUTE_SEED) -> np.ndarray:
    """routing.py:213-232."""
    parents = num_experts // 2
    base = balanced_hash_table(vocab_size, parents, top_k, layer_index, route_seed)
    return hierarchical_expand(base, parents, num_experts, layer_index, route_seed)


def route_table(strategy: str, vocab_size: int, num_experts: int, top_k: int,
                layer_index: int = 0, route_seed: int = DEFAULT_ROUTE_SEED,
                hash_count: int = 2) -> np.ndarray:
    """Dispatch on the strategy value strings of config.py:51-58."""
    if strategy == "token_id_multi_hash":
        return multi_hash_table(vocab_size, num_experts, top_k, layer_index, route_seed, hash_count)
    if strategy == "token_id_affine_hash":
        return affine_hash_table(vocab_size, num_experts, top_k, layer_index, route_seed)
    if strategy == "token_id_balanced_hash":
        return balanced_hash_table(vocab_size, num_experts, top_k, layer_index, route_seed)
    if strategy == "modulo_cyclic":
        return modulo_cyclic_table(vocab_size, num_experts, top_k, layer_index, route_seed)
    if strategy == "token_id_hierarchical_hash":
        return hierarchical_hash_table(vocab_size, num_experts, top_k, layer_index, route_seed)
    raise ValueError(strategy)


def pair_metadata(routes: np.ndarray, num_experts: int) -> Tuple[np.ndarray, np.ndarray]:
    """routing.py:262-311: uint8 code = lexicographic pair index | swap bit."""
    pairs = [(a, b) for a in range(num_experts) for b in range(a + 1, num_experts)]
    index = {p: i for i, p in enumerate(pairs)}
    swap_bit = 0x8 if len(pairs) <= 8 else 0x20
    codes = np.empty(routes.shape[1], dtype=np.uint8)
    for t in range(routes.shape[1]):
        p, s = int(routes[0, t]), int(routes[1, t])
        lo, hi = min(p, s), max(p, s)
        codes[t] = index[(lo, hi)] | (swap_bit if p == hi else 0)
    return codes, np.asarray(pairs, dtype=np.int32).reshape(-1, 2)


def gather_routes(table: np.ndarray, token_ids: np.ndarray) -> np.ndarray:
    """engine.py:316-318: clamp ids into [0, V-1] and gather ``[k, N]``."""
    ids = np.clip(np.asarray(token_ids, dtype=np.int64).reshape(-1), 0, table.shape[1] - 1)
    return table[:, ids]


def counting_partition(routes: np.ndarray, num_experts: int, order: int):
    """Expert-contiguous partition of the k*N assignments ``a = slot*N + t``.

    ORDER_TOKEN follows triton_token_routed.py:211-277 (segment order = token
    order); ORDER_ASSIGNMENT follows the stable sort of :2320-2351 (segment
    order = assignment index).  Returns (sorted int64[kN], inverse int64[kN],
    offsets int32[E+1], counts int32[E]) with inverse[sorted[r]] = r.
    """
    k, n = routes.shape
    experts = routes.reshape(-1).astype(np.int64)
    a = np.arange(k * n, dtype=np.int64)
    token = a % n if n else a
    if order == ORDER_TOKEN:
        key = experts * max(n, 1) + token
    elif order == ORDER_ASSIGNMENT:
        key = experts * max(k * n, 1) + a
    else:
        raise ValueError(order)
    sorted_idx = np.argsort(key, kind="stable").astype(np.int64)
    inverse = np.empty_like(sorted_idx)
    inverse[sorted_idx] = np.arange(k * n, dtype=np.int64)
    counts = np.bincount(experts, minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return sorted_idx, inverse, offsets, counts


def brute_force_partition(routes: np.ndarray, num_experts: int, order: int):
    """Pure-Python definition (small inputs): walk experts, emit matches in order."""
    k, n = routes.shape
    out = []
    for e in range(num_experts):
        if order == ORDER_TOKEN:
            for t in range(n):
                for s in range(k):
                    if int(routes[s, t]) == e:
                        out.append(s * n + t)
        else:
            for a in range(k * n):
                if int(routes[a // n, a % n]) == e:
                    out.append(a)
    return np.asarray(out, dtype=np.int64)


# ---------------------------------------------------------------------------
# floating point layer
# ---------------------------------------------------------------------------

def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    return F.silu(gate) * up


def reference_topk_swiglu(flat_x, routes, gate_w, up_w, down_w, route_weights):
    """engine.py:66-104: masked dense loop over experts, summed in expert order.

    ``routes`` [k, N] int64, ``route_weights`` [k] (per slot constants,
    engine.py:371) broadcast over tokens; computed in ``flat_x.dtype``.
    """
    rw = torch.as_tensor(route_weights, dtype=flat_x.dtype, device=flat_x.device).view(-1, 1).expand(routes.shape)
    out = torch.zeros_like(flat_x)
    for e in range(gate_w.shape[0]):
        tw = (routes.eq(e).to(flat_x.dtype) * rw).sum(dim=0)
        xa = flat_x * tw.ne(0).to(flat_x.dtype).unsqueeze(-1)
        inter = silu_mul(xa @ gate_w[e], xa @ up_w[e])
        out = out + (inter @ down_w[e]).to(out.dtype) * tw.unsqueeze(-1)
    return out


def shared_swiglu(flat_x, shared_gate_w, shared_up_w, shared_down_w):
    """engine.py:333-349 with nn.Linear weights ``[out, in]``."""
    if shared_gate_w is None or shared_gate_w.numel() == 0:
        return torch.zeros_like(flat_x)
    return F.linear(silu_mul(F.linear(flat_x, shared_gate_w), F.linear(flat_x, shared_up_w)),
                    shared_down_w)


def engine_forward(x, token_ids, table, params: dict, *, route_weights: Sequence[float],
                   shared_scale: float = 1.0, routed_scale: float = 1.0,
                   active_experts: Optional[int] = None, active_width: Optional[int] = None):
    """engine.py:534-579 (PYTORCH backend): a*shared + b*routed, shape of ``x``.

    ``params``: expert_gate/up [E,H,W], expert_down [E,W,H], shared_* [out,in]
    (absent or empty when shared_width == 0).  Active capacity slices a prefix
    (engine.py:320-331); ``table`` must already be the active table.
    """
    shape = x.shape
    flat_x = x.reshape(-1, shape[-1])
    ids = torch.as_tensor(token_ids).reshape(-1).clamp(0, table.shape[1] - 1)
    routes = torch.as_tensor(table)[:, ids]
    g, u, d = params["expert_gate"], params["expert_up"], params["expert_down"]
    if active_experts is not None or active_width is not None:
        ea = active_experts or g.shape[0]
        wa = active_width or g.shape[2]
        g, u, d = g[:ea, :, :wa], u[:ea, :, :wa], d[:ea, :wa, :]
    shared = shared_swiglu(flat_x, params.get("shared_gate"), params.get("shared_up"),
                           params.get("shared_down"))
    routed = reference_topk_swiglu(flat_x, routes, g, u, d, route_weights)
    return (shared_scale * shared + routed_scale * routed).view(shape)


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm.forward's formula (complexity/core/normalization/norms.py:53-55):
    x * rsqrt(mean(x^2) + eps) * weight, in x's dtype."""
    variance = x.pow(2).mean(-1, keepdim=True)
    return weight * (x * torch.rsqrt(variance + eps))


def engine_forward_norm_residual(x, token_ids, table, params: dict, norm_weight, eps: float, **kw):
    """The MLP half of a block with its post-attention RMSNorm
    (complexity/models/block.py:271-278): x + engine_forward(rms_norm(x))."""
    return x + engine_forward(rms_norm(x, norm_weight, eps), token_ids, table, params, **kw)


def engine_backward(x, token_ids, table, params: dict, dout, *, route_weights: Sequence[float],
                    shared_scale: float = 1.0, routed_scale: float = 1.0,
                    active_experts: Optional[int] = None, active_width: Optional[int] = None):
    """Gradients of ``engine_forward`` for an output gradient ``dout``:
    {"x", "shared_gate", "shared_up", "shared_down", "expert_gate",
    "expert_up", "expert_down"} (full parameter shapes; entries outside the
    active capacity are zero).  This is what the reference's PYTORCH backend
    returns through autograd, and what its Triton path's autograd Functions
    (triton_token_routed.py:1616-1833) compute for the routed branch.
    """
    leaves = {"x": x.detach().clone().requires_grad_(True)}
    for name, t in params.items():
        if t is not None and t.numel():
            leaves[name] = t.detach().clone().requires_grad_(True)
    p = {k: v for k, v in leaves.items() if k != "x"}
    out = engine_forward(leaves["x"], token_ids, table, p, route_weights=route_weights,
                         shared_scale=shared_scale, routed_scale=routed_scale,
                         active_experts=active_experts, active_width=active_width)
    names = list(leaves)
    grads = torch.autograd.grad(out, [leaves[n] for n in names], grad_outputs=dout.to(out.dtype),
                                allow_unused=True)
    return {n: (torch.zeros_like(leaves[n]) if g is None else g) for n, g in zip(names, grads)}


def swiglu_backward(x, dout, gate_w, up_w, down_w, mult=1.0):
    """Closed-form backward of y = (m * silu(x Wg^T) * (x Wu^T)) Wd^T per row.

    x, dout: [R, H]; gate_w, up_w: [F, H]; down_w: [H, F]; mult: scalar or
    [R, F] (the route weight of a routed row, the shared scale otherwise).
    Returns (dg, du, h): the gradients at the gate and up pre-activations and
    the forward's m * silu(g) * u, each [R, F]; silu'(g) = s + g s (1 - s)
    with s = sigmoid(g).
    """
    g = x @ gate_w.T
    u = x @ up_w.T
    dh = dout @ down_w
    s = torch.sigmoid(g)
    dm = dh * mult
    return dm * u * (s + g * s * (1 - s)), dm * g * s, mult * g * s * u


def naive_engine_output(x, token_ids, table, params: dict, *, route_weights,
                        shared_scale=1.0, routed_scale=1.0):
    """Token-by-token definition (tests/test_tr_hash_engine.py:183-206)."""
    B, T, H = x.shape
    out = torch.empty_like(x)
    for b in range(B):
        for t in range(T):
            xv = x[b, t]
            tid = min(max(int(token_ids[b, t]), 0), table.shape[1] - 1)
            if params.get("shared_gate") is None or params["shared_gate"].numel() == 0:
                shared = torch.zeros_like(xv)
            else:
                hs = F.silu(params["shared_gate"] @ xv) * (params["shared_up"] @ xv)
                shared = params["shared_down"] @ hs
            routed = torch.zeros_like(xv)
            for s in range(table.shape[0]):
                e = int(table[s, tid])
                inter = F.silu(xv @ params["expert_gate"][e]) * (xv @ params["expert_up"][e])
                routed = routed + route_weights[s] * (inter @ params["expert_down"][e])
            out[b, t] = shared_scale * shared + routed_scale * routed
    return out


def normwise_rel_err(actual: torch.Tensor, expected: torch.Tensor) -> float:
    """max|a - e| / max|e| in float64 (the parity metric of this build)."""
    a = actual.detach().to(torch.float64).cpu()
    e = expected.detach().to(torch.float64).cpu()
    denom = e.abs().max().item()
    return float((a - e).abs().max().item() / (denom if denom > 0 else 1.0))


# ---------------------------------------------------------------------------
# fp8 (OCP e4m3) per-output-channel quantisation used by the quantised path
# ---------------------------------------------------------------------------

E4M3_MAX = 448.0


def quantize_e4m3(weight: torch.Tensor, reduce_dim: int):
    """Per-output-channel scale = amax/448 over ``reduce_dim`` (the K axis).

    Returns (q float8_e4m3fn, scale float32 with ``reduce_dim`` removed).
    """
    w = weight.detach().to(torch.float32)
    amax = w.abs().amax(dim=reduce_dim, keepdim=True)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    q = (w / scale).clamp(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return q, scale.squeeze(reduce_dim)


def dequantize_e4m3(q: torch.Tensor, scale: torch.Tensor, reduce_dim: int) -> torch.Tensor:
    return q.to(torch.float32) * scale.unsqueeze(reduce_dim)


def block_exponents_e4m3(amax) -> np.ndarray:
    """Power-of-two block scale exponents for e4m3 codes (the block-scaled
    W8A8 h; no reference counterpart): the smallest integer e with
    amax <= 448 * 2^e, from frexp (amax = m * 2^k, m in [0.5, 1): e = k - 9,
    plus 1 when m > 0.875 = 448 / 2^9), clamped to [-126, 126]; 0 where amax
    is 0 or not finite."""
    a = np.asarray(amax, dtype=np.float32)
    m, k = np.frexp(a)
    e = k.astype(np.int64) - 9 + (m > np.float32(0.875))
    e = np.clip(e, -126, 126)
    return np.where((a > 0) & np.isfinite(a), e, 0)


def quantize_blocks_e4m3(h: torch.Tensor, block: int = 32):
    """h [n, f] (f a multiple of ``block``) as e4m3 codes with one exponent
    per row and block of ``block`` columns: (codes float8_e4m3fn [n, f],
    exponents int64 [n, f / block]); code = e4m3(clamp(h * 2^-e, +-448)),
    round to nearest even.  A block's maximum ignores NaN."""
    hf = h.detach().to(torch.float32)
    n, f = hf.shape
    hb = hf.reshape(n, f // block, block)
    amax = torch.nan_to_num(hb.abs(), nan=0.0).amax(dim=-1)
    e = torch.from_numpy(block_exponents_e4m3(amax.numpy()))
    scaled = hb * torch.exp2(-e.to(torch.float32)).unsqueeze(-1)
    q = torch.where(scaled > E4M3_MAX, E4M3_MAX, torch.where(scaled < -E4M3_MAX, -E4M3_MAX, scaled))
    return q.to(torch.float8_e4m3fn).reshape(n, f), e


def dequantize_blocks_e4m3(q: torch.Tensor, e: torch.Tensor, block: int = 32) -> torch.Tensor:
    n, f = q.shape
    qb = q.to(torch.float32).reshape(n, f // block, block)
    return (qb * torch.exp2(e.to(torch.float32)).unsqueeze(-1)).reshape(n, f)


def engine_forward_w8a8(x, token_ids, table, params: dict, *, h_blocks: bool = False, **kw):
    """engine_forward with the shared gate|up fed per-token e4m3 activations
    (the W8A8 path, which has no reference counterpart: the reference has no
    fp8): the shared branch sees dequantize(quantize_e4m3(x over each row)),
    the routed experts see x.  h_blocks: the down projection sees h through
    quantize_blocks_e4m3 (blocks of 32 features), else h itself."""
    shape = x.shape
    flat = x.reshape(-1, shape[-1]).to(torch.float32)
    q, s = quantize_e4m3(flat, 1)
    xq = dequantize_e4m3(q, s, 1).to(x.dtype)
    g = params.get("shared_gate")
    shared_params = {k: v for k, v in params.items() if not k.startswith("shared_")}
    routed = engine_forward(x, token_ids, table, shared_params, **kw)
    if g is None or g.numel() == 0:
        return routed
    h = silu_mul(F.linear(xq, g), F.linear(xq, params["shared_up"]))
    if h_blocks:
        hq, he = quantize_blocks_e4m3(h)
        h = dequantize_blocks_e4m3(hq, he).to(h.dtype)
    shared = F.linear(h, params["shared_down"]).view(shape)
    return routed + kw.get("shared_scale", 1.0) * shared


def e4m3_decode_table() -> np.ndarray:
    """All 256 OCP e4m3fn codes decoded from the format definition (NaN = 0x7F/0xFF)."""
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = math.nan
        elif exp == 0:
            out[code] = sign * man * 2.0 ** -9
        else:
            out[code] = sign * (1 + man / 8.0) * 2.0 ** (exp - 7)
    return out
