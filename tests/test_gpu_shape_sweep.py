"""Seeded sweep of irregular layer shapes: TRHashEngine on the HIP backend vs
the CPU oracle of the universal dispatch (engine.py:66-104, 534-579).

Each case draws, from its own seed, a hidden size (not always a multiple of
64 or of 16 bytes), a shared width (0 = no shared branch), the expert count,
top-k, expert width, token count (both sides of the 128-token decode
kernels), precision, routing strategy, route weights, output scales and the
HIP strategy (dense-routed or grouped).  The bounds are the north-star ones:
normwise max relative error 1e-4 for fp32 and 2e-2 for bf16 (the bf16 cases
against an fp32 oracle fed the same bf16-rounded inputs and weights).
"""

import random

import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = {"fp32": 1e-4, "bf16": 2e-2}
CASES = 32


def _draw(case: int) -> dict:
    r = random.Random(0x5EED + case)
    E = r.choice([1, 2, 4, 8, 16])
    k = r.choice([t for t in (1, 2, 4) if t <= E])
    raw = [r.uniform(0.2, 1.0) for _ in range(k)]
    weights = tuple(v / sum(raw) for v in raw) if r.random() < 0.5 else ()
    n = r.choice([1, 2, 7, 8, 16, 17, 63, 64, 65, 128, 129, 300, 777])
    b = r.choice([d for d in (1, 2, 3) if n % d == 0])
    return dict(
        hidden=r.choice([8, 16, 20, 24, 40, 72, 100, 136, 264, 520]),
        shared=r.choice([0, 8, 24, 40, 100, 200, 520, 1000]),
        E=E, k=k, weights=weights,
        W=r.choice([1, 3, 8, 12, 24, 64, 100]),
        batch=b, seq=n // b,
        vocab=r.choice([257, 1000, 5000]),
        # hierarchical routing needs an even expert count >= 4 and k <= E / 2
        routing=r.choice(["modulo_cyclic", "token_id_balanced_hash", "token_id_multi_hash"]
                         + (["token_id_hierarchical_hash"] if E >= 4 and E % 2 == 0 and k <= E // 2 else [])),
        dtype=r.choice(["fp32", "bf16"]),
        strategy=r.choice(["dense", "grouped"]),
        shared_scale=r.choice([1.0, 0.5, 1.25]),
        routed_scale=r.choice([1.0, 2.0]),
        seed=r.randrange(1 << 30),
    )


def _oracle(engine, x, ids):
    cfg = engine.config
    p = {n: getattr(engine, n).detach().float().cpu() for n in ("expert_gate", "expert_up", "expert_down")}
    if engine.shared_gate is not None:
        for n in ("shared_gate", "shared_up", "shared_down"):
            p[n] = getattr(engine, n).weight.detach().float().cpu()
    return O.engine_forward(
        x.float().cpu(), ids.cpu(), engine._active_route_table.cpu(), p, route_weights=cfg.route_weights,
        shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale,
        active_experts=engine.active_num_experts, active_width=engine.active_expert_width)


@pytest.mark.parametrize("case", range(CASES))
def test_irregular_shapes_match_oracle(gpu, case):
    from complexity_amd.tr_hash import TRHashBackend, TRHashEngine, TRHashEngineConfig

    c = _draw(case)
    print(f"case {case}: {c}", flush=True)
    torch.manual_seed(c["seed"])
    engine = TRHashEngine(TRHashEngineConfig(
        hidden_size=c["hidden"], vocab_size=c["vocab"], num_experts=c["E"], top_k=c["k"],
        shared_width=c["shared"], expert_width=c["W"], routing_strategy=c["routing"],
        route_weights=c["weights"], shared_output_scale=c["shared_scale"],
        routed_output_scale=c["routed_scale"], precision=c["dtype"], backend="hip")).to(gpu)
    act = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    engine = engine.to(act)
    engine.routed_strategy = c["strategy"]
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), device=gpu)
    x = torch.randn(c["batch"], c["seq"], c["hidden"], device=gpu, dtype=act)
    with torch.no_grad():
        out = engine(x, ids)
    torch.cuda.synchronize()
    assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
    assert out.shape == x.shape and out.dtype == act
    err = O.normwise_rel_err(out, _oracle(engine, x, ids))
    assert err <= BOUND[c["dtype"]], (c, err)


BWD_CASES = 16


@pytest.mark.parametrize("case", range(BWD_CASES))
def test_irregular_shapes_backward_match_oracle(gpu, case):
    """The differentiable HIP call on the same kind of draws (hidden rounded up
    to a multiple of 8, the HIP backward's requirement): the gradients of x
    and of every parameter against autograd of the oracle's forward in f64."""
    from complexity_amd.tr_hash import TRHashBackend, TRHashEngine, TRHashEngineConfig

    c = _draw(1000 + case)
    c["hidden"] += -c["hidden"] % 8
    print(f"backward case {case}: {c}", flush=True)
    torch.manual_seed(c["seed"])
    engine = TRHashEngine(TRHashEngineConfig(
        hidden_size=c["hidden"], vocab_size=c["vocab"], num_experts=c["E"], top_k=c["k"],
        shared_width=c["shared"], expert_width=c["W"], routing_strategy=c["routing"],
        route_weights=c["weights"], shared_output_scale=c["shared_scale"],
        routed_output_scale=c["routed_scale"], precision=c["dtype"], backend="hip")).to(gpu)
    act = torch.bfloat16 if c["dtype"] == "bf16" else torch.float32
    engine = engine.to(act)
    engine.routed_strategy = c["strategy"]
    ids = torch.randint(0, c["vocab"], (c["batch"], c["seq"]), device=gpu)
    x = torch.randn(c["batch"], c["seq"], c["hidden"], device=gpu, dtype=act).requires_grad_(True)
    dout = torch.randn(c["batch"], c["seq"], c["hidden"], device=gpu, dtype=act)
    out = engine(x, ids)
    assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
    out.backward(dout)
    torch.cuda.synchronize()
    got = {"x": x.grad}
    names = ["expert_gate", "expert_up", "expert_down"]
    params = {n: getattr(engine, n) for n in names}
    if engine.shared_gate is not None:
        for n in ("shared_gate", "shared_up", "shared_down"):
            params[n] = getattr(engine, n).weight
    got.update({n: p.grad for n, p in params.items()})
    cfg = engine.config
    ref = O.engine_backward(
        x.detach().cpu().double(), ids.cpu(), engine._active_route_table.cpu(),
        {n: p.detach().cpu().double() for n, p in params.items()}, dout.cpu().double(),
        route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale,
        routed_scale=cfg.routed_output_scale, active_experts=engine.active_num_experts,
        active_width=engine.active_expert_width)
    for name, r in ref.items():
        g = got[name]
        assert g is not None and g.shape == r.shape, (name, c)
        err = O.normwise_rel_err(g, r)
        assert err <= BOUND[c["dtype"]], (name, c, err)
