"""TRHashEngine on the HIP backend vs the CPU oracle of the universal dispatch.

Bounds (normwise max|got - ref| / max|ref|, the north-star metric): 1e-4 for
fp32, 2e-2 for bf16, 5e-2 for fp8 (against the oracle run on the engine's own
dequantised e4m3 weights).  The bf16 cases are compared with an fp32 oracle
fed the same bf16-rounded inputs and weights.
"""

import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = {"fp32": 1e-4, "bf16": 2e-2, "fp8": 5e-2}


def _oracle_params(engine, dequant_fp8=False):
    p = {}
    names = ["expert_gate", "expert_up", "expert_down"]
    for n in names:
        if dequant_fp8:
            p[n] = O.dequantize_e4m3(getattr(engine, n + "_fp8").cpu(), getattr(engine, n + "_scale").cpu(), 1)
        else:
            p[n] = getattr(engine, n).detach().float().cpu()
    if engine.shared_gate is not None:
        for n in ("shared_gate", "shared_up", "shared_down"):
            if dequant_fp8:
                p[n] = O.dequantize_e4m3(getattr(engine, n + "_fp8").cpu(), getattr(engine, n + "_scale").cpu(), 1)
            else:
                p[n] = getattr(engine, n).weight.detach().float().cpu()
    return p


def _oracle(engine, x, ids, rows=None, dequant_fp8=False, dtype=torch.float32):
    """The oracle on the engine's weights and x, computed in `dtype` (fp32: the
    bf16-rounded inputs widened; bf16: the reference formula in bf16)."""
    cfg = engine.config
    table = engine._active_route_table.cpu().numpy()
    p = {k: v.to(dtype) for k, v in _oracle_params(engine, dequant_fp8).items()}
    xr = x.cpu().to(dtype)
    idr = ids.cpu()
    if rows is not None:
        xr = xr.reshape(-1, xr.shape[-1])[rows].unsqueeze(0)
        idr = idr.reshape(-1)[rows].unsqueeze(0)
    return O.engine_forward(
        xr, idr, torch.from_numpy(table), p, route_weights=cfg.route_weights,
        shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale,
        active_experts=engine.active_num_experts, active_width=engine.active_expert_width)


def _run(engine, x, ids):
    from complexity_amd.tr_hash import TRHashBackend

    with torch.no_grad():
        out = engine(x, ids)
    torch.cuda.synchronize()
    assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
    return out


@pytest.mark.parametrize("E", [4, 8])
def test_reference_fused_shape_fp32(gpu, E):
    """The reference's own fused-vs-pytorch shape (test_tr_hash_engine.py:328-398)."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(29)
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=16, vocab_size=257, num_experts=E, top_k=2,
                                             shared_width=24, expert_width=8, precision="fp32",
                                             backend="hip")).to(gpu)
    ids = torch.randint(0, 257, (2, 11), device=gpu)
    x = torch.randn(2, 11, 16, device=gpu)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["fp32"]


def test_fp32_residual_with_bf16_expert_weights(gpu):
    """test_tr_hash_engine.py:401-433: x stays fp32, experts run in bf16."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(31)
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=16, vocab_size=257, num_experts=4, top_k=2,
                                             shared_width=0, expert_width=8, precision="bf16",
                                             backend="hip")).to(gpu).to(torch.bfloat16).eval()
    ids = torch.randint(0, 257, (1, 19), device=gpu)
    x = torch.randn(1, 19, 16, device=gpu)
    out = _run(engine, x, ids)
    assert out.dtype is torch.float32
    ref = _oracle(engine, x.to(torch.bfloat16), ids)
    assert O.normwise_rel_err(out, ref) <= BOUND["bf16"]


@pytest.mark.parametrize("E,k,weights,S,H,W", [
    (2, 1, None, 48, 64, 32),
    (8, 4, None, 40, 24, 12),
    (16, 4, (0.4, 0.2, 0.2, 0.2), 64, 128, 64),
    (4, 2, (0.7, 0.3), 0, 96, 64),
    (16, 2, None, 200, 136, 128),
])
@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
def test_engine_shapes(gpu, E, k, weights, S, H, W, dtype):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(E * 100 + k)
    cfg = TRHashEngineConfig(hidden_size=H, vocab_size=3001, num_experts=E, top_k=k, shared_width=S,
                             expert_width=W, routing_strategy="token_id_multi_hash",
                             route_weights=weights or (), routed_output_scale=2.0, shared_output_scale=0.5,
                             precision=dtype, backend="hip")
    engine = TRHashEngine(cfg).to(gpu)
    if dtype == "bf16":
        engine = engine.to(torch.bfloat16)
    ids = torch.randint(-5, 3010, (3, 171), device=gpu)
    x = torch.randn(3, 171, H, device=gpu)
    if dtype == "bf16":
        x = x.to(torch.bfloat16)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND[dtype]


def test_c1_fp32_full_size(gpu):
    from complexity_amd import workloads as Wl

    w = Wl.C1
    engine = Wl.build_engine(w, gpu, backend="hip")
    x, ids = Wl.make_hidden(w).to(gpu), Wl.make_token_ids(w).to(gpu)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["fp32"]


@pytest.mark.parametrize("name", ["c2_bf16_prefill_16384", "c3_bf16_decode_64"])
def test_bf16_layer_full_size(gpu, name):
    """Against the fp32 oracle fed the same bf16-rounded inputs (every row) and
    against the bf16 oracle, the reference formula computed in bf16 (every row
    at C3; a fixed 2048-row sample at C2, where every token's output depends
    only on its own row and id)."""
    from complexity_amd import workloads as Wl

    w = Wl.WORKLOADS[name]
    engine = Wl.build_engine(w, gpu, backend="hip")
    x, ids = Wl.make_hidden(w).to(gpu).to(torch.bfloat16), Wl.make_token_ids(w).to(gpu)
    out = _run(engine, x, ids)
    err32 = O.normwise_rel_err(out, _oracle(engine, x, ids))
    rows = None
    if w.tokens > 2048:
        rows = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(0))[:2048]
    ref16 = _oracle(engine, x, ids, rows=rows, dtype=torch.bfloat16)
    got = out.reshape(-1, w.hidden) if rows is None else out.reshape(-1, w.hidden)[rows.to(gpu)]
    err16 = O.normwise_rel_err(got, ref16.reshape(-1, w.hidden))
    print(f"\n{name}: normwise error vs fp32 oracle {err32:.3e}, vs bf16 oracle {err16:.3e}")
    assert err32 <= BOUND["bf16"]
    assert err16 <= BOUND["bf16"]


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("tokens", [512, 2048, 4096, 8192])
def test_bf16_layer_between_decode_and_c2(gpu, strategy, tokens):
    """C2's layer at token counts where the launch shapes change: 64-row
    tiles where larger ones leave CUs idle (512, 2048), the ping-pong gate|up
    from half a round of 256 x 256 tiles (2048: 192 tiles, 4096: 384), the
    256 x 256 down from 512 tiles (8192).  Every row against the fp32 oracle
    fed the same bf16 inputs."""
    from dataclasses import replace

    from complexity_amd import workloads as Wl

    w = replace(Wl.C2, name=f"bf16_{tokens}", batch=max(1, tokens // 2048), seq=min(tokens, 2048))
    assert w.tokens == tokens
    engine = Wl.build_engine(w, gpu, backend="hip")
    engine.routed_strategy = strategy
    x, ids = Wl.make_hidden(w).to(gpu).to(torch.bfloat16), Wl.make_token_ids(w).to(gpu)
    out = _run(engine, x, ids)
    assert engine._packed.strategy == strategy
    err = O.normwise_rel_err(out, _oracle(engine, x, ids))
    print(f"\nbf16 {tokens} tokens {strategy}: normwise error vs fp32 oracle {err:.3e}")
    assert err <= BOUND["bf16"]


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("tokens", [512, 8192])
def test_fp32_layer_between_decode_and_c2(gpu, strategy, tokens):
    """C1's fp32 layer at 512 tokens (64 x 64 down and 64 x 128 gate|up
    tiles) and 8192 (the large fp32 tiles), every row against the oracle."""
    from dataclasses import replace

    from complexity_amd import workloads as Wl

    w = replace(Wl.C1, name=f"fp32_{tokens}", batch=max(1, tokens // 2048), seq=min(tokens, 2048))
    assert w.tokens == tokens
    engine = Wl.build_engine(w, gpu, backend="hip")
    engine.routed_strategy = strategy
    x, ids = Wl.make_hidden(w).to(gpu), Wl.make_token_ids(w).to(gpu)
    out = _run(engine, x, ids)
    assert engine._packed.strategy == strategy
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["fp32"]


@pytest.mark.parametrize("layer", [0, 7, 15])
def test_c4_decode_layers(gpu, layer):
    """C4's MLP in greedy decode: 8 tokens, the route table of layer `layer`
    of the 16-layer model (routing.py:114 layer salt)."""
    from complexity_amd import workloads as Wl

    w = Wl.C4_DECODE
    engine = Wl.build_engine(w, gpu, backend="hip", seed=layer, layer_index=layer)
    x, ids = Wl.make_hidden(w, seed=layer).to(gpu).to(torch.bfloat16), Wl.make_token_ids(w, seed=layer).to(gpu)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["bf16"]


@pytest.mark.parametrize("name", ["c5_fp8_32768", "c5_fp8_32768_active_8x128"])
def test_fp8_layer_full_size(gpu, name):
    """Whole layer at N=32768; the oracle checks a fixed sample of 1024 rows
    (every token's output depends only on its own row and id)."""
    from complexity_amd import workloads as Wl

    w = Wl.WORKLOADS[name]
    engine = Wl.build_engine(w, gpu, backend="hip")
    x, ids = Wl.make_hidden(w).to(gpu).to(torch.bfloat16), Wl.make_token_ids(w).to(gpu)
    out = _run(engine, x, ids)
    rows = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(0))[:1024]
    ref = _oracle(engine, x, ids, rows=rows, dequant_fp8=True)
    got = out.reshape(-1, w.hidden)[rows.to(gpu)]
    assert O.normwise_rel_err(got, ref.reshape(-1, w.hidden)) <= BOUND["fp8"]


def test_fp8_quantisation_matches_oracle(gpu):
    from complexity_amd import workloads as Wl

    w = Wl.C5
    engine = Wl.build_engine(w, gpu, backend="hip")
    for n in ("expert_gate", "expert_down", "shared_up", "shared_down"):
        master = getattr(engine, n) if n.startswith("expert") else getattr(engine, n).weight
        q, s = O.quantize_e4m3(master.detach().float().cpu(), 1)
        assert torch.equal(getattr(engine, n + "_fp8").cpu().view(torch.uint8), q.view(torch.uint8)), n
        assert torch.equal(getattr(engine, n + "_scale").cpu(), s), n


def test_active_capacity_on_hip_matches_oracle_and_restores(gpu):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(5)
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=64, vocab_size=997, num_experts=8, top_k=2,
                                             shared_width=96, expert_width=48,
                                             routing_strategy="token_id_balanced_hash", precision="fp32",
                                             backend="hip")).to(gpu)
    ids = torch.randint(0, 997, (2, 50), device=gpu)
    x = torch.randn(2, 50, 64, device=gpu)
    full = _run(engine, x, ids)
    engine.set_active_capacity(num_experts=4, expert_width=20)
    reduced = _run(engine, x, ids)
    assert O.normwise_rel_err(reduced, _oracle(engine, x, ids)) <= BOUND["fp32"]
    assert not torch.allclose(full, reduced)
    engine.set_active_capacity(num_experts=8, expert_width=48)
    assert torch.equal(_run(engine, x, ids), full)


def test_partition_orders_give_identical_outputs(gpu):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(9)
    common = dict(hidden_size=64, vocab_size=997, num_experts=4, top_k=2, shared_width=64, expert_width=64,
                  precision="fp32")
    a = TRHashEngine(TRHashEngineConfig(**common, backend="hip")).to(gpu)
    b = TRHashEngine(TRHashEngineConfig(**common, backend="cggr")).to(gpu)
    b.load_state_dict(a.state_dict())
    ids = torch.randint(0, 997, (4, 33), device=gpu)
    x = torch.randn(4, 33, 64, device=gpu)
    with torch.no_grad():
        ya, yb = a(x, ids), b(x, ids)
    assert a.last_backend.partition == "token" and b.last_backend.partition == "assignment"
    assert torch.equal(ya, yb)


def test_residual_fused_into_down_epilogue(gpu):
    from complexity_amd import workloads as Wl

    w = Wl.C3
    engine = Wl.build_engine(w, gpu, backend="hip")
    x, ids = Wl.make_hidden(w).to(gpu).to(torch.bfloat16), Wl.make_token_ids(w).to(gpu)
    res = torch.randn_like(x)
    with torch.no_grad():
        fused = engine.forward_with_residual(x, ids, res)
        plain = engine(x, ids)
    assert O.normwise_rel_err(fused, (plain.float() + res.float())) <= 1e-2


def test_empty_batch(gpu):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    engine = TRHashEngine(TRHashEngineConfig(hidden_size=16, vocab_size=97, precision="fp32",
                                             backend="hip")).to(gpu)
    with torch.no_grad():
        out = engine(torch.zeros(0, 5, 16, device=gpu), torch.zeros(0, 5, dtype=torch.long, device=gpu))
    assert out.shape == (0, 5, 16)


def test_graph_backend_replays_hip_kernels(gpu):
    """Captured HIP path: several replays with eager work between them, each
    checked against the eager result (no memset nodes are recorded)."""
    from complexity_amd.tr_hash import GraphBucket, TRHashEngine, TRHashEngineConfig

    torch.manual_seed(11)
    common = dict(hidden_size=128, vocab_size=997, num_experts=4, top_k=2, shared_width=256, expert_width=64,
                  precision="bf16", phase="inference")
    graph = TRHashEngine(TRHashEngineConfig(**common, backend="cuda_graph",
                                            graph_buckets=(GraphBucket(4, 16),))).to(gpu).to(torch.bfloat16).eval()
    eager = TRHashEngine(TRHashEngineConfig(**common, backend="hip")).to(gpu).to(torch.bfloat16).eval()
    eager.load_state_dict(graph.state_dict())
    with torch.no_grad():
        for step in range(4):
            ids = torch.randint(0, 997, (3, 10), device=gpu)
            x = torch.randn(3, 10, 128, device=gpu, dtype=torch.bfloat16)
            got = graph(x, ids)
            _ = torch.randn(1000, device=gpu).sum()  # unrelated eager work
            torch.cuda.synchronize()
            assert torch.equal(got, eager(x, ids)), step


@pytest.mark.parametrize("tokens", [(4, 16), (64, 1)])
def test_graph_replay_follows_weight_changes(gpu, tokens):
    """A captured graph reads the packed weights it captured.  After
    load_state_dict (new weights), an in-place update, a routing-strategy
    change or quantize_fp8_(), replays must give the eager result of the new
    weights (the runner re-captures), and the old pack must not be read after
    it was freed.  (64, 1) takes the decode kernels and their split-K
    scratch, which each captured graph owns."""
    from complexity_amd.tr_hash import GraphBucket, TRHashEngine, TRHashEngineConfig

    torch.manual_seed(13)
    b, t = tokens
    common = dict(hidden_size=128, vocab_size=997, num_experts=4, top_k=2, shared_width=256, expert_width=64,
                  precision="bf16", phase="inference")
    graph = TRHashEngine(TRHashEngineConfig(**common, backend="cuda_graph",
                                            graph_buckets=(GraphBucket(b, t),))).to(gpu).to(torch.bfloat16).eval()
    eager = TRHashEngine(TRHashEngineConfig(**common, backend="hip")).to(gpu).to(torch.bfloat16).eval()
    ids = torch.randint(0, 997, (b, t), device=gpu)
    x = torch.randn(b, t, 128, device=gpu, dtype=torch.bfloat16)

    def check(tag):
        with torch.no_grad():
            got = graph(x, ids)
            torch.cuda.empty_cache()   # freed packs would now be reused or unmapped
            _ = torch.randn(1 << 20, device=gpu).sum()
            torch.cuda.synchronize()
            want = eager(x, ids)
        assert torch.equal(got, want), tag

    eager.load_state_dict(graph.state_dict())
    check("initial")
    other = TRHashEngine(TRHashEngineConfig(**common, backend="hip", route_seed=7)).to(gpu).to(torch.bfloat16)
    sd = {k: v for k, v in other.state_dict().items() if "route" not in k and "fused" not in k}
    graph.load_state_dict(sd, strict=False)
    eager.load_state_dict(sd, strict=False)
    check("load_state_dict")
    with torch.no_grad():
        graph.expert_down.mul_(1.5)
        eager.expert_down.mul_(1.5)
    check("in-place update")
    graph.routed_strategy = eager.routed_strategy = "grouped"
    check("strategy")
    graph.quantize_fp8_()
    eager.quantize_fp8_()
    check("quantize_fp8_")


def test_quantized_bf16_engine_under_autograd_takes_the_universal_path(gpu):
    """quantize_fp8_() on a bf16-config engine: differentiable calls resolve
    to PYTORCH (the e4m3 packs have no backward) and match the oracle on the
    dequantised weights; no-grad calls stay on HIP."""
    from complexity_amd.tr_hash import TRHashBackend, TRHashEngine, TRHashEngineConfig

    torch.manual_seed(17)
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=128, vocab_size=997, num_experts=4, top_k=2,
                                             shared_width=256, expert_width=64, precision="bf16",
                                             routing_strategy="token_id_multi_hash")).to(gpu).to(torch.bfloat16)
    engine.quantize_fp8_()
    ids = torch.randint(0, 997, (2, 200), device=gpu)
    x = torch.randn(2, 200, 128, device=gpu, dtype=torch.bfloat16, requires_grad=True)
    out = engine(x, ids)
    assert engine.last_backend.selected is TRHashBackend.PYTORCH
    assert any("e4m3" in r for r in engine.last_backend.reasons)
    out.float().square().sum().backward()
    torch.cuda.synchronize()
    assert x.grad is not None and torch.isfinite(x.grad.float()).all()
    ref = _oracle(engine, x.detach(), ids, dequant_fp8=True)
    assert O.normwise_rel_err(out.detach(), ref) <= BOUND["fp8"]
    with torch.no_grad():
        hip = engine(x.detach(), ids)
    assert engine.last_backend.selected is TRHashBackend.HIP
    assert O.normwise_rel_err(hip, ref) <= BOUND["fp8"]


@pytest.mark.parametrize("strategy", ["grouped", "dense"])
@pytest.mark.parametrize("E,k,weights", [(16, 2, (0.7, 0.3)), (8, 4, (0.4, 0.3, 0.2, 0.1))])
def test_repeated_experts_per_token_match_oracle(gpu, strategy, E, k, weights):
    """A loaded table whose slots name one expert twice for some ids (the
    reference accepts such tables where it compiles no top-2 pair metadata:
    more than 8 experts or top_k != 2): the reference sums both slots'
    weights (engine.py:94); the grouped path gives each slot its own
    partition row and sums them in the un-permute."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(19)
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=128, vocab_size=997, num_experts=E, top_k=k,
                                             shared_width=256, expert_width=64, precision="fp32",
                                             route_weights=weights, routed_output_scale=2.0,
                                             routing_strategy="token_id_multi_hash")).to(gpu)
    table = engine.route_table.clone()
    table[1, :300] = table[0, :300]
    engine.load_route_table(table)
    engine.routed_strategy = strategy
    ids = torch.randint(0, 997, (3, 400), device=gpu)
    ids[0, :300] = torch.arange(300, device=gpu)
    x = torch.randn(3, 400, 128, device=gpu)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["fp32"]


def test_fp32_layer_at_prefill_size(gpu):
    """C1's fp32 layer at C2's 16384 tokens: the large-tile fp32 kernels."""
    from dataclasses import replace

    from complexity_amd import workloads as Wl

    w = replace(Wl.C1, name="fp32_16384", batch=8, seq=2048, ids="zipf")
    engine = Wl.build_engine(w, gpu, backend="hip")
    x, ids = Wl.make_hidden(w).to(gpu), Wl.make_token_ids(w).to(gpu)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["fp32"]


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("E,k,S,W,dtype,weights", [
    (4, 2, 3072, 64, "bf16", None),
    (4, 2, 256, 64, "fp32", (0.7, 0.3)),
    (8, 4, 96, 12, "fp32", None),
    (2, 1, 0, 40, "bf16", None),
    (16, 2, 512, 32, "bf16", None),
])
def test_routed_strategies_agree_with_oracle(gpu, strategy, E, k, S, W, dtype, weights):
    """Both HIP strategies (dense-routed and grouped) on the same engine."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(E + k + S + W)
    H = 128
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=H, vocab_size=5000, num_experts=E, top_k=k,
                                             shared_width=S, expert_width=W, routing_strategy="token_id_multi_hash",
                                             route_weights=weights or (), routed_output_scale=2.0,
                                             shared_output_scale=0.5, precision=dtype, backend="hip")).to(gpu)
    if dtype == "bf16":
        engine = engine.to(torch.bfloat16)
    engine.routed_strategy = strategy
    ids = torch.randint(0, 5000, (2, 300), device=gpu)
    x = torch.randn(2, 300, H, device=gpu, dtype=torch.bfloat16 if dtype == "bf16" else torch.float32)
    out = _run(engine, x, ids)
    assert engine._packed.strategy == strategy
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND[dtype]
    engine.set_active_capacity(num_experts=max(k, E // 2), expert_width=max(1, W // 2))
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND[dtype]


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("n", [7, 300])
def test_out_of_range_token_ids_are_clamped(gpu, strategy, n):
    """engine.py:316-318 clamps ids into [0, V-1] before the gather; the
    dense-routed kernels (tile and decode shapes) gather routes themselves."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    torch.manual_seed(n)
    engine = TRHashEngine(TRHashEngineConfig(hidden_size=128, vocab_size=1000, num_experts=4, top_k=2,
                                             shared_width=256, expert_width=64, precision="bf16",
                                             backend="hip")).to(gpu).to(torch.bfloat16)
    engine.routed_strategy = strategy
    ids = torch.randint(-50, 1050, (1, n), device=gpu)
    x = torch.randn(1, n, 128, device=gpu, dtype=torch.bfloat16)
    out = _run(engine, x, ids)
    assert O.normwise_rel_err(out, _oracle(engine, x, ids)) <= BOUND["bf16"]
    clamped = _run(engine, x, ids.clamp(0, 999))
    assert torch.equal(out, clamped)


def test_fp8_state_dict_loads_into_the_hip_path(gpu):
    """F3 on the HIP backend: an fp8 engine's state dict (e4m3 codes, scales,
    route table) loaded into an engine of another seed and route seed repacks
    the kernel weights and reproduces the outputs bit for bit; the result
    matches the oracle on the dequantised weights."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    common = dict(hidden_size=256, vocab_size=1000, num_experts=4, top_k=2, shared_width=512, expert_width=64,
                  precision="fp8", backend="hip")
    torch.manual_seed(21)
    a = TRHashEngine(TRHashEngineConfig(**common)).to(gpu).eval()
    torch.manual_seed(22)
    b = TRHashEngine(TRHashEngineConfig(**common, route_seed=0x13579BD)).to(gpu).eval()
    ids = torch.randint(0, 1000, (2, 40), device=gpu)
    x = torch.randn(2, 40, 256, device=gpu).to(torch.bfloat16)
    _run(b, x, ids)   # b's own packs exist before the load
    b.load_state_dict(a.state_dict())
    ya, yb = _run(a, x, ids), _run(b, x, ids)
    assert torch.equal(ya, yb)
    assert O.normwise_rel_err(ya, _oracle(a, x, ids, dequant_fp8=True)) <= BOUND["fp8"]


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("experts,top_k", [(8, 4), (16, 4), (16, 2), (2, 1)])
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_expert_topk_matrix_against_oracle(gpu, strategy, experts, top_k, precision):
    """The FUSED/CGGR-vs-PYTORCH checks of test_tr_hash_engine.py:328-398 and
    test_tr_hash_fused_kernel_parity.py:148-201, widened to the supported
    (E, k) matrix and both routed strategies; shape (2, 11, 16) at V = 257 as
    there, plus a 300-token batch (tile kernels) with ragged widths."""
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    print(f"matrix {strategy} E={experts} k={top_k} {precision}", flush=True)
    dt = torch.float32 if precision == "fp32" else torch.bfloat16
    for (b, t, hidden, shared, width) in ((2, 11, 16, 24, 8), (3, 100, 72, 200, 40)):
        torch.manual_seed(experts * 10 + top_k + hidden)
        eng = TRHashEngine(TRHashEngineConfig(hidden_size=hidden, vocab_size=257, num_experts=experts, top_k=top_k,
                                              shared_width=shared, expert_width=width, precision=precision,
                                              backend="hip")).to(gpu)
        with torch.no_grad():
            for p in eng.parameters():
                p.normal_(0.0, 0.2)
        eng = eng.to(dt).eval()
        eng.routed_strategy = strategy
        x = torch.randn(b, t, hidden, device=gpu).to(dt)
        ids = torch.randint(0, 257, (b, t), device=gpu)
        out = _run(eng, x, ids)
        assert O.normwise_rel_err(out, _oracle(eng, x, ids)) <= BOUND[precision]
