"""CPU tests of the host package: the mirror of the reference's TR-Hash API.

They follow the behaviours the reference's own tests pin
(tests/test_tr_hash_engine.py, tests/test_tr_hash_dynamic_moe.py,
tests/test_tr_hash_fused_kernel_parity.py) on the product modules, with the
routing checked against the golden vectors written from the reference, and
the PYTORCH (universal) backend checked against the CPU oracle.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from complexity_amd.core.mlp import MLPConfig, TRHashEngineMLP
from complexity_amd.core.registry import MLP_REGISTRY
from complexity_amd.tr_hash import (
    GraphBucket,
    TRHashBackend,
    TRHashEngine,
    TRHashEngineConfig,
    TRHashPhase,
    TRHashPrecision,
    TRHashStrategy,
)
from complexity_amd.tr_hash.buckets import GraphBucketPlanner
from complexity_amd.tr_hash.capabilities import select_backend, supports_fused_cuda, supports_hip_backward
from complexity_amd.tr_hash.routing import (
    build_route_table,
    compile_top2_pair_metadata,
    decode_top2_pair_metadata,
    mix32,
)
from oracle import trmoe_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"


def _digest(table) -> str:
    return hashlib.sha256(np.ascontiguousarray(np.asarray(table), dtype=np.int64).tobytes()).hexdigest()


def _config(**kw) -> TRHashEngineConfig:
    base = dict(hidden_size=32, vocab_size=257, num_experts=4, top_k=2, shared_width=48, expert_width=16,
                routing_strategy=TRHashStrategy.MULTI_HASH)
    base.update(kw)
    return TRHashEngineConfig(**base)


# --------------------------------------------------------------------------- config


@pytest.mark.parametrize("num_experts", [1, 2, 3, 4, 5, 8, 16, 32])
@pytest.mark.parametrize("top_k", [1, 2, 3, 4])
def test_supported_expert_and_topk_matrix(num_experts, top_k):
    ok = num_experts in (1, 2, 4, 8, 16) and top_k in (1, 2, 4) and top_k <= num_experts
    if ok:
        cfg = _config(num_experts=num_experts, top_k=top_k)
        assert len(cfg.route_weights) == top_k
        assert abs(sum(cfg.route_weights) - 1.0) < 1e-6
    else:
        with pytest.raises(ValueError):
            _config(num_experts=num_experts, top_k=top_k)


@pytest.mark.parametrize("kw", [dict(route_hash_count=1), dict(route_hash_count=9), dict(route_weights=(0.7, 0.7)),
                                dict(route_weights=(1.5, -0.5)), dict(route_weights=(1.0,)),
                                dict(shared_width=-1), dict(expert_width=0)])
def test_config_rejects_invalid_values(kw):
    with pytest.raises(ValueError):
        _config(**kw)


def test_cuda_graph_config_is_inference_only_and_requires_buckets():
    with pytest.raises(ValueError):
        _config(backend=TRHashBackend.CUDA_GRAPH, phase=TRHashPhase.INFERENCE)
    with pytest.raises(ValueError):
        _config(backend=TRHashBackend.CUDA_GRAPH, graph_buckets=(GraphBucket(1, 8),))
    cfg = _config(backend=TRHashBackend.CUDA_GRAPH, phase=TRHashPhase.INFERENCE,
                  graph_buckets=(GraphBucket(4, 64), GraphBucket(1, 8)))
    assert [b.token_capacity for b in cfg.graph_buckets] == [8, 256]


def test_cuda_graph_bucket_selection_is_smallest_containing_shape():
    planner = GraphBucketPlanner([GraphBucket(8, 128), GraphBucket(1, 64), GraphBucket(2, 32), GraphBucket(4, 16)])
    # (1, 64) and (4, 16) hold 64 tokens each: ties go to the smaller batch
    assert planner.select(1, 16) == GraphBucket(1, 64)
    assert planner.select(3, 16) == GraphBucket(4, 16)
    assert planner.select(2, 20) == GraphBucket(2, 32)
    assert planner.select(1, 40) == GraphBucket(1, 64)
    assert planner.select(3, 100) == GraphBucket(8, 128)
    with pytest.raises(ValueError):
        planner.select(9, 1)
    with pytest.raises(ValueError):
        planner.select(0, 1)


# --------------------------------------------------------------------------- routing


def test_mix32_matches_oracle_on_edge_values():
    vals = np.array([0, 1, 2, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF, 0x9E3779B1, 12345678], dtype=np.uint64)
    got = mix32(torch.from_numpy(vals.astype(np.int64))).numpy().astype(np.uint64)
    assert np.array_equal(got, O.mix32(vals))


def test_product_route_tables_match_every_reference_digest():
    data = json.loads((GOLDEN / "route_digests.json").read_text())
    assert data["route_seed"] == 0x71D5A17
    for case in data["cases"]:
        cfg = TRHashEngineConfig(hidden_size=8, vocab_size=case["vocab_size"], num_experts=case["num_experts"],
                                 top_k=case["top_k"], shared_width=8, expert_width=8,
                                 routing_strategy=TRHashStrategy(case["strategy"]),
                                 layer_index=case["layer_index"], route_hash_count=case["hash_count"])
        table = build_route_table(cfg)
        assert table.dtype == torch.int64 and tuple(table.shape) == (case["top_k"], case["vocab_size"])
        assert table[:, :32].tolist() == case["head"], case
        assert _digest(table.numpy()) == case["sha256"], case


@pytest.mark.parametrize("experts", [4, 8, 16])
def test_product_full_table_matches_reference_vectors(experts):
    golden = np.load(GOLDEN / "route_tables_v32000.npz")[f"multi_e{experts}_l0"].astype(np.int64)
    cfg = TRHashEngineConfig(hidden_size=8, vocab_size=32000, num_experts=experts, top_k=2, shared_width=8,
                             expert_width=8, routing_strategy=TRHashStrategy.MULTI_HASH)
    assert np.array_equal(build_route_table(cfg).numpy(), golden)


def test_route_tables_are_deterministic_distinct_and_use_every_expert():
    for strategy in TRHashStrategy:
        for experts, k in ((4, 2), (8, 4), (16, 2)):
            cfg = _config(vocab_size=4096, num_experts=experts, top_k=k, routing_strategy=strategy)
            a, b = build_route_table(cfg), build_route_table(cfg)
            assert torch.equal(a, b)
            assert int(a.min()) >= 0 and int(a.max()) < experts
            srt = a.sort(dim=0).values
            assert bool((srt[1:] != srt[:-1]).all()), strategy
            assert set(a[0].tolist()) == set(range(experts)), strategy


def test_multi_hash_routes_depend_on_every_hash_channel_and_layer():
    base = build_route_table(_config(vocab_size=4096, route_hash_count=2))
    assert not torch.equal(base, build_route_table(_config(vocab_size=4096, route_hash_count=3)))
    assert not torch.equal(base, build_route_table(_config(vocab_size=4096, layer_index=1)))
    assert not torch.equal(base, build_route_table(_config(vocab_size=4096, route_seed=7)))


@pytest.mark.parametrize("strategy", ["modulo_cyclic", "token_id_balanced_hash", "token_id_affine_hash",
                                      "token_id_multi_hash"])
@pytest.mark.parametrize("experts", [2, 4, 8])
def test_compact_top2_pair_metadata_matches_reference_and_round_trips(strategy, experts):
    gold = np.load(GOLDEN / "pair_codes_v997.npz")
    routes = torch.from_numpy(gold[f"{strategy}_e{experts}_routes"].astype(np.int64))
    codes, pairs = compile_top2_pair_metadata(routes, num_experts=experts)
    assert np.array_equal(codes.numpy(), gold[f"{strategy}_e{experts}_codes"])
    assert np.array_equal(pairs.numpy(), gold[f"{strategy}_e{experts}_pairs"])
    assert torch.equal(decode_top2_pair_metadata(codes, pairs), routes)


def test_compact_pair_metadata_rejects_unsupported_shape():
    with pytest.raises(ValueError):
        compile_top2_pair_metadata(torch.zeros(3, 10, dtype=torch.long), num_experts=4)
    with pytest.raises(ValueError):
        compile_top2_pair_metadata(torch.zeros(2, 10, dtype=torch.long), num_experts=16)


# --------------------------------------------------------------------------- backend policy


def test_auto_backend_on_cpu_is_pytorch_with_reason():
    d = select_backend(_config(), device_type="cpu")
    assert d.requested is TRHashBackend.AUTO and d.selected is TRHashBackend.PYTORCH
    assert d.reasons


def test_auto_backend_on_gpu_selects_hip_also_under_autograd():
    cfg = _config()
    d = select_backend(cfg, device_type="cuda", hip_available=True, cggr_available=False, fused_cuda_available=False)
    assert d.selected is TRHashBackend.HIP
    # the HIP backend has a backward for bf16/f32 weights and hidden % 8 == 0
    d = select_backend(cfg, device_type="cuda", hip_available=True, cggr_available=False,
                       fused_cuda_available=False, autograd=True)
    assert d.selected is TRHashBackend.HIP and not d.reasons
    assert supports_hip_backward(cfg)
    # otherwise differentiable calls resolve to PYTORCH with the reason
    for cfg in (_config(hidden_size=36), _config(precision=TRHashPrecision.FP8)):
        assert not supports_hip_backward(cfg)
        d = select_backend(cfg, device_type="cuda", hip_available=True, cggr_available=False,
                           fused_cuda_available=False, autograd=True)
        assert d.selected is TRHashBackend.PYTORCH and any("backward" in r for r in d.reasons)


def test_quantized_copies_keep_differentiable_calls_off_hip():
    """An engine quantised with quantize_fp8_() computes from e4m3 copies
    whatever its config precision: differentiable calls resolve to PYTORCH
    (AUTO) or raise (explicit HIP), like an fp8 config."""
    cfg = _config()
    assert supports_hip_backward(cfg) and not supports_hip_backward(cfg, quantized_weights=True)
    d = select_backend(cfg, device_type="cuda", hip_available=True, cggr_available=False,
                       fused_cuda_available=False, autograd=True, quantized_weights=True)
    assert d.selected is TRHashBackend.PYTORCH and any("e4m3" in r for r in d.reasons)
    d = select_backend(cfg, device_type="cuda", hip_available=True, cggr_available=False,
                       fused_cuda_available=False, autograd=False, quantized_weights=True)
    assert d.selected is TRHashBackend.HIP
    with pytest.raises(RuntimeError, match="e4m3"):
        select_backend(_config(backend=TRHashBackend.HIP), device_type="cuda", hip_available=True, autograd=True,
                       quantized_weights=True)


def test_quantize_clears_the_cached_decision(monkeypatch):
    """The decision cache is keyed on the e4m3 state: a grad-enabled forward
    after quantize_fp8_() no longer reuses the bf16 decision."""
    from complexity_amd.tr_hash import capabilities

    monkeypatch.setattr(capabilities, "_hip_available", lambda: True)
    eng = _engine()

    class _Fake:   # the two attributes _decide reads of a ROCm activation
        device = torch.device("cuda")
        requires_grad = True

    fake = _Fake()
    with torch.enable_grad():
        assert eng._decide(fake).selected is TRHashBackend.HIP
        eng.quantize_fp8_()
        assert eng._decide(fake).selected is TRHashBackend.PYTORCH


def test_save_refuses_e4m3_packs():
    from complexity_amd import ops

    packed = ops.PackedLayer(act_dtype=torch.bfloat16, num_experts=4, expert_width=64,
                             expert_gate_up=torch.zeros(4, 128, 64, dtype=torch.float8_e4m3fn))
    assert packed.fp8
    assert not ops.PackedLayer(act_dtype=torch.bfloat16, num_experts=4, expert_width=64,
                               expert_gate_up=torch.zeros(4, 128, 64, dtype=torch.bfloat16)).fp8
    with pytest.raises(ValueError, match="inference-only"):
        ops.layer_forward(torch.zeros(2, 64), torch.zeros(2, dtype=torch.long), torch.zeros(2, 8, dtype=torch.long),
                          packed, (0.5, 0.5), 1.0, 1.0, save=True)


def test_fp8_activation_modes_are_validated():
    from complexity_amd import ops

    assert [ops.fp8_activation_mode(m) for m in (False, True, "gate_up")] == [False, True, "gate_up"]
    for bad in ("all", 1, None, "down"):
        with pytest.raises(ValueError, match="fp8_activations"):
            ops.fp8_activation_mode(bad)
    with pytest.raises(ValueError, match="fp8_activations"):
        ops.layer_forward(torch.zeros(2, 64), torch.zeros(2, dtype=torch.long), torch.zeros(2, 8, dtype=torch.long),
                          ops.PackedLayer(act_dtype=torch.bfloat16, num_experts=4, expert_width=64), (0.5, 0.5),
                          1.0, 1.0, act_fp8="both")


def test_missing_library_on_gpu_fails_loudly(monkeypatch):
    monkeypatch.delenv("TRMOE_ALLOW_PYTORCH_FALLBACK", raising=False)
    with pytest.raises(RuntimeError):
        select_backend(_config(), device_type="cuda", hip_available=False, cggr_available=False,
                       fused_cuda_available=False)
    monkeypatch.setenv("TRMOE_ALLOW_PYTORCH_FALLBACK", "1")
    d = select_backend(_config(), device_type="cuda", hip_available=False, cggr_available=False,
                       fused_cuda_available=False)
    assert d.selected is TRHashBackend.PYTORCH and any("unavailable" in r for r in d.reasons)


def test_explicit_backends_resolve_with_reasons():
    fused = _config(backend=TRHashBackend.FUSED_CUDA)
    d = select_backend(fused, device_type="cuda", hip_available=True, cggr_available=False, fused_cuda_available=False)
    assert d.selected is TRHashBackend.HIP and d.reasons
    with pytest.raises(RuntimeError):
        select_backend(_config(backend=TRHashBackend.FUSED_CUDA, num_experts=16), device_type="cuda",
                       hip_available=True, cggr_available=False, fused_cuda_available=False)
    cggr = _config(backend=TRHashBackend.CGGR, num_experts=16)
    d = select_backend(cggr, device_type="cuda", hip_available=True, cggr_available=False, fused_cuda_available=False)
    assert d.selected is TRHashBackend.HIP and d.partition == "assignment"
    with pytest.raises(RuntimeError):
        select_backend(_config(backend=TRHashBackend.HIP), device_type="cpu")
    d = select_backend(_config(backend=TRHashBackend.HIP), device_type="cuda", hip_available=True, autograd=True)
    assert d.selected is TRHashBackend.HIP
    with pytest.raises(RuntimeError):
        select_backend(_config(backend=TRHashBackend.HIP, hidden_size=36), device_type="cuda", hip_available=True,
                       autograd=True)


def test_fused_eligibility_is_the_reference_pair_shape():
    assert supports_fused_cuda(_config(num_experts=4, top_k=2))
    assert supports_fused_cuda(_config(num_experts=8, top_k=2))
    assert not supports_fused_cuda(_config(num_experts=16, top_k=2))
    assert not supports_fused_cuda(_config(num_experts=4, top_k=1))


@pytest.mark.parametrize("precision", [TRHashPrecision.INT8])
def test_int8_fails_explicitly(precision):
    with pytest.raises(NotImplementedError):
        select_backend(_config(precision=precision), device_type="cpu")


# --------------------------------------------------------------------------- engine (PYTORCH backend, CPU)


def _engine(seed=0, **kw):
    torch.manual_seed(seed)
    cfg = _config(precision=TRHashPrecision.FP32, **kw)
    eng = TRHashEngine(cfg).eval()
    with torch.no_grad():
        for p in eng.parameters():
            p.normal_(0.0, 0.2)
    return eng


def test_pytorch_backend_matches_token_by_token_definition():
    eng = _engine()
    x = torch.randn(2, 9, 32)
    ids = torch.randint(0, 257, (2, 9))
    with torch.no_grad():
        out = eng(x, ids)
    assert eng.last_backend.selected is TRHashBackend.PYTORCH
    params = {"expert_gate": eng.expert_gate, "expert_up": eng.expert_up, "expert_down": eng.expert_down,
              "shared_gate": eng.shared_gate.weight, "shared_up": eng.shared_up.weight,
              "shared_down": eng.shared_down.weight}
    want = O.naive_engine_output(x.double(), ids, eng.route_table, {k: v.double() for k, v in params.items()},
                                 route_weights=eng.config.route_weights)
    assert torch.allclose(out.double(), want, rtol=1e-5, atol=1e-5)


def test_norm_residual_on_cpu_is_the_reference_block_formula():
    """forward_norm_residual off the HIP backend: RMSNorm as norms.py:53-55
    writes it, then residual + forward (block.py:271-278); also through the
    MLP wrapper's norm-module form."""
    eng = _engine()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 9, 32, generator=g) * 2.0
    ids = torch.randint(0, 257, (2, 9), generator=g)
    nw = torch.rand(32, generator=g) + 0.5
    with torch.no_grad():
        out = eng.forward_norm_residual(x, ids, nw, 1e-6)
    assert eng.last_backend.selected is TRHashBackend.PYTORCH
    params = {"expert_gate": eng.expert_gate, "expert_up": eng.expert_up, "expert_down": eng.expert_down,
              "shared_gate": eng.shared_gate.weight, "shared_up": eng.shared_up.weight,
              "shared_down": eng.shared_down.weight}
    want = O.engine_forward_norm_residual(x.double(), ids, eng.route_table, {k: v.double() for k, v in params.items()},
                                          nw.double(), 1e-6, route_weights=eng.config.route_weights)
    assert torch.allclose(out.double(), want, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        eng.forward_norm_residual(x, ids, nw[:16], 1e-6)


def test_fp8_state_dict_round_trips_through_safetensors(tmp_path):
    """F3: an fp8 engine's e4m3 weights, scales and persisted route table go
    to disk with safetensors and come back into an engine built from another
    seed and route seed: same keys as the reference plus the fp8 buffers,
    identical tensors, identical outputs (the table is transplanted, not
    regenerated; docs/tr-hash-engine.md:64-66)."""
    from safetensors.torch import load_file, save_file

    torch.manual_seed(1)
    a = TRHashEngine(_config(precision=TRHashPrecision.FP8)).eval()
    with torch.no_grad():
        for p in a.parameters():
            p.normal_(0.0, 0.2)
    a.quantize_fp8_()
    sd = a.state_dict()
    for key in ("route_table", "fused_route_codes", "fused_expert_pairs", "expert_gate_fp8", "expert_gate_scale",
                "shared_down_fp8", "shared_down_scale"):
        assert key in sd, key
    assert sd["expert_gate_fp8"].dtype == torch.float8_e4m3fn
    path = tmp_path / "layer.safetensors"
    save_file({k: v.contiguous() for k, v in sd.items()}, str(path))

    torch.manual_seed(2)
    b = TRHashEngine(_config(precision=TRHashPrecision.FP8, route_seed=0x1234567)).eval()
    assert not torch.equal(b.route_table, a.route_table)
    b.load_state_dict(load_file(str(path)))
    for k, v in a.state_dict().items():
        assert torch.equal(b.state_dict()[k].view(torch.uint8) if v.dtype == torch.float8_e4m3fn
                           else b.state_dict()[k], v.view(torch.uint8) if v.dtype == torch.float8_e4m3fn else v), k
    x = torch.randn(2, 7, 32)
    ids = torch.randint(0, 257, (2, 7))
    with torch.no_grad():
        assert torch.equal(a(x, ids), b(x, ids))


def test_load_route_table_transplants_and_validates():
    eng = _engine()
    other = _engine(route_seed=0x2468ACE)
    assert not torch.equal(eng.route_table, other.route_table)
    eng.load_route_table(other.route_table)
    assert torch.equal(eng.route_table, other.route_table)
    assert torch.equal(eng._active_route_table, other.route_table)
    bad = other.route_table.clone()
    bad[0, 0] = eng.config.num_experts
    with pytest.raises(ValueError):
        eng.load_route_table(bad)
    with pytest.raises(ValueError):
        eng.load_route_table(other.route_table[:, :10])


def test_capacity_change_and_table_load_invalidate_captured_graphs():
    """test_tr_hash_dynamic_moe.py:166-170: captured graphs are dropped when
    the routing they baked in changes."""
    eng = _engine(num_experts=8, top_k=2)
    eng._graph_pool["sentinel"] = object()
    eng.set_active_capacity(num_experts=4)
    assert eng._graph_pool == {}
    eng._graph_pool["sentinel"] = object()
    eng.load_route_table(eng.route_table.clone())
    assert eng._graph_pool == {}


def test_quantize_and_module_moves_invalidate_captured_graphs():
    """A captured graph holds the addresses of the packs and parameters it
    read: quantize_fp8_() and _apply (.to(), .float(), ...) drop it."""
    eng = _engine(num_experts=4, top_k=2)
    eng._graph_pool["sentinel"] = object()
    eng.quantize_fp8_()
    assert eng._graph_pool == {}
    eng._graph_pool["sentinel"] = object()
    eng.to(torch.float64)
    assert eng._graph_pool == {}


def test_engine_materialises_every_shared_swiglu_projection():
    """test_tr_hash_shared_swiglu_contract.py:103-125: gate/up [S, H] and
    down [H, S] exist as linears whenever shared_width > 0."""
    eng = TRHashEngine(_config(hidden_size=32, shared_width=16, expert_width=8))
    assert tuple(eng.shared_gate.weight.shape) == (16, 32)
    assert tuple(eng.shared_up.weight.shape) == (16, 32)
    assert tuple(eng.shared_down.weight.shape) == (32, 16)
    none = TRHashEngine(_config(hidden_size=32, shared_width=0, expert_width=8))
    assert none.shared_gate is None and none.shared_up is None and none.shared_down is None


def test_capability_summary_contract_is_stable_across_shapes():
    keys = None
    for experts, k in ((4, 2), (16, 2), (8, 4), (1, 1)):
        summary = _engine(num_experts=experts, top_k=k).capability_summary()
        json.dumps(summary)
        assert len(summary) == 21
        keys = keys or set(summary)
        assert set(summary) == keys
        assert summary["selected_backend"] == "pytorch"


def test_default_active_capacity_equals_allocation_and_restriction_routes_to_active_pool():
    eng = _engine(num_experts=8, top_k=2)
    assert (eng.active_num_experts, eng.active_expert_width) == (8, 16)
    eng.set_active_capacity(num_experts=4)
    assert int(eng._active_route_table.max()) < 4


def test_reduced_capacity_changes_output_and_restoring_reproduces_it():
    eng = _engine(num_experts=8, top_k=2)
    x = torch.randn(1, 12, 32)
    ids = torch.randint(0, 257, (1, 12))
    with torch.no_grad():
        full = eng(x, ids)
        eng.set_active_capacity(num_experts=4, expert_width=8)
        reduced = eng(x, ids)
        eng.set_active_capacity(num_experts=8, expert_width=16)
        restored = eng(x, ids)
    assert reduced.shape == full.shape
    assert not torch.allclose(reduced, full)
    assert torch.equal(restored, full)


@pytest.mark.parametrize("kw", [dict(num_experts=3), dict(num_experts=16), dict(expert_width=17),
                                dict(expert_width=0), dict(num_experts=1)])
def test_set_active_capacity_rejects_invalid_requests(kw):
    eng = _engine(num_experts=8, top_k=2)
    with pytest.raises(ValueError):
        eng.set_active_capacity(**kw)


def test_fp8_quantization_matches_oracle_e4m3():
    eng = _engine()
    eng.quantize_fp8_()
    for name, w in (("expert_gate", eng.expert_gate), ("expert_down", eng.expert_down),
                    ("shared_up", eng.shared_up.weight), ("shared_down", eng.shared_down.weight)):
        q, s = O.quantize_e4m3(w.detach().float(), reduce_dim=1)  # the K axis of every weight
        assert torch.equal(getattr(eng, name + "_fp8").view(torch.uint8), q.view(torch.uint8)), name
        assert torch.equal(getattr(eng, name + "_scale"), s), name


# --------------------------------------------------------------------------- MLP adapter


def _mlp_config(**kw):
    base = dict(hidden_size=32, intermediate_size=64, vocab_size=257, num_experts=4, top_k=2,
                routing_strategy="token_id_multi_hash")
    base.update(kw)
    return MLPConfig(**base)


def test_mlp_registry_builds_the_engine_and_requires_token_ids():
    for name in ("tr_hash_engine", "tr_hash_moe"):
        mlp = MLP_REGISTRY.build(name, _mlp_config())
        assert isinstance(mlp, TRHashEngineMLP)
    mlp = MLP_REGISTRY.build("tr_hash_engine", _mlp_config())
    with pytest.raises(ValueError):
        mlp(torch.randn(1, 4, 32))
    out = mlp(torch.randn(1, 4, 32), token_ids=torch.randint(0, 257, (1, 4)))
    assert out.shape == (1, 4, 32)


@pytest.mark.parametrize("kw,expected", [
    ({"use_custom_kernels": False}, TRHashBackend.PYTORCH),
    ({"use_custom_kernels": " False "}, TRHashBackend.PYTORCH),
    ({"use_custom_kernels": "hip"}, TRHashBackend.HIP),
    ({}, TRHashBackend.AUTO),
    ({"use_custom_kernels": True}, TRHashBackend.AUTO),
    ({"use_cggr": True}, TRHashBackend.CGGR),
    ({"use_cggr": " TRUE"}, TRHashBackend.CGGR),
    # the kernel switch is read first (tr_hash_engine.py:59-62)
    ({"use_custom_kernels": False, "use_cggr": True}, TRHashBackend.PYTORCH),
])
def test_use_custom_kernels_switch_maps_to_backends(kw, expected):
    """The reference's backend policy (core/mlp/tr_hash_engine.py:52-63),
    plus "hip" forcing the gfx950 kernels."""
    mlp = TRHashEngineMLP(_mlp_config(**kw))
    assert mlp.engine.config.backend is expected


def test_mlp_adapter_exposes_dynamic_capacity_controls():
    mlp = TRHashEngineMLP(_mlp_config(num_experts=8))
    mlp.set_active_experts(4)
    mlp.set_active_expert_width(4)
    assert (mlp.engine.active_num_experts, mlp.engine.active_expert_width) == (4, 4)


def test_shared_lora_adapters_resolve_to_pytorch_with_reason(monkeypatch):
    """A shared adapter without LoRALinear's surface (reference
    engine.py:337-345, lora.py:37-90) keeps the layer on the universal path;
    an explicit HIP request raises."""
    import types

    from complexity_amd.tr_hash import TRHashEngine
    from complexity_amd.tr_hash import capabilities as caps

    monkeypatch.setattr(caps, "_hip_available", lambda: True)

    class _Adapter(torch.nn.Module):
        is_lora_adapter = True

        def __init__(self, base):
            super().__init__()
            self.base = base

        def forward(self, x):
            return self.base(x)

    fake_cuda = types.SimpleNamespace(device=types.SimpleNamespace(type="cuda"), requires_grad=False)
    with torch.no_grad():
        engine = TRHashEngine(_config())
        assert engine._decide(fake_cuda).selected is TRHashBackend.HIP
        engine.shared_gate = _Adapter(engine.shared_gate)
        d = engine._decide(fake_cuda)
        assert d.selected is TRHashBackend.PYTORCH and any("LoRA" in r for r in d.reasons)
        hip = TRHashEngine(_config(backend=TRHashBackend.HIP))
        hip.shared_up = _Adapter(hip.shared_up)
        with pytest.raises(RuntimeError, match="LoRA"):
            hip._decide(fake_cuda)


class _LinearLoRA(torch.nn.Module):
    """LoRALinear's surface (reference complexity/training/lora.py:37-90)."""

    is_lora_adapter = True

    def __init__(self, base, rank=3, alpha=6.0, dropout=0.0, dtype=torch.float64):
        super().__init__()
        self.base = base.to(dtype)
        self.scaling = alpha / rank
        self.dropout = torch.nn.Dropout(dropout) if dropout else torch.nn.Identity()
        self.lora_A = torch.nn.Parameter(torch.randn(rank, base.in_features, dtype=dtype))
        self.lora_B = torch.nn.Parameter(torch.randn(base.out_features, rank, dtype=dtype))
        self.base.requires_grad_(False)

    def forward(self, x):
        return self.base(x) + torch.nn.functional.linear(
            torch.nn.functional.linear(self.dropout(x), self.lora_A), self.lora_B) * self.scaling


class _ExpertLoRA(torch.nn.Module):
    """LoRAExpertTensor's parametrization surface (lora.py:93-165)."""

    def __init__(self, base, rank=2):
        super().__init__()
        E, fan_in, fan_out = base.shape
        self.lora_A = torch.nn.Parameter(torch.randn(E, fan_in, rank))
        self.lora_B = torch.nn.Parameter(torch.randn(E, rank, fan_out))
        self.calls = 0

    def forward(self, base):
        self.calls += 1
        return torch.baddbmm(base, self.lora_A, self.lora_B, alpha=0.5)


def test_merged_lora_weight_equals_the_adapter():
    """The HIP backend serves a shared LoRALinear by base + scaling * B @ A:
    same output and same factor gradients as the adapter's own two-step
    forward (f64, eval)."""
    from complexity_amd.tr_hash import weights as Wt

    torch.manual_seed(3)
    a = _LinearLoRA(torch.nn.Linear(24, 40, bias=False))
    x = torch.randn(7, 24, dtype=torch.float64)
    dy = torch.randn(7, 40, dtype=torch.float64)
    direct = a(x)
    gA, gB = torch.autograd.grad(direct, [a.lora_A, a.lora_B], dy)
    merged = torch.nn.functional.linear(x, Wt.merged_lora_weight(a))
    mA, mB = torch.autograd.grad(merged, [a.lora_A, a.lora_B], dy)
    assert torch.allclose(merged, direct, rtol=0, atol=1e-12)
    assert torch.allclose(mA, gA, rtol=0, atol=1e-10) and torch.allclose(mB, gB, rtol=0, atol=1e-10)


def test_weights_key_follows_parametrized_factors_without_materialising():
    """The pack cache key changes when a parametrization's factor changes in
    place, never materialises a weight, and is None (not cacheable) while a
    parametrization is in training mode; materialize() runs each once."""
    from torch.nn.utils import parametrize

    from complexity_amd.tr_hash import weights as Wt

    engine = TRHashEngine(_config())
    engine.requires_grad_(False)
    adapters = {}
    for name in Wt.EXPERT_NAMES:
        adapters[name] = _ExpertLoRA(getattr(engine, name))
        parametrize.register_parametrization(engine, name, adapters[name])
        adapters[name].calls = 0                     # registration evaluates it once
    engine.eval()
    k1 = Wt.weights_key(engine)
    assert k1 is not None and Wt.weights_key(engine) == k1
    assert all(a.calls == 0 for a in adapters.values())
    assert Wt.stored_dtype(engine, "expert_gate") == torch.float32
    with torch.no_grad():
        adapters["expert_up"].lora_B.add_(1.0)
    k2 = Wt.weights_key(engine)
    assert k2 != k1
    with torch.no_grad():
        engine.parametrizations["expert_down"].original.mul_(2.0)
    assert Wt.weights_key(engine) != k2
    got = Wt.materialize(engine)
    assert [a.calls for a in adapters.values()] == [1, 1, 1]
    assert torch.equal(got["expert_up"], adapters["expert_up"](engine.parametrizations["expert_up"].original))
    engine.train()
    assert Wt.weights_key(engine) is None

    # shared LoRA adapters: keyed on base and factors
    plain = TRHashEngine(_config()).eval()
    plain.shared_gate = _LinearLoRA(plain.shared_gate, dtype=torch.float32)
    k3 = Wt.weights_key(plain)
    with torch.no_grad():
        plain.shared_gate.lora_A.mul_(0.5)
    assert Wt.weights_key(plain) != k3


def test_shared_lora_with_merged_weights_selects_hip(monkeypatch):
    """LoRALinear adapters keep the HIP backend while their dropout is
    inactive; active dropout (training mode, p > 0) resolves to PYTORCH with a
    reason, and an explicit HIP request raises."""
    import types

    from complexity_amd.tr_hash import capabilities as caps

    monkeypatch.setattr(caps, "_hip_available", lambda: True)
    fake_cuda = types.SimpleNamespace(device=types.SimpleNamespace(type="cuda"), requires_grad=False)
    with torch.no_grad():
        engine = TRHashEngine(_config())
        for name in ("shared_gate", "shared_up", "shared_down"):
            setattr(engine, name, _LinearLoRA(getattr(engine, name), dropout=0.1, dtype=torch.float32))
        engine.eval()
        assert engine._decide(fake_cuda).selected is TRHashBackend.HIP
        engine.train()
        d = engine._decide(fake_cuda)
        assert d.selected is TRHashBackend.PYTORCH and any("LoRA dropout" in r for r in d.reasons)
        engine.shared_up.dropout = torch.nn.Identity()
        engine.shared_gate.dropout.p = 0.0
        engine.shared_down.dropout.p = 0.0
        assert engine._decide(fake_cuda).selected is TRHashBackend.HIP
        hip = TRHashEngine(_config(backend=TRHashBackend.HIP))
        hip.shared_gate = _LinearLoRA(hip.shared_gate, dropout=0.1, dtype=torch.float32)
        with pytest.raises(RuntimeError, match="LoRA dropout"):
            hip._decide(fake_cuda)


def test_device_guard_is_transparent_for_host_tensors():
    """The entry points' device guard only switches devices for a GPU tensor
    on a non-current device; for other arguments it calls straight through."""
    from complexity_amd import ops

    calls = []

    @ops._on_tensor_device
    def probe(x, k=1):
        calls.append((x.device.type, k))
        return x * k

    out = probe(torch.ones(2), k=3)
    assert torch.equal(out, torch.full((2,), 3.0)) and calls == [("cpu", 3)]
    assert probe.__name__ == "probe"
    for name in ("layer_forward", "layer_backward", "route_sort", "pack_dense_routed", "pack_fragments",
                 "rms_row_scale"):
        assert getattr(ops, name).__wrapped__ is not None
