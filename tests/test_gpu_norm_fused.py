"""F2: the block's post-attention RMSNorm fused into the gate|up kernels.

``TRHashEngine.forward_norm_residual(x, ids, norm_weight, eps)`` is
``x + forward(rmsnorm(x))`` (complexity/models/block.py:271-278 with
RMSNorm, complexity/core/normalization/norms.py:46-55); the oracle is
``engine_forward_norm_residual``.  Decode sizes (dense strategy) compute the
per-token scale inside the decode kernel; larger calls and the grouped
strategy take it from ``trmoe_rms_row_scale``.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = {"fp32": 1e-4, "bf16": 2e-2}


def _params(engine):
    p = {n: getattr(engine, n).detach().float().cpu() for n in ("expert_gate", "expert_up", "expert_down")}
    if engine.shared_gate is not None:
        for n in ("shared_gate", "shared_up", "shared_down"):
            p[n] = getattr(engine, n).weight.detach().float().cpu()
    return p


def _oracle(engine, x, ids, nw, eps):
    cfg = engine.config
    return O.engine_forward_norm_residual(
        x.float().cpu(), ids.cpu(), engine._active_route_table.cpu(), _params(engine), nw.float().cpu(), eps,
        route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale,
        active_experts=engine.active_num_experts, active_width=engine.active_expert_width)


def _norm_weight(hidden, device, dtype, seed=5):
    g = torch.Generator().manual_seed(seed)
    return (torch.rand(hidden, generator=g) + 0.5).to(device=device, dtype=dtype)


@pytest.mark.parametrize("name,strategy", [
    ("c3_bf16_decode_64", "auto"),
    ("c4_bf16_decode_8", "auto"),
    ("c3_bf16_decode_64", "grouped"),
    ("c1_fp32_2048", "auto"),
    ("c1_fp32_2048", "grouped"),
    ("c2_bf16_prefill_16384", "auto"),
])
def test_norm_residual_layer(gpu, name, strategy):
    from complexity_amd import workloads as Wl
    from complexity_amd.tr_hash import TRHashBackend

    print(f"norm residual {name} {strategy}", flush=True)
    w = Wl.WORKLOADS[name]
    engine = Wl.build_engine(w, gpu, backend="hip")
    if strategy != "auto":
        engine.routed_strategy = strategy
    dt = torch.float32 if w.dtype == "fp32" else torch.bfloat16
    x = (Wl.make_hidden(w).to(gpu) * 2.5).to(dt)   # the norm must undo the scale
    ids = Wl.make_token_ids(w).to(gpu)
    nw = _norm_weight(w.hidden, gpu, dt)
    with torch.no_grad():
        out = engine.forward_norm_residual(x, ids, nw, 1e-6)
    torch.cuda.synchronize()
    assert engine.last_backend.selected is TRHashBackend.HIP
    bound = BOUND["fp32" if dt == torch.float32 else "bf16"]
    if w.tokens > 4096:
        rows = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(1))[:1024]
        xr, ir = x.reshape(-1, w.hidden)[rows.to(gpu)].unsqueeze(0), ids.reshape(-1)[rows.to(gpu)].unsqueeze(0)
        ref = _oracle(engine, xr, ir, nw, 1e-6)
        got = out.reshape(-1, w.hidden)[rows.to(gpu)].unsqueeze(0)
    else:
        ref = _oracle(engine, x, ids, nw, 1e-6)
        got = out
    assert O.normwise_rel_err(got, ref) <= bound
    # the MLP term alone (the residual dominates the sum above): the same
    # fused pack and scales through ops.layer_forward without the residual
    from complexity_amd import ops

    packed = engine._hip_packed(nw)
    flat = x.reshape(-1, w.hidden)
    with torch.no_grad():
        mlp = ops.layer_forward(flat, ids.reshape(-1), engine._active_route_table, packed,
                                engine.config.route_weights, engine.config.shared_output_scale,
                                engine.config.routed_output_scale, norm_eps=1e-6)
    cfg = engine.config
    xs = flat if w.tokens <= 4096 else flat[rows.to(gpu)]
    ids_s = ids.reshape(-1) if w.tokens <= 4096 else ids.reshape(-1)[rows.to(gpu)]
    mlp_s = mlp if w.tokens <= 4096 else mlp[rows.to(gpu)]
    ref_mlp = O.engine_forward(O.rms_norm(xs.float().cpu(), nw.float().cpu(), 1e-6), ids_s.cpu(),
                               engine._active_route_table.cpu(), _params(engine), route_weights=cfg.route_weights,
                               shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale,
                               active_experts=engine.active_num_experts, active_width=engine.active_expert_width)
    assert O.normwise_rel_err(mlp_s, ref_mlp) <= bound


def test_norm_residual_autograd_runs_the_unfused_path(gpu):
    """Under autograd the norm runs as the reference writes it (differentiable)
    and the MLP through the HIP autograd Function; the values agree."""
    from complexity_amd import workloads as Wl

    w = Wl.C3
    engine = Wl.build_engine(w, gpu, backend="hip")
    x = (Wl.make_hidden(w).to(gpu) * 2.5).to(torch.bfloat16)
    ids = Wl.make_token_ids(w).to(gpu)
    nw = _norm_weight(w.hidden, gpu, torch.bfloat16)
    with torch.no_grad():
        fused = engine.forward_norm_residual(x, ids, nw, 1e-6)
    xg = x.clone().requires_grad_(True)
    out = engine.forward_norm_residual(xg, ids, nw, 1e-6)
    out.float().sum().backward()
    assert xg.grad is not None and torch.isfinite(xg.grad.float()).all()
    assert O.normwise_rel_err(out.detach(), fused) <= 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,hidden", [(1, 200), (5, 100), (64, 896), (300, 104), (4096, 896)])
def test_rms_row_scale_kernel(gpu, dtype, n, hidden):
    """hidden = 100/104 leave a tail after the last whole 16-byte chunk."""
    from complexity_amd import ops

    g = torch.Generator().manual_seed(n + hidden)
    x = (torch.randn(n, hidden, generator=g) * 3.0).to(dtype)
    r = ops.rms_row_scale(x.to(gpu), 1e-6).cpu()
    ref = torch.rsqrt(x.double().pow(2).mean(-1) + 1e-6)
    assert torch.allclose(r.double(), ref, rtol=1e-5, atol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 7, 64, 128, 129, 700])
def test_shared_gate_up_rms(gpu, dtype, n):
    """Kernel level: packs of W * norm_weight, scales from the decode kernel
    (n <= 128, eps) and from trmoe_rms_row_scale, against
    silu(xn Wg^T) * (xn Wu^T) with xn = rmsnorm(x)."""
    from complexity_amd import ops

    H, S, eps = 200, 320, 1e-5
    g = torch.Generator().manual_seed(n)
    x = (torch.randn(n, H, generator=g) * 2.0).to(dtype)
    wg, wu = (torch.randn(S, H, generator=g) * 0.1).to(dtype), (torch.randn(S, H, generator=g) * 0.1).to(dtype)
    nw = (torch.rand(H, generator=g) + 0.5).to(dtype)
    xn = O.rms_norm(x.double(), nw.double(), eps)
    ref = F.silu(xn @ wg.double().T) * (xn @ wu.double().T)
    fold = lambda w: (w.float() * nw.float()[None, :]).to(dtype)
    pg, _ = ops.pack_linear_gate_up(fold(wg).to(gpu), fold(wu).to(gpu))
    xg = x.to(gpu)
    r = ops.rms_row_scale(xg, eps)
    got = ops.shared_gate_up(xg, pg, None, S, row_scale=r).cpu()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert O.normwise_rel_err(got[:, :S], ref) <= tol
    if n <= 128:
        got_in = ops.shared_gate_up(xg, pg, None, S, rms_eps=eps).cpu()
        assert O.normwise_rel_err(got_in[:, :S], ref) <= tol
        # the in-kernel scales and the row-scale kernel's agree to fp32 rounding
        assert O.normwise_rel_err(got_in.float(), got.float()) <= (1e-5 if dtype == torch.float32 else 1e-2)
    else:
        with pytest.raises(ValueError, match="128"):
            ops.shared_gate_up(xg, pg, None, S, rms_eps=eps)


def _small_engine(gpu, dtype, strategy, fp8=False):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    engine = TRHashEngine(TRHashEngineConfig(hidden_size=256, vocab_size=5000, num_experts=4, top_k=2,
                                             shared_width=384, expert_width=64,
                                             routing_strategy="token_id_multi_hash", routed_output_scale=2.0,
                                             shared_output_scale=0.5, precision="fp8" if fp8 else dtype,
                                             backend="hip")).to(gpu)
    if dtype != "fp32":
        engine = engine.to(torch.bfloat16)
    engine.routed_strategy = strategy
    if fp8:
        engine.quantize_fp8_()
    return engine


@pytest.mark.parametrize("dtype,strategy,tokens", [
    ("fp32", "dense", 300), ("bf16", "dense", 300), ("bf16", "grouped", 300), ("bf16", "dense", 40),
])
def test_norm_residual_backward_on_rmsnorm_kernels(gpu, dtype, strategy, tokens):
    """Under autograd the norm runs on the RMSNorm kernels and the MLP on the
    HIP autograd Function: the output and the gradients of x, the norm weight
    and two layer weights match f64 autograd of the oracle."""
    print(f"norm residual backward {dtype} {strategy} {tokens}", flush=True)
    dt = torch.float32 if dtype == "fp32" else torch.bfloat16
    engine = _small_engine(gpu, dtype, strategy)
    g = torch.Generator().manual_seed(tokens)
    ids = torch.randint(0, 5000, (2, tokens // 2), generator=g).to(gpu)
    x = (torch.randn(2, tokens // 2, 256, generator=g) * 2.5).to(gpu, dt)
    nw = _norm_weight(256, gpu, dt).requires_grad_(True)
    dout = (torch.randn(2, tokens // 2, 256, generator=g) * 0.1).to(gpu, dt)
    xg = x.detach().clone().requires_grad_(True)
    out = engine.forward_norm_residual(xg, ids, nw, 1e-6)
    assert engine.last_norm == "rmsnorm"
    out.backward(dout)
    torch.cuda.synchronize()

    cfg = engine.config
    d = torch.float64
    leaves = {"x": x.detach().cpu().to(d).requires_grad_(True), "nw": nw.detach().cpu().to(d).requires_grad_(True)}
    p = {k: v.to(d) for k, v in _params(engine).items()}
    for k in ("shared_down", "expert_gate"):
        p[k] = leaves[k] = p[k].clone().requires_grad_(True)
    ref = O.engine_forward_norm_residual(
        leaves["x"], ids.cpu(), engine._active_route_table.cpu(), p, leaves["nw"], 1e-6,
        route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale)
    names = list(leaves)
    grads = dict(zip(names, torch.autograd.grad(ref, [leaves[n] for n in names], dout.detach().cpu().to(d))))
    got = {"x": xg.grad, "nw": nw.grad, "shared_down": engine.shared_down.weight.grad,
           "expert_gate": engine.expert_gate.grad}
    bound = BOUND[dtype]
    assert O.normwise_rel_err(out.detach(), ref.detach()) <= bound
    for n in names:
        assert got[n] is not None, n
        assert O.normwise_rel_err(got[n].float().cpu(), grads[n]) <= bound, (n, O.normwise_rel_err(got[n], grads[n]))


def test_norm_residual_fp8_runs_the_rmsnorm_kernel(gpu):
    """fp8 weights cannot take the norm weight in their packs: the norm runs on
    the RMSNorm kernel, then the fp8 layer (against the oracle on the
    dequantised weights, bound 5e-2)."""
    engine = _small_engine(gpu, "bf16", "grouped", fp8=True)
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, 5000, (1, 700), generator=g).to(gpu)
    # small x (the norm is scale-free) so that out - x keeps the MLP term's bits
    x = (torch.randn(1, 700, 256, generator=g) * 0.02).to(gpu, torch.bfloat16)
    nw = _norm_weight(256, gpu, torch.bfloat16)
    with torch.no_grad():
        out = engine.forward_norm_residual(x, ids, nw, 1e-6)
    torch.cuda.synchronize()
    assert engine.last_norm == "rmsnorm"
    p = {}
    for n in ("expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up", "shared_down"):
        p[n] = O.dequantize_e4m3(getattr(engine, n + "_fp8").cpu(), getattr(engine, n + "_scale").cpu(), 1)
    cfg = engine.config
    ref = O.engine_forward(O.rms_norm(x.float().cpu(), nw.float().cpu(), 1e-6), ids.cpu(),
                           engine._active_route_table.cpu(), p, route_weights=cfg.route_weights,
                           shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale)
    mlp = out.float().cpu() - x.float().cpu()
    assert O.normwise_rel_err(mlp, ref) <= 5e-2
