"""Backward of the HIP layer (the reference's autograd surface) vs the oracle.

Kernel level: the token-reduction weight-gradient GEMM against a torch fp32
product (dense, gathered, segmented, split), the SwiGLU backward kernels
against the oracle's closed form (``swiglu_backward``, pinned to autograd of
the forward on the CPU), the grouped linear against per-expert products.
Layer level: gradients of x and of every parameter through
``TRHashEngine`` on the HIP backend against ``engine_backward`` (autograd of
the oracle's universal forward, pinned to central differences on the CPU).

Bounds: normwise max|got - ref| / max|ref| <= 1e-4 for fp32, 2e-2 for bf16
(the north-star forward tolerances); outputs and weight gradients are
rounded to the parameter dtype, accumulation is fp32.
"""

import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = {"fp32": 1e-4, "bf16": 2e-2}
# token-reduction GEMM alone: fp32 accumulation, one rounding of the output
GEMM_BOUND = {"fp32": 1e-5, "bf16": 8e-3}
DT = {"fp32": torch.float32, "bf16": torch.bfloat16}


def _err(got, ref):
    return O.normwise_rel_err(got.float().cpu(), ref.float().cpu())


# --------------------------------------------------------------------------- weight_grad


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("T,M,N", [(1, 64, 64), (63, 136, 264), (777, 896, 256), (4096, 64, 64),
                                   (2048, 512, 896)])
def test_weight_grad_dense(gpu, dtype, T, M, N):
    from complexity_amd import ops

    print(f"weight_grad dense {dtype} T={T} M={M} N={N}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(T + M + N)
    a = torch.randn(T, M, generator=g).to(DT[dtype]).to(gpu)
    b = torch.randn(T, N, generator=g).to(DT[dtype]).to(gpu)
    out = ops.weight_grad(a, b, M, N, T)
    torch.cuda.synchronize()
    ref = a.float().T @ b.float()
    assert out.shape == (1, M, N)
    assert _err(out[0], ref) <= GEMM_BOUND[dtype]


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("gather", ["a", "b"])
def test_weight_grad_segments_gathered(gpu, dtype, gather):
    """Expert segments (one empty, one longer than a staging block) with one
    operand read through a partition index mod n (as the routed grads do)."""
    from complexity_amd import ops

    print(f"weight_grad segments {dtype} gather={gather}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(3)
    counts = [700, 0, 2500, 33, 1]
    E, n = len(counts), 1600
    rows = sum(counts)
    offsets = torch.tensor([0] + list(torch.tensor(counts).cumsum(0)), dtype=torch.int32)
    idx = torch.randint(0, 2 * n, (rows,), generator=g)   # values slot*n + t, 2 slots
    M, N = 72, 136
    if gather == "a":
        a = torch.randn(n, M, generator=g).to(DT[dtype])
        b = torch.randn(rows, N, generator=g).to(DT[dtype])
        a_rows = a[idx % n]
        b_rows = b
    else:
        a = torch.randn(rows, M, generator=g).to(DT[dtype])
        b = torch.randn(n, N, generator=g).to(DT[dtype])
        a_rows = a
        b_rows = b[idx % n]
    out = ops.weight_grad(a.to(gpu), b.to(gpu), M, N, rows,
                          a_gather=idx.to(gpu) if gather == "a" else None,
                          b_gather=idx.to(gpu) if gather == "b" else None, gather_mod=n,
                          offsets=offsets.to(gpu), segments=E)
    torch.cuda.synchronize()
    for e in range(E):
        s0, s1 = int(offsets[e]), int(offsets[e + 1])
        ref = a_rows[s0:s1].float().T @ b_rows[s0:s1].float()
        if s1 == s0:
            assert out[e].abs().max().item() == 0, e
        else:
            assert _err(out[e], ref) <= GEMM_BOUND[dtype], e


def test_weight_grad_is_deterministic(gpu):
    from complexity_amd import ops

    g = torch.Generator(device="cpu").manual_seed(1)
    a = torch.randn(8192, 128, generator=g).to(torch.bfloat16).to(gpu)
    b = torch.randn(8192, 64, generator=g).to(torch.bfloat16).to(gpu)
    r1 = ops.weight_grad(a, b, 128, 64, 8192)
    r2 = ops.weight_grad(a, b, 128, 64, 8192)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2)


# --------------------------------------------------------------------------- SwiGLU backward


def _split_dgu(dgu, F):
    v = dgu.view(dgu.shape[0], F // 32, 2, 32)
    return v[:, :, 0].reshape(dgu.shape[0], F), v[:, :, 1].reshape(dgu.shape[0], F)


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("n,H,S", [(1, 64, 96), (300, 128, 256), (1000, 896, 3072)])
def test_shared_swiglu_backward(gpu, dtype, n, H, S):
    from complexity_amd import ops

    print(f"shared_swiglu_backward {dtype} n={n} H={H} S={S}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(n + S)
    x = torch.randn(n, H, generator=g).to(DT[dtype])
    dout = torch.randn(n, H, generator=g).to(DT[dtype])
    wg = (torch.randn(S, H, generator=g) * H ** -0.5).to(DT[dtype])
    wu = (torch.randn(S, H, generator=g) * H ** -0.5).to(DT[dtype])
    wd = (torch.randn(H, S, generator=g) * S ** -0.5).to(DT[dtype])
    gu, _ = ops.pack_linear_gate_up(wg.to(gpu), wu.to(gpu))
    wdt = ops.pack_linear_down_t(wd.to(gpu))
    dgu, hm = ops.shared_swiglu_backward(x.to(gpu), dout.to(gpu), gu, wdt, S, 1.5)
    torch.cuda.synchronize()
    F = -(-S // 128) * 128
    dg, du = _split_dgu(dgu, F)
    rdg, rdu, rh = O.swiglu_backward(x.double(), dout.double(), wg.double(), wu.double(), wd.double(), 1.5)
    assert _err(dg[:, :S], rdg) <= BOUND[dtype]
    assert _err(du[:, :S], rdu) <= BOUND[dtype]
    assert _err(hm[:, :S], rh) <= BOUND[dtype]
    if F > S:   # padded features: zero weights give zero gradients
        assert dg[:, S:].abs().max().item() == 0 and hm[:, S:].abs().max().item() == 0
    # the training forward's saved gate|up outputs instead of the recomputation
    hs, gus = ops.shared_gate_up(x.to(gpu), gu, None, S, save=True)
    h_plain = ops.shared_gate_up(x.to(gpu), gu, None, S)
    dgu2, hm2 = ops.shared_swiglu_backward(x.to(gpu), dout.to(gpu), gu, wdt, S, 1.5, gu=gus)
    torch.cuda.synchronize()
    assert _err(hs, h_plain) <= BOUND[dtype]   # other tiles, same h to rounding
    g_ref = (x.double() @ wg.double().T, x.double() @ wu.double().T)
    sg, su = _split_dgu(gus, F)
    assert _err(sg[:, :S], g_ref[0]) <= BOUND[dtype] and _err(su[:, :S], g_ref[1]) <= BOUND[dtype]
    dg2, du2 = _split_dgu(dgu2, F)
    assert _err(dg2[:, :S], rdg) <= BOUND[dtype]
    assert _err(du2[:, :S], rdu) <= BOUND[dtype]
    assert _err(hm2[:, :S], rh) <= BOUND[dtype]


@pytest.mark.parametrize("S,E,W,n", [(3072, 4, 64, 16384), (256, 4, 64, 700), (96, 3, 40, 300)])
def test_weight_grad_mapped_matches_the_strided_views(gpu, S, E, W, n):
    """trmoe_weight_grad_mapped (dense strategy's dWgu in row mode, dWd in
    column mode) against trmoe_weight_grad plus the unmapped path's views:
    the same fp32 partials summed in the same order, so bit-identical."""
    from complexity_amd import ops

    print(f"weight_grad_mapped S={S} E={E} W={W} n={n}", flush=True)
    H = 128 if n < 16384 else 896
    s_pad, w_pad = -(-S // 128) * 128, -(-W // 64) * 64
    F_ = s_pad + E * w_pad
    g = torch.Generator(device="cpu").manual_seed(S + E + W + n)
    dgu = (torch.randn(n, 2 * F_, generator=g) * 0.1).to(torch.bfloat16).to(gpu)
    x = torch.randn(n, H, generator=g).to(torch.bfloat16).to(gpu)
    dout = torch.randn(n, H, generator=g).to(torch.bfloat16).to(gpu)
    hm = torch.randn(n, F_, generator=g).to(torch.bfloat16).to(gpu)
    roff, rstride, coff, cstride, offs = ops._dense_grad_maps(S, E, W, H, x.device)
    flat = torch.full((offs[-1],), float("nan"), dtype=torch.bfloat16, device=gpu)
    ops.weight_grad_mapped(dgu, x, 2 * F_, H, n, 1, roff, rstride, flat)
    ops.weight_grad_mapped(dout, hm, H, F_, n, 2, coff, cstride, flat)
    dwgu = ops.weight_grad(dgu, x, 2 * F_, H, n)[0]
    dwd = ops.weight_grad(dout, hm, H, F_, n)[0]
    torch.cuda.synchronize()
    assert not torch.isnan(flat).any()
    o_gate, o_up, o_sd, o_eg, o_eu, o_ed, _ = offs
    g_rows, u_rows = ops._gate_up_rows(dwgu, F_)
    sh, ew = S * H, E * W * H
    assert torch.equal(flat[o_gate:o_gate + sh].view(S, H), g_rows[:S])
    assert torch.equal(flat[o_up:o_up + sh].view(S, H), u_rows[:S])
    assert torch.equal(flat[o_sd:o_sd + sh].view(H, S), dwd[:, :S])
    assert torch.equal(flat[o_eg:o_eg + ew].view(E, H, W), g_rows[s_pad:].view(E, w_pad, H)[:, :W].transpose(1, 2))
    assert torch.equal(flat[o_eu:o_eu + ew].view(E, H, W), u_rows[s_pad:].view(E, w_pad, H)[:, :W].transpose(1, 2))
    assert torch.equal(flat[o_ed:o_ed + ew].view(E, W, H),
                       dwd[:, s_pad:].reshape(H, E, w_pad)[:, :, :W].permute(1, 2, 0))


def test_shared_swiglu_backward_persistent(gpu):
    """Saved bf16 g|u at a size that fills a round of CUs: the dh GEMM runs
    on the persistent stream (256 x 256 tiles, ragged last row tile, padded
    features past S), checked against the closed form in fp64."""
    from complexity_amd import ops

    n, H, S = 5500, 896, 3000
    print(f"shared_swiglu_backward persistent bf16 n={n} H={H} S={S}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(7)
    x = torch.randn(n, H, generator=g).to(torch.bfloat16).to(gpu)
    dout = torch.randn(n, H, generator=g).to(torch.bfloat16).to(gpu)
    wg = (torch.randn(S, H, generator=g) * H ** -0.5).to(torch.bfloat16).to(gpu)
    wu = (torch.randn(S, H, generator=g) * H ** -0.5).to(torch.bfloat16).to(gpu)
    wd = (torch.randn(H, S, generator=g) * S ** -0.5).to(torch.bfloat16).to(gpu)
    gu, _ = ops.pack_linear_gate_up(wg, wu)
    wdt = ops.pack_linear_down_t(wd)
    _, gus = ops.shared_gate_up(x, gu, None, S, save=True)
    dgu, hm = ops.shared_swiglu_backward(x, dout, gu, wdt, S, 1.5, gu=gus)
    torch.cuda.synchronize()
    F = -(-S // 128) * 128
    # the closed form from the same bf16-rounded g|u the kernel reads
    sg, su = _split_dgu(gus, F)
    gd, ud = sg[:, :S].double(), su[:, :S].double()
    dh = dout.double() @ wd.double()
    s = torch.sigmoid(gd)
    rdg, rdu, rh = 1.5 * dh * ud * (s + gd * s * (1 - s)), 1.5 * dh * gd * s, 1.5 * gd * s * ud
    dg, du = _split_dgu(dgu, F)
    assert _err(dg[:, :S], rdg) <= BOUND["bf16"]
    assert _err(du[:, :S], rdu) <= BOUND["bf16"]
    assert _err(hm[:, :S], rh) <= BOUND["bf16"]
    assert dg[:, S:].abs().max().item() == 0 and du[:, S:].abs().max().item() == 0
    assert hm[:, S:].abs().max().item() == 0
    # and the full closed form from x
    odg, odu, oh = O.swiglu_backward(x.double(), dout.double(), wg.double(), wu.double(), wd.double(), 1.5)
    assert _err(dg[:, :S], odg) <= BOUND["bf16"] and _err(du[:, :S], odu) <= BOUND["bf16"]
    assert _err(hm[:, :S], oh) <= BOUND["bf16"]


@pytest.mark.parametrize("dtype", ["fp32", "bf16"])
@pytest.mark.parametrize("E,k,W,n", [(4, 2, 64, 500), (16, 2, 256, 300), (8, 4, 40, 129), (2, 1, 128, 1)])
def test_routed_swiglu_backward_and_grouped_linear(gpu, dtype, E, k, W, n):
    from complexity_amd import ops

    print(f"routed_swiglu_backward {dtype} E={E} k={k} W={W} n={n}", flush=True)
    H = 128
    g = torch.Generator(device="cpu").manual_seed(E * W + n)
    x = torch.randn(n, H, generator=g).to(DT[dtype])
    dout = torch.randn(n, H, generator=g).to(DT[dtype])
    gate = (torch.randn(E, H, W, generator=g) * H ** -0.5).to(DT[dtype])
    up = (torch.randn(E, H, W, generator=g) * H ** -0.5).to(DT[dtype])
    down = (torch.randn(E, W, H, generator=g) * W ** -0.5).to(DT[dtype])
    table = torch.from_numpy(O.multi_hash_table(5000, E, k, 0))
    ids = torch.randint(0, 5000, (n,), generator=g)
    rw = (0.6, 0.4, 0.3, 0.2)[:k] if k > 1 else (1.0,)
    sorted_idx, inverse, offsets, _ = ops.route_sort(ids.to(gpu), table.to(gpu), E, ops.ORDER_TOKEN)
    egu, _ = ops.pack_expert_gate_up(gate.to(gpu), up.to(gpu))
    edt = ops.pack_expert_down_t(down.to(gpu))
    dgu, hm = ops.routed_swiglu_backward(x.to(gpu), dout.to(gpu), sorted_idx, offsets, E, k, egu, edt, W, rw, 2.0)
    wp = -(-W // 64) * 64
    egut = ops.pack_gate_up_t(egu, H)
    dxa = ops.grouped_linear(dgu, 2 * wp, offsets, E, egut, H)
    torch.cuda.synchronize()
    dg, du = _split_dgu(dgu, wp)
    srt, off = sorted_idx.cpu(), offsets.cpu()
    for e in range(E):
        s0, s1 = int(off[e]), int(off[e + 1])
        if s1 == s0:
            continue
        t = srt[s0:s1] % n
        mult = (2.0 * torch.tensor(rw, dtype=torch.float64)[srt[s0:s1] // n]).unsqueeze(1)
        rdg, rdu, rh = O.swiglu_backward(x[t].double(), dout[t].double(), gate[e].T.double(), up[e].T.double(),
                                         down[e].T.double(), mult)
        assert _err(dg[s0:s1, :W], rdg) <= BOUND[dtype], e
        assert _err(du[s0:s1, :W], rdu) <= BOUND[dtype], e
        assert _err(hm[s0:s1, :W], rh) <= BOUND[dtype], e
        # data gradient of the routed rows: [dg|du] . [Wg_e; Wu_e]
        ref_dx = dg[s0:s1, :W].double().cpu() @ gate[e].T.double() + du[s0:s1, :W].double().cpu() @ up[e].T.double()
        assert _err(dxa[s0:s1], ref_dx) <= BOUND[dtype], e


# --------------------------------------------------------------------------- layer


def _engine(gpu, dtype, E, k, S, W, H, weights, strategy):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    engine = TRHashEngine(TRHashEngineConfig(hidden_size=H, vocab_size=5000, num_experts=E, top_k=k,
                                             shared_width=S, expert_width=W, routing_strategy="token_id_multi_hash",
                                             route_weights=weights or (), routed_output_scale=2.0,
                                             shared_output_scale=0.5, precision=dtype, backend="hip")).to(gpu)
    if dtype == "bf16":
        engine = engine.to(torch.bfloat16)
    engine.routed_strategy = strategy
    return engine


def _oracle_grads(engine, x, ids, dout, device="cpu", dtype=torch.float64):
    cfg = engine.config
    params = {n: getattr(engine, n).detach().to(device, dtype) for n in ("expert_gate", "expert_up", "expert_down")}
    if engine.shared_gate is not None:
        for n in ("shared_gate", "shared_up", "shared_down"):
            params[n] = getattr(engine, n).weight.detach().to(device, dtype)
    return O.engine_backward(x.detach().to(device, dtype), ids.to(device), engine._active_route_table.to(device),
                             params, dout.to(device, dtype), route_weights=cfg.route_weights,
                             shared_scale=cfg.shared_output_scale, routed_scale=cfg.routed_output_scale,
                             active_experts=engine.active_num_experts, active_width=engine.active_expert_width)


def _hip_grads(engine, x, ids, dout, residual=None):
    from complexity_amd.tr_hash import TRHashBackend

    engine.zero_grad(set_to_none=True)
    xg = x.detach().clone().requires_grad_(True)
    if residual is None:
        out = engine(xg, ids)
    else:
        out = engine.forward_with_residual(xg, ids, residual)
    assert engine.last_backend.selected is TRHashBackend.HIP, engine.last_backend
    out.backward(dout)
    torch.cuda.synchronize()
    grads = {"x": xg.grad}
    for n in ("expert_gate", "expert_up", "expert_down"):
        grads[n] = getattr(engine, n).grad
    if engine.shared_gate is not None:
        for n in ("shared_gate", "shared_up", "shared_down"):
            grads[n] = getattr(engine, n).weight.grad
    return out, grads


def _check(got, ref, dtype):
    for name, r in ref.items():
        g = got[name]
        assert g is not None, name
        assert g.shape == r.shape, (name, g.shape, r.shape)
        assert _err(g, r) <= BOUND[dtype], (name, _err(g, r))


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("E,k,S,W,dtype,weights", [
    (4, 2, 256, 64, "fp32", (0.7, 0.3)),
    (4, 2, 512, 64, "bf16", None),
    (8, 4, 96, 12, "fp32", None),
    (2, 1, 0, 40, "bf16", None),
    (16, 2, 128, 32, "bf16", None),
])
def test_layer_backward_matches_oracle(gpu, strategy, E, k, S, W, dtype, weights):
    print(f"layer backward {strategy} E={E} k={k} S={S} W={W} {dtype}", flush=True)
    torch.manual_seed(E + k + S + W)
    H = 128
    engine = _engine(gpu, dtype, E, k, S, W, H, weights, strategy)
    ids = torch.randint(0, 5000, (2, 300), device=gpu)
    x = torch.randn(2, 300, H, device=gpu, dtype=DT[dtype])
    dout = torch.randn(2, 300, H, device=gpu, dtype=DT[dtype])
    _, got = _hip_grads(engine, x, ids, dout)
    assert engine._packed.strategy == strategy
    _check(got, _oracle_grads(engine, x, ids, dout), dtype)


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
def test_layer_backward_active_capacity_and_residual(gpu, strategy):
    print(f"layer backward active/residual {strategy}", flush=True)
    torch.manual_seed(3)
    engine = _engine(gpu, "fp32", 8, 2, 192, 48, 64, None, strategy)
    engine.set_active_capacity(num_experts=4, expert_width=20)
    ids = torch.randint(0, 5000, (3, 70), device=gpu)
    x = torch.randn(3, 70, 64, device=gpu)
    res = torch.randn(3, 70, 64, device=gpu, requires_grad=True)
    dout = torch.randn(3, 70, 64, device=gpu)
    out, got = _hip_grads(engine, x, ids, dout, residual=res)
    ref = _oracle_grads(engine, x, ids, dout)
    _check(got, ref, "fp32")
    assert torch.equal(res.grad, dout)
    # parameter rows/columns outside the active capacity get zero gradient
    assert got["expert_gate"][4:].abs().max().item() == 0
    assert got["expert_gate"][:, :, 20:].abs().max().item() == 0
    assert got["expert_down"][:, 20:].abs().max().item() == 0


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
def test_layer_backward_active_capacity_bf16_saved(gpu, strategy):
    """bf16 at reduced active capacity above the decode sizes: the forward
    saves g|u (and h), and the dense strategy's weight gradients come from
    the flat mapped buffer as views, copied into full-size zero tensors."""
    print(f"layer backward active bf16 saved {strategy}", flush=True)
    torch.manual_seed(5)
    engine = _engine(gpu, "bf16", 8, 2, 256, 64, 128, None, strategy)
    engine.set_active_capacity(num_experts=4, expert_width=40)
    ids = torch.randint(0, 5000, (2, 150), device=gpu)              # 300 tokens > 128
    x = torch.randn(2, 150, 128, device=gpu, dtype=torch.bfloat16)
    dout = (torch.randn(2, 150, 128, device=gpu) * 0.1).to(torch.bfloat16)
    out, got = _hip_grads(engine, x, ids, dout)
    assert engine._packed.strategy == strategy
    _check(got, _oracle_grads(engine, x, ids, dout), "bf16")
    assert got["expert_gate"][4:].abs().max().item() == 0
    assert got["expert_up"][:, :, 40:].abs().max().item() == 0
    assert got["expert_down"][:, 40:].abs().max().item() == 0
    assert got["expert_down"][4:].abs().max().item() == 0


def test_layer_backward_frozen_weights_and_no_grad_x(gpu):
    """needs_input_grad: only the requested gradients are produced."""
    torch.manual_seed(4)
    engine = _engine(gpu, "bf16", 4, 2, 256, 64, 128, None, "grouped")
    for p in engine.parameters():
        p.requires_grad_(False)
    engine.expert_down.requires_grad_(True)
    ids = torch.randint(0, 5000, (1, 200), device=gpu)
    x = torch.randn(1, 200, 128, device=gpu, dtype=torch.bfloat16)
    dout = torch.randn(1, 200, 128, device=gpu, dtype=torch.bfloat16)
    out = engine(x, ids)
    out.backward(dout)
    torch.cuda.synchronize()
    ref = _oracle_grads(engine, x, ids, dout)
    assert engine.shared_gate.weight.grad is None and engine.expert_gate.grad is None
    assert _err(engine.expert_down.grad, ref["expert_down"]) <= BOUND["bf16"]


def test_c2_bf16_layer_backward_full_size(gpu):
    """C2 (bf16, 16384 tokens, Zipf ids) through autograd on the HIP backend,
    against autograd of the oracle's forward in fp32 on the GPU."""
    from complexity_amd import workloads as Wl

    print("layer backward C2 full size", flush=True)
    w = Wl.C2
    engine = Wl.build_engine(w, gpu, backend="hip")
    x = Wl.make_hidden(w).to(gpu).to(torch.bfloat16)
    ids = Wl.make_token_ids(w).to(gpu)
    dout = (torch.randn(x.shape, device=gpu) * 0.1).to(torch.bfloat16)
    _, got = _hip_grads(engine, x, ids, dout)
    ref = _oracle_grads(engine, x, ids, dout, device=gpu, dtype=torch.float32)
    _check(got, ref, "bf16")


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("tokens", [2048, 8192])
def test_c2_shape_layer_backward_mid_sizes(gpu, strategy, tokens):
    """C2's layer (bf16, Zipf ids) at 2048 and 8192 tokens through autograd,
    both routed strategies: the weight gradients' split counts and the
    persistent SwiGLU backward's grid differ from C2's 16384 tokens."""
    from dataclasses import replace

    from complexity_amd import workloads as Wl

    print(f"layer backward C2 shape {tokens} tokens {strategy}", flush=True)
    w = replace(Wl.C2, name=f"bf16_{tokens}", batch=tokens // 2048, seq=2048)
    engine = Wl.build_engine(w, gpu, backend="hip")
    engine.routed_strategy = strategy
    x = Wl.make_hidden(w).to(gpu).to(torch.bfloat16)
    ids = Wl.make_token_ids(w).to(gpu)
    dout = (torch.randn(x.shape, device=gpu, generator=torch.Generator(device=gpu).manual_seed(tokens)) *
            0.1).to(torch.bfloat16)
    _, got = _hip_grads(engine, x, ids, dout)
    assert engine._packed.strategy == strategy
    ref = _oracle_grads(engine, x, ids, dout, device=gpu, dtype=torch.float32)
    _check(got, ref, "bf16")


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
@pytest.mark.parametrize("n", [1, 5, 64, 129])
def test_layer_backward_decode_sizes(gpu, strategy, n):
    """Few tokens: the data gradient runs on the decode-shape down kernels
    (K = 2F) and most expert segments are empty."""
    print(f"layer backward decode sizes {strategy} n={n}", flush=True)
    torch.manual_seed(n)
    engine = _engine(gpu, "bf16", 4, 2, 512, 64, 256, None, strategy)
    ids = torch.randint(0, 5000, (1, n), device=gpu)
    x = torch.randn(1, n, 256, device=gpu, dtype=torch.bfloat16)
    dout = torch.randn(1, n, 256, device=gpu, dtype=torch.bfloat16)
    _, got = _hip_grads(engine, x, ids, dout)
    _check(got, _oracle_grads(engine, x, ids, dout), "bf16")


def test_c1_fp32_layer_backward_full_size(gpu):
    """C1 (fp32, 2048 tokens, multi-hash, uniform ids) through autograd."""
    from complexity_amd import workloads as Wl

    print("layer backward C1 full size", flush=True)
    w = Wl.C1
    engine = Wl.build_engine(w, gpu, backend="hip")
    x = Wl.make_hidden(w).to(gpu)
    ids = Wl.make_token_ids(w).to(gpu)
    dout = torch.randn(x.shape, device=gpu) * 0.1
    _, got = _hip_grads(engine, x, ids, dout)
    ref = _oracle_grads(engine, x, ids, dout, device=gpu, dtype=torch.float64)
    _check(got, ref, "fp32")


@pytest.mark.parametrize("strategy", ["dense", "grouped"])
def test_layer_backward_out_of_range_ids(gpu, strategy):
    torch.manual_seed(2)
    engine = _engine(gpu, "fp32", 4, 2, 128, 64, 128, None, strategy)
    ids = torch.randint(-30, 5030, (2, 90), device=gpu)
    x = torch.randn(2, 90, 128, device=gpu)
    dout = torch.randn(2, 90, 128, device=gpu)
    _, got = _hip_grads(engine, x, ids, dout)
    _check(got, _oracle_grads(engine, x, ids, dout), "fp32")
