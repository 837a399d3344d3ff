"""W8A8 shared gate|up (e4m3 activations with per-token scales, e4m3 MFMA).

The reference has no fp8 path; the oracle is the engine's own weight
quantizer applied to token rows (``quantize_e4m3`` over each row) followed by
the layer's formula (``engine_forward_w8a8``), pinned in tests/test_oracle.py.

* trmoe_quantize_rows_e4m3 is byte work: codes and scales bit for bit.
* trmoe_shared_gate_up_a8 multiplies the same e4m3 values the oracle
  dequantizes, so only fp32 summation order and the bf16 rounding of h
  differ: normwise bound 1e-2.
* trmoe_shared_gate_up_a8_mx (h as block-scaled e4m3): every block's largest
  code in [224, 448] (the exponent is the smallest that fits), padding
  features code 0 / exponent 0, and the oracle's block quantizer applied to
  the same kernel's bf16 h (trmoe_shared_gate_up_a8, pinned to f64 above)
  agrees up to what bf16 rounding moves.
* trmoe_shared_down_combine_a8 on oracle-quantized h: 1e-2 against f64 on
  the dequantized values (only fp32 summation order and bf16 outputs differ).
* The C5 layer with fp8_activations True (its h block-scaled e4m3 into the
  W8A8 down) and "gate_up" (W8A8 gate|up only), full and active capacity:
  2e-2 against the W8A8 oracle of that mode and the north-star 5e-2 against
  the plain (W8A16) oracle, on sampled rows.
* C5's layer at 512, 2048 and 8192 tokens (the small e4m3 tiles, one round
  of 256 x 256): W8A16 and W8A8 with block-scaled h against their oracles.
* The CUDA_GRAPH backend with fp8_activations: replays equal the eager HIP
  layer bit for bit, and flipping the switch after capture re-captures.
* Shapes the W8A8 kernels do not take fall back (bf16 h into the W8A16 down,
  or the whole layer W8A16), checked against the oracle of the path taken.
"""

import pytest
import torch
import torch.nn.functional as F

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu


def _special_rows(k, dtype):
    """A zero row, a row with one large value and the rest in e4m3's
    subnormal range after scaling, a row holding a NaN, and a row of ties."""
    rows = torch.zeros(4, k)
    rows[1] = torch.linspace(-0.02, 0.02, k)                # / (300 / 448): subnormal and small normal codes
    rows[1, 3] = 300.0
    rows[2] = torch.linspace(-2.0, 2.0, k)
    rows[2, 5] = float("nan")
    # x / scale lands halfway between e4m3 neighbours: scale 1 (max 448),
    # values 1.0625 and 17 (ties between 1.0 / 1.125 and 16 / 18)
    rows[3, 0] = 448.0
    rows[3, 1::2] = 1.0625
    rows[3, 2::2] = -17.0
    return rows.to(dtype)


@pytest.mark.parametrize("dtype,n,k", [
    (torch.bfloat16, 1, 128), (torch.bfloat16, 300, 2048), (torch.bfloat16, 4097, 896),
    (torch.bfloat16, 33, 4096), (torch.float32, 5, 2048), (torch.float32, 64, 256),
])
def test_quantize_rows_bit_exact(gpu, dtype, n, k):
    from complexity_amd import ops

    print(f"quantize rows {dtype} {n}x{k}", flush=True)
    g = torch.Generator().manual_seed(n + k)
    x = (torch.randn(n, k, generator=g) * torch.exp2(torch.randint(-8, 8, (n, 1), generator=g).float())).to(dtype)
    x = torch.cat([x, _special_rows(k, dtype)])
    q, s = ops.quantize_rows_e4m3(x.to(gpu))
    torch.cuda.synchronize()
    ref_q, ref_s = O.quantize_e4m3(x.float(), 1)
    got, ref = q.cpu().view(torch.uint8), ref_q.view(torch.uint8)
    nan_row = n + 2
    keep = torch.ones(x.shape[0], dtype=torch.bool)
    keep[nan_row] = False
    assert torch.equal(s.cpu(), ref_s)
    assert torch.equal(got[keep], ref[keep])
    finite = ~torch.isnan(x[nan_row].float())
    assert torch.equal(got[nan_row][finite], ref[nan_row][finite])
    assert bool(((got[nan_row][~finite] & 0x7F) == 0x7F).all())


def test_quantize_rows_every_bf16_value(gpu):
    """Rows whose maximum is 448 have scale 1, so every finite bf16 value
    (clamped to +-448) is its own quotient: the conversion's rounding against
    torch's over all of them (every e4m3 value, the subnormal steps, the ties
    and both zeros)."""
    from complexity_amd import ops

    bits = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    vals = torch.where(torch.isfinite(bits), bits, torch.zeros_like(bits)).clamp(-448, 448).reshape(32, 2048)
    vals[:, 0] = 448.0
    q, s = ops.quantize_rows_e4m3(vals.to(gpu))
    torch.cuda.synchronize()
    ref_q, ref_s = O.quantize_e4m3(vals.float(), 1)
    assert torch.equal(s.cpu(), ref_s) and bool((ref_s == 1.0).all())
    assert torch.equal(q.cpu().view(torch.uint8), ref_q.view(torch.uint8))


def _engine(gpu, hidden, shared, experts=4, width=64):
    from complexity_amd.tr_hash import TRHashEngine, TRHashEngineConfig

    engine = TRHashEngine(TRHashEngineConfig(hidden_size=hidden, vocab_size=5000, num_experts=experts, top_k=2,
                                             shared_width=shared, expert_width=width,
                                             routing_strategy="token_id_multi_hash", routed_output_scale=2.0,
                                             shared_output_scale=0.5, precision="fp8", backend="hip")).to(gpu)
    engine = engine.to(torch.bfloat16)
    engine.routed_strategy = "grouped"
    engine.quantize_fp8_()
    return engine.eval()


def _deq(engine, name):
    return O.dequantize_e4m3(getattr(engine, name + "_fp8").cpu(), getattr(engine, name + "_scale").cpu(), 1)


@pytest.mark.parametrize("hidden,shared,n", [(256, 384, 300), (128, 128, 1), (2048, 5632, 4096), (896, 3072, 777)])
def test_shared_gate_up_a8(gpu, hidden, shared, n):
    """h against silu(xq Wgq^T) * (xq Wuq^T) in f64 on the same e4m3 values
    (rows sampled above 1024 tokens)."""
    from complexity_amd import ops

    print(f"gate_up a8 H={hidden} S={shared} n={n}", flush=True)
    engine = _engine(gpu, hidden, shared)
    g = torch.Generator().manual_seed(hidden + n)
    x = (torch.randn(n, hidden, generator=g) * 1.5).to(gpu, torch.bfloat16)
    packed = engine._hip_packed()
    xq, xs = ops.quantize_rows_e4m3(x)
    h = ops.shared_gate_up_a8(xq, xs, packed.shared_gate_up, packed.shared_gate_up_scale, shared)
    torch.cuda.synchronize()
    rows = torch.arange(n) if n <= 1024 else torch.randperm(n, generator=g)[:1024]
    xd = O.dequantize_e4m3(xq.cpu()[rows], xs.cpu()[rows], 1).double()
    ref = O.silu_mul(F.linear(xd, _deq(engine, "shared_gate").double()),
                     F.linear(xd, _deq(engine, "shared_up").double()))
    got = h[:, :shared].cpu()[rows].double()
    assert O.normwise_rel_err(got, ref) <= 1e-2, O.normwise_rel_err(got, ref)


@pytest.mark.parametrize("hidden,shared,n", [(256, 384, 300), (128, 300, 1), (2048, 5632, 4096), (896, 3072, 777)])
def test_shared_gate_up_a8_block_scaled_h(gpu, hidden, shared, n):
    """The block quantizer on the kernel's own h: trmoe_shared_gate_up_a8
    gives the same accumulators rounded to bf16 (its h is pinned against the
    f64 oracle by test_shared_gate_up_a8), so the codes and exponents are
    checked against the oracle's rule applied to that bf16 h: exactly, except
    where the bf16 rounding of h lands exactly on a boundary of the rule
    (a block maximum of 448 * 2^e, an e4m3 rounding midpoint), where the
    kernel's fp32 h may fall on either side."""
    from complexity_amd import ops

    print(f"gate_up a8 mx H={hidden} S={shared} n={n}", flush=True)
    engine = _engine(gpu, hidden, shared)
    g = torch.Generator().manual_seed(hidden + n + 1)
    x = (torch.randn(n, hidden, generator=g) * 1.5).to(gpu, torch.bfloat16)
    packed = engine._hip_packed()
    xq, xs = ops.quantize_rows_e4m3(x)
    hq, hs = ops.shared_gate_up_a8_mx(xq, xs, packed.shared_gate_up, packed.shared_gate_up_scale, shared)
    hb = ops.shared_gate_up_a8(xq, xs, packed.shared_gate_up, packed.shared_gate_up_scale, shared)
    torch.cuda.synchronize()
    f_pad = hq.shape[1]
    assert f_pad == -(-shared // 128) * 128 and hs.shape == (n, f_pad // 32)
    rows = torch.arange(n) if n <= 1024 else torch.randperm(n, generator=g)[:1024]
    q = hq.cpu()[rows]
    e = hs.cpu()[rows].long() - 127
    h = hb.cpu()[rows].float()
    # padding features: code 0, exponent 0
    assert bool((q.float()[:, shared:] == 0).all())
    assert bool((e[:, -(-shared // 32):] == 0).all())
    # the exponent is the smallest that fits: every block's largest code in [224, 448]
    qb = q.float().reshape(len(rows), -1, 32).abs().amax(-1)
    nz = qb > 0
    assert bool(((qb[nz] >= 224) & (qb[nz] <= 448)).all())
    _, want_e = O.quantize_blocks_e4m3(h)
    # 448 * 2^e is a bf16 number: the kernel's fp32 maximum may lie just above
    # a bf16 maximum that equals it, and then the kernel's exponent is one more
    bmax = h.abs().reshape(len(rows), -1, 32).amax(-1)
    edge = bmax == 448.0 * torch.exp2(want_e.float())
    assert bool(((e == want_e) | (edge & (e == want_e + 1))).all())

    def e4m3(v):
        return torch.where(v > 448, 448.0, torch.where(v < -448, -448.0, v)).to(torch.float8_e4m3fn)

    # codes under the kernel's own exponents.  e4m3 rounding midpoints are
    # bf16 numbers too, so bf16 h can only round differently from the
    # kernel's fp32 h where it sits exactly on one: there either neighbour
    scaled = h * torch.exp2(-e.repeat_interleave(32, dim=1).float())
    own = e4m3(scaled)
    tie = e4m3(scaled * (1 + 2.0 ** -20)).view(torch.uint8) != e4m3(scaled * (1 - 2.0 ** -20)).view(torch.uint8)
    same = q.view(torch.uint8) == own.view(torch.uint8)
    assert bool((same | tie).all())
    lo, hi = e4m3(scaled * (1 - 2.0 ** -20)).float(), e4m3(scaled * (1 + 2.0 ** -20)).float()
    assert bool((same | (q.float() == torch.minimum(lo, hi)) | (q.float() == torch.maximum(lo, hi))).all())
    got = O.dequantize_blocks_e4m3(q, e)
    assert O.normwise_rel_err(got[:, :shared].double(), h[:, :shared].double()) <= 2.0 ** -4


@pytest.mark.parametrize("hidden,shared,n,routed,residual", [
    (256, 384, 300, True, False), (128, 128, 1, False, True), (2048, 5632, 4096, True, False),
    (896, 3072, 777, True, True)])
def test_shared_down_combine_a8(gpu, hidden, shared, n, routed, residual):
    from complexity_amd import ops

    print(f"down a8 H={hidden} S={shared} n={n} routed={routed} residual={residual}", flush=True)
    engine = _engine(gpu, hidden, shared)
    packed = engine._hip_packed()
    g = torch.Generator().manual_seed(hidden + shared + n)
    h = torch.randn(n, shared, generator=g) * torch.exp2(torch.randint(-6, 6, (n, shared // 32), generator=g)
                                                         .float()).repeat_interleave(32, dim=1)
    hq, he = O.quantize_blocks_e4m3(h)
    hd = O.dequantize_blocks_e4m3(hq, he).double()
    rw = (0.6, 0.4)
    y = inv = res = None
    ref = 0.5 * (hd @ _deq(engine, "shared_down").double().T)
    if routed:
        y = torch.randn(2 * n, hidden, generator=g).to(torch.bfloat16)
        inv = torch.randperm(2 * n, generator=g).reshape(2, n)
        ref = ref + 2.0 * (rw[0] * y.double()[inv[0]] + rw[1] * y.double()[inv[1]])
    if residual:
        res = torch.randn(n, hidden, generator=g).to(torch.bfloat16)
        ref = ref + res.double()
    out = ops.shared_down_combine_a8(
        hq.to(gpu), (he + 127).to(torch.uint8).to(gpu), shared, packed.shared_down, packed.shared_down_scale, hidden,
        None if y is None else y.to(gpu), None if inv is None else inv.to(gpu), 2, rw, 0.5, 2.0,
        None if res is None else res.to(gpu))
    torch.cuda.synchronize()
    assert O.normwise_rel_err(out.cpu().double(), ref) <= 1e-2, O.normwise_rel_err(out.cpu().double(), ref)


@pytest.mark.parametrize("mode", [True, "gate_up"])
@pytest.mark.parametrize("name", ["c5_fp8_32768", "c5_fp8_32768_active_8x128"])
def test_c5_layer_with_fp8_activations(gpu, name, mode):
    """C5 (hidden 2048, shared 5632, 16 x 256 experts, 32768 tokens; the
    active variant runs 8 experts x 128 features) with fp8_activations
    against the W8A8 oracle and the plain W8A16 oracle."""
    from complexity_amd import ops
    from complexity_amd import workloads as Wl
    from complexity_amd.tr_hash import TRHashBackend

    print(f"W8A8 layer {name} mode {mode}", flush=True)
    w = Wl.WORKLOADS[name]
    engine = Wl.build_engine(w, gpu, backend="hip")
    engine.fp8_activations = mode
    x = Wl.make_hidden(w).to(gpu).to(torch.bfloat16)
    ids = Wl.make_token_ids(w).to(gpu)
    calls = []
    names = ("shared_gate_up_a8_mx", "shared_down_combine_a8", "shared_gate_up_a8")
    saved = {k: getattr(ops, k) for k in names}

    def counted(k):
        def f(*a, **kw):
            calls.append(k)
            return saved[k](*a, **kw)
        return f

    for k in names:
        setattr(ops, k, counted(k))
    try:
        with torch.no_grad():
            out = engine(x, ids)
            want = ["shared_gate_up_a8_mx", "shared_down_combine_a8"] if mode is True else ["shared_gate_up_a8"]
            assert calls == want
            engine.fp8_activations = False
            plain = engine(x, ids)
            assert calls == want
    finally:
        for k in names:
            setattr(ops, k, saved[k])
    torch.cuda.synchronize()
    assert engine.last_backend.selected is TRHashBackend.HIP
    rows = torch.randperm(w.tokens, generator=torch.Generator().manual_seed(2))[:1024]
    xr = x.reshape(-1, w.hidden)[rows.to(gpu)].float().cpu()
    ir = ids.reshape(-1)[rows.to(gpu)].cpu()
    p = {n: _deq(engine, n) for n in ("expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up",
                                      "shared_down")}
    cfg = engine.config
    kw = dict(route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale,
              routed_scale=cfg.routed_output_scale, active_experts=w.active_experts,
              active_width=w.active_width)
    table = engine._active_route_table.cpu()
    ref8 = O.engine_forward_w8a8(xr, ir, table, p, h_blocks=mode is True, **kw)
    ref = O.engine_forward(xr, ir, table, p, **kw)
    got = out.reshape(-1, w.hidden)[rows.to(gpu)].float().cpu()
    e8, e = O.normwise_rel_err(got, ref8), O.normwise_rel_err(got, ref)
    print(f"C5 W8A8 ({mode}): {e8:.3e} vs the W8A8 oracle, {e:.3e} vs the W8A16 oracle", flush=True)
    assert e8 <= 2e-2
    assert e <= 5e-2
    # the flag changes only the shared gate|up: without it the layer is the W8A16 one
    assert O.normwise_rel_err(plain.reshape(-1, w.hidden)[rows.to(gpu)].float().cpu(), ref) <= 5e-2


@pytest.mark.parametrize("tokens", [512, 2048, 8192])
def test_fp8_layer_between_decode_and_c5(gpu, tokens):
    """C5's layer (e4m3 weights, hidden 2048, shared 5632, 16 x 256 experts)
    at token counts where the launch shapes change: 64-row tiles for e4m3
    weights where larger ones leave CUs idle (512, 2048), one round or more
    of 256 x 256 tiles (8192).  W8A16 against the dequantised-weight oracle,
    then W8A8 with block-scaled h against the W8A8 oracle, on the same engine
    and inputs (up to 1024 sampled rows).  e4m3 weights take the grouped
    strategy (the dense-routed one needs bf16/f32 weights)."""
    from dataclasses import replace

    from complexity_amd import workloads as Wl

    print(f"fp8 layer {tokens} tokens", flush=True)
    w = replace(Wl.C5, name=f"fp8_{tokens}", batch=max(1, tokens // 2048), seq=min(tokens, 2048))
    assert w.tokens == tokens
    engine = Wl.build_engine(w, gpu, backend="hip")
    x = Wl.make_hidden(w).to(gpu).to(torch.bfloat16)
    ids = Wl.make_token_ids(w).to(gpu)
    with torch.no_grad():
        out16 = engine(x, ids)
        engine.fp8_activations = True
        out8 = engine(x, ids)
    torch.cuda.synchronize()
    assert engine._packed.strategy == "grouped"
    rows = torch.randperm(tokens, generator=torch.Generator().manual_seed(3))[:1024]
    xr = x.reshape(-1, w.hidden)[rows.to(gpu)].float().cpu()
    ir = ids.reshape(-1)[rows.to(gpu)].cpu()
    p = {n: _deq(engine, n) for n in ("expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up",
                                      "shared_down")}
    cfg = engine.config
    kw = dict(route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale,
              routed_scale=cfg.routed_output_scale)
    table = engine._active_route_table.cpu()
    ref = O.engine_forward(xr, ir, table, p, **kw)
    ref8 = O.engine_forward_w8a8(xr, ir, table, p, h_blocks=True, **kw)
    e16 = O.normwise_rel_err(out16.reshape(-1, w.hidden)[rows.to(gpu)].float().cpu(), ref)
    e8 = O.normwise_rel_err(out8.reshape(-1, w.hidden)[rows.to(gpu)].float().cpu(), ref8)
    print(f"fp8 {tokens}: W8A16 {e16:.3e}, W8A8 {e8:.3e}", flush=True)
    assert e16 <= 5e-2
    assert e8 <= 2e-2


def test_graph_backend_with_fp8_activations(gpu):
    """CUDA_GRAPH over an e4m3 layer above decode sizes (256 tokens): replays
    with eager work between them equal the eager HIP layer with the same
    switch, before and after fp8_activations is changed on the captured
    engine (the runner captures again), and the replays of the three modes
    differ (the switch reached the captured kernels)."""
    from complexity_amd.tr_hash import GraphBucket, TRHashEngine, TRHashEngineConfig

    torch.manual_seed(19)
    common = dict(hidden_size=256, vocab_size=997, num_experts=4, top_k=2, shared_width=384, expert_width=64,
                  precision="fp8", phase="inference", routing_strategy="token_id_multi_hash")
    graph = TRHashEngine(TRHashEngineConfig(**common, backend="cuda_graph",
                                            graph_buckets=(GraphBucket(2, 128),))).to(gpu).to(torch.bfloat16)
    eager = TRHashEngine(TRHashEngineConfig(**common, backend="hip")).to(gpu).to(torch.bfloat16)
    eager.load_state_dict(graph.state_dict())
    for e in (graph, eager):
        e.routed_strategy = "grouped"
        e.quantize_fp8_()
        e.eval()
    results = {}
    with torch.no_grad():
        for flag in (True, False, "gate_up", True):
            graph.fp8_activations = eager.fp8_activations = flag
            for step in range(3):
                g = torch.Generator().manual_seed(step)
                ids = torch.randint(0, 997, (2, 100 + 14 * step), generator=g).to(gpu)
                x = torch.randn(2, 100 + 14 * step, 256, generator=g).to(gpu, torch.bfloat16)
                got = graph(x, ids)
                _ = torch.randn(1 << 16, device=gpu).sum()  # unrelated eager work
                torch.cuda.synchronize()
                want = eager(x, ids)
                assert torch.equal(got, want), (flag, step)
                results[(flag, step)] = got
    assert not torch.equal(results[(True, 0)], results[(False, 0)])
    assert not torch.equal(results[(True, 0)], results[("gate_up", 0)])


@pytest.mark.parametrize("hidden,shared,want", [
    (256, 300, ["shared_gate_up_a8"]),                                 # S % 128 != 0: bf16 h, W8A16 down
    (192, 384, []),                                                    # hidden % 128 != 0: W8A16
    (256, 384, ["shared_gate_up_a8_mx", "shared_down_combine_a8"]),
])
def test_fp8_activations_falls_back_by_shape(gpu, hidden, shared, want):
    """fp8_activations=True takes the W8A8 kernels the shapes allow, and the
    output matches the oracle of the path taken (2e-2)."""
    from complexity_amd import ops

    print(f"W8A8 fallback H={hidden} S={shared}", flush=True)
    engine = _engine(gpu, hidden, shared)
    engine.fp8_activations = True
    g = torch.Generator().manual_seed(hidden + shared)
    x = torch.randn(2, 150, hidden, generator=g).to(gpu, torch.bfloat16)
    ids = torch.randint(0, 5000, (2, 150), generator=g).to(gpu)
    names = ("shared_gate_up_a8_mx", "shared_down_combine_a8", "shared_gate_up_a8")
    saved = {k: getattr(ops, k) for k in names}
    calls = []

    def counted(k):
        def f(*a, **kw):
            calls.append(k)
            return saved[k](*a, **kw)
        return f

    for k in names:
        setattr(ops, k, counted(k))
    try:
        with torch.no_grad():
            out = engine(x, ids)
    finally:
        for k in names:
            setattr(ops, k, saved[k])
    torch.cuda.synchronize()
    assert calls == want
    p = {n: _deq(engine, n) for n in ("expert_gate", "expert_up", "expert_down", "shared_gate", "shared_up",
                                      "shared_down")}
    cfg = engine.config
    kw = dict(route_weights=cfg.route_weights, shared_scale=cfg.shared_output_scale,
              routed_scale=cfg.routed_output_scale)
    xr, ir, table = x.float().cpu(), ids.cpu(), engine._active_route_table.cpu()
    if want:
        ref = O.engine_forward_w8a8(xr, ir, table, p, h_blocks=len(want) == 2, **kw)
    else:
        ref = O.engine_forward(xr, ir, table, p, **kw)
    assert O.normwise_rel_err(out.float().cpu(), ref) <= 2e-2, O.normwise_rel_err(out.float().cpu(), ref)
