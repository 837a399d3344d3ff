"""Each HIP kernel family against a float64 CPU reference of the same op.

Tolerances are normwise (max|got - ref| / max|ref|): 1e-5 for fp32 inputs,
1e-2 for bf16 inputs (one bf16 rounding of the output), fp8 weights are
compared against the dequantised weights at the bf16 bound.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def nerr(got, ref):
    return O.normwise_rel_err(got.double(), ref.double())


def _rand(*shape, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def test_fp8_to_bf16_conversion_is_exact_for_all_codes(gpu):
    """pack + a 1x1 identity GEMM would hide a wrong decode: check the decode
    itself through the gate/up kernel with x = unit vectors."""
    from complexity_amd import ops

    codes = torch.arange(256, dtype=torch.uint8)
    codes[0x7F] = 0
    codes[0xFF] = 0  # NaN codes are never produced by the quantiser
    H, S = 256, 128
    # gate weights: row f holds code f at column f (diagonal), up weights = 1.0 (code 0x38)
    wg = torch.zeros(S, H, dtype=torch.uint8)
    wu = torch.full((S, H), 0x38, dtype=torch.uint8)
    x = torch.zeros(H, H)
    x[torch.arange(H), torch.arange(H)] = 1.0
    # two passes cover the 256 codes with S = 128 features
    for half in range(2):
        wg.zero_()
        for f in range(S):
            wg[f, half * 128 + f] = codes[half * 128 + f]
        pg, sg = ops.pack_linear_gate_up(wg.view(torch.float8_e4m3fn).to(gpu), wu.view(torch.float8_e4m3fn).to(gpu),
                                        torch.ones(S, device=gpu), torch.ones(S, device=gpu))
        h = ops.shared_gate_up(x.to(torch.bfloat16).to(gpu), pg, sg, S).float().cpu()
        for f in range(S):
            row = half * 128 + f
            g = O.e4m3_decode_table()[int(codes[row])]
            expect = g / (1.0 + np.exp(-g)) * 1.0 if g == g else 0.0
            got = float(h[row, f])
            assert abs(got - expect) <= 2 ** -7 * abs(expect) + 1e-30, (row, got, expect)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,H,S", [(1, 64, 64), (200, 96, 160), (513, 896, 384), (64, 40, 100)])
def test_shared_gate_up(gpu, dtype, N, H, S):
    from complexity_amd import ops

    x = _rand(N, H, seed=1)
    wg, wu = _rand(S, H, scale=0.1, seed=2), _rand(S, H, scale=0.1, seed=3)
    xd = x.to(dtype)
    pg, _ = ops.pack_linear_gate_up(wg.to(dtype).to(gpu), wu.to(dtype).to(gpu))
    h = ops.shared_gate_up(xd.to(gpu), pg, None, S).cpu()
    xr, gr, ur = xd.double(), wg.to(dtype).double(), wu.to(dtype).double()
    ref = F.silu(xr @ gr.T) * (xr @ ur.T)
    assert h.shape[1] == (S + 127) // 128 * 128
    assert nerr(h[:, :S], ref) <= TOL[dtype]
    assert (h[:, S:] == 0).all()


def test_shared_gate_up_unaligned_rows(gpu):
    """x with a row stride that is not a multiple of 8 takes the scalar loads."""
    from complexity_amd import ops

    N, H, S = 77, 36, 64
    base = _rand(N, H + 3, seed=4).to(torch.bfloat16)
    x = base[:, 1 : H + 1]  # misaligned view
    wg, wu = _rand(S, H, scale=0.1, seed=5).to(torch.bfloat16), _rand(S, H, scale=0.1, seed=6).to(torch.bfloat16)
    pg, _ = ops.pack_linear_gate_up(wg.to(gpu), wu.to(gpu))
    xg = base.to(gpu)[:, 1 : H + 1]
    h = ops.shared_gate_up(xg, pg, None, S).cpu()
    ref = F.silu(x.double() @ wg.double().T) * (x.double() @ wu.double().T)
    assert nerr(h[:, :S], ref) <= 1e-2


def test_shared_gate_up_fp8_weights(gpu):
    from complexity_amd import ops

    N, H, S = 300, 256, 256
    x = _rand(N, H, seed=7).to(torch.bfloat16)
    wg, wu = _rand(S, H, scale=0.02, seed=8), _rand(S, H, scale=0.02, seed=9)
    qg, sg = O.quantize_e4m3(wg, 1)
    qu, su = O.quantize_e4m3(wu, 1)
    pg, ps = ops.pack_linear_gate_up(qg.to(gpu), qu.to(gpu), sg.to(gpu), su.to(gpu))
    h = ops.shared_gate_up(x.to(gpu), pg, ps, S).cpu()
    dg, du = O.dequantize_e4m3(qg, sg, 1).double(), O.dequantize_e4m3(qu, su, 1).double()
    ref = F.silu(x.double() @ dg.T) * (x.double() @ du.T)
    assert nerr(h[:, :S], ref) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_y,with_res", [(True, False), (True, True), (False, False)])
def test_shared_down_combine(gpu, dtype, with_y, with_res):
    from complexity_amd import ops

    N, S, H, k = 333, 320, 200, 2
    h = _rand(N, S, seed=10).to(dtype)
    wd = _rand(H, S, scale=0.05, seed=11).to(dtype)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    hpad = torch.zeros(N, (S + 127) // 128 * 128, dtype=dtype)
    hpad[:, :S] = h
    y = _rand(k * N, H, seed=12).to(dtype)
    perm = torch.randperm(k * N, generator=torch.Generator().manual_seed(13))
    res = _rand(N, H, seed=14).to(dtype)
    rw = (0.7, 0.3)
    out = ops.shared_down_combine(hpad.to(gpu), S, pd, None, H, y.to(gpu) if with_y else None,
                                  perm.to(gpu) if with_y else None, k, rw, 0.5, 2.0,
                                  res.to(gpu) if with_res else None).cpu()
    ref = 0.5 * (h.double() @ wd.double().T)
    if with_y:
        yr = y.double()
        ref = ref + 2.0 * (rw[0] * yr[perm[:N]] + rw[1] * yr[perm[N:]])
    if with_res:
        ref = ref + res.double()
    assert nerr(out, ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_combine_without_shared(gpu, dtype):
    from complexity_amd import ops

    N, H, k = 129, 72, 4
    y = _rand(k * N, H, seed=15).to(dtype)
    perm = torch.randperm(k * N, generator=torch.Generator().manual_seed(16))
    rw = (0.4, 0.3, 0.2, 0.1)
    out = ops.combine(y.to(gpu), perm.to(gpu), N, k, rw, 1.5).cpu()
    yr = y.double()
    ref = 1.5 * sum(rw[j] * yr[perm[j * N:(j + 1) * N]] for j in range(k))
    assert nerr(out, ref) <= TOL[dtype]


def _routed_ref(x, table, ids, gate, up, down, order):
    routes = O.gather_routes(table, ids)
    k, n = routes.shape
    s, _, off, _ = O.counting_partition(routes, gate.shape[0], order)
    y = torch.empty(k * n, x.shape[1], dtype=torch.float64)
    xr = x.double()
    for e in range(gate.shape[0]):
        rows = torch.from_numpy(s[off[e]:off[e + 1]])
        if rows.numel() == 0:
            continue
        xt = xr[rows % n]
        hh = F.silu(xt @ gate[e].double()) * (xt @ up[e].double())
        y[off[e]:off[e + 1]] = hh @ down[e].double()
    return y


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("E,k,H,W,n", [(4, 2, 96, 64, 700), (8, 4, 64, 12, 300), (16, 2, 128, 256, 900),
                                        (2, 1, 40, 8, 33), (4, 2, 896, 64, 2048), (16, 2, 2048, 256, 1200)])
@pytest.mark.parametrize("two_pass", [True, False])
def test_routed_experts(gpu, dtype, E, k, H, W, n, two_pass):
    from complexity_amd import ops

    table = O.route_table("token_id_multi_hash", 500, E, k, 0)
    rng = np.random.default_rng(E + k + W)
    ids = rng.integers(0, 500, n)
    x = _rand(n, H, seed=20).to(dtype)
    gate, up = _rand(E, H, W, scale=0.1, seed=21).to(dtype), _rand(E, H, W, scale=0.1, seed=22).to(dtype)
    down = _rand(E, W, H, scale=0.1, seed=23).to(dtype)
    order = O.ORDER_TOKEN
    s, inv, off, cnt = ops.route_sort(torch.from_numpy(ids).to(gpu), torch.from_numpy(table).to(gpu), E, order)
    pgu, _ = ops.pack_expert_gate_up(gate.to(gpu), up.to(gpu))
    pd, _ = ops.pack_expert_down(down.to(gpu))
    y = ops.routed_experts(x.to(gpu), s, off, E, k, pgu, None, pd, None, W, two_pass=two_pass).cpu()
    ref = _routed_ref(x, table, ids, gate, up, down, order)
    assert nerr(y, ref) <= TOL[dtype]


@pytest.mark.parametrize("two_pass", [True, False])
def test_routed_experts_fp8_and_active_slice(gpu, two_pass):
    """fp8 expert weights, packed from an active-capacity prefix view."""
    from complexity_amd import ops

    E, k, H, W, n = 16, 2, 256, 256, 1500
    Ea, Wa = 8, 128
    table = O.route_table("token_id_multi_hash", 32000, Ea, k, 0)
    ids = np.random.default_rng(3).integers(0, 32000, n)
    x = _rand(n, H, seed=30).to(torch.bfloat16)
    gate, up, down = _rand(E, H, W, scale=0.02, seed=31), _rand(E, H, W, scale=0.02, seed=32), \
        _rand(E, W, H, scale=0.02, seed=33)
    qg, sg = O.quantize_e4m3(gate, 1)
    qu, su = O.quantize_e4m3(up, 1)
    qd, sd = O.quantize_e4m3(down, 1)
    s, inv, off, cnt = ops.route_sort(torch.from_numpy(ids).to(gpu), torch.from_numpy(table).to(gpu), Ea)
    pgu, pgus = ops.pack_expert_gate_up(qg.to(gpu)[:Ea, :, :Wa], qu.to(gpu)[:Ea, :, :Wa],
                                        sg.to(gpu)[:Ea, :Wa], su.to(gpu)[:Ea, :Wa])
    pd, pds = ops.pack_expert_down(qd.to(gpu)[:Ea, :Wa, :], sd.to(gpu)[:Ea])
    y = ops.routed_experts(x.to(gpu), s, off, Ea, k, pgu, pgus, pd, pds, Wa, two_pass=two_pass).cpu()
    dg = O.dequantize_e4m3(qg, sg, 1)[:Ea, :, :Wa]
    du = O.dequantize_e4m3(qu, su, 1)[:Ea, :, :Wa]
    dd = O.dequantize_e4m3(qd, sd, 1)[:Ea, :Wa, :]
    ref = _routed_ref(x, table, ids, dg, du, dd, O.ORDER_TOKEN)
    assert nerr(y, ref) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,H,S", [(4100, 256, 3072), (16384, 896, 3072)])
def test_shared_gate_up_big_tiles(gpu, dtype, N, H, S):
    """Shapes that select the 256x256 workgroup tile (with an M tail)."""
    from complexity_amd import ops

    x = _rand(N, H, seed=40).to(dtype)
    wg, wu = _rand(S, H, scale=0.05, seed=41).to(dtype), _rand(S, H, scale=0.05, seed=42).to(dtype)
    pg, _ = ops.pack_linear_gate_up(wg.to(gpu), wu.to(gpu))
    h = ops.shared_gate_up(x.to(gpu), pg, None, S).cpu()
    rows = torch.randperm(N, generator=torch.Generator().manual_seed(1))[:512]
    rows = torch.cat([rows, torch.arange(N - 40, N)])
    xr = x[rows].double()
    ref = F.silu(xr @ wg.double().T) * (xr @ wu.double().T)
    assert nerr(h[rows, :S], ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N,S,H", [(16384, 3072, 896), (9000, 1024, 2048), (4096, 512, 896)])
def test_shared_down_combine_big_tiles(gpu, dtype, N, S, H):
    """256x224 (H = 896) and 256x256 (H = 2048) down tiles, with M tails."""
    from complexity_amd import ops

    k = 2
    h = _rand(N, S, scale=0.5, seed=43).to(dtype)
    wd = _rand(H, S, scale=0.05, seed=44).to(dtype)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    y = _rand(k * N, H, seed=45).to(dtype)
    perm = torch.randperm(k * N, generator=torch.Generator().manual_seed(46))
    hp = torch.zeros(N, (S + 127) // 128 * 128, dtype=dtype)
    hp[:, :S] = h
    out = ops.shared_down_combine(hp.to(gpu), S, pd, None, H, y.to(gpu), perm.to(gpu), k, (0.5, 0.5), 1.0,
                                  1.0).cpu()
    rows = torch.cat([torch.randperm(N, generator=torch.Generator().manual_seed(2))[:512], torch.arange(N - 40, N)])
    yr = y.double()
    ref = h[rows].double() @ wd.double().T + 0.5 * (yr[perm[rows]] + yr[perm[N + rows]])
    assert nerr(out[rows], ref) <= TOL[dtype]


@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("S", [64, 128, 192, 320])
def test_fp8_down_three_stage_ring_short_k(gpu, S, with_res):
    """The ping-pong down with e4m3 weights runs three LDS stages; K = 64,
    128, 192 and 320 give 1, 2, 3 and 5 stages, covering the prologue that
    requests fewer than three and the loop's last waits.  8197 tokens x 2048
    hidden = 33 x 8 tiles (a round and a ragged row tile); with the residual
    the LDS-tile epilogue, without it the stores from the accumulators."""
    from complexity_amd import ops

    N, H = 8197, 2048
    h = _rand(N, S, scale=0.5, seed=70 + S).to(torch.bfloat16)
    wd = _rand(H, S, scale=0.05, seed=71 + S)
    q, sc = O.quantize_e4m3(wd, 1)
    pd, ps = ops.pack_linear_down(q.to(gpu), sc.to(gpu))
    hpad = torch.zeros(N, (S + 127) // 128 * 128, dtype=torch.bfloat16)
    hpad[:, :S] = h
    res = _rand(N, H, seed=72 + S).to(torch.bfloat16)
    out = ops.shared_down_combine(hpad.to(gpu), S, pd, ps, H, None, None, 1, (1.0,), 0.5, 1.0,
                                  res.to(gpu) if with_res else None).cpu()
    ref = 0.5 * (h.double() @ O.dequantize_e4m3(q, sc, 1).double().T)
    if with_res:
        ref = ref + res.double()
    row_err = (out.double() - ref).norm(dim=1) / ref.norm(dim=1)
    assert row_err.max().item() <= TOL[torch.bfloat16], int(row_err.argmax())


@pytest.mark.parametrize("with_y,with_res", [(False, False), (False, True), (True, True)])
def test_shared_down_combine_ping_pong_every_row(gpu, with_y, with_res):
    """bf16 down at H = 896 on the ping-pong kernel (at least 256 tiles of
    256 x 256, the last column tile half zero weight rows).  Every row is
    checked against a float64 product, so a block stored at the wrong rows
    or columns, or one never stored, fails; 16384 + 37 rows leave a ragged
    last row tile.  Both epilogues: stores from the accumulators (no y, no
    residual) and the LDS tile that adds y and the residual."""
    from complexity_amd import ops

    N, S, H, k = 16384 + 37, 3072, 896, 2
    h, wd, hpad, y, perm, res = _down_case(N, S, H, k, torch.bfloat16, 60)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    rw = (0.7, 0.3)
    out = ops.shared_down_combine(hpad.to(gpu), S, pd, None, H, y.to(gpu) if with_y else None,
                                  perm.to(gpu) if with_y else None, k, rw, 0.5, 2.0,
                                  res.to(gpu) if with_res else None).cpu()
    ref = 0.5 * (h.double() @ wd.double().T)
    if with_y:
        yr = y.double()
        ref = ref + 2.0 * (rw[0] * yr[perm[:N]] + rw[1] * yr[perm[N:]])
    if with_res:
        ref = ref + res.double()
    row_err = (out.double() - ref).norm(dim=1) / ref.norm(dim=1)
    assert row_err.max().item() <= TOL[torch.bfloat16], int(row_err.argmax())
    # per 32-column block of every row tile: catches a block written to the
    # wrong place even where a row's norm would dilute it
    blk = (out.double() - ref).reshape(N, H // 32, 32).norm(dim=2) / ref.reshape(N, H // 32, 32).norm(dim=2)
    assert blk.max().item() <= 4 * TOL[torch.bfloat16]


# --------------------------------------------------------------------------- decode-shape kernels


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [1, 8, 31, 33, 64, 65, 127, 128])
def test_shared_gate_up_decode_shapes(gpu, dtype, N):
    """M <= 128 runs the split-K-across-waves kernel; K not a multiple of the
    wave split and ragged M are covered."""
    from complexity_amd import ops

    H, S = 200, 320
    x = _rand(N, H, seed=31).to(dtype)
    wg, wu = _rand(S, H, scale=0.1, seed=32).to(dtype), _rand(S, H, scale=0.1, seed=33).to(dtype)
    pg, _ = ops.pack_linear_gate_up(wg.to(gpu), wu.to(gpu))
    h = ops.shared_gate_up(x.to(gpu), pg, None, S).cpu()
    ref = F.silu(x.double() @ wg.double().T) * (x.double() @ wu.double().T)
    assert nerr(h[:, :S], ref) <= TOL[dtype]
    assert (h[:, S:] == 0).all()


@pytest.mark.parametrize("N", [1, 64, 128])
def test_shared_gate_up_decode_fp8(gpu, N):
    from complexity_amd import ops

    H, S = 2048, 384
    x = _rand(N, H, seed=34).to(torch.bfloat16)
    wg, wu = _rand(S, H, scale=0.02, seed=35), _rand(S, H, scale=0.02, seed=36)
    qg, sg = O.quantize_e4m3(wg, 1)
    qu, su = O.quantize_e4m3(wu, 1)
    pg, ps = ops.pack_linear_gate_up(qg.to(gpu), qu.to(gpu), sg.to(gpu), su.to(gpu))
    h = ops.shared_gate_up(x.to(gpu), pg, ps, S).cpu()
    dg, du = O.dequantize_e4m3(qg, sg, 1).double(), O.dequantize_e4m3(qu, su, 1).double()
    ref = F.silu(x.double() @ dg.T) * (x.double() @ du.T)
    assert nerr(h[:, :S], ref) <= 1e-2


def _down_case(N, S, H, k, dtype, seed):
    h = _rand(N, S, seed=seed).to(dtype)
    wd = _rand(H, S, scale=0.05, seed=seed + 1).to(dtype)
    hpad = torch.zeros(N, (S + 127) // 128 * 128, dtype=dtype)
    hpad[:, :S] = h
    y = _rand(k * N, H, seed=seed + 2).to(dtype)
    perm = torch.randperm(k * N, generator=torch.Generator().manual_seed(seed + 3))
    res = _rand(N, H, seed=seed + 4).to(dtype)
    return h, wd, hpad, y, perm, res


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("N", [1, 8, 64, 100, 128])
@pytest.mark.parametrize("with_y,with_res", [(True, True), (False, False)])
def test_shared_down_combine_decode_shapes(gpu, dtype, N, with_y, with_res):
    from complexity_amd import ops

    S, H, k = 3328, 896, 2
    h, wd, hpad, y, perm, res = _down_case(N, S, H, k, dtype, 40)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    rw = (0.7, 0.3)
    out = ops.shared_down_combine(hpad.to(gpu), S, pd, None, H, y.to(gpu) if with_y else None,
                                  perm.to(gpu) if with_y else None, k, rw, 0.5, 2.0,
                                  res.to(gpu) if with_res else None).cpu()
    ref = 0.5 * (h.double() @ wd.double().T)
    if with_y:
        yr = y.double()
        ref = ref + 2.0 * (rw[0] * yr[perm[:N]] + rw[1] * yr[perm[N:]])
    if with_res:
        ref = ref + res.double()
    assert nerr(out, ref) <= TOL[dtype]


def test_shared_down_combine_decode_without_workspace_uses_tile_kernel(gpu):
    """The split-K path and the tile kernel (no workspace) agree, and the
    split-K result is identical from call to call (fixed reduction order)."""
    import ctypes

    from complexity_amd import _native, ops

    N, S, H, k = 64, 3328, 896, 2
    h, wd, hpad, y, perm, res = _down_case(N, S, H, k, torch.bfloat16, 50)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    hg, yg, pg_, rg = hpad.to(gpu), y.to(gpu), perm.to(gpu), res.to(gpu)
    a = ops.shared_down_combine(hg, S, pd, None, H, yg, pg_, k, (0.5, 0.5), 1.0, 1.0, rg)
    b = ops.shared_down_combine(hg, S, pd, None, H, yg, pg_, k, (0.5, 0.5), 1.0, 1.0, rg)
    assert torch.equal(a, b)
    lib = _native.load()
    out = torch.empty(N, H, dtype=torch.bfloat16, device=gpu)
    rw = (ctypes.c_float * 4)(0.5, 0.5, 0.0, 0.0)
    st = lib.trmoe_shared_down_combine(_native.BF16, _native.BF16, hg.data_ptr(), N, S, hg.stride(0), pd.data_ptr(),
                                       None, H, yg.data_ptr(), H, pg_.data_ptr(), k,
                                       ctypes.cast(rw, ctypes.c_void_p), 1.0, 1.0, rg.data_ptr(), H,
                                       out.data_ptr(), H, None, 0,
                                       ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _native.check(st, "trmoe_shared_down_combine")
    assert nerr(a.cpu(), out.cpu()) <= 1e-2


@pytest.mark.parametrize("N", [16, 64, 128])
def test_decode_down_split_k_reduction_is_repeatable(gpu, N):
    """Decode-sized down GEMM: the split-K partials are summed in split order,
    so 40 calls in a row, every other one behind a cache-evicting write,
    give bit-identical outputs within the bf16 bound of the reference."""
    from complexity_amd import ops

    S, H, k = 3328, 896, 2
    h, wd, hpad, y, perm, res = _down_case(N, S, H, k, torch.bfloat16, 70)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    hg, yg, pg_, rg = hpad.to(gpu), y.to(gpu), perm.to(gpu), res.to(gpu)
    evict = torch.empty(1 << 28, dtype=torch.float32, device=gpu)
    outs = []
    for i in range(40):
        if i % 2:
            evict.add_(1.0)
        outs.append(ops.shared_down_combine(hg, S, pd, None, H, yg, pg_, k, (0.6, 0.4), 0.5, 2.0, rg))
    torch.cuda.synchronize()
    for i, o in enumerate(outs[1:], 1):
        assert torch.equal(o, outs[0]), f"call {i} differs from call 0"
    ref = 0.5 * (h.double() @ wd.double().T) + 2.0 * (0.6 * y.double()[perm[:N]] + 0.4 * y.double()[perm[N:]])
    ref = ref + res.double()
    assert nerr(outs[0].cpu(), ref) <= TOL[torch.bfloat16]


def test_shared_down_combine_decode_fp8(gpu):
    from complexity_amd import ops

    N, S, H = 64, 1024, 2048
    h = _rand(N, S, seed=60).to(torch.bfloat16)
    wd = _rand(H, S, scale=0.02, seed=61)
    q, s = O.quantize_e4m3(wd, 1)
    pd, ps = ops.pack_linear_down(q.to(gpu), s.to(gpu))
    out = ops.shared_down_combine(h.to(gpu), S, pd, ps, H, None, None, 2, (0.5, 0.5), 1.0, 1.0).cpu()
    ref = h.double() @ O.dequantize_e4m3(q, s, 1).double().T
    assert nerr(out, ref) <= 1e-2


@pytest.mark.parametrize("routed", [False, True])
def test_prefill_gate_up_every_row_and_repeatable_with_cold_caches(gpu, routed):
    """Regression test for an LDS race in the prefill gate|up main loop: one
    wave refilled a stage while other waves of its group could still be
    reading it, so with cold caches a few rows per call came out wrong (too
    few to move a normwise bound over sampled rows).  At the C2 shape (16384
    tokens, 256-row tiles plus the 128-row tail launch over the expert
    columns) every row is checked against a torch fp32 reference, and calls
    separated by a cache-evicting write agree bit for bit."""
    from complexity_amd import ops
    from complexity_amd import workloads as W

    w = W.C2
    eng = W.build_engine(w, gpu, backend="hip")
    p = eng._hip_packed()
    x = W.make_hidden(w).to(gpu).to(torch.bfloat16).reshape(-1, w.hidden).contiguous()
    ids = W.make_token_ids(w).to(gpu).reshape(-1).contiguous()
    table = eng._active_route_table
    rw, shared_scale, routed_scale = eng.config.route_weights, 0.5, 2.0
    S, E, Wd = p.shared_width, p.num_experts, p.expert_width
    xf = x.float()
    g = xf @ eng.shared_gate.weight.detach().float().T
    u = xf @ eng.shared_up.weight.detach().float().T
    if routed:
        F_ = p.dense_features
        ref = torch.zeros(x.shape[0], F_, device=gpu)
        ref[:, :S] = shared_scale * F.silu(g) * u
        routes = table[:, ids]  # [k, N]
        for e in range(E):
            mult = sum(routed_scale * rw[j] * (routes[j] == e).float() for j in range(routes.shape[0]))
            ge = xf @ eng.expert_gate.detach()[e].float()
            ue = xf @ eng.expert_up.detach()[e].float()
            c0 = (S + 127) // 128 * 128 + e * ((Wd + 63) // 64 * 64)  # shared block, then 64-aligned experts
            ref[:, c0:c0 + Wd] = mult[:, None] * F.silu(ge) * ue

        def call():
            return ops.dense_routed_gate_up(x, p.dense_gate_up, S, E, Wd, ids, table, rw, shared_scale, routed_scale)
    else:
        pg, _ = ops.pack_linear_gate_up(eng.shared_gate.weight.detach(), eng.shared_up.weight.detach())
        ref = F.silu(g) * u

        def call():
            return ops.shared_gate_up(x, pg, None, S)[:, :S]

    evict = torch.empty(1 << 28, dtype=torch.float32, device=gpu)  # 1 GiB: more than L2 and MALL together
    outs = []
    for _ in range(6):
        evict.add_(1.0)
        outs.append(call())
    torch.cuda.synchronize()
    first = outs[0]
    for i, o in enumerate(outs[1:], 1):
        assert torch.equal(o.view(torch.int16), first.view(torch.int16)), f"call {i} differs from call 0"
    # every row: max |h - ref| within two bf16 roundings of the row's largest value
    err = (first.float() - ref).abs().amax(1)
    scale = ref.abs().amax(1).clamp_min(1e-6)
    worst = int(torch.argmax(err / scale))
    assert float(err[worst] / scale[worst]) <= 2 ** -7, (worst, float(err[worst]), float(scale[worst]))


@pytest.mark.parametrize("nbytes,blocks", [(16, 1), (4096 + 16 * 7, 3), (18 << 20, 512)])
def test_stream_read_folds_every_word_once(gpu, nbytes, blocks):
    """The streaming-floor kernel reads each 16-byte chunk exactly once: the
    XOR of its per-workgroup words equals the XOR of all 32-bit words."""
    from complexity_amd import ops

    g = torch.Generator().manual_seed(nbytes)
    words = torch.randint(-(2 ** 31), 2 ** 31 - 1, (nbytes // 4,), generator=g, dtype=torch.int64).to(torch.int32)
    sink = torch.zeros(blocks, dtype=torch.int32, device=gpu)
    ops.stream_read(words.to(gpu), sink)
    got = 0
    for v in sink.cpu().tolist():
        got ^= v & 0xFFFFFFFF
    want = int(np.bitwise_xor.reduce(words.numpy().view(np.uint32)))
    assert got == want
