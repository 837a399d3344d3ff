"""Pin the CPU oracle: golden vectors from the reference, closed forms, brute force.

These run without a GPU.  The oracle is the checker of every GPU parity test,
so each of its functions is checked here by something other than a retyped
copy of itself.
"""

import ctypes
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import trmoe_oracle as O

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"


def _digest(table):
    return hashlib.sha256(np.ascontiguousarray(table, dtype=np.int64).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def coracle():
    lib_path = ROOT / "oracle" / "lib" / "liboracle_route.so"
    if not lib_path.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "-s"], check=True)
    lib = ctypes.CDLL(str(lib_path))
    lib.oracle_mix32.restype = ctypes.c_uint32
    lib.oracle_mix32.argtypes = [ctypes.c_uint32]
    lib.oracle_multi_hash_table.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
                                            ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]
    lib.oracle_partition.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def c_partition(lib, routes, E, order):
    k, n = routes.shape
    r = np.ascontiguousarray(routes, dtype=np.int64)
    s = np.empty(k * n, np.int64)
    inv = np.empty(k * n, np.int64)
    off = np.empty(E + 1, np.int32)
    cnt = np.empty(E, np.int32)
    st = lib.oracle_partition(r.ctypes.data, n, k, E, order, s.ctypes.data, inv.ctypes.data, off.ctypes.data,
                              cnt.ctypes.data)
    assert st == 0
    return s, inv, off, cnt


# ---------------------------------------------------------------------------
# mix32 / route tables
# ---------------------------------------------------------------------------

def test_mix32_inverts_through_published_lowbias32_inverse():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.integers(0, 2**32, 100000, dtype=np.uint64),
                        np.array([0, 1, 2**31, 2**32 - 1], dtype=np.uint64)])
    assert np.array_equal(O.mix32_inverse(O.mix32(v)), v)
    assert int(O.mix32(np.array([0], dtype=np.uint64))[0]) == 0


def test_c_and_numpy_mix32_agree(coracle):
    rng = np.random.default_rng(1)
    for v in rng.integers(0, 2**32, 2000, dtype=np.uint64):
        assert coracle.oracle_mix32(int(v)) == int(O.mix32(np.array([v]))[0])


def test_every_reference_route_digest():
    data = json.loads((GOLDEN / "route_digests.json").read_text())
    assert data["route_seed"] == O.DEFAULT_ROUTE_SEED
    for case in data["cases"]:
        table = O.route_table(case["strategy"], case["vocab_size"], case["num_experts"], case["top_k"],
                              case["layer_index"], hash_count=case["hash_count"])
        assert table[:, :32].tolist() == case["head"], case
        assert _digest(table) == case["sha256"], case


@pytest.mark.parametrize("experts", [4, 8, 16])
def test_full_v32000_tables_match_reference_and_c_oracle(coracle, experts):
    golden = np.load(GOLDEN / "route_tables_v32000.npz")[f"multi_e{experts}_l0"].astype(np.int64)
    numpy_table = O.multi_hash_table(32000, experts, 2, 0)
    c_table = np.empty((2, 32000), np.int64)
    assert coracle.oracle_multi_hash_table(32000, experts, 2, 0, O.DEFAULT_ROUTE_SEED, 2,
                                           c_table.ctypes.data) == 0
    assert np.array_equal(numpy_table, golden)
    assert np.array_equal(c_table, golden)


def test_multi_hash_has_no_score_ties_at_measured_shapes():
    """top-k order then never depends on a tie-break rule."""
    for experts in (4, 8, 16):
        for layer in (0, 7, 15):
            s = np.sort(O.multi_hash_scores(32000, experts, layer), axis=1)
            assert not (s[:, 1:] == s[:, :-1]).any()


def test_route_table_invariants_from_reference_tests():
    """tests/test_tr_hash_engine.py:51-90 on the oracle: distinct and balanced."""
    for strategy, tol in (("modulo_cyclic", 1), ("token_id_balanced_hash", 1),
                          ("token_id_affine_hash", 80), ("token_id_multi_hash", 80)):
        for experts, k in ((2, 1), (4, 2), (8, 4), (16, 4)):
            t = O.route_table(strategy, 997, experts, k, 3)
            assert all(len(set(col)) == k for col in t.T.tolist())
            for row in t:
                c = np.bincount(row, minlength=experts)
                assert c.max() - c.min() <= tol


def test_pair_metadata_matches_reference_and_round_trips():
    z = np.load(GOLDEN / "pair_codes_v997.npz")
    for key in [k for k in z.files if k.endswith("_codes")]:
        stem = key[: -len("_codes")]
        routes = z[stem + "_routes"].astype(np.int64)
        experts = int(stem.rsplit("_e", 1)[1])
        codes, pairs = O.pair_metadata(routes, experts)
        assert np.array_equal(codes, z[key])
        assert np.array_equal(pairs, z[stem + "_pairs"])
        # decode by the definition: pair index + swap bit
        swap_bit = 0x8 if len(pairs) <= 8 else 0x20
        idx = codes & (swap_bit - 1)
        sw = (codes & swap_bit) != 0
        dec0 = np.where(sw, pairs[idx, 1], pairs[idx, 0])
        dec1 = np.where(sw, pairs[idx, 0], pairs[idx, 1])
        assert np.array_equal(np.stack([dec0, dec1]), routes)


# ---------------------------------------------------------------------------
# counting partition
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("order", [O.ORDER_TOKEN, O.ORDER_ASSIGNMENT])
@pytest.mark.parametrize("experts,k", [(1, 1), (2, 1), (4, 2), (8, 2), (8, 4), (16, 4), (16, 2)])
def test_partition_brute_force_numpy_and_c(coracle, order, experts, k):
    rng = np.random.default_rng(experts * 10 + k + 100 * order)
    table = O.route_table("token_id_multi_hash" if experts > 1 else "modulo_cyclic", 257, experts, k, 1)
    for n in (0, 1, 7, 64, 300):
        ids = rng.integers(-5, 270, n)  # includes out-of-range ids: clamped
        routes = O.gather_routes(table, ids)
        s, inv, off, cnt = O.counting_partition(routes, experts, order)
        assert np.array_equal(s, O.brute_force_partition(routes, experts, order))
        cs, cinv, coff, ccnt = c_partition(coracle, routes, experts, order)
        assert np.array_equal(s, cs) and np.array_equal(inv, cinv)
        assert np.array_equal(off, coff) and np.array_equal(cnt, ccnt)
        # invariants: permutation, inverse, histogram, segment membership, order
        assert np.array_equal(np.sort(s), np.arange(k * n))
        assert np.array_equal(inv[s], np.arange(k * n))
        flat = routes.reshape(-1)
        assert np.array_equal(cnt, np.bincount(flat, minlength=experts))
        for e in range(experts):
            seg = s[off[e]:off[e + 1]]
            assert (flat[seg] == e).all()
            key = seg % max(n, 1) if order == O.ORDER_TOKEN else seg
            assert (np.diff(key) > 0).all()


@pytest.mark.parametrize("order", [O.ORDER_TOKEN, O.ORDER_ASSIGNMENT])
@pytest.mark.parametrize("experts,k", [(2, 2), (4, 4), (8, 2), (16, 4)])
def test_partition_with_repeated_experts_per_token(coracle, order, experts, k):
    """Tables whose slots may name one expert twice for a token (a loaded
    table need not be distinct): every assignment keeps its own row, and the
    token order breaks (expert, token) ties by slot."""
    rng = np.random.default_rng(experts * 31 + k + order)
    for n in (1, 5, 64, 300):
        routes = rng.integers(0, experts, (k, n)).astype(np.int64)
        routes[:, 0] = routes[0, 0]   # token 0: every slot the same expert
        s, inv, off, cnt = O.counting_partition(routes, experts, order)
        assert np.array_equal(s, O.brute_force_partition(routes, experts, order))
        cs, cinv, coff, ccnt = c_partition(coracle, routes, experts, order)
        assert np.array_equal(s, cs) and np.array_equal(inv, cinv)
        assert np.array_equal(off, coff) and np.array_equal(cnt, ccnt)
        assert np.array_equal(np.sort(s), np.arange(k * n))
        assert np.array_equal(inv[s], np.arange(k * n))
        flat = routes.reshape(-1)
        for e in range(experts):
            seg = s[off[e]:off[e + 1]]
            assert (flat[seg] == e).all()
            key = (seg % n) * k + seg // n if order == O.ORDER_TOKEN else seg
            assert (np.diff(key) > 0).all()


def test_token_and_assignment_orders_differ_but_share_offsets():
    table = O.route_table("token_id_multi_hash", 1000, 4, 2, 0)
    ids = np.arange(0, 1000, 3)
    routes = O.gather_routes(table, ids)
    a = O.counting_partition(routes, 4, O.ORDER_TOKEN)
    b = O.counting_partition(routes, 4, O.ORDER_ASSIGNMENT)
    assert np.array_equal(a[2], b[2]) and np.array_equal(a[3], b[3])
    assert not np.array_equal(a[0], b[0])


# ---------------------------------------------------------------------------
# floating-point layer
# ---------------------------------------------------------------------------

def _params(E, H, W, S, seed=0, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    p = {
        "expert_gate": torch.randn(E, H, W, generator=g, dtype=dtype) * 0.3,
        "expert_up": torch.randn(E, H, W, generator=g, dtype=dtype) * 0.3,
        "expert_down": torch.randn(E, W, H, generator=g, dtype=dtype) * 0.3,
    }
    if S:
        p["shared_gate"] = torch.randn(S, H, generator=g, dtype=dtype) * 0.3
        p["shared_up"] = torch.randn(S, H, generator=g, dtype=dtype) * 0.3
        p["shared_down"] = torch.randn(H, S, generator=g, dtype=dtype) * 0.3
    return p


@pytest.mark.parametrize("E,k,S,weights,scales", [
    (2, 1, 12, (1.0,), (1.0, 1.0)),
    (4, 2, 12, (0.5, 0.5), (1.0, 2.0)),
    (4, 2, 0, (0.7, 0.3), (0.5, 1.0)),
    (8, 4, 12, (0.4, 0.2, 0.2, 0.2), (1.0, 1.0)),
    (16, 4, 12, (0.25,) * 4, (1.0, 1.0)),
])
def test_masked_dense_matches_token_loop(E, k, S, weights, scales):
    """engine.py:66-104 vs the reference test's token-by-token loop."""
    H, W, V = 8, 4, 101
    p = _params(E, H, W, S)
    table = torch.from_numpy(O.route_table("token_id_multi_hash", V, E, k, 0))
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 5, H, generator=g, dtype=torch.float64)
    ids = torch.randint(-3, V + 3, (2, 5), generator=g)
    a = O.engine_forward(x, ids, table, p, route_weights=weights, shared_scale=scales[0],
                         routed_scale=scales[1])
    b = O.naive_engine_output(x, ids, table, p, route_weights=weights, shared_scale=scales[0],
                              routed_scale=scales[1])
    assert torch.allclose(a, b, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("E,k", [(4, 2), (8, 4)])
def test_masked_dense_sums_repeated_slots_like_the_token_loop(E, k):
    """A table whose slots repeat an expert for some tokens: the masked
    formula's weight sum_j w_j [route_j == e] (engine.py:94) equals the token
    loop's one term per slot."""
    H, W, V, S = 8, 4, 53, 6
    p = _params(E, H, W, S, seed=4)
    rng = np.random.default_rng(E + k)
    table = torch.from_numpy(rng.integers(0, E, (k, V)).astype(np.int64))
    table[:, :5] = table[0, :5]     # ids 0..4: every slot the same expert
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 7, H, generator=g, dtype=torch.float64)
    ids = torch.randint(0, V, (3, 7), generator=g)
    ids[0, :5] = torch.arange(5)
    weights = tuple(np.linspace(1.0, 2.0, k) / np.linspace(1.0, 2.0, k).sum())
    a = O.engine_forward(x, ids, table, p, route_weights=weights, routed_scale=2.0)
    b = O.naive_engine_output(x, ids, table, p, route_weights=weights, routed_scale=2.0)
    assert torch.allclose(a, b, atol=1e-12, rtol=1e-12)


def test_shared_swiglu_matches_explicit_formula():
    H, S = 6, 10
    p = _params(1, H, 4, S)
    x = torch.randn(7, H, dtype=torch.float64)
    got = O.shared_swiglu(x, p["shared_gate"], p["shared_up"], p["shared_down"])
    for t in range(7):
        g = sum(p["shared_gate"][:, i] * x[t, i] for i in range(H))
        u = sum(p["shared_up"][:, i] * x[t, i] for i in range(H))
        h = g / (1 + torch.exp(-g)) * u
        ref = torch.stack([sum(p["shared_down"][c, j] * h[j] for j in range(S)) for c in range(H)])
        assert torch.allclose(got[t], ref, atol=1e-12)


def test_active_capacity_slices_prefix():
    H, W, S, V = 8, 6, 0, 97
    p = _params(8, H, W, S)
    table4 = torch.from_numpy(O.route_table("token_id_multi_hash", V, 4, 2, 0))
    x = torch.randn(1, 9, H, dtype=torch.float64)
    ids = torch.arange(9).view(1, 9)
    full = {k2: v for k2, v in p.items()}
    got = O.engine_forward(x, ids, table4, full, route_weights=(0.5, 0.5), active_experts=4, active_width=3)
    sliced = {"expert_gate": p["expert_gate"][:4, :, :3], "expert_up": p["expert_up"][:4, :, :3],
              "expert_down": p["expert_down"][:4, :3, :]}
    ref = O.naive_engine_output(x, ids, table4, sliced, route_weights=(0.5, 0.5))
    assert torch.allclose(got, ref, atol=1e-12)


def test_e4m3_decode_table_matches_torch_float8():
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).to(torch.float64).numpy()
    mine = O.e4m3_decode_table()
    nan = np.isnan(mine)
    assert np.array_equal(nan, np.isnan(ref))
    assert np.array_equal(mine[~nan], ref[~nan])
    assert mine[0x7E] == 448.0 and mine[0x01] == 2.0 ** -9


def test_quantize_e4m3_scale_and_error_bound():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(3, 64, 16, generator=g) * 0.02
    q, s = O.quantize_e4m3(w, 1)
    assert s.shape == (3, 16)
    deq = O.dequantize_e4m3(q, s, 1)
    assert torch.allclose(w.abs().amax(dim=1), deq.abs().amax(dim=1), rtol=1e-6, atol=0)
    # e4m3 has a 3-bit mantissa: relative rounding error <= 2^-4 for normal values
    rel = ((deq - w).abs() / w.abs().clamp_min(1e-30))
    normal = w.abs() >= s.unsqueeze(1) * 2.0 ** -6
    assert rel[normal].max() <= 2.0 ** -4 + 1e-6


# --------------------------------------------------------------------------- backward


def _tiny_layer(seed, E=3, H=6, S=5, W=4, k=2, n=7, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    params = {
        "expert_gate": torch.randn(E, H, W, generator=g, dtype=dtype) * 0.5,
        "expert_up": torch.randn(E, H, W, generator=g, dtype=dtype) * 0.5,
        "expert_down": torch.randn(E, W, H, generator=g, dtype=dtype) * 0.5,
    }
    if S:
        params["shared_gate"] = torch.randn(S, H, generator=g, dtype=dtype) * 0.5
        params["shared_up"] = torch.randn(S, H, generator=g, dtype=dtype) * 0.5
        params["shared_down"] = torch.randn(H, S, generator=g, dtype=dtype) * 0.5
    x = torch.randn(1, n, H, generator=g, dtype=dtype)
    ids = torch.randint(0, 50, (1, n), generator=g)
    table = torch.from_numpy(O.multi_hash_table(50, E, k, 0))
    dout = torch.randn(1, n, H, generator=g, dtype=dtype)
    return x, ids, table, params, dout


@pytest.mark.parametrize("S,active", [(5, None), (0, None), (5, (2, 3))])
def test_engine_backward_matches_central_differences(S, active):
    """Directional derivatives of <engine_forward, dout> by central differences
    in f64 pin every gradient engine_backward returns (names, shapes, scales)."""
    x, ids, table, params, dout = _tiny_layer(7, S=S)
    kw = dict(route_weights=(0.7, 0.3), shared_scale=1.5, routed_scale=2.0)
    if active:
        kw.update(active_experts=active[0], active_width=active[1])
        table = torch.from_numpy(O.multi_hash_table(50, active[0], 2, 0))
    grads = O.engine_backward(x, ids, table, params, dout, **kw)

    def loss(xx, pp):
        return float((O.engine_forward(xx, ids, table, pp, **kw) * dout).sum())

    g = torch.Generator().manual_seed(11)
    eps = 1e-6
    for name in ["x", *params]:
        base = x if name == "x" else params[name]
        for _ in range(3):
            v = torch.randn(base.shape, generator=g, dtype=base.dtype)
            plus = {**params}
            minus = {**params}
            if name == "x":
                lp, lm = loss(x + eps * v, params), loss(x - eps * v, params)
            else:
                plus[name], minus[name] = base + eps * v, base - eps * v
                lp, lm = loss(x, plus), loss(x, minus)
            fd = (lp - lm) / (2 * eps)
            an = float((grads[name] * v).sum())
            assert abs(fd - an) <= 1e-6 * max(1.0, abs(fd)), (name, fd, an)
    if active:
        E, W = active
        assert grads["expert_gate"][E:].abs().max() == 0 and grads["expert_gate"][:, :, W:].abs().max() == 0
        assert grads["expert_down"][E:].abs().max() == 0 and grads["expert_down"][:, W:].abs().max() == 0


def test_swiglu_backward_closed_form_matches_autograd():
    g = torch.Generator().manual_seed(5)
    R, H, F_ = 9, 6, 7
    x = torch.randn(R, H, generator=g, dtype=torch.float64)
    dout = torch.randn(R, H, generator=g, dtype=torch.float64)
    wg = torch.randn(F_, H, generator=g, dtype=torch.float64, requires_grad=True)
    wu = torch.randn(F_, H, generator=g, dtype=torch.float64)
    wd = torch.randn(H, F_, generator=g, dtype=torch.float64)
    mult = torch.rand(R, F_, generator=g, dtype=torch.float64)
    gate = (x @ wg.T).detach().requires_grad_(True)
    up = (x @ wu.T).detach().requires_grad_(True)
    h = mult * torch.nn.functional.silu(gate) * up
    y = h @ wd.T
    dg_ref, du_ref = torch.autograd.grad(y, [gate, up], grad_outputs=dout)
    dg, du, hm = O.swiglu_backward(x, dout, wg.detach(), wu, wd, mult)
    torch.testing.assert_close(dg, dg_ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(du, du_ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(hm, h.detach(), rtol=1e-12, atol=1e-12)


# --------------------------------------------------------------------------- RMSNorm (F2)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_rms_norm_matches_torch_rms_norm(dtype):
    """The oracle's restatement of norms.py:53-55 against torch's own
    implementation of the same normalisation."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(37, 96, generator=g, dtype=dtype) * 3.0
    w = torch.rand(96, generator=g, dtype=dtype) + 0.5
    ref = F.rms_norm(x, (96,), weight=w, eps=1e-6)
    assert torch.allclose(O.rms_norm(x, w, 1e-6), ref, rtol=1e-6 if dtype == torch.float64 else 1e-5, atol=0)


def test_rms_norm_constant_rows_closed_form():
    """A row of constant c normalises to sign(c) * weight (up to eps)."""
    w = torch.linspace(0.5, 2.0, 64, dtype=torch.float64)
    x = torch.tensor([[2.5] * 64, [-0.75] * 64], dtype=torch.float64)
    y = O.rms_norm(x, w, 0.0)
    assert torch.allclose(y[0], w, atol=1e-12)
    assert torch.allclose(y[1], -w, atol=1e-12)


@pytest.mark.parametrize("eps", [1e-6, 0.5])
def test_rms_norm_gradients_match_central_differences(eps):
    """The RMSNorm kernels' backward is checked against autograd of the
    oracle; that autograd is pinned here by central differences of
    <rms_norm(x, w), dout> in f64, entry by entry in x and w (a large eps
    keeps its term visible)."""
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(3, 8, generator=g, dtype=torch.float64) * 2.0).requires_grad_(True)
    w = (torch.rand(8, generator=g, dtype=torch.float64) + 0.5).requires_grad_(True)
    dout = torch.randn(3, 8, generator=g, dtype=torch.float64)
    gx, gw = torch.autograd.grad((O.rms_norm(x, w, eps) * dout).sum(), (x, w))

    def f(xv, wv):
        return float((O.rms_norm(xv, wv, eps) * dout).sum())

    h = 1e-6
    with torch.no_grad():
        for t, grad in ((x, gx), (w, gw)):
            flat, gflat = t.view(-1), grad.reshape(-1)
            for i in range(flat.numel()):
                keep = float(flat[i])
                flat[i] = keep + h
                up = f(x, w)
                flat[i] = keep - h
                down = f(x, w)
                flat[i] = keep
                assert abs((up - down) / (2 * h) - float(gflat[i])) <= 1e-7 * max(1.0, abs(float(gflat[i])))


def test_norm_residual_oracle_composes():
    """engine_forward_norm_residual is x + engine_forward(rms_norm(x))."""
    g = torch.Generator().manual_seed(3)
    H, S, E, W, V = 32, 48, 4, 8, 50
    params = {
        "shared_gate": torch.randn(S, H, generator=g) * 0.1, "shared_up": torch.randn(S, H, generator=g) * 0.1,
        "shared_down": torch.randn(H, S, generator=g) * 0.1,
        "expert_gate": torch.randn(E, H, W, generator=g) * 0.1, "expert_up": torch.randn(E, H, W, generator=g) * 0.1,
        "expert_down": torch.randn(E, W, H, generator=g) * 0.1,
    }
    table = torch.as_tensor(O.multi_hash_table(V, E, 2, 0))
    x = torch.randn(2, 5, H, generator=g)
    ids = torch.randint(0, V, (2, 5), generator=g)
    nw = torch.rand(H, generator=g) + 0.5
    got = O.engine_forward_norm_residual(x, ids, table, params, nw, 1e-6, route_weights=(0.6, 0.4))
    xn = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * nw
    want = x + O.engine_forward(xn, ids, table, params, route_weights=(0.6, 0.4))
    assert torch.allclose(got, want, atol=1e-6)


# --------------------------------------------------------------------------- W8A8 (e4m3 activations)


def _w8a8_params(g, H=64, S=96, E=4, W=16):
    return {
        "shared_gate": torch.randn(S, H, generator=g) * 0.1, "shared_up": torch.randn(S, H, generator=g) * 0.1,
        "shared_down": torch.randn(H, S, generator=g) * 0.1,
        "expert_gate": torch.randn(E, H, W, generator=g) * 0.1, "expert_up": torch.randn(E, H, W, generator=g) * 0.1,
        "expert_down": torch.randn(E, W, H, generator=g) * 0.1,
    }


def test_w8a8_oracle_is_exact_on_representable_rows():
    """Rows of e4m3 grid values times 2^j whose maximum magnitude is 448 * 2^j
    quantize exactly (scale 2^j), so the W8A8 forward equals the plain one."""
    g = torch.Generator().manual_seed(21)
    params = _w8a8_params(g)
    grid = torch.from_numpy(O.e4m3_decode_table()).float()
    grid = grid[torch.isfinite(grid)]
    rows = grid[torch.randint(0, grid.numel(), (10, 64), generator=g)]
    rows[:, 0] = 448.0
    x = rows * torch.exp2(torch.randint(-12, -6, (10, 1), generator=g).float())
    ids = torch.randint(0, 50, (10,), generator=g)
    table = torch.from_numpy(O.multi_hash_table(50, 4, 2, 0))
    kw = dict(route_weights=(0.5, 0.5), shared_scale=0.7, routed_scale=1.3)
    assert torch.equal(O.engine_forward_w8a8(x, ids, table, params, **kw), O.engine_forward(x, ids, table, params, **kw))


def test_w8a8_oracle_quantizes_the_shared_branch_only():
    g = torch.Generator().manual_seed(22)
    params = _w8a8_params(g)
    x = torch.randn(40, 64, generator=g)
    ids = torch.randint(0, 50, (40,), generator=g)
    table = torch.from_numpy(O.multi_hash_table(50, 4, 2, 0))
    kw = dict(route_weights=(0.5, 0.5), shared_scale=0.7, routed_scale=1.3)
    no_shared = {k: v for k, v in params.items() if not k.startswith("shared_")}
    assert torch.equal(O.engine_forward_w8a8(x, ids, table, no_shared, **kw),
                       O.engine_forward(x, ids, table, no_shared, **kw))
    ref = O.engine_forward(x, ids, table, params, **kw)
    got = O.engine_forward_w8a8(x, ids, table, params, **kw)
    err = O.normwise_rel_err(got, ref)
    assert 0.0 < err < 5e-2, err


# --------------------------------------------------------------------------- block-scaled e4m3 h


def _smallest_exponent(a: float) -> int:
    """Brute force in float64 (448 * 2^e is exact there): the smallest e with a <= 448 * 2^e."""
    e = -140
    while a > 448.0 * 2.0 ** e:
        e += 1
    return e


def test_block_exponents_against_brute_force():
    rng = np.random.default_rng(5)
    vals = [np.float32(v) for v in rng.lognormal(0.0, 12.0, 3000)]
    for j in range(-120, 121, 7):   # the boundaries 448 * 2^j and their float32 neighbours
        b = np.float32(448.0 * 2.0 ** j)
        vals += [b, np.nextafter(b, np.float32(np.inf)), np.nextafter(b, np.float32(0))]
    vals += [np.float32(224.0), np.float32(224.5), np.float32(1e-40), np.float32(3e38)]
    got = O.block_exponents_e4m3(np.array(vals, dtype=np.float32))
    for v, e in zip(vals, got):
        want = min(max(_smallest_exponent(float(v)), -126), 126)
        assert e == want, (float(v), int(e), want)
    special = O.block_exponents_e4m3(np.array([0.0, np.inf, np.nan, -0.0], dtype=np.float32))
    assert special.tolist() == [0, 0, 0, 0]


def test_quantize_blocks_codes_in_range_and_exact_blocks():
    g = torch.Generator().manual_seed(31)
    h = torch.randn(50, 128, generator=g) * torch.exp2(torch.randint(-20, 20, (50, 1), generator=g).float())
    h[3, 32:64] = 0.0   # an all-zero block
    q, e = O.quantize_blocks_e4m3(h)
    qb = q.float().reshape(50, 4, 32).abs().amax(-1)
    nz = qb > 0
    # the exponent is the smallest that fits: the block's largest code is in [224, 448]
    assert bool(((qb[nz] >= 224) & (qb[nz] <= 448)).all())
    assert e[3, 1] == 0 and not bool(nz[3, 1])
    d = O.dequantize_blocks_e4m3(q, e)
    big = h.abs() >= 2.0 ** -6 * 2.0 ** e.repeat_interleave(32, dim=1).float()   # e4m3 normals
    assert bool(((d - h).abs()[big] <= h.abs()[big] * 2.0 ** -4).all())       # half an e4m3 ulp
    # blocks of e4m3 grid values with maximum 448 * 2^j come back unchanged
    grid = torch.from_numpy(O.e4m3_decode_table()).float()
    grid = grid[torch.isfinite(grid)]
    exact = grid[torch.randint(0, grid.numel(), (6, 64), generator=g)]
    exact[:, 0] = 448.0
    exact[:, 32] = -448.0
    exact = exact * torch.exp2(torch.randint(-30, 30, (6, 1), generator=g).float())
    q2, e2 = O.quantize_blocks_e4m3(exact)
    assert torch.equal(O.dequantize_blocks_e4m3(q2, e2), exact)


def test_w8a8_oracle_with_block_scaled_h():
    g = torch.Generator().manual_seed(23)
    params = _w8a8_params(g, S=128)
    x = torch.randn(40, 64, generator=g)
    ids = torch.randint(0, 50, (40,), generator=g)
    table = torch.from_numpy(O.multi_hash_table(50, 4, 2, 0))
    kw = dict(route_weights=(0.5, 0.5), shared_scale=0.7, routed_scale=1.3)
    a = O.engine_forward_w8a8(x, ids, table, params, **kw)
    b = O.engine_forward_w8a8(x, ids, table, params, h_blocks=True, **kw)
    err = O.normwise_rel_err(b, a)
    assert 0.0 < err < 4e-2, err
