"""Fragment-major weight copies for the decode kernels.

The copy only changes how the decode kernels load weights (1 KiB
contiguous per 16-row x 64-byte MFMA fragment instead of 16 rows x 64
bytes), not what they compute: outputs must be bit-identical to the plain
decode path, and the layout itself is checked against a torch permutation.
"""

import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu


def _rand(*shape, scale=1.0, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cols", [64, 200, 896])
def test_fragment_layout(gpu, dtype, cols):
    from complexity_amd import ops

    rows = 48
    ld = (cols + 7) // 8 * 8
    w = torch.zeros(rows, ld, dtype=dtype)
    w[:, :cols] = _rand(rows, cols, seed=cols).to(dtype)
    frag, c = ops.pack_fragments(w.to(gpu), cols)
    assert c == cols
    eb = w.element_size()
    G = (cols * eb + 63) // 64
    wb = torch.zeros(rows, G * 64, dtype=torch.uint8)
    wb[:, : cols * eb] = w.view(torch.uint8)[:, : cols * eb]
    # [block][g][q][i][16 bytes] from [row = 16 block + i][64 g + 16 q + byte]
    want = wb.view(rows // 16, 16, G, 4, 16).permute(0, 2, 3, 1, 4).reshape(-1)
    assert torch.equal(frag.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 8, 17, 64, 100, 128])
def test_gate_up_with_fragments_is_bit_identical(gpu, dtype, n):
    from complexity_amd import ops

    H, S = 200, 320
    x = _rand(n, H, seed=n).to(dtype).to(gpu)
    wg, wu = _rand(S, H, scale=0.1, seed=1).to(dtype), _rand(S, H, scale=0.1, seed=2).to(dtype)
    pg, _ = ops.pack_linear_gate_up(wg.to(gpu), wu.to(gpu))
    fr = ops.pack_fragments(pg, H)
    assert torch.equal(ops.shared_gate_up(x, pg, None, S), ops.shared_gate_up(x, pg, None, S, w_frag=fr))
    # with the fused RMSNorm scales too
    a = ops.shared_gate_up(x, pg, None, S, rms_eps=1e-5)
    b = ops.shared_gate_up(x, pg, None, S, rms_eps=1e-5, w_frag=fr)
    assert torch.equal(a, b)
    with pytest.raises(ValueError, match="cols"):
        ops.shared_gate_up(x, pg, None, S, w_frag=(fr[0], H + 8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n", [1, 8, 16, 17, 64, 128])
@pytest.mark.parametrize("hidden", [896, 72])
def test_down_with_fragments_is_bit_identical(gpu, dtype, n, hidden):
    """8-column tiles (n <= 16) start at every multiple of 8, so half of them
    sit in the second half of a 16-row fragment block."""
    from complexity_amd import ops

    S = 3328 if hidden == 896 else 200
    h = _rand(n, S, seed=n + hidden).to(dtype)
    hp = torch.zeros(n, (S + 127) // 128 * 128, dtype=dtype)
    hp[:, :S] = h
    wd = _rand(hidden, S, scale=0.05, seed=3).to(dtype)
    pd, _ = ops.pack_linear_down(wd.to(gpu))
    fr = ops.pack_fragments(pd, S)
    res = _rand(n, hidden, seed=9).to(dtype).to(gpu)
    a = ops.shared_down_combine(hp.to(gpu), S, pd, None, hidden, None, None, 2, (0.5, 0.5), 0.7, 1.0, res)
    b = ops.shared_down_combine(hp.to(gpu), S, pd, None, hidden, None, None, 2, (0.5, 0.5), 0.7, 1.0, res,
                                w_frag=fr)
    assert torch.equal(a, b)
    ref = 0.7 * (h.double() @ wd.double().T) + res.double().cpu()
    assert O.normwise_rel_err(b, ref) <= (1e-5 if dtype == torch.float32 else 1e-2)


@pytest.mark.parametrize("name", ["c3_bf16_decode_64", "c4_bf16_decode_8"])
def test_decode_layer_uses_fragments_and_matches_oracle(gpu, name):
    """The engine's decode-sized calls build the fragment copies once and
    match both the plain kernels (bit for bit) and the oracle."""
    from complexity_amd import ops
    from complexity_amd import workloads as Wl

    w = Wl.WORKLOADS[name]
    engine = Wl.build_engine(w, gpu, backend="hip")
    x, ids = Wl.make_hidden(w).to(gpu).to(torch.bfloat16), Wl.make_token_ids(w).to(gpu)
    with torch.no_grad():
        out = engine(x, ids)
    packed = engine._hip_packed()
    assert set(packed.frag) == {"dense_gate_up", "dense_down"}
    flat = x.reshape(-1, w.hidden)
    plain = ops.PackedLayer(**{k: getattr(packed, k) for k in (
        "act_dtype", "num_experts", "expert_width", "strategy", "shared_width", "dense_gate_up", "dense_down",
        "dense_features")})
    plain.fragments = lambda name, cols: None
    cfg = engine.config
    with torch.no_grad():
        ref_plain = ops.layer_forward(flat, ids.reshape(-1), engine._active_route_table, plain, cfg.route_weights,
                                      cfg.shared_output_scale, cfg.routed_output_scale)
    assert torch.equal(out.reshape(-1, w.hidden), ref_plain)
