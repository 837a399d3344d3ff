"""Host logic of the mapped weight gradients (no GPU): the destination maps
of ops._dense_grad_maps, applied on the CPU the way k_wgrad_reduce applies
them, must place dWgu [2F, H] (packed gate|up rows) and dWd [H, F] exactly
where the strided views of the unmapped path put them."""

import pytest
import torch

from complexity_amd import ops


def _apply_rows(flat, mat, off, stride):
    # mode 1: flat[off[i] + j * stride[i]] = mat[i, j]
    n = mat.shape[1]
    j = torch.arange(n, dtype=torch.int64)
    for i in range(mat.shape[0]):
        if off[i] >= 0:
            flat[off[i] + j * stride[i]] = mat[i]


def _apply_cols(flat, mat, off, stride):
    # mode 2: flat[off[j] + i * stride[j]] = mat[i, j]
    m = mat.shape[0]
    i = torch.arange(m, dtype=torch.int64)
    for j in range(mat.shape[1]):
        if off[j] >= 0:
            flat[off[j] + i * stride[j]] = mat[:, j]


@pytest.mark.parametrize("S,E,W,H", [(256, 4, 64, 32), (96, 8, 12, 16), (0, 2, 40, 24), (128, 16, 32, 8),
                                     (300, 3, 100, 8)])
def test_dense_grad_maps_match_the_strided_views(S, E, W, H):
    s_pad, w_pad = -(-S // 128) * 128, -(-W // 64) * 64
    F_ = s_pad + E * w_pad
    g = torch.Generator().manual_seed(S + E + W + H)
    dwgu = torch.randn(2 * F_, H, generator=g)
    dwd = torch.randn(H, F_, generator=g)
    roff, rstride, coff, cstride, offs = ops._dense_grad_maps(S, E, W, H, "cpu")
    flat = torch.full((offs[-1],), float("nan"))
    _apply_rows(flat, dwgu, roff, rstride)
    _apply_cols(flat, dwd, coff, cstride)
    assert not torch.isnan(flat).any(), "every parameter element is written once"
    o_gate, o_up, o_sd, o_eg, o_eu, o_ed, _ = offs
    # the unmapped path's views (ops.layer_backward, dense strategy)
    g_rows, u_rows = ops._gate_up_rows(dwgu, F_)
    sh, ew = S * H, E * W * H
    if S:
        assert torch.equal(flat[o_gate:o_gate + sh].view(S, H), g_rows[:S])
        assert torch.equal(flat[o_up:o_up + sh].view(S, H), u_rows[:S])
        assert torch.equal(flat[o_sd:o_sd + sh].view(H, S), dwd[:, :S])
    eg = g_rows[s_pad:].view(E, w_pad, H)[:, :W].transpose(1, 2)
    eu = u_rows[s_pad:].view(E, w_pad, H)[:, :W].transpose(1, 2)
    ed = dwd[:, s_pad:].reshape(H, E, w_pad)[:, :, :W].permute(1, 2, 0)
    assert torch.equal(flat[o_eg:o_eg + ew].view(E, H, W), eg)
    assert torch.equal(flat[o_eu:o_eu + ew].view(E, H, W), eu)
    assert torch.equal(flat[o_ed:o_ed + ew].view(E, W, H), ed)


def test_dense_grad_maps_skip_padding_rows_and_columns():
    S, E, W, H = 96, 2, 40, 8
    roff, _, coff, _, _ = ops._dense_grad_maps(S, E, W, H, "cpu")
    s_pad, w_pad = 128, 64
    p = torch.arange(roff.numel())
    f = 32 * (p // 64) + p % 32
    fe = f - s_pad
    pad = ((f >= S) & (f < s_pad)) | ((f >= s_pad) & (fe % w_pad >= W))
    assert bool((roff[pad] < 0).all()) and bool((roff[~pad] >= 0).all())
    c = torch.arange(coff.numel())
    cpad = ((c >= S) & (c < s_pad)) | ((c >= s_pad) & ((c - s_pad) % w_pad >= W))
    assert bool((coff[cpad] < 0).all()) and bool((coff[~cpad] >= 0).all())


def test_mapped_destination_guard(tmp_path):
    """trmoe::mapped_dest, the reduction's write guard, built for the host:
    real destinations pass; a skipped row, a destination at or past out_elems
    and a negative one (bad maps from a C-ABI caller) are not written."""
    import shutil
    import subprocess
    from pathlib import Path

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is not installed")
    root = Path(__file__).resolve().parents[1]
    exe = tmp_path / "map_guard"
    subprocess.run([hipcc, "-x", "hip", "--offload-host-only", "-O1", "-I", str(root / "complexity-framework_amd/csrc"),
                    str(root / "tests/map_guard_check.cpp"), "-o", str(exe)], check=True)
    S, E, W, H = 256, 4, 64, 32
    roff, rstride, coff, cstride, offs = ops._dense_grad_maps(S, E, W, H, "cpu")
    total = int(offs[-1])
    cases, want = [], []
    for i in range(roff.numel()):              # every real row destination, first and last column
        o, st = int(roff[i]), int(rstride[i])
        for j in (0, H - 1):
            cases.append((o, j, st, total))
            want.append(o + j * st if o >= 0 else -1)
    cases += [(-1, 0, 1, total), (total - 1, 0, 5, total), (total - 1, 1, 1, total), (0, total, 1, total),
              (5, 1, -6, total), (5, 1, -5, total), (0, 3, 2, 7)]
    want += [-1, total - 1, -1, -1, -1, 0, 6]
    out = subprocess.run([str(exe)], input="\n".join(" ".join(map(str, c)) for c in cases), capture_output=True,
                         text=True, check=True).stdout.split()
    assert [int(v) for v in out] == want
