"""RMSNorm kernels (trmoe_rmsnorm_forward / _backward) against the oracle.

The forward is the reference's RMSNorm (complexity/core/normalization/
norms.py:46-55); the oracle is ``rms_norm`` in f64 and its gradients are f64
autograd of it (pinned by central differences in tests/test_oracle.py).
Bounds, normwise max|got - ref| / max|ref|: 1e-5 for fp32 and 1e-2 for bf16
(inputs and outputs rounded to bf16; the product's bound is 2e-2).  The
per-token scale r is checked to 1e-5 relative in both dtypes.
"""

import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu

BOUND = {torch.float32: 1e-5, torch.bfloat16: 1e-2}

SHAPES = [
    (torch.float32, 1, 896),
    (torch.float32, 7, 8),            # one 32-byte row: lanes past the row idle
    (torch.float32, 300, 2048),       # eight chunks per lane
    (torch.bfloat16, 5, 16),
    (torch.bfloat16, 64, 896),
    (torch.bfloat16, 4097, 896),      # more rows than 4 x 1024 backward workgroups
    (torch.bfloat16, 33, 4096),       # eight chunks per lane
    (torch.bfloat16, 1000, 2048),
]


def _inputs(dtype, n, hidden, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, hidden, generator=g) * 2.0).to(dtype)
    w = (torch.rand(hidden, generator=g) + 0.5).to(dtype)
    dy = (torch.randn(n, hidden, generator=g) * 0.5).to(dtype)
    return x, w, dy


def _oracle(x, w, dy, eps):
    xd = x.double().requires_grad_(True)
    wd = w.double().requires_grad_(True)
    y = O.rms_norm(xd, wd, eps)
    dx, dw = torch.autograd.grad(y, (xd, wd), dy.double())
    return y.detach(), dx, dw


def _err(got, ref):
    return O.normwise_rel_err(got.double().cpu(), ref)


@pytest.mark.parametrize("dtype,n,hidden", SHAPES)
def test_rmsnorm_forward_and_backward(gpu, dtype, n, hidden):
    from complexity_amd import ops

    print(f"rmsnorm {dtype} n={n} hidden={hidden}", flush=True)
    eps = 1e-6
    x, w, dy = _inputs(dtype, n, hidden, n + hidden)
    y, r = ops.rmsnorm_forward(x.to(gpu), w.to(gpu), eps)
    dx, dw = ops.rmsnorm_backward(x.to(gpu), w.to(gpu), r, dy.to(gpu))
    torch.cuda.synchronize()
    ref_y, ref_dx, ref_dw = _oracle(x, w, dy, eps)
    ref_r = torch.rsqrt(x.double().pow(2).mean(-1) + eps)
    assert torch.allclose(r.double().cpu(), ref_r, rtol=1e-5, atol=0)
    assert y.dtype == dtype and dx.dtype == dtype and dw.dtype == dtype
    assert _err(y, ref_y) <= BOUND[dtype], _err(y, ref_y)
    assert _err(dx, ref_dx) <= BOUND[dtype], _err(dx, ref_dx)
    assert _err(dw, ref_dw) <= BOUND[dtype], _err(dw, ref_dw)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_backward_residual_gradient_and_determinism(gpu, dtype):
    """dres is added to dx (also in place, dres = dx's buffer); the weight
    gradient is bit-identical across calls (partials summed in fixed order)."""
    from complexity_amd import ops

    x, w, dy = _inputs(dtype, 2000, 896, 3)
    dres = (torch.randn(2000, 896, generator=torch.Generator().manual_seed(4)) * 0.3).to(dtype)
    xg, wg, dyg = x.to(gpu), w.to(gpu), dy.to(gpu)
    _, r = ops.rmsnorm_forward(xg, wg, 1e-5)
    dx0, dw0 = ops.rmsnorm_backward(xg, wg, r, dyg)
    dx1, dw1 = ops.rmsnorm_backward(xg, wg, r, dyg, dres=dres.to(gpu))
    torch.cuda.synchronize()
    _, ref_dx, ref_dw = _oracle(x, w, dy, 1e-5)
    assert _err(dx1, ref_dx + dres.double()) <= BOUND[dtype]
    assert torch.equal(dw0, dw1)
    # in place: the residual gradient's buffer receives dx
    buf = dres.to(gpu)
    lib = ops._lib()
    from complexity_amd import _native as N
    code = ops.dtype_code(dtype)
    ws_bytes = lib.trmoe_rmsnorm_backward_workspace_bytes(code, 2000, 896)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    dw2 = torch.empty(896, dtype=dtype, device=gpu)
    st = lib.trmoe_rmsnorm_backward(code, ops._p(xg), 2000, 896, 896, ops._p(wg), ops._p(r), ops._p(dyg), 896,
                                    ops._p(buf), 896, ops._p(buf), 896, ops._p(dw2), ops._p(ws), ws_bytes,
                                    ops._stream(xg))
    N.check(st, "trmoe_rmsnorm_backward")
    torch.cuda.synchronize()
    assert torch.equal(buf, dx1)
    assert torch.equal(dw2, dw0)


def test_rmsnorm_empty_rows(gpu):
    """No tokens: an empty dx and a zero weight gradient."""
    from complexity_amd import ops

    x = torch.empty(0, 896, dtype=torch.bfloat16, device=gpu)
    w = torch.ones(896, dtype=torch.bfloat16, device=gpu)
    y, r = ops.rmsnorm_forward(x, w, 1e-6)
    dx, dw = ops.rmsnorm_backward(x, w, r, x)
    torch.cuda.synchronize()
    assert y.shape == (0, 896) and dx.shape == (0, 896)
    assert torch.equal(dw, torch.zeros_like(dw))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rmsnorm_function_strided_input(gpu, dtype):
    """RMSNormFunction on a column slice of a wider buffer (a row stride
    larger than hidden) matches the oracle's forward and gradients."""
    from complexity_amd.tr_hash.hip_autograd import RMSNormFunction

    x, w, dy = _inputs(dtype, 129, 256, 9)
    wide = torch.zeros(129, 384, dtype=dtype)
    wide[:, 64:320] = x
    xg = wide.to(gpu)[:, 64:320].detach().requires_grad_(True)
    wg = w.to(gpu).requires_grad_(True)
    y = RMSNormFunction.apply(xg, wg, 1e-6)
    y.backward(dy.to(gpu))
    torch.cuda.synchronize()
    ref_y, ref_dx, ref_dw = _oracle(x, w, dy, 1e-6)
    assert _err(y.detach(), ref_y) <= BOUND[dtype]
    assert _err(xg.grad, ref_dx) <= BOUND[dtype]
    assert _err(wg.grad, ref_dw) <= BOUND[dtype]
