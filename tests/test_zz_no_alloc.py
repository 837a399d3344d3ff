"""trmoe_route_sort_noalloc, the K1 entry point that allocates nothing (its
histogram scratch is a static device array), against trmoe_route_sort with
a caller workspace: bit-exact outputs on calls in a row on one stream, each
smaller than the one before, so a call that finds the previous call's
histograms in the shared array must not be affected by them."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _outputs(n, k, E, dev):
    return (torch.full((k, n), -7, dtype=torch.int64, device=dev),
            torch.full((k * n,), -7, dtype=torch.int64, device=dev),
            torch.full((k * n,), -7, dtype=torch.int64, device=dev),
            torch.full((E + 1,), -7, dtype=torch.int32, device=dev),
            torch.full((E,), -7, dtype=torch.int32, device=dev))


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _with_workspace(lib, ids, table, E, order):
    from complexity_amd import _native

    k, vocab = table.shape
    n = ids.numel()
    routes, srt, inv, off, cnt = _outputs(n, k, E, ids.device)
    ws_bytes = lib.trmoe_route_sort_workspace_bytes(n, k, E, order)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=ids.device)
    st = lib.trmoe_route_sort(_p(ids), n, _p(table), vocab, k, E, order, _p(routes), _p(srt), _p(inv), _p(off),
                              _p(cnt), _p(ws), ws_bytes, _stream(ids.device))
    _native.check(st, "trmoe_route_sort")
    return routes, srt, inv, off, cnt


def _no_alloc(lib, ids, table, E, order):
    from complexity_amd import _native

    k, vocab = table.shape
    n = ids.numel()
    routes, srt, inv, off, cnt = _outputs(n, k, E, ids.device)
    st = lib.trmoe_route_sort_noalloc(_p(ids), n, _p(table), vocab, k, E, order, _p(routes), _p(srt), _p(inv),
                                      _p(off), _p(cnt), _stream(ids.device))
    _native.check(st, "trmoe_route_sort_noalloc")
    return routes, srt, inv, off, cnt


@pytest.mark.parametrize("order", [0, 1])
def test_no_alloc_route_sort_matches_the_workspace_call(gpu, order):
    from complexity_amd import _native
    from oracle import trmoe_oracle as O

    lib = _native.load()
    rng = np.random.default_rng(41 + order)
    table16 = torch.from_numpy(O.multi_hash_table(32000, 16, 2, 0)).to(gpu)
    table4 = torch.from_numpy(O.multi_hash_table(32000, 4, 2, 0)).to(gpu)
    # 32768 tokens x 2 slots = 256 chunks of 256 items: 256 blocks x 16
    # experts, the whole 16 KiB scratch; then 70000 tokens (547 chunks, 3 per
    # block, 183 blocks), 20000 tokens at E = 4 (157 blocks), and one block
    # (no scratch)
    cases = [(32768, table16, 16), (70000, table16, 16), (20000, table4, 4), (300, table16, 16)]
    for n, table, E in cases:
        ids = torch.from_numpy(rng.integers(-5, 32005, n)).to(gpu)
        want = _with_workspace(lib, ids, table, E, order)
        got = _no_alloc(lib, ids, table, E, order)
        torch.cuda.synchronize()
        for name, a, b in zip(("routes", "sorted", "inverse", "offsets", "counts"), got, want):
            assert torch.equal(a, b), (n, E, order, name)


def test_no_alloc_route_sort_validates_like_the_workspace_call(gpu):
    from complexity_amd import _native

    lib = _native.load()
    ids = torch.zeros(4, dtype=torch.int64, device=gpu)
    table = torch.zeros(2, 10, dtype=torch.int64, device=gpu)
    routes, srt, inv, off, cnt = _outputs(4, 2, 17, gpu)
    st = lib.trmoe_route_sort_noalloc(_p(ids), 4, _p(table), 10, 2, 17, 0, _p(routes), _p(srt), _p(inv), _p(off),
                                      _p(cnt), _stream(gpu))
    assert st == _native.ERR_INVALID and b"num_experts" in lib.trmoe_last_error()
