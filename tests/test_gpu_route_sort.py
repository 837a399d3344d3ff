"""K1 on the GPU vs the oracle: routes, partition, inverse, offsets, counts bit-exact."""

import numpy as np
import pytest
import torch

from oracle import trmoe_oracle as O

pytestmark = pytest.mark.gpu


def _check(gpu, table_np, ids_np, E, order):
    from complexity_amd import ops

    table = torch.from_numpy(table_np).to(gpu)
    ids = torch.from_numpy(np.asarray(ids_np, dtype=np.int64)).to(gpu)
    s, inv, off, cnt, routes = ops.route_sort(ids, table, E, order, return_routes=True)
    torch.cuda.synchronize()
    r_ref = O.gather_routes(table_np, ids_np)
    s_ref, inv_ref, off_ref, cnt_ref = O.counting_partition(r_ref, E, order)
    assert np.array_equal(routes.cpu().numpy(), r_ref)
    assert np.array_equal(off.cpu().numpy(), off_ref)
    assert np.array_equal(cnt.cpu().numpy(), cnt_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    assert np.array_equal(inv.cpu().numpy(), inv_ref)


@pytest.mark.parametrize("order", [O.ORDER_TOKEN, O.ORDER_ASSIGNMENT])
@pytest.mark.parametrize("E,k", [(1, 1), (2, 1), (4, 2), (8, 2), (8, 4), (16, 2), (16, 4)])
def test_route_sort_small_and_ragged(gpu, order, E, k):
    strategy = "modulo_cyclic" if E == 1 else "token_id_multi_hash"
    table = O.route_table(strategy, 997, E, k, 3)
    rng = np.random.default_rng(E * 7 + k + order)
    for n in (0, 1, 63, 64, 255, 1000, 1024, 1025, 4097):
        ids = rng.integers(-10, 1010, n)  # out-of-range ids exercise the clamp
        _check(gpu, table, ids, E, order)


@pytest.mark.parametrize("order", [O.ORDER_TOKEN, O.ORDER_ASSIGNMENT])
@pytest.mark.parametrize("E,k", [(2, 2), (4, 4), (8, 2), (16, 4)])
def test_route_sort_repeated_experts_per_token(gpu, order, E, k):
    """Tables whose slots repeat an expert for a token: one partition row per
    assignment, ties broken by slot (single- and multi-block launches)."""
    rng = np.random.default_rng(E * 13 + k + order)
    table = rng.integers(0, E, (k, 503)).astype(np.int64)
    table[:, :40] = table[0, :40]
    for n in (1, 100, 2000, 40000):
        ids = rng.integers(0, 503, n)
        ids[: min(n, 40)] = np.arange(min(n, 40))
        _check(gpu, table, ids, E, order)


@pytest.mark.parametrize("n", [2048 * 1024 // 2 + 77, 3 * 65536 + 5])
def test_route_sort_many_chunks_per_block(gpu, n):
    """Beyond 256 blocks x 256 items the blocks take several chunks each."""
    table = O.multi_hash_table(32000, 16, 2, 0)
    rng = np.random.default_rng(n)
    ids = rng.integers(0, 32000, n)
    _check(gpu, table, ids, 16, O.ORDER_TOKEN)
    _check(gpu, table, ids, 16, O.ORDER_ASSIGNMENT)


@pytest.mark.parametrize("order", [O.ORDER_TOKEN, O.ORDER_ASSIGNMENT])
def test_route_sort_c2_zipf_prefill(gpu, order):
    from complexity_amd import workloads as W

    table = O.multi_hash_table(32000, 4, 2, 0)
    ids = W.make_token_ids(W.C2, seed=0).reshape(-1).numpy()
    _check(gpu, table, ids, 4, order)


def test_route_sort_c3_decode(gpu):
    from complexity_amd import workloads as W

    table = O.multi_hash_table(32000, 4, 2, 0)
    ids = W.make_token_ids(W.C3, seed=0).reshape(-1).numpy()
    _check(gpu, table, ids, 4, O.ORDER_TOKEN)


@pytest.mark.parametrize("E", [16, 8])
def test_route_sort_c5_scaled(gpu, E):
    from complexity_amd import workloads as W

    table = O.multi_hash_table(32000, E, 2, 0)
    ids = W.make_token_ids(W.C5, seed=0).reshape(-1).numpy()
    _check(gpu, table, ids, E, O.ORDER_ASSIGNMENT)
    _check(gpu, table, ids, E, O.ORDER_TOKEN)


def test_route_sort_is_deterministic_across_launches(gpu):
    from complexity_amd import ops

    table = torch.from_numpy(O.multi_hash_table(32000, 16, 4, 0)).to(gpu)
    ids = torch.randint(0, 32000, (50000,), device=gpu)
    first = ops.route_sort(ids, table, 16)
    for _ in range(3):
        again = ops.route_sort(ids, table, 16)
        for a, b in zip(first, again):
            assert torch.equal(a, b)


def test_route_sort_rejects_bad_arguments(gpu):
    from complexity_amd import ops

    table = torch.zeros(2, 10, dtype=torch.int64, device=gpu)
    ids = torch.zeros(4, dtype=torch.int64, device=gpu)
    with pytest.raises(ValueError, match="num_experts"):
        ops.route_sort(ids, table, 17)
    with pytest.raises(ValueError, match="top_k cannot exceed"):
        ops.route_sort(ids, table, 1)
