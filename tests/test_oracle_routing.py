"""Pins the oracle's routing tables (op moe_routing; tables of tools/kernels/abi/trtllm_bmm.py:19-27,
capacity :50-60) on the CPU against a brute-force stable sort and the tables' invariants."""
import numpy as np
import pytest

from kern_amd import workload as wl


@pytest.mark.parametrize("T,E,k,start,local", [(64, 16, 4, 0, 16), (37, 16, 4, 4, 8), (1, 8, 2, 0, 8),
                                               (300, 224, 16, 56, 56), (0, 8, 2, 0, 8), (600, 4, 2, 0, 4)])
def test_routing_bruteforce(oracle, T, E, k, start, local):
    ids = wl.topk_ids(T * 31 + E, T, E, k) if T else np.zeros((0, k), np.int32)
    t = oracle.routing(ids, start, local)
    flat = ids.reshape(-1) - start
    is_local = (flat >= 0) & (flat < local)
    counts = np.bincount(flat[is_local], minlength=local)
    np.testing.assert_array_equal(t["counts"][:local], counts)
    slots = -(-counts // 128)
    off = np.concatenate([[0], np.cumsum(slots)[:-1]])
    np.testing.assert_array_equal(t["counts"][local:], off)
    S = int(slots.sum())
    assert t["num_non_exiting"][0] == S and t["total_padded"][0] == 128 * S
    # expected permutation: stable sort of local expanded rows by expert
    order = np.argsort(np.where(is_local, flat, local), kind="stable")[: int(is_local.sum())]
    perm = np.full(T * k, -1)
    for e in range(local):
        rows = order[flat[order] == e]
        perm[rows] = off[e] * 128 + np.arange(len(rows))
    np.testing.assert_array_equal(t["exp2perm"].reshape(-1), perm)
    rm = np.full(S * 128, -1)
    rm[perm[perm >= 0]] = np.nonzero(perm >= 0)[0] // k
    np.testing.assert_array_equal(t["route_map"][: S * 128], rm)
    for s in range(S):
        e = t["cta_batch"][s]
        assert off[e] <= s < off[e] + slots[e]
        assert t["cta_limit"][s] == min((s + 1) * 128, off[e] * 128 + counts[e])
        assert t["cta_limit"][s] > s * 128      # every live slot has at least one row
    # slot bound of the manifest grid.y: experts + ceil(tokens*topk/128) (trtllm_bmm.py:58-60)
    assert S <= local + -(-T * k // 128)
    assert S <= oracle.max_ctas(T, k, local, 128) or T * k < local


def test_max_ctas_formula(oracle):
    # trtllm_bmm.py:50-55: min(E, T*k) + (T*k - min(E, T*k)) // tile
    assert oracle.max_ctas(512, 8, 256, 128) == 256 + (4096 - 256) // 128
    assert oracle.max_ctas(1, 8, 256, 128) == 8
    assert oracle.max_ctas(8192, 16, 56, 128) == 56 + (131072 - 56) // 128
