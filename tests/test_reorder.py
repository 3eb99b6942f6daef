"""Bucket processing order and bucket reorder (host logic, CPU): the
library's gt_bucket_order against the reference header compiled in place
(src/bucket_order.hpp:161-262), and gt_bucket_reorder against the CPU
restatement of compute_bucket_reorder (src/bucket.cu:8363-8412), itself
pinned by the closed form (stable argsort of processing positions)."""
import numpy as np
import pytest

import gt_oracle as O
import gtann

needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference harness not built")


def _graph(rng, B, K, kind):
    g = rng.integers(0, B, size=(B, K)).astype(np.uint32)
    if kind == "knn-like":      # nearby buckets, self in column 0 as a self-kNN would have it
        g = ((np.arange(B)[:, None] + rng.integers(-6, 7, size=(B, K))) % B).astype(np.uint32)
        g[:, 0] = np.arange(B)
    elif kind == "padded":      # invalid entries and repeats
        g[rng.random((B, K)) < 0.2] = 0xFFFFFFFF
        g[:, -1] = g[:, 0]
    elif kind == "components":  # disconnected blocks of 10 buckets
        blk = np.arange(B) // 10 * 10
        g = (blk[:, None] + rng.integers(0, 10, size=(B, K))) % B
        g = g.astype(np.uint32)
    elif kind == "sparse":      # most rows empty
        g[rng.random(B) < 0.7] = 0xFFFFFFFF
    return g


@needs_ref
@pytest.mark.parametrize("B,K", [(1, 4), (2, 1), (17, 4), (300, 8), (2000, 32)])
@pytest.mark.parametrize("kind", ["random", "knn-like", "padded", "components", "sparse"])
@pytest.mark.parametrize("window", [1, 5, 64])
def test_bucket_order_matches_reference(B, K, kind, window):
    rng = np.random.default_rng(B * 31 + K + window)
    g = _graph(rng, B, K, kind)
    ours = gtann.bucket_order(g, window)
    np.testing.assert_array_equal(ours, O.ref_bucket_order(g, window))
    assert sorted(ours.tolist()) == list(range(B))


def test_bucket_order_empty_and_no_columns():
    assert gtann.bucket_order(np.zeros((0, 4), np.uint32), 8).size == 0
    # no edges at all: start at the first bucket, then the smallest free ids
    np.testing.assert_array_equal(gtann.bucket_order(np.zeros((5, 0), np.uint32), 8), np.arange(5))


@pytest.mark.parametrize("N,nb", [(1, 1), (1000, 20), (200000, 513)])
def test_bucket_reorder_matches_oracle_and_closed_form(N, nb):
    rng = np.random.default_rng(N + nb)
    assign = rng.integers(0, nb, size=N).astype(np.int32)
    assign[:nb] = np.arange(nb)[:min(nb, N)] if N >= nb else assign[:nb]
    order = rng.permutation(nb).astype(np.int32)
    cids = rng.choice(N, size=min(N, 7), replace=False)
    inv, off, cn = gtann.bucket_reorder(assign, nb, order, cids=cids)
    oi, oo = O.bucket_reorder(assign, nb, order)
    np.testing.assert_array_equal(inv, oi)
    np.testing.assert_array_equal(off, oo)
    # closed form: points by (processing position of their bucket, old id)
    pos = np.empty(nb, np.int64)
    pos[order] = np.arange(nb)
    np.testing.assert_array_equal(oi, np.argsort(pos[assign], kind="stable"))
    np.testing.assert_array_equal(oo, np.concatenate([[0], np.cumsum(np.bincount(assign, minlength=nb)[order])]))
    perm = np.empty(N, np.int64)
    perm[inv] = np.arange(N)
    np.testing.assert_array_equal(cn, perm[cids])


def test_bucket_reorder_rejects_bad_input():
    with pytest.raises(gtann.GtannError, match="no bucket"):
        gtann.bucket_reorder(np.array([0, 3], np.int32), 2, np.array([1, 0], np.int32))
    with pytest.raises(gtann.GtannError, match="permutation"):
        gtann.bucket_reorder(np.array([0, 1], np.int32), 2, np.array([1, 1], np.int32))
