"""Rows longer than 256 floats (config C4, D = 960): the wide fused kNN
kernel and every stage that reads vectors, against the CPU oracle.  Integer
data below 120 keeps every fp32 sum exact up to D = 1024 (1024 * 119^2 <
2^24), so these comparisons are bit-exact."""
import numpy as np
import pytest

import gt_oracle as O
import synth
from helpers import assert_knn_close, assert_knn_equal

pytestmark = pytest.mark.gpu


def _int_data(n, d, seed, hi=120):
    return np.random.default_rng(seed).integers(0, hi, size=(n, d)).astype(np.float32)


@pytest.mark.parametrize("n,d,k", [(2000, 960, 96), (1500, 300, 32), (700, 1024, 48), (300, 288, 7)])
def test_knn_exact_wide_bitexact(ctx, n, d, k):
    X = _int_data(n, d, seed=n + d)
    print(f"wide exact n={n} d={d} k={k}", flush=True)
    ids, dist = ctx.knn_exact(X, k)
    rid, rd = O.knn_exact(X, k)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_wide_split_pool_and_queries(ctx):
    X = _int_data(20000, 960, seed=3)
    q = np.random.default_rng(4).choice(len(X), size=200, replace=False)
    ids, dist = ctx.knn_exact(X, 64, queries=q)
    rid, rd = O.knn_exact(X, 64, queries=q)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_wide_float_c4_and_ip(ctx):
    X, _ = synth.generate("C4", n=3000)
    ids, dist = ctx.knn_exact(X, 48)
    rid, rd = O.knn_exact(X, 48)
    assert_knn_close(X, np.arange(len(X)), ids, dist, rid, rd)
    Xn = X / np.linalg.norm(X, axis=1, keepdims=True)
    ids, dist = ctx.knn_exact(Xn, 32, metric="ip")
    rid, rd = O.knn_exact(Xn, 32, metric=1)
    # the library reports the inner product (descending); the oracle its negation
    assert_knn_close(Xn, np.arange(len(Xn)), ids, -dist, rid, rd, metric="ip")


def test_knn_wide_bucketed(ctx):
    X = _int_data(6000, 960, seed=5)
    rng = np.random.default_rng(6)
    nb = 12
    assign = rng.integers(0, nb, size=len(X))
    order = np.argsort(assign, kind="stable").astype(np.int32)
    offsets = np.searchsorted(assign[order], np.arange(nb + 1)).astype(np.int64)
    probe = np.stack([rng.permutation(np.delete(np.arange(nb), b))[:3] for b in range(nb)]).astype(np.int32)
    ids, d = ctx.knn_bucketed(X, offsets, order, probe, 96)
    rid, rd = O.knn_bucketed(X, offsets, order, probe, 96)
    assert_knn_equal(ids, d, rid, rd)


def test_wide_stages_refine_occlusion_assign(ctx):
    X = _int_data(3000, 960, seed=7)
    ex_i, ex_d = O.knn_exact(X, 32)
    # refinement of a degraded table
    bi, bd = ex_i.copy(), ex_d.copy()
    bi[:, 16:], bd[:, 16:] = -1, np.inf
    gi, gd = ctx.refine_2hop(X, bi, bd, 8)
    oi, od = O.refine_2hop(X, bi, bd, 8)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)
    # occlusion prune
    np.testing.assert_array_equal(ctx.prune_occlusion(X, ex_i, 16), O.prune_occlusion(X, ex_i.astype(np.int64), 16))
    # top-2 assignment against centroids
    C = X[::100].copy()
    t2, d2 = ctx.assign_top2(X, C)
    diff = ((X[:, None, :].astype(np.int64) - C[None, :, :].astype(np.int64)) ** 2).sum(axis=2)
    order = np.lexsort((np.broadcast_to(np.arange(len(C)), diff.shape), diff), axis=1)[:, :2]
    np.testing.assert_array_equal(t2.astype(np.int64), order)
    np.testing.assert_array_equal(d2, np.take_along_axis(diff, order, 1).astype(np.float32))


def test_build_graph_c4_small(ctx):
    X, _ = synth.generate("C4", n=20000)
    res = ctx.build_graph(X, n_buckets=10, nprobe=1, M=96, K=48, rounds=2)
    q = np.arange(0, len(X), 97)
    ex_i, _ = O.knn_exact(X, 48, queries=q)
    rec = np.mean([len(np.intersect1d(res.knn_ids[qq, :48], ex_i[r])) / 48 for r, qq in enumerate(q)])
    assert rec > 0.9, rec
    g = res.graph
    assert g.shape == (len(X), 48) and (g < len(X)).all()
    assert (g != np.arange(len(X))[:, None]).all()
    san = O.sanitize(res.knn_ids)
    fwd, rc, _ = O.cagra_prune(san, 48)
    assert rc == 0
    np.testing.assert_array_equal(g, O.reverse_merge(fwd))
