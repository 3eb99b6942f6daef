"""GPU parity of the kNN stages (fused MFMA distance + top-M kernel) against the
CPU oracle, through the C ABI.

Integer-valued data (every distance exact in fp32) must match bit for bit;
float data must match within 1e-5 relative with ids identical except ties.
"""
import numpy as np
import pytest

import gt_oracle as O
import synth
from helpers import assert_knn_close, assert_knn_equal

pytestmark = pytest.mark.gpu


def _int_data(n, d, seed, hi=256):
    rng = np.random.default_rng(seed)
    return rng.integers(0, hi, size=(n, d)).astype(np.float32)


@pytest.mark.parametrize("n,d,k", [(3000, 128, 64), (777, 96, 32), (1000, 100, 17), (257, 32, 128), (5, 8, 4)])
def test_knn_exact_integer_bitexact(ctx, n, d, k):
    X = _int_data(n, d, seed=n + d)
    k = min(k, n - 1)
    ids, dist = ctx.knn_exact(X, k)
    rid, rd = O.knn_exact(X, k)
    assert_knn_equal(ids, dist, rid, rd)


@pytest.mark.parametrize("k", [1, 2, 3, 4, 5])
def test_knn_exact_short_lists(ctx, k):
    # lists of at most 4 entries are merged one lane per query; 5 takes the wave-wide merge
    X = _int_data(3000, 64, seed=40 + k, hi=8)      # many ties
    ids, dist = ctx.knn_exact(X, k)
    rid, rd = O.knn_exact(X, k)
    assert_knn_equal(ids, dist, rid, rd)
    q = np.random.default_rng(k).choice(3000, size=100, replace=False)
    ids, dist = ctx.knn_exact(np.tile(X, (8, 1)), k, queries=q)   # pool split + partial merge
    rid, rd = O.knn_exact(np.tile(X, (8, 1)), k, queries=q)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_exact_query_subset_split_pool(ctx):
    # few queries, large pool: exercises the pool-split + partial-merge path
    X = _int_data(40000, 128, seed=1)
    q = np.random.default_rng(2).choice(40000, size=300, replace=False)
    ids, dist = ctx.knn_exact(X, 32, queries=q)
    rid, rd = O.knn_exact(X, 32, queries=q)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_exact_duplicates_and_ties(ctx):
    X = _int_data(2000, 128, seed=3, hi=3)       # tiny range: massive ties
    X[100] = X[200]
    ids, dist = ctx.knn_exact(X, 64)
    rid, rd = O.knn_exact(X, 64)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_exact_float_c1(ctx):
    X, _ = synth.generate("C1", n=3000)
    ids, dist = ctx.knn_exact(X, 64)
    rid, rd = O.knn_exact(X, 64)
    assert_knn_close(X, np.arange(len(X)), ids, dist, rid, rd, rtol=1e-5)


def test_knn_exact_ip_c3(ctx):
    X, _ = synth.generate("C3", n=3000)
    ids, dist = ctx.knn_exact(X, 32, metric="ip")
    rid, rd = O.knn_exact(X, 32, metric=1)
    # the library reports the inner product (descending); the oracle its negation
    assert_knn_close(X, np.arange(len(X)), ids, -dist, rid, rd, rtol=1e-5, metric="ip")


def test_knn_exact_int8(ctx):
    X, _ = synth.generate("C5", n=2000)
    ids, dist = ctx.knn_exact(X, 32)
    rid, rd = O.knn_exact(X.astype(np.float32), 32)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_exact_uint8(ctx):
    X = np.random.default_rng(5).integers(0, 256, size=(1500, 128)).astype(np.uint8)
    ids, dist = ctx.knn_exact(X, 16)
    rid, rd = O.knn_exact(X.astype(np.float32), 16)
    assert_knn_equal(ids, dist, rid, rd)


def test_assign_top2(ctx):
    X = _int_data(5000, 128, seed=6)
    C = X[np.random.default_rng(7).choice(5000, 300, replace=False)]
    top2, d2 = ctx.assign_top2(X, C)
    Xi, Ci = X.astype(np.int64), C.astype(np.int64)
    for q in range(0, 5000, 37):
        dd = ((Ci - Xi[q]) ** 2).sum(axis=1)
        o = np.lexsort((np.arange(300), dd))[:2]
        assert top2[q].tolist() == o.tolist()
        assert d2[q].tolist() == dd[o].astype(np.float32).tolist()


def _buckets(rng, N, B):
    lab = rng.integers(0, B, size=N)
    lab[:B] = np.arange(B)
    order = np.argsort(lab, kind="stable")
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    return np.cumsum(off), order.astype(np.int32)


@pytest.mark.parametrize("N,B,P,M", [(6000, 12, 3, 64), (3000, 5, 4, 32), (2500, 40, 0, 16), (4000, 9, 2, 96)])
def test_knn_bucketed_bitexact(ctx, N, B, P, M):
    rng = np.random.default_rng(N + B)
    X = _int_data(N, 128, seed=N)
    off, mem = _buckets(rng, N, B)
    probe = np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32) \
        if P else np.zeros((B, 0), np.int32)
    ids, dist = ctx.knn_bucketed(X, off, mem, probe, M)
    rid, rd = O.knn_bucketed(X, off, mem, probe, M)
    assert_knn_equal(ids, dist, rid, rd)


def test_knn_bucketed_merge_rounds(ctx):
    rng = np.random.default_rng(11)
    N, B, M = 5000, 10, 32
    X = _int_data(N, 128, seed=12)
    run = None
    ref = None
    for r in range(3):
        off, mem = _buckets(rng, N, B)
        probe = np.stack([rng.permutation(np.delete(np.arange(B), b))[:2] for b in range(B)]).astype(np.int32)
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, running=run)
        ni, nd = O.knn_bucketed(X, off, mem, probe, M)
        ref = (ni, nd) if ref is None else O.merge_rounds(*ref, ni, nd)
        run = (ids, dist)
        assert_knn_equal(ids, dist, *ref)


def test_knn_bucketed_all_probed_is_exact_c1(ctx):
    # C1's rule (nprobe = buckets - 1): the pooled kNN is the exact kNN
    X, _ = synth.generate("C1", n=4000)
    X = np.rint(X * 8)   # integer-valued copy of the C1 recipe: exact distances
    rng = np.random.default_rng(13)
    off, mem = _buckets(rng, 4000, 16)
    probe = np.array([[b2 for b2 in range(16) if b2 != b] for b in range(16)], np.int32)
    ids, dist = ctx.knn_bucketed(X, off, mem, probe, 64)
    rid, rd = O.knn_exact(X, 64)
    assert_knn_equal(ids, dist, rid, rd)


def test_merge_rounds_gpu(ctx):
    rng = np.random.default_rng(14)
    X = _int_data(3000, 64, seed=15, hi=20)
    a = O.knn_exact(X, 48)
    # two partial views of the exact lists (random subsets, still sorted)
    views = []
    for s in range(2):
        keep = rng.random(a[0].shape) < 0.6
        vi = np.full_like(a[0], -1)
        vd = np.full_like(a[1], np.inf)
        for q in range(3000):
            k = np.nonzero(keep[q])[0]
            vi[q, :len(k)], vd[q, :len(k)] = a[0][q, k], a[1][q, k]
        views.append((vi, vd))
    gi, gd = ctx.merge_rounds(*views[0], *views[1])
    ri, rd = O.merge_rounds(*views[0], *views[1])
    assert_knn_equal(gi, gd, ri, rd)


def test_refine_2hop_gpu(ctx):
    X = _int_data(3000, 128, seed=16, hi=64)
    rng = np.random.default_rng(17)
    off, mem = _buckets(rng, 3000, 30)
    probe = np.stack([rng.permutation(np.delete(np.arange(30), b))[:1] for b in range(30)]).astype(np.int32)
    ids, dist = O.knn_bucketed(X, off, mem, probe, 32)
    gi, gd = ctx.refine_2hop(X, ids, dist, S=8, passes=2)
    ri, rd = O.refine_2hop(X, ids, dist, 8)
    ri, rd = O.refine_2hop(X, ri, rd, 8)
    assert_knn_equal(gi, gd, ri, rd)


def test_refine_hand_traced_known_answer_gpu(ctx):
    from test_oracle import REFINE_KAT_OUT_D, REFINE_KAT_OUT_IDS, refine_kat_input
    X, ids, d = refine_kat_input()
    gi, gd = ctx.refine_2hop(X, ids, d, S=2, passes=1)
    assert gi.tolist() == REFINE_KAT_OUT_IDS
    assert gd.tolist() == REFINE_KAT_OUT_D


def test_invalid_arguments_raise(ctx):
    import gtann
    X = _int_data(100, 16, seed=18)
    with pytest.raises(gtann.GtannError):
        ctx.knn_exact(X, 0)
    with pytest.raises(gtann.GtannError):
        ctx.knn_exact(np.zeros((10, 1040), np.float32), 4)   # D > 1024 not supported
    off = np.array([0, 50], np.int64)   # does not cover all points
    with pytest.raises(gtann.GtannError):
        ctx.knn_bucketed(X, off, np.arange(100, dtype=np.int32), np.zeros((1, 0), np.int32), 8)


@pytest.mark.parametrize("n,nb,D,lo,hi", [(30000, 300, 128, -128, 128), (20000, 500, 128, -2, 3),
                                           (20000, 250, 256, -128, 128), (12000, 40, 32, 0, 2),
                                           (30000, 900, 128, -128, 128)])
def test_bucketing_resident_centroids(ctx, n, nb, D, lo, hi):
    """Lloyd steps, probe table and top-2 assignment of int8 rows with the
    centroids held in LDS (up to 512 of 128 bytes, 288 of 256; 900 take the
    staged kernel either way): the staged kernel's build, table and graph bit
    for bit.  Values in [-2, 3) and [0, 2) give ties among centroids."""
    from helpers import debug_opts
    rng = np.random.default_rng(n + nb + D)
    X = rng.integers(lo, hi, size=(n, D)).astype(np.int8)
    kw = dict(n_buckets=nb, nprobe=1, M=32, K=16, rounds=2)
    print(f"resident centroids n={n} buckets={nb} D={D}", flush=True)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, knn_resident=False):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists.view(np.uint32), b.knn_dists.view(np.uint32))
    np.testing.assert_array_equal(a.graph, b.graph)


@pytest.mark.parametrize("k", [1, 3, 4])
def test_knn_exact_short_lists_resident(ctx, k):
    # exact kNN of a small int8 set with k <= 4 (self excluded) takes the
    # LDS-resident kernel: the staged kernel's lists bit for bit
    from helpers import debug_opts
    rng = np.random.default_rng(k)
    X = rng.integers(-3, 4, size=(2500, 64)).astype(np.int8)
    a = ctx.knn_exact(X, k)
    with debug_opts(ctx, knn_resident=False):
        b = ctx.knn_exact(X, k)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
    rid, rd = O.knn_exact(X.astype(np.float32), k)
    assert_knn_equal(a[0], a[1], rid, rd)
