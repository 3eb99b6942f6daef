"""The collect + select kNN path (int8 rows, 4 < M <= 64) against the CPU
oracle and against the merging kernel.

The bucketed passes on int8 rows append every key at or below a query's
threshold to its candidate slots and select the top-M afterwards; the
threshold of an unseeded pass comes from the scan's first tiles, and a query
whose slots fill up is compacted to its M smallest keys.  Integer rows give
exact distances, so every comparison here is bit-exact, ties included
(order (distance, id)).
"""

import numpy as np
import pytest

import gt_oracle as O
from helpers import assert_knn_equal, debug_opts

pytestmark = pytest.mark.gpu


def _data(n, d, seed, lo=-128, hi=128):
    return np.random.default_rng(seed).integers(lo, hi, size=(n, d)).astype(np.int8)


def _buckets(rng, N, B, sizes=None):
    if sizes is None:
        lab = rng.integers(0, B, size=N)
        lab[:B] = np.arange(B)
    else:
        lab = np.repeat(np.arange(B), sizes)
        rng.shuffle(lab)
    order = np.argsort(lab, kind="stable")
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    return np.cumsum(off), order.astype(np.int32)


def _probe(rng, B, P):
    if P == 0:
        return np.zeros((B, 0), np.int32)
    return np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32)


@pytest.mark.parametrize("N,D,B,P,M,metric", [
    (6000, 128, 6, 0, 64, "l2"),     # own buckets only, pools of ~1000 rows
    (6000, 128, 6, 1, 64, "l2"),
    (5000, 96, 8, 2, 48, "l2"),
    (4000, 32, 5, 1, 17, "l2"),      # M <= 32: 16-key lanes
    (3000, 256, 4, 0, 32, "l2"),
    (3000, 64, 12, 0, 5, "l2"),
    (4000, 128, 6, 1, 64, "ip"),
    (3000, 96, 5, 0, 33, "ip"),
])
def test_collect_unseeded_matches_oracle(ctx, N, D, B, P, M, metric):
    rng = np.random.default_rng(N + D + M)
    X = _data(N, D, seed=D + M)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, P)
    print(f"collect unseeded N={N} D={D} B={B} P={P} M={M} {metric}", flush=True)
    ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, metric=metric)
    ri, rd = O.knn_bucketed(X.astype(np.float32), off, mem, probe, M, metric=1 if metric == "ip" else 0)
    got_d = -dist if metric == "ip" else dist
    assert_knn_equal(ids, got_d, ri, rd)


def test_collect_small_and_tiny_buckets(ctx):
    # pools shorter than the threshold window, shorter than M, a single row
    rng = np.random.default_rng(5)
    sizes = [1, 2, 30, 63, 64, 65, 200, 257, 900, 2000]
    N = sum(sizes)
    X = _data(N, 128, seed=6)
    off, mem = _buckets(rng, N, len(sizes), sizes)
    for P in (0, 1):
        probe = _probe(rng, len(sizes), P)
        print(f"collect small buckets P={P}", flush=True)
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, 64)
        ri, rd = O.knn_bucketed(X.astype(np.float32), off, mem, probe, 64)
        assert_knn_equal(ids, dist, ri, rd)


def test_collect_ties_and_duplicates(ctx):
    # rows over {0, 1}: few distinct distances, many duplicates at distance 0;
    # the kept set and its order are decided by ids at every threshold
    rng = np.random.default_rng(7)
    N = 5000
    X = _data(N, 32, seed=8, lo=0, hi=2)
    X[100:400] = X[99]          # 301 copies of one row
    off, mem = _buckets(rng, N, 4)
    probe = _probe(rng, 4, 1)
    print("collect ties", flush=True)
    ids, dist = ctx.knn_bucketed(X, off, mem, probe, 64)
    ri, rd = O.knn_bucketed(X.astype(np.float32), off, mem, probe, 64)
    np.testing.assert_array_equal(ids, ri)
    np.testing.assert_array_equal(dist, rd)


def test_collect_seeded_without_cap_compacts(ctx):
    # a running table of padding seeds every query with +inf: every pool row
    # passes and each query's slots are compacted many times
    rng = np.random.default_rng(9)
    N, B, M = 8000, 4, 64
    X = _data(N, 128, seed=10)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    run = (np.full((N, M), -1, np.int32), np.full((N, M), np.inf, np.float32))
    print("collect seeded with +inf", flush=True)
    ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, running=run)
    ri, rd = O.knn_bucketed(X.astype(np.float32), off, mem, probe, M)
    assert_knn_equal(ids, dist, ri, rd)


def test_collect_rounds_match_oracle(ctx):
    rng = np.random.default_rng(13)
    N, B, M = 6000, 8, 64
    X = _data(N, 128, seed=14, lo=-30, hi=31)
    Xf = X.astype(np.float32)
    run = ref = None
    for r in range(3):
        off, mem = _buckets(rng, N, B)
        probe = _probe(rng, B, 1)
        print(f"collect round {r}", flush=True)
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, running=run)
        ni, nd = O.knn_bucketed(Xf, off, mem, probe, M)
        ref = (ni, nd) if ref is None else O.merge_rounds(*ref, ni, nd)
        run = (ids, dist)
        assert_knn_equal(ids, dist, *ref)


def _mixed_running(ids, dist, other_ids, other_dist):
    """Running rows of every shape the in-place merge meets: a pass's own
    table (its keys come back: no fresh key), padding only (every key fresh,
    more than M), a short prefix + padding (threshold +inf), the row with a
    middle stretch removed (+ padding), and the row of another bucketing's
    table.  Every distance is the pair's exact one, as in a build."""
    N, M = ids.shape
    ri, rd = ids.copy(), dist.copy()
    k = np.arange(N) % 5
    ri[k == 1], rd[k == 1] = -1, np.inf
    ri[k == 2, 5:], rd[k == 2, 5:] = -1, np.inf
    sel = np.flatnonzero(k == 3)
    keep = np.r_[0:M // 4, M // 2:M]
    ri[sel, :len(keep)], rd[sel, :len(keep)] = ids[sel][:, keep], dist[sel][:, keep]
    ri[sel, len(keep):], rd[sel, len(keep):] = -1, np.inf
    ri[k == 4], rd[k == 4] = other_ids[k == 4], other_dist[k == 4]
    return ri, rd


@pytest.mark.parametrize("M,metric", [(64, "l2"), (33, "l2"), (17, "l2"), (64, "ip")])
def test_collect_merge_mixed_running_rows(ctx, M, metric):
    # a seeded pass merged into the running table in place: rows without
    # keys, rows whose keys all repeat running ids, rows with a few fresh
    # keys and rows with more than M, all against the oracle's pass +
    # cross-round merge
    rng = np.random.default_rng(31 + M)
    N, B = 7000, 7
    X = _data(N, 96, seed=32 + M, lo=-40, hi=41)
    mi = 1 if metric == "ip" else 0
    sign = -1 if metric == "ip" else 1
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    ai, ad = O.knn_bucketed(X.astype(np.float32), off, mem, probe, M, metric=mi)
    off3, mem3 = _buckets(rng, N, B)
    bi, bd = O.knn_bucketed(X.astype(np.float32), off3, mem3, _probe(rng, B, 1), M, metric=mi)
    ri, rd = _mixed_running(ai, ad, bi, bd)
    off2, mem2 = _buckets(rng, N, B)
    probe2 = _probe(rng, B, 1)
    print(f"collect merge into mixed running rows M={M} {metric}", flush=True)
    ids, dist = ctx.knn_bucketed(X, off2, mem2, probe2, M, metric=metric, running=(ri, sign * rd))
    ni, nd = O.knn_bucketed(X.astype(np.float32), off2, mem2, probe2, M, metric=mi)
    ei, ed = O.merge_rounds(ri, rd, ni, nd)
    np.testing.assert_array_equal(ids, ei)
    np.testing.assert_array_equal((sign * dist).view(np.uint32), ed.view(np.uint32))


def test_collect_equals_merging_kernel(ctx):
    # the same passes through the kernel that merges as it scans
    rng = np.random.default_rng(15)
    N, B, M = 20000, 16, 64
    X = _data(N, 128, seed=16, lo=-60, hi=61)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    a = ctx.knn_bucketed(X, off, mem, probe, M)
    b2 = ctx.knn_bucketed(X, off, mem, probe, M, running=a)
    with debug_opts(ctx, knn_collect=False):
        print("merging kernel", flush=True)
        c = ctx.knn_bucketed(X, off, mem, probe, M)
        c2 = ctx.knn_bucketed(X, off, mem, probe, M, running=c)
    for x, y in ((a, c), (b2, c2)):
        np.testing.assert_array_equal(x[0], y[0])
        np.testing.assert_array_equal(x[1], y[1])


@pytest.mark.parametrize("cfg,n,nb,skips", [("C2", 60000, 16, True), ("C5", 80000, 16, False),
                                            ("C2", 30000, 3, False)])
def test_chunk_pruning_is_exact(ctx, cfg, n, nb, skips):
    """The int8 collect kernel skips pool chunks whose bounding sphere is
    farther from every query of the block than its threshold: the tables and
    graphs equal a build that scans every chunk, bit for bit.  On the C2
    mixture (60 rows per cluster here) fewer pairs are computed; an 80,000-row
    slice of C5's 4,096-cluster mixture has 20 rows per cluster, so chunks
    span clusters and nothing is skipped."""
    import synth
    X, _ = synth.generate(cfg, n=n)
    kw = dict(n_buckets=nb, nprobe=1, M=64, K=32, rounds=2)
    print(f"pruning {cfg} n={n} buckets={nb}", flush=True)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, knn_prune=False):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists.view(np.uint32), b.knn_dists.view(np.uint32))
    np.testing.assert_array_equal(a.graph, b.graph)
    done, full = a.stats["knn_pairs_computed"], b.stats["knn_pairs_computed"]
    print(f"  pairs computed {done:.4g} of {full:.4g}", flush=True)
    if skips:
        assert done < full


def test_chunk_pruning_uniform_rows(ctx):
    # unclustered rows: chunks' spheres overlap every query; same table
    rng = np.random.default_rng(21)
    X = rng.integers(-127, 128, size=(20000, 64)).astype(np.int8)
    kw = dict(n_buckets=8, nprobe=2, M=32, K=16, rounds=2)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, knn_prune=False):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.graph, b.graph)


@pytest.mark.parametrize("window", [2, 16, 32])
def test_collect_threshold_window_sizes(ctx, window):
    # the unseeded pass's threshold window (32 tiles on builds of 2^22 rows
    # or more) changes how many keys are collected, never the lists
    rng = np.random.default_rng(41)
    N, B = 9000, 3
    X = _data(N, 128, seed=42, lo=-20, hi=21)
    off, mem = _buckets(rng, N, B)
    probe = _probe(rng, B, 1)
    print(f"collect window {window}", flush=True)
    with debug_opts(ctx, knn_window=window):
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, 64)
    ri, rd = O.knn_bucketed(X.astype(np.float32), off, mem, probe, 64)
    assert_knn_equal(ids, dist, ri, rd)
