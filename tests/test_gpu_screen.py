"""The fp16 screen ahead of fp32 collect passes (knn_screen; forced on
here with knn_screen=2, which also screens passes below the default's size
threshold).

The screen keeps, for each 128-query work item, the pool rows whose fp16
key less a rigorous bound on its gap to the fp32 key is at or below some
query's threshold -- the running M-th distance of a seeded pass, or in an
unseeded pass an upper bound on the pool's M-th smallest fp32 key from the
screen's own window (fp16 key plus the bound); the fp32 pass then scans only
those rows.  It must change nothing: every pass here is compared with the
unscreened pass from the same running table, ids and distance bits equal.
The cases press on the bound: rows far from the origin (the L2 key's
cancellation, where the norm term of the bound decides), rows of tiny and
of huge scale (the power-of-two scale of the fp16 copy), duplicated rows
(ties at the threshold), inner products of rows of varied norm, running
tables with padding (+inf thresholds: every row kept), every padded width
the screen takes (32 .. 160), and whole builds, resident and out of core
(compact output rows).  The unscreened passes are
themselves checked against the CPU oracle in tests/test_gpu_collect_f32.py
and tests/test_gpu_float.py.
"""

import numpy as np
import pytest

import synth
from helpers import debug_opts

pytestmark = pytest.mark.gpu


def _buckets(rng, N, B):
    lab = rng.integers(0, B, size=N)
    lab[:B] = np.arange(B)
    order = np.argsort(lab, kind="stable")
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    return np.cumsum(off), order.astype(np.int32)


def _probe(rng, B, P):
    if P == 0:
        return np.zeros((B, 0), np.int32)
    return np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32)


def _data(kind, n, d, seed):
    rng = np.random.default_rng(seed)
    if kind in ("C1", "C3"):
        X, _ = synth.generate(kind, n=n)
        return X
    C = rng.normal(size=(40, d)).astype(np.float32)
    X = C[rng.integers(0, 40, n)] + 0.3 * rng.normal(size=(n, d)).astype(np.float32)
    if kind == "offset":      # |x|^2 ~ 3e7 against distances ~ 10: the key cancels
        X = X + 500.0
    elif kind == "dup":       # every row four times: ties at every threshold
        X = np.repeat(X[: n // 4], 4, axis=0)
        X = X[rng.permutation(len(X))]
    elif kind == "scaled":    # rows of norms over three orders of magnitude
        X = X * np.exp(rng.uniform(-3.5, 3.5, size=(n, 1))).astype(np.float32)
    elif kind == "tiny":      # elements near fp16's subnormals before scaling
        X = X * np.float32(1e-9)
    elif kind == "huge":      # elements far beyond fp16's range before scaling
        X = X * np.float32(1e12)
    return np.ascontiguousarray(X, dtype=np.float32)


def _equal(x, y):
    np.testing.assert_array_equal(x[0], y[0])
    np.testing.assert_array_equal(x[1].view(np.uint32), y[1].view(np.uint32))


@pytest.mark.parametrize("kind,N,D,B,P,M,metric", [
    ("C1", 6000, 128, 12, 2, 64, "l2"),
    ("C3", 6000, 96, 12, 2, 64, "ip"),
    ("gauss", 4000, 32, 6, 1, 32, "l2"),
    ("gauss", 4000, 64, 6, 1, 17, "ip"),
    ("gauss", 3000, 160, 5, 1, 48, "l2"),
    ("gauss", 3000, 160, 5, 1, 64, "ip"),
    ("offset", 4000, 128, 6, 1, 32, "l2"),
    ("dup", 4000, 96, 6, 1, 32, "l2"),
    ("dup", 4000, 96, 6, 1, 32, "ip"),
    ("scaled", 4000, 128, 6, 1, 32, "ip"),
    ("scaled", 4000, 64, 6, 1, 32, "l2"),
    ("tiny", 3000, 96, 5, 1, 32, "l2"),
    ("huge", 3000, 64, 5, 1, 32, "ip"),
])
def test_screened_passes_equal_unscreened(ctx, kind, N, D, B, P, M, metric):
    X = _data(kind, N, D, seed=N + D + M)
    N = len(X)
    rng = np.random.default_rng(7 * N + M)
    print(f"screen rounds {kind} N={N} D={D} B={B} P={P} M={M} {metric}", flush=True)
    run = None   # the first pass unseeded: the screen's own window bound
    for r in range(3):
        off, mem = _buckets(rng, N, B)
        probe = _probe(rng, B, P)
        with debug_opts(ctx, knn_screen=2):
            got = ctx.knn_bucketed(X, off, mem, probe, M, metric=metric, running=run)
        with debug_opts(ctx, knn_screen=0):
            want = ctx.knn_bucketed(X, off, mem, probe, M, metric=metric, running=run)
        _equal(got, want)
        run = want


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_screen_with_padded_running_lists(ctx, metric):
    # a first round of small buckets without probes leaves lists with
    # (-1, +inf) padding: those queries keep their whole pools
    X = _data("gauss", 4000, 96, seed=11)
    N = len(X)
    rng = np.random.default_rng(12)
    off, mem = _buckets(rng, N, 400)
    # unseeded pools of fewer than M rows: the window bound is +inf
    with debug_opts(ctx, knn_screen=2):
        run = ctx.knn_bucketed(X, off, mem, _probe(rng, 400, 0), 32, metric=metric)
    with debug_opts(ctx, knn_screen=0):
        _equal(run, ctx.knn_bucketed(X, off, mem, _probe(rng, 400, 0), 32, metric=metric))
    assert (run[0] < 0).any()
    off, mem = _buckets(rng, N, 6)
    probe = _probe(rng, 6, 1)
    with debug_opts(ctx, knn_screen=2):
        got = ctx.knn_bucketed(X, off, mem, probe, 32, metric=metric, running=run)
    with debug_opts(ctx, knn_screen=0):
        want = ctx.knn_bucketed(X, off, mem, probe, 32, metric=metric, running=run)
    _equal(got, want)


@pytest.mark.parametrize("cfg,N", [("C3", 30000), ("C1", 20000)])
def test_screened_build_equals_unscreened(ctx, cfg, N):
    X, _ = synth.generate(cfg, n=N)
    metric = synth.CONFIGS[cfg].metric
    kw = dict(n_buckets=16, nprobe=1, M=64, K=32, rounds=2, metric=metric)
    print(f"screened build {cfg} N={N}", flush=True)
    with debug_opts(ctx, knn_screen=2):
        a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, knn_screen=0):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists.view(np.uint32), b.knn_dists.view(np.uint32))
    np.testing.assert_array_equal(a.graph, b.graph)
    # the screen dropped pool rows: the fp32 passes computed fewer pairs
    sa, sb = a.stats, b.stats
    print(f"  pairs {sa['knn_pairs']:.4g}, fp32 pairs screened {sa['knn_pairs_computed']:.4g}, "
          f"unscreened {sb['knn_pairs_computed']:.4g}", flush=True)
    assert sb["knn_pairs_computed"] == sb["knn_pairs"]
    assert sa["knn_pairs_computed"] < 0.8 * sa["knn_pairs"]


@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_screened_out_of_core_build_equals_unscreened(ctx, metric):
    # bucket chunks with compact output rows (each work item's rows through
    # its out_base), seeded from the host-resident running table
    X = _data("gauss", 40000, 96, seed=21)
    if metric == "ip":
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    kw = dict(n_buckets=24, M=32, K=16, rounds=2, nprobe=1, metric=metric, device_budget_mb=24)
    print(f"screened out-of-core build {metric}", flush=True)
    with debug_opts(ctx, knn_screen=2):
        a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, knn_screen=0):
        b = ctx.build_graph(X, **kw)
    assert a.stats["ooc_chunks"] > 3
    assert a.stats["knn_pairs_computed"] < a.stats["knn_pairs"]
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists.view(np.uint32), b.knn_dists.view(np.uint32))
    np.testing.assert_array_equal(a.graph, b.graph)
