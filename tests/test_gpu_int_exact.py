"""Float rows whose values are all integers in [-128, 127] or [0, 255] run the
point kNN on the int8 matrix cores (gt_build_params.int_exact, on by
default).  Every distance is then an exact integer below 2^24 in both the
int8 and the fp32 kernel, so the two builds must agree bit for bit: table,
distances and graph, Lloyd-moved (fp32) centroids included."""
import numpy as np
import pytest

import gt_oracle as O
import synth
from helpers import assert_knn_equal

pytestmark = pytest.mark.gpu


def _both(ctx, X, **kw):
    a = ctx.build_graph(X, int_exact=True, **kw)
    b = ctx.build_graph(X, int_exact=False, **kw)
    return a, b


@pytest.mark.parametrize("lo,hi,metric", [(0, 256, "l2"), (-128, 128, "l2"), (-40, 41, "ip")])
def test_builds_identical(ctx, lo, hi, metric):
    rng = np.random.default_rng(hi - lo)
    X = rng.integers(lo, hi, size=(20000, 96)).astype(np.float32)
    X[:, :6] = (np.arange(20000)[:, None] % 11 * (hi - lo) // 11 + lo).astype(np.float32)   # structure
    a, b = _both(ctx, X, n_buckets=16, nprobe=2, M=48, K=24, rounds=2, kmeans_iters=3, metric=metric)
    assert a.stats["knn_int8"] == 1 and b.stats["knn_int8"] == 0
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists.view(np.uint32), b.knn_dists.view(np.uint32))
    np.testing.assert_array_equal(a.graph, b.graph)


def test_c2_shape_build_identical(ctx):
    X, _ = synth.generate("C2", n=60000)
    a, b = _both(ctx, X, n_buckets=32, M=64, K=32, rounds=2)
    assert a.stats["knn_int8"] == 1
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.graph, b.graph)


@pytest.mark.parametrize("bad", ["fraction", "range", "negative_with_255"])
def test_non_int8_rows_stay_fp32(ctx, bad):
    rng = np.random.default_rng(3)
    X = rng.integers(0, 200, size=(3000, 64)).astype(np.float32)
    if bad == "fraction":
        X[1234, 5] += 0.5
    elif bad == "range":
        X[77, 3] = 300.0
    else:
        X[5, 0], X[6, 1] = -1.0, 255.0   # fits neither [-128, 127] nor [0, 255]
    a = ctx.build_graph(X, n_buckets=4, M=16, K=8, rounds=1, kmeans_iters=0)
    assert a.stats["knn_int8"] == 0
    b = ctx.build_graph(X, n_buckets=4, M=16, K=8, rounds=1, kmeans_iters=0, int_exact=False)
    np.testing.assert_array_equal(a.graph, b.graph)


def test_exact_knn_on_integer_float_rows(ctx):
    # gt_knn_exact always takes the int8 path for such rows: bit-exact vs the oracle
    rng = np.random.default_rng(4)
    X = rng.integers(0, 256, size=(4000, 128)).astype(np.float32)
    ids, d = ctx.knn_exact(X, 32)
    rid, rd = O.knn_exact(X, 32)
    assert_knn_equal(ids, d, rid, rd)
