"""Float-data build paths against the CPU oracle.

* Multi-round seeded bucketed kNN on float rows (C1 L2, C3 inner product, C4
  L2 at D = 960): each round's GPU table against the oracle's bucketed kNN of
  the same buckets merged into the oracle's running table; distances within
  1e-5 relative (plus the fp32 expanded-form floor of tests/helpers.py), ids
  equal except among ties.
* Whole builds on float data (C3 inner product, C1 L2): recall of the
  pre-prune table against the oracle's exact kNN, every returned distance the
  pair's own distance, and the graph equal, bit for bit, to the oracle's
  sanitize + CAGRA prune + reverse merge of the returned table.
"""
import numpy as np
import pytest

import gt_oracle as O
import synth
from helpers import assert_knn_close, floor_report

pytestmark = pytest.mark.gpu


def _buckets(rng, N, B):
    lab = rng.integers(0, B, size=N)
    lab[:B] = np.arange(B)
    order = np.argsort(lab, kind="stable")
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    return np.cumsum(off), order.astype(np.int32)


def _probe(rng, B, P):
    return np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32)


FLOOR_DECIDED_MAX = {"C1": 0.06, "C3": 0.0, "C4": 0.0005}


@pytest.mark.parametrize("cfg,N,B,P,M,rounds", [("C1", 6000, 12, 2, 64, 3), ("C3", 6000, 12, 2, 64, 3),
                                                ("C4", 3000, 8, 2, 96, 2)])
def test_knn_bucketed_float_rounds_match_oracle(ctx, cfg, N, B, P, M, rounds):
    X, _ = synth.generate(cfg, n=N)
    metric = synth.CONFIGS[cfg].metric
    mcode = 1 if metric == "ip" else 0
    rng = np.random.default_rng(N + B + M)
    run = ref = None
    print(f"float rounds {cfg} N={N} B={B} P={P} M={M}", flush=True)
    for r in range(rounds):
        off, mem = _buckets(rng, N, B)
        probe = _probe(rng, B, P)
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, metric=metric, running=run)
        ni, nd = O.knn_bucketed(X, off, mem, probe, M, metric=mcode)
        ref = (ni, nd) if ref is None else O.merge_rounds(*ref, ni, nd)
        run = (ids, dist)
        got_d = -dist if metric == "ip" else dist   # the library reports the inner product itself
        assert_knn_close(X, np.arange(N), ids, got_d, ref[0], ref[1], rtol=1e-5, metric=metric)
    st = floor_report()
    print(f"  floor statistics {cfg}: {st}", flush=True)
    # share of distance positions whose error exceeds 1e-5 relative (decided
    # by the floor): measured C1 5.2 % (88 % of rows), C3 none, C4 0.014 %
    assert st["positions_floor_decided"] <= FLOOR_DECIDED_MAX[cfg]


def _check_build(ctx, X, metric, n_buckets, M, K, min_recall, sample=1000):
    N = len(X)
    res = ctx.build_graph(X, n_buckets=n_buckets, nprobe=1, M=M, K=K, rounds=2, metric=metric)
    ids, dist = res.knn_ids, res.knn_dists
    assert (ids >= 0).all() and (ids < N).all()
    assert (ids != np.arange(N)[:, None]).all()
    assert all(len(set(r)) == M for r in ids[::97].tolist())
    # every distance is the pair's own distance (fp32 expanded form vs float64)
    X64 = X.astype(np.float64)
    rows = np.arange(0, N, 53)
    v = X64[ids[rows]]
    if metric == "ip":
        true = (v * X64[rows][:, None, :]).sum(-1)
        assert np.abs(dist[rows] - true).max() <= 1e-5 * np.abs(true).max() + 2.0 ** -21 * np.sqrt(X.shape[1])
        assert (np.diff(dist, axis=1) <= 0).all()       # descending inner product
    else:
        true = ((v - X64[rows][:, None, :]) ** 2).sum(-1)
        n2 = (X64 ** 2).sum(1)
        tol = 1e-5 * true + (n2[rows][:, None] + n2[ids[rows]]) * 2.0 ** -22 * np.sqrt(X.shape[1])
        assert (np.abs(dist[rows] - true) <= tol).all()
        assert (np.diff(dist, axis=1) >= 0).all()
    # recall@32 against the oracle's exact kNN on a sample
    q = np.sort(np.random.default_rng(3).choice(N, sample, replace=False))
    ex_i, _ = O.knn_exact(X, 32, queries=q, metric=1 if metric == "ip" else 0)
    rec = np.mean([len(np.intersect1d(ids[qq, :32], ex_i[j])) / 32 for j, qq in enumerate(q)])
    print(f"  build {metric} N={N}: recall@32 {rec:.4f}", flush=True)
    assert rec >= min_recall
    # the graph stages are integer: bit-exact given the returned table
    fwd, rc, _ = O.cagra_prune(O.sanitize(ids), K)
    assert rc == 0
    np.testing.assert_array_equal(res.graph, O.reverse_merge(fwd))


def test_build_graph_c3_inner_product(ctx):
    X, _ = synth.generate("C3", n=50000)
    print("build C3 IP N=50000", flush=True)
    _check_build(ctx, X, "ip", n_buckets=13, M=64, K=32, min_recall=0.97)


def test_build_graph_c1_float_l2(ctx):
    X, _ = synth.generate("C1", n=10000)
    print("build C1 L2 float N=10000", flush=True)
    _check_build(ctx, X, "l2", n_buckets=16, M=64, K=32, min_recall=0.97)
