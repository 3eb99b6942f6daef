"""Out-of-core stages on the GPU: the windowed prune against the oracle, the
multi-chunk reverse merge and the out-of-core build (a device budget far
below the tables) against their resident counterparts, bit for bit."""
import numpy as np
import pytest

import gt_oracle as O
from helpers import bucketed_graph

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed,N,nb,M,K,W,budget", [
    (1, 3000, 30, 32, 16, 4, 0),            # one chunk
    (2, 3000, 30, 32, 16, 4, 200_000),      # several chunks of positions
    (3, 20000, 64, 64, 32, 5, 1_000_000),
    (4, 4000, 12, 100, 40, 3, 600_000),     # two list halves (M > 64)
    (5, 2000, 50, 16, 8, 1, 30_000),        # windows of the own bucket only
])
def test_prune_windowed_matches_oracle(ctx, seed, N, nb, M, K, W, budget):
    rng = np.random.default_rng(seed)
    G, off, win, wl = bucketed_graph(rng, N, nb, M, W)
    print(f"windowed N={N} nb={nb} M={M} K={K} W={W} budget={budget}", flush=True)
    ref, rc, _ = O.prune_windowed(G, off, win, wl, K)
    assert rc == 0
    got = ctx.prune_windowed(G, off, win, wl, K, device_budget_bytes=budget)
    bad = np.nonzero((got != ref).any(axis=1))[0]
    assert len(bad) == 0, f"{len(bad)} rows differ, first {bad[:5].tolist()}"


def test_prune_windowed_full_windows_equal_prune(ctx):
    rng = np.random.default_rng(9)
    G, off, _, _ = bucketed_graph(rng, 5000, 20, 32, 2)
    nb = len(off) - 1
    win = np.tile(np.arange(nb, dtype=np.int32), (nb, 1))
    got = ctx.prune_windowed(G, off, win, np.full(nb, nb, np.int32), 16, device_budget_bytes=0)
    np.testing.assert_array_equal(got, ctx.cagra_prune(G.view(np.uint32), 16))


def test_prune_windowed_padding_and_errors(ctx):
    import gtann
    rng = np.random.default_rng(4)
    G, off, win, wl = bucketed_graph(rng, 2000, 10, 24, 3, pad=0.2)
    ref, rc, _ = O.prune_windowed(G, off, win, wl, 8)
    if rc == 0:
        np.testing.assert_array_equal(ctx.prune_windowed(G, off, win, wl, 8, device_budget_bytes=100_000), ref)
    G[7, :20] = -1   # fewer than K valid candidates
    with pytest.raises(gtann.GtannError):
        ctx.prune_windowed(G, off, win, wl, 8)
    bad_win = win.copy()
    bad_win[0, 0] = len(off)   # a position beyond the buckets
    with pytest.raises(gtann.GtannError):
        ctx.prune_windowed(G, off, bad_win, wl, 8)


@pytest.mark.parametrize("N,K,hub,budget", [(60000, 32, True, 2_000_000), (30000, 16, False, 600_000),
                                            (5000, 48, True, 1_500_000), (100000, 32, False, 0),
                                            (40000, 32, "spread", 1_000_000)])
def test_reverse_merge_chunked_equals_resident(ctx, N, K, hub, budget):
    """Hubs send a destination chunk more edges than its share of the budget:
    one row with 10 % of all edges (merged alone), or 30 % of the edges over
    the first 2,000 rows (merged in row ranges that fit)."""
    rng = np.random.default_rng(N + K)
    F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
    if hub == "spread":
        sel = rng.random((N, K)) < 0.3
        F[sel] = rng.integers(0, 2000, size=int(sel.sum())).astype(np.uint32)
    elif hub:
        F[rng.random((N, K)) < 0.1] = 7
    print(f"chunked merge N={N} K={K} hub={hub} budget={budget}", flush=True)
    np.testing.assert_array_equal(ctx.reverse_merge_chunked(F, budget), ctx.reverse_merge(F))


def test_reverse_merge_chunked_oracle_and_errors(ctx):
    import gtann
    rng = np.random.default_rng(3)
    F = rng.integers(0, 3000, size=(3000, 24)).astype(np.uint32)
    np.testing.assert_array_equal(ctx.reverse_merge_chunked(F, 100_000), O.reverse_merge(F))
    F[5, 3] = 3000
    with pytest.raises(gtann.GtannError):
        ctx.reverse_merge_chunked(F, 100_000)


def _int_data(N, D, seed):
    rng = np.random.default_rng(seed)
    C = rng.integers(0, 256, size=(64, D))
    X = C[rng.integers(0, 64, N)] + rng.normal(0, 12, size=(N, D))
    return np.clip(np.rint(X), 0, 255).astype(np.float32)


@pytest.mark.parametrize("rounds,nprobe,metric", [(2, 1, "l2"), (3, 2, "l2"), (1, 0, "l2"), (2, 1, "ip")])
def test_build_out_of_core_equals_resident(ctx, rounds, nprobe, metric):
    """A device budget far below the tables: the running table lives in host
    memory and moves bucket chunk by bucket chunk; the prune and the reverse
    merge run in row chunks.  Same table and graph as the resident build."""
    if metric == "ip":
        rng = np.random.default_rng(8)
        X = rng.normal(size=(40000, 48)).astype(np.float32)
        X /= np.linalg.norm(X, axis=1, keepdims=True)
    else:
        X = _int_data(60000, 64, rounds)
    kw = dict(n_buckets=24, M=32, K=16, rounds=rounds, nprobe=nprobe, metric=metric)
    print(f"ooc build rounds={rounds} nprobe={nprobe} metric={metric}", flush=True)
    res = ctx.build_graph(X, **kw)
    ooc = ctx.build_graph(X, device_budget_mb=24, **kw)
    assert res.stats["ooc_chunks"] == 0 and ooc.stats["ooc_chunks"] > 3
    np.testing.assert_array_equal(ooc.knn_ids, res.knn_ids)
    np.testing.assert_array_equal(ooc.knn_dists, res.knn_dists)
    np.testing.assert_array_equal(ooc.graph, res.graph)


def test_build_out_of_core_c2(ctx):
    """Configuration C2 (1M x 128 integer-valued rows, 256 buckets, 64 -> 32)
    with a 512 MiB device budget for the tables (the resident build holds
    about 4.3 GB): identical table and graph."""
    import synth
    X, _ = synth.generate("C2")
    kw = dict(n_buckets=256, M=64, K=32, rounds=2, nprobe=1)
    print("ooc build C2", flush=True)
    res = ctx.build_graph(X, **kw)
    ooc = ctx.build_graph(X, device_budget_mb=512, **kw)
    print(f"ooc chunks {ooc.stats['ooc_chunks']}, {ooc.stats['t_total']:.2f} s "
          f"(resident {res.stats['t_total']:.3f} s)", flush=True)
    assert ooc.stats["ooc_chunks"] > 10
    assert np.array_equal(ooc.knn_ids, res.knn_ids) and np.array_equal(ooc.knn_dists, res.knn_dists)
    assert np.array_equal(ooc.graph, res.graph)


def test_build_out_of_core_rejects_refinement(ctx):
    import gtann
    X = _int_data(5000, 32, 1)
    with pytest.raises(gtann.GtannError):
        ctx.build_graph(X, n_buckets=8, M=16, K=8, refine_passes=1, device_budget_mb=1)
