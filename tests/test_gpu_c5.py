"""C5's own code paths against the CPU oracle, bit for bit.

C5 (10M x 128 int8, M 64 -> K 32) reaches two variants no smaller
configuration does:

* the prune of a table of 2 GiB or more (N * M * 4 bytes) fetches neighbour
  rows with 64-bit addresses instead of buffer loads; ``prune_flat_rows``
  forces that variant on small tables, which are compared with the oracle's
  CAGRA prune (src/prune_windowed_core.hpp:177-263) at M 64 and 96 with
  padding, repeated ids and spilled hash buckets;
* its rounds run int8 rows through the collect + select kNN at bucket sizes
  of about 5,000 rows.  A C5-shaped slice (200,000 rows of the C5 mixture, 40
  balanced buckets, one probe bucket, 2 rounds) is checked round by round
  against the oracle's bucketed kNN and cross-round merge, and a whole build
  of the same slice against the oracle's sanitize + prune + reverse merge of
  the table it returns, with both prune variants.
"""
import numpy as np
import pytest

import gt_oracle as O
import synth
from helpers import debug_opts

pytestmark = pytest.mark.gpu


def _rand_graph(rng, N, M, pad):
    G = rng.integers(0, N, size=(N, M)).astype(np.int32)
    G[rng.random((N, M)) < pad] = -1
    G[::7, 3] = G[::7, 1]        # repeated ids
    return G


@pytest.mark.parametrize("N,M,K,pad", [(1500, 64, 32, 0.002), (1000, 96, 48, 0.002), (3000, 32, 16, 0.0),
                                       (40000, 64, 32, 0.0), (600, 128, 64, 0.001)])
def test_prune_flat_rows_matches_oracle(ctx, N, M, K, pad):
    rng = np.random.default_rng(N + 3 * M)
    G = _rand_graph(rng, N, M, pad)
    ref, rc, _ = O.cagra_prune(G, K)
    assert rc == 0
    print(f"flat-row prune N={N} M={M} K={K}", flush=True)
    with debug_opts(ctx, prune_flat_rows=True):
        got = ctx.cagra_prune(G, K)
    np.testing.assert_array_equal(got, ref)
    np.testing.assert_array_equal(ctx.cagra_prune(G, K), ref)   # the buffer-load variant


@pytest.mark.parametrize("M,K,nbk", [(64, 32, 128), (96, 48, 256)])
def test_prune_flat_rows_spilled_buckets(ctx, M, K, nbk):
    # ids sharing a few home buckets of the per-row hash table (bits 15.. of
    # v * 0x9E3779B1 mod 2^32): full buckets spill, lookups probe several
    rng = np.random.default_rng(M + 1)
    N = 30000
    v = np.arange(N, dtype=np.uint64)
    home = ((v * 0x9E3779B1) % (1 << 32) >> 15) & (nbk - 1)
    G = rng.choice(np.flatnonzero(home < 3), size=(N, M)).astype(np.int32)
    G[::5, 1] = G[::5, 0]
    ref, rc, _ = O.cagra_prune(G, K)
    assert rc == 0
    with debug_opts(ctx, prune_flat_rows=True):
        np.testing.assert_array_equal(ctx.cagra_prune(G, K), ref)


def _c5_slice(n=200000):
    X, _ = synth.generate("C5", n=n)
    assert X.dtype == np.int8
    return X


def _balanced_buckets(X, B, seed):
    """Data-point centroids, nearest-two assignment with the two-choice rule
    of src/bucket.cu:2276-2302 (2nd bucket if its size < 0.8 x the 1st's,
    sizes counted in point order), probe = nearest other centroid."""
    rng = np.random.default_rng(seed)
    N = len(X)
    Xf = X.astype(np.float32)
    C = Xf[np.sort(rng.choice(N, B, replace=False))]
    t2 = np.argsort((C ** 2).sum(1)[None, :] - 2.0 * Xf @ C.T, axis=1, kind="stable")[:, :2]
    size = np.zeros(B, np.int64)
    lab = np.empty(N, np.int64)
    for i, (a, b) in enumerate(t2.tolist()):
        lab[i] = b if size[b] < 0.8 * size[a] else a
        size[lab[i]] += 1
    order = np.argsort(lab, kind="stable").astype(np.int32)
    off = np.zeros(B + 1, np.int64)
    np.add.at(off, lab + 1, 1)
    cd = ((C[:, None, :] - C[None, :, :]) ** 2).sum(-1)
    np.fill_diagonal(cd, np.inf)
    return np.cumsum(off), order, cd.argmin(1).astype(np.int32)[:, None]


def test_c5_shaped_rounds_match_oracle(ctx):
    X = _c5_slice()
    N, M = len(X), 64
    run = ref = None
    for r in range(2):
        off, mem, probe = _balanced_buckets(X, 40, seed=42 + r)
        print(f"C5 slice round {r + 1}: buckets {np.diff(off).min()}..{np.diff(off).max()} rows", flush=True)
        ids, dist = ctx.knn_bucketed(X, off, mem, probe, M, running=run)
        ni, nd = O.knn_bucketed_int(X, off, mem, probe, M)
        ref = (ni, nd) if ref is None else O.merge_rounds(*ref, ni, nd)
        np.testing.assert_array_equal(ids, ref[0])
        np.testing.assert_array_equal(dist.view(np.uint32), ref[1].view(np.uint32))
        run = (ids, dist)


def test_c5_shaped_build_graph_matches_oracle(ctx):
    X = _c5_slice()
    N = len(X)
    kw = dict(n_buckets=40, nprobe=1, M=64, K=32, rounds=2)
    print("C5 slice build", flush=True)
    res = ctx.build_graph(X, **kw)
    ids = res.knn_ids
    assert (ids >= 0).all() and (ids < N).all() and (ids != np.arange(N)[:, None]).all()
    # every distance is the pair's exact integer distance, rows ascending
    Xi = X.astype(np.int64)
    rows = np.arange(0, N, 101)
    true = ((Xi[ids[rows]] - Xi[rows][:, None, :]) ** 2).sum(-1)
    np.testing.assert_array_equal(res.knn_dists[rows], true.astype(np.float32))
    assert (np.diff(res.knn_dists, axis=1) >= 0).all()
    fwd, rc, _ = O.cagra_prune(O.sanitize(ids), 32)
    assert rc == 0
    ref = O.reverse_merge(fwd)
    np.testing.assert_array_equal(res.graph, ref)
    with debug_opts(ctx, prune_flat_rows=True):
        flat = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(flat.knn_ids, ids)
    np.testing.assert_array_equal(flat.graph, ref)
