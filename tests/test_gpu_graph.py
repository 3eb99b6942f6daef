"""GPU parity of the integer graph stages (sanitize, CAGRA prune, reverse-edge
merge, translate, end-to-end build) against the CPU oracle and the
reference's golden fixtures.  All bit-exact."""
import os

import numpy as np
import pytest

import gt_oracle as O
import synth
from helpers import debug_opts

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rand_graph(rng, N, M, pad=0.0, dup=True):
    if dup:
        G = rng.integers(0, N, size=(N, M)).astype(np.int32)
    else:
        G = np.stack([rng.permutation(np.delete(np.arange(N), i))[:M] for i in range(N)]).astype(np.int32)
    if pad:
        G[rng.random((N, M)) < pad] = -1
    return G


@pytest.mark.parametrize("M", [64, 32, 128, 16, 48, 7])
def test_sanitize_gpu(ctx, M):
    # the vector kernel (M in 16, 32, 64, 128) and the one-wave-per-row kernel
    rng = np.random.default_rng(M)
    N = 503
    G = rng.integers(-1, N + 100, size=(N, M)).astype(np.int32)
    G[3] = -1
    G[4] = 4
    G[N - 1] = N - 1   # self only: the fallback wraps to row 0
    G[7, :M // 2] = -5
    np.testing.assert_array_equal(ctx.sanitize(G), O.sanitize(G))


def test_prune_golden(ctx):
    z = np.load(os.path.join(GOLDEN, "prune_golden.npz"))
    import gtann
    for c in range(6):
        G, K = z[f"prune{c}_G"], int(z[f"prune{c}_K"])
        if int(z[f"prune{c}_rc"]) == 0:
            np.testing.assert_array_equal(ctx.cagra_prune(G, K), z[f"prune{c}_out"])
        else:
            with pytest.raises(gtann.GtannError) as e:
                ctx.cagra_prune(G, K)
            assert e.value.code == gtann.GT_EFEWCAND


@pytest.mark.parametrize("N,M,K,pad,dup", [(2000, 64, 32, 0.0, False), (1500, 64, 32, 0.0, True),
                                           (1000, 96, 48, 0.0, True), (800, 128, 64, 0.0, True),
                                           (3000, 32, 16, 0.001, True), (50, 7, 3, 0.0, True)])
def test_prune_random(ctx, N, M, K, pad, dup):
    rng = np.random.default_rng(N + M)
    G = _rand_graph(rng, N, M, pad, dup)
    ref, rc, _ = O.cagra_prune(G, K)
    assert rc == 0
    np.testing.assert_array_equal(ctx.cagra_prune(G, K), ref)


@pytest.mark.parametrize("M,K,nbk", [(64, 32, 128), (128, 64, 256)])
def test_prune_spilled_buckets(ctx, M, K, nbk):
    # rows drawn from ids that share a handful of home buckets of the
    # kernel's per-row hash table (multiplicative hash, bits 15.. of
    # v * 0x9E3779B1 mod 2^32): full buckets spill into the next ones, so
    # lookups probe several buckets (the path random rows rarely reach)
    rng = np.random.default_rng(M)
    N = 40000
    v = np.arange(N, dtype=np.uint64)
    home = ((v * 0x9E3779B1) % (1 << 32) >> 15) & (nbk - 1)
    pool = np.flatnonzero(home < 3)
    G = rng.choice(pool, size=(N, M)).astype(np.int32)
    G[::5, 1] = G[::5, 0]                        # repeated ids
    ref, rc, _ = O.cagra_prune(G, K)
    assert rc == 0
    np.testing.assert_array_equal(ctx.cagra_prune(G, K), ref)


def test_prune_few_candidates_error(ctx):
    import gtann
    G = np.array([[1, -1, -1], [0, 2, -1], [0, 1, -1]], np.int32)
    with pytest.raises(gtann.GtannError) as e:
        ctx.cagra_prune(G, 2)
    assert e.value.code == gtann.GT_EFEWCAND


def _assert_rows_equal(got, ref, F):
    bad = np.nonzero((got != ref).any(axis=1))[0]
    if len(bad):
        j = int(bad[0])
        raise AssertionError(f"{len(bad)} rows differ, first {j} (in-degree {int((F == j).sum())}):\n"
                             f"fwd {F[j].tolist()}\nref {ref[j].tolist()}\ngot {got[j].tolist()}")


def test_reverse_merge_golden(ctx):
    z = np.load(os.path.join(GOLDEN, "revmerge_golden.npz"))
    for c in range(4):
        F = z[f"rev{c}_F"]
        _assert_rows_equal(ctx.reverse_merge(F), z[f"rev{c}_out"], F)


@pytest.mark.parametrize("N,K,hub", [(5000, 32, False), (3000, 48, True), (2000, 64, True), (700, 1, False),
                                     (1000, 7, True), (30, 16, False), (100, 32, True), (60000, 32, True)])
def test_reverse_merge_random(ctx, N, K, hub):
    rng = np.random.default_rng(N * K)
    F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
    if hub:
        F[rng.random((N, K)) < 0.2] = 3
        F[rng.random((N, K)) < 0.05] = 5
    _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_csr_path(ctx):
    """The global-atomic CSR path (graphs beyond the binned path's limits),
    forced by revmerge_path='csr', gives the same rows."""
    with debug_opts(ctx, revmerge_path="csr"):
        for N, K in [(5000, 32), (3000, 48), (700, 1)]:
            rng = np.random.default_rng(N + K)
            F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
            F[rng.random((N, K)) < 0.2] = 3
            _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_two_kernel_path_forced(ctx):
    """The two-kernel merge wherever it applies (revmerge_path='rv'),
    including the output degrees and bin widths the default leaves to the
    binned merge (K > 32, 2^11-row bins) and rows beyond its LDS capacity."""
    with debug_opts(ctx, revmerge_path="rv"):
        for N, K, hub in [(3000, 48, True), (2000, 64, True), (70000, 48, False), (700, 1, False),
                          (5000, 32, True), (60000, 32, True), (2200000, 2, False)]:
            rng = np.random.default_rng(N * 11 + K)
            F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
            if hub:
                F[rng.random((N, K)) < 0.2] = 3
                F[rng.random((N, K)) < 0.05] = 5
            print(f"rv path N={N} K={K} hub={hub}", flush=True)
            _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_superbin_path_forced(ctx):
    """The two-kernel merge behind a level of superbins (revmerge_path='rv2',
    the default beyond 2^21 rows): several superbins at these sizes, K from 1
    to 64; the hub graphs send a quarter of all edges to two rows of the first
    superbin, so its level-two blocks overflow and the rows are redone by the
    binned merge."""
    with debug_opts(ctx, revmerge_path="rv2"):
        for N, K, hub in [(3000, 48, True), (70000, 48, False), (60000, 32, True), (200000, 32, False),
                          (2000, 64, True), (700, 1, False), (50000, 16, False), (131104, 24, False)]:
            rng = np.random.default_rng(N * 13 + K)
            F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
            if hub:
                F[rng.random((N, K)) < 0.2] = 3
                F[rng.random((N, K)) < 0.05] = 5
            print(f"rv2 path N={N} K={K} hub={hub}", flush=True)
            _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


@pytest.mark.parametrize("K", [8, 32])
def test_reverse_merge_default_beyond_2_21_rows(ctx, K):
    # graphs beyond 2^21 rows take the superbin path by default (C5's shape
    # at K 32, 2.2 M rows), checked against the oracle
    rng = np.random.default_rng(K)
    N = 2_200_000
    F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
    print(f"default path N={N} K={K}", flush=True)
    _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_binned_path(ctx):
    """The binned merge through global grouping (graphs between the two-kernel
    merge's 2^11 * 8192 rows and 2^26), forced by revmerge_path='binned'."""
    with debug_opts(ctx, revmerge_path="binned"):
        for N, K in [(5000, 32), (3000, 48), (700, 1), (20000, 16)]:
            rng = np.random.default_rng(N * 7 + K)
            F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
            F[rng.random((N, K)) < 0.2] = 3
            _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_oversize_bins(ctx):
    """256-row bins of the two-kernel merge around its fast path's limits
    (9,087 keys of LDS group buffer at this size, 9,216 in registers): bins
    beyond them go to the deferred kernel.  In-degrees set exactly: bin 5 36
    per row (9,216 keys), bin 9 40 (10,240), bin 30 72 in its first half and
    0 in its second (9,216 keys on 128 rows); every other bin about 8,100."""
    rng = np.random.default_rng(11)
    N, K = 256 * 48, 32
    deg = np.zeros(N, np.int64)
    deg[256 * 5:256 * 6] = 36
    deg[256 * 9:256 * 10] = 40
    deg[256 * 30:256 * 30 + 128] = 72
    rest = np.ones(N, bool)
    rest[256 * 5:256 * 6] = rest[256 * 9:256 * 10] = rest[256 * 30:256 * 31] = False
    left = N * K - deg.sum()
    idx = np.flatnonzero(rest)
    deg[idx] = left // len(idx)
    deg[idx[:left % len(idx)]] += 1
    F = rng.permutation(np.repeat(np.arange(N), deg)).reshape(N, K).astype(np.uint32)
    keys = np.bincount(F.ravel() >> 8, minlength=48)
    assert keys[5] == 9216 and keys[9] == 10240 and keys[30] == 9216
    _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


@pytest.mark.parametrize("N,K", [(200000, 32), (70000, 64), (33, 8), (4097 * 32, 16)])
def test_reverse_merge_bin_edges(ctx, N, K):
    # sizes around the bin boundaries (a last bin of one row; many bins),
    # long in-lists (> 64 keys) and rows without any reverse edge
    rng = np.random.default_rng(N ^ K)
    F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
    F[rng.random((N, K)) < 0.01] = N - 1
    F[:, K // 2:][rng.random((N, K - K // 2)) < 0.3] = 0
    _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_distinct_rows_with_hubs(ctx):
    # rows without repeated ids (as the prune writes them) and a skewed
    # in-degree: the long in-lists take the chunked selection, not the
    # repeated-source fallback
    rng = np.random.default_rng(17)
    N, K = 30000, 32
    w = 1.0 / (1.0 + np.arange(N)) ** 0.9
    w /= w.sum()
    draws = rng.choice(N, size=(N, 6 * K), p=w)
    rows = []
    for r in draws:
        u, first = np.unique(r, return_index=True)
        rows.append(u[np.argsort(first)][:K])   # distinct ids in draw order
    assert min(len(r) for r in rows) == K
    F = np.stack(rows).astype(np.uint32)[rng.permutation(N)]
    assert np.bincount(F.ravel(), minlength=N).max() > 1000
    _assert_rows_equal(ctx.reverse_merge(F), O.reverse_merge(F), F)


def test_reverse_merge_out_of_range(ctx):
    import gtann
    F = np.zeros((10, 4), np.uint32)
    F[2, 1] = 10
    with pytest.raises(gtann.GtannError):
        ctx.reverse_merge(F)


def test_optimize_equals_prune_then_merge(ctx):
    rng = np.random.default_rng(5)
    G = _rand_graph(rng, 3000, 64, 0.0, False).view(np.uint32)
    ref, rc, _ = O.cagra_prune(G, 32)
    ref = O.reverse_merge(ref)
    np.testing.assert_array_equal(ctx.optimize(G, 32), ref)


def test_translate_gpu(ctx):
    z = np.load(os.path.join(GOLDEN, "translate_golden.npz"))
    for c in range(2):
        np.testing.assert_array_equal(ctx.translate(z[f"tr{c}_g"], z[f"tr{c}_inv"]), z[f"tr{c}_out"])
    import gtann
    with pytest.raises(gtann.GtannError):
        ctx.translate(np.zeros((3, 2), np.uint32), np.array([0, 0, 1], np.uint32))


def _structural(graph, N, K):
    assert graph.shape == (N, K)
    assert (graph < N).all()
    assert (graph != np.arange(N)[:, None]).all(), "self loop"


def test_build_graph_c1_end_to_end(ctx):
    """The whole build on C1 with every bucket probed: the pre-prune table is the
    exact kNN and the final graph equals oracle prune + merge of it."""
    X, _ = synth.generate("C1")
    X = np.rint(X * 8).astype(np.float32)   # integer-valued C1: exact distances
    res = ctx.build_graph(X, n_buckets=16, nprobe=15, M=64, K=32, rounds=1)
    ex_i, ex_d = O.knn_exact(X, 64)
    np.testing.assert_array_equal(res.knn_ids, ex_i)
    np.testing.assert_array_equal(res.knn_dists, ex_d)
    san = O.sanitize(res.knn_ids)
    fwd, rc, _ = O.cagra_prune(san, 32)
    assert rc == 0
    np.testing.assert_array_equal(res.graph, O.reverse_merge(fwd))
    _structural(res.graph, len(X), 32)


@pytest.mark.parametrize("n_buckets,nprobe", [(400, 0), (60, 1)])
def test_build_graph_padded_table(ctx, n_buckets, nprobe):
    """Buckets smaller than M + 1: the table carries -1 padding, which the
    build's sanitize replaces before the prune; the graph equals the oracle's
    sanitize + prune + merge of the returned table."""
    X, _ = synth.generate("C1", n=4000)
    X = np.rint(X * 8).astype(np.float32)
    res = ctx.build_graph(X, n_buckets=n_buckets, nprobe=nprobe, M=32, K=16, rounds=1, kmeans_iters=0,
                          balance=0.0)
    if n_buckets == 400:
        assert (res.knn_ids < 0).any()
    fwd, rc, _ = O.cagra_prune(O.sanitize(res.knn_ids), 16)
    assert rc == 0
    np.testing.assert_array_equal(res.graph, O.reverse_merge(fwd))


def test_build_graph_recall_c2_small(ctx):
    X, _ = synth.generate("C2", n=60000)
    res = ctx.build_graph(X, n_buckets=16, M=64, K=32, rounds=2)
    q = np.random.default_rng(0).choice(len(X), 500, replace=False)
    ex_i, _ = O.knn_exact(X, 32, queries=q)
    rec = np.mean([len(np.intersect1d(res.knn_ids[qq, :32], ex_i[r])) / 32 for r, qq in enumerate(q)])
    assert rec > 0.9, rec
    _structural(res.graph, len(X), 32)
    # the final graph is exactly oracle(prune + merge) of the returned table
    san = O.sanitize(res.knn_ids)
    np.testing.assert_array_equal(ctx.sanitize(res.knn_ids), san)
    fwd, rc, _ = O.cagra_prune(san, 32)
    assert rc == 0
    gfwd = ctx.cagra_prune(san, 32)
    _assert_rows_equal(gfwd, fwd, san)
    _assert_rows_equal(ctx.reverse_merge(fwd), O.reverse_merge(fwd), fwd)
    _assert_rows_equal(res.graph, O.reverse_merge(fwd), fwd)


# ------------------------------------------------------- Python-pipeline stages

def _int_data(rng, N, D, hi=255):
    return rng.integers(0, hi + 1, size=(N, D)).astype(np.float32)


@pytest.mark.parametrize("N,D,M,maxdeg", [(3000, 128, 64, 32), (2000, 100, 64, 0), (1500, 32, 20, 8),
                                          (1200, 64, 96, 48), (900, 96, 128, 64), (64, 32, 40, 0)])
def test_prune_occlusion_matches_oracle(ctx, N, D, M, maxdeg):
    rng = np.random.default_rng(N + M)
    X = _int_data(rng, N, D)
    nb = rng.integers(-1, N + 5, size=(N, M)).astype(np.int32)    # padding, out of range
    nb[::7, 0] = np.arange(0, N, 7)                                # self
    nb[::5, 3] = nb[::5, 2]                                        # duplicates
    print(f"occlusion N={N} D={D} M={M} maxdeg={maxdeg}", flush=True)
    got = ctx.prune_occlusion(X, nb, maxdeg)
    want = O.prune_occlusion(X, nb.astype(np.int64), maxdeg)
    np.testing.assert_array_equal(got, want)


def test_prune_occlusion_on_knn_lists_u8(ctx):
    rng = np.random.default_rng(3)
    X = rng.integers(0, 256, size=(4000, 128)).astype(np.uint8)
    ids, _ = O.knn_exact(X.astype(np.float32), 64)
    got = ctx.prune_occlusion(X, ids, 32)
    want = O.prune_occlusion(X.astype(np.float32), ids.astype(np.int64), 32)
    np.testing.assert_array_equal(got, want)


def test_prune_occlusion_float_data(ctx):
    # non-integer data: a decision can flip only on a near-tie of fp32 sums
    X, _ = synth.generate("C1", n=3000)
    ids, _ = O.knn_exact(X, 48)
    got = ctx.prune_occlusion(X, ids, 24)
    want = O.prune_occlusion(X, ids.astype(np.int64), 24)
    assert (got == want).all(axis=1).mean() >= 0.999


def test_prune_occlusion_matches_reference_python(ctx):
    # fixtures written by bd/prune.py:prune_graph itself (tests/golden/make_golden_py.py):
    # integer cases exact, float cases at least 1e-3 relative from every tie
    z = np.load(os.path.join(GOLDEN, "pyref_golden.npz"))
    n = len([k for k in z.files if k.endswith("_nb")])
    for c in range(n):
        print(f"occlusion vs prune_graph case {c} ({z[f'occ{c}_kind']})", flush=True)
        got = ctx.prune_occlusion(z[f"occ{c}_X"], z[f"occ{c}_nb"].astype(np.int32), int(z[f"occ{c}_maxdeg"]))
        np.testing.assert_array_equal(got.astype(np.int64), z[f"occ{c}_out"], err_msg=f"case {c}")


def test_reverse_insert_matches_reference_python(ctx):
    # fixtures written by bd/build_bucket.py:_apply_reverse_edges itself, tie-free tables
    z = np.load(os.path.join(GOLDEN, "pyref_golden.npz"))
    n = len([k for k in z.files if k.startswith("rin") and k.endswith("_out_ids")])
    for c in range(n):
        print(f"reverse insert vs _apply_reverse_edges case {c}", flush=True)
        gi, gd = ctx.reverse_insert(z[f"rin{c}_ids"], z[f"rin{c}_d"])
        np.testing.assert_array_equal(gi, z[f"rin{c}_out_ids"], err_msg=f"case {c}")
        np.testing.assert_array_equal(gd, z[f"rin{c}_out_d"], err_msg=f"case {c}")


def _offer_table(rng, X, M):
    ids, d = O.knn_exact(X, M)
    # degrade: drop some true neighbours so that offers exist
    N = len(X)
    keep = rng.random((N, M)) < 0.7
    far = rng.integers(0, N, size=(N, M)).astype(np.int32)
    Xi = X.astype(np.int64)
    ids = np.where(keep, ids, far).astype(np.int32)
    d = ((Xi[ids] - Xi[:, None, :]) ** 2).sum(axis=2).astype(np.float32)
    d[ids == np.arange(N)[:, None]] = np.inf
    ids[ids == np.arange(N)[:, None]] = -1
    o = np.lexsort((ids.view(np.uint32), d), axis=1)
    return np.take_along_axis(ids, o, 1), np.take_along_axis(d, o, 1)


@pytest.mark.parametrize("N,D,M", [(3000, 32, 64), (2000, 16, 32), (1000, 8, 128), (500, 4, 16)])
def test_reverse_insert_matches_oracle(ctx, N, D, M):
    rng = np.random.default_rng(N * 3 + M)
    X = _int_data(rng, N, D, 15)
    ids, d = _offer_table(rng, X, M)
    print(f"reverse insert N={N} D={D} M={M}", flush=True)
    gi, gd = ctx.reverse_insert(ids, d)
    oi, od = O.reverse_insert(ids, d)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


def test_reverse_insert_hub_and_repeats(ctx):
    # one target offered by nearly every row (>> 64 offers: several chunks),
    # repeated offers of the same source, padded rows
    rng = np.random.default_rng(9)
    N, M = 1500, 16
    ids = rng.integers(0, N, size=(N, M)).astype(np.int32)
    d = np.sort(rng.integers(1, 50, size=(N, M)).astype(np.float32), axis=1)
    ids[:, 0] = 7
    d[:, 0] = rng.integers(0, 3, size=N)
    ids[::3, 1] = ids[::3, 0]
    d[::3, 1] = d[::3, 0]
    d[7] = 1000.0
    ids[11, 8:], d[11, 8:] = -1, np.inf
    o = np.lexsort((ids.view(np.uint32), d), axis=1)
    ids, d = np.take_along_axis(ids, o, 1), np.take_along_axis(d, o, 1)
    gi, gd = ctx.reverse_insert(ids, d)
    oi, od = O.reverse_insert(ids, d)
    np.testing.assert_array_equal(gi, oi)
    np.testing.assert_array_equal(gd, od)


def test_reverse_insert_out_of_range(ctx):
    import gtann
    ids = np.zeros((10, 4), np.int32)
    ids[3, 2] = 10
    with pytest.raises(gtann.GtannError) as e:
        ctx.reverse_insert(ids, np.ones((10, 4), np.float32))
    assert e.value.code == gtann.GT_EINVAL


def test_build_graph_reverse_edges_rounds(ctx):
    # the Python pipeline's rounds (full table + reverse edges + merge) equal
    # the oracle's composition of the same steps on the GPU's own round tables
    X, _ = synth.generate("C1", n=4000)
    X = np.rint(X * 8).astype(np.float32)   # integer-valued: exact, symmetric distances
    r = ctx.build_graph(X, n_buckets=8, nprobe=7, M=32, K=16, rounds=2, kmeans_iters=0, reverse_edges=True,
                        prune=False)
    ex_i, ex_d = O.knn_exact(X, 32)
    # the probes cover every bucket, so each round's table is exact, and an
    # offer below a row's worst is then already in the row: the result is
    # the exact table
    np.testing.assert_array_equal(r.knn_ids, ex_i)
    np.testing.assert_array_equal(r.knn_dists, ex_d)
    assert r.graph is None
    # one probe: the rounds are approximate; the merged table keeps its
    # invariants (sorted, no self, no duplicates, exact distances)
    r2 = ctx.build_graph(X, n_buckets=8, nprobe=1, M=32, K=16, rounds=2, kmeans_iters=0, reverse_edges=True,
                         prune=False)
    d2 = r2.knn_dists
    assert (np.diff(d2, axis=1) >= 0).all()
    assert (d2 >= ex_d).all()
    for q in range(0, len(X), 97):
        v = r2.knn_ids[q][r2.knn_ids[q] >= 0]
        assert len(set(v.tolist())) == len(v) and q not in v
        np.testing.assert_array_equal(d2[q][:len(v)], ((X[v] - X[q]) ** 2).sum(axis=1))


def test_build_graph_wide_probe_table(ctx):
    """nprobe above the kernels' list length (probe table computed exactly on
    the host): with every other bucket probed the table is the exact kNN."""
    rng = np.random.default_rng(31)
    X = rng.integers(0, 40, size=(12000, 32)).astype(np.float32)
    res = ctx.build_graph(X, n_buckets=160, nprobe=159, M=32, K=16, rounds=1, kmeans_iters=1)
    ex_i, ex_d = O.knn_exact(X, 32)
    np.testing.assert_array_equal(res.knn_ids, ex_i)
    np.testing.assert_array_equal(res.knn_dists, ex_d)


def test_sub_centroid_order_does_not_change_the_build(ctx):
    """The unseeded own-bucket pass scans members ordered by nearest
    sub-centroid; the exact top-M does not depend on the order of the pool,
    so the two-choice order (sub_order=False) gives the same table and graph."""
    import synth
    X, _ = synth.generate("C2", n=40000)
    kw = dict(n_buckets=12, nprobe=2, M=64, K=32, rounds=2)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, sub_order=False):
        b = ctx.build_graph(X, **kw)
        c = ctx.build_graph(X.astype(np.float32) + 0.25, **kw)   # float rows: the fp32 kernel
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists, b.knn_dists)
    np.testing.assert_array_equal(a.graph, b.graph)
    d = ctx.build_graph(X.astype(np.float32) + 0.25, **kw)
    np.testing.assert_array_equal(c.knn_ids, d.knn_ids)
    np.testing.assert_array_equal(c.graph, d.graph)


@pytest.mark.parametrize("dtype,n_buckets", [("f32", 37), ("i8", 24), ("f32", 300)])
def test_lloyd_device_csr_matches_host(ctx, dtype, n_buckets):
    """The Lloyd steps group the sampled rows by nearest centroid on the
    device (stable counting sort); the host's counting sort
    (lloyd_host_csr=True) gives the same CSR, hence the same centroids and the
    same build.  300 buckets over 40,000 rows leaves some centroids with few
    or no sampled members."""
    import synth
    X, _ = synth.generate("C2", n=40000)
    if dtype == "i8":
        X = (X.astype(np.int64) - 128).clip(-128, 127).astype(np.int8)
    print(f"lloyd csr {dtype} buckets={n_buckets}", flush=True)
    kw = dict(n_buckets=n_buckets, nprobe=1, M=32, K=16, rounds=2, kmeans_iters=3)
    a = ctx.build_graph(X, **kw)
    with debug_opts(ctx, lloyd_host_csr=True):
        b = ctx.build_graph(X, **kw)
    np.testing.assert_array_equal(a.knn_ids, b.knn_ids)
    np.testing.assert_array_equal(a.knn_dists, b.knn_dists)
    np.testing.assert_array_equal(a.graph, b.graph)
