"""Pins the CPU oracle (oracle/gt_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something other than itself: the
reference's golden fixtures (tests/golden/, written from the reference's own
headers), hand-computed known answers, closed forms, and independent numpy
brute force on integer data.
"""
import os

import numpy as np
import pytest

import gt_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _np_knn(X, k, metric="l2"):
    """independent brute force: int64 arithmetic on integer data, lexsort by (d, id)"""
    Xi = X.astype(np.int64)
    N = len(X)
    ids = np.empty((N, k), np.int64)
    ds = np.empty((N, k), np.int64)
    for q in range(N):
        if metric == "ip":
            d = -(Xi @ Xi[q])
        else:
            d = ((Xi - Xi[q]) ** 2).sum(axis=1)
        order = np.lexsort((np.arange(N), d))
        order = order[order != q][:k]
        ids[q], ds[q] = order, d[order]
    return ids, ds


# ---------------------------------------------------------------- kNN

def test_knn_exact_line_known_answer():
    # points on a line at 0, 1, 3, 6, 10: neighbours of x=3 are 1 (d=4), then
    # 0 and 6 tied at d=9 (lower id first), then 10 (d=49)
    X = np.array([[0], [1], [3], [6], [10]], np.float32)
    ids, d = O.knn_exact(X, 4)
    assert ids[2].tolist() == [1, 0, 3, 4]
    assert d[2].tolist() == [4.0, 9.0, 9.0, 49.0]
    assert ids[0].tolist() == [1, 2, 3, 4] and d[0].tolist() == [1, 9, 36, 100]


def test_knn_exact_matches_numpy_bruteforce_integer():
    rng = np.random.default_rng(3)
    X = rng.integers(0, 256, size=(300, 128)).astype(np.float32)
    X[7] = X[11]   # duplicate point: distance 0
    ids, d = O.knn_exact(X, 20)
    rid, rd = _np_knn(X, 20)
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_array_equal(d, rd.astype(np.float32))
    assert ids[7, 0] == 11 and d[7, 0] == 0.0


def test_knn_exact_ip_equals_l2_on_unit_vectors():
    # <x,y> = 1 - |x-y|^2 / 2 on the unit sphere: identical rankings
    rng = np.random.default_rng(4)
    X = rng.standard_normal((400, 32)).astype(np.float32)
    X /= np.linalg.norm(X, axis=1, keepdims=True)
    i_ip, d_ip = O.knn_exact(X, 10, metric=1)
    i_l2, d_l2 = O.knn_exact(X, 10, metric=0)
    np.testing.assert_allclose(-d_ip, 1 - d_l2 / 2, atol=1e-6)
    assert (i_ip == i_l2).mean() > 0.99


def test_knn_exact_query_subset_and_keep_self():
    rng = np.random.default_rng(5)
    X = rng.integers(0, 50, size=(120, 16)).astype(np.float32)
    q = np.array([5, 17, 100])
    ids, d = O.knn_exact(X, 5, queries=q)
    full, fd = O.knn_exact(X, 5)
    np.testing.assert_array_equal(ids, full[q])
    ids2, d2 = O.knn_exact(X, 5, queries=q, exclude_self=False)
    assert (ids2[:, 0] == q).all() and (d2[:, 0] == 0).all()


def _buckets(rng, N, B):
    lab = rng.integers(0, B, size=N)
    lab[:B] = np.arange(B)
    order = np.argsort(lab, kind="stable")
    offsets = np.zeros(B + 1, np.int64)
    np.add.at(offsets, lab + 1, 1)
    return np.cumsum(offsets), order.astype(np.int32), lab


def test_knn_bucketed_all_probed_equals_exact():
    # config C1's rule: nprobe = buckets - 1 makes the pooled kNN exact
    rng = np.random.default_rng(6)
    X = rng.integers(0, 256, size=(500, 64)).astype(np.float32)
    off, mem, _ = _buckets(rng, 500, 8)
    probe = np.array([[b2 for b2 in range(8) if b2 != b] for b in range(8)], np.int32)
    ids, d = O.knn_bucketed(X, off, mem, probe, 16)
    eids, ed = O.knn_exact(X, 16)
    np.testing.assert_array_equal(ids, eids)
    np.testing.assert_array_equal(d, ed)


def test_knn_bucketed_matches_numpy_per_bucket():
    rng = np.random.default_rng(7)
    N, B, P, M = 400, 10, 2, 12
    X = rng.integers(0, 100, size=(N, 32)).astype(np.float32)
    off, mem, lab = _buckets(rng, N, B)
    probe = np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32)
    ids, d = O.knn_bucketed(X, off, mem, probe, M)
    Xi = X.astype(np.int64)
    for q in range(0, N, 7):
        b = lab[q]
        pool = np.concatenate([np.nonzero(lab == bb)[0] for bb in [b, *probe[b]]])
        pool = pool[pool != q]
        dd = ((Xi[pool] - Xi[q]) ** 2).sum(axis=1)
        o = np.lexsort((pool, dd))[:M]
        np.testing.assert_array_equal(ids[q], pool[o])
        np.testing.assert_array_equal(d[q], dd[o].astype(np.float32))


@pytest.mark.parametrize("N,B,P,M,D,dtype", [(3000, 6, 2, 64, 128, np.int8), (500, 5, 1, 100, 32, np.int8),
                                             (60, 4, 3, 64, 8, np.int8), (1200, 7, 1, 32, 96, np.float32)])
def test_knn_bucketed_int_matches_c_oracle(N, B, P, M, D, dtype):
    """The BLAS restatement for integer rows (used at C5's bucket sizes) equals
    the C loop bit for bit: duplicated rows (distance-0 ties broken by id),
    pools shorter than M, an out-of-range probe, a bucket probing itself."""
    rng = np.random.default_rng(N + M)
    if dtype == np.int8:
        X = rng.integers(-127, 128, size=(N, D)).astype(np.int8)
    else:
        X = rng.integers(0, 256, size=(N, D)).astype(np.float32)
    X[5] = X[7]
    X[11] = X[7]
    off, mem, _ = _buckets(rng, N, B)
    probe = np.stack([rng.permutation(np.delete(np.arange(B), b))[:P] for b in range(B)]).astype(np.int32)
    probe[0, 0] = -1
    probe[1, 0] = 1
    a = O.knn_bucketed(X, off, mem, probe, M)
    b = O.knn_bucketed_int(X, off, mem, probe, M, query_chunk=97)
    np.testing.assert_array_equal(a[0], b[0])
    np.testing.assert_array_equal(a[1].view(np.uint32), b[1].view(np.uint32))


def test_knn_bucketed_int_rejects_non_integer_rows():
    X = np.full((10, 4), 0.5, np.float32)
    with pytest.raises(ValueError):
        O.knn_bucketed_int(X, np.array([0, 10]), np.arange(10, dtype=np.int32), np.zeros((1, 0), np.int32), 4)


def test_merge_rounds_union_dedup():
    rng = np.random.default_rng(8)
    X = rng.integers(0, 60, size=(300, 16)).astype(np.float32)
    ex_i, ex_d = O.knn_exact(X, 10)
    # two "rounds" each seeing a random half of the true neighbours plus junk
    Xi = X.astype(np.int64)
    rounds = []
    for r in range(2):
        ri = np.full((300, 10), -1, np.int32)
        rd = np.full((300, 10), np.inf, np.float32)
        for q in range(300):
            cand = rng.choice(np.delete(np.arange(300), q), size=14, replace=False)
            cand = np.union1d(cand, ex_i[q][rng.random(10) < 0.6])
            dd = ((Xi[cand] - Xi[q]) ** 2).sum(axis=1)
            o = np.lexsort((cand, dd))[:10]
            ri[q, :len(o)], rd[q, :len(o)] = cand[o], dd[o]
        rounds.append((ri, rd))
    mi, md = O.merge_rounds(*rounds[0], *rounds[1])
    for q in range(300):
        u = np.union1d(rounds[0][0][q], rounds[1][0][q])
        u = u[u >= 0]
        dd = ((Xi[u] - Xi[q]) ** 2).sum(axis=1)
        o = np.lexsort((u, dd))[:10]
        np.testing.assert_array_equal(mi[q, :len(o)], u[o])
    # merging the exact table with anything drawn from the same distances is a no-op
    mi2, md2 = O.merge_rounds(ex_i, ex_d, *rounds[0])
    np.testing.assert_array_equal(mi2, ex_i)


# ---------------------------------------------------------------- sanitize

def test_sanitize_known_answers():
    knn = np.array([[-1, 2, 0, 5],      # row 0: -1 -> 2, self 0 -> 2, 5 out of range -> 2
                    [1, -1, -1, -1],    # row 1: only self -> fallback (1+1)%3 = 2
                    [0, 1, -1, 2]], np.int32)
    out = O.sanitize(knn)
    assert out.tolist() == [[2, 2, 2, 2], [2, 2, 2, 2], [0, 1, 0, 0]]


# ---------------------------------------------------------------- prune

def test_prune_select_known_answer():
    # point 0 ranks ids 1..5; rows of 1,2 are built so the detour counts are
    # {0,0,1,1,2} (test_prune_windowed_core.cpp:93-105 pattern): K=3 keeps ranks 0,1,2
    G = np.zeros((6, 5), np.int32)
    G[0] = [1, 2, 3, 4, 5]
    G[1] = [3, 5, 0, 0, 0]
    G[2] = [4, 5, 0, 0, 0]
    assert O.detour_counts(G, 0).tolist() == [0, 0, 1, 1, 2]
    out, rc, _ = O.cagra_prune(G, 3)
    assert rc == 0 and out[0].tolist() == [1, 2, 3]
    out, rc, _ = O.cagra_prune(G, 5)
    assert out[0].tolist() == [1, 2, 3, 4, 5]


def _naive_counts(G, a):
    """direct triple loop of test_prune_windowed_core.cpp:42-63"""
    M = G.shape[1]
    row = G[a]
    cnt = np.zeros(M, np.int64)
    for kad in range(M - 1):
        d = row[kad]
        if d < 0 or d >= len(G):
            continue
        for kab in range(kad + 1, M):
            if row[kab] >= 0 and row[kab] in G[d]:
                cnt[kab] += 1
    return cnt


def test_prune_counts_match_naive_definition():
    rng = np.random.default_rng(9)
    G = rng.integers(-1, 50, size=(50, 10)).astype(np.int32)
    for a in range(50):
        np.testing.assert_array_equal(O.detour_counts(G, a), _naive_counts(G, a))


def test_prune_fewer_candidates_error():
    G = np.array([[1, -1, -1], [0, 2, -1], [0, 1, -1]], np.int32)
    out, rc, bad = O.cagra_prune(G, 2)
    assert rc == O.OR_EFEWCAND and bad == 0


def test_prune_matches_reference_golden():
    z = np.load(os.path.join(GOLDEN, "prune_golden.npz"))
    for c in range(6):
        G, K = z[f"prune{c}_G"], int(z[f"prune{c}_K"])
        out, rc, _ = O.cagra_prune(G, K)
        assert rc == int(z[f"prune{c}_rc"])
        if rc == 0:
            np.testing.assert_array_equal(out, z[f"prune{c}_out"])
        np.testing.assert_array_equal(O.detour_counts(G, 0), z[f"prune{c}_counts0"])


@pytest.mark.skipif(not O.ref_available(), reason="reference harness not built here")
def test_prune_matches_reference_random():
    rng = np.random.default_rng(10)
    for t in range(20):
        N, M = int(rng.integers(20, 120)), int(rng.integers(3, 40))
        K = int(rng.integers(1, M + 1))
        G = rng.integers(-1, N, size=(N, M)).astype(np.int32)
        a, rc, _ = O.cagra_prune(G, K)
        b, rc2 = O.ref_cagra_prune(G, K)
        assert rc == rc2
        if rc == 0:
            np.testing.assert_array_equal(a, b)


# ---------------------------------------------------------------- reverse merge

def test_prune_windowed_known_answer():
    # two buckets {0, 1, 2} and {3, 4, 5}; row 0 = [1, 3, 4, 2] in rank order.
    # Full window: D=1 (rank 0) holds 4; D=3 (rank 1, other bucket) holds 4
    # and 2; D=4 (rank 2) holds 2 -> counts [0, 0, 2, 2] -> K=3: [1, 3, 4].
    # Window of position 0 = {0}: only D=1 counts -> [0, 0, 1, 0] -> [1, 3, 2].
    G = np.array([[1, 3, 4, 2], [0, 4, 5, 5], [0, 1, 3, 4], [2, 5, 4, 0], [2, 0, 3, 5], [3, 4, 0, 1]], np.int32)
    off = np.array([0, 3, 6], np.uint32)
    own = np.array([[0, 0], [1, 0]], np.int32), np.array([1, 1], np.int32)
    both = np.array([[0, 1], [0, 1]], np.int32), np.array([2, 2], np.int32)
    out, rc, _ = O.prune_windowed(G, off, *own, 3)
    assert rc == 0 and out[0].tolist() == [1, 3, 2]
    out, rc, _ = O.prune_windowed(G, off, *both, 3)
    assert rc == 0 and out[0].tolist() == [1, 3, 4]
    full, _, _ = O.cagra_prune(G, 3)
    assert (out == full).all()


def test_prune_windowed_full_windows_equal_prune():
    from helpers import bucketed_graph
    rng = np.random.default_rng(11)
    G, off, _, _ = bucketed_graph(rng, 2000, 17, 24, 3)
    nb = len(off) - 1
    win = np.tile(np.arange(nb, dtype=np.int32), (nb, 1))
    out, rc, _ = O.prune_windowed(G, off, win, np.full(nb, nb, np.int32), 12)
    ref, rc2, _ = O.cagra_prune(G, 12)
    assert rc == rc2 == 0 and (out == ref).all()


@pytest.mark.skipif(not O.ref_available(), reason="reference harness not built here")
@pytest.mark.parametrize("seed,N,nb,M,K,W,pad", [(1, 3000, 30, 32, 16, 4, 0.0), (2, 1500, 9, 64, 32, 2, 0.0),
                                                 (3, 2500, 40, 20, 10, 6, 0.05)])
def test_prune_windowed_matches_reference_random(seed, N, nb, M, K, W, pad):
    """The reference's own BucketWindow prune (src/prune_windowed_core.hpp),
    compiled in place, on random bucketed tables with padding and repeats."""
    from helpers import bucketed_graph
    rng = np.random.default_rng(seed)
    G, off, win, wl = bucketed_graph(rng, N, nb, M, W, pad=pad)
    out, rc, _ = O.prune_windowed(G, off, win, wl, K)
    ref, rrc = O.ref_prune_windowed(G, off, win, wl, K)
    assert rc == rrc
    if rc == 0:
        assert (out == ref).all()
        full, _, _ = O.cagra_prune(G, K)
        assert (out != full).any()   # the windows decide some rows


def test_merge_row_truncation_known_answer():
    # test_edge_chunk_accumulator.cpp:185-220: 5 candidates for 3 free slots
    row = O.merge_row([0, 1, 2, 3, 4, 5], [13, 11, 14, 12, 10])
    assert row.tolist() == [0, 1, 2, 13, 11, 14]


def test_reverse_merge_matches_reference_golden():
    z = np.load(os.path.join(GOLDEN, "revmerge_golden.npz"))
    for c in range(4):
        np.testing.assert_array_equal(O.reverse_merge(z[f"rev{c}_F"]), z[f"rev{c}_out"])


@pytest.mark.skipif(not O.ref_available(), reason="reference harness not built here")
def test_reverse_merge_matches_reference_random():
    rng = np.random.default_rng(11)
    for t in range(20):
        N, K = int(rng.integers(5, 200)), int(rng.integers(1, 40))
        F = rng.integers(0, N, size=(N, K)).astype(np.uint32)
        np.testing.assert_array_equal(O.reverse_merge(F), O.ref_reverse_merge(F))


def test_translate_matches_reference_golden():
    z = np.load(os.path.join(GOLDEN, "translate_golden.npz"))
    for c in range(2):
        np.testing.assert_array_equal(O.translate(z[f"tr{c}_g"], z[f"tr{c}_inv"]), z[f"tr{c}_out"])


def test_translate_rejects_non_permutation():
    with pytest.raises(RuntimeError):
        O.translate(np.zeros((3, 2), np.uint32), np.array([0, 0, 1], np.uint32))


# ---------------------------------------------------------------- refine

def test_refine_fixed_point_and_monotone():
    rng = np.random.default_rng(12)
    X = rng.integers(0, 40, size=(300, 16)).astype(np.float32)
    ex_i, ex_d = O.knn_exact(X, 12)
    ri, rd = O.refine_2hop(X, ex_i, ex_d, 6)
    np.testing.assert_array_equal(ri, ex_i)     # exact kNN is a fixed point
    # a damaged table only improves, elementwise
    bi, bd = ex_i.copy(), ex_d.copy()
    bi[:, 6:], bd[:, 6:] = -1, np.inf
    ri, rd = O.refine_2hop(X, bi, bd, 6)
    assert (rd <= bd).all()
    assert ((ri >= 0).sum(axis=1) >= (bi >= 0).sum(axis=1)).all()
    for q in range(0, 300, 13):                 # every kept distance is exact
        v = ri[q][ri[q] >= 0]
        np.testing.assert_array_equal(rd[q][:len(v)], ((X[v] - X[q]) ** 2).sum(axis=1))


# Hand-traced known answer of one refinement pass (src/bucket.cu:4754-4850),
# M = 3, S = 2, eight 2-D integer points.  Each input row holds ids sorted by
# their true squared distance (not the exact kNN).  The candidates of a are
# columns 0..S-1 of the rows of its first S neighbours; self, ids already in
# a's row and repeated candidates drop out; a candidate enters only if its
# distance is strictly below a's 3rd distance; the row becomes the first 3 of
# row + candidates by (distance, id).
REFINE_KAT_X = np.array([[0, 0], [3, 0], [4, 0], [20, 20], [-1, 0], [0, 1], [0, 6], [6, 0]], np.float32)
REFINE_KAT_IDS = np.array([[1, 2, 7],    # a=0: kth 36
                           [2, 0, 4],    # col 0 = 2 is in row 0 (dedup); col 2 = 4 (d0 = 1) lies beyond S
                           [1, 6, 3],    # col 1 = 6: d(0,6) = 36 = row 0's kth, id 6 < 7 (strict <)
                           [7, 2, 1],
                           [0, 5, 7],
                           [0, 4, 1],
                           [5, 0, 1],
                           [0, 5, 6]],   # row 7 is row 0's 3rd neighbour (hop beyond S): its 5 has d0 = 1
                          np.int32)
REFINE_KAT_OUT_IDS = [[1, 2, 7],   # nothing enters: 2 dedup, 0 self, 1 dedup, 6 tied with kth
                      [2, 0, 4],   # 6 (45) not below 16; 0 and 2 self / in row
                      [1, 0, 5],   # 0 (16) via hop 1, 5 (17) via hop 6; 0 again via 6 is a repeat
                      [6, 7, 2],   # 6 (596) via hop 2 ties 7 (596): lower id first; 0 (800), 5 (761) too far
                      [0, 5, 1],   # 1 (16) and 2 (25) via hop 0, both below 49
                      [0, 4, 1],   # 2 (17) not below 10
                      [5, 0, 4],   # 4 (37) via hop 5; 2 (52) not below 45
                      [2, 1, 0]]   # 1 (9), 2 (4) via hop 0, 4 (49) via hop 5, all below 72
REFINE_KAT_OUT_D = [[9, 16, 36], [1, 9, 16], [1, 16, 17], [596, 596, 656],
                    [1, 2, 16], [1, 2, 10], [25, 36, 37], [4, 9, 36]]


def refine_kat_input():
    X = REFINE_KAT_X
    d = np.array([[((X[a] - X[v]) ** 2).sum() for v in REFINE_KAT_IDS[a]] for a in range(8)], np.float32)
    return X, REFINE_KAT_IDS.copy(), d


def test_refine_hand_traced_known_answer():
    X, ids, d = refine_kat_input()
    assert (np.diff(d, axis=1) >= 0).all()
    ri, rd = O.refine_2hop(X, ids, d, 2)
    assert ri.tolist() == REFINE_KAT_OUT_IDS
    assert rd.tolist() == REFINE_KAT_OUT_D


def test_refine_two_hop_property():
    """After one pass, every 2-hop candidate v of a (column < S of the row of
    one of a's first S neighbours, v != a) is in a's new row unless its
    distance is not below the new row's last distance; and every entry of the
    new row is either from a's old row or such a candidate, with its exact
    distance."""
    rng = np.random.default_rng(13)
    N, D, M, S = 400, 6, 10, 4
    X = rng.integers(0, 200, size=(N, D)).astype(np.float32)
    X64 = X.astype(np.float64)
    ids = np.stack([rng.permutation(np.delete(np.arange(N), a))[:M] for a in range(N)]).astype(np.int32)
    d = np.array([((X64[ids[a]] - X64[a]) ** 2).sum(1) for a in range(N)], np.float32)
    o = np.argsort(d, axis=1, kind="stable")
    ids, d = np.take_along_axis(ids, o, 1), np.take_along_axis(d, o, 1)
    ri, rd = O.refine_2hop(X, ids, d, S)
    changed = 0
    for a in range(N):
        cand = {int(v) for u in ids[a, :S] for v in ids[u, :S] if v != a}
        allowed = cand | set(ids[a].tolist())
        assert set(ri[a].tolist()) <= allowed
        assert len(set(ri[a].tolist())) == M
        np.testing.assert_array_equal(rd[a], ((X64[ri[a]] - X64[a]) ** 2).sum(1).astype(np.float32))
        for v in cand:
            dv = float(((X64[v] - X64[a]) ** 2).sum())
            assert v in ri[a] or dv >= rd[a, -1]
        changed += int((ri[a] != ids[a]).any())
    assert changed > N // 2


# ---------------------------------------------------------------- fixtures from the reference's Python
# tests/golden/pyref_golden.npz is written by tests/golden/make_golden_py.py,
# which imports bd/prune.py:prune_graph and bd/build_bucket.py:_apply_reverse_edges
# in the build container, on inputs whose results no tie order or float32
# summation order can change.

def _pyref():
    return np.load(os.path.join(GOLDEN, "pyref_golden.npz"))


def test_occlusion_prune_matches_reference_python():
    z = _pyref()
    n = len([k for k in z.files if k.endswith("_nb")])
    assert n >= 7
    for c in range(n):
        got = O.prune_occlusion(z[f"occ{c}_X"], z[f"occ{c}_nb"], int(z[f"occ{c}_maxdeg"]))
        np.testing.assert_array_equal(got, z[f"occ{c}_out"], err_msg=f"case {c} ({z[f'occ{c}_kind']})")


def test_reverse_insert_matches_reference_python():
    z = _pyref()
    n = len([k for k in z.files if k.startswith("rin") and k.endswith("_out_ids")])
    assert n >= 4
    for c in range(n):
        ri, rd = O.reverse_insert(z[f"rin{c}_ids"], z[f"rin{c}_d"])
        np.testing.assert_array_equal(ri, z[f"rin{c}_out_ids"], err_msg=f"case {c}")
        np.testing.assert_array_equal(rd, z[f"rin{c}_out_d"], err_msg=f"case {c}")


# ---------------------------------------------------------------- occlusion prune

def test_occlusion_prune_line_known_answer():
    # v = 0 at x=0 with neighbours at 1, 2, -3: sorted 1 (d=1), 2 (d=4), -3 (d=9);
    # 2 is occluded by 1 (d(1,2)=1 < 4); -3 is not (d(1,-3)=16 > 9)
    X = np.array([[0], [1], [2], [-3]], np.float32)
    nb = np.array([[2, 1, 3], [0, 2, 3], [1, 0, 3], [0, 1, 2]], np.int64)
    out = O.prune_occlusion(X, nb, 0)
    assert out[0].tolist() == [1, 3, -1]
    out = O.prune_occlusion(X, nb, 1)
    assert out[0].tolist() == [1, -1, -1]


# ---------------------------------------------------------------- reverse-edge insertion

def test_reverse_insert_line_known_answer():
    # points at 0, 1, 3, 7 (squared distances); an approximate table in which
    # row 2 misses 1 (d=4) and row 0 misses 2 (d=9).  Offers: 1->2 (4 < 16)
    # enters row 2; 2->0 (9 < 49) enters row 0; 3->2 (16) is not below row 2's
    # worst (16); offers already in the target row are dropped.
    ids = np.array([[1, 3], [0, 2], [0, 3], [2, 1]], np.int32)
    d = np.array([[1, 49], [1, 4], [9, 16], [16, 36]], np.float32)
    ri, rd = O.reverse_insert(ids, d)
    assert ri.tolist() == [[1, 2], [0, 2], [1, 0], [2, 1]]
    assert rd.tolist() == [[1, 9], [1, 4], [4, 9], [16, 36]]


def test_reverse_insert_exact_table_is_fixed_point():
    # with distinct distances every offer below b's worst is one of b's exact
    # nearest neighbours, so it is already in b's row
    rng = np.random.default_rng(5)
    X = rng.standard_normal((600, 8)).astype(np.float32)
    ids, d = O.knn_exact(X, 12)
    ri, rd = O.reverse_insert(ids, d)
    np.testing.assert_array_equal(ri, ids)
    np.testing.assert_array_equal(rd, d)


def test_reverse_insert_rows_are_m_smallest_of_row_and_offers():
    rng = np.random.default_rng(6)
    N, M = 400, 10
    ids = np.stack([rng.permutation(N)[:M] for _ in range(N)]).astype(np.int32)
    d = np.sort(rng.integers(0, 1000, size=(N, M)).astype(np.float32), axis=1)
    ids[rng.random((N, M)) < 0.05] = -1
    d[ids < 0] = np.inf
    o = np.argsort(d, axis=1, kind="stable")
    ids, d = np.take_along_axis(ids, o, 1), np.take_along_axis(d, o, 1)
    ri, rd = O.reverse_insert(ids, d)
    worst = d.max(axis=1)
    offers = [[] for _ in range(N)]
    for a in range(N):
        for k in range(M):
            b = ids[a, k]
            if b >= 0 and d[a, k] < worst[b] and a not in ids[b]:
                offers[b].append((float(d[a, k]), a))
    for b in range(N):
        pool = sorted([(float(x), int(i) & 0xFFFFFFFF) for x, i in zip(d[b], ids[b])] + offers[b])
        if not offers[b]:
            assert ri[b].tolist() == ids[b].tolist()
            continue
        got = [(float(x), int(i) & 0xFFFFFFFF) for x, i in zip(rd[b], ri[b])]
        assert got == sorted(got)
        # every entry left out is not below the last kept one
        left = list(pool)
        for g in got:
            left.remove(g)
        assert all(x >= got[-1] for x in left)


# ---------------------------------------------------------------- the timed CPU baseline

def test_knn_exact_blas_port_matches_oracle():
    # bd/build_knn.py's blocked BLAS kNN restated in numpy (the CPU baseline of
    # bench.py): tie-free float data, several query and base blocks
    rng = np.random.default_rng(21)
    X = rng.standard_normal((2500, 24)).astype(np.float32)
    bi, bd = O.knn_exact_blas(X, 16, base_chunk=600, query_chunk=700)
    oi, od = O.knn_exact(X, 16)
    np.testing.assert_array_equal(bi, oi)
    np.testing.assert_allclose(bd, od, rtol=1e-5, atol=1e-5)
    q = np.array([0, 5, 2499, 1200])
    si, _ = O.knn_exact_blas(X, 16, queries=q, base_chunk=1000, query_chunk=4)
    np.testing.assert_array_equal(si, oi[q])


@pytest.mark.skipif(not O.ref_available(), reason="reference harness not built here")
def test_reference_openmp_prune_and_merge_equal_serial():
    rng = np.random.default_rng(22)
    G = rng.integers(0, 4000, size=(4000, 32)).astype(np.int32)
    a, rc = O.ref_cagra_prune(G, 16)
    b, rc2 = O.ref_cagra_prune_omp(G, 16)
    assert rc == rc2 == 0
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(O.ref_reverse_merge(a), O.ref_reverse_merge_omp(a))
