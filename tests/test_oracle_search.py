"""Pins of the search oracle (bd/search.py:20-90 restated in oracle/gt_oracle.c):
hand-traced known answers, the exact-search closed form, and the reference's
own C++ search compiled in place.  CPU only."""
import numpy as np
import pytest

import gt_oracle as O

BAD = -1   # an id outside [0, N): skipped


def _line(xs):
    """1-D points as (N, 1) float32 rows."""
    return np.asarray(xs, np.float32)[:, None]


def test_tie_at_the_ef_th_distance_is_expanded():
    # q = 0; ids: 0 at 5 (d 25), 1 at 3 (d 9), 2 at -3 (d 9), 3 at 1 (d 1).
    # entry 0 -> expand 0: 1 replaces 0 (9 < 25); 2 ties (9) and stays out.
    # pop (9, 1): 9 > 9 is false -> expand 1 (nothing new); pop (9, 2): still
    # not > 9 -> expand 2 -> finds 3 (d 1).  A ">=" stop rule would end at
    # the pop of (9, 1) and return id 1.
    X = _line([5, 3, -3, 1])
    g = np.array([[1, 2], [0, BAD], [3, BAD], [BAD, BAD]])
    ids, d, ex = O.search(X, g, _line([0]), np.array([[0]]), topk=1, ef=1)
    assert ids.tolist() == [[3]] and d.tolist() == [[1.0]]
    assert ex.tolist() == [4]


def test_closer_point_replaces_first_slot_of_the_maximum():
    # q = 0; entries 1 (d 4) and 2 (d 4) fill ef = 2 slots [1, 2]; expanding 1
    # finds 3 (d 1), which replaces slot 0 (id 1, the first maximum), so the
    # answer is [3, 2].  Replacing the last maximum would give [3, 1].
    X = _line([50, 2, -2, 1])
    g = np.array([[BAD], [3], [BAD], [BAD]])
    ids, d, _ = O.search(X, g, _line([0]), np.array([[1, 2]]), topk=2, ef=2)
    assert ids.tolist() == [[3, 2]] and d.tolist() == [[1.0, 4.0]]


def test_short_result_is_padded():
    X = _line([0, 1, 2, 3])
    g = np.array([[1], [BAD], [BAD], [BAD]])
    ids, d, _ = O.search(X, g, _line([0.25]), np.array([[0]]), topk=4, ef=4)
    assert ids.tolist() == [[0, 1, -1, -1]]
    assert d[0, 2:].tolist() == [np.inf, np.inf]


def test_ef_at_least_n_on_a_connected_graph_is_exact():
    rng = np.random.default_rng(0)
    N, D = 600, 16
    X = rng.integers(0, 50, size=(N, D)).astype(np.float32)
    # ring plus random chords: connected
    g = np.stack([(np.arange(N) + 1) % N, (np.arange(N) - 1) % N,
                  rng.integers(0, N, N), rng.integers(0, N, N)], axis=1)
    Q = rng.integers(0, 50, size=(20, D)).astype(np.float32)
    ent = rng.integers(0, N, size=(20, 1))
    ids, d, _ = O.search(X, g, Q, ent, topk=10, ef=N)
    D2 = ((Q[:, None, :].astype(np.float64) - X[None, :, :]) ** 2).sum(-1)
    for i in range(20):
        order = np.lexsort((np.arange(N), D2[i]))[:10]
        np.testing.assert_array_equal(d[i], D2[i, order].astype(np.float32))
        # equal distances may come in another id order; the sets per distance agree
        for v in np.unique(d[i]):
            assert set(ids[i][d[i] == v]) <= set(np.nonzero(D2[i] == v)[0])


def test_duplicate_ids_in_a_row_are_visited_once():
    X = _line([0, 1, 2])
    g = np.array([[1, 1, 2, 2], [BAD] * 4, [BAD] * 4])
    ids, d, ex = O.search(X, g, _line([0]), np.array([[0]]), topk=3, ef=3)
    assert ids.tolist() == [[0, 1, 2]] and ex.tolist() == [3]


@pytest.mark.skipif(not O.ref_search_available(), reason="reference search not built (needs /root/reference)")
@pytest.mark.parametrize("ef,topk,deg", [(10, 10, 16), (32, 10, 16), (64, 20, 24), (200, 10, 32)])
def test_matches_reference_cpp_search(ef, topk, deg):
    """bd/search.cpp and bd/search.py agree on tie-free float data with one
    entry point (distinct distances: no tie order; one entry: the C++ best
    list starts as a valid heap), so the C++ reference pins the oracle there."""
    rng = np.random.default_rng(ef + deg)
    N, D, nq = 3000, 24, 64
    X = rng.standard_normal((N, D)).astype(np.float32)
    Q = rng.standard_normal((nq, D)).astype(np.float32)
    knn, _ = O.knn_exact(X, deg - 4)
    g = np.concatenate([knn, rng.integers(0, N, size=(N, 4))], axis=1).astype(np.int64)
    rid, rd, ent = O.ref_search(X, g, Q, topk, ef, num_entry=1)
    ids, d, _ = O.search(X, g, Q, ent, topk, ef)
    np.testing.assert_array_equal(ids, rid)
    np.testing.assert_allclose(d, rd, rtol=1e-6)
