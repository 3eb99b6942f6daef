"""CPU oracle for the bucketed CAGRA-style graph build -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker / the timed CPU
baseline.  The shipped library never routes through it.

ctypes bindings over ``oracle/liboracle_gt.so`` (built from gt_oracle.c by
``oracle/Makefile``) plus optional bindings over ``oracle/_ref/libgtann_ref.so``
(the reference's own headers compiled in place, present only where
/root/reference was available at build time).

How each oracle function is pinned (what checks it besides itself):

* ``knn_exact`` -- brute force restatement of bd/build_knn.py:17-149.  Pinned by
  closed forms in tests/test_oracle.py: a 1-D line with hand-computed
  neighbours, the IP/L2 identity on unit vectors (<x,y> = 1 - |x-y|^2/2),
  duplicated points giving distance 0, and an independent numpy brute force
  on integer data.
* ``knn_bucketed`` -- restates src/bucket.cu:5331-5347 + 4101-4265.  Pinned by
  the identity "all buckets probed == exact kNN" (config C1 has nprobe =
  buckets-1) and by a numpy per-bucket brute force.
* ``merge_rounds`` -- src/bucket.cu:5021-5053.  Pinned by the identity
  merge(exact, anything-from-the-same-distance-function) == exact, and by a
  numpy union/dedup/sort restatement on random tables.
* ``sanitize`` -- src/optimize.cu:89-134.  Pinned by hand-written known
  answers (padding, self, out-of-range, empty row fallback (i+1)%N).
* ``cagra_prune`` / ``detour_counts`` -- src/prune_windowed_core.hpp:177-263.
  Pinned bit-exactly against the reference header itself (``ref_*``) on
  random graphs incl. duplicates and padding, and the reference's KAT
  (detour {0,0,1,1,2} -> ids {10,11,12}, test_prune_windowed_core.cpp:93-105).
* ``reverse_merge`` / ``merge_row`` -- src/edge_chunk_accumulator.hpp:235-284,
  471-494.  Pinned against the reference header (``ref_reverse_merge``) and
  its truncation KAT (test_edge_chunk_accumulator.cpp:185-220).
* ``refine_2hop`` -- src/bucket.cu:4754-4850.  Pinned by a hand-traced known
  answer on eight 2-D integer points (tests/test_oracle.py, REFINE_KAT_*)
  that a no-op, an S cutoff off by one on either the hop or the column
  index, ``<=`` in place of ``<`` against the row's M-th distance, and a
  missing dedup against the row each fail; by the two-hop property on random
  integer tables (every 2-hop candidate is in the new row or not below its
  last distance; every new entry comes from the old row or the candidates,
  with its exact distance); by the fixed point on exact kNN input and by
  monotone distances.
* ``translate`` -- src/translate_graph_ids.hpp:75.  Pinned against the
  reference header (``ref_translate``).
* ``prune_occlusion`` -- bd/prune.py:8-83.  Pinned by a hand-computed 1-D
  example and bit for bit against the reference's own ``prune_graph``
  (imported in the build container by tests/golden/make_golden_py.py;
  fixtures in tests/golden/pyref_golden.npz): integer cases with distinct
  candidate distances (one on a coarse 2-D grid where d(u,z) == d(v,z) is
  frequent, so ``<`` is pinned) and float cases at least 1e-3 relative from
  every tie.  np.argsort's order among equal distances and float32 summation
  order on near-ties stay "parity unpinned"; the oracle orders ties by column.
* ``reverse_insert`` -- bd/build_bucket.py:473-543.  Pinned bit for bit
  against the reference's own ``_apply_reverse_edges`` (same fixture file:
  tie-free tables, padded rows), by a hand-computed 1-D known answer, by the
  fixed point "an exact kNN table with distinct distances does not change",
  and by the characterisation of each new row as the M smallest of (row,
  surviving offers).  torch.topk's order among equal distances is "parity
  unpinned"; the oracle orders ties by id.
* ``search`` -- bd/search.py:20-90 (graph_search_single).  Pinned by two
  hand-traced known answers (a tie at the ef-th distance is still expanded,
  ``>`` not ``>=``; a closer point replaces the FIRST slot holding the
  maximum), by the closed form "ef >= N on a connected graph returns the
  exact top-k", and against the reference's own C++ search
  (bd/search.cpp:33-137, compiled in place into ``_ref/``) on tie-free float
  data with one entry point, where the two reference versions agree.  The
  reference's np.argsort order among equal distances and its BLAS float32
  summation order are "parity unpinned"; the oracle sorts ties by slot and
  sums in four partial sums by dimension mod 4 (the kernel's order).
* ``bucket_reorder`` -- src/bucket.cu:8363-8412 (compute_bucket_reorder).
  Pinned by the closed form "inverse_perm = stable argsort of each point's
  processing position, offsets = running sums of bucket sizes in processing
  order" on random assignments.  The bucket order itself is checked against
  the reference header (``ref_bucket_order``, src/bucket_order.hpp:161-262).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_gt.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libgtann_ref.so")
_REF_SEARCH_PATH = os.path.join(_HERE, "_ref", "libgtann_ref_search.so")

OR_OK, OR_EINVAL, OR_ENOMEM, OR_EFEWCAND = 0, -1, -2, -4

_lib = None
_ref = None
_ref_search = None


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle not built: {_LIB_PATH} (run `make -C oracle`)")
        L = C.CDLL(_LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        L.or_knn_exact.argtypes = [vp, i64, i64, i32, vp, i64, i32, i32, vp, vp]
        L.or_knn_bucketed.argtypes = [vp, i64, i64, i32, vp, vp, i64, vp, i32, i32, vp, vp]
        L.or_merge_rounds.argtypes = [vp, vp, vp, vp, i64, i32, vp, vp]
        L.or_sanitize.argtypes = [vp, i64, i32, vp]
        L.or_sanitize.restype = i64
        L.or_cagra_prune.argtypes = [vp, i64, i32, i32, vp, vp]
        L.or_prune_windowed.argtypes = [vp, i64, i32, vp, i32, vp, vp, i32, i32, vp, vp]
        L.or_detour_counts.argtypes = [vp, i64, i32, i64, vp]
        L.or_reverse_merge.argtypes = [vp, i64, i32, vp]
        L.or_reverse_insert.argtypes = [vp, vp, i64, i32]
        L.or_merge_row.argtypes = [vp, vp, C.c_uint32, C.c_uint32]
        L.or_merge_row.restype = None
        L.or_refine_2hop.argtypes = [vp, i64, i64, i32, vp, vp, i32, i32, vp, vp]
        L.or_translate.argtypes = [vp, vp, i64, i32, vp]
        L.or_prune_occlusion.argtypes = [vp, i64, i64, vp, i32, i32, vp]
        L.or_search.argtypes = [vp, i64, i64, vp, i32, vp, i64, vp, i32, i32, i32, i32, vp, vp, vp]
        L.or_bucket_reorder.argtypes = [vp, i64, i64, vp, vp, vp]
        L.or_bucket_reorder.restype = i64
        L.or_num_threads.restype = i32
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(_REF_PATH)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference harness not built: {_REF_PATH}")
        R = C.CDLL(_REF_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int32
        R.ref_cagra_prune.argtypes = [vp, i64, i32, i32, vp]
        R.ref_prune_windowed.argtypes = [vp, i64, i32, vp, i32, vp, vp, i32, i32, vp]
        R.ref_cagra_prune_omp.argtypes = [vp, i64, i32, i32, vp]
        R.ref_reverse_merge_omp.argtypes = [vp, i64, i32, vp]
        R.ref_detour_counts.argtypes = [vp, i64, i32, i64, vp]
        R.ref_reverse_merge.argtypes = [vp, i64, i32, vp]
        R.ref_translate.argtypes = [vp, vp, i64, i32, vp]
        cp = C.c_char_p
        R.ref_write_graph.argtypes = [cp, vp, i64, i32]
        R.ref_write_vector_knn.argtypes = [cp, vp, i64, i32]
        R.ref_write_u32_vector.argtypes = [cp, vp, i64]
        R.ref_read_graph.argtypes = [cp, vp, i64, C.POINTER(i64), C.POINTER(i32)]
        R.ref_read_vector_knn.argtypes = [cp, vp, i64, C.POINTER(i64), C.POINTER(i32)]
        R.ref_read_dataset.argtypes = [cp, vp, i64, C.POINTER(i32), C.POINTER(i32)]
        R.ref_bucket_order.argtypes = [vp, i64, i32, i32, vp]
        R.ref_write_bucket_offsets.argtypes = [cp, vp, i64]
        R.ref_write_bucket_process_order.argtypes = [cp, vp, i64]
        R.ref_read_bucket_offsets.argtypes = [cp, vp, i64, C.POINTER(i64)]
        R.ref_read_bucket_process_order.argtypes = [cp, vp, i64, C.POINTER(i64)]
        _ref = R
    return _ref


def _f32(X):
    return np.ascontiguousarray(X, dtype=np.float32)


def _check(rc, what):
    if rc != OR_OK:
        raise RuntimeError(f"{what} failed with code {rc}")


def num_threads() -> int:
    return int(lib().or_num_threads())


def knn_exact(X, k, queries=None, metric=0, exclude_self=True):
    X = _f32(X)
    N, D = X.shape
    q = np.arange(N, dtype=np.int64) if queries is None else np.ascontiguousarray(queries, dtype=np.int64)
    ids = np.empty((len(q), k), np.int32)
    d = np.empty((len(q), k), np.float32)
    _check(lib().or_knn_exact(_p(X), N, D, metric, _p(q), len(q), k, int(exclude_self), _p(ids), _p(d)),
           "or_knn_exact")
    return ids, d


def knn_exact_blas(X, k, queries=None, base_chunk=262144, query_chunk=8192):
    """The reference's CPU exact kNN, bd/build_knn.py:17-149, restated in
    numpy: per query block and base block, dots by BLAS (A @ B.T, float32),
    d = |a|^2 + |b|^2 - 2 a.b, self (same global id) set to +inf, the block's
    top-k by np.argpartition + np.argsort, merged into the running top-k the
    same way (_merge_topk).  Returns (ids int64, dists float32) for `queries`
    (global ids, default all rows).  The timed CPU baseline of bench.py; the
    order among equal distances is numpy's, as in the reference."""
    X = np.ascontiguousarray(X, np.float32)
    N = X.shape[0]
    norms = np.sum(X ** 2, axis=1).astype(np.float32)
    q = np.arange(N) if queries is None else np.asarray(queries, np.int64)
    out_i = np.full((len(q), k), -1, np.int64)
    out_d = np.full((len(q), k), np.inf, np.float32)
    for a0 in range(0, len(q), query_chunk):
        qa = q[a0:a0 + query_chunk]
        A, a2 = X[qa], norms[qa]
        cur_i = np.full((len(qa), k), -1, np.int64)
        cur_d = np.full((len(qa), k), np.inf, np.float32)
        for b0 in range(0, N, base_chunk):
            b1 = min(N, b0 + base_chunk)
            dist = a2[:, None] + norms[b0:b1][None, :] - 2.0 * (A @ X[b0:b1].T)
            own = (qa >= b0) & (qa < b1)
            dist[np.nonzero(own)[0], qa[own] - b0] = np.inf
            if k < dist.shape[1]:
                part = np.argpartition(dist, kth=k - 1, axis=1)[:, :k]
            else:
                part = np.tile(np.arange(dist.shape[1]), (dist.shape[0], 1))
            row = np.arange(dist.shape[0])[:, None]
            cd, ci = dist[row, part], part + b0
            o = np.argsort(cd, axis=1)
            add_d, add_i = np.take_along_axis(cd, o, 1), np.take_along_axis(ci, o, 1)
            cat_i, cat_d = np.hstack([cur_i, add_i]), np.hstack([cur_d, add_d])
            sel = np.argpartition(cat_d, kth=k - 1, axis=1)[:, :k]
            cur_i, cur_d = cat_i[row, sel], cat_d[row, sel]
            o = np.argsort(cur_d, axis=1)
            cur_i, cur_d = np.take_along_axis(cur_i, o, 1), np.take_along_axis(cur_d, o, 1)
        out_i[a0:a0 + len(qa)] = cur_i
        out_d[a0:a0 + len(qa)] = cur_d
    return out_i, out_d


def knn_bucketed(X, offsets, members, probe, M, metric=0):
    X = _f32(X)
    N, D = X.shape
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    members = np.ascontiguousarray(members, dtype=np.int32)
    probe = np.ascontiguousarray(probe, dtype=np.int32)
    nB = len(offsets) - 1
    P = probe.shape[1] if probe.ndim == 2 else 0
    ids = np.empty((N, M), np.int32)
    d = np.empty((N, M), np.float32)
    _check(lib().or_knn_bucketed(_p(X), N, D, metric, _p(offsets), _p(members), nB, _p(probe), P, M,
                                 _p(ids), _p(d)), "or_knn_bucketed")
    return ids, d


def knn_bucketed_int(X, offsets, members, probe, M, query_chunk=512, threads=None):
    """``knn_bucketed`` (L2) for integer rows of magnitude <= 255 with
    D * 255^2 < 2^24 (int8 datasets, integer-valued float rows), restated
    with BLAS for sizes the C loop cannot finish in seconds: every product
    sum is an integer below 2^24, so the float32 GEMM is exact, the distance
    |q|^2 + |p|^2 - 2 q.p is an exact integer, and the int64 key
    (distance << 32 | id) is the same total order as the C oracle's
    (distance, id).  Pool = the bucket's members, then those of its probe
    buckets (out-of-range and repeated probes skipped), the query itself
    excluded, as src/bucket.cu:5331-5347 + 4101-4265.  Query blocks run on
    `threads` host threads (default: all), one BLAS thread each.  Pinned
    against ``knn_bucketed`` in tests/test_oracle.py."""
    from concurrent.futures import ThreadPoolExecutor
    Xi = np.asarray(X)
    if not np.issubdtype(Xi.dtype, np.integer):
        if not np.array_equal(Xi, np.rint(Xi)):
            raise ValueError("knn_bucketed_int needs integer-valued rows")
    if np.abs(Xi).max(initial=0) > 255 or Xi.shape[1] * 255 ** 2 >= 1 << 24:
        raise ValueError("knn_bucketed_int needs |x| <= 255 and D * 255^2 < 2^24")
    Xf = np.ascontiguousarray(Xi, np.float32)
    N = Xf.shape[0]
    n2 = (Xi.astype(np.int64) ** 2).sum(1)
    offsets = np.asarray(offsets, np.int64)
    members = np.asarray(members, np.int64)
    probe = np.asarray(probe, np.int64).reshape(len(offsets) - 1, -1)
    nB = len(offsets) - 1
    ids = np.full((N, M), -1, np.int32)
    d = np.full((N, M), np.inf, np.float32)
    big = np.iinfo(np.int64).max
    pools = []
    for b in range(nB):
        segs = [b]
        for pb in probe[b]:
            if 0 <= pb < nB and pb not in segs:
                segs.append(int(pb))
        pools.append(np.concatenate([members[offsets[s]:offsets[s + 1]] for s in segs]))

    def block(b, q0):
        pool = pools[b]
        q = members[offsets[b] + q0:min(offsets[b + 1], offsets[b] + q0 + query_chunk)]
        kk = min(M, len(pool))
        dot = (Xf[q] @ Xf[pool].T).astype(np.int64)
        key = ((n2[q][:, None] + n2[pool][None, :] - 2 * dot) << 32) | pool[None, :]
        key[np.arange(len(q)), q0 + np.arange(len(q))] = big   # the query itself (own rows come first)
        if kk < len(pool):
            key = np.partition(key, kk - 1, axis=1)[:, :kk]
        key.sort(axis=1)
        valid = key != big
        ids[q, :kk] = np.where(valid, key & 0xFFFFFFFF, -1).astype(np.int32)
        d[q, :kk] = np.where(valid, (key >> 32).astype(np.float32), np.float32(np.inf))

    jobs = [(b, q0) for b in range(nB) for q0 in range(0, int(offsets[b + 1] - offsets[b]), query_chunk)]
    try:
        from threadpoolctl import threadpool_limits
        limit = threadpool_limits(limits=1, user_api="blas")
    except Exception:
        limit = None
    try:
        with ThreadPoolExecutor(max_workers=threads or os.cpu_count() or 1) as ex:
            for f in [ex.submit(block, b, q0) for b, q0 in jobs]:
                f.result()
    finally:
        if limit is not None:
            limit.unregister() if hasattr(limit, "unregister") else limit.__exit__(None, None, None)
    return ids, d


def merge_rounds(run_ids, run_d, new_ids, new_d):
    run_ids = np.ascontiguousarray(run_ids, np.int32)
    new_ids = np.ascontiguousarray(new_ids, np.int32)
    run_d = np.ascontiguousarray(run_d, np.float32)
    new_d = np.ascontiguousarray(new_d, np.float32)
    N, M = run_ids.shape
    oi = np.empty((N, M), np.int32)
    od = np.empty((N, M), np.float32)
    _check(lib().or_merge_rounds(_p(run_ids), _p(run_d), _p(new_ids), _p(new_d), N, M, _p(oi), _p(od)),
           "or_merge_rounds")
    return oi, od


def sanitize(knn):
    knn = np.ascontiguousarray(knn, np.int32)
    N, M = knn.shape
    out = np.empty((N, M), np.uint32)
    lib().or_sanitize(_p(knn), N, M, _p(out))
    return out


def cagra_prune(G, K):
    """Returns (out, rc, bad_row)."""
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    out = np.zeros((N, K), np.uint32)
    bad = np.zeros(1, np.int64)
    rc = lib().or_cagra_prune(_p(G), N, M, K, _p(out), _p(bad))
    return out, rc, int(bad[0])


def prune_windowed(G, offsets, win, win_len, K):
    """Windowed CAGRA prune (src/prune_windowed_core.hpp:177-263 with bucket
    windows); returns (out, rc, bad_row)."""
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    off = np.ascontiguousarray(offsets, np.uint32)
    win = np.ascontiguousarray(win, np.int32)
    wl = np.ascontiguousarray(win_len, np.int32)
    out = np.zeros((N, K), np.uint32)
    bad = np.zeros(1, np.int64)
    rc = lib().or_prune_windowed(_p(G), N, M, _p(off), len(off) - 1, _p(win), _p(wl), win.shape[1], K, _p(out),
                                 _p(bad))
    return out, rc, int(bad[0])


def detour_counts(G, a):
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    cnt = np.empty(M, np.uint32)
    _check(lib().or_detour_counts(_p(G), N, M, a, _p(cnt)), "or_detour_counts")
    return cnt


def reverse_insert(ids, d):
    """bd/build_bucket.py:473-543 on a copy of (ids, d); returns (ids, d)."""
    ids = np.ascontiguousarray(ids, np.int32).copy()
    d = np.ascontiguousarray(d, np.float32).copy()
    N, M = ids.shape
    _check(lib().or_reverse_insert(_p(ids), _p(d), N, M), "or_reverse_insert")
    return ids, d


def reverse_merge(fwd):
    fwd = np.ascontiguousarray(fwd, np.uint32)
    N, K = fwd.shape
    out = np.empty((N, K), np.uint32)
    _check(lib().or_reverse_merge(_p(fwd), N, K, _p(out)), "or_reverse_merge")
    return out


def merge_row(row, rank_sorted_src):
    row = np.array(row, dtype=np.uint32)
    src = np.ascontiguousarray(rank_sorted_src, np.uint32)
    lib().or_merge_row(_p(row), _p(src), len(src), len(row))
    return row


def refine_2hop(X, ids, d, S, metric=0):
    X = _f32(X)
    N, D = X.shape
    ids = np.ascontiguousarray(ids, np.int32)
    d = np.ascontiguousarray(d, np.float32)
    M = ids.shape[1]
    oi = np.empty_like(ids)
    od = np.empty_like(d)
    _check(lib().or_refine_2hop(_p(X), N, D, metric, _p(ids), _p(d), M, S, _p(oi), _p(od)), "or_refine_2hop")
    return oi, od


def translate(g, inv):
    g = np.ascontiguousarray(g, np.uint32)
    inv = np.ascontiguousarray(inv, np.uint32)
    N, K = g.shape
    out = np.empty((N, K), np.uint32)
    _check(lib().or_translate(_p(g), _p(inv), N, K, _p(out)), "or_translate")
    return out


def prune_occlusion(X, nb, max_degree):
    X = _f32(X)
    N, D = X.shape
    nb = np.ascontiguousarray(nb, np.int64)
    M = nb.shape[1]
    out = np.empty((N, M), np.int64)
    _check(lib().or_prune_occlusion(_p(X), N, D, _p(nb), M, int(max_degree or 0), _p(out)),
           "or_prune_occlusion")
    return out


def search(X, graph, Q, entries, topk, ef, metric=0):
    """(ids int32 (nq, topk), keys float32, expansions int64 (nq,)); entries
    (nq, E) int32 in processing order, -1 = none.  ef is raised to topk as
    bd/search.py:164 does."""
    X = _f32(X)
    Q = _f32(Q)
    N, D = X.shape
    g = np.ascontiguousarray(graph).astype(np.int64)
    g = np.where((g >= 0) & (g < N), g, 0xFFFFFFFF).astype(np.uint32)
    deg = g.shape[1]
    ent = np.ascontiguousarray(entries, np.int32)
    if ent.ndim == 1:
        ent = ent[:, None]
    nq = Q.shape[0]
    ef = max(int(ef), int(topk))
    ids = np.empty((nq, topk), np.int32)
    d = np.empty((nq, topk), np.float32)
    ex = np.empty(nq, np.int64)
    _check(lib().or_search(_p(X), N, D, _p(g), deg, _p(Q), nq, _p(ent), ent.shape[1], topk, ef, metric,
                           _p(ids), _p(d), _p(ex)), "or_search")
    return ids, d, ex


def bucket_reorder(assign, nb, order):
    """(inverse_perm uint32 (placed,), offsets uint32 (nb + 1,))."""
    assign = np.ascontiguousarray(assign, np.int32)
    order = np.ascontiguousarray(order, np.int32)
    N = len(assign)
    inv = np.empty(N, np.uint32)
    off = np.empty(nb + 1, np.uint32)
    placed = lib().or_bucket_reorder(_p(assign), N, nb, _p(order), _p(inv), _p(off))
    if placed < 0:
        raise RuntimeError(f"or_bucket_reorder failed: {placed}")
    return inv[:placed], off


# ---- the reference's own code, compiled in place (test-time only) ----

def ref_search_available() -> bool:
    return os.path.exists(_REF_SEARCH_PATH)


def ref_search(X, graph, Q, topk, ef, num_entry, seed=42):
    """bd/search.cpp's graph_search_single over every query with one
    std::mt19937(seed) as its search_graph_recall does, plus the entry points
    it drew (nq, num_entry; -1 past the distinct ones, in draw order)."""
    global _ref_search
    if _ref_search is None:
        R = C.CDLL(_REF_SEARCH_PATH)
        vp, i32 = C.c_void_p, C.c_int32
        R.ref_graph_search.argtypes = [vp, i32, i32, vp, i32, vp, i32, i32, i32, i32, C.c_uint32, vp, vp, vp]
        _ref_search = R
    X = _f32(X)
    Q = _f32(Q)
    N, D = X.shape
    g = np.ascontiguousarray(graph, np.int64)
    nq = Q.shape[0]
    ids = np.empty((nq, topk), np.int64)
    d = np.empty((nq, topk), np.float32)
    ent = np.empty((nq, num_entry), np.int32)
    _check(_ref_search.ref_graph_search(_p(X), N, D, _p(g), g.shape[1], _p(Q), nq, topk, ef, num_entry, seed,
                                        _p(ids), _p(d), _p(ent)), "ref_graph_search")
    return ids, d, ent


def ref_cagra_prune(G, K):
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    out = np.zeros((N, K), np.uint32)
    rc = ref().ref_cagra_prune(_p(G), N, M, K, _p(out))
    return out, rc


def ref_cagra_prune_omp(G, K):
    """The reference's prune as its CLI runs it: rows over OpenMP threads
    (src/prune_windowed.cpp:97); same output as ref_cagra_prune."""
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    out = np.zeros((N, K), np.uint32)
    rc = ref().ref_cagra_prune_omp(_p(G), N, M, K, _p(out))
    return out, rc


def ref_reverse_merge_omp(fwd):
    fwd = np.ascontiguousarray(fwd, np.uint32)
    N, K = fwd.shape
    out = np.empty((N, K), np.uint32)
    _check(ref().ref_reverse_merge_omp(_p(fwd), N, K, _p(out)), "ref_reverse_merge_omp")
    return out


def ref_prune_windowed(G, offsets, win, win_len, K):
    """The reference's own windowed prune (BucketWindow per position,
    compute_detour_counts + select_pruned_row), rows in the given order."""
    R = ref()
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    off = np.ascontiguousarray(offsets, np.uint32)
    win = np.ascontiguousarray(win, np.int32)
    wl = np.ascontiguousarray(win_len, np.int32)
    out = np.zeros((N, K), np.uint32)
    rc = R.ref_prune_windowed(_p(G), N, M, _p(off), len(off) - 1, _p(win), _p(wl), win.shape[1], K, _p(out))
    return out, rc


def ref_detour_counts(G, a):
    G = np.ascontiguousarray(G).view(np.int32) if np.asarray(G).dtype == np.uint32 else \
        np.ascontiguousarray(G, np.int32)
    N, M = G.shape
    cnt = np.empty(M, np.uint32)
    _check(ref().ref_detour_counts(_p(G), N, M, a, _p(cnt)), "ref_detour_counts")
    return cnt


def ref_reverse_merge(fwd):
    fwd = np.ascontiguousarray(fwd, np.uint32)
    N, K = fwd.shape
    out = np.empty((N, K), np.uint32)
    _check(ref().ref_reverse_merge(_p(fwd), N, K, _p(out)), "ref_reverse_merge")
    return out


def ref_translate(g, inv):
    g = np.ascontiguousarray(g, np.uint32)
    inv = np.ascontiguousarray(inv, np.uint32)
    N, K = g.shape
    out = np.empty((N, K), np.uint32)
    _check(ref().ref_translate(_p(g), _p(inv), N, K, _p(out)), "ref_translate")
    return out


# ---- on-disk formats through the reference's own writers/readers (src/graph_io.hpp, src/load.hpp)

def ref_write_graph(path, g):
    g = np.ascontiguousarray(g, np.uint32)
    _check(ref().ref_write_graph(str(path).encode(), _p(g), g.shape[0], g.shape[1]), "ref_write_graph")


def ref_write_vector_knn(path, ids):
    ids = np.ascontiguousarray(ids, np.int32)
    _check(ref().ref_write_vector_knn(str(path).encode(), _p(ids), ids.shape[0], ids.shape[1]),
           "ref_write_vector_knn")


def ref_write_u32_vector(path, v):
    v = np.ascontiguousarray(v, np.uint32)
    _check(ref().ref_write_u32_vector(str(path).encode(), _p(v), v.size), "ref_write_u32_vector")


def _ref_read(fn, path, dtype, cap, nt, wt):
    buf = np.empty(cap, dtype)
    n, w = nt(), wt()
    _check(fn(str(path).encode(), _p(buf), cap, C.byref(n), C.byref(w)), fn.__name__)
    return buf[: int(n.value) * int(w.value)].reshape(int(n.value), int(w.value))


def ref_read_graph(path, cap=1 << 24):
    return _ref_read(ref().ref_read_graph, path, np.uint32, cap, C.c_int64, C.c_int32)


def ref_read_vector_knn(path, cap=1 << 24):
    return _ref_read(ref().ref_read_vector_knn, path, np.int32, cap, C.c_int64, C.c_int32)


def ref_read_dataset(path, cap=1 << 24):
    """float32 (N, D) as the C++ pipeline reads it (.i8bin signed)."""
    return _ref_read(ref().ref_read_dataset, path, np.float32, cap, C.c_int32, C.c_int32)


def ref_bucket_order(graph, window):
    g = np.ascontiguousarray(graph, np.uint32)
    B, K = g.shape
    out = np.empty(B, np.int32)
    _check(ref().ref_bucket_order(_p(g), B, K, window, _p(out)), "ref_bucket_order")
    return out


def ref_write_bucket_offsets(path, off):
    off = np.ascontiguousarray(off, np.uint32)
    _check(ref().ref_write_bucket_offsets(str(path).encode(), _p(off), len(off)), "ref_write_bucket_offsets")


def ref_write_bucket_process_order(path, order):
    order = np.ascontiguousarray(order, np.int32)
    _check(ref().ref_write_bucket_process_order(str(path).encode(), _p(order), len(order)),
           "ref_write_bucket_process_order")


def _ref_read_vec(fn, path, dtype, cap):
    out = np.empty(cap, dtype)
    n = C.c_int64()
    _check(fn(str(path).encode(), _p(out), cap, C.byref(n)), fn.__name__)
    return out[:n.value].copy()


def ref_read_bucket_offsets(path, cap=1 << 22):
    return _ref_read_vec(ref().ref_read_bucket_offsets, path, np.uint32, cap)


def ref_read_bucket_process_order(path, cap=1 << 22):
    return _ref_read_vec(ref().ref_read_bucket_process_order, path, np.int32, cap)
