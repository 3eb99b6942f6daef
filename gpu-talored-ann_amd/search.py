"""Graph search and index comparison with the interface of bd/search.py.

Same functions, arguments, defaults, outputs and report lines as the
reference script; the per-query beam search runs on the GPU
(``gtann.Context.search``, the C ABI's ``gt_search``), with the entry points
drawn on the host exactly as the reference draws them
(``np.random.default_rng(42)``, ``np.unique(rng.integers(0, N, num_entry))``
per query, bd/search.py:41-42,163).

    python search.py search --base B --query Q --index neighbors.npy --gt gt.ibin
                            [--topk 10] [--ef 200] [--num-entry 4] [--normalize]
    python search.py compare --index1 A.npy --index2 B.npy [--k_cmp K] [--save_csv F]

Results equal the reference's except in the order of equal distances (the
reference sorts its result list with numpy's unstable argsort; here ties keep
their result-slot order) and in the last bits of float distances (the
reference sums with BLAS; here in dimension order).
"""
from __future__ import annotations

import argparse
import os
import time
from typing import Optional, Tuple

import numpy as np

import gtann
from load import get_ext, load_bigann_to_f32, load_ibin, load_neighbors   # noqa: F401  (the reference's imports)

_ctx = None


def _context(ctx=None):
    global _ctx
    if ctx is not None:
        return ctx
    if _ctx is None:
        _ctx = gtann.Context()
    return _ctx


def draw_entries(rng: np.random.Generator, N: int, nq: int, num_entry: int) -> np.ndarray:
    """(nq, max(1, num_entry)) int32: per query the sorted distinct ids the
    reference draws (bd/search.py:41-42), -1 padded."""
    E = max(1, num_entry)
    out = np.full((nq, E), -1, np.int32)
    for i in range(nq):
        e = np.unique(rng.integers(0, N, size=E, endpoint=False))
        out[i, :len(e)] = e
    return out


def graph_search(Q: np.ndarray, base: np.ndarray, graph: np.ndarray, topk: int, ef: int, rng: np.random.Generator,
                 num_entry: int = 1, ctx=None) -> Tuple[np.ndarray, np.ndarray]:
    """graph_search_single over every row of Q in one GPU call; the rng is
    consumed per query in order, as the reference's loop does.  Returns
    (ids int64 (nq, topk) -1 padded, dists float32 (nq, topk) +inf padded)."""
    Q = np.atleast_2d(Q)
    ent = draw_entries(rng, base.shape[0], Q.shape[0], num_entry)
    ids, d, _ = _context(ctx).search(base, graph, Q, topk=topk, ef=max(ef, topk), entries=ent)
    return ids.astype(np.int64), d


def graph_search_single(
    q: np.ndarray,
    base: np.ndarray,
    graph: np.ndarray,
    topk: int,
    ef: int,
    rng: np.random.Generator,
    num_entry: int = 1,
    ctx=None,
) -> Tuple[np.ndarray, np.ndarray]:
    """bd/search.py:20-90: (indices int64, dists) of at most topk results."""
    ids, d = graph_search(np.asarray(q)[None, :], base, graph, topk, ef, rng, num_entry, ctx)
    keep = ids[0] >= 0
    return ids[0][keep], d[0][keep].astype(np.float32)


# ---------------------------------------------------------------- set arithmetic over padded id rows

_SENT = np.iinfo(np.int64).min


def _distinct_rows(x: np.ndarray, valid_only: bool, side: int) -> np.ndarray:
    """Each row sorted, with repeats (and negative ids when valid_only)
    replaced by sentinels that are unique per position and per side, so they
    never pair with anything."""
    s = np.sort(np.asarray(x, np.int64), axis=1)
    drop = np.zeros(s.shape, bool)
    drop[:, 1:] = s[:, 1:] == s[:, :-1]
    if valid_only:
        drop |= s < 0
    sent = _SENT + side + 2 * np.arange(s.shape[1], dtype=np.int64)[None, :]
    return np.where(drop, sent, s)


def _set_sizes(a: np.ndarray, b: np.ndarray, valid_only: bool = True, chunk: int = 65536):
    """Per row i: (|A_i ∩ B_i|, |A_i|, |B_i|) over the distinct values of
    a[i] and b[i] (ids >= 0 only when valid_only).  A value common to both
    rows appears exactly twice in the sorted concatenation of the two
    distinct rows, as a pair of equal neighbours."""
    n = a.shape[0]
    inter = np.empty(n, np.int64)
    na = np.empty(n, np.int64)
    nb = np.empty(n, np.int64)
    for r0 in range(0, n, chunk):
        da = _distinct_rows(a[r0:r0 + chunk], valid_only, 0)
        db = _distinct_rows(b[r0:r0 + chunk], valid_only, 1)
        na[r0:r0 + chunk] = (da > _SENT + 2 * da.shape[1]).sum(axis=1)
        nb[r0:r0 + chunk] = (db > _SENT + 2 * db.shape[1]).sum(axis=1)
        both = np.sort(np.concatenate([da, db], axis=1), axis=1)
        inter[r0:r0 + chunk] = (both[:, 1:] == both[:, :-1]).sum(axis=1)
    return inter, na, nb


def recall_vs_gt(pred: np.ndarray, gt: np.ndarray, topk: int) -> Tuple[float, float, float]:
    """The three figures of bd/search.py:95-127:
      * hit GT[:,0]: the query's first ground-truth id is among its predictions;
      * hit any:     the prediction row and the ground-truth row share a value;
      * mean overlap: |distinct valid ids of pred[:, :k] ∩ those of gt[:, :k]| / k,
        k = min(topk, prediction width, ground-truth width), averaged over queries."""
    pred = np.asarray(pred, np.int64)
    gt = np.asarray(gt, np.int64)
    nq = pred.shape[0]
    if nq == 0:
        return 0.0, 0.0, float("nan")
    r_first = float((pred == gt[:, :1]).any(axis=1).mean())
    r_any = float((_set_sizes(pred, gt, valid_only=False)[0] > 0).mean())
    k = min(topk, pred.shape[1], gt.shape[1])
    overlap = _set_sizes(pred[:, :k], gt[:, :k])[0]
    return r_first, r_any, float((overlap / float(k)).mean())


def _load_search_inputs(base_path: str, query_path: str, index_path: str, gt_path: str):
    """(base, queries, graph, ground truth), shapes checked against each
    other with the reference's messages."""
    base, N, D = load_bigann_to_f32(base_path)
    Q, nq, dq = load_bigann_to_f32(query_path)
    graph = load_neighbors(index_path)
    GT, gt_nq, _ = load_ibin(gt_path)
    for ok, msg in ((dq == D, f"Dim mismatch: base D={D}, query D={dq}"),
                    (graph.shape[0] == N, "Index N mismatch with base"),
                    (gt_nq == nq, "GT nq mismatch with query")):
        if not ok:
            raise ValueError(msg)
    return base, Q, graph, GT


def search_graph_recall(base_path: str, query_path: str, index_path: str, gt_path: str, topk: int, ef: int,
                        num_entry: int, normalize: bool = False, ctx=None):
    base, Q, neighbors, GT = _load_search_inputs(base_path, query_path, index_path, gt_path)
    nq = Q.shape[0]
    if normalize:   # cosine search: unit rows (the 1e-12 keeps zero rows finite)
        print("[eval] L2-normalizing base & queries")
        for X in (base, Q):
            X /= np.linalg.norm(X, axis=1, keepdims=True) + 1e-12

    rng = np.random.default_rng(42)
    ef = max(ef, topk)
    print("[eval] start searching ...")
    t0 = time.perf_counter()
    preds, _ = graph_search(Q, base, neighbors, topk, ef, rng, num_entry, ctx)
    elapsed = time.perf_counter() - t0

    r_first, r_any, recall = recall_vs_gt(preds, GT, topk)
    print("\n======== Recall vs GT ========")
    print(f"Recall@{topk} (hit GT[:,0])         : {r_first:.6f}")
    print(f"Recall@{topk} (hit any of GT[:,:]) : {r_any:.6f}")
    print(f"Recall@{topk} (recall mean overlap): {recall:.6f}")
    print(f"[eval] {nq} queries in {elapsed:.3f} s ({nq / max(elapsed, 1e-9):.0f} QPS, host draw included)")
    return r_first, r_any, recall


def compare_indices_setwise(index_a_path: str, index_b_path: str, k_cmp: Optional[int] = None,
                            save_csv: Optional[str] = None):
    """bd/search.py:193-262: MeanOverlap@k, HitsAny@k, SetEqual@k of the first
    k columns of two indices (k = min widths unless k_cmp)."""
    A = load_neighbors(index_a_path)
    B = load_neighbors(index_b_path)
    if A.ndim != 2 or B.ndim != 2:
        raise ValueError("indices must be 2D")
    if A.shape[0] != B.shape[0]:
        raise ValueError(f"N mismatch: A={A.shape[0]}, B={B.shape[0]}")
    N, Ma, Mb = A.shape[0], A.shape[1], B.shape[1]
    k = min(Ma, Mb) if k_cmp is None else min(int(k_cmp), Ma, Mb)
    if k <= 0:
        raise ValueError("k_cmp must be > 0")
    inter, deg_a, deg_b = _set_sizes(A[:, :k], B[:, :k])
    overlaps = (inter / float(k)).astype(np.float32)
    mean_overlap = float(overlaps.mean()) if N > 0 else 0.0
    hits_any_rate = float((inter >= 1).mean()) if N > 0 else 0.0
    set_equal_rate = float(((deg_a == k) & (deg_b == k) & (inter == k)).mean()) if N > 0 else 0.0
    print("\n======= Index Comparison (set-wise) =======")
    print(f"N={N}, k={k} (A:{Ma}, B:{Mb})")
    print(f"MeanOverlap@{k} (|A∩B|/k) : {mean_overlap:.6f}")
    print(f"HitsAny@{k}               : {hits_any_rate:.6f}")
    print(f"SetEqual@{k}              : {set_equal_rate:.6f}")
    if save_csv is not None:
        os.makedirs(os.path.dirname(save_csv) or ".", exist_ok=True)
        with open(save_csv, "w") as f:
            f.write("node,intersect_size,deg_A,deg_B,overlap\n")
            f.writelines(f"{i},{c},{x},{y},{o:.6f}\n" for i, (c, x, y, o) in
                         enumerate(zip(inter.tolist(), deg_a.tolist(), deg_b.tolist(), overlaps.tolist())))
        print(f"[compare] per-node stats saved to: {save_csv}")
    return {"mean_overlap": mean_overlap, "hits_any": hits_any_rate, "set_equal": set_equal_rate, "k": k}


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    ap_s = sub.add_parser("search", help="Run graph search")
    ap_s.add_argument("--base", type=str, required=True, help="Path to base vectors (.fbin/.bin/.u8bin/.i8bin)")
    ap_s.add_argument("--query", type=str, required=True, help="Path to query vectors (.fbin/.bin/.u8bin/.i8bin)")
    ap_s.add_argument("--index", type=str, required=True, help="neighbors.npy (N, M)")
    ap_s.add_argument("--gt", type=str, required=True, help="groundtruth .ibin (nq, k_gt)")
    ap_s.add_argument("--topk", type=int, default=10, help="return top-k results")
    ap_s.add_argument("--ef", type=int, default=200, help="efSearch breadth (>= topk)")
    ap_s.add_argument("--num-entry", type=int, default=4, help="number of random entry points per query")
    ap_s.add_argument("--normalize", action="store_true", help="L2-normalize rows for cosine search")
    ap_c = sub.add_parser("compare", help="Compare two indices (set-wise)")
    ap_c.add_argument("--index1", type=str, required=True, help="first index npy")
    ap_c.add_argument("--index2", type=str, required=True, help="second index npy")
    ap_c.add_argument("--k_cmp", type=int, default=None, help="use top-k for comparison")
    ap_c.add_argument("--save_csv", type=str, default=None)
    args = ap.parse_args(argv)
    if args.cmd == "search":
        search_graph_recall(args.base, args.query, args.index, args.gt, args.topk, args.ef, args.num_entry,
                            args.normalize)
    else:
        compare_indices_setwise(args.index1, args.index2, args.k_cmp, args.save_csv)


if __name__ == "__main__":
    main()
