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
from typing import List, Optional, Tuple

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


def l2sqr(a: np.ndarray, b: np.ndarray) -> float:
    diff = a - b
    return float(diff.dot(diff))


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


def recall_vs_gt(pred: np.ndarray, gt: np.ndarray, topk: int) -> Tuple[float, float, float]:
    """bd/search.py:95-127: (hit GT[:,0], hit any of GT, mean overlap of the
    first min(topk, pred width, gt width) columns, -1 ignored)."""
    nq = pred.shape[0]
    hit_first = 0
    hit_any = 0
    for i in range(nq):
        if gt[i, 0] in pred[i]:
            hit_first += 1
        if np.intersect1d(pred[i], gt[i], assume_unique=False).size > 0:
            hit_any += 1
    r_first = hit_first / float(nq) if nq > 0 else 0.0
    r_any = hit_any / float(nq) if nq > 0 else 0.0
    k = min(topk, pred.shape[1], gt.shape[1])
    total = 0.0
    for i in range(nq):
        a = pred[i, :k]
        b = gt[i, :k]
        a = a[a >= 0]
        b = b[b >= 0]
        total += len(set(a.tolist()).intersection(set(b.tolist()))) / float(k)
    recall = total / float(nq)
    return r_first, r_any, recall


def search_graph_recall(base_path: str, query_path: str, index_path: str, gt_path: str, topk: int, ef: int,
                        num_entry: int, normalize: bool = False, ctx=None):
    base, N, D = load_bigann_to_f32(base_path)
    Q, nq, dq = load_bigann_to_f32(query_path)
    if dq != D:
        raise ValueError(f"Dim mismatch: base D={D}, query D={dq}")
    neighbors = load_neighbors(index_path)
    if neighbors.shape[0] != N:
        raise ValueError("Index N mismatch with base")
    GT, gt_nq, k_gt = load_ibin(gt_path)
    if gt_nq != nq:
        raise ValueError("GT nq mismatch with query")

    if normalize:
        print("[eval] L2-normalizing base & queries")

        def norm_rows(X):
            n = np.linalg.norm(X, axis=1, keepdims=True) + 1e-12
            X /= n
        norm_rows(base)
        norm_rows(Q)

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
    Ak = A[:, :k].astype(np.int64, copy=False)
    Bk = B[:, :k].astype(np.int64, copy=False)
    overlaps = np.empty(N, dtype=np.float32)
    hits_any = 0
    set_equal = 0
    rows: List[tuple] = []
    for i in range(N):
        a = Ak[i][Ak[i] >= 0]
        b = Bk[i][Bk[i] >= 0]
        SA, SB = set(a.tolist()), set(b.tolist())
        inter = len(SA & SB)
        overlaps[i] = inter / float(k)
        hits_any += inter >= 1
        set_equal += len(SA) == len(SB) == k and inter == k
        if save_csv is not None:
            rows.append((i, inter, len(SA), len(SB), overlaps[i]))
    mean_overlap = float(overlaps.mean()) if N > 0 else 0.0
    hits_any_rate = hits_any / float(N) if N > 0 else 0.0
    set_equal_rate = set_equal / float(N) if N > 0 else 0.0
    print("\n======= Index Comparison (set-wise) =======")
    print(f"N={N}, k={k} (A:{Ma}, B:{Mb})")
    print(f"MeanOverlap@{k} (|A∩B|/k) : {mean_overlap:.6f}")
    print(f"HitsAny@{k}               : {hits_any_rate:.6f}")
    print(f"SetEqual@{k}              : {set_equal_rate:.6f}")
    if save_csv is not None:
        os.makedirs(os.path.dirname(save_csv) or ".", exist_ok=True)
        with open(save_csv, "w") as f:
            f.write("node,intersect_size,deg_A,deg_B,overlap\n")
            for (i, inter, la, lb, ov) in rows:
                f.write(f"{i},{inter},{la},{lb},{ov:.6f}\n")
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
