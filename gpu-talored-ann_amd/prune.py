#!/usr/bin/env python3
"""Graph pruning with the interface of bd/prune.py, on the GPU.

``prune_graph(X, neighbors, max_degree=None, algo="occlusion")`` returns an
int64 (N, M) array with -1 padding, like bd/prune.py:8-83:

* ``algo="occlusion"`` (the reference's algorithm): per point v the valid
  neighbours (not -1, not out of range, not v) are ordered by squared L2
  distance to v; walking that order a neighbour z is dropped when an earlier
  kept u has d(u, z) < d(v, z); the kept ids are truncated to max_degree.
  Ties in d(v, .) keep the column order (numpy's argsort order among ties is
  not specified by the reference).
* ``algo="cagra"``: the bucket2 pipeline's prune -- sanitize, CAGRA
  rank-based detour-count prune to max_degree, reverse-edge merge
  (src/optimize.cu:89-134, 395-397) -- written into the same (N, M) shape.

The same checks as the reference raise ValueError.  ``prune_existing_index``
and the ``prune_existing`` command mirror bd/prune.py:86-151 and take
``--algo``.
"""
from __future__ import annotations

import argparse

import numpy as np

import gtann
from load import load_bigann_to_f32, load_neighbors

ALGOS = ("occlusion", "cagra")


def prune_graph(X, neighbors, max_degree: int | None = None, algo: str = "occlusion",
                ctx: gtann.Context | None = None) -> np.ndarray:
    if algo not in ALGOS:
        raise ValueError(f"algo must be one of {ALGOS}")
    X = np.asarray(X, dtype=np.float32)
    N, D = X.shape
    nb = np.asarray(neighbors)
    if nb.ndim != 2:
        raise ValueError("neighbors must be 2D")
    if nb.shape[0] != N:
        raise ValueError(f"N mismatch: X has {N}, neighbors has {nb.shape[0]}")
    if nb.dtype.kind not in "iu":
        raise ValueError("neighbors must be integer dtype")
    M = nb.shape[1]
    # ids outside [0, N) are dropped either way; keep them out of int32 range issues
    nb32 = np.where((nb >= 0) & (nb < N), nb, -1).astype(np.int32)
    own = ctx is None
    ctx = ctx or gtann.Context()
    try:
        if algo == "occlusion":
            out = ctx.prune_occlusion(X, nb32, max_degree or 0).astype(np.int64)
        else:
            if not max_degree or max_degree <= 0 or max_degree > min(M, 64):
                raise ValueError("cagra prune needs 1 <= max_degree <= min(M, 64)")
            g = ctx.optimize(ctx.sanitize(nb32), int(max_degree))
            out = -np.ones((N, M), dtype=np.int64)
            out[:, :max_degree] = g
    finally:
        if own:
            ctx.close()
    return out


def prune_existing_index(data_path: str, index_in: str, index_out: str, max_degree: int,
                         algo: str = "occlusion"):
    X, N, D = load_bigann_to_f32(data_path)
    print(f"[prune_existing] loaded base: {X.shape}, dtype={X.dtype}")
    nb = load_neighbors(index_in)
    print(f"[prune_existing] loaded index: {nb.shape}, dtype={nb.dtype}")
    if nb.shape[0] != N:
        raise ValueError(f"N mismatch: base={N}, index={nb.shape[0]}")
    print(f"[prune_existing] pruning ({algo}) with max_degree={max_degree} ...")
    pruned = prune_graph(X, nb, max_degree=max_degree, algo=algo)
    np.save(index_out, pruned.astype(np.int64))
    print(f"[prune_existing] pruned index saved to: {index_out}")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    ap_pe = sub.add_parser("prune_existing", help="Prune an existing index and save")
    ap_pe.add_argument("--data", type=str, required=True)
    ap_pe.add_argument("--index_in", type=str, required=True)
    ap_pe.add_argument("--index_out", type=str, required=True)
    ap_pe.add_argument("--max_degree", type=int, required=True)
    ap_pe.add_argument("--algo", type=str, default="occlusion", choices=ALGOS)
    args = ap.parse_args()
    # the reference dispatches on "prune", which its parser never produces
    # (bd/prune.py:141-149); here the registered command runs
    if args.cmd == "prune_existing":
        prune_existing_index(args.data, args.index_in, args.index_out, args.max_degree, args.algo)


if __name__ == "__main__":
    main()
