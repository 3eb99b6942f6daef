#!/usr/bin/env python3
"""Bucketed kNN graph build with the interface of bd/build_bucket.py, on the GPU.

Same command line (bd/build_bucket.py:748-764) and outputs
(``neighbors_k{k}m{m}[t{t}].npy`` int64, ``neighbors_dist...npy`` float32,
``meta...npy``; :844-854).  Per round (seed + round): B = max(1, N // 32)
buckets (:405), centroids refined by ``--kmeans-iters`` Lloyd iterations,
top-2 balanced assignment, each bucket's pool = its own points + the points of
its ``--k`` nearest buckets, the m nearest pool points of every point (self
excluded), then reverse-edge insertion (:473-543); the t round tables are
merged keeping the m nearest distinct ids (:640-671).

All of it runs in libgtann (gt_build_graph with reverse_edges = 1), with the
reference's rules where they fix the result and this build's where they are
randomised or tie-dependent: centroids start from a seeded sample (the
reference uses torch k-means++), the balance rule is the two-choice rule of
the C++ pipeline (a point moves to its second bucket when that one is below
``0.8 x`` the first; ``--balance-slack`` is accepted and not used), and
ties are ordered by id.  ``--force-cpu``/``--use-bf16``/chunk sizes are
accepted and ignored: distances are fp32 on the matrix cores.
"""
from __future__ import annotations

import argparse
import os

import numpy as np

import gtann
from load import get_ext, load_bigann_bin, load_dataset


def build_index(X, k: int, m: int, t: int = 1, seed: int = 0, kmeans_iters: int = 5, balance: bool = True,
                ctx: gtann.Context | None = None):
    """(neighbors int64 (N, m), dists float32 (N, m)) of the multi-round build."""
    N = X.shape[0]
    B = max(1, N // 32)
    if k >= B:
        raise ValueError(f"--k ({k}) must be below the number of buckets ({B})")
    own = ctx is None
    ctx = ctx or gtann.Context()
    try:
        r = ctx.build_graph(X, n_buckets=B, nprobe=k, M=m, rounds=t, kmeans_iters=kmeans_iters,
                            balance=0.8 if balance else 0.0, seed=seed, reverse_edges=True, prune=False)
    finally:
        if own:
            ctx.close()
    return r.knn_ids.astype(np.int64), r.knn_dists.astype(np.float32), r.stats


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--data", type=str, required=True)
    ap.add_argument("--k", type=int, required=True)
    ap.add_argument("--m", type=int, required=True)
    ap.add_argument("--out_dir", type=str, required=True)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--assign-batch", type=int, default=65536)
    ap.add_argument("--matmul-chunk", type=int, default=262144)
    ap.add_argument("--query-chunk", type=int, default=32768)
    ap.add_argument("--base-chunk", type=int, default=262144)
    ap.add_argument("--force-cpu", action="store_true")
    ap.add_argument("--use-bf16", action="store_true")
    ap.add_argument("--prune_max_degree", type=int, default=64)
    ap.add_argument("--kmeans-iters", type=int, default=5)
    ap.add_argument("--no-balance", action="store_true")
    ap.add_argument("--balance-slack", type=int, default=4)
    ap.add_argument("--t", type=int, default=1)
    args = ap.parse_args()
    if args.force_cpu:
        print("[note] --force-cpu ignored: this build runs on the GPU only")
    os.makedirs(args.out_dir, exist_ok=True)
    # .fbin/.bin/.u8bin/.i8bin in their stored type; .ibin as float32 (bd/load.py:106-109)
    X = load_bigann_bin(args.data).numpy() if get_ext(args.data) == ".ibin" else load_dataset(args.data)
    N, D = X.shape
    print(f"Loaded X: shape=({N}, {D}), dtype={X.dtype}")
    neighbors, dists, stats = build_index(X, args.k, args.m, args.t, args.seed, args.kmeans_iters,
                                          not args.no_balance)
    print(f"[build] {stats['t_total']:.3f} s (bucketing {stats['t_bucketing']:.3f}, knn {stats['t_knn']:.3f}, "
          f"reverse edges + merge {stats['t_merge']:.3f})")
    suffix = f"_k{args.k}m{args.m}" + (f"t{args.t}" if args.t > 1 else "")
    np.save(os.path.join(args.out_dir, f"neighbors{suffix}.npy"), neighbors)
    np.save(os.path.join(args.out_dir, f"neighbors_dist{suffix}.npy"), dists)
    meta = {"N": int(N), "D": int(D), "k": int(args.k), "m": int(args.m), "t": int(args.t)}
    np.save(os.path.join(args.out_dir, f"meta{suffix}.npy"), meta, allow_pickle=True)
    print(f"Done. Files written to: {args.out_dir}")


if __name__ == "__main__":
    main()
