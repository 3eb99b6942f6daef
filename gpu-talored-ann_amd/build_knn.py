#!/usr/bin/env python3
"""Exact self-excluded kNN with the interface of bd/build_knn.py, on the GPU.

``build_exact_knn(data_path, k, out_dir, query_chunk, base_chunk)`` writes
``exact_knn_idx.npy`` (int64, -1 padding) and ``exact_knn_dist.npy``
(float32, squared L2, +inf padding) like bd/build_knn.py:98-149 and returns
the two paths.  The whole dataset goes to HBM and one fused MFMA
distance/top-k pass replaces the blocked CPU GEMM + argpartition; the chunk
sizes are accepted for compatibility and do not change the result.  Rows are
ascending by (distance, id) -- the reference's order among equal distances
is numpy's argpartition/argsort order.
"""
from __future__ import annotations

import argparse
import os
from typing import Tuple

import numpy as np

import gtann
from load import load_bigann_to_f32, save_npy


def build_exact_knn(data_path: str, k: int, out_dir: str, query_chunk: int = 8192,
                    base_chunk: int = 262144, ctx: gtann.Context | None = None) -> Tuple[str, str]:
    X, N, D = load_bigann_to_f32(data_path)
    print(f"[exact] Loaded X: {X.shape}, dtype={X.dtype}")
    own = ctx is None
    ctx = ctx or gtann.Context()
    try:
        ids, d = ctx.knn_exact(X, k)
    finally:
        if own:
            ctx.close()
    os.makedirs(out_dir, exist_ok=True)
    idx_path = os.path.join(out_dir, "exact_knn_idx.npy")
    dist_path = os.path.join(out_dir, "exact_knn_dist.npy")
    save_npy(idx_path, ids.astype(np.int64))
    save_npy(dist_path, d.astype(np.float32))
    print(f"[exact] saved: {idx_path}")
    print(f"[exact] saved: {dist_path}")
    return idx_path, dist_path


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    ap_b = sub.add_parser("build", help="Build exact kNN for dataset")
    ap_b.add_argument("--data", type=str, required=True)
    ap_b.add_argument("--k", type=int, required=True)
    ap_b.add_argument("--out_dir", type=str, required=True)
    ap_b.add_argument("--query-chunk", type=int, default=8192)
    ap_b.add_argument("--base-chunk", type=int, default=262144)
    args = ap.parse_args()
    if args.cmd == "build":
        build_exact_knn(args.data, args.k, args.out_dir, args.query_chunk, args.base_chunk)


if __name__ == "__main__":
    main()
