"""Benchmark of the bucketed CAGRA-style graph build on one MI355X.

A step is one whole graph build -- 2 rounds of (centroids refined by 3 Lloyd
iterations on a training subset -> probe table -> top-2 assignment -> fused
MFMA kNN over every bucket's pool (own bucket + 1 probe bucket) -> cross-round
merge), sanitize, CAGRA prune, reverse-edge merge -- of configuration C2
(1,000,000 x 128 fp32 integer-valued points, L2, 256 buckets, M 64 -> K 32)
with the dataset already resident in HBM.  Prints one JSON line.

`roofline` is the kNN kernel of the rounds (knn_i8_kernel when the rows are
integers, as C2's are; knn_fused_kernel / knn_wide_kernel otherwise):
achieved = the algorithmic ops of its launches (2*D per scanned (query, pool
row) pair) over their summed duration, both measured by the library with HIP
events on its stream.  `traffic` is read from
profiles/<kernel>_<config>_traffic.json (knn_i8_C2_traffic.json for the
default run), the rocprofv3 FETCH_SIZE/WRITE_SIZE measurement of the same
launches (commands in profiles/knn_i8_C2_build.md), when the knobs are the
defaults.

`search` (after the build) runs the search entry point on workload S2 (the
C2 shape with a 16-dimensional latent structure: a connected graph, unlike
the clustered C mixtures, whose graphs split per cluster): the S2 graph is
built with the same knobs, then 10,000 held-out queries, topk 10, 4 entry
points, ef 64 and the reference CLI's 200; QPS from the device time of the
search kernels, recall@10 against the exact top-10 among the base points,
and the CPU restatement timed on a sample of the queries beside it.

    python bench.py [--gpus 1] [--steps 3] [--warmup 1] [--config C2]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gpu-talored-ann_amd"))

PEAK_FP32_MFMA = 157.3e12   # MI355X dense fp32 matrix, FLOP/s
PEAK_INT8_MFMA = 5.0e15     # MI355X dense int8 matrix, OP/s
PEAK_HBM = 8.0e12           # MI355X HBM3E, B/s


def recall_at(approx, exact, k):
    return float(np.mean([len(np.intersect1d(approx[i, :k], exact[i, :k])) / k for i in range(len(exact))]))


def cpu_baseline(X, knn_ids, K, n_sample):
    """The CPU restatement of the reference path (exact kNN -> sanitize ->
    CAGRA prune -> reverse merge, oracle/gt_oracle.c) timed on this host on a
    bounded sample and extrapolated to the whole build."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import gt_oracle as O
    N = len(X)
    rng = np.random.default_rng(1)
    q = np.sort(rng.choice(N, n_sample, replace=False))
    t0 = time.perf_counter()
    O.knn_exact(X, knn_ids.shape[1], queries=q)
    t_knn = (time.perf_counter() - t0) * N / n_sample
    # prune of the sampled rows needs every row they reference: time the
    # whole-table sanitize + prune + merge on the GPU's own kNN table
    t0 = time.perf_counter()
    san = O.sanitize(knn_ids)
    fwd, rc, _ = O.cagra_prune(san, K)
    t_prune = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.reverse_merge(fwd)
    t_merge = time.perf_counter() - t0
    total = t_knn + t_prune + t_merge
    return {
        "value": N / total / 1e6, "unit": "Mpts/s", "cores": O.num_threads(), "kind": "port",
        "sample": f"exact kNN of {n_sample} random queries vs all {N} points, extrapolated x{N / n_sample:.0f} "
                  f"({t_knn:.1f} s); sanitize+prune ({t_prune:.1f} s) and reverse merge ({t_merge:.1f} s) "
                  f"measured on the full table",
        "seconds_extrapolated": total,
    }


def search_leg(ctx, torch, name, nq, kw, efs, cpu_sample):
    """The search entry point on a graph built from workload `name`: nq
    held-out queries of the same distribution, the reference CLI's topk 10 /
    num_entry 4 (bd/search.py:280-283), recall@10 against the exact top-10
    among the base points, device time of the search kernels from the
    library; the CPU restatement (oracle/gt_oracle.c) timed on cpu_sample
    queries at the largest ef."""
    import synth
    cfg = synth.CONFIGS[name]
    X, Q = synth.generate(name, queries=nq)
    Xd = torch.from_numpy(X).cuda()
    graph = ctx.build_graph(Xd, n_buckets=cfg.buckets, M=cfg.M, K=cfg.K, metric=cfg.metric, **kw).graph
    N, D = Xd.shape
    nq = len(Q)
    Qd = torch.from_numpy(Q).cuda()
    qids = torch.arange(N, N + nq, device="cuda", dtype=torch.int64)
    ex_i, _ = ctx.knn_exact(torch.cat([Xd, Qd]), 32, queries=qids, metric=cfg.metric)
    ex = ex_i.cpu().numpy()
    gt = [row[(row >= 0) & (row < N)][:10] for row in ex]
    deg = int(graph.shape[1])
    runs = []
    for ef in efs:
        ctx.search(Xd, graph, Qd, topk=10, ef=ef, num_entry=4, metric=cfg.metric)   # warm-up
        ids, _, st = ctx.search(Xd, graph, Qd, topk=10, ef=ef, num_entry=4, metric=cfg.metric)
        ids = ids.cpu().numpy()
        rec = float(np.mean([len(np.intersect1d(ids[i], gt[i])) / 10 for i in range(nq)]))
        # algorithmic bytes: one graph row per expansion, one fp32 row per distance
        nbytes = st["expansions"] * deg * 4 + st["visited"] * D * 4 + nq * D * 4
        runs.append({
            "ef": ef, "qps": nq / st["t_search"], "ms": st["t_search"] * 1e3, "recall@10": rec,
            "expansions_per_query": st["expansions"] / nq, "visited_per_query": st["visited"] / nq,
            "requeued": st["requeued"],
            "roofline": {"bound": "hbm", "achieved": nbytes / st["t_search"] / 1e9, "peak": 8000.0, "unit": "GB/s",
                         "frac": nbytes / st["t_search"] / PEAK_HBM, "bytes": nbytes,
                         "note": "one wave per query, latency-bound (serial best-first steps)"},
        })
        print(f"[bench] search ef={ef}: {runs[-1]['qps']:.0f} QPS, recall@10 {rec:.4f}", file=sys.stderr,
              flush=True)
    out = {"kernel": "graph_search_kernel", "workload": f"{name}: {N} x {D} {cfg.dtype}, graph degree {deg}",
           "queries": nq, "topk": 10, "num_entry": 4, "runs": runs}
    if cpu_sample:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import gt_oracle as O
        rng = np.random.default_rng(2)
        ent = rng.integers(0, N, size=(cpu_sample, 4)).astype(np.int32)
        g = graph.cpu().numpy().view(np.uint32)
        t0 = time.perf_counter()
        O.search(X, g, Q[:cpu_sample], ent, 10, efs[-1], metric=1 if cfg.metric == "ip" else 0)
        t = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": cpu_sample / t, "unit": "QPS", "cores": O.num_threads(), "kind": "port",
                               "sample": f"{cpu_sample} queries at ef {efs[-1]}"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="C2")
    ap.add_argument("--rounds", type=int, default=2)
    ap.add_argument("--kmeans-iters", type=int, default=3)
    ap.add_argument("--nprobe", type=int, default=1)
    ap.add_argument("--reference-knobs", action="store_true",
                    help="the reference's own bucketing settings: 3 rounds, sampled data points as "
                         "centroids, nprobe = ceil(20000 / avg bucket)")
    ap.add_argument("--cpu-sample", type=int, default=2000)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--search-queries", type=int, default=10000,
                    help="held-out queries of the search leg (0 = skip it)")
    ap.add_argument("--search-config", default="S2", help="workload of the search leg")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run one device-to-device copy of this many MiB first (calibrates the "
                         "FETCH_SIZE/WRITE_SIZE counters of rocprofv3 --pmc against known bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the bucketed build would shard by bucket, but no multi-GPU path exists)",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import gtann
    import synth

    cfg = synth.CONFIGS[args.config]
    t0 = time.perf_counter()
    X, _ = synth.generate(args.config)
    print(f"[bench] {args.config} generated {X.shape} {X.dtype} in {time.perf_counter() - t0:.1f} s",
          file=sys.stderr, flush=True)
    N, D = X.shape
    Xd = torch.from_numpy(X).cuda()
    if args.copy_probe_mib:
        src = torch.empty(args.copy_probe_mib << 18, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        del src, dst
    torch.cuda.synchronize()
    ctx = gtann.Context(0)
    if args.reference_knobs:
        args.rounds, args.kmeans_iters, args.nprobe = 3, 0, -1
    kw = dict(n_buckets=cfg.buckets, M=cfg.M, K=cfg.K, rounds=args.rounds, metric=cfg.metric,
              kmeans_iters=args.kmeans_iters, nprobe=args.nprobe)
    for _ in range(args.warmup):
        ctx.build_graph(Xd, **kw)
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)
    stats = []
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = ctx.build_graph(Xd, **kw)
        stats.append(res.stats)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps

    # quality: recall of the pre-prune table vs exact kNN on 10,000 sampled points
    q = np.random.default_rng(0).choice(N, 10000, replace=False)
    ex_i, _ = ctx.knn_exact(Xd, 64, queries=torch.from_numpy(q).cuda(), metric=cfg.metric)
    ex_i = ex_i.cpu().numpy()
    knn = res.knn_ids.cpu().numpy()
    rec = {f"recall@{k}": recall_at(knn[q], ex_i, k) for k in (1, 10, 32, 64)}
    graph = res.graph.cpu().numpy().view(np.uint32)
    structural = {
        "bad_ids": int((graph >= N).sum()),
        "self_loops": int((graph == np.arange(N, dtype=np.uint32)[:, None]).sum()),
        "dup_edges": int(sum(len(r) - len(np.unique(r)) for r in graph[:20000])),
        "degree": int(graph.shape[1]),
    }

    s = {k: float(np.mean([st[k] for st in stats])) for k in stats[0]}
    launches = max(1, int(round(s["knn_launches"])))
    knn_launch_s = s["t_knn"] / launches
    flops_launch = s["knn_flops"] / launches
    achieved = flops_launch / knn_launch_s
    traffic = None
    kbase = "knn_i8" if bool(round(s["knn_int8"])) else ("knn_fused" if D <= 256 else "knn_wide")
    tfile = os.path.join(ROOT, "profiles", f"{kbase}_{args.config}_traffic.json")
    default_knobs = (args.rounds, args.kmeans_iters, args.nprobe) == (2, 3, 1)
    if default_knobs and os.path.exists(tfile):
        with open(tfile) as f:
            traffic = json.load(f).get("bytes_per_launch")
    prune_bytes = N * (4 * cfg.M + 4 * cfg.M * (cfg.M - 1) + 4 * cfg.K)
    merge_bytes = 28 * N * cfg.K

    # integer-typed datasets of up to 256 dimensions run the int8 kernel, and
    # so do float datasets whose values are all integers in [-128, 127] or
    # [0, 255] (the library's int_exact: exact, the fp32 kernel's keys)
    int8 = bool(round(s["knn_int8"]))
    dtype = "i8" if int8 else "fp32"
    mip = 1 if cfg.metric == "ip" else 0
    if int8:
        kname, peak, punit = f"knn_i8_kernel<{-(-D // 32) * 32}, {mip}>", PEAK_INT8_MFMA, "TOP/s"
    elif D <= 256:
        kname, peak, punit = f"knn_fused_kernel<{-(-D // 32) * 32}, {mip}>", PEAK_FP32_MFMA, "TFLOP/s"
    else:
        kname, peak, punit = f"knn_wide_kernel<{mip}>", PEAK_FP32_MFMA, "TFLOP/s"
    out = {
        "metric": f"graph build Mpts/s at {N // 1000000 if N >= 1000000 else N}"
                  f"{'M' if N >= 1000000 else ''}x{D} {'fp32' if cfg.dtype == 'f32' else cfg.dtype} deg{cfg.K} "
                  f"(build seconds = ms_per_step/1000)",
        "value": N / wall / 1e6,
        "unit": "Mpts/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype if cfg.dtype != "f32" or not int8 else "i8 (exact: integer-valued fp32 rows, int32 sums)",
        "data": "synthetic (seeded Gaussian mixture, gpu-talored-ann_amd/synth.py)",
        "config": {
            "workload": f"{args.config}: {N} x {D} {cfg.dtype}, {cfg.metric.upper()}, {cfg.buckets} buckets, "
                        f"M {cfg.M} -> K {cfg.K}, {args.rounds} rounds, {args.kmeans_iters} Lloyd iterations, "
                        f"nprobe {args.nprobe if args.nprobe >= 0 else 'ceil(20000/avg bucket)'}",
            "points": N, "dim": D, "buckets": cfg.buckets, "M": cfg.M, "K": cfg.K, "rounds": args.rounds,
            "kmeans_iters": args.kmeans_iters, "nprobe": args.nprobe,
        },
        "build_seconds": wall,
        **rec,
        "structural": structural,
        "stages_s": {k: s[k] for k in ("t_prepare", "t_bucketing", "t_knn", "t_merge", "t_refine", "t_prune",
                                       "t_revmerge", "t_download", "t_total")},
        "roofline": {
            "kernel": kname + " (one launch per round; round 1 split in two when probing)",
            "bound": "mfma", "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": punit,
            "frac": achieved / peak, "traffic": traffic,
            "flops_per_launch": flops_launch, "launch_ms": knn_launch_s * 1e3, "launches": launches,
        },
        "roofline_prune": {"bound": "hbm", "achieved": prune_bytes / s["t_prune"] / 1e9, "peak": 8000.0,
                           "unit": "GB/s", "frac": prune_bytes / s["t_prune"] / PEAK_HBM,
                           "bytes": prune_bytes, "includes": "sanitize + prune"},
        "roofline_revmerge": {"bound": "hbm", "achieved": merge_bytes / s["t_revmerge"] / 1e9, "peak": 8000.0,
                              "unit": "GB/s", "frac": merge_bytes / s["t_revmerge"] / PEAK_HBM,
                              "bytes": merge_bytes, "includes": "count + scan + scatter + merge"},
        "max_pool": int(s["max_pool"]), "max_bucket": int(s["max_bucket"]),
    }
    if int8 and cfg.dtype == "f32":
        # the same build on the fp32 kernel (int_exact off): its time, its
        # fraction of the fp32 matrix peak, and the check that both paths
        # return the same table and graph
        kw32 = dict(kw, int_exact=False)
        ctx.build_graph(Xd, **kw32)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        st32 = []
        for _ in range(max(1, min(args.steps, 3))):
            r32 = ctx.build_graph(Xd, **kw32)
            st32.append(r32.stats)
        torch.cuda.synchronize()
        wall32 = (time.perf_counter() - t1) / len(st32)
        s32 = {k: float(np.mean([st[k] for st in st32])) for k in st32[0]}
        l32 = max(1, int(round(s32["knn_launches"])))
        ach32 = (s32["knn_flops"] / l32) / (s32["t_knn"] / l32)
        same = bool(torch.equal(r32.knn_ids, res.knn_ids) and torch.equal(r32.graph, res.graph))
        out["fp32_path"] = {
            "note": "int_exact=0: same dataset on knn_fused_kernel (fp32 matrix cores)",
            "value": N / wall32 / 1e6, "unit": "Mpts/s", "ms_per_step": wall32 * 1e3,
            "identical_table_and_graph": same,
            "roofline": {"kernel": f"knn_fused_kernel<{-(-D // 32) * 32}, {mip}>", "bound": "mfma",
                         "achieved": ach32 / 1e12, "peak": PEAK_FP32_MFMA / 1e12, "unit": "TFLOP/s",
                         "frac": ach32 / PEAK_FP32_MFMA, "launch_ms": s32["t_knn"] / l32 * 1e3},
        }
        del r32
    if args.search_queries > 0:
        del Xd, res
        out["search"] = search_leg(ctx, torch, args.search_config, args.search_queries,
                                   dict(rounds=args.rounds, kmeans_iters=args.kmeans_iters, nprobe=args.nprobe),
                                   (64, 200), 0 if args.no_cpu else 500)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(X, knn, cfg.K, args.cpu_sample)
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
