"""Benchmark of the bucketed CAGRA-style graph build on one MI355X.

A step is one whole graph build -- 2 rounds of (centroids refined by 3 Lloyd
iterations on a training subset -> probe table -> top-2 assignment -> fused
MFMA kNN over every bucket's pool (own bucket + 1 probe bucket) -> cross-round
merge), sanitize, CAGRA prune, reverse-edge merge -- of configuration C2
(1,000,000 x 128 fp32 integer-valued points, L2, 256 buckets, M 64 -> K 32)
with the dataset already resident in HBM.  Prints one JSON line.

`roofline` is the kNN kernel of the rounds (knn_i8_collect_kernel +
knn_select_kernel when the rows are integers, as C2's are;
knn_f32_collect_kernel + knn_select_kernel for float rows up to 160
dimensions, behind the fp16 screen (knn_screen_kernel) on passes of at least
2^27 pairs; knn_wide_kernel beyond): achieved = the algorithmic ops of its launches
(2*D per scanned (query, pool row) pair) over their summed duration, both
measured by the library with HIP events on its stream.  `traffic` is read
from profiles/<kernel>_<config>_traffic.json (knn_i8_collect_C2_traffic.json
for the default run), the rocprofv3 FETCH_SIZE/WRITE_SIZE measurement of the
same launches (commands in profiles/knn_i8_collect_C2_build.md), when the
knobs are the defaults.  `roofline_prune` / `roofline_revmerge`: the
algorithmic bytes of sanitize + prune and of the reverse merge over their
event times.  `--refine-passes P` adds a `refine` leg (the same build with P
refinement passes: ms per pass, recall before and after, refine_2hop_kernel's
row-gather rate); the `configs` leg reports one pass on C3 and C4.

`search` (after the build) runs the search entry point on workload S2 (the
C2 shape with a 16-dimensional latent structure: a connected graph, unlike
the clustered C mixtures, whose graphs split per cluster): the S2 graph is
built with the same knobs, then 10,000 held-out queries, topk 10, 4 entry
points, ef 64 and the reference CLI's 200; QPS from the device time of the
search kernels, recall@10 against the exact top-10 among the base points,
and the CPU restatement timed on a sample of the queries beside it.

Beside `value` (dataset resident in HBM), the line carries the other two
build-time definitions: `host_to_host` (dataset in host memory, graph and
table back in host memory) and `file_io` (the gtann CLI's bucket2 from a
.fbin file to the reference's output files, a separate process);
`reference_knobs` (3 rounds, KMeans|| data-point centroids, nprobe =
ceil(20000 / avg bucket)) on the same data; `configs` (C1, C3, C4, C5 with the default
knobs: build time, recall@32, kernel fraction of peak); and `cpu_baseline`,
the reference's CPU path on this host (numpy BLAS blocked kNN as
bd/build_knn.py, the reference's own prune and merge headers compiled in
place) on a bounded sample.

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


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(X, knn_ids, K, n_sample, graph=None):
    """The reference's CPU path timed on this host: exact kNN as
    bd/build_knn.py:17-149 computes it (numpy: BLAS A @ B.T over 262,144-row
    base blocks, argpartition + argsort per block and per merge;
    oracle/gt_oracle.py knn_exact_blas) on a bounded sample of queries,
    extrapolated to all N; then sanitize and the reference's own prune and
    rank-ordered reverse merge (src/prune_windowed_core.hpp,
    src/edge_chunk_accumulator.hpp compiled in place into oracle/_ref, rows over
    OpenMP threads as src/prune_windowed.cpp:97 runs them) on the GPU's whole
    kNN table; the CPU restatement in oracle/gt_oracle.c when the reference
    build is absent.  With the GPU's graph given, also reports whether it
    equals the CPU path's prune + merge of the same table bit for bit."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import gt_oracle as O
    N = len(X)
    M = knn_ids.shape[1]
    rng = np.random.default_rng(1)
    q = np.sort(rng.choice(N, n_sample, replace=False))
    t0 = time.perf_counter()
    O.knn_exact_blas(X, M, queries=q, query_chunk=n_sample)
    t_knn_sample = time.perf_counter() - t0
    t_knn = t_knn_sample * N / n_sample
    san = O.sanitize(knn_ids)
    ref = O.ref_available()
    t0 = time.perf_counter()
    if ref:
        fwd, rc = O.ref_cagra_prune_omp(san, K)
    else:
        fwd, rc, _ = O.cagra_prune(san, K)
    t_prune = time.perf_counter() - t0
    t0 = time.perf_counter()
    if ref:
        fin = O.ref_reverse_merge_omp(fwd)
    else:
        fin = O.reverse_merge(fwd)
    t_merge = time.perf_counter() - t0
    same = None if graph is None or rc != 0 else bool(np.array_equal(np.asarray(fin).view(np.uint32), graph))
    total = t_knn + t_prune + t_merge
    try:
        from threadpoolctl import threadpool_info
        blas = [(i.get("internal_api"), i.get("num_threads")) for i in threadpool_info() if i.get("user_api") == "blas"]
    except Exception:
        blas = []
    threads = O.num_threads()
    return {
        "value": N / total / 1e6, "unit": "Mpts/s", "cores": threads, "kind": "port",
        "cpu": cpu_model(), "host_cpus": os.cpu_count(), "blas": blas,
        "parts": {"knn": "port: numpy restatement of bd/build_knn.py:17-149 (BLAS GEMM; argpartition/argsort "
                         "on one thread, as the reference)",
                  "prune_merge": ("reference: prune_windowed_core.hpp + edge_chunk_accumulator.hpp compiled in "
                                  "place (oracle/_ref), OpenMP over rows") if ref else
                                 "port: oracle/gt_oracle.c (reference build absent)"},
        "sample": f"exact kNN of {n_sample} random queries vs all {N} points ({t_knn_sample:.1f} s), extrapolated "
                  f"x{N / n_sample:.0f}; sanitize + prune ({t_prune:.1f} s) and reverse merge ({t_merge:.1f} s) "
                  f"on the whole table",
        "stages_s": {"knn_extrapolated": t_knn, "prune": t_prune, "reverse_merge": t_merge},
        "seconds_extrapolated": total,
        "gpu_graph_identical_to_cpu_prune_merge": same,
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


def knn_roofline(s, D, metric, M=64):
    """Roofline of the round launches of the kNN kernel from the library's
    own event times (mean build stats s).  Integer rows with lists of at most
    64 run as one launch of several kernels (chunk_bounds_kernel: the
    pruning spheres; knn_i8_collect_kernel keeps the pairs under a per-query
    bound; knn_select_kernel reduces them to the top M, or for a seeded pass
    knn_merge_fresh_kernel merges them into the running table, the rows with
    more than M fresh keys through a listed knn_select_kernel +
    knn_merge_run_kernel); the library times the launch as one.

    `achieved`/`frac`: the algorithmic ops, 2*D per (query, pool row) pair of
    the bucketed scan (every pair of every pool, what the reference's GEMM
    computes), over the launch time.  The int8 kernel skips pool chunks whose
    bounding sphere lies beyond every query's bound, so it multiplies fewer
    pairs: `ops_executed_per_launch` / `frac_executed` count those (the
    pairs the MFMAs actually computed, counted on the device).  On fp32 rows
    the fp16 screen (knn_screen_kernel) first computes every pair of each
    work item on the fp16 matrix cores and the fp32 collect kernel then
    scans only the item's union of rows that can reach a list: there
    `pairs_executed_share` is the share of pairs left to the fp32 MFMAs."""
    launches = max(1, int(round(s["knn_launches"])))
    launch_s = s["t_knn"] / launches
    flops = s["knn_flops"] / launches
    pairs = max(float(s.get("knn_pairs", 0.0)), 1.0)
    done = float(s.get("knn_pairs_computed", 0.0)) or pairs
    executed = flops * done / pairs
    int8 = bool(round(s["knn_int8"]))
    mip = 1 if metric == "ip" else 0
    if int8:
        dp = -(-D // 32) * 32
        kname = (f"knn_i8_collect_kernel<{dp}, {mip}> + knn_select_kernel" if 4 < M <= 64 and dp <= 256
                 else f"knn_i8_kernel<{dp}, {mip}>")
        peak, unit = PEAK_INT8_MFMA, "TOP/s"
    elif D <= 256:
        dp = -(-D // 32) * 32
        kname = (f"knn_f32_collect_kernel<{dp}, {mip}> + knn_select_kernel" if 4 < M <= 64 and dp <= 160
                 else f"knn_fused_kernel<{dp}, {mip}>")
        peak, unit = PEAK_FP32_MFMA, "TFLOP/s"
        if done < pairs and 4 < M <= 64 and dp <= 160:   # the fp16 screen ran
            kname = f"knn_screen_kernel<{dp}, {mip}> (fp16) + " + kname
    else:
        kname, peak, unit = f"knn_wide_kernel<{mip}>", PEAK_FP32_MFMA, "TFLOP/s"
    return {"kernel": kname, "bound": "mfma", "achieved": flops / launch_s / 1e12, "peak": peak / 1e12,
            "unit": unit, "frac": flops / launch_s / peak, "flops_per_launch": flops,
            "ops_executed_per_launch": executed, "pairs_executed_share": done / pairs,
            "frac_executed": executed / launch_s / peak,
            "launch_ms": launch_s * 1e3, "launches": launches}


def traffic_file(kernel, config):
    """rocprofv3 FETCH+WRITE bytes per round launch of `kernel` on `config`
    (profiles/<kernel>_<config>_traffic.json, named for the launch's
    distance kernel: a leading fp16 screen is part of the same launch), or
    None."""
    main = kernel.split(" + ")[1] if kernel.startswith("knn_screen_kernel") else kernel
    base = main.split("<")[0].replace("_kernel", "")
    path = os.path.join(ROOT, "profiles", f"{base}_{config}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    return {"bytes_per_launch": d.get("bytes_per_launch"), "mfma_busy_pct": d.get("mfma_busy_pct"),
            "source": d.get("source")}


def mean_stats(stats):
    return {k: float(np.mean([st[k] for st in stats])) for k in stats[0]}


def timed_builds(ctx, torch, X, kw, steps, warmup=1):
    for _ in range(warmup):
        ctx.build_graph(X, **kw)
    torch.cuda.synchronize()
    stats = []
    t0 = time.perf_counter()
    res = None
    for _ in range(steps):
        res = ctx.build_graph(X, **kw)
        stats.append(res.stats)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps, mean_stats(stats), res


def host_to_host_leg(ctx, torch, X, kw, steps):
    """Build seconds with the dataset in host memory and the graph and the
    pre-prune table (ids and distances) back in host memory: the upload,
    the download and pageable-memory staging included."""
    wall, s, res = timed_builds(ctx, torch, X, kw, steps)
    N = len(X)
    return {"ms_per_step": wall * 1e3, "value": N / wall / 1e6, "unit": "Mpts/s",
            "prepare_incl_upload_ms": s["t_prepare"] * 1e3, "download_ms": s["t_download"] * 1e3,
            "outputs": "graph (N x K uint32) + pre-prune table (N x M int32 ids, float32 distances), host memory",
            "input": "dataset as a host numpy array (pageable memory)"}, res


def pinned_graph_leg(ctx, torch, X, kw, steps):
    """Build seconds as the survey defines them: the dataset in (pinned)
    host memory, the final N x K graph back in (pinned) host memory, no
    pre-prune table; the upload and the download are inside the timed
    region."""
    N = len(X)
    Xp = torch.from_numpy(X).pin_memory()
    g = torch.empty((N, kw["K"]), dtype=torch.int32, pin_memory=True)
    ctx.build_graph(Xp, return_knn=False, graph_out=g, **kw)
    stats = []
    t0 = time.perf_counter()
    for _ in range(steps):
        stats.append(ctx.build_graph(Xp, return_knn=False, graph_out=g, **kw).stats)
    wall = (time.perf_counter() - t0) / steps
    s = mean_stats(stats)
    return {"ms_per_step": wall * 1e3, "value": N / wall / 1e6, "unit": "Mpts/s",
            "upload_and_prepare_ms": s["t_prepare"] * 1e3, "download_ms": s["t_download"] * 1e3,
            "input": "dataset in pinned host memory", "output": "graph (N x K uint32) in pinned host memory"}, g


def file_io_leg(X, cfg, args):
    """Build seconds from a .fbin file to the reference's output files: the
    gtann CLI's bucket2 subcommand (read the dataset, build, inline reorder,
    write data_reordered, inverse_perm, bucket files, centroid kNN,
    vector_knn, vector_dists, neighbors.npy and final_graph), as a separate
    process; wall time includes process start and GPU initialisation."""
    import re
    import shutil
    import subprocess
    import tempfile
    import gtann_io
    exe = os.path.join(ROOT, "gpu-talored-ann_amd", "bin", "gtann")
    if not os.path.exists(exe):
        return {"skipped": "gtann CLI not built"}
    N = len(X)
    tmp = tempfile.mkdtemp(prefix="gtann_bench_", dir=os.environ.get("TMPDIR", "/tmp"))
    try:
        path = os.path.join(tmp, "base.fbin")
        gtann_io.write_dataset(path, X)
        cmd = [exe, "bucket2", "-i", path, "-o", os.path.join(tmp, "out"), "--centroid-ratio", repr(cfg.buckets / N),
               "--nprobe", str(args.nprobe if args.nprobe > 0 else 1), "--neighbors-m", str(cfg.M),
               "--fused-optimize-degree", str(cfg.K), "-t", str(args.rounds), "--kmeans-iters",
               str(args.kmeans_iters), "--knn-k", "32"]
        t0 = time.perf_counter()
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
        wall = time.perf_counter() - t0
        if r.returncode != 0:
            return {"error": f"gtann bucket2 exited {r.returncode}: {r.stderr.strip()[-300:]}"}
        m = re.search(r"read ([0-9.]+) s\s+build ([0-9.]+) s.*reorder ([0-9.]+) s\s+write ([0-9.]+) s", r.stdout)
        out = {"wall_s": wall, "value": N / wall / 1e6, "unit": "Mpts/s", "command": " ".join(
            ["gtann"] + cmd[1:3] + ["base.fbin"] + cmd[4:5] + ["out"] + cmd[6:])}
        if m:
            rd, bd, ro, wr = (float(m.group(k)) for k in range(1, 5))
            out.update({"read_s": rd, "build_s": bd, "reorder_s": ro, "write_s": wr,
                        "process_and_init_s": wall - rd - bd - ro - wr})
        files = os.listdir(os.path.join(tmp, "out"))
        out["output_dir"] = files[0] if files else None
        return out
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def recall32(ctx, torch, Xd, knn, metric, n_sample=10000):
    N = Xd.shape[0]
    q = np.random.default_rng(0).choice(N, min(N, n_sample), replace=False)
    ex_i, _ = ctx.knn_exact(Xd, 32, queries=torch.from_numpy(q).cuda(), metric=metric)
    return recall_at(knn[q], ex_i.cpu().numpy(), 32)


def mean_candidates(knn, S, n_sample=2000):
    """Mean number of distinct 2-hop candidates per point that refinement
    computes a distance for: the first S neighbours of the first S
    neighbours, minus invalid ids, the point itself and its own row."""
    N = knn.shape[0]
    rows = np.random.default_rng(1).choice(N, min(N, n_sample), replace=False)
    tot = 0
    for a in rows:
        own = knn[a]
        hop1 = own[:S][(own[:S] >= 0) & (own[:S] < N)]
        c = knn[hop1, :S].ravel()
        c = np.setdiff1d(c[(c >= 0) & (c < N) & (c != a)], own)
        tot += len(c)
    return tot / len(rows)


def refine_leg(ctx, torch, Xd, knn, kw, metric, rec_before, passes=1, S=16, steps=2):
    """The same build with refinement (passes x 2-hop pull join of sample S)
    after the rounds: refine ms per pass, recall@32 before and after, and the
    row-gather rate of refine_2hop_kernel.  Every candidate costs one Dp-float
    row read (from L2 or the MALL when the candidate's bucket is resident
    there, else from HBM); a point also reads its row, its list and its S
    neighbours' lists and writes its list: the HBM minimum of a pass is the
    dataset plus the two tables."""
    N, D = Xd.shape
    Dp = -(-D // 32) * 32
    M = knn.shape[1]
    nc = mean_candidates(knn, S)
    wall, s, res = timed_builds(ctx, torch, Xd, dict(kw, refine_passes=passes, refine_sample=S), steps)
    t = s["t_refine"] / passes
    gather = N * nc * Dp * 4
    hbm_min = N * Dp * 4 + 2 * N * M * 8
    rec = recall32(ctx, torch, Xd, res.knn_ids.cpu().numpy(), metric)
    del res
    return {"passes": passes, "sample": S, "ms_per_build": wall * 1e3, "refine_ms_per_pass": t * 1e3,
            "recall@32_before": rec_before, "recall@32_after": rec,
            "candidates_per_point": nc,
            "roofline_refine": {"kernel": f"refine_2hop_kernel<{2 if Dp <= 256 else 4}>", "bound": "hbm",
                                "achieved": hbm_min / t / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                                "frac": hbm_min / t / PEAK_HBM, "bytes": hbm_min,
                                "row_gather_bytes": gather, "row_gather_GBps": gather / t / 1e9,
                                "note": "bytes = dataset + table in + table out (the HBM minimum of a pass); the "
                                        "kernel is bound by its candidate-row gathers (row_gather_GBps, mostly "
                                        "served by L2 and the MALL: the points go in bucket order)"}}


def configs_leg(ctx, torch, names, steps):
    """Every other BASELINE configuration once more with the default knobs:
    build time, recall@32 on a 10,000-point sample (all of C1) against the
    exact kNN, and the kNN kernel's fraction of its matrix peak."""
    import synth
    out = {}
    for name in names:
        cfg = synth.CONFIGS[name]
        t0 = time.perf_counter()
        X, _ = synth.generate(name)
        tg = time.perf_counter() - t0
        Xd = torch.from_numpy(X).cuda()
        N, D = Xd.shape
        kw = dict(n_buckets=cfg.buckets, M=cfg.M, K=cfg.K, metric=cfg.metric, rounds=2, kmeans_iters=3, nprobe=1)
        wall, s, res = timed_builds(ctx, torch, Xd, kw, steps)
        knn = res.knn_ids.cpu().numpy()
        rec = recall32(ctx, torch, Xd, knn, cfg.metric)
        out[name] = {"workload": f"{name}: {N} x {D} {cfg.dtype}, {cfg.metric.upper()}, {cfg.buckets} buckets, "
                                 f"M {cfg.M} -> K {cfg.K}, 2 rounds, 3 Lloyd iterations, nprobe 1",
                     "ms_per_step": wall * 1e3, "value": N / wall / 1e6, "unit": "Mpts/s", "recall@32": rec,
                     "knn_roofline": dict(knn_roofline(s, D, cfg.metric, cfg.M),
                                          rocprof=traffic_file(knn_roofline(s, D, cfg.metric, cfg.M)["kernel"], name)),
                     "prune_frac_hbm": N * (4 * cfg.M + 4 * cfg.M * (cfg.M - 1) + 4 * cfg.K) / s["t_prune"] / PEAK_HBM,
                     "revmerge_frac_hbm": 28 * N * cfg.K / s["t_revmerge"] / PEAK_HBM,
                     "stages_s": {k: s[k] for k in ("t_prepare", "t_bucketing", "t_knn", "t_merge", "t_prune",
                                                    "t_revmerge", "t_total")}}
        if name in ("C3", "C4"):
            # refinement after the rounds: one pass of sample 16
            out[name]["refine"] = refine_leg(ctx, torch, Xd, knn, kw, cfg.metric, rec)
        print(f"[bench] {name}: {wall * 1e3:.1f} ms, recall@32 {rec:.4f} (data generated in {tg:.1f} s)",
              file=sys.stderr, flush=True)
        del Xd, res, X
        torch.cuda.empty_cache()
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
                    help="headline at the reference's own bucketing settings: 3 rounds, KMeans|| data-point "
                         "centroids, nprobe = ceil(20000 / avg bucket) (also reported as reference_knobs)")
    ap.add_argument("--no-ref-knobs", action="store_true", help="skip the reference_knobs builds")
    ap.add_argument("--cpu-sample", type=int, default=2048)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-io", action="store_true", help="skip the host-to-host and file-I/O legs")
    ap.add_argument("--configs", default="C1,C3,C4,C5",
                    help="other configurations built once more with the default knobs ('' = none)")
    ap.add_argument("--search-queries", type=int, default=10000,
                    help="held-out queries of the search leg (0 = skip it)")
    ap.add_argument("--search-config", default="S2", help="workload of the search leg")
    ap.add_argument("--refine-passes", type=int, default=0,
                    help="also build --config with this many refinement passes after the rounds and report them "
                         "(the headline build has none)")
    ap.add_argument("--refine-sample", type=int, default=16)
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
    ref_kw = dict(rounds=3, kmeans_iters=0, nprobe=-1)
    if args.reference_knobs:
        args.rounds, args.kmeans_iters, args.nprobe = ref_kw["rounds"], ref_kw["kmeans_iters"], ref_kw["nprobe"]
    base_kw = dict(n_buckets=cfg.buckets, M=cfg.M, K=cfg.K, metric=cfg.metric)
    kw = dict(base_kw, rounds=args.rounds, kmeans_iters=args.kmeans_iters, nprobe=args.nprobe)
    wall, s, res = timed_builds(ctx, torch, Xd, kw, args.steps, args.warmup)
    print("[bench] timed builds done", file=sys.stderr, flush=True)

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

    roof = knn_roofline(s, D, cfg.metric, cfg.M)
    int8 = bool(round(s["knn_int8"]))
    default_knobs = (args.rounds, args.kmeans_iters, args.nprobe) == (2, 3, 1)
    tr = traffic_file(roof["kernel"], args.config) if default_knobs else None
    traffic = tr["bytes_per_launch"] if tr else None
    prune_bytes = N * (4 * cfg.M + 4 * cfg.M * (cfg.M - 1) + 4 * cfg.K)
    merge_bytes = 28 * N * cfg.K
    # integer-typed datasets of up to 256 dimensions run the int8 kernel, and
    # so do float datasets whose values are all integers in [-128, 127] or
    # [0, 255] (the library's int_exact: exact, the fp32 kernel's keys)
    dtype = "i8" if int8 else "fp32"
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
            "timed_region": "dataset resident in HBM (torch tensor) to graph and table in HBM",
        },
        "build_seconds": wall,
        **rec,
        "structural": structural,
        "stages_s": {k: s[k] for k in ("t_prepare", "t_bucketing", "t_knn", "t_merge", "t_refine", "t_prune",
                                       "t_revmerge", "t_download", "t_total")},
        "roofline": dict(roof, kernel=roof["kernel"] + " (one launch per round; round 1 split in two when probing)",
                         traffic=traffic),
        "roofline_prune": {"bound": "hbm", "achieved": prune_bytes / s["t_prune"] / 1e9, "peak": 8000.0,
                           "unit": "GB/s", "frac": prune_bytes / s["t_prune"] / PEAK_HBM,
                           "bytes": prune_bytes, "includes": "sanitize + prune"},
        "roofline_revmerge": {"bound": "hbm", "achieved": merge_bytes / s["t_revmerge"] / 1e9, "peak": 8000.0,
                              "unit": "GB/s", "frac": merge_bytes / s["t_revmerge"] / PEAK_HBM,
                              "bytes": merge_bytes, "includes": "scatter + merge (+ slow rows)"},
        "max_pool": int(s["max_pool"]), "max_bucket": int(s["max_bucket"]),
    }
    if int8 and cfg.dtype == "f32":
        # the same build on the fp32 kernel (int_exact off), first without
        # the fp16 screen (every pair on the fp32 matrix cores: the fp32
        # distance kernel's own fraction of the fp32 peak), then as the
        # library runs it by default (behind the screen); both checked to
        # return the int8 path's table and graph
        ctx.set_debug(knn_screen=0)
        try:
            w32, s32, r32 = timed_builds(ctx, torch, Xd, dict(kw, int_exact=False), max(1, min(args.steps, 3)))
        finally:
            ctx.set_debug()
        same = bool(torch.equal(r32.knn_ids, res.knn_ids) and torch.equal(r32.graph, res.graph))
        r = knn_roofline(s32, D, cfg.metric, cfg.M)
        del r32
        wsc, ssc, rsc = timed_builds(ctx, torch, Xd, dict(kw, int_exact=False), max(1, min(args.steps, 3)))
        same_sc = bool(torch.equal(rsc.knn_ids, res.knn_ids) and torch.equal(rsc.graph, res.graph))
        rs = knn_roofline(ssc, D, cfg.metric, cfg.M)
        del rsc
        out["fp32_path"] = {
            "note": "int_exact=0, knn_screen=0: same dataset, every pair on the fp32 matrix cores "
                    "(knn_f32_collect_kernel + knn_select_kernel)",
            "value": N / w32 / 1e6, "unit": "Mpts/s", "ms_per_step": w32 * 1e3,
            "identical_table_and_graph": same,
            "roofline": dict({k: r[k] for k in ("kernel", "bound", "achieved", "peak", "unit", "frac", "launch_ms")},
                             rocprof=traffic_file(r["kernel"], args.config)),
            "screened": {
                "note": "int_exact=0 with the default fp16 screen: the fp32 collect kernel scans only each work "
                        "item's rows that can reach a list",
                "value": N / wsc / 1e6, "unit": "Mpts/s", "ms_per_step": wsc * 1e3,
                "identical_table_and_graph": same_sc, "knn_launch_ms": rs["launch_ms"],
                "fp32_pairs_share": rs["pairs_executed_share"]},
        }
    if args.refine_passes > 0:
        out["refine"] = refine_leg(ctx, torch, Xd, knn, kw, cfg.metric, rec["recall@32"], args.refine_passes,
                                   args.refine_sample, max(1, min(args.steps, 2)))
        print("[bench] refine leg done", file=sys.stderr, flush=True)
    if not args.reference_knobs and not args.no_ref_knobs:
        # the reference's own knobs on the same data
        wr, sr, rr = timed_builds(ctx, torch, Xd, dict(base_kw, **ref_kw), max(1, min(args.steps, 2)))
        out["reference_knobs"] = {
            "knobs": "3 rounds, KMeans|| data-point centroids (D^2 oversampling, no Lloyd; src/bucket.cu:2833-3168), "
                     "nprobe = ceil(20000 / avg bucket) (sk/scripts/params.sh:12, sk/scripts/dataset_env.py:56)",
            "ms_per_step": wr * 1e3, "value": N / wr / 1e6, "unit": "Mpts/s",
            "recall@32": recall_at(rr.knn_ids.cpu().numpy()[q], ex_i, 32),
            "knn_roofline": knn_roofline(sr, D, cfg.metric, cfg.M)}
        del rr
    if not args.no_io:
        h2h, rh = host_to_host_leg(ctx, torch, X, kw, max(1, min(args.steps, 2)))
        h2h["identical_graph_to_device_run"] = bool((rh.graph == graph).all())
        out["host_to_host"] = h2h
        del rh
        pg, gp = pinned_graph_leg(ctx, torch, X, kw, max(1, min(args.steps, 3)))
        pg["identical_graph_to_device_run"] = bool((gp.numpy().view(np.uint32) == graph).all())
        out["host_to_host_graph_pinned"] = pg
        del gp
        out["file_io"] = file_io_leg(X, cfg, args)
        print("[bench] host-to-host and file-I/O legs done", file=sys.stderr, flush=True)
    if args.search_queries > 0:
        del Xd, res
        torch.cuda.empty_cache()
        out["search"] = search_leg(ctx, torch, args.search_config, args.search_queries,
                                   dict(rounds=args.rounds, kmeans_iters=args.kmeans_iters, nprobe=args.nprobe),
                                   (64, 200), 0 if args.no_cpu else 500)
    names = [c for c in args.configs.split(",") if c and c != args.config]
    if names:
        out["configs"] = configs_leg(ctx, torch, names, max(1, min(args.steps, 2)))
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(X, knn, cfg.K, args.cpu_sample, graph)
    ctx.close()
    # the north star's gates in one short object at the end of the line
    ns = {"build_ms": round(wall * 1e3, 3), "Mpts_s": round(N / wall / 1e6, 3),
          "recall@32": round(rec["recall@32"], 4), "recall_gate_0.95": rec["recall@32"] >= 0.95,
          "knn_kernel": roof["kernel"].split(" (")[0], "knn_frac_of_peak": round(roof["frac"], 4),
          "knn_pairs_executed_share": round(roof["pairs_executed_share"], 4),
          "knn_frac_of_peak_executed": round(roof["frac_executed"], 4),
          "knn_launch_ms": round(roof["launch_ms"], 3),
          "knn_traffic_gb_per_launch": round(traffic / 1e9, 3) if traffic else None,
          "knn_mfma_busy_pct": (tr or {}).get("mfma_busy_pct"),
          "prune_frac_hbm": round(out["roofline_prune"]["frac"], 4),
          "revmerge_frac_hbm": round(out["roofline_revmerge"]["frac"], 4)}
    if "fp32_path" in out:
        fp = out["fp32_path"]
        ns["fp32_knn_frac_of_fp32_peak"] = round(fp["roofline"]["frac"], 4)
        ns["fp32_mfma_busy_pct"] = (fp["roofline"].get("rocprof") or {}).get("mfma_busy_pct")
        ns["fp32_identical_table_and_graph"] = fp["identical_table_and_graph"]
        ns["fp32_screened_ms"] = round(fp["screened"]["ms_per_step"], 3)
        ns["fp32_screened_identical_table_and_graph"] = fp["screened"]["identical_table_and_graph"]
    if "cpu_baseline" in out:
        ns["graph_identical_to_cpu_prune_merge"] = out["cpu_baseline"]["gpu_graph_identical_to_cpu_prune_merge"]
    if "host_to_host_graph_pinned" in out:
        ns["host_to_host_graph_pinned_ms"] = round(out["host_to_host_graph_pinned"]["ms_per_step"], 3)
    if "configs" in out:
        ns["configs"] = {k: {"ms": round(v["ms_per_step"], 2), "recall@32": round(v["recall@32"], 4),
                             "knn_frac": round(v["knn_roofline"]["frac"], 3),
                             "knn_mfma_busy_pct": ((v["knn_roofline"].get("rocprof") or {}).get("mfma_busy_pct")),
                             "prune_frac_hbm": round(v["prune_frac_hbm"], 3),
                             "revmerge_frac_hbm": round(v["revmerge_frac_hbm"], 3)} for k, v in out["configs"].items()}
    out["north_star"] = ns
    print(f"[bench] north_star {json.dumps(ns)}", file=sys.stderr, flush=True)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
