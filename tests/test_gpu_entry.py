"""End-to-end checks of the drop-in entry points on the GPU: the gtann CLI
(one subcommand per reference executable, writing the reference's file
layouts) and the Python mirrors of bd/build_knn.py, bd/prune.py and
bd/build_bucket.py -- against the CPU oracle, bit-exact on integer data."""
import os
import subprocess
import sys

import numpy as np
import pytest

import gt_oracle as O
import gtann_io as io
import synth

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gpu-talored-ann_amd")
EXE = os.path.join(PKG, "bin", "gtann")


def _c1_int(n=4000):
    X, _ = synth.generate("C1", n=n)
    return np.rint(X * 8).astype(np.float32)


def _run(args, **kw):
    print("run:", " ".join(map(str, args)), flush=True)
    r = subprocess.run([EXE] + [str(a) for a in args], capture_output=True, text=True, timeout=120, **kw)
    assert r.returncode == 0, r.stderr + r.stdout
    return r


def test_cli_bucket2_and_pipeline_tools(tmp_path, ctx):
    import gtann
    X = _c1_int()
    N = len(X)
    data = tmp_path / "base.fbin"
    io.write_dataset(data, X)
    # 16 buckets, every bucket probed: the table is the exact kNN
    _run(["bucket2", "-i", data, "-o", tmp_path / "out", "--centroid-ratio", 16 / N, "--nprobe", 15, "--knn-k", 8,
          "--neighbors-m", 64, "-t", 1, "--fused-optimize-degree", 32, "--kmeans-iters", 0, "--cache-mb", 64])
    d = tmp_path / "out" / "k8p15m64t1"
    ex_i, ex_d = O.knn_exact(X, 64)
    fwd, rc, _ = O.cagra_prune(O.sanitize(ex_i), 32)
    assert rc == 0
    final = O.reverse_merge(fwd)
    np.testing.assert_array_equal(io.read_graph(d / "final_graph.bin"), final)   # the input's ids

    # round-1 reorder artifacts: the same build through the library, then the
    # processing order and the new-id layout
    res = ctx.build_graph(X, n_buckets=16, nprobe=15, M=64, K=32, rounds=1, kmeans_iters=0, prune=False,
                          round1_bucket=True, centroid_knn_k=15)
    np.testing.assert_array_equal(io.read_graph(d / "centroid_pool.bin"), res.centroid_knn)
    cg = np.ascontiguousarray(res.centroid_knn[:, :8])
    np.testing.assert_array_equal(io.read_graph(d / "centroid_knn.bin"), cg)
    order = gtann.bucket_order(cg, 32)                     # window: 4 x knn-k
    np.testing.assert_array_equal(io.read_bucket_process_order(d / "bucket_process_order.bin"), order)
    inv, off, _ = gtann.bucket_reorder(res.round1_bucket, 16, order)
    np.testing.assert_array_equal(io.read_inverse_perm(d / "inverse_perm.bin"), inv)
    np.testing.assert_array_equal(io.read_bucket_offsets(d / "bucket_offsets.bin"), off)
    for q in range(16):   # position q's range holds bucket order[q]
        assert (res.round1_bucket[inv[off[q]:off[q + 1]]] == order[q]).all()
    perm = np.empty(N, np.int64)
    perm[inv] = np.arange(N)
    np.testing.assert_array_equal(io.read_dataset(str(d / "data_reordered.fbin")), X[inv])
    ids_new = io.read_vector_knn(d / "vector_knn.bin")
    np.testing.assert_array_equal(ids_new, perm[ex_i[inv]].astype(np.int32))
    np.testing.assert_array_equal(io.read_vector_dists(d / "vector_dists.bin"), ex_d[inv])
    np.testing.assert_array_equal(np.load(d / "neighbors.npy"), ids_new.astype(np.int64))

    # Step 5 files of the last round (src/bucket.cu:3434-3510, 9552-9568), in
    # new ids: the same build's last-round buckets and centroid rows
    last = ctx.build_graph(X, n_buckets=16, nprobe=15, M=64, K=32, rounds=1, kmeans_iters=0, prune=False,
                           last_round=True)
    assert (last.last_bucket[last.last_centroids] == np.arange(16)).all()   # KMeans|| seeds: data points
    bnew = last.last_bucket[inv]
    data_ref = np.concatenate([np.flatnonzero(bnew == c) for c in range(16)]).astype("<i4")
    counts = np.bincount(bnew, minlength=16)
    offs = np.concatenate([[0], np.cumsum(counts)[:-1]]) * 4
    rec = np.zeros(16, dtype=[("off", "<i8"), ("count", "<i4")])   # packed: 12 bytes a record
    rec["off"], rec["count"] = offs, counts
    index_ref = np.array([16, N], "<i8").tobytes() + rec.tobytes()
    assert (d / "bucket_data.bin").read_bytes() == data_ref.tobytes()
    assert (d / "bucket_index.bin").read_bytes() == index_ref
    cent_ref = np.concatenate([[16], perm[last.last_centroids]]).astype("<i8")
    assert (d / "centroid_global_indices.bin").read_bytes() == cent_ref.tobytes()
    bi, bd = io.read_bucket_files(d / "bucket_index.bin", d / "bucket_data.bin")
    for c in range(16):
        np.testing.assert_array_equal(bd[c], np.flatnonzero(bnew == c))
    np.testing.assert_array_equal(io.read_centroid_indices(d / "centroid_global_indices.bin"),
                                  perm[last.last_centroids])

    # optimize (prune + reverse merge) of the reordered table
    fwd_n, rc, _ = O.cagra_prune(O.sanitize(ids_new), 32)
    final_n = O.reverse_merge(fwd_n)
    _run(["optimize", "-i", d / "data_reordered.fbin", "-g", d / "vector_knn.bin", "-o", tmp_path / "g2.bin",
          "--output-degree", 32, "--skip-sort"])
    np.testing.assert_array_equal(io.read_graph(tmp_path / "g2.bin"), final_n)
    # the out-of-core path's tools: prune_windowed -> optimize_chunked -m E (+ translate to the input's ids)
    _run(["prune_windowed", "-k", d / "vector_knn.bin", "-i", d / "data_reordered.fbin", "-o", tmp_path / "fwd.bin",
          "--output-degree", 32, "--bucket-offsets", d / "bucket_offsets.bin", "--cache-mb", 8])
    np.testing.assert_array_equal(io.read_graph(tmp_path / "fwd.bin"), fwd_n)
    _run(["optimize_chunked", "-g", tmp_path / "fwd.bin", "-o", tmp_path / "e.bin", "-m", "E",
          "--inverse-perm", d / "inverse_perm.bin", "--final-output", tmp_path / "final.bin"])
    np.testing.assert_array_equal(io.read_graph(tmp_path / "e.bin"), final_n)
    # with a budget below the graph: destination chunks, the same rows
    _run(["optimize_chunked", "-g", tmp_path / "fwd.bin", "-o", tmp_path / "e2.bin", "-m", "E",
          "--gpu-budget-mb", 1])
    np.testing.assert_array_equal(io.read_graph(tmp_path / "e2.bin"), final_n)
    # the windowed prune: position q's window = q + the positions of its
    # bucket's centroid-kNN neighbours (src/prune_windowed.cpp:370-385)
    _run(["prune_windowed", "-k", d / "vector_knn.bin", "-i", d / "data_reordered.fbin", "-o", tmp_path / "fw.bin",
          "--output-degree", 32, "--bucket-offsets", d / "bucket_offsets.bin", "--bucket-process-order",
          d / "bucket_process_order.bin", "-c", d / "centroid_knn.bin", "--cache-mb", 1])
    pos_of = np.empty(16, np.int64)
    pos_of[order] = np.arange(16)
    win = np.zeros((16, 9), np.int32)
    wl = np.zeros(16, np.int32)
    for q in range(16):
        w = sorted({q} | {int(pos_of[b]) for b in cg[order[q]] if b != order[q] and b < 16})
        win[q, :len(w)] = w
        wl[q] = len(w)
    ref_w, rc, _ = O.prune_windowed(ids_new, off, win, wl, 32)
    assert rc == 0
    np.testing.assert_array_equal(io.read_graph(tmp_path / "fw.bin"), ref_w)
    np.testing.assert_array_equal(io.read_graph(tmp_path / "final.bin"), O.translate(final_n, inv))
    _run(["translate_ids", "-g", tmp_path / "e.bin", "-p", d / "inverse_perm.bin", "-o", tmp_path / "t.bin"])
    np.testing.assert_array_equal(io.read_graph(tmp_path / "t.bin"), O.translate(final_n, inv))


def test_permute_rows_and_remap_table(ctx):
    import gtann
    rng = np.random.default_rng(12)
    N = 5000
    inv = rng.permutation(N).astype(np.uint32)
    perm = np.empty(N, np.int64)
    perm[inv] = np.arange(N)
    for X in (rng.standard_normal((N, 37)).astype(np.float32), rng.integers(0, 256, (N, 13)).astype(np.uint8),
              rng.integers(-128, 128, (N, 64)).astype(np.int8), rng.standard_normal((N, 128)).astype(np.float32)):
        np.testing.assert_array_equal(ctx.permute_rows(X, inv), X[inv])
    ids = rng.integers(-1, N, size=(N, 24)).astype(np.int32)
    ids[5, 3] = N + 7   # out of range -> -1
    exp = np.where(ids[inv] >= 0, perm[np.clip(ids[inv], 0, N - 1)], -1)
    exp[np.nonzero(inv == 5)[0][0], 3] = -1
    np.testing.assert_array_equal(ctx.remap_table(ids, inv), exp.astype(np.int32))
    bad = inv.copy()
    bad[0] = bad[1]
    with pytest.raises(gtann.GtannError, match="permutation"):
        ctx.permute_rows(np.zeros((N, 4), np.float32), bad)
    with pytest.raises(gtann.GtannError, match="permutation"):
        ctx.remap_table(ids, bad)


def test_cli_knn_u8_and_i8(tmp_path):
    rng = np.random.default_rng(4)
    for ext, dt in ((".u8bin", np.uint8), (".i8bin", np.int8)):
        lo, hi = (0, 256) if dt == np.uint8 else (-128, 128)
        X = rng.integers(lo, hi, size=(3000, 96)).astype(dt)
        io.write_dataset(tmp_path / f"x{ext}", X)
        _run(["knn", "-i", tmp_path / f"x{ext}", "-o", tmp_path / ext[1:], "-k", 24])
        ex_i, ex_d = O.knn_exact(X.astype(np.float32), 24)
        np.testing.assert_array_equal(io.read_vector_knn(tmp_path / ext[1:] / "vector_knn.bin"), ex_i)
        np.testing.assert_array_equal(np.load(tmp_path / ext[1:] / "exact_knn_dist.npy"), ex_d)


def test_cli_bucket2_multi_round_recall(tmp_path):
    X, _ = synth.generate("C2", n=50000)
    io.write_dataset(tmp_path / "c2.fbin", X)
    r = _run(["bucket2", "-i", tmp_path / "c2.fbin", "-o", tmp_path / "o", "--centroid-ratio", 0.00032,
              "--nprobe", 1, "--knn-k", 8, "--neighbors-m", 64, "-t", 2, "--fused-optimize-degree", 32, "--skip-npy"])
    assert "build" in r.stdout
    d = tmp_path / "o" / "k8p1m64t2"
    ids = io.read_vector_knn(d / "vector_knn.bin")          # new ids
    inv = io.read_inverse_perm(d / "inverse_perm.bin")
    perm = np.empty(len(X), np.int64)
    perm[inv] = np.arange(len(X))
    assert not (d / "neighbors.npy").exists()
    q = np.arange(0, len(X), 173)
    ex_i, _ = O.knn_exact(X, 32, queries=q)
    rec = np.mean([len(np.intersect1d(inv[ids[perm[qq], :32]], ex_i[j])) / 32 for j, qq in enumerate(q)])
    assert rec > 0.9, rec
    g = io.read_graph(d / "final_graph.bin")
    assert g.shape == (len(X), 32) and (g < len(X)).all()
    # --gpu-limit far below the tables: the out-of-core build writes the same files
    _run(["bucket2", "-i", tmp_path / "c2.fbin", "-o", tmp_path / "o2", "--centroid-ratio", 0.00032,
          "--nprobe", 1, "--knn-k", 8, "--neighbors-m", 64, "-t", 2, "--fused-optimize-degree", 32, "--skip-npy",
          "--gpu-limit", 32 << 20])
    d2 = tmp_path / "o2" / "k8p1m64t2"
    np.testing.assert_array_equal(io.read_vector_knn(d2 / "vector_knn.bin"), ids)
    np.testing.assert_array_equal(io.read_graph(d2 / "final_graph.bin"), g)


def test_python_build_knn_mirror(tmp_path, ctx):
    import build_knn
    rng = np.random.default_rng(2)
    X = rng.integers(0, 256, size=(2500, 128)).astype(np.uint8)
    io.write_dataset(tmp_path / "x.u8bin", X)
    ip, dp = build_knn.build_exact_knn(str(tmp_path / "x.u8bin"), 16, str(tmp_path / "o"), ctx=ctx)
    ids, d = np.load(ip), np.load(dp)
    assert ids.dtype == np.int64 and d.dtype == np.float32
    ex_i, ex_d = O.knn_exact(X.astype(np.float32), 16)
    np.testing.assert_array_equal(ids, ex_i)
    np.testing.assert_array_equal(d, ex_d)


def test_python_prune_mirror(tmp_path, ctx):
    import prune
    X = _c1_int(3000)
    ex_i, _ = O.knn_exact(X, 48)
    nb = ex_i.astype(np.int64)
    nb[5, 3] = 10 ** 10                       # out of range: dropped
    out = prune.prune_graph(X, nb, 24, ctx=ctx)
    assert out.dtype == np.int64 and out.shape == nb.shape
    np.testing.assert_array_equal(out, O.prune_occlusion(X, nb, 24))
    out = prune.prune_graph(X, nb, None, ctx=ctx)
    np.testing.assert_array_equal(out, O.prune_occlusion(X, nb, 0))
    cg = prune.prune_graph(X, ex_i, 32, algo="cagra", ctx=ctx)
    fwd, rc, _ = O.cagra_prune(O.sanitize(ex_i), 32)
    np.testing.assert_array_equal(cg[:, :32], O.reverse_merge(fwd).astype(np.int64))
    assert (cg[:, 32:] == -1).all()
    with pytest.raises(ValueError):
        prune.prune_graph(X, nb[:10], 8, ctx=ctx)
    with pytest.raises(ValueError):
        prune.prune_graph(X, nb.astype(np.float32), 8, ctx=ctx)
    # the prune_existing command end to end
    io.write_dataset(tmp_path / "x.fbin", X)
    np.save(tmp_path / "in.npy", nb)
    subprocess.run([sys.executable, os.path.join(PKG, "prune.py"), "prune_existing", "--data", str(tmp_path / "x.fbin"),
                    "--index_in", str(tmp_path / "in.npy"), "--index_out", str(tmp_path / "out.npy"),
                    "--max_degree", "24"], check=True, timeout=120)
    np.testing.assert_array_equal(np.load(tmp_path / "out.npy"), O.prune_occlusion(X, nb, 24))


def test_python_build_bucket_mirror(tmp_path):
    X = _c1_int(4096)
    io.write_dataset(tmp_path / "x.fbin", X)
    # 128 buckets of ~32; --k 127 probes every other bucket: each round is
    # exact and reverse insertion leaves an exact table unchanged
    cmd = [sys.executable, os.path.join(PKG, "build_bucket.py"), "--data", str(tmp_path / "x.fbin"), "--k", "127",
           "--m", "32", "--out_dir", str(tmp_path / "o"), "--t", "2", "--kmeans-iters", "2"]
    print("run:", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True, timeout=180)
    nbr = np.load(tmp_path / "o" / "neighbors_k127m32t2.npy")
    dst = np.load(tmp_path / "o" / "neighbors_dist_k127m32t2.npy")
    meta = np.load(tmp_path / "o" / "meta_k127m32t2.npy", allow_pickle=True).item()   # written by this test
    assert meta == {"N": 4096, "D": 128, "k": 127, "m": 32, "t": 2}
    ex_i, ex_d = O.knn_exact(X, 32)
    np.testing.assert_array_equal(nbr, ex_i.astype(np.int64))
    np.testing.assert_array_equal(dst, ex_d)
