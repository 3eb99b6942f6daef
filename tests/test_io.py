"""On-disk formats: this build's writers and readers (Python gtann_io, the
C++ gtann_io.hpp used by the gtann CLI, the load.py mirror) against the
reference's own writers and readers (src/graph_io.hpp, src/load.hpp compiled
into oracle/_ref) -- byte for byte."""
import os
import subprocess

import numpy as np
import pytest

import gt_oracle as O
import gtann_io as io
import load as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR = os.path.join(ROOT, "gpu-talored-ann_amd", "csrc")
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="reference harness not built")


def _bytes(p):
    with open(p, "rb") as f:
        return f.read()


def _contents():
    """the deterministic contents tests/io_driver.cpp writes"""
    N, W, D = 37, 5, 7
    i = np.arange(N * W)
    knn = np.where(i % 11 == 0, -1, (i * 7) % N).astype(np.int32).reshape(N, W)
    dist = (0.25 * i).astype(np.float32).reshape(N, W)
    g = ((i * 13) % N).astype(np.uint32).reshape(N, W)
    j = np.arange(N * D)
    x = (0.5 * j - 3.0).astype(np.float32).reshape(N, D)
    u8 = ((j * 5) % 256).astype(np.uint8).reshape(N, D)
    i8 = (((j * 5) % 256) - 128).astype(np.int8).reshape(N, D)
    perm = ((np.arange(N) * 5) % N).astype(np.uint32)
    return dict(knn=knn, dist=dist, g=g, x=x, u8=u8, i8=i8, perm=perm)


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    d = tmp_path_factory.mktemp("iodrv")
    exe = d / "io_driver"
    subprocess.run(["g++", "-O1", "-std=c++17", "-I", HDR, "-o", str(exe),
                    os.path.join(ROOT, "tests", "io_driver.cpp")], check=True)
    out = d / "files"
    out.mkdir()
    subprocess.run([str(exe), "write", str(out)], check=True)
    return exe, out


@needs_ref
def test_python_writers_match_reference_bytes(tmp_path):
    c = _contents()
    io.write_vector_knn(tmp_path / "a.bin", c["knn"])
    O.ref_write_vector_knn(tmp_path / "b.bin", c["knn"])
    assert _bytes(tmp_path / "a.bin") == _bytes(tmp_path / "b.bin")
    io.write_graph(tmp_path / "c.bin", c["g"])
    O.ref_write_graph(tmp_path / "d.bin", c["g"])
    assert _bytes(tmp_path / "c.bin") == _bytes(tmp_path / "d.bin")
    io.write_inverse_perm(tmp_path / "e.bin", c["perm"])
    O.ref_write_u32_vector(tmp_path / "f.bin", c["perm"])
    assert _bytes(tmp_path / "e.bin") == _bytes(tmp_path / "f.bin")


@needs_ref
def test_cpp_writers_match_reference_bytes(driver, tmp_path):
    _, out = driver
    c = _contents()
    O.ref_write_vector_knn(tmp_path / "knn.bin", c["knn"])
    assert _bytes(out / "vector_knn.bin") == _bytes(tmp_path / "knn.bin")
    O.ref_write_graph(tmp_path / "g.bin", c["g"])
    assert _bytes(out / "graph.bin") == _bytes(tmp_path / "g.bin")
    O.ref_write_u32_vector(tmp_path / "p.bin", c["perm"])
    assert _bytes(out / "inverse_perm.bin") == _bytes(tmp_path / "p.bin")
    # vector_dists.bin has the vector_knn layout with float payload
    raw = _bytes(out / "vector_dists.bin")
    assert raw[:12] == _bytes(tmp_path / "knn.bin")[:12]
    np.testing.assert_array_equal(np.frombuffer(raw[12:], np.float32).reshape(37, 5), c["dist"])


@needs_ref
def test_readers_agree_with_reference(driver):
    _, out = driver
    c = _contents()
    np.testing.assert_array_equal(io.read_vector_knn(out / "vector_knn.bin"), O.ref_read_vector_knn(out / "vector_knn.bin"))
    np.testing.assert_array_equal(io.read_graph(out / "graph.bin"), O.ref_read_graph(out / "graph.bin"))
    np.testing.assert_array_equal(io.read_vector_dists(out / "vector_dists.bin"), c["dist"])
    np.testing.assert_array_equal(io.read_inverse_perm(out / "inverse_perm.bin"), c["perm"])
    for name, key in (("x.fbin", "x"), ("x.u8bin", "u8"), ("x.i8bin", "i8")):
        mine = io.read_dataset(out / name)
        np.testing.assert_array_equal(mine, c[key])
        # the C++ pipeline's reader (src/load.hpp) converts .i8bin as signed
        np.testing.assert_array_equal(O.ref_read_dataset(out / name), mine.astype(np.float32))


def test_cpp_reader_and_npy(driver):
    exe, out = driver
    c = _contents()
    for name, key in (("x.fbin", "x"), ("x.u8bin", "u8"), ("x.i8bin", "i8")):
        r = subprocess.run([str(exe), "read", str(out / name)], check=True, capture_output=True, text=True)
        n, d, s = r.stdout.split()
        assert (int(n), int(d)) == c[key].shape
        assert float(s) == pytest.approx(float(c[key].astype(np.float64).sum()))
    ids = np.load(out / "ids.npy")
    assert ids.dtype == np.int64
    np.testing.assert_array_equal(ids, c["knn"])
    dist = np.load(out / "dist.npy")
    np.testing.assert_array_equal(dist, c["dist"])
    with open(out / "ids.npy", "rb") as f:
        head = f.read(10)
    assert (10 + int.from_bytes(head[8:10], "little")) % 64 == 0


def test_python_loader_mirror(driver, tmp_path):
    _, out = driver
    c = _contents()
    # bd/load.py reads .i8bin bytes as uint8 (its own pipeline's reading)
    X, N, D = L.load_bigann_to_f32(str(out / "x.i8bin"))
    np.testing.assert_array_equal(X, c["i8"].view(np.uint8).astype(np.float32))
    X, N, D = L.load_bigann_to_f32(str(out / "x.fbin"))
    np.testing.assert_array_equal(X, c["x"])
    np.testing.assert_array_equal(L.load_dataset(str(out / "x.i8bin")), c["i8"])
    t = L.load_bigann_bin(str(out / "x.u8bin"))
    np.testing.assert_array_equal(t.numpy(), c["u8"].astype(np.float32))
    raw = _bytes(out / "x.fbin")
    (tmp_path / "x.xyz").write_bytes(raw)
    with pytest.raises(ValueError):
        L.load_bigann_to_f32(str(tmp_path / "x.xyz"))
    # truncated payload
    (tmp_path / "t.fbin").write_bytes(raw[:-4])
    with pytest.raises(ValueError):
        L.load_bigann_to_f32(str(tmp_path / "t.fbin"))
    with pytest.raises(ValueError):
        io.read_dataset(tmp_path / "t.fbin")
    # neighbors.npy rules (bd/load.py:60-88)
    np.save(tmp_path / "n32.npy", np.array([[1, -1], [0, 1]], np.int32))
    assert L.load_neighbors(str(tmp_path / "n32.npy")).dtype == np.int64
    np.save(tmp_path / "bad.npy", np.array([[1, -2]], np.int32))
    with pytest.raises(ValueError):
        L.load_neighbors(str(tmp_path / "bad.npy"))
    np.save(tmp_path / "f.npy", np.zeros((2, 2), np.float32))
    with pytest.raises(ValueError):
        L.load_neighbors(str(tmp_path / "f.npy"))
    # ground truth .ibin
    gt = np.arange(12, dtype=np.int32).reshape(3, 4)
    with open(tmp_path / "gt.ibin", "wb") as f:
        f.write(np.array([3, 4], "<i4").tobytes() + gt.tobytes())
    G, n, k = L.load_ibin(str(tmp_path / "gt.ibin"))
    np.testing.assert_array_equal(G, gt)


def test_cli_rejects_bad_arguments():
    exe = os.path.join(ROOT, "gpu-talored-ann_amd", "bin", "gtann")
    if not os.path.exists(exe):
        pytest.skip("CLI not built")
    r = subprocess.run([exe, "bucket2", "--bogus", "1"], capture_output=True, text=True)
    assert r.returncode == 1 and "FATAL: unknown option --bogus" in r.stderr
    r = subprocess.run([exe, "bucket2", "-i", "x.fbin"], capture_output=True, text=True)
    assert r.returncode == 1 and "missing required option --output" in r.stderr
    r = subprocess.run([exe, "optimize_chunked", "-g", "f.bin", "-o", "o.bin", "-m", "A"], capture_output=True,
                       text=True)
    assert r.returncode == 1 and "only method E" in r.stderr
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 1


def _bucket_contents():
    """the bucket files tests/io_driver.cpp writes"""
    boff = np.concatenate([[0], np.cumsum([(b * 3) % 5 for b in range(11)])]).astype(np.uint32)
    bord = np.array([(b * 7) % 11 for b in range(11)], np.int32)
    return boff, bord


@needs_ref
def test_bucket_files_match_reference_bytes(driver, tmp_path):
    _, out = driver
    boff, bord = _bucket_contents()
    O.ref_write_bucket_offsets(tmp_path / "o.bin", boff)
    O.ref_write_bucket_process_order(tmp_path / "p.bin", bord)
    assert _bytes(out / "bucket_offsets.bin") == _bytes(tmp_path / "o.bin")
    assert _bytes(out / "bucket_process_order.bin") == _bytes(tmp_path / "p.bin")
    io.write_bucket_offsets(tmp_path / "o2.bin", boff)
    io.write_bucket_process_order(tmp_path / "p2.bin", bord)
    assert _bytes(tmp_path / "o2.bin") == _bytes(tmp_path / "o.bin")
    assert _bytes(tmp_path / "p2.bin") == _bytes(tmp_path / "p.bin")
    np.testing.assert_array_equal(O.ref_read_bucket_offsets(out / "bucket_offsets.bin"), boff)
    np.testing.assert_array_equal(O.ref_read_bucket_process_order(out / "bucket_process_order.bin"), bord)
    np.testing.assert_array_equal(io.read_bucket_offsets(tmp_path / "o.bin"), boff)
    np.testing.assert_array_equal(io.read_bucket_process_order(tmp_path / "p.bin"), bord)
