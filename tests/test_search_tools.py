"""Host-side parts of the search entry point (CPU): the recall and set-wise
comparison of bd/search.py:95-127 and :193-262 in the Python mirror and in
the `gtann compare` subcommand, against hand-computed values."""
import os
import subprocess

import numpy as np
import pytest

import search

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "gpu-talored-ann_amd", "bin", "gtann")


def test_recall_vs_gt_known_values():
    pred = np.array([[1, 2, 3], [7, 8, -1], [4, 5, 6]])
    gt = np.array([[1, 9, 3, 0], [9, 7, 2, 2], [0, 1, 2, 3]], np.int32)
    r_first, r_any, recall = search.recall_vs_gt(pred, gt, 3)
    # row 0: gt0=1 in pred; overlap {1,3} of gt[:3]={1,9,3} -> 2/3
    # row 1: gt0=9 not in pred; any: 7; overlap {7} of {9,7,2} -> 1/3
    # row 2: nothing
    assert r_first == pytest.approx(1 / 3)
    assert r_any == pytest.approx(2 / 3)
    assert recall == pytest.approx((2 / 3 + 1 / 3 + 0) / 3)


def _write_npy(path, a):
    np.save(path, a)


def test_compare_known_values(tmp_path, capsys):
    A = np.array([[1, 2, 3], [4, 5, -1], [7, 8, 9]], np.int64)
    B = np.array([[3, 2, 1, 0], [4, 6, 5, 5], [0, 0, 0, 0]], np.int64)
    _write_npy(tmp_path / "a.npy", A)
    _write_npy(tmp_path / "b.npy", B)
    r = search.compare_indices_setwise(str(tmp_path / "a.npy"), str(tmp_path / "b.npy"),
                                       save_csv=str(tmp_path / "o.csv"))
    # k = 3: row0 {1,2,3}={3,2,1} -> 3 equal; row1 {4,5} vs {4,6,5} -> 2; row2 {7,8,9} vs {0} -> 0
    assert r["k"] == 3
    assert r["mean_overlap"] == pytest.approx((1 + 2 / 3 + 0) / 3)
    assert r["hits_any"] == pytest.approx(2 / 3)
    assert r["set_equal"] == pytest.approx(1 / 3)
    csv = (tmp_path / "o.csv").read_text().splitlines()
    assert csv[0] == "node,intersect_size,deg_A,deg_B,overlap"
    assert csv[2] == "1,2,2,3,0.666667"


@pytest.mark.skipif(not os.path.exists(EXE), reason="gtann CLI not built")
def test_cli_compare_matches_mirror(tmp_path):
    rng = np.random.default_rng(0)
    A = rng.integers(-1, 50, size=(500, 16)).astype(np.int64)
    B = np.where(rng.random((500, 16)) < 0.7, A, rng.integers(-1, 50, size=(500, 16)))
    np.save(tmp_path / "a.npy", A)
    np.save(tmp_path / "b.npy", B.astype(np.int32))   # int32 index files are read too
    r = subprocess.run([EXE, "compare", "--index1", str(tmp_path / "a.npy"), "--index2", str(tmp_path / "b.npy"),
                        "--k-cmp", "10", "--save-csv", str(tmp_path / "c.csv")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    vals = {ln.split(":")[0].split("@")[0].strip(): float(ln.split(":")[-1])
            for ln in r.stdout.splitlines() if "@10" in ln}
    m = search.compare_indices_setwise(str(tmp_path / "a.npy"), str(tmp_path / "b.npy"), k_cmp=10,
                                       save_csv=str(tmp_path / "p.csv"))
    assert vals["MeanOverlap"] == pytest.approx(m["mean_overlap"], abs=2e-6)
    assert vals["HitsAny"] == pytest.approx(m["hits_any"], abs=2e-6)
    assert vals["SetEqual"] == pytest.approx(m["set_equal"], abs=2e-6)
    # per-node rows agree (the C++ CSV counts distinct ids, as the reference's sets do)
    assert (tmp_path / "c.csv").read_text() == (tmp_path / "p.csv").read_text()


@pytest.mark.skipif(not os.path.exists(EXE), reason="gtann CLI not built")
def test_cli_search_rejects_bad_options(tmp_path):
    r = subprocess.run([EXE, "search", "--bogus", "1"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "unknown option" in r.stderr


def test_vectorised_metrics_equal_per_row_set_definitions():
    # rows with -1 padding and repeated ids on both sides
    rng = np.random.default_rng(8)
    pred = rng.integers(-1, 40, size=(500, 10))
    gt = rng.integers(-1, 40, size=(500, 25))
    r_first, r_any, rec = search.recall_vs_gt(pred, gt, 10)
    k = 10
    first = np.mean([gt[i, 0] in pred[i].tolist() for i in range(500)])
    anyh = np.mean([len(set(pred[i].tolist()) & set(gt[i].tolist())) > 0 for i in range(500)])
    ov = np.mean([len({v for v in pred[i, :k] if v >= 0} & {v for v in gt[i, :k] if v >= 0}) / k
                  for i in range(500)])
    assert (r_first, r_any) == (first, anyh)
    assert abs(rec - ov) < 1e-12
    inter, na, nb = search._set_sizes(pred, gt)
    for i in range(500):
        A = {v for v in pred[i] if v >= 0}
        B = {v for v in gt[i] if v >= 0}
        assert (inter[i], na[i], nb[i]) == (len(A & B), len(A), len(B))
