"""Writes tests/golden/pyref_golden.npz from the reference's own Python
functions, imported in the build container only (the reference never
travels to the GPU box; the fixtures are data):

  * bd/prune.py:8-83 `prune_graph` (occlusion prune);
  * bd/build_bucket.py:473-543 `_apply_reverse_edges` (reverse-edge insertion).

Inputs are chosen so that the parts of the reference that no restatement
can pin (numpy argsort / torch.topk order among equal keys, float32
summation order) cannot decide any output:

  * occlusion prune, integer case: integer coordinates with D * 1000^2 < 2^24,
    so every distance is exact in float32 in any summation order; a point's
    candidate distances are distinct (argsort order unique); equalities
    d(u, z) == d(v, z) are kept on purpose -- they pin the strict `<`;
  * occlusion prune, float case: non-integer coordinates, and every
    comparison the prune makes (candidate order and each d(u, z) against
    d(v, z)) is at least 1e-3 relative away from a tie;
  * reverse-edge insertion: tables with globally distinct finite distances
    (so torch.topk has no ties to order), rows without repeated ids, some
    rows padded with (-1, +inf).

Run (needs /root/reference):

    python tests/golden/make_golden_py.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_BD = os.environ.get("GTANN_REF_BD", "/root/reference/bucketDemo")


def _sqd(X, i, j):
    t = X[i].astype(np.float64) - X[j].astype(np.float64)
    return float(t @ t)


def _drop_float_near_ties(X, nb, eps):
    """A candidate z becomes -1 unless, against every candidate u kept
    before it, |d(v,z) - d(v,u)|, |d(u,z) - d(v,z)| and |d(z,u) - d(v,u)|
    all exceed eps relative (float64): no decision of the prune is then
    within eps of a tie."""
    N = X.shape[0]
    nb = nb.copy()
    for v in range(N):
        kept = []
        for k in range(nb.shape[1]):
            z = int(nb[v, k])
            if not (0 <= z < N) or z == v:
                continue
            dvz = _sqd(X, v, z)
            ok = True
            for u in kept:
                dvu = _sqd(X, v, u)
                duz = _sqd(X, u, z)
                if (abs(dvz - dvu) <= eps * max(dvz, dvu) or abs(duz - dvz) <= eps * dvz
                        or abs(duz - dvu) <= eps * dvu):
                    ok = False
                    break
            if ok:
                kept.append(z)
            else:
                nb[v, k] = -1
    return nb


def _drop_tied_candidates(X, nb):
    """A candidate whose distance to the point equals an earlier candidate's
    becomes -1, so every point's candidate distances are distinct."""
    N = X.shape[0]
    nb = nb.copy()
    for v in range(N):
        seen = set()
        for k in range(nb.shape[1]):
            z = int(nb[v, k])
            if not (0 <= z < N) or z == v:
                continue
            dz = _sqd(X, v, z)
            if dz in seen:
                nb[v, k] = -1
            seen.add(dz)
    return nb


def prune_cases(rng):
    cases = []
    # integer coordinates: exact distances, distinct per point, equalities in d(u,z) vs d(v,z) allowed
    for (N, D, M, lo, hi, maxdeg, pad, self_loops) in [(40, 4, 8, 0, 40, 0, 0.0, False),
                                                       (120, 8, 16, 0, 1000, 6, 0.05, True),
                                                       (200, 3, 24, -30, 30, 10, 0.1, True),
                                                       (64, 16, 64, 0, 255, 0, 0.0, False)]:
        X = rng.integers(lo, hi + 1, size=(N, D)).astype(np.float32)
        nb = np.stack([rng.permutation(N)[:M] for _ in range(N)]).astype(np.int64)
        if not self_loops:
            for v in range(N):
                nb[v][nb[v] == v] = -1
        if pad:
            nb[rng.random((N, M)) < pad] = -1
        nb = _drop_tied_candidates(X, nb)
        cases.append(("int", X, nb, maxdeg))
    # candidates = each point's exact 24 nearest (distinct distances first):
    # coarse 2-D integer grid, where d(u, z) == d(v, z) happens often
    N, M = 300, 24
    X = rng.integers(0, 21, size=(N, 2)).astype(np.float32)
    X64 = X.astype(np.float64)
    dd = ((X64[:, None, :] - X64[None, :, :]) ** 2).sum(-1)
    np.fill_diagonal(dd, np.inf)
    nb = np.argsort(dd, axis=1, kind="stable")[:, :M].astype(np.int64)
    cases.append(("int", X, _drop_tied_candidates(X, nb), 0))
    # float coordinates with a clear margin on every decision
    for (N, D, M, maxdeg) in [(60, 8, 12, 0), (100, 16, 20, 8)]:
        X = (rng.standard_normal((N, D)) * 3.0).astype(np.float32)
        nb = np.stack([rng.permutation(np.delete(np.arange(N), v))[:M] for v in range(N)]).astype(np.int64)
        nb = _drop_float_near_ties(X, nb, 1e-3)
        cases.append(("float", X, nb, maxdeg))
    return cases


def reverse_cases(rng):
    cases = []
    for (N, m, pad_rows) in [(30, 4, 0.0), (200, 16, 0.1), (500, 32, 0.05), (100, 64, 0.2)]:
        ids = np.stack([rng.permutation(np.delete(np.arange(N), a))[:m] for a in range(N)]).astype(np.int64)
        # globally distinct finite distances, each row ascending
        vals = rng.permutation(N * m * 8)[:N * m].astype(np.float64) * 0.25 + 1.0
        d = np.sort(vals.reshape(N, m), axis=1).astype(np.float32)
        assert len(np.unique(d)) == d.size
        for a in np.nonzero(rng.random(N) < pad_rows)[0]:
            k = int(rng.integers(1, m))   # keep k entries, pad the rest
            ids[a, k:] = -1
            d[a, k:] = np.inf
        cases.append((ids, d, m))
    return cases


def main():
    if not os.path.isdir(REF_BD):
        sys.exit(f"reference tree not found at {REF_BD}")
    sys.path.insert(0, REF_BD)
    import torch
    from prune import prune_graph              # bd/prune.py:8
    from build_bucket import _apply_reverse_edges   # bd/build_bucket.py:473

    rng = np.random.default_rng(20261202)
    out = {}
    for c, (kind, X, nb, maxdeg) in enumerate(prune_cases(rng)):
        res = prune_graph(X, nb, maxdeg if maxdeg > 0 else None)
        out[f"occ{c}_kind"] = np.array(kind)
        out[f"occ{c}_X"] = X
        out[f"occ{c}_nb"] = nb
        out[f"occ{c}_maxdeg"] = np.int32(maxdeg)
        out[f"occ{c}_out"] = np.asarray(res, np.int64)
    for c, (ids, d, m) in enumerate(reverse_cases(rng)):
        ti = torch.from_numpy(ids.copy())
        td = torch.from_numpy(d.copy())
        _apply_reverse_edges(ti, td, m)
        out[f"rin{c}_ids"] = ids.astype(np.int32)
        out[f"rin{c}_d"] = d
        out[f"rin{c}_out_ids"] = ti.numpy().astype(np.int32)
        out[f"rin{c}_out_d"] = td.numpy().astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "pyref_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "pyref_golden.npz"))


if __name__ == "__main__":
    main()
