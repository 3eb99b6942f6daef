"""Comparison helpers shared by the parity tests."""
import contextlib

import numpy as np


@contextlib.contextmanager
def debug_opts(ctx, **opts):
    """The context's path selection (gt_set_debug) for the duration of a
    block, back to the defaults afterwards."""
    ctx.set_debug(**opts)
    try:
        yield
    finally:
        ctx.set_debug()


def exact_dist(X, q, ids, metric="l2"):
    """float64 distance keys of (q, ids) -- the tie arbiter."""
    X64 = X.astype(np.float64)
    v = X64[ids]
    if metric == "ip":
        return -(v @ X64[q])
    return ((v - X64[q]) ** 2).sum(axis=1)


def assert_knn_equal(ids, d, ref_ids, ref_d):
    """Bit-exact: integer-valued data, every distance exact."""
    np.testing.assert_array_equal(ids, ref_ids)
    np.testing.assert_array_equal(d.view(np.uint32), ref_d.view(np.uint32))


FLOOR_STATS = {"positions": 0, "floor_decided": 0, "rows": 0, "rows_floor_decided": 0}
# largest error seen per (metric, D), in ulps of the operand magnitude (the
# calibration of FLOOR_ULPS; printed at the end of a session that saw any)
ERR_ULPS_MAX = {}

# The absolute floor per (metric, D), in ulps of the operand magnitude
# (|q|^2 + |p|^2 for L2, 2 |q| |p| for the inner product): twice the largest
# error measured on the float tests' data (the GPU suite prints the maxima at
# the end: L2 D = 96 11.3, D = 128 13.7, D = 960 5.9; IP D = 96 5.0, D = 960
# 3.0; D > 256 sums per 32-dimension chunk, hence the smaller error).  A
# (metric, D) without a measurement has no floor: calibrate it first.
FLOOR_ULPS = {("l2", 96): 23.0, ("l2", 128): 28.0, ("l2", 960): 12.0, ("ip", 96): 10.0, ("ip", 960): 6.0}


def floor_report(reset=True):
    """FLOOR_STATS as fractions (and reset it)."""
    s = dict(FLOOR_STATS)
    if reset:
        for k in FLOOR_STATS:
            FLOOR_STATS[k] = 0
    return {"positions": s["positions"], "rows": s["rows"],
            "positions_floor_decided": s["floor_decided"] / max(s["positions"], 1),
            "rows_floor_decided": s["rows_floor_decided"] / max(s["rows"], 1)}


def assert_knn_close(X, queries, ids, d, ref_ids, ref_d, rtol=1e-5, metric="l2"):
    """Float data: distances within rtol relative (positionwise, both lists are
    sorted), ids identical except where the reference's distance at that
    position is tied within rtol by the GPU's id (checked in float64).

    The absolute floor covers the cancellation of |q|^2 + |p|^2 - 2q.p in fp32
    (the reference's own formula: cuBLAS L2Expanded, src/bucket.cu:4603-4687):
    FLOOR_ULPS[(metric, D)] ulps of the operand magnitude |q|^2 + |p|^2 (2|q||p|
    for the inner product), twice the largest error measured for that D, which
    for clustered data is what bounds the error of small distances.  Returns
    the number of id mismatches (all of them ties); FLOOR_STATS counts the
    positions checked and those whose error exceeds rtol relative, i.e. where
    the floor, not the relative bound, decided."""
    X64 = X.astype(np.float64)
    n2 = (X64 ** 2).sum(axis=1)
    nmis = 0
    for r in range(ids.shape[0]):
        q = int(queries[r])
        valid = ref_ids[r] >= 0
        assert ((ids[r] >= 0) == valid).all(), f"row {r}: padding differs"
        k = int(valid.sum())
        key = (metric, int(X.shape[1]))
        assert key in FLOOR_ULPS, f"no measured float floor for {key}: calibrate FLOOR_ULPS first"
        ulps = FLOOR_ULPS[key]
        if metric == "ip":
            scale = np.sqrt(n2[q] * n2[np.maximum(ref_ids[r, :k], 0)]) * 2.0 ** -24 * 2 * ulps
        else:
            scale = (n2[q] + n2[np.maximum(ref_ids[r, :k], 0)]) * 2.0 ** -24 * ulps
        tol = rtol * np.abs(ref_d[r, :k]) + scale
        diff = np.abs(d[r, :k].astype(np.float64) - ref_d[r, :k].astype(np.float64))
        if k:
            ERR_ULPS_MAX[key] = max(ERR_ULPS_MAX.get(key, 0.0), float((diff / (scale / ulps)).max()))
        assert (diff <= tol).all(), f"row {r}: distance off by {diff.max()} (tol {tol[diff.argmax()]})"
        beyond = int((diff > rtol * np.abs(ref_d[r, :k])).sum())
        FLOOR_STATS["positions"] += k
        FLOOR_STATS["floor_decided"] += beyond
        FLOOR_STATS["rows"] += 1
        FLOOR_STATS["rows_floor_decided"] += int(beyond > 0)
        mis = np.nonzero(ids[r, :k] != ref_ids[r, :k])[0]
        if len(mis):
            nmis += len(mis)
            true = exact_dist(X, q, ids[r, mis], metric)
            refd = exact_dist(X, q, ref_ids[r, mis], metric)
            t2 = rtol * np.abs(refd) + scale[mis]
            assert (np.abs(true - refd) <= t2).all(), f"row {r}: id mismatch beyond ties at {mis}"
        assert len(set(ids[r, :k].tolist())) == k, f"row {r}: duplicate ids"
    return nmis


def bucketed_graph(rng, N, nb, M, W, outside=0.3, pad=0.0):
    """A candidate table in a bucket-contiguous id space (the layout of the
    windowed prune): nb buckets of random sizes, each row's candidates drawn
    mostly from its own bucket and a few others, some padding (-1) and
    repeated ids; per bucket position a window of itself plus up to W - 1
    random positions.  Returns (G int32 (N, M), offsets uint32 (nb + 1),
    win int32 (nb, W), win_len int32 (nb,))."""
    cuts = np.sort(rng.choice(np.arange(1, N), nb - 1, replace=False))
    off = np.concatenate([[0], cuts, [N]]).astype(np.uint32)
    pos = np.searchsorted(off, np.arange(N), side="right") - 1
    G = np.empty((N, M), np.int32)
    for a in range(N):
        lo, hi = int(off[pos[a]]), int(off[pos[a] + 1])
        own = rng.integers(lo, hi, M)
        far = rng.integers(0, N, M)
        row = np.where(rng.random(M) < outside, far, own)
        row[row == a] = (a + 1) % N
        G[a] = row
    if pad:
        G[rng.random((N, M)) < pad] = -1
    win = np.zeros((nb, W), np.int32)
    wl = np.zeros(nb, np.int32)
    for p in range(nb):
        ws = [p] + [int(q) for q in rng.integers(0, nb, W - 1) if q != p]
        ws = sorted(set(ws))[:W]
        win[p, :len(ws)] = ws
        wl[p] = len(ws)
    return G, off, win, wl
