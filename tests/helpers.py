"""Comparison helpers shared by the parity tests."""
import numpy as np


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


def assert_knn_close(X, queries, ids, d, ref_ids, ref_d, rtol=1e-5, metric="l2"):
    """Float data: distances within rtol relative (positionwise, both lists are
    sorted), ids identical except where the reference's distance at that
    position is tied within rtol by the GPU's id (checked in float64).

    The absolute floor covers the cancellation of |q|^2 + |p|^2 - 2q.p in fp32:
    a few ulps of the operand magnitude |q|^2 + |p|^2, which for clustered data
    is what bounds the error of small distances."""
    X64 = X.astype(np.float64)
    n2 = (X64 ** 2).sum(axis=1)
    nmis = 0
    for r in range(ids.shape[0]):
        q = int(queries[r])
        valid = ref_ids[r] >= 0
        assert ((ids[r] >= 0) == valid).all(), f"row {r}: padding differs"
        k = int(valid.sum())
        if metric == "ip":
            scale = np.sqrt(n2[q] * n2[np.maximum(ref_ids[r, :k], 0)]) * 2.0 ** -20
        else:
            scale = (n2[q] + n2[np.maximum(ref_ids[r, :k], 0)]) * 2.0 ** -21
        tol = rtol * np.abs(ref_d[r, :k]) + scale
        diff = np.abs(d[r, :k].astype(np.float64) - ref_d[r, :k].astype(np.float64))
        assert (diff <= tol).all(), f"row {r}: distance off by {diff.max()} (tol {tol[diff.argmax()]})"
        mis = np.nonzero(ids[r, :k] != ref_ids[r, :k])[0]
        if len(mis):
            nmis += len(mis)
            true = exact_dist(X, q, ids[r, mis], metric)
            refd = exact_dist(X, q, ref_ids[r, mis], metric)
            t2 = rtol * np.abs(refd) + scale[mis]
            assert (np.abs(true - refd) <= t2).all(), f"row {r}: id mismatch beyond ties at {mis}"
        assert len(set(ids[r, :k].tolist())) == k, f"row {r}: duplicate ids"
    return nmis
