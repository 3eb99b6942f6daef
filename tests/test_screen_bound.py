"""The fp16 screen's error bound, checked on the CPU.

The screen (gpu-talored-ann_amd/csrc/screen_kernels.hip) keeps a pool row p
for query q when the fp16 key minus e(q, p) is at most q's threshold; its
lists stay exact only if e bounds the gap between the fp16 key and the fp32
key everywhere.  Here both keys are computed the way the two paths compute
them -- rows scaled by 2^k (k = 15 - E, max |x| < 2^E) and rounded to fp16
(numpy's round-to-nearest-even, as the conversion kernel), float32 sums --
and the gap is compared with the kernel's e, written out again from its
derivation (L2: 2 c |q||p| + 2^-9 (|q| + |p|) + R (|q|^2 + |p|^2) + A; IP:
(c + R) |q||p| + 2^-10 (|q| + |p|) + A, in scaled units, c = 2^-10 + 2^-12,
R = 2^-19, A = 2^-20).  The adversarial rows put every element just below
an fp16 rounding midpoint, so every product's rounding error has the same
sign: the gap then reaches about 2^-10 |q||p|, close to the bound, and a
bound built on half that rounding error (2^-11) fails the test.
"""
import numpy as np
import pytest

C = 2.0 ** -10 + 2.0 ** -12
R = 2.0 ** -19
A = 2.0 ** -20


def _scale(X):
    n2 = np.max(np.einsum("ij,ij->i", X.astype(np.float32), X.astype(np.float32), dtype=np.float32))
    _, E = np.frexp(np.sqrt(np.float32(n2)) * np.float32(1.0000002))
    return 15 - int(E)


def _keys(Q, P, metric, c=C):
    k = _scale(np.vstack([Q, P]))
    s = np.float32(2.0 ** k)
    Qh = (Q * s).astype(np.float16).astype(np.float32)
    Ph = (P * s).astype(np.float16).astype(np.float32)
    d16 = Qh @ Ph.T                                           # float32 sums (any order is within the bound)
    d32 = Q @ P.T                                             # the fp32 path's dot products
    qn = np.einsum("ij,ij->i", Q, Q, dtype=np.float32)
    pn = np.einsum("ij,ij->i", P, P, dtype=np.float32)
    s2 = 4.0 ** k
    if metric == "l2":
        k16 = (qn[:, None].astype(np.float64) * s2 + pn[None, :] * s2 - 2.0 * d16.astype(np.float64))
        k32 = (np.float32(-2.0) * d32 + (pn[None, :] + qn[:, None])).astype(np.float64) * s2
    else:
        k16 = -d16.astype(np.float64)
        k32 = -d32.astype(np.float64) * s2
    qr = np.sqrt(qn.astype(np.float64)) * 2.0 ** k
    pr = np.sqrt(pn.astype(np.float64)) * 2.0 ** k
    if metric == "l2":
        e = 2 * c * qr[:, None] * pr[None, :] + 2.0 ** -9 * (qr[:, None] + pr[None, :]) + \
            R * (qr[:, None] ** 2 + pr[None, :] ** 2) + A
    else:
        e = (c + R) * qr[:, None] * pr[None, :] + 2.0 ** -10 * (qr[:, None] + pr[None, :]) + A
    return np.abs(k16 - k32), e


def _adversarial(n, d, rng):
    # elements just below the midpoint between two fp16 values: every one
    # rounds down by almost half an ulp (2^-11 of itself)
    base = 1.0 + rng.integers(0, 1024, size=(n, d)) / 1024.0            # fp16 values in [1, 2)
    x = base + (2.0 ** -11) * (1.0 - 2.0 ** -8)                           # just under the midpoint
    return (x * 2.0 ** -1).astype(np.float32)                             # max |x| well inside 2^E


DATA = {
    "gauss": lambda rng: rng.standard_normal((300, 128)).astype(np.float32),
    "offset": lambda rng: (500.0 + rng.standard_normal((300, 128))).astype(np.float32),
    "scaled": lambda rng: (rng.standard_normal((300, 64)) *
                           np.exp(rng.uniform(-3.5, 3.5, size=(300, 1)))).astype(np.float32),
    "tiny": lambda rng: (rng.standard_normal((300, 96)) * 1e-9).astype(np.float32),
    "huge": lambda rng: (rng.standard_normal((300, 96)) * 1e12).astype(np.float32),
    "adversarial": lambda rng: _adversarial(300, 160, rng),
}


@pytest.mark.parametrize("kind", sorted(DATA))
@pytest.mark.parametrize("metric", ["l2", "ip"])
def test_fp16_key_within_bound(kind, metric):
    rng = np.random.default_rng(sorted(DATA).index(kind))
    X = DATA[kind](rng)
    if metric == "ip" and kind in ("gauss", "adversarial"):
        X = X / np.linalg.norm(X, axis=1, keepdims=True).astype(np.float32)
    gap, e = _keys(X[:150], X[150:], metric)
    assert np.all(gap <= e), (kind, metric, float(np.max(gap / e)))


def test_bound_is_nearly_tight_on_aligned_rounding():
    # the aligned rounding errors come within a factor 2 of the bound, and a
    # bound on half the rounding error would not hold
    rng = np.random.default_rng(5)
    X = _adversarial(300, 160, rng)
    gap, e = _keys(X[:150], X[150:], "ip")
    assert np.max(gap / e) > 0.5
    gap_half, e_half = _keys(X[:150], X[150:], "ip", c=2.0 ** -11)
    assert np.any(gap_half > e_half)
