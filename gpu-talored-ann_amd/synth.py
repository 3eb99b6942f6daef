"""Seeded synthetic datasets of the five benchmark configurations.

Each configuration is a Gaussian mixture drawn with numpy's PCG64 from a
fixed seed, so the same bytes come out on every machine with this image.
Parameters the benchmark description leaves open are fixed here:

  C1  10,000 x 128 fp32, 64 centres U[-10,10]^128, sigma 1, L2, 16 buckets, 64 -> 32
  C2  1,000,000 x 128 fp32 integer-valued, 1,000 centres U[0,255]^128, sigma 20,
      rounded and clipped to [0,255], L2, 256 buckets, 64 -> 32 (+10,000 held-out queries)
  C3  1,000,000 x 96 fp32, 500 centres N(0, I), sigma 0.3 (relative to unit-norm
      centres: centres are normalised first), rows L2-normalised, IP, 256 buckets, 64 -> 32
  C4  1,000,000 x 960 fp32, 200 centres U[0,1]^960, sigma 0.1, L2, 512 buckets, 96 -> 48
  C5  10,000,000 x 128 int8, 4,096 centres U[-100,100]^128, sigma 15, rounded and
      clipped to [-127,127], L2, 2,048 buckets, 64 -> 32
  S2  the search workload: 1,000,000 x 128 fp32 integer-valued, a 16-dimensional
      latent Gaussian (sd 24 per latent axis) through a random orthonormal
      128 x 16 map, plus N(0, 2^2) noise, centred at 128, rounded and clipped
      to [0,255]; L2, 256 buckets, 64 -> 32.  The C configurations are
      mixtures of well separated clusters, so any kNN-derived graph of them
      splits into one component per cluster and a search from random entry
      points only reaches its query's cluster by chance; S2 has the low
      intrinsic dimension and the connected graph of real descriptor sets.

Points are assigned to clusters uniformly at random.  `n` scales a
configuration down (same recipe, first `n` points of the stream) for tests.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

BASE_SEED = 42


@dataclass(frozen=True)
class Config:
    name: str
    n: int
    dim: int
    metric: str
    buckets: int
    M: int
    K: int
    dtype: str


CONFIGS = {
    "C1": Config("C1", 10_000, 128, "l2", 16, 64, 32, "f32"),
    "C2": Config("C2", 1_000_000, 128, "l2", 256, 64, 32, "f32"),
    "C3": Config("C3", 1_000_000, 96, "ip", 256, 64, 32, "f32"),
    "C4": Config("C4", 1_000_000, 960, "l2", 512, 96, 48, "f32"),
    "C5": Config("C5", 10_000_000, 128, "l2", 2048, 64, 32, "i8"),
    "S2": Config("S2", 1_000_000, 128, "l2", 256, 64, 32, "f32"),
}


def _rng(cfg: str, stream: int = 0):
    return np.random.default_rng([BASE_SEED, int(cfg[1:]), stream])


def _mixture(rng, n, centres, sigma, chunk=1 << 18):
    k, dim = centres.shape
    out = np.empty((n, dim), np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        lab = rng.integers(0, k, size=e - s)
        out[s:e] = centres[lab] + sigma * rng.standard_normal((e - s, dim), dtype=np.float32)
    return out


def generate(cfg: str, n: int | None = None, queries: int = 0):
    """Returns (X, Q): base points and `queries` held-out points of the same mixture."""
    c = CONFIGS[cfg]
    n = c.n if n is None else n
    rng = _rng(cfg, 0)
    if cfg == "C1":
        centres = rng.uniform(-10, 10, size=(64, c.dim)).astype(np.float32)
        X = _mixture(rng, n + queries, centres, 1.0)
    elif cfg == "C2":
        centres = rng.uniform(0, 255, size=(1000, c.dim)).astype(np.float32)
        X = np.clip(np.rint(_mixture(rng, n + queries, centres, 20.0)), 0, 255).astype(np.float32)
    elif cfg == "C3":
        centres = rng.standard_normal((500, c.dim)).astype(np.float32)
        centres /= np.linalg.norm(centres, axis=1, keepdims=True)
        X = _mixture(rng, n + queries, centres, 0.3 / np.sqrt(c.dim))
        X /= np.linalg.norm(X, axis=1, keepdims=True)
        X = X.astype(np.float32)
    elif cfg == "C4":
        centres = rng.uniform(0, 1, size=(200, c.dim)).astype(np.float32)
        X = _mixture(rng, n + queries, centres, 0.1)
    elif cfg == "S2":
        basis, _ = np.linalg.qr(rng.standard_normal((c.dim, 16)))
        basis = basis.astype(np.float32)
        X = np.empty((n + queries, c.dim), np.float32)
        for s in range(0, n + queries, 1 << 18):
            e = min(n + queries, s + (1 << 18))
            z = 24.0 * rng.standard_normal((e - s, 16), dtype=np.float32)
            X[s:e] = 128.0 + z @ basis.T + 2.0 * rng.standard_normal((e - s, c.dim), dtype=np.float32)
        X = np.clip(np.rint(X), 0, 255).astype(np.float32)
    elif cfg == "C5":
        centres = rng.uniform(-100, 100, size=(4096, c.dim)).astype(np.float32)
        X = np.clip(np.rint(_mixture(rng, n + queries, centres, 15.0)), -127, 127).astype(np.int8)
    else:
        raise KeyError(cfg)
    return X[:n], X[n:]
