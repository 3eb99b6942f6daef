"""Dataset and index loaders with the interface of bd/load.py.

Same names, return values and errors as the reference's Python loaders, so
that scripts written against them run unchanged:

* ``load_bigann_to_f32`` (bd/load.py:15-41): ``.fbin``/``.bin`` as float32,
  ``.u8bin`` and ``.i8bin`` read as uint8 and cast to float32 -- the Python
  pipeline's own reading (the C++ pipeline, and ``gtann_io.read_dataset``,
  read ``.i8bin`` as signed int8);
* ``load_ibin`` (bd/load.py:43-58), ``load_neighbors`` (bd/load.py:60-88),
  ``load_bigann_bin`` (bd/load.py:94-137, ``.fbin``/``.ibin``/``.u8bin`` to a
  float32 torch tensor), ``save_npy``.

``load_dataset`` is this build's addition: the stored element type, for the
GPU entry points (the device converts).
"""
from __future__ import annotations

import os
from typing import Tuple

import numpy as np

import gtann_io


def get_ext(path: str) -> str:
    return os.path.splitext(path)[1].lower()


def _header(path: str) -> Tuple[int, int]:
    with open(path, "rb") as f:
        head = f.read(8)
    if len(head) < 8:
        raise ValueError(f"File too small: {path}")
    N, D = np.frombuffer(head, dtype="<i4")
    return int(N), int(D)


def load_bigann_to_f32(path: str) -> Tuple[np.ndarray, int, int]:
    ext = get_ext(path)
    N, D = _header(path)
    if ext in (".fbin", ".bin"):
        dt = np.float32
    elif ext in (".u8bin", ".i8bin"):
        dt = np.uint8
    else:
        raise ValueError(f"Unsupported data ext: {ext}")
    raw = np.fromfile(path, dtype=dt, count=N * D, offset=8)
    if raw.size != N * D:
        raise ValueError("Size mismatch for fbin" if dt == np.float32 else "Size mismatch for u8bin/i8bin")
    return raw.reshape(N, D).astype(np.float32, copy=False), N, D


def load_dataset(path: str) -> np.ndarray:
    """(N, D) in the stored element type: float32, uint8 or signed int8."""
    return gtann_io.read_dataset(path)


def load_ibin(path: str) -> Tuple[np.ndarray, int, int]:
    N, D = _header(path)
    G = np.fromfile(path, dtype=np.int32, count=N * D, offset=8)
    if G.size != N * D:
        raise ValueError("Size mismatch for ibin")
    return G.reshape(N, D), N, D


def load_neighbors(path: str) -> np.ndarray:
    idx = np.load(path)   # allow_pickle stays False
    if idx.ndim != 2:
        raise ValueError(f"Expected 2D neighbors matrix, got shape={idx.shape}")
    if not np.issubdtype(idx.dtype, np.integer):
        raise ValueError(f"neighbors must be integer dtype, got {idx.dtype}")
    if idx.dtype != np.int64:
        if np.any(idx < -1):
            raise ValueError("neighbors matrix contains invalid negative ids (< -1), or out of uint64 range")
        idx = idx.astype(np.int64, copy=False)
    return idx


def load_bigann_bin(path: str):
    import torch
    ext = get_ext(path)
    dt = {".fbin": np.float32, ".ibin": np.int32, ".u8bin": np.uint8}.get(ext)
    if dt is None:
        raise ValueError(f"Unsupported extension: {ext}")
    N, D = _header(path)
    expected = N * D * np.dtype(dt).itemsize
    got = os.path.getsize(path) - 8
    if got != expected:
        raise ValueError(f"Data size mismatch: expect {expected} bytes for N={N},D={D}, got {got}.")
    arr = np.fromfile(path, dtype=dt, count=N * D, offset=8).reshape(N, D)
    return torch.from_numpy(arr.astype(np.float32))


def save_npy(path: str, arr: np.ndarray):
    d = os.path.dirname(path)
    if d:
        os.makedirs(d, exist_ok=True)
    np.save(path, arr)
