"""Readers and writers of the pipeline's on-disk files (numpy).

Byte layouts, identical with the reference's files:

* dataset ``.fbin``/``.bin`` float32, ``.u8bin`` uint8, ``.i8bin`` int8:
  ``int32 N, int32 D`` then N*D elements (src/load.hpp:67-117).
  ``read_dataset`` returns the stored element type (int8 signed, as the C++
  pipeline reads it); ``load.load_bigann_to_f32`` keeps the Python pipeline's
  own reading of ``.i8bin`` as uint8 (bd/load.py:34-38).
* ``vector_knn.bin``: ``int64 N, int32 M, int32[N*M]``, -1 padding
  (src/graph_io.hpp:26-30, 286-329).
* ``vector_dists.bin``: ``int64 N, int32 M, float32[N*M]`` (src/bucket.cu:5563-5573).
* graphs (forward, cagra, ``final_graph.bin``): ``int64 N, int32 K, uint32[N*K]``
  (src/graph_io.hpp:8-11, 50-96).
* ``inverse_perm.bin``: raw ``uint32[N]`` (src/graph_io.hpp:369-377).
* ground truth ``.ibin``: ``int32 N, int32 K, int32[N*K]`` (bd/load.py:43-58).
* ``bucket_offsets.bin``: ``int32 n_buckets, uint32[n_buckets+1]`` and
  ``bucket_process_order.bin``: ``int32 n, int32[n]`` (src/graph_io.hpp:178-244);
  ``centroid_knn.bin`` / ``centroid_pool.bin`` use the graph layout.
* ``bucket_index.bin``: ``int64 n_buckets, int64 N``, then per bucket a
  packed ``int64 byte offset, int32 count``; ``bucket_data.bin``: the int32
  point ids of each bucket in turn; ``centroid_global_indices.bin``:
  ``int64 n, int64[n]`` (src/bucket.cu:3434-3510, 9561-9568).
"""
from __future__ import annotations

import os
import struct

import numpy as np

_DATASET_DTYPES = {".fbin": np.float32, ".bin": np.float32, ".u8bin": np.uint8, ".i8bin": np.int8}


def dataset_dtype(path: str):
    ext = os.path.splitext(path)[1].lower()
    if ext not in _DATASET_DTYPES:
        raise ValueError(f"unsupported dataset extension {ext!r} (.fbin/.bin/.u8bin/.i8bin)")
    return _DATASET_DTYPES[ext]


def _read_header(f, fmt, path):
    raw = f.read(struct.calcsize(fmt))
    if len(raw) < struct.calcsize(fmt):
        raise ValueError(f"file too small for its header: {path}")
    return struct.unpack("<" + fmt, raw)


def read_dataset(path: str, mmap: bool = False) -> np.ndarray:
    """(N, D) array in the file's own element type."""
    dt = np.dtype(dataset_dtype(path))
    with open(path, "rb") as f:
        N, D = _read_header(f, "ii", path)
    if N <= 0 or D <= 0:
        raise ValueError(f"bad header (N={N}, D={D}): {path}")
    need = 8 + N * D * dt.itemsize
    if os.path.getsize(path) < need:
        raise ValueError(f"size mismatch: {path} holds {os.path.getsize(path)} bytes, header needs {need}")
    if mmap:
        return np.memmap(path, dtype=dt, mode="r", offset=8, shape=(N, D))
    with open(path, "rb") as f:
        f.seek(8)
        return np.fromfile(f, dtype=dt, count=N * D).reshape(N, D)


def write_dataset(path: str, X: np.ndarray) -> None:
    dt = np.dtype(dataset_dtype(path))
    X = np.ascontiguousarray(X)
    if X.dtype != dt:
        raise ValueError(f"{path} stores {dt}, array is {X.dtype}")
    N, D = X.shape
    with open(path, "wb") as f:
        f.write(struct.pack("<ii", N, D))
        X.tofile(f)


def _read_table(path: str, dtype) -> np.ndarray:
    with open(path, "rb") as f:
        N, W = _read_header(f, "qi", path)
        if N <= 0 or W <= 0:
            raise ValueError(f"bad header (N={N}, width={W}): {path}")
        a = np.fromfile(f, dtype=dtype, count=N * W)
    if a.size != N * W:
        raise ValueError(f"short payload: {path}")
    return a.reshape(N, W)


def _write_table(path: str, a: np.ndarray, dtype) -> None:
    a = np.ascontiguousarray(a, dtype=dtype)
    if a.ndim != 2:
        raise ValueError("table must be 2-D")
    with open(path, "wb") as f:
        f.write(struct.pack("<qi", a.shape[0], a.shape[1]))
        a.tofile(f)


def read_vector_knn(path: str) -> np.ndarray:
    return _read_table(path, np.int32)


def write_vector_knn(path: str, ids: np.ndarray) -> None:
    _write_table(path, ids, np.int32)


def read_vector_dists(path: str) -> np.ndarray:
    return _read_table(path, np.float32)


def write_vector_dists(path: str, d: np.ndarray) -> None:
    _write_table(path, d, np.float32)


def read_graph(path: str) -> np.ndarray:
    return _read_table(path, np.uint32)


def write_graph(path: str, g: np.ndarray) -> None:
    _write_table(path, g, np.uint32)


def read_inverse_perm(path: str) -> np.ndarray:
    if os.path.getsize(path) % 4:
        raise ValueError(f"size is not a multiple of 4: {path}")
    return np.fromfile(path, dtype=np.uint32)


def write_inverse_perm(path: str, p: np.ndarray) -> None:
    np.ascontiguousarray(p, dtype=np.uint32).tofile(path)


def read_ibin(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        N, K = _read_header(f, "ii", path)
        a = np.fromfile(f, dtype=np.int32, count=N * K)
    if a.size != N * K:
        raise ValueError(f"size mismatch for ibin: {path}")
    return a.reshape(N, K)


def write_bucket_offsets(path: str, off: np.ndarray) -> None:
    off = np.ascontiguousarray(off, dtype=np.uint32)
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(off) - 1))
        off.tofile(f)


def read_bucket_offsets(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        (n,) = _read_header(f, "i", path)
        if n <= 0:
            raise ValueError(f"bad bucket-offsets header: {path}")
        a = np.fromfile(f, dtype=np.uint32, count=n + 1)
    if a.size != n + 1:
        raise ValueError(f"short payload: {path}")
    return a


def write_bucket_process_order(path: str, order: np.ndarray) -> None:
    order = np.ascontiguousarray(order, dtype=np.int32)
    with open(path, "wb") as f:
        f.write(struct.pack("<i", len(order)))
        order.tofile(f)


def read_bucket_process_order(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        (n,) = _read_header(f, "i", path)
        if n <= 0:
            raise ValueError(f"bad bucket-process-order header: {path}")
        a = np.fromfile(f, dtype=np.int32, count=n)
    if a.size != n:
        raise ValueError(f"short payload: {path}")
    return a


def read_bucket_files(index_path: str, data_path: str):
    """(records, buckets): the (offset, count) records of bucket_index.bin and
    the int32 ids of every bucket from bucket_data.bin."""
    with open(index_path, "rb") as f:
        nb, n = struct.unpack("<qq", f.read(16))
        rec = np.frombuffer(f.read(12 * nb), dtype=[("off", "<i8"), ("count", "<i4")])
    if len(rec) != nb:
        raise ValueError(f"{index_path}: truncated index")
    data = np.fromfile(data_path, dtype="<i4")
    return rec, [data[o // 4:o // 4 + c] for o, c in zip(rec["off"].tolist(), rec["count"].tolist())]


def read_centroid_indices(path: str) -> np.ndarray:
    with open(path, "rb") as f:
        (n,) = struct.unpack("<q", f.read(8))
        v = np.frombuffer(f.read(8 * n), dtype="<i8")
    if len(v) != n:
        raise ValueError(f"{path}: truncated")
    return v.astype(np.int64)
