"""ctypes binding of libgtann.so (include/gtann.h) -- the gfx950 graph build.

Arrays may be numpy arrays (host memory) or torch tensors (host or device
memory of the context's GPU); device tensors are used in place by the
library.  Every call goes to the HIP library; there is no CPU fallback, and
a missing library raises immediately.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libgtann.so")

GT_OK, GT_EINVAL, GT_ENOMEM, GT_EDEVICE, GT_EFEWCAND = 0, -1, -2, -3, -4
DTYPES = {"f32": 0, "u8": 1, "i8": 2}
METRICS = {"l2": 0, "ip": 1}

# symbols the C ABI must export (checked by the CPU tests)
EXPORTS = (
    "gt_create", "gt_destroy", "gt_last_error", "gt_version", "gt_knn_exact", "gt_assign_top2",
    "gt_knn_bucketed", "gt_merge_rounds", "gt_refine_2hop", "gt_sanitize", "gt_cagra_prune",
    "gt_reverse_merge", "gt_optimize", "gt_translate", "gt_build_params_default", "gt_build_graph",
    "gt_prune_occlusion", "gt_reverse_insert", "gt_search_params_default", "gt_search", "gt_build_graph_ex",
    "gt_bucket_order", "gt_bucket_reorder", "gt_permute_rows", "gt_remap_table", "gt_optimize_noalloc",
    "gt_reverse_merge_chunked", "gt_prune_windowed", "gt_debug_opts_default", "gt_set_debug",
)
SEEDING = {"auto": 0, "kmeans||": 1, "uniform": 2}
REVMERGE_PATHS = {"auto": 0, "rv": 1, "binned": 2, "csr": 3, "rv2": 4}


class GtannError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"gtann error {code}: {msg}")
        self.code = code


class BuildParams(C.Structure):
    _fields_ = [
        ("metric", C.c_int32), ("n_buckets", C.c_int32), ("nprobe", C.c_int32), ("M", C.c_int32),
        ("K", C.c_int32), ("rounds", C.c_int32), ("refine_passes", C.c_int32), ("refine_sample", C.c_int32),
        ("kmeans_iters", C.c_int32), ("balance", C.c_float), ("seed", C.c_uint64),
        ("reverse_edges", C.c_int32), ("int_exact", C.c_int32), ("device_budget_mb", C.c_int32),
        ("seeding", C.c_int32), ("kmeans_train_fraction", C.c_float),
    ]


class DebugOpts(C.Structure):
    _fields_ = [
        ("knn_collect", C.c_int32), ("revmerge_path", C.c_int32), ("sub_order", C.c_int32),
        ("lloyd_host_csr", C.c_int32), ("prune_flat_rows", C.c_int32), ("knn_stats", C.c_int32),
        ("knn_prune", C.c_int32), ("bucket_host_csr", C.c_int32), ("knn_resident", C.c_int32),
        ("knn_window", C.c_int32), ("knn_screen", C.c_int32),
    ]


class BuildStats(C.Structure):
    _fields_ = [
        ("t_total", C.c_double), ("t_prepare", C.c_double), ("t_bucketing", C.c_double), ("t_knn", C.c_double),
        ("t_merge", C.c_double), ("t_refine", C.c_double), ("t_prune", C.c_double), ("t_revmerge", C.c_double),
        ("t_download", C.c_double), ("knn_flops", C.c_double), ("knn_pairs", C.c_double),
        ("max_pool", C.c_int64), ("max_bucket", C.c_int64), ("knn_launches", C.c_int64), ("knn_int8", C.c_int64),
        ("ooc_chunks", C.c_int64), ("knn_pairs_computed", C.c_double),
    ]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


class BuildExtras(C.Structure):
    _fields_ = [("round1_bucket", C.c_void_p), ("centroid_knn", C.c_void_p), ("centroid_knn_k", C.c_int32),
                ("reserved_", C.c_int32), ("last_bucket", C.c_void_p), ("last_centroids", C.c_void_p)]


class SearchParams(C.Structure):
    _fields_ = [
        ("topk", C.c_int32), ("ef", C.c_int32), ("num_entry", C.c_int32), ("metric", C.c_int32),
        ("seed", C.c_uint64), ("visited_slots", C.c_int32), ("reserved_", C.c_int32),
    ]


class SearchStats(C.Structure):
    _fields_ = [("t_total", C.c_double), ("t_search", C.c_double), ("expansions", C.c_int64),
                ("visited", C.c_int64), ("requeued", C.c_int64)]

    def as_dict(self):
        return {name: getattr(self, name) for name, _ in self._fields_}


_lib = None


def _torch_hip_runtime():
    """Path of the HIP runtime bundled with PyTorch-ROCm, or None."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return None
    path = os.path.join(list(spec.submodule_search_locations)[0], "lib", "libamdhip64.so")
    return path if os.path.exists(path) else None


def lib():
    """Loads libgtann.so; raises if it has not been built.

    One HIP runtime per process: PyTorch-ROCm ships its own libamdhip64
    (soname libamdhip64.so.7, the same as /opt/rocm's) and asks for it by a
    different name, so a process that loaded /opt/rocm's runtime through this
    library first would get a second runtime from torch, which cannot acquire
    the GPU.  When torch is installed its runtime is loaded first (without
    importing torch), and libgtann.so binds to it; with torch imported
    earlier this is the runtime already in the process."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"HIP library missing: {LIB_PATH} (run __graft_entry__.build())")
        rt = _torch_hip_runtime()
        if rt is not None:
            C.CDLL(rt, mode=C.RTLD_GLOBAL)
        L = C.CDLL(LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int32
        L.gt_create.argtypes = [C.c_int, C.POINTER(vp)]
        L.gt_destroy.argtypes = [vp]
        L.gt_destroy.restype = None
        L.gt_last_error.argtypes = [vp]
        L.gt_last_error.restype = C.c_char_p
        L.gt_version.restype = C.c_char_p
        L.gt_knn_exact.argtypes = [vp, vp, i64, i32, C.c_int, C.c_int, vp, i64, i32, vp, vp]
        L.gt_assign_top2.argtypes = [vp, vp, i64, i32, C.c_int, C.c_int, vp, i64, vp, vp]
        L.gt_knn_bucketed.argtypes = [vp, vp, i64, i32, C.c_int, C.c_int, vp, vp, i64, vp, i32, i32, vp, vp, C.c_int]
        L.gt_merge_rounds.argtypes = [vp, vp, vp, vp, vp, i64, i32, vp, vp]
        L.gt_refine_2hop.argtypes = [vp, vp, i64, i32, C.c_int, C.c_int, i32, i32, i32, vp, vp]
        L.gt_sanitize.argtypes = [vp, vp, i64, i32, vp]
        L.gt_cagra_prune.argtypes = [vp, vp, i64, i32, i32, vp]
        L.gt_reverse_merge.argtypes = [vp, vp, i64, i32, vp]
        L.gt_reverse_merge_chunked.argtypes = [vp, vp, i64, i32, i64, vp]
        L.gt_prune_windowed.argtypes = [vp, vp, i64, i32, vp, i32, vp, vp, i32, i32, i64, vp]
        L.gt_optimize.argtypes = [vp, vp, i64, i32, i32, vp]
        L.gt_optimize_noalloc.argtypes = [vp, vp, i64, i32, i32, vp]
        L.gt_translate.argtypes = [vp, vp, vp, i64, i32, vp]
        L.gt_prune_occlusion.argtypes = [vp, vp, i64, i32, C.c_int, vp, i32, i32, vp]
        L.gt_reverse_insert.argtypes = [vp, vp, vp, i64, i32]
        L.gt_build_params_default.argtypes = [C.POINTER(BuildParams)]
        L.gt_build_params_default.restype = None
        L.gt_build_graph.argtypes = [vp, vp, i64, i32, C.c_int, C.POINTER(BuildParams), vp, vp, vp,
                                     C.POINTER(BuildStats)]
        L.gt_build_graph_ex.argtypes = [vp, vp, i64, i32, C.c_int, C.POINTER(BuildParams), vp, vp, vp,
                                        C.POINTER(BuildStats), C.POINTER(BuildExtras)]
        L.gt_bucket_order.argtypes = [vp, vp, i64, i32, i32, vp]
        L.gt_bucket_reorder.argtypes = [vp, vp, i64, i64, vp, vp, i64, vp, vp, vp]
        L.gt_permute_rows.argtypes = [vp, vp, i64, i32, C.c_int, vp, vp]
        L.gt_remap_table.argtypes = [vp, vp, i64, i32, vp, vp]
        L.gt_search_params_default.argtypes = [C.POINTER(SearchParams)]
        L.gt_search_params_default.restype = None
        L.gt_search.argtypes = [vp, vp, i64, i32, C.c_int, vp, i32, vp, i64, vp, i32, C.POINTER(SearchParams),
                                vp, vp, C.POINTER(SearchStats)]
        L.gt_debug_opts_default.argtypes = [C.POINTER(DebugOpts)]
        L.gt_debug_opts_default.restype = None
        L.gt_set_debug.argtypes = [vp, C.POINTER(DebugOpts)]
        _lib = L
    return _lib


def _is_torch(a):
    return type(a).__module__.startswith("torch")


def _ptr(a):
    if a is None:
        return None
    if _is_torch(a):
        if not a.is_contiguous():
            raise ValueError("tensor must be contiguous")
        return C.c_void_p(a.data_ptr())
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("array must be C-contiguous")
    return C.c_void_p(a.ctypes.data)


def _np(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _dtype_code(X):
    if _is_torch(X):
        import torch
        m = {torch.float32: 0, torch.uint8: 1, torch.int8: 2}
    else:
        m = {np.dtype(np.float32): 0, np.dtype(np.uint8): 1, np.dtype(np.int8): 2}
    if X.dtype not in m:
        raise ValueError(f"unsupported dtype {X.dtype} (float32, uint8, int8)")
    return m[X.dtype]


def _empty_like_input(X, shape, dtype):
    """Output buffer on the same side (host/device) as the input."""
    if _is_torch(X):
        import torch
        tmap = {np.int32: torch.int32, np.float32: torch.float32, np.uint32: torch.int32, np.int64: torch.int64}
        return torch.empty(shape, dtype=tmap[dtype], device=X.device)
    return np.empty(shape, dtype=dtype)


def _as_u32(a):
    if _is_torch(a):
        return a
    return a.view(np.uint32) if a.dtype == np.int32 else _np(a, np.uint32)


@dataclass
class BuildResult:
    graph: object
    knn_ids: object
    knn_dists: object
    stats: dict
    round1_bucket: object = None
    centroid_knn: object = None
    last_bucket: object = None
    last_centroids: object = None


def _host_check(rc, what):
    if rc != GT_OK:
        msg = lib().gt_last_error(None)
        raise GtannError(rc, f"{what}: {msg.decode() if msg else ''}")


def bucket_order(graph, window):
    """DiskJoin processing order of the flat (B, K) bucket graph
    (src/bucket_order.hpp:161-262); host-side, no GPU needed."""
    g = _np(graph, np.uint32)
    B, K = g.shape
    out = np.empty(B, np.int32)
    _host_check(lib().gt_bucket_order(None, _ptr(g), B, K, int(window), _ptr(out)), "gt_bucket_order")
    return out


def bucket_reorder(assignment, n_buckets, order, cids=None):
    """(inverse_perm uint32 (N,), bucket_offsets uint32 (n_buckets + 1,),
    new ids of `cids` or None) -- compute_bucket_reorder
    (src/bucket.cu:8363-8412); host-side, no GPU needed."""
    a = _np(assignment, np.int32)
    o = _np(order, np.int32)
    N = len(a)
    inv = np.empty(N, np.uint32)
    off = np.empty(n_buckets + 1, np.uint32)
    c = None if cids is None else _np(cids, np.int64)
    cn = None if c is None else np.empty(len(c), np.uint32)
    _host_check(lib().gt_bucket_reorder(None, _ptr(a), N, n_buckets, _ptr(o), _ptr(c), 0 if c is None else len(c),
                                        _ptr(inv), _ptr(off), _ptr(cn)), "gt_bucket_reorder")
    return inv, off, cn


class Context:
    """One device + stream + workspaces (gt_create / gt_destroy)."""

    def __init__(self, device: int = 0):
        self._h = C.c_void_p()
        rc = lib().gt_create(device, C.byref(self._h))
        if rc != GT_OK:
            raise GtannError(rc, f"gt_create(device={device}) failed")

    def close(self):
        if self._h:
            lib().gt_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != GT_OK:
            msg = lib().gt_last_error(self._h)
            raise GtannError(rc, f"{what}: {msg.decode() if msg else ''}")

    def set_debug(self, **opts):
        """Path selection (gt_set_debug): every choice gives the same results.
        Keywords: knn_collect (bool), revmerge_path ('auto'|'rv'|'binned'|'csr'|'rv2'),
        sub_order (bool), lloyd_host_csr (bool), prune_flat_rows (bool),
        knn_stats (bool), knn_prune (bool), bucket_host_csr (bool),
        knn_resident (bool), knn_window (even tiles, 0 = by size),
        knn_screen (0 off, 1 by pass size, 2 always).  No keywords: the
        defaults."""
        o = DebugOpts()
        lib().gt_debug_opts_default(C.byref(o))
        for k, v in opts.items():
            if k == "revmerge_path":
                v = REVMERGE_PATHS[v] if isinstance(v, str) else int(v)
            elif k not in {f for f, _ in DebugOpts._fields_}:
                raise ValueError(f"unknown debug option {k!r}")
            setattr(o, k, int(v))
        self._check(lib().gt_set_debug(self._h, C.byref(o)), "gt_set_debug")

    # ---------------------------------------------------------------- stages

    def knn_exact(self, X, k, queries=None, metric="l2"):
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
        N, D = X.shape
        q = None
        nq = N
        if queries is not None:
            q = queries if _is_torch(queries) else _np(queries, np.int64)
            nq = int(q.shape[0])
        ids = _empty_like_input(X, (nq, k), np.int32)
        d = _empty_like_input(X, (nq, k), np.float32)
        self._check(lib().gt_knn_exact(self._h, _ptr(X), N, D, _dtype_code(X), METRICS[metric], _ptr(q), nq, k,
                                       _ptr(ids), _ptr(d)), "gt_knn_exact")
        return ids, d

    def assign_top2(self, X, Cm, metric="l2"):
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
            Cm = np.ascontiguousarray(Cm, dtype=X.dtype)
        N, D = X.shape
        top2 = _empty_like_input(X, (N, 2), np.int32)
        d2 = _empty_like_input(X, (N, 2), np.float32)
        self._check(lib().gt_assign_top2(self._h, _ptr(X), N, D, _dtype_code(X), METRICS[metric], _ptr(Cm),
                                         int(Cm.shape[0]), _ptr(top2), _ptr(d2)), "gt_assign_top2")
        return top2, d2

    def knn_bucketed(self, X, offsets, members, probe, M, metric="l2", running=None):
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
        N, D = X.shape
        offsets = _np(offsets, np.int64)
        members = _np(members, np.int32)
        probe = _np(probe, np.int32)
        P = probe.shape[1] if probe.ndim == 2 else 0
        if running is None:
            ids = _empty_like_input(X, (N, M), np.int32)
            d = _empty_like_input(X, (N, M), np.float32)
            merge = 0
        else:
            ids = running[0].copy() if not _is_torch(running[0]) else running[0].clone()
            d = running[1].copy() if not _is_torch(running[1]) else running[1].clone()
            merge = 1
        self._check(lib().gt_knn_bucketed(self._h, _ptr(X), N, D, _dtype_code(X), METRICS[metric], _ptr(offsets),
                                          _ptr(members), len(offsets) - 1, _ptr(probe), P, M, _ptr(ids), _ptr(d),
                                          merge), "gt_knn_bucketed")
        return ids, d

    def merge_rounds(self, run_ids, run_d, new_ids, new_d):
        run_ids, new_ids = _np(run_ids, np.int32), _np(new_ids, np.int32)
        run_d, new_d = _np(run_d, np.float32), _np(new_d, np.float32)
        N, M = run_ids.shape
        oi = np.empty((N, M), np.int32)
        od = np.empty((N, M), np.float32)
        self._check(lib().gt_merge_rounds(self._h, _ptr(run_ids), _ptr(run_d), _ptr(new_ids), _ptr(new_d), N, M,
                                          _ptr(oi), _ptr(od)), "gt_merge_rounds")
        return oi, od

    def refine_2hop(self, X, ids, d, S, passes=1, metric="l2"):
        X = np.ascontiguousarray(X)
        N, D = X.shape
        ids = _np(ids, np.int32).copy()
        d = _np(d, np.float32).copy()
        M = ids.shape[1]
        self._check(lib().gt_refine_2hop(self._h, _ptr(X), N, D, _dtype_code(X), METRICS[metric], M, S, passes,
                                         _ptr(ids), _ptr(d)), "gt_refine_2hop")
        return ids, d

    def sanitize(self, knn):
        knn = _np(knn, np.int32)
        N, M = knn.shape
        out = np.empty((N, M), np.uint32)
        self._check(lib().gt_sanitize(self._h, _ptr(knn), N, M, _ptr(out)), "gt_sanitize")
        return out

    def cagra_prune(self, knn, K):
        knn = _as_u32(knn)
        N, M = knn.shape
        out = np.empty((N, K), np.uint32)
        self._check(lib().gt_cagra_prune(self._h, _ptr(knn), N, M, K, _ptr(out)), "gt_cagra_prune")
        return out

    def reverse_merge(self, fwd):
        fwd = _np(fwd, np.uint32)
        N, K = fwd.shape
        out = np.empty((N, K), np.uint32)
        self._check(lib().gt_reverse_merge(self._h, _ptr(fwd), N, K, _ptr(out)), "gt_reverse_merge")
        return out

    def reverse_merge_chunked(self, fwd, device_budget_bytes=0):
        """Out-of-core reverse merge (optimize_chunked -m E with several
        chunks): the same rows as reverse_merge, within a device budget."""
        fwd = _np(fwd, np.uint32)
        N, K = fwd.shape
        out = np.empty((N, K), np.uint32)
        self._check(lib().gt_reverse_merge_chunked(self._h, _ptr(fwd), N, K, int(device_budget_bytes), _ptr(out)),
                    "gt_reverse_merge_chunked")
        return out

    def prune_windowed(self, cand, offsets, win, win_len, K, device_budget_bytes=0):
        """Windowed CAGRA prune (prune_windowed_gpu::run_chunked, candidates in
        rank order) of int32 cand (N, M) in the bucket-contiguous id space:
        offsets (n_buckets + 1) by processing position, win (n_buckets, W)
        window positions, win_len (n_buckets)."""
        cand = _np(cand, np.int32)
        N, M = cand.shape
        off = _np(offsets, np.uint32)
        win = _np(win, np.int32)
        wl = _np(win_len, np.int32)
        nb = off.shape[0] - 1
        if win.ndim != 2 or win.shape[0] != nb or wl.shape != (nb,):
            raise ValueError("win must be (n_buckets, W) and win_len (n_buckets,)")
        out = np.empty((N, K), np.uint32)
        self._check(lib().gt_prune_windowed(self._h, _ptr(cand), N, M, _ptr(off), nb, _ptr(win), _ptr(wl),
                                            win.shape[1], K, int(device_budget_bytes), _ptr(out)),
                    "gt_prune_windowed")
        return out

    def optimize(self, knn, K):
        knn = _as_u32(knn)
        N, M = knn.shape
        out = np.empty((N, K), np.uint32)
        self._check(lib().gt_optimize(self._h, _ptr(knn), N, M, K, _ptr(out)), "gt_optimize")
        return out

    def optimize_noalloc(self, knn, K, out=None):
        """gt_optimize_noalloc: knn (N, M) int32/uint32 and out (N, K)
        int32/uint32 must be contiguous device tensors of one GPU (this
        context's); the library allocates nothing."""
        import torch
        ok_dt = (torch.int32, getattr(torch, "uint32", torch.int32))
        if not (_is_torch(knn) and knn.is_cuda):
            raise ValueError("optimize_noalloc needs a device tensor")
        if knn.dim() != 2 or knn.dtype not in ok_dt or not knn.is_contiguous():
            raise ValueError(f"knn must be a contiguous 2-D int32 tensor, got {knn.dtype} {tuple(knn.shape)}")
        N, M = knn.shape
        if out is None:
            out = torch.empty((N, K), dtype=torch.int32, device=knn.device)
        if not (_is_torch(out) and out.is_cuda and out.device == knn.device):
            raise ValueError("out must be a device tensor on knn's device")
        if out.dtype not in ok_dt or tuple(out.shape) != (N, K) or not out.is_contiguous():
            raise ValueError(f"out must be a contiguous int32 ({N}, {K}) tensor, got {out.dtype} {tuple(out.shape)}")
        self._check(lib().gt_optimize_noalloc(self._h, _ptr(knn), N, M, K, _ptr(out)), "gt_optimize_noalloc")
        return out

    def prune_occlusion(self, X, nb, max_degree=0):
        """Occlusion prune (bd/prune.py:8-83); returns int32 (N, M), -1 padded."""
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
        N, D = X.shape
        nb = _np(nb, np.int32)
        if nb.ndim != 2 or nb.shape[0] != N:
            raise ValueError(f"neighbors must be ({N}, M), got {nb.shape}")
        M = nb.shape[1]
        out = np.empty((N, M), np.int32)
        self._check(lib().gt_prune_occlusion(self._h, _ptr(X), N, D, _dtype_code(X), _ptr(nb), M,
                                             int(max_degree or 0), _ptr(out)), "gt_prune_occlusion")
        return out

    def reverse_insert(self, ids, d):
        """Reverse-edge insertion (bd/build_bucket.py:473-543); returns new (ids, d)."""
        ids = _np(ids, np.int32).copy()
        d = _np(d, np.float32).copy()
        N, M = ids.shape
        self._check(lib().gt_reverse_insert(self._h, _ptr(ids), _ptr(d), N, M), "gt_reverse_insert")
        return ids, d

    def translate(self, g, inv):
        g = _np(g, np.uint32)
        inv = _np(inv, np.uint32)
        N, K = g.shape
        out = np.empty((N, K), np.uint32)
        self._check(lib().gt_translate(self._h, _ptr(g), _ptr(inv), N, K, _ptr(out)), "gt_translate")
        return out

    def build_graph(self, X, *, n_buckets=0, nprobe=1, M=64, K=32, rounds=2, refine_passes=0, refine_sample=16,
                    kmeans_iters=3, balance=0.8, seed=42, metric="l2", return_knn=True, reverse_edges=False,
                    prune=True, centroid_knn_k=0, round1_bucket=False, int_exact=True, device_budget_mb=0,
                    seeding="auto", kmeans_train_fraction=0.0, last_round=False, graph_out=None):
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
        N, D = X.shape
        p = BuildParams()
        lib().gt_build_params_default(C.byref(p))
        p.metric, p.n_buckets, p.nprobe, p.M, p.K = METRICS[metric], n_buckets, nprobe, M, K
        p.rounds, p.refine_passes, p.refine_sample, p.kmeans_iters = rounds, refine_passes, refine_sample, kmeans_iters
        p.balance, p.seed, p.reverse_edges = balance, seed, int(bool(reverse_edges))
        p.int_exact = int(bool(int_exact))
        p.device_budget_mb = int(device_budget_mb)
        p.seeding = SEEDING[seeding] if isinstance(seeding, str) else int(seeding)
        p.kmeans_train_fraction = float(kmeans_train_fraction)
        if graph_out is not None:
            if tuple(graph_out.shape) != (N, K) or np.dtype(str(graph_out.dtype).replace("torch.", "")).itemsize != 4:
                raise ValueError(f"graph_out must be a ({N}, {K}) 32-bit array")
            graph = graph_out
        else:
            graph = _empty_like_input(X, (N, K), np.uint32) if prune else None
        ids = _empty_like_input(X, (N, M), np.int32) if return_knn else None
        d = _empty_like_input(X, (N, M), np.float32) if return_knn else None
        st = BuildStats()
        ex = BuildExtras()
        nb = min(max(1, n_buckets if n_buckets > 0 else N // 4000), N)
        r1 = np.empty(N, np.int32) if round1_bucket else None
        ck = np.empty((nb, centroid_knn_k), np.uint32) if centroid_knn_k > 0 else None
        ex.round1_bucket = None if r1 is None else r1.ctypes.data
        ex.centroid_knn = None if ck is None else ck.ctypes.data
        ex.centroid_knn_k = centroid_knn_k
        lb = np.empty(N, np.int32) if last_round else None
        lc = np.empty(nb, np.int64) if last_round else None
        ex.last_bucket = None if lb is None else lb.ctypes.data
        ex.last_centroids = None if lc is None else lc.ctypes.data
        self._check(lib().gt_build_graph_ex(self._h, _ptr(X), N, D, _dtype_code(X), C.byref(p), _ptr(ids), _ptr(d),
                                            _ptr(graph), C.byref(st), C.byref(ex)), "gt_build_graph_ex")
        if graph is not None and not _is_torch(graph):
            graph = graph.view(np.uint32)
        return BuildResult(graph=graph, knn_ids=ids, knn_dists=d, stats=st.as_dict(), round1_bucket=r1,
                           centroid_knn=ck, last_bucket=lb, last_centroids=lc)

    def permute_rows(self, X, inverse_perm):
        """out row n = X row inverse_perm[n] (data_reordered)."""
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
        N, D = X.shape
        inv = _np(inverse_perm, np.uint32)
        out = np.empty_like(X) if not _is_torch(X) else X.new_empty(X.shape)
        if _is_torch(X):
            import torch
            codes = {torch.float32: 0, torch.uint8: 1, torch.int8: 2}
        else:
            codes = {np.dtype(np.float32): 0, np.dtype(np.uint8): 1, np.dtype(np.int8): 2}
        self._check(lib().gt_permute_rows(self._h, _ptr(X), N, D, codes[X.dtype], _ptr(inv), _ptr(out)),
                    "gt_permute_rows")
        return out

    def remap_table(self, ids, inverse_perm):
        """Per-point id table in new ids: out[n] = perm[ids[inverse_perm[n]]]."""
        ids = _np(ids, np.int32)
        N, M = ids.shape
        inv = _np(inverse_perm, np.uint32)
        out = np.empty_like(ids)
        self._check(lib().gt_remap_table(self._h, _ptr(ids), N, M, _ptr(inv), _ptr(out)), "gt_remap_table")
        return out

    def search(self, X, graph, Q, *, topk=10, ef=200, num_entry=4, entries=None, metric="l2", seed=42,
               visited_slots=0):
        """Beam search (bd/search.py:20-90 per query) of the rows of Q over
        `graph` (N, degree); ids outside [0, N) in the graph are skipped.
        entries: (nq, E) int entry points in processing order (< 0 skipped),
        or None to let the library draw `num_entry` per query.  Returns
        (ids int32 (nq, topk), dists float32, stats dict)."""
        if not _is_torch(X):
            X = np.ascontiguousarray(X)
            Q = np.ascontiguousarray(Q, dtype=X.dtype)
        N, D = X.shape
        if Q.shape[1] != D:
            raise ValueError(f"query dimension {Q.shape[1]} != base dimension {D}")
        if _is_torch(graph):
            g = graph
        else:
            g = np.asarray(graph)
            if g.dtype != np.uint32:
                g64 = g.astype(np.int64)
                g = np.where((g64 >= 0) & (g64 < N), g64, 0xFFFFFFFF).astype(np.uint32)
            g = np.ascontiguousarray(g)
        if g.shape[0] != N:
            raise ValueError(f"graph must have {N} rows, got {g.shape[0]}")
        nq = int(Q.shape[0])
        E = 0
        ent = None
        if entries is not None:
            ent = entries if _is_torch(entries) else _np(np.asarray(entries).reshape(nq, -1), np.int32)
            E = int(ent.shape[1])
        p = SearchParams()
        lib().gt_search_params_default(C.byref(p))
        p.topk, p.ef, p.num_entry, p.metric = topk, ef, num_entry, METRICS[metric]
        p.seed, p.visited_slots = seed, visited_slots
        ids = _empty_like_input(X, (nq, topk), np.int32)
        d = _empty_like_input(X, (nq, topk), np.float32)
        st = SearchStats()
        self._check(lib().gt_search(self._h, _ptr(X), N, D, _dtype_code(X), _ptr(g), int(g.shape[1]), _ptr(Q), nq,
                                    _ptr(ent), E, C.byref(p), _ptr(ids), _ptr(d), C.byref(st)), "gt_search")
        return ids, d, st.as_dict()
