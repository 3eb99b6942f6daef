"""CPU checks of the C-ABI library: it loads without a GPU, exports every
entry point include/gtann.h declares, and fails cleanly where no device exists."""
import ctypes as C
import os
import re

import numpy as np

import gtann

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "gtann.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|void|const char\*)\s+(gt_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("gt_create", "gt_destroy", "gt_last_error", "gt_knn_exact", "gt_assign_top2",
                     "gt_knn_bucketed", "gt_refine_2hop", "gt_sanitize", "gt_cagra_prune",
                     "gt_reverse_merge", "gt_optimize", "gt_translate", "gt_build_graph"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = gtann.lib()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in gtann.h but not exported"
    assert set(gtann.EXPORTS) <= set(declared_functions())


def test_version_and_defaults():
    lib = gtann.lib()
    assert lib.gt_version().startswith(b"gtann")
    p = gtann.BuildParams()
    lib.gt_build_params_default(C.byref(p))
    assert (p.M, p.K, p.rounds, p.nprobe, p.kmeans_iters, p.seed) == (64, 32, 2, 1, 3, 42)
    assert abs(p.balance - 0.8) < 1e-6


def test_create_without_device_fails_cleanly():
    lib = gtann.lib()
    h = C.c_void_p()
    rc = lib.gt_create(0, C.byref(h))
    if rc == gtann.GT_OK:          # a GPU is visible: nothing to check here
        lib.gt_destroy(h)
    else:
        assert rc == gtann.GT_EDEVICE and not h.value
    assert lib.gt_create(-1, C.byref(h)) == gtann.GT_EDEVICE
    assert lib.gt_last_error(None) == b"null context"


def test_null_context_is_rejected():
    lib = gtann.lib()
    X = np.zeros((4, 8), np.float32)
    ids = np.zeros((4, 2), np.int32)
    d = np.zeros((4, 2), np.float32)
    rc = lib.gt_knn_exact(None, X.ctypes.data, 4, 8, 0, 0, None, 4, 2, ids.ctypes.data, d.ctypes.data)
    assert rc == gtann.GT_EINVAL


def test_one_hip_runtime_with_torch():
    # libgtann.so and PyTorch must share one HIP runtime, whichever is loaded
    # first (two runtimes in one process cannot both acquire the GPU)
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r); import gtann; gtann.lib(); import torch; "
            "m = {l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}; print(len(m))"
            % os.path.join(ROOT, "gpu-talored-ann_amd"))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True)
    assert out.stdout.strip() == "1"
