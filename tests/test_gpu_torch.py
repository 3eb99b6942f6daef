"""Device-tensor callers: inputs written asynchronously on PyTorch's default
stream right before a call must be read after that work completes (the
library's stream is a blocking stream, ordered after the legacy null
stream).  Results must equal those of the same call on host arrays."""
import numpy as np
import pytest

import gt_oracle as O

pytestmark = pytest.mark.gpu


def _busy_then_copy(torch, src):
    """X = src, queued on the default stream behind ~tens of ms of matmuls."""
    X = torch.zeros_like(src)
    a = torch.randn(4096, 4096, device=src.device)
    for _ in range(24):
        a = a @ a
        a = a / a.norm()
    X.copy_(src)
    return X


def test_knn_exact_reads_async_written_device_input(ctx):
    import torch
    rng = np.random.default_rng(31)
    Xh = rng.integers(0, 256, size=(6000, 128)).astype(np.float32)
    ref_i, ref_d = ctx.knn_exact(Xh, 16)
    src = torch.from_numpy(Xh).cuda()
    torch.cuda.synchronize()
    X = _busy_then_copy(torch, src)
    ids, d = ctx.knn_exact(X, 16)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_i)
    np.testing.assert_array_equal(d.cpu().numpy().view(np.uint32), ref_d.view(np.uint32))
    oi, _ = O.knn_exact(Xh, 16)
    np.testing.assert_array_equal(ref_i, oi)


def test_build_and_optimize_read_async_written_device_inputs(ctx):
    import torch
    rng = np.random.default_rng(32)
    Xh = rng.integers(0, 256, size=(8000, 64)).astype(np.float32)
    ref = ctx.build_graph(Xh, n_buckets=8, nprobe=2, M=32, K=16, rounds=2)
    src = torch.from_numpy(Xh).cuda()
    torch.cuda.synchronize()
    X = _busy_then_copy(torch, src)
    res = ctx.build_graph(X, n_buckets=8, nprobe=2, M=32, K=16, rounds=2)
    np.testing.assert_array_equal(np.asarray(res.knn_ids.cpu()), ref.knn_ids)
    np.testing.assert_array_equal(np.asarray(res.graph.cpu()).view(np.uint32), ref.graph.view(np.uint32))
    # the graph stages on a table written the same way
    kn = torch.from_numpy(ref.knn_ids.astype(np.int32)).cuda()
    torch.cuda.synchronize()
    kn2 = _busy_then_copy(torch, kn)
    g = ctx.optimize(kn2, 16)   # host output, device input
    np.testing.assert_array_equal(np.asarray(g).view(np.uint32), ref.graph.view(np.uint32))
