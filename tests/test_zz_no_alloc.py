"""gt_optimize_noalloc (prune + reverse merge with the library's fixed
per-GPU scratch array, no allocation) against gt_optimize, bit for bit,
through the C ABI on device tensors: two calls in a row, the second on a
smaller input, so stale scratch contents from the first call would show."""
import numpy as np
import pytest

import gtann

pytestmark = pytest.mark.gpu


def _table(rng, N, M):
    G = rng.integers(0, N, size=(N, M)).astype(np.int32)
    G[rng.random((N, M)) < 0.02] = -1
    return G


def _check(ctx, torch, G, K):
    want = ctx.optimize(G, K)                       # allocating entry point, host buffers
    kn = torch.from_numpy(G).cuda()
    out = torch.full((G.shape[0], K), -7, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    got = ctx.optimize_noalloc(kn, K, out)
    np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), want)


def test_noalloc_matches_optimize_twice_shrinking(ctx):
    import torch
    rng = np.random.default_rng(71)
    print("noalloc: N=32768 M=64 K=32", flush=True)
    _check(ctx, torch, _table(rng, 32768, 64), 32)     # N*K = 2^20, the maximum
    print("noalloc: N=3000 M=48 K=24", flush=True)
    _check(ctx, torch, _table(rng, 3000, 48), 24)


def test_noalloc_rejects_beyond_maximum_and_host_buffers(ctx):
    import torch
    G = torch.zeros((32769, 64), dtype=torch.int32, device="cuda")
    with pytest.raises(gtann.GtannError) as e:
        ctx.optimize_noalloc(G, 32)
    assert e.value.code == gtann.GT_EINVAL and "scratch maximum" in str(e.value)
    out = np.empty((100, 8), np.int32)
    h = np.zeros((100, 16), np.int32)
    rc = gtann.lib().gt_optimize_noalloc(ctx._h, h.ctypes.data, 100, 16, 8, out.ctypes.data)
    assert rc == gtann.GT_EINVAL


def test_noalloc_few_candidates_error(ctx):
    import torch
    G = np.full((500, 16), -1, np.int32)
    G[:, :4] = np.random.default_rng(3).integers(0, 500, size=(500, 4))
    with pytest.raises(gtann.GtannError) as e:
        ctx.optimize_noalloc(torch.from_numpy(G).cuda(), 8)
    assert e.value.code == gtann.GT_EFEWCAND
    # the next call after an error still gives the right graph
    rng = np.random.default_rng(5)
    _check(ctx, torch, _table(rng, 2000, 32), 16)
