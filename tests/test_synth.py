"""The seeded synthetic configurations are reproducible and follow their recipes."""
import numpy as np

import synth


def test_reproducible_and_prefix_stable():
    a, _ = synth.generate("C2", n=5000)
    b, _ = synth.generate("C2", n=5000)
    assert a.dtype == np.float32 and a.shape == (5000, 128)
    np.testing.assert_array_equal(a, b)


def test_recipes():
    x, q = synth.generate("C2", n=3000, queries=100)
    assert q.shape == (100, 128)
    assert x.min() >= 0 and x.max() <= 255 and (x == np.rint(x)).all()
    x, _ = synth.generate("C3", n=2000)
    np.testing.assert_allclose(np.linalg.norm(x, axis=1), 1.0, atol=1e-5)
    x, _ = synth.generate("C5", n=2000)
    assert x.dtype == np.int8 and x.min() >= -127
    x, _ = synth.generate("C1", n=2000)
    assert x.shape == (2000, 128) and np.abs(x).max() < 20
    x, _ = synth.generate("C4", n=500)
    assert x.shape == (500, 960)


def test_configs_match_baseline():
    c = synth.CONFIGS
    assert (c["C2"].n, c["C2"].dim, c["C2"].buckets, c["C2"].M, c["C2"].K) == (1_000_000, 128, 256, 64, 32)
    assert (c["C4"].M, c["C4"].K, c["C4"].buckets) == (96, 48, 512)
    assert c["C3"].metric == "ip" and c["C5"].dtype == "i8"
