"""The synthetic-input generator: SplitMix64 known answers and distribution checks."""
import numpy as np

from gomlx_hip import synth


def test_splitmix64_published_vector():
    # Published SplitMix64 outputs for state 1234567 (reference implementation by
    # S. Vigna, prng.di.unimi.it/splitmix64.c).
    got = synth.splitmix64(1234567, 5).tolist()
    assert got == [6457827717110365317, 3203168211198807973, 9817491932198370423,
                   4593380528125082431, 16408922859458223821]


def test_normal_moments_and_determinism():
    a = synth.normal(1001, (1 << 18,), std=2.0)
    assert a.dtype == np.float32
    assert abs(float(a.mean())) < 0.02 and abs(float(a.std()) - 2.0) < 0.02
    assert np.array_equal(a, synth.normal(1001, (1 << 18,), std=2.0))
    assert not np.array_equal(a[:100], synth.normal(1002, (100,), std=2.0))


def test_uniform_int_range():
    v = synth.uniform_int(5001, (8, 1024), 0, 32000)
    assert v.dtype == np.int32 and v.min() >= 0 and v.max() < 32000


def test_normal_device_matches_host_stream():
    """The torch form (run here on the CPU) draws the same SplitMix64 stream: equal
    to the numpy form value for value on a ragged shape, odd length included."""
    import torch  # noqa: F401
    for shape in ((3, 1000, 77), (5,), (1, 1)):
        a = synth.normal(3001, shape, std=0.125, mean=0.5)
        b = synth.normal_device(3001, shape, std=0.125, mean=0.5, device="cpu").numpy()
        assert b.shape == a.shape and np.max(np.abs(a - b)) <= np.spacing(np.abs(a)).max()
