"""The measurement protocol's counter-based generator, CPU side
(oracle.synth / loom_oracle_synth), pinned without trusting its own code:

- the counter stream: numpy restates splitmix64 (uint64 wraparound) on the
  same counters and the uniform draws must equal a + (b - a) * u exactly
  (one fused rounding in fp32, so within half an ulp of the fp64 value);
- Box-Muller: the fp32 normals must match sqrt(-2 ln u1) cos(2 pi u2) in
  fp64 from the same bits to 1e-6 absolute (the hand-written ln and cos
  polynomials, the exponent and octant splits);
- bf16 output is the round-to-nearest-even of the fp32 output;
- element i depends on (seed, i) only: a prefix is the same whatever n;
- distributions: Kolmogorov-Smirnov against N(0, 1) and U[-1, 1) on 2^18
  draws, and the moments of a scaled N(0.5, 0.02).
The GPU generator (loom_hip_synth) is checked bit for bit against this one
in tests/test_gpu_synth.py.
"""
import numpy as np
import pytest
from scipy import stats

import oracle

M64 = np.uint64((1 << 64) - 1)


def mix(z):
    z = z.astype(np.uint64)
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def bits(seed, n):
    i = np.arange(n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return mix(np.uint64(seed) * np.uint64(0xD1B54A32D192ED03) + i * np.uint64(0x9E3779B97F4A7C15))


@pytest.mark.parametrize("seed", [0, 1, 12345, (1 << 64) - 1])
def test_uniform_is_the_counter_stream(seed):
    n = 4096
    z = bits(seed, n)
    u = (z >> np.uint64(40)).astype(np.float64) * 2.0 ** -24
    got = oracle.synth((n,), seed, "uniform", -1.0, 1.0, bf16=False).astype(np.float64)
    exp = -1.0 + 2.0 * u
    # fmaf(b - a, u, a) rounds once: within half an fp32 ulp of the exact value
    assert np.all(np.abs(got - exp) <= np.spacing(np.abs(exp).astype(np.float32)) * 0.5 + 1e-30)


@pytest.mark.parametrize("seed", [3, 77, 2 ** 40 + 5])
def test_normal_is_box_muller(seed):
    n = 1 << 16
    z = bits(seed, n)
    u1 = ((z >> np.uint64(40)) + np.uint64(1)).astype(np.float64) * 2.0 ** -24
    u2 = ((z >> np.uint64(16)) & np.uint64(0xFFFFFF)).astype(np.float64) * 2.0 ** -24
    exp = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    got = oracle.synth((n,), seed, "normal", 0.0, 1.0, bf16=False).astype(np.float64)
    assert np.max(np.abs(got - exp)) < 1e-6


def test_bf16_is_rounded_fp32_and_prefix_independent():
    f = oracle.synth((3, 1000), 9, "normal", 0.25, 2.0, bf16=False)
    h = oracle.synth((3, 1000), 9, "normal", 0.25, 2.0)
    assert h.dtype == np.uint16 and np.array_equal(h, oracle.to_bf16(f))
    assert np.array_equal(oracle.synth((10,), 9, "normal", 0.25, 2.0, bf16=False),
                          f.reshape(-1)[:10])
    assert not np.array_equal(oracle.synth((10,), 10, "normal", 0.25, 2.0), h.reshape(-1)[:10])


def test_distributions():
    n = 1 << 18
    x = oracle.synth((n,), 21, "normal", 0.0, 1.0, bf16=False).astype(np.float64)
    assert stats.kstest(x, "norm").pvalue > 1e-3
    u = oracle.synth((n,), 22, "uniform", -1.0, 1.0, bf16=False).astype(np.float64)
    assert stats.kstest(u, "uniform", args=(-1.0, 2.0)).pvalue > 1e-3
    assert u.min() >= -1.0 and u.max() < 1.0
    y = oracle.synth((n,), 23, "normal", 0.5, 0.02, bf16=False).astype(np.float64)
    assert abs(y.mean() - 0.5) < 1e-3 and abs(y.std() - 0.02) < 1e-3


def test_rejects_bad_arguments():
    with pytest.raises(KeyError):
        oracle.synth((4,), 0, "poisson")


def test_square_root_is_correctly_rounded():
    """The generator's square root (integer arithmetic, so host and device
    agree) equals IEEE sqrt rounded to nearest: every float of two binades
    and a log sweep over the generator's inputs (0 and -2 ln u1 <= 33.3)."""
    m = np.arange(1 << 23, dtype=np.uint32)
    xs = [((np.uint32(e) << np.uint32(23)) | m).view(np.float32) for e in (127, 128)]
    xs.append(np.geomspace(1e-30, 40.0, 1 << 20).astype(np.float32))
    xs.append(np.array([0.0, -0.0, 1.0, 4.0, 33.27106, 2.0 ** -24], np.float32))
    x = np.concatenate(xs)
    got = oracle.synth_sqrt(x)
    exp = np.sqrt(np.maximum(x, 0.0)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), np.abs(exp).view(np.uint32))
