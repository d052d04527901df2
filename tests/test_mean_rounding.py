"""The mean pooling rounding used by the HIP kernels, checked on the CPU.

The kernels divide a bag's fp32 sum `a` by its length L as RN32(RN64(a * RN64(1/L))) when the
quotient is in the fp32 normal range (|a| >= 2^-126 * L) and by IEEE fp32 division otherwise.
The oracle divides with IEEE fp32 division (baseline/infer.py:256-263 pools in fp32). These tests
restate the kernel's arithmetic with numpy's IEEE fp64/fp32 operations and compare bit for bit.
"""
import numpy as np

FLT_MIN = np.float32(2.0 ** -126)


def kernel_mean(a, L):
    a = np.asarray(a, np.float32)
    L = np.asarray(L, np.int64)
    inv = 1.0 / L.astype(np.float64)
    q = (a.astype(np.float64) * inv).astype(np.float32)
    fl = L.astype(np.float32)
    slow = np.abs(a) < FLT_MIN * fl
    with np.errstate(invalid="ignore", over="ignore"):
        q[slow] = (a[slow] / fl[slow]).astype(np.float32)
    return q


def ieee_mean(a, L):
    with np.errstate(invalid="ignore", over="ignore"):
        return (np.asarray(a, np.float32) / np.asarray(L, np.int64).astype(np.float32)).astype(np.float32)


def same_bits(x, y):
    x, y = np.asarray(x, np.float32), np.asarray(y, np.float32)
    nan = np.isnan(x) & np.isnan(y)
    return np.all(nan | (x.view(np.uint32) == y.view(np.uint32)))


def test_random_sums_and_lengths():
    rng = np.random.default_rng(0)
    n = 2_000_000
    a = rng.standard_normal(n).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, n).astype(np.float32)
    L = np.concatenate([rng.integers(1, 300, n // 2), rng.integers(1, 1 << 24, n - n // 2)])
    assert same_bits(kernel_mean(a, L), ieee_mean(a, L))


def test_all_bit_patterns_sampled():
    # fp32 bit patterns over every exponent, including subnormals, Inf and NaN
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 1 << 32, 3_000_000, dtype=np.uint64).astype(np.uint32)
    a = bits.view(np.float32)
    L = rng.integers(1, 5000, len(a))
    assert same_bits(kernel_mean(a, L), ieee_mean(a, L))


def test_exact_quotients_and_near_midpoints():
    # a = q * L for representable q (exact quotient), and a one ulp either side of it
    rng = np.random.default_rng(2)
    L = rng.integers(1, 4097, 500_000)
    q = rng.standard_normal(len(L)).astype(np.float32)
    a = (q.astype(np.float64) * L).astype(np.float32)
    for x in (a, np.nextafter(a, np.float32(np.inf)), np.nextafter(a, np.float32(-np.inf))):
        assert same_bits(kernel_mean(x, L), ieee_mean(x, L))


def test_subnormal_quotients_take_the_division():
    # quotients at and below 2^-126, where fp32 midpoints can be hit exactly (e.g. 9 * 2^-149 / 6)
    a = np.array([9 * 2.0 ** -149, 3 * 2.0 ** -149, 2.0 ** -126, -(2.0 ** -125), 1e-40, 0.0, -0.0], np.float32)
    for L in (1, 2, 3, 6, 7, 1 << 20):
        Ls = np.full(len(a), L)
        assert same_bits(kernel_mean(a, Ls), ieee_mean(a, Ls))
    # exact midpoints that the fp64 product alone rounds the wrong way (found by search):
    # a / L = (2k+1) * 2^-150
    for L, m in ((98, 147), (150, 2175), (154, 2233), (182, 1183), (186, 1209)):
        a1 = np.array([m * 2.0 ** -149, -m * 2.0 ** -149], np.float32)
        wrong = (a1.astype(np.float64) * (1.0 / np.float64(L))).astype(np.float32)
        assert not same_bits(wrong, ieee_mean(a1, [L, L]))
        assert same_bits(kernel_mean(a1, [L, L]), ieee_mean(a1, [L, L]))
    rng = np.random.default_rng(3)
    m = rng.integers(1, 1 << 23, 1_000_000)
    tiny = (m * 2.0 ** -149).astype(np.float32)
    L = rng.integers(1, 64, len(m))
    assert same_bits(kernel_mean(tiny, L), ieee_mean(tiny, L))
