"""The oracle's fp16 rounding (the KV rows of the engine's flagged fp16 KV
mode) against numpy's binary16 conversion, an independent round-to-nearest-
even implementation: random values over the whole range, every halfway point
between neighbouring halves of a few binades, subnormals and the overflow
boundary."""
import numpy as np

import _native as N

O = N.oracle()


def rh(xs):
    return np.array([O.or_round_half(float(x)) for x in np.asarray(xs, np.float32)], np.float32)


def ref(xs):
    return np.asarray(xs, np.float32).astype(np.float16).astype(np.float32)


def same(a, b):
    return np.array_equal(a, b) or np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(
        a[~np.isnan(a)], b[~np.isnan(b)])


def test_round_half_random_values():
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 1 << 32, 20000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    x = np.concatenate([x, rng.normal(0, 3, 20000).astype(np.float32),
                        rng.normal(0, 1e-5, 5000).astype(np.float32)])
    assert same(rh(x), ref(x))


def test_round_half_ties_subnormals_and_overflow():
    # halfway points between consecutive halves (ties go to the even one),
    # and their fp32 neighbours, in normal and subnormal binades
    h = np.arange(0, 0x7C00, 97, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    near = np.concatenate([mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    edge = np.array([65504.0, 65519.99, 65520.0, 70000.0, 2.0 ** -24, 2.0 ** -25, 2.0 ** -26,
                     3 * 2.0 ** -26, 2.0 ** -14, 0.0, -0.0, np.inf, -np.inf, np.nan], np.float32)
    for xs in (near, -near, edge):
        assert same(rh(xs), ref(xs))
