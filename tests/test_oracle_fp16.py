"""Pins the oracle's binary16 conversions against numpy's IEEE casts.

numpy implements float16<->float32 with round-to-nearest-even, the same
rounding as cuda_fp16's __float2half / __half2float used by the reference
kernels (e.g. flash_decode_q1_opt.cuh:457,534).
"""
import numpy as np

from oracle import oracle


def test_h2f_all_65536_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    h = bits.view(np.float16)
    got = oracle.h2f(h)
    want = h.astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _boundary_floats():
    """Every binary16 value, its float32 neighbours, and the exact midpoints
    between consecutive binary16 values (ties) with their neighbours."""
    h = np.arange(0, 0x7C01, dtype=np.uint32).astype(np.uint16).view(np.float16)
    f = h.astype(np.float64)
    mids = (f[:-1] + f[1:]) / 2.0                      # exact in float32 (<= 12 significant bits)
    vals = np.concatenate([f, mids, [65504.0, 65519.99, 65520.0, 65536.0, 1e30, 2.0 ** -25,
                                     2.0 ** -26, 1e-30, 1e-45]]).astype(np.float32)
    ub = vals.view(np.uint32)
    near = np.concatenate([ub, ub + 1, ub - 1]).view(np.float32)
    near = near[np.isfinite(near)]
    return np.concatenate([near, -near, [np.inf, -np.inf]]).astype(np.float32)


def test_f2h_rne_ties_overflow_subnormals():
    x = _boundary_floats()
    got = oracle.f2h(x).view(np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(float(x[i]), hex(got[i]), hex(want[i])) for i in bad[:5]]


def test_f2h_random_bit_patterns():
    rng = np.random.default_rng(1234)
    x = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    got = oracle.f2h(x).view(np.uint16)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f2h_nan_stays_nan():
    x = np.array([np.nan, -np.nan], np.float32)
    assert np.all(np.isnan(oracle.f2h(x).astype(np.float32)))
