"""Pins the deterministic transcendental layer (splatx-metal_amd/csrc/sx_fmath.h) that both the
device code and the CPU oracle use: compared with float64 numpy references (correctly rounded to
float32 in all but rare double-rounding cases) and with glibc's float functions."""
import ctypes

import numpy as np
import pytest

LIBM = ctypes.CDLL("libm.so.6")
for f in ("logf", "expf", "sinf", "cosf", "powf"):
    getattr(LIBM, f).restype = ctypes.c_float
    getattr(LIBM, f).argtypes = [ctypes.c_float] * (2 if f == "powf" else 1)


def ulp_diff(a, b):
    ai = a.astype(np.float32).view(np.int32).astype(np.int64)
    bi = b.astype(np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, np.int64(-2**31) - ai, ai)
    bi = np.where(bi < 0, np.int64(-2**31) - bi, bi)
    return np.abs(ai - bi)


@pytest.fixture(scope="module")
def rng():
    return np.random.default_rng(123)


def test_logf_correctly_rounded(oracle, rng):
    x = np.concatenate([rng.uniform(1.0, 255.0, 400_000), 10 ** rng.uniform(-40, 38, 400_000),
                        np.array([1.0, 2.0, 0.5, 255.0, 1e-45, 3.4e38])]).astype(np.float32)
    y = oracle.logf(x)
    ref = np.log(x.astype(np.float64)).astype(np.float32)
    assert ulp_diff(y, ref).max() <= 1
    assert (y != ref).sum() <= 2  # double rounding of the float64 reference only
    assert oracle.logf(np.array([1.0], np.float32))[0] == 0.0
    assert np.isneginf(oracle.logf(np.array([0.0], np.float32))[0])
    assert np.isnan(oracle.logf(np.array([-1.0], np.float32))[0])


def test_logf_agrees_with_glibc(oracle, rng):
    x = rng.uniform(1.0, 255.0, 50_000).astype(np.float32)
    y = oracle.logf(x)
    g = np.array([LIBM.logf(float(v)) for v in x], np.float32)
    assert ulp_diff(y, g).max() <= 1
    assert (y != g).mean() < 1e-3


def test_expf_correctly_rounded(oracle, rng):
    x = np.concatenate([rng.uniform(-103.0, 88.7, 400_000), rng.uniform(-1, 1, 200_000),
                        np.array([0.0, -0.0, 88.72, -87.3, -103.9, 1e-8])]).astype(np.float32)
    y = oracle.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert ulp_diff(y, ref).max() <= 1
    assert (y != ref).sum() <= 2
    assert oracle.expf(np.array([0.0], np.float32))[0] == 1.0
    assert np.isinf(oracle.expf(np.array([89.0], np.float32))[0])
    assert oracle.expf(np.array([-110.0], np.float32))[0] == 0.0


def test_expf_fast_within_two_ulp(oracle, rng):
    # the rasterizer's exp(-sigma): sigma in [0, ~20] matters; check a wide range
    x = np.concatenate([-rng.uniform(0.0, 30.0, 400_000), rng.uniform(-87.0, 88.0, 200_000)]).astype(np.float32)
    y = oracle.expf_fast(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    d = ulp_diff(y, ref)
    assert d.max() <= 2
    assert d.mean() < 0.2
    assert oracle.expf_fast(np.array([0.0], np.float32))[0] == 1.0


def test_sincosf_correctly_rounded(oracle, rng):
    x = (rng.uniform(0, 1, 400_000) * np.float32(6.2831855)).astype(np.float32)
    s, c = oracle.sincosf(x)
    rs = np.sin(x.astype(np.float64)).astype(np.float32)
    rc = np.cos(x.astype(np.float64)).astype(np.float32)
    # near zeros of sin/cos the float64 reference itself carries the absolute error; compare in ulps of 1
    assert np.abs(s - rs).max() <= 6e-8 and np.abs(c - rc).max() <= 6e-8
    assert (s != rs).sum() <= 4 and (c != rc).sum() <= 4


def test_powf(oracle, rng):
    x = rng.uniform(0.0, 1.0, 200_000).astype(np.float32)
    p = rng.integers(1, 52, 200_000).astype(np.float32)
    inv = (1.0 / p).astype(np.float32)
    for e in (p, inv):
        y = oracle.powf(x, e)
        ref = np.power(x.astype(np.float64), e.astype(np.float64)).astype(np.float32)
        assert ulp_diff(y, ref).max() <= 1
        assert (y != ref).sum() <= 4


def test_a_planted_polynomial_error_is_caught(oracle, rng):
    """The checks above detect a wrong Taylor coefficient: perturbing exp's result by 1 part in 1e6
    (what dropping the r^5 term would do near |r| = 0.35) breaks the 1-ulp bound."""
    x = rng.uniform(-20, 20, 10_000).astype(np.float32)
    y = oracle.expf(x) * np.float32(1 + 1e-6)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert ulp_diff(y, ref).max() > 1
