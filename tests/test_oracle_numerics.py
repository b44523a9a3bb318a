"""CPU: the oracle's scalar numerics against library routines and closed forms.

exp (Cody-Waite + Taylor) against float64 exp, F16 conversion against numpy's IEEE
float16 cast, half_sat against its definition (common/math.h:33-40), silu/sigmoid against
float64 formulas.
"""
import numpy as np
import pytest


def _ulp32(x):
    x = np.abs(np.asarray(x, np.float32))
    return np.spacing(x).astype(np.float64)


def test_exp_accuracy_sweep(orc):
    lib = orc.lib()
    xs = np.concatenate([np.linspace(-103.9, 88.7, 120001, dtype=np.float32),
                         np.random.default_rng(1).uniform(-20, 20, 40000).astype(np.float32),
                         np.float32([0.0, -0.0, 1e-8, -1e-8, 0.34657, -0.34657, 0.5, -0.5, 1.0, 88.0])])
    got = np.array([lib.or_exp(float(x)) for x in xs], np.float32)
    ref = np.exp(xs.astype(np.float64))
    # Error in units of the float result's spacing; subnormal results use the subnormal ulp.
    ulps = np.abs(got.astype(np.float64) - ref) / np.maximum(_ulp32(ref.astype(np.float32)), 2.0 ** -149)
    assert ulps.max() <= 2.0, (ulps.max(), xs[np.argmax(ulps)])


def test_exp_special_cases(orc):
    lib = orc.lib()
    assert lib.or_exp(0.0) == 1.0
    assert lib.or_exp(float("-inf")) == 0.0
    assert lib.or_exp(float("inf")) == float("inf")
    assert np.isnan(lib.or_exp(float("nan")))
    assert lib.or_exp(-105.0) == 0.0
    assert lib.or_exp(89.0) == float("inf")
    # Deep subnormal range is still monotone and non-negative.
    vals = [lib.or_exp(x) for x in np.linspace(-103.5, -87.0, 500)]
    assert all(b >= a for a, b in zip(vals, vals[1:])) and vals[0] >= 0.0


def _rand_floats(n, seed):
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    return f[np.isfinite(f)]


def test_f32_to_f16_matches_ieee_cast(orc):
    lib = orc.lib()
    xs = np.concatenate([
        _rand_floats(20000, 2),
        np.random.default_rng(3).uniform(-70000, 70000, 5000).astype(np.float32),
        np.random.default_rng(4).uniform(-1e-4, 1e-4, 5000).astype(np.float32),   # f16 subnormals
        np.float32([65504, 65519.99, 65520, -65520, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 2 ** -14, 0.0, -0.0]),
    ])
    got = np.array([lib.or_f32_to_f16(float(x)) for x in xs], np.uint16)
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)
    back = np.array([lib.or_f16_to_f32(int(h)) for h in ref], np.float32)
    assert np.array_equal(back, ref.view(np.float16).astype(np.float32))


def test_half_sat_definition(orc):
    lib = orc.lib()
    sub = np.uint32([0x00000001, 0x007FFFFF, 0x80000001, 0x80400000]).view(np.float32)
    for x in sub:  # F32 subnormals (either sign) -> +0
        assert lib.or_half_sat(float(x)) == 0x0000
    assert lib.or_half_sat(float("nan")) == 0x7E00
    assert lib.or_half_sat(70000.0) == 0x7BFF and lib.or_half_sat(-70000.0) == 0xFBFF
    assert lib.or_half_sat(65519.0) == 0x7BFF
    assert lib.or_half_sat(float("inf")) == 0x7BFF and lib.or_half_sat(float("-inf")) == 0xFBFF
    assert lib.or_half_sat(-0.0) == 0x8000
    xs = np.random.default_rng(5).uniform(-60000, 60000, 3000).astype(np.float32)
    got = np.array([lib.or_half_sat(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, xs.astype(np.float16).view(np.uint16))


def test_silu_sigmoid_against_float64(orc):
    lib = orc.lib()
    xs = np.concatenate([np.linspace(-30, 30, 6001), [0.0, 1e-6, -1e-6]]).astype(np.float32)
    x64 = xs.astype(np.float64)
    sil = np.array([lib.or_silu(float(x)) for x in xs], np.float32)
    sig = np.array([lib.or_sigmoid(float(x)) for x in xs], np.float32)
    sil_ref = x64 / (1.0 + np.exp(-x64))
    sig_ref = 1.0 / (1.0 + np.exp(-x64))
    assert (np.abs(sil - sil_ref) <= 4 * np.maximum(_ulp32(sil_ref), 2.0 ** -149)).all()
    assert (np.abs(sig - sig_ref) <= 4 * np.maximum(_ulp32(sig_ref), 2.0 ** -149)).all()
