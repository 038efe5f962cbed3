"""Pins the oracle's ops::rms_norm restatement (ggml_rms_norm + ggml_mul,
src/core/ops.hpp:76-80) with closed forms and invariants, not by retyping
its formula."""
import numpy as np
import pytest

import kd_oracle as orc


def test_known_vector_closed_form():
    # x = (3, 4, 0, ...): mean of squares 25/128, so y = x / sqrt(25/128 + eps)
    x = np.zeros((1, 128), np.float32)
    x[0, 0], x[0, 1] = 3.0, 4.0
    eps = 1e-6
    y = orc.rms_norm(x, None, eps)
    want = x / np.sqrt(25.0 / 128.0 + eps)
    np.testing.assert_allclose(y, want, rtol=2e-7, atol=0)


def test_constant_row_and_weight():
    # a constant row c normalises to c / sqrt(c^2 + eps); the weight scales each column
    w = np.linspace(-2.0, 2.0, 128, dtype=np.float32)
    for c in (1e-3, 0.5, 7.0, -123.0):
        x = np.full((1, 128), c, np.float32)
        y = orc.rms_norm(x, w, 1e-6)
        want = (c / np.sqrt(np.float64(c) ** 2 + 1e-6)) * w.astype(np.float64)
        np.testing.assert_allclose(y[0], want, rtol=3e-7, atol=1e-12)


def test_unit_rms_and_scale_invariance():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((64, 128)).astype(np.float32) * rng.uniform(0.01, 50, (64, 1)).astype(np.float32)
    y = orc.rms_norm(x, None, 0.0)
    ms = (y.astype(np.float64) ** 2).mean(axis=1)
    np.testing.assert_allclose(ms, 1.0, rtol=2e-6)
    # rms(a x) == rms(x) for a power of two (exact scaling in binary)
    y2 = orc.rms_norm(x * np.float32(8.0), None, 0.0)
    np.testing.assert_array_equal(y, y2)


def test_eps_dominates_tiny_rows():
    x = np.full((1, 128), 1e-6, np.float32)
    y = orc.rms_norm(x, None, 1e-6)
    np.testing.assert_allclose(y, 1e-6 / np.sqrt(1e-12 + 1e-6), rtol=1e-6)


def test_rows_independent_and_zero_row():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    x[1] = 0.0
    y = orc.rms_norm(x, None, 1e-6)
    np.testing.assert_array_equal(y[1], 0.0)
    np.testing.assert_array_equal(y[0], orc.rms_norm(x[0:1], None, 1e-6)[0])
    np.testing.assert_array_equal(y[2], orc.rms_norm(x[2:3], None, 1e-6)[0])


@pytest.mark.parametrize("mutate", ["no_sqrt", "sum_not_mean", "weight_before"])
def test_planted_mistakes_fail(mutate):
    """Plausible restatement mistakes, planted on the CPU, break the checks above."""
    x = np.zeros((1, 128), np.float32)
    x[0, 0], x[0, 1] = 3.0, 4.0
    w = np.linspace(0.5, 1.5, 128, dtype=np.float32)
    xd = x.astype(np.float64)
    if mutate == "no_sqrt":
        bad = xd / (25.0 / 128.0 + 1e-6)
    elif mutate == "sum_not_mean":
        bad = xd / np.sqrt(25.0 + 1e-6)
    else:
        bad = (xd * w) / np.sqrt(((xd * w) ** 2).mean() + 1e-6)
    good = orc.rms_norm(x, w, 1e-6)
    assert not np.allclose(good, bad, rtol=1e-4, atol=0)
