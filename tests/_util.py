"""Comparison helpers shared by the tests."""
from __future__ import annotations

import numpy as np

# Tolerances:
#   exact ops: bit-identical;
#   f32 norm / rope / activation: |got - exp| <= 1e-5 * |exp| + ATOL_X * |x|;
#   f16-stored tensors with f32 arithmetic: <= 2e-3 relative.
# ATOL_X = 2^-22 (4 f32 ulps of the input's magnitude) is the absolute floor
# of ops whose ggml formula itself cancels (1 + erf, log(1 + e^x)): there the
# result carries an absolute error of a few ulps of |x| in any f32
# evaluation, so no relative bound can hold near the cancellation.
RTOL_F32 = 1e-5
ATOL_X = 2.0 ** -22
RTOL_F16 = 2e-3


def bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return a.view({4: np.uint32, 2: np.uint16}[a.dtype.itemsize])


def assert_bitexact(got: np.ndarray, exp: np.ndarray, what: str = ""):
    got = np.asarray(got)
    exp = np.asarray(exp)
    assert got.shape == exp.shape, f"{what}: shape {got.shape} != {exp.shape}"
    assert got.dtype == exp.dtype, f"{what}: dtype {got.dtype} != {exp.dtype}"
    gn, en = np.isnan(got.astype(np.float32)), np.isnan(exp.astype(np.float32))
    assert np.array_equal(gn, en), f"{what}: NaN positions differ"
    diff = bits(got)[~gn] != bits(exp)[~en]
    n = int(diff.sum())
    if n:
        g, e = got[~gn][diff], exp[~en][diff]
        raise AssertionError(f"{what}: {n} of {got.size} elements differ; first got {g[:4]} expected {e[:4]}")


def rel_err(got: np.ndarray, exp: np.ndarray) -> float:
    g = np.asarray(got, dtype=np.float64)
    e = np.asarray(exp, dtype=np.float64)
    d = np.abs(g - e)
    return float(np.max(d / np.maximum(np.abs(e), 1e-30))) if d.size else 0.0


def assert_close(got, exp, x=None, rtol=RTOL_F32, atol_x=ATOL_X, what=""):
    """|got - exp| <= rtol |exp| + atol_x |x| elementwise (x: the op's input)."""
    g = np.asarray(got, dtype=np.float64)
    e = np.asarray(exp, dtype=np.float64)
    assert g.shape == e.shape, f"{what}: shape {g.shape} != {e.shape}"
    gn, en = np.isnan(g), np.isnan(e)
    assert np.array_equal(gn, en), f"{what}: NaN positions differ"
    g, e = g[~gn], e[~en]
    bound = rtol * np.abs(e)
    if x is not None:
        bound = bound + atol_x * np.abs(np.asarray(x, dtype=np.float64).reshape(-1)[~gn.reshape(-1)])
    d = np.abs(g - e)
    bad = d > bound
    if bad.any():
        i = int(np.argmax(d - bound))
        raise AssertionError(f"{what}: {int(bad.sum())} of {g.size} out of tolerance; worst got {g[i]!r} "
                             f"expected {e[i]!r} bound {bound[i]!r}")


def exact_fraction(got, exp) -> float:
    return float(np.mean(bits(np.asarray(got)) == bits(np.asarray(exp))))
