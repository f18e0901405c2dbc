"""How far the ops built on the device's transcendentals (expf, logf,
tanhf, erff, sinf) land from the oracle (glibc's), measured at the
configurations' shapes and over every f16-representable input: the maximum
relative error, the share of bit-identical results, and how many elements
need the absolute floor 2^-22 |x| of the test bar because their error
exceeds 1e-5 |exp|.  Each measurement is printed (pytest -s shows the table)
and held to the bar of tests/_util.py; the relative part alone (1e-5, the
f32 tolerance of the path) is asserted for every op whose formula does not
cancel."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import ATOL_X, RTOL_F32, assert_close

pytestmark = pytest.mark.gpu

# The ops whose ggml formula cancels near some input (1 + erf(x/sqrt2) for
# x << 0, log(1 + e^x) for x << 0 and x*tanh(softplus(x)) after it): there
# the result is a small difference of O(1) terms, so an f32 evaluation
# carries an absolute error of a few ulps of the terms, not of the result.
CANCELS = {"GELU_ERF", "SOFTPLUS", "MISH"}


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stats(got, exp, x):
    g, e, xx = (np.asarray(a, dtype=np.float64).reshape(-1) for a in (got, exp, x))
    fin = np.isfinite(e) & np.isfinite(g)
    g, e, xx = g[fin], e[fin], xx[fin]
    d = np.abs(g - e)
    nz = e != 0
    rel = float(np.max(d[nz] / np.abs(e[nz]))) if nz.any() else 0.0
    exact = float(np.mean(np.asarray(got).reshape(-1)[fin].view(np.uint32) ==
                          np.asarray(exp).reshape(-1)[fin].view(np.uint32)))
    beyond = d > RTOL_F32 * np.abs(e)
    return rel, exact, int(beyond.sum()), int(g.size), float(np.max(d[beyond] / np.abs(xx[beyond]))) if beyond.any() else 0.0


def report(name, where, got, exp, x):
    rel, exact, n_floor, n, floor_ratio = stats(got, exp, x)
    print(f"\nLIBM {name:9s} {where:22s} max rel {rel:.3e}  bit-exact {100 * exact:7.3f}%  "
          f"beyond 1e-5 rel: {n_floor} of {n} (max |d|/|x| there {floor_ratio:.2e}, floor {ATOL_X:.2e})", flush=True)
    assert_close(got, exp, x=x, what=f"{name} {where}")
    if name not in CANCELS:
        assert n_floor == 0, f"{name} {where}: {n_floor} elements beyond 1e-5 relative"
    return rel, exact, n_floor


OPS = ["GELU_ERF", "SILU", "TANH", "SOFTPLUS", "SIN", "MISH"]


@pytest.mark.parametrize("op", OPS)
def test_config_shape(cbx, oracle, op):
    """[512,4096] of N(0,1) (the prefill FFN shape; the CFM estimator runs
    gelu_erf on (1024, T_mel) rows of the same magnitude)."""
    x = W.prefill_inputs()["ffn"]
    got = host(cbx.unary(getattr(cbx, op), dev(x)))
    exp = oracle.unary(getattr(oracle, op), x, nth=8)
    report(op, "[512,4096] N(0,1)", got, exp, x)


@pytest.mark.parametrize("op", OPS)
def test_every_f16_value(cbx, oracle, op):
    """Every finite f16-representable input as f32 (|x| up to 65504)."""
    codes = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    x = codes[np.isfinite(codes)]
    got = host(cbx.unary(getattr(cbx, op), dev(x)))
    exp = oracle.unary(getattr(oracle, op), x)
    report(op, "all f16 values", got, exp, x)


@pytest.mark.parametrize("shape", [(1, 6000, 256), (1, 48000, 128)])
def test_snake_stage_shapes(cbx, oracle, shape):
    """Snake x + sin^2(alpha x)/alpha at two vocoder stages (channel
    innermost, alpha ~ U(0.5, 1.5)): its own sin^2 against glibc's sinf."""
    B, T, Ch = shape
    x = W.normal(W.seed_of(4, 2), shape)
    a, ai = W.snake_alpha(Ch)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    exp = oracle.snake(x, a, ai, nth=8)
    report("SNAKE", f"[{B},{Ch},{T}]", got, exp, x)
