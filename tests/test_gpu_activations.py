"""Activations through the C ABI vs the oracle.

Exact: GELU (fp16 table), LeakyReLU, SQR.  Device transcendentals (expf,
logf, tanhf, erff, sinf) are held to |d| <= 1e-5 |exp| + 2^-22 |x|."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import RTOL_F16, assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_prefill_gelu(cbx, oracle):
    """tanh-GELU over [512,4096] (fp16-table semantics): bit-exact."""
    x = W.prefill_inputs()["ffn"]
    assert_bitexact(host(cbx.gelu(dev(x))), oracle.unary(oracle.GELU, x, nth=8), "gelu")


def test_gelu_all_codes_and_edges(cbx, oracle):
    codes = np.arange(65536, dtype=np.uint16).view(np.float16)
    # f16 path: the table itself
    assert_bitexact(host(cbx.gelu(dev(codes))), oracle.unary(oracle.GELU, codes), "gelu f16 codes")
    # f32 path at every f16 value, the +-10 clamps, ties between f16 neighbours
    x = np.concatenate([codes.astype(np.float32),
                        np.array([-10.0, 10.0, np.nextafter(-10, 0), np.nextafter(10, 0), -1e30, 1e30,
                                  np.inf, -np.inf, 0.0, -0.0], dtype=np.float32),
                        W.normal(51, (4099,), 0.0, 4.0)])
    x = x[~np.isnan(x)]
    assert_bitexact(host(cbx.gelu(dev(x))), oracle.unary(oracle.GELU, x), "gelu f32 edges")


def test_gelu_large_all_codes(cbx, oracle):
    """A large tensor (full grid of workgroups): every f16 code as an f32
    input, shuffled, plus the clamps, in a ragged length."""
    codes = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    codes = codes[~np.isnan(codes)]
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.permutation(np.tile(codes, 5)),
                        np.array([-10.0, 10.0, np.nextafter(-10, 0), np.nextafter(10, 0), 9.9995, -9.9995, np.nan],
                                 dtype=np.float32),
                        W.normal(57, (1003,), 0.0, 6.0)])
    got = host(cbx.gelu(dev(x)))
    assert_bitexact(got, oracle.unary(oracle.GELU, x, nth=8), "gelu lds path")


OPS = ["GELU_ERF", "SILU", "TANH", "SOFTPLUS", "SIN", "MISH"]


@pytest.mark.parametrize("op", OPS)
def test_transcendental_ops(cbx, oracle, op):
    x = np.concatenate([W.normal(52, (200_003,), 0.0, 3.0),
                        np.array([0.0, -0.0, 20.0, np.nextafter(20, 0), 21.0, -20.0, -88.0, 88.0, 1e-30, -1e-30],
                                 dtype=np.float32)])
    got = host(cbx.unary(getattr(cbx, op), dev(x)))
    exp = oracle.unary(getattr(oracle, op), x)
    assert_close(got, exp, x=x, what=op)
    # f16 storage
    xh = x.astype(np.float16)
    goth = host(cbx.unary(getattr(cbx, op), dev(xh)))
    exph = oracle.unary(getattr(oracle, op), xh)
    assert_close(goth.astype(np.float32), exph.astype(np.float32), x=xh.astype(np.float32), rtol=RTOL_F16,
                 atol_x=2.0 ** -11, what=op + " f16")


def test_sqr_leaky_exact(cbx, oracle):
    x = np.concatenate([W.normal(53, (100_001,)), np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, -1e-40],
                                                           dtype=np.float32)])
    assert_bitexact(host(cbx.sqr(dev(x))), oracle.unary(oracle.SQR, x), "sqr")
    for slope in (0.1, 0.01):
        assert_bitexact(host(cbx.leaky_relu(dev(x), slope)), oracle.leaky_relu(x, slope), f"leaky {slope}")
    xn = np.array([np.nan, 1.0, -1.0], dtype=np.float32)
    got = host(cbx.leaky_relu(dev(xn), 0.1))
    assert_bitexact(got, oracle.leaky_relu(xn, 0.1), "leaky nan -> 0 as ggml")


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_swiglu(cbx, oracle, dtype):
    """SiLU(gate) * up: decode [1,4096] f32 and 64 streams [64,4096] f16."""
    n = 1 if dtype == np.float32 else 64
    g = W.normal(W.seed_of(1, 5) + n, (n, 4096)).astype(dtype)
    u = W.normal(W.seed_of(1, 6) + n, (n, 4096)).astype(dtype)
    got = host(cbx.swiglu(dev(g), dev(u)))
    exp = oracle.swiglu(g, u)
    rtol = 1e-5 if dtype == np.float32 else RTOL_F16
    assert_close(got.astype(np.float32), exp.astype(np.float32), rtol=rtol, what="swiglu")


@pytest.mark.parametrize("C,T", [(256, 6000), (128, 4800), (64, 12000), (36, 1001)])
def test_snake_channel_inner(cbx, oracle, C, T):
    """Reference layout (C, T): ne0 = C, alpha per channel along ne0."""
    x = W.normal(W.seed_of(4, 0) + C, (T, C))
    a = W.uniform_range(W.seed_of(4, 1) + C, (C,), 0.5, 1.5)
    ai = (1.0 / (a.astype(np.float32) + np.float32(1e-9))).astype(np.float32)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    assert_close(got, oracle.snake(x, a, ai, nth=8), x=x, what=f"snake inner {C}")


def test_snake_channel_outer_and_leaky(cbx, oracle):
    """Time-innermost layout [C, T]: alpha of ne (1, C)."""
    C, T = 64, 12001
    x = W.normal(W.seed_of(4, 2), (C, T))
    a = W.uniform_range(W.seed_of(4, 3), (C, 1), 0.5, 1.5)
    ai = (1.0 / (a + np.float32(1e-9))).astype(np.float32)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    assert_close(got, oracle.snake(x, a, ai), x=x, what="snake outer")
    assert_bitexact(host(cbx.leaky_relu(dev(x), 0.1)), oracle.leaky_relu(x, 0.1), "leaky")


def test_snake_zero_and_specials(cbx, oracle):
    """x = 0 gives 0; alpha broadcast over a batched tensor."""
    x = W.normal(54, (3, 40, 64))
    x[0, 0, :] = 0.0
    a = W.uniform_range(55, (64,), 0.5, 1.5)
    ai = (1.0 / (a + np.float32(1e-9))).astype(np.float32)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    assert not got[0, 0].any()
    assert_close(got, oracle.snake(x, a, ai), x=x, what="snake batch")


def test_snake_argument_range(cbx, oracle):
    """Snake's sin^2 across magnitudes from 2^-30 to 2^30 (the compact
    reduction below 2^16, the library sinf above), next to multiples of
    pi/2 (where sin^2 and cos^2 = 1 - sin^2 take turns), and at 0, +-Inf and
    NaN, against the oracle (glibc sinf)."""
    rng = np.random.default_rng(57)
    mag = np.exp2(rng.uniform(-30, 30, 20000))
    k = rng.integers(-40000, 40000, 20000)
    near = k * (np.pi / 2) + rng.uniform(-1e-3, 1e-3, 20000)
    x = np.concatenate([mag * rng.choice([-1.0, 1.0], 20000), near, [0.0, -0.0, np.inf, -np.inf, np.nan, 65535.9,
                        65536.0, -65536.0, 1e30, -3e38]]).astype(np.float32)
    x = x[: x.size // 64 * 64].reshape(-1, 64)
    a = W.uniform_range(58, (64,), 0.5, 1.5)
    ai = (1.0 / (a + np.float32(1e-9))).astype(np.float32)
    with np.errstate(invalid="ignore", over="ignore"):
        exp = oracle.snake(x, a, ai)
    got = host(cbx.snake(dev(x), dev(a), dev(ai)))
    fin = np.isfinite(x)
    assert_close(np.where(fin, got, 0), np.where(fin, exp, 0), x=np.where(fin, x, 0), what="snake range")
    assert np.array_equal(np.isnan(got), np.isnan(exp))


def test_non_contiguous_rows(cbx, oracle):
    big = W.normal(56, (50, 300))
    view = big[:, 7:263]
    got = host(cbx.silu(dev(big)[:, 7:263]))
    assert_close(got, oracle.unary(oracle.SILU, np.ascontiguousarray(view)), x=view, what="silu view")
    got = host(cbx.gelu(dev(big)[:, 7:263]))
    assert_bitexact(got, oracle.unary(oracle.GELU, np.ascontiguousarray(view)), "gelu view")
