"""Pins of the CPU oracle (oracle/cbx_oracle.c) against independent facts.

Each oracle function is checked against something that does not share its
code: numpy's own float16 conversion and float32 arithmetic, float64
closed forms, exact invariants (power-of-two scale invariance, the identity
rotation at position 0, the NORMAL/NEOX pairing permutation), brute force on
tiny inputs, and the reference's own NumPy op texts (restated in float64).
A plausible slip (dropped term, wrong sign, swapped operand, wrong index)
fails at least one test here."""
import math

import numpy as np
import pytest

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import ATOL_X, assert_bitexact, assert_close

# --------------------------------------------------------------------------- #
# f16 conversion
# --------------------------------------------------------------------------- #


def test_fp16_to_fp32_all_codes(oracle):
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_fp32(int(c)) for c in codes], dtype=np.float32)
    assert_bitexact(got, ref, "f16->f32")


def test_fp32_to_fp16_matches_numpy(oracle):
    rng = np.random.default_rng(1)
    # random bit patterns over the whole f32 range, plus every f16 midpoint (ties) and its neighbours
    xs = [rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)]
    f = np.arange(0, 0x7c00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mid = ((f[:-1] + f[1:]) / 2).astype(np.float32)
    xs += [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0)), -mid]
    xs += [np.array([65504, 65519.99, 65520, 1e-8, 2.9802322e-08, 2.98023259e-08, -0.0, 0.0, np.inf, -np.inf],
                    dtype=np.float32)]
    x = np.concatenate(xs)
    x = x[~np.isnan(x)]
    got = np.array([oracle.fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref), int((got != ref).sum())


# --------------------------------------------------------------------------- #
# Q8_0
# --------------------------------------------------------------------------- #


def _q8_blocks(d_codes, rng):
    rows = []
    for d in d_codes:
        blk = bytearray(int(d).to_bytes(2, "little"))
        blk += rng.integers(-128, 128, 32).astype(np.int8).tobytes()
        rows.append(np.frombuffer(bytes(blk), dtype=np.uint8))
    return np.concatenate(rows).reshape(1, -1)


def test_q8_0_dequant_closed_form(oracle):
    rng = np.random.default_rng(2)
    d_codes = [0x3C00, 0x1400, 0x0001, 0x8000, 0x7BFF, 0x0400, 0x3555, 0xBC00] + list(rng.integers(0, 0x7c00, 24))
    q = _q8_blocks(d_codes, rng)
    got = oracle.dequantize_q8_0(q)
    blocks = q.reshape(-1, 34)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32)
    qs = blocks[:, 2:].view(np.int8).astype(np.float32)
    ref = (qs * d).astype(np.float32).reshape(1, -1)
    assert_bitexact(got, ref, "dequant")


def test_workload_q8_0_tables_match_the_oracle_quantizer(oracle):
    """The synthetic Q8_0 tables of the workloads come from the same rule."""
    x = W.normal(W.seed_of(5, 0), (300, 1024), 0.0, 0.02)
    x[0, :32] = 0.0                     # an all-zero block: d = 0
    assert np.array_equal(W.quantize_q8_0(x), oracle.quantize_q8_0(x))


def test_q8_0_quantize_rule_and_roundtrip(oracle):
    x = W.normal(3, (16, 1024), 0.0, 0.02)
    x[0, :32] = 0.0
    x[1, :32] = np.linspace(-1, 1, 32, dtype=np.float32)
    q = oracle.quantize_q8_0(x)
    blocks = q.reshape(-1, 34)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(blocks[:, :2].copy().view(np.float16).reshape(-1), d.astype(np.float16))
    inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    x0 = (xb * inv[:, None]).astype(np.float32).astype(np.float64)
    qref = np.where(x0 >= 0, np.floor(x0 + 0.5), np.ceil(x0 - 0.5))          # roundf: half away from zero
    assert np.array_equal(blocks[:, 2:].view(np.int8).astype(np.float64), qref)
    back = oracle.dequantize_q8_0(q).reshape(-1, 32)
    dh = blocks[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
    # |q*dh - x| <= |q*d - x| + |q| |dh - d| <= d/2 + 127 |dh - d|  (plus f32 rounding)
    bound = 0.5 * d * 1.001 + 127.0 * np.abs(dh - d) + 1e-12
    assert np.all(np.abs(back - xb) <= bound[:, None])


# --------------------------------------------------------------------------- #
# GELU table
# --------------------------------------------------------------------------- #


def _gelu64(x):
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def test_gelu_table_against_float32_emulation(oracle):
    """Every finite entry equals numpy's op-by-op float32 evaluation of
    0.5x(1 + tanh(sqrt(2/pi) x (1 + 0.044715 x x))) with a correctly rounded
    tanh, then f16 rounding -- independent code, same formula and order."""
    tab = oracle.gelu_table(0)
    x = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    ok = np.isfinite(x)
    f = np.float32
    with np.errstate(all="ignore"):
        inner = (f(1.0) + (f(0.044715) * x) * x).astype(f)
        arg = ((f(0.79788456080286535587989211986876) * x) * inner).astype(f)
        t = np.tanh(arg.astype(np.float64)).astype(f)
        g = ((f(0.5) * x) * (f(1.0) + t)).astype(f)
    ref = g.astype(np.float16).view(np.uint16)
    assert np.array_equal(tab[ok], ref[ok])
    # away from the negative-tail cancellation the f32 formula is within one
    # f16 step of the exact function
    sel = ok & (x > -2.0) & (np.abs(x) > 1e-3)
    gf = tab[sel].view(np.float16).astype(np.float64)
    exact = _gelu64(x[sel])
    assert np.all(np.abs(gf - exact) <= np.abs(exact) * 2.0 ** -10 + 1e-7)
    # the ISO-C and FMA-contracted evaluations differ in at most a handful of codes
    assert int((oracle.gelu_table(1) != tab).sum()) < 16


def test_gelu_f32_clamps_and_lookup(oracle):
    x = np.array([-10.0, -9.999, 10.0, 9.999, -1e30, 1e30, 0.5, -0.5], dtype=np.float32)
    got = oracle.unary(oracle.GELU, x)
    tab = oracle.gelu_table(0)
    assert got[0] == 0.0 and got[2] == 10.0 and got[4] == 0.0 and got[5] == np.float32(1e30)
    for i in (1, 3, 6, 7):
        h = x[i:i + 1].astype(np.float16).view(np.uint16)[0]
        assert got[i] == tab[h:h + 1].view(np.float16).astype(np.float32)[0]


# --------------------------------------------------------------------------- #
# norms
# --------------------------------------------------------------------------- #


def _ln64(x, eps):
    x = x.astype(np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps)


@pytest.mark.parametrize("n", [1, 7, 80, 1024, 5120])
def test_norm_float64(oracle, n):
    x = W.normal(4 + n, (9, n), 0.3, 2.0)
    y = oracle.norm(x, 1e-5)
    ref = _ln64(x, 1e-5)
    assert np.max(np.abs(y - ref)) < 2e-6 * max(1.0, np.abs(ref).max())


def test_norm_invariants(oracle):
    x = W.normal(5, (4, 256))
    y = oracle.norm(x, 0.0)
    # power-of-two scaling is exact through every step when eps = 0
    assert_bitexact(oracle.norm(x * np.float32(8.0), 0.0), y, "scale invariance")
    assert np.allclose(y.astype(np.float64).mean(-1), 0, atol=1e-6)
    assert np.allclose((y.astype(np.float64) ** 2).mean(-1), 1, atol=1e-5)
    c = np.full((2, 100), -7.5, dtype=np.float32)
    assert not oracle.norm(c, 1e-5).any()


def test_layer_norm_affine_composition(oracle):
    x = W.normal(6, (5, 64))
    w = W.normal(7, (64,), 1.0, 0.5)
    b = W.normal(8, (64,), 0.0, 0.5)
    y = oracle.layer_norm(x, w, b, 1e-5)
    n = oracle.norm(x, 1e-5)
    assert_bitexact(y, (n * w).astype(np.float32) + b, "norm*w+b in f32")
    assert_bitexact(oracle.layer_norm(x, None, None, 1e-5), n, "no affine")


def test_rms_norm_float64_and_invariants(oracle):
    x = W.normal(9, (6, 1024))
    y = oracle.rms_norm(x, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-5)
    assert np.max(np.abs(y - ref)) < 2e-6
    assert_bitexact(oracle.rms_norm(x * np.float32(0.25), 0.0), oracle.rms_norm(x, 0.0), "scale invariance")
    g = W.normal(10, (1024,), 1.0, 0.1)
    assert_bitexact(oracle.rms_norm_mul(x, g, 1e-5), (y * g).astype(np.float32), "rms*g")


def test_rms_norm_f16_storage_rounds_once(oracle):
    x = W.normal(11, (3, 256)).astype(np.float16)
    g = W.normal(12, (256,), 1.0, 0.1)
    y = oracle.rms_norm_mul(x, g, 1e-5)
    ref = oracle.rms_norm_mul(x.astype(np.float32), g, 1e-5).astype(np.float16)
    assert_bitexact(y, ref, "f16 = round(f32 result)")


def test_group_norm_float64_and_one_group(oracle):
    x = W.normal(13, (2, 12, 3, 10), 1.0, 3.0)     # ggml ne (10, 3, 12, 2): channels 12
    y = oracle.group_norm(x, 4, 1e-5)
    xd = x.astype(np.float64).reshape(2, 4, -1)
    ref = ((xd - xd.mean(-1, keepdims=True)) / np.sqrt(xd.var(-1, keepdims=True) + 1e-5)).reshape(x.shape)
    assert np.max(np.abs(y - ref)) < 3e-6
    y1 = oracle.group_norm(x, 1, 1e-5).reshape(2, -1)
    assert np.max(np.abs(y1 - oracle.norm(x.reshape(2, -1), 1e-5))) < 1e-6
    # ceil split: 10 channels in 3 groups -> 4, 4, 2
    x2 = W.normal(14, (1, 10, 1, 8))
    y2 = oracle.group_norm(x2, 3, 1e-5)
    for lo, hi in ((0, 4), (4, 8), (8, 10)):
        assert abs(float(y2[0, lo:hi].astype(np.float64).mean())) < 1e-6


def test_group_norm_affine_mish(oracle):
    x = W.normal(15, (1, 8, 1, 50))
    w = W.normal(16, (1, 8, 1, 1), 1.0, 0.2)
    b = W.normal(17, (1, 8, 1, 1), 0.0, 0.2)
    gn = oracle.group_norm(x, 2, 1e-5)
    aff = ((gn * w).astype(np.float32) + b).astype(np.float32)
    assert_bitexact(oracle.group_norm_affine(x, 2, 1e-5, w, b, False), aff, "affine per channel")
    m = oracle.group_norm_affine(x, 2, 1e-5, w, b, True)
    assert_close(m, _mish64(aff), x=aff, what="mish")


# --------------------------------------------------------------------------- #
# RoPE
# --------------------------------------------------------------------------- #


def test_rope_theta_recurrence_and_cache(oracle):
    """cache = (cos, sin) of theta_i = p * ts^i formed as an iterated f32 product."""
    ts = np.float32(oracle.theta_scale_f32(10000.0, 64))
    # powf(10000, -1/32) correctly rounded: float64 pow rounded to f32
    assert ts == np.float32(10000.0 ** (-2.0 / 64))
    for p in (0, 1, 29, 1999, 2047):
        cache = oracle.rope_cache(p, 64)
        th = np.float32(p)
        for i in range(32):
            c64, s64 = math.cos(float(th)), math.sin(float(th))
            assert abs(cache[2 * i] - c64) <= 1.2e-7 and abs(cache[2 * i + 1] - s64) <= 1.2e-7
            th = np.float32(th * ts)


def test_rope_identity_norms_and_float64(oracle):
    x = W.normal(18, (5, 3, 64))
    pos = np.array([0, 1, 7, 300, 2047], dtype=np.int32)
    y = oracle.rope_ext(x, pos, 64)
    assert_bitexact(y[0], x[0], "position 0")
    n0 = x[..., :32].astype(np.float64) ** 2 + x[..., 32:].astype(np.float64) ** 2
    n1 = y[..., :32].astype(np.float64) ** 2 + y[..., 32:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)
    for t, p in enumerate(pos):
        cache = oracle.rope_cache(int(p), 64).astype(np.float64)
        c, s = cache[0::2], cache[1::2]
        x0, x1 = x[t, :, :32].astype(np.float64), x[t, :, 32:].astype(np.float64)
        ref = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
        # two f32 products and one sum: within 2^-22 (|x0| + |x1|)
        mag = np.concatenate([np.abs(x0) + np.abs(x1)] * 2, axis=-1)
        assert np.all(np.abs(y[t] - ref) <= 2.0 ** -22 * mag)


def test_rope_normal_is_permuted_neox(oracle):
    """NORMAL pairs (2i, 2i+1), NEOX pairs (i, i + n/2): the same rotation up to a permutation."""
    x = W.normal(19, (7, 2, 64))
    pos = np.arange(7, dtype=np.int32) * 5
    perm = np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)])   # interleaved -> halves
    y_normal = oracle.rope_ext(x, pos, 64, mode=0)
    y_neox = oracle.rope_ext(np.ascontiguousarray(x[..., perm]), pos, 64, mode=2)
    assert_bitexact(np.ascontiguousarray(y_normal[..., perm]), y_neox, "pairing permutation")


def test_rope_partial_dims_copy_tail(oracle):
    x = W.normal(20, (3, 2, 64))
    y = oracle.rope_ext(x, np.array([3, 4, 5], dtype=np.int32), 16)
    assert_bitexact(y[..., 16:], x[..., 16:], "tail")


def test_rope_matches_reference_numpy_form_small_positions(oracle):
    """scripts/reference_s3_encoder.py:110-127 (pow-based freqs, textbook
    half-split) agrees with ggml's iterated form where theta is small."""
    T, H, D = 12, 4, 64
    x = W.normal(21, (T, H, D))
    freqs = 1.0 / (10000.0 ** (np.arange(0, D, 2).astype(np.float32) / D))
    ang = np.outer(np.arange(T).astype(np.float32), freqs)
    cos, sin = np.cos(ang), np.sin(ang)
    cf = np.concatenate([cos, cos], -1)[:, None, :]
    sf = np.concatenate([sin, sin], -1)[:, None, :]
    rot = np.concatenate([-x[..., D // 2:], x[..., :D // 2]], -1)
    ref = x * cf + rot * sf
    y = oracle.rope_ext(x, np.arange(T, dtype=np.int32), D)
    assert np.max(np.abs(y - ref)) < 2e-5


def test_rope_yarn_corr_dims(oracle):
    import ctypes

    L = oracle.lib()
    dims = np.zeros(2, dtype=np.float32)
    L.cbxo_rope_yarn_corr_dims(128, 4096, 10000.0, 32.0, 1.0, dims.ctypes.data)

    def cd(beta):
        return 128 * math.log(4096 / (beta * 2 * math.pi)) / (2 * math.log(10000.0))

    assert dims[0] == max(0.0, math.floor(cd(32.0))) and dims[1] == min(127.0, math.ceil(cd(1.0)))
    del ctypes


# YaRN (Peng et al. 2023, "YaRN: Efficient Context Window Extension of Large
# Language Models"): each rotary pair mixes the extrapolated angle (the
# position's own) with the interpolated one (freq_scale times it) by a ramp
# that is 1 (no interpolation) for high-frequency pairs below the low
# correction dim and 0 above the high one, linear in between, and the
# magnitude is scaled by 1 + 0.1 ln(1 / freq_scale).  The oracle's cache is
# checked against these properties, not against its own formula.

def _corr(oracle, n_dims, n_ctx, base, beta_fast, beta_slow):
    dims = np.zeros(2, dtype=np.float32)
    oracle.lib().cbxo_rope_yarn_corr_dims(n_dims, n_ctx, base, beta_fast, beta_slow, dims.ctypes.data)
    return dims


def _angles(cache):
    c, s = cache[0::2].astype(np.float64), cache[1::2].astype(np.float64)
    return np.arctan2(s, c), np.hypot(c, s)


def _theta64(p, n_dims, base):
    return p * base ** (-2.0 * np.arange(n_dims // 2) / n_dims)


@pytest.mark.parametrize("fs", [0.25, 0.5, 0.125])
def test_rope_yarn_full_extrapolation_and_interpolation(oracle, fs):
    n, base, ctx, p, attn = 64, 10000.0, 4096, 3, 1.5
    m = attn * (1.0 + 0.1 * math.log(1.0 / fs))
    th = _theta64(p, n, base)
    tol = lambda t: (np.arange(n // 2) + 2) * 2.0 ** -22 * np.abs(t) + 1e-6  # noqa: E731
    # every pair below the low correction dim: pure extrapolation
    lo = _corr(oracle, n, ctx, base, 0.01, 0.001)
    assert lo[0] >= n // 2
    ang, mag = _angles(oracle.rope_cache(p, n, base, fs, 1.0, attn, ctx, 0.01, 0.001))
    assert np.all(np.abs(ang - th) <= tol(th)) and np.allclose(mag, m, rtol=1e-6)
    # correction dims at 0: pair 0 extrapolates, all others interpolate
    hi = _corr(oracle, n, ctx, base, 1000.0, 1000.0)
    assert hi[0] == 0 and hi[1] <= 0
    ang, mag = _angles(oracle.rope_cache(p, n, base, fs, 1.0, attn, ctx, 1000.0, 1000.0))
    exp = np.concatenate([th[:1], fs * th[1:]])
    assert np.all(np.abs(ang - exp) <= tol(exp)) and np.allclose(mag, m, rtol=1e-6)
    # ext_factor 0: plain interpolation, magnitude attn_factor alone
    ang, mag = _angles(oracle.rope_cache(p, n, base, fs, 0.0, attn, ctx, 0.01, 0.001))
    assert np.all(np.abs(ang - fs * th) <= tol(fs * th)) and np.allclose(mag, attn, rtol=1e-6)


@pytest.mark.parametrize("ext", [1.0, 0.5])
def test_rope_yarn_ramp_is_linear_between_correction_dims(oracle, ext):
    n, base, ctx, p, fs = 128, 10000.0, 4096, 1, 0.25
    bf, bs = 32.0, 1.0
    low, high = (float(v) for v in _corr(oracle, n, ctx, base, bf, bs))
    assert 0 < low < high < n // 2 - 1
    ang, _ = _angles(oracle.rope_cache(p, n, base, fs, ext, 1.0, ctx, bf, bs))
    th = _theta64(p, n, base)
    mix = (ang - fs * th) / (th - fs * th)     # 1 = extrapolated angle, 0 = interpolated
    i = np.arange(n // 2)
    # mixes well resolved (angles above 1e-3 rad): the mix is ext below the
    # low dim, 0 above the high dim, and falls linearly in between
    ok = (th - fs * th) > 1e-3
    assert np.allclose(mix[ok & (i <= low)], ext, atol=1e-3)
    assert np.allclose(mix[ok & (i >= high)], 0.0, atol=1e-3)
    mid = ok & (i > low) & (i < high)
    assert mid.sum() >= 4
    slope = np.diff(mix[mid])
    assert np.all(slope < 0) and np.allclose(slope, -ext / (high - low), atol=2e-3)


def test_rope_freq_factors_divide_the_position(oracle):
    """A power-of-two freq factor 2^k on pair i makes that pair's angle the
    one of position p / 2^k, exactly (the iterated f32 angle scales by 2^k
    without rounding), with or without YaRN; so the factor divides, and
    pair i reads factor i."""
    n, base, p = 64, 10000.0, 96
    k = np.array([(3 * i) % 6 for i in range(n // 2)])
    ff = (2.0 ** k).astype(np.float32)
    for fs, ext in ((1.0, 0.0), (0.25, 1.0)):
        kw = dict(freq_base=base, freq_scale=fs, ext_factor=ext, n_ctx_orig=4096, beta_fast=32.0, beta_slow=1.0)
        got = oracle.rope_cache(p, n, freq_factors=ff, **kw)
        for i in range(n // 2):
            plain = oracle.rope_cache(p // 2 ** int(k[i]), n, **kw)
            assert_bitexact(got[2 * i:2 * i + 2], plain[2 * i:2 * i + 2], what=f"pair {i}, fs {fs}")
    ones = oracle.rope_cache(p, n, freq_factors=np.ones(n // 2, np.float32), freq_base=base)
    assert_bitexact(ones, oracle.rope_cache(p, n, freq_base=base), what="unit freq factors")


def test_rope_attn_factor_scales_exactly(oracle):
    x = W.normal(W.seed_of(31, 0), (5, 4, 64), 0.0, 1.0)
    pos = np.array([0, 7, 100, 513, 2047], dtype=np.int32)
    y1 = oracle.rope_ext(x, pos, 64, attn_factor=1.0)
    y2 = oracle.rope_ext(x, pos, 64, attn_factor=2.0)
    assert_bitexact(y2, 2.0 * y1, what="attn_factor 2")


# --------------------------------------------------------------------------- #
# activations
# --------------------------------------------------------------------------- #


def _mish64(x):
    x = np.asarray(x, dtype=np.float64)
    sp = np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))
    return x * np.tanh(sp)


CLOSED = {
    "SILU": lambda x: x / (1.0 + np.exp(-x)),
    "TANH": np.tanh,
    "SOFTPLUS": lambda x: np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20)))),
    "SIN": np.sin,
    "SQR": lambda x: x * x,
    "MISH": _mish64,
    "GELU_ERF": lambda x: 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0))),
}


@pytest.mark.parametrize("op", sorted(CLOSED))
def test_unary_float64(oracle, op):
    x = np.concatenate([W.normal(22, (20_001,), 0.0, 4.0),
                        np.array([0.0, 20.0, 20.5, -30.0, 1e-20], dtype=np.float32)])
    got = oracle.unary(getattr(oracle, op), x)
    ref = CLOSED[op](x.astype(np.float64))
    # f32 evaluation of the ggml formula vs the exact function: a few ulps,
    # plus the formula's own absolute floor where it cancels
    assert_close(got, ref, x=x, rtol=4e-7 if op != "MISH" else 1e-6, atol_x=ATOL_X, what=op)


def test_leaky_relu_exact(oracle):
    x = np.concatenate([W.normal(23, (1000,)), np.array([0.0, -0.0, np.nan, np.inf, -np.inf], dtype=np.float32)])
    for slope in (0.1, 0.01):
        got = oracle.leaky_relu(x, slope)
        with np.errstate(invalid="ignore"):
            ref = np.where(x > 0, x, np.float32(0)) + np.float32(slope) * np.where(x < 0, x, np.float32(0))
        assert_bitexact(got, ref.astype(np.float32), "leaky")
    assert oracle.leaky_relu(np.array([np.nan], dtype=np.float32), 0.1)[0] == 0.0


def test_swiglu_float64(oracle):
    g = W.normal(24, (3, 4096))
    u = W.normal(25, (3, 4096))
    got = oracle.swiglu(g, u)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    assert_close(got, gd / (1 + np.exp(-gd)) * ud, rtol=6e-7, what="swiglu")
    assert_bitexact(got, (oracle.unary(oracle.SILU, g) * u).astype(np.float32), "silu(g)*u")


def test_snake_float64_and_reference_form(oracle):
    """hift_vocoder.cpp:64-73 / reference_hift_vocoder.py:140-145."""
    C, T = 16, 300
    x = W.normal(26, (T, C), 0.0, 2.0)          # ggml (C, T): channel innermost
    a = W.uniform_range(27, (C,), 0.5, 1.5)
    ai = (1.0 / (a + np.float32(1e-9))).astype(np.float32)
    got = oracle.snake(x, a, ai)
    xd, ad = x.astype(np.float64), a.astype(np.float64)
    ref = xd + (1.0 / (ad + 1e-9)) * np.sin(xd * ad) ** 2
    assert_close(got, ref, x=x, rtol=1e-6, what="snake")
    z = oracle.snake(np.zeros((2, C), np.float32), a, ai)
    assert not z.any()
    # channel-outer layout: alpha of ne (1, C)
    xo = np.ascontiguousarray(x.T)
    got_o = oracle.snake(xo, a.reshape(C, 1), ai.reshape(C, 1))
    assert_bitexact(got_o, np.ascontiguousarray(got.T), "layouts agree")


# --------------------------------------------------------------------------- #
# gather, broadcast, cast
# --------------------------------------------------------------------------- #


def test_get_rows_numpy(oracle):
    tab = W.normal(28, (50, 33))
    ids = np.array([0, 49, 3, 3, 17], dtype=np.int32)
    assert_bitexact(oracle.get_rows(tab, ids), tab[ids], "f32")
    t16 = tab.astype(np.float16)
    assert_bitexact(oracle.get_rows(t16, ids), t16[ids].astype(np.float32), "f16")
    # batched: dst[:, i10, i11] = src[:, ids[i10, i11], i11]
    src = W.normal(29, (4, 6, 8))
    idb = W.randint(30, (4, 3), 0, 6)
    ref = np.stack([src[b][idb[b]] for b in range(4)])
    assert_bitexact(oracle.get_rows(src, idb), ref, "batched")
    with pytest.raises(ValueError):
        oracle.get_rows(tab, np.array([50], dtype=np.int32))


def test_get_rows_add_and_broadcast(oracle):
    inp = W.prefill_inputs()
    ids, pid = inp["ids"][:32], inp["pos_ids"][:32]
    got = oracle.get_rows_add(inp["table"], ids, inp["pos_table"], pid)
    assert_bitexact(got, inp["table"][ids] + inp["pos_table"][pid], "tok+pos")
    a = W.normal(31, (2, 3, 8))
    b = W.normal(32, (1, 3, 4))          # repeats along ne0 (x2) and ne2 (x2)
    assert_bitexact(oracle.add(a, b), a + np.tile(b, (2, 1, 2)), "add repeat")
    assert_bitexact(oracle.mul(a, b), a * np.tile(b, (2, 1, 2)), "mul repeat")


def test_cpy_numpy(oracle):
    x = W.normal(33, (10, 100), 0.0, 1e4)
    assert_bitexact(oracle.cpy(x, np.float16), x.astype(np.float16), "f32->f16")
    h = x.astype(np.float16)
    assert_bitexact(oracle.cpy(h, np.float32), h.astype(np.float32), "f16->f32")


def test_thread_count_does_not_change_results(oracle):
    x = W.normal(34, (37, 513))
    for fn in (lambda n: oracle.norm(x, 1e-5, nth=n), lambda n: oracle.unary(oracle.SILU, x, nth=n)):
        assert_bitexact(fn(1), fn(7), "threads")


# --------------------------------------------------------------------------- #
# attention epilogue: scale -> diag_mask_inf -> soft_max
# --------------------------------------------------------------------------- #

def _softmax64(x):
    """The reference's NumPy text (scripts/reference_t3_forward.py:87-89) in float64."""
    x = x.astype(np.float64)
    m = x.max(-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(-1, keepdims=True)


def test_scale_and_diag_mask_exact(oracle):
    x = W.normal(120, (2, 3, 5, 7))
    assert_bitexact(oracle.scale(x, 0.125), (x * np.float32(0.125)).astype(np.float32), "scale")
    m = oracle.diag_mask_inf(x, 2)
    i = np.arange(7)[None, :]
    j = np.arange(5)[:, None]
    masked = np.broadcast_to(i > 2 + j, x.shape)
    assert np.all(np.isneginf(m[masked])) and np.array_equal(m[~masked], x[~masked])


@pytest.mark.parametrize("n", [1, 2, 33, 500, 4097])
def test_soft_max_float64_and_invariants(oracle, n):
    x = W.normal(121 + n, (6, n), 0.0, 3.0)
    y = oracle.soft_max(x)
    assert np.max(np.abs(y - _softmax64(x))) < 4e-7
    assert np.allclose(y.astype(np.float64).sum(-1), 1.0, atol=2e-6)
    # a constant row gives exactly (float)(1.0 / n)
    c = np.full((3, n), 2.5, dtype=np.float32)
    assert_bitexact(oracle.soft_max(c), np.full((3, n), np.float32(1.0 / n)), "constant row")


def test_causal_attention_matches_reference_text(oracle):
    """scores/sqrt(Hd), triu(k=1) masked to -inf, softmax (reference_t3_forward.py:113-120)
    equals scale -> diag_mask_inf(n_past=0) -> soft_max; masked entries are exactly 0."""
    H, L, Hd = 4, 37, 64
    s = W.normal(122, (H, L, L), 0.0, 8.0)
    y = oracle.scale_diag_mask_soft_max(s, 1.0 / math.sqrt(Hd), 0)
    causal = np.triu(np.ones((L, L), dtype=bool), k=1)
    ref = _softmax64(np.where(causal[None], -np.inf, s.astype(np.float64) / math.sqrt(Hd)))
    assert np.max(np.abs(y - ref)) < 4e-7
    assert not y[:, causal].any()
    # incremental decode: one new query row after n_past cached keys sees every key
    q = W.normal(123, (H, 1, 50))
    y1 = oracle.scale_diag_mask_soft_max(q, 0.125, 49)
    assert_bitexact(y1, oracle.scale_diag_mask_soft_max(q, 0.125, -1), "n_past masks nothing")
    assert np.max(np.abs(y1 - _softmax64(q * np.float32(0.125)))) < 4e-7


# ---- conv1d (HiFT conv_1d_f32 with the fused prologue) ---------------------------

def _conv_brute(xh, wh, stride, pad, dil):
    """float64 brute force over f16-rounded operands: x [B, T, C], w [Co, C, K]."""
    B, T, C = xh.shape
    Co, _, K = wh.shape
    T_out = (T + 2 * pad - dil * (K - 1) - 1) // stride + 1
    out = np.zeros((B, T_out, Co))
    for t in range(T_out):
        for k in range(K):
            ti = t * stride + k * dil - pad
            if 0 <= ti < T:
                out[:, t, :] += xh[:, ti, :] @ wh[:, :, k].T
    return out


@pytest.mark.parametrize("stride,pad,dil", [(1, 2, 1), (1, 10, 5), (2, 3, 1), (15, 7, 1), (3, 0, 2)])
def test_conv1d_matches_brute_force(oracle, stride, pad, dil):
    """im2col semantics (tap k reads time t*stride + k*dil - pad, zero
    outside), f16 operands, exact products: against float64 brute force."""
    rng = np.random.default_rng(stride * 10 + dil)
    x = rng.standard_normal((2, 61, 12)).astype(np.float32)
    w = rng.standard_normal((8, 12, 5)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    got = oracle.conv1d(x, w, stride, pad, dil, bias=b)
    ref = _conv_brute(x.astype(np.float16).astype(np.float64), w.astype(np.float16).astype(np.float64), stride, pad,
                      dil)
    assert got.shape == ref.shape
    assert np.array_equal(got, (ref.astype(np.float32) + b).astype(np.float32))


def test_conv1d_identity_and_prologues(oracle):
    """K = 1 with the identity weight returns f16(pro(x)) exactly; the snake
    and leaky prologues equal the oracle's own snake / leaky_relu ops; the
    residual is added last (ggml_add(x, h))."""
    rng = np.random.default_rng(3)
    C = 16
    x = (rng.standard_normal((1, 40, C)) * 3).astype(np.float32)
    eye = np.eye(C, dtype=np.float32)[:, :, None]
    f16 = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
    assert np.array_equal(oracle.conv1d(x, eye), f16(x))
    a = rng.uniform(0.5, 1.5, C).astype(np.float32)
    ai = (np.float32(1) / (a + np.float32(1e-9))).astype(np.float32)
    assert np.array_equal(oracle.conv1d(x, eye, prologue=oracle.CONV_PRO_SNAKE, alpha=a, alpha_inv=ai),
                          f16(oracle.snake(x, a, ai)))
    assert np.array_equal(oracle.conv1d(x, eye, prologue=oracle.CONV_PRO_LEAKY, slope=0.1),
                          f16(oracle.leaky_relu(x, 0.1)))
    r = rng.standard_normal((1, 40, C)).astype(np.float32)
    bias = rng.standard_normal(C).astype(np.float32)
    assert np.array_equal(oracle.conv1d(x, eye, bias=bias, res=r), (r + (f16(x) + bias)).astype(np.float32))


def test_conv1d_f16_weights_equal_rounded_f32(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((30, 8)).astype(np.float32)
    w = rng.standard_normal((4, 8, 3)).astype(np.float32)
    assert np.array_equal(oracle.conv1d(x, w, pad=1), oracle.conv1d(x, w.astype(np.float16), pad=1))


# ---- conv_transpose1d (HiFT ups.i: ggml_conv_transpose_1d + crop + bias) ----------

@pytest.mark.parametrize("stride,K,pad", [(8, 16, 4), (5, 11, 3), (3, 7, 2), (1, 3, 1), (3, 2, 0), (4, 9, 0)])
def test_conv_transpose1d_matches_torch(oracle, stride, K, pad):
    """Against torch's conv_transpose1d in float64 on the same f16-rounded
    operands (weight [C_in, C_out, K], padding = the crop from each end):
    the HiFT upsamplers (8, 16, 4), (5, 11, 3), (3, 7, 2), stride 1, and a
    kernel shorter than the stride (outputs with no tap)."""
    import torch
    rng = np.random.default_rng(stride * 100 + K)
    x = rng.standard_normal((2, 23, 12)).astype(np.float32)
    w = rng.standard_normal((12, 8, K)).astype(np.float32)
    b = rng.standard_normal(8).astype(np.float32)
    got = oracle.conv_transpose1d(x, w, stride, pad, bias=b)
    xh = torch.from_numpy(x.astype(np.float16).astype(np.float64)).transpose(1, 2)
    wh = torch.from_numpy(w.astype(np.float16).astype(np.float64))
    ref = torch.nn.functional.conv_transpose1d(xh, wh, stride=stride, padding=pad).transpose(1, 2).numpy()
    assert got.shape == ref.shape == (2, 22 * stride + K - 2 * pad, 8)
    # the oracle rounds the f64 sum to f32 once, then adds the bias in f32
    assert np.array_equal(got, (ref.astype(np.float32) + b).astype(np.float32))


@pytest.mark.parametrize("stride,K,pad", [(8, 16, 4), (5, 11, 3), (2, 5, 1)])
def test_conv_transpose1d_is_the_adjoint_of_conv1d(oracle, stride, K, pad):
    """<convT_w(x), y> = <x, conv_w(y)>: the transposed conv is the adjoint
    of conv1d with the same array as its [C_out', C_in', K] weight, stride
    and padding.  f16-exact operands, so both sides are sums of the same
    exact products."""
    rng = np.random.default_rng(K)
    f16 = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
    x = f16(rng.standard_normal((17, 6)))
    w = f16(rng.standard_normal((6, 5, K)))
    T_out = 16 * stride + K - 2 * pad
    y = f16(rng.standard_normal((T_out, 5)))
    lhs = np.sum(oracle.conv_transpose1d(x, w, stride, pad).astype(np.float64) * y)
    cy = oracle.conv1d(y, w, stride, pad)
    assert cy.shape == x.shape
    rhs = np.sum(x.astype(np.float64) * cy)
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + 1.0)


def test_conv_transpose1d_repeat_and_prologue(oracle):
    """K = stride with w[ci][co][k] = (ci == co): every input row repeats
    stride times (nearest upsampling), then the crop; the leaky prologue is
    the oracle's leaky_relu, rounded to f16; F16 weights equal rounded F32."""
    rng = np.random.default_rng(9)
    C, s = 8, 5
    x = (rng.standard_normal((30, C)) * 2).astype(np.float32)
    w = np.repeat(np.eye(C, dtype=np.float32)[:, :, None], s, axis=2)
    f16 = lambda a: a.astype(np.float16).astype(np.float32)  # noqa: E731
    up = np.repeat(f16(x), s, axis=0)
    assert np.array_equal(oracle.conv_transpose1d(x, w, s, 0), up)
    assert np.array_equal(oracle.conv_transpose1d(x, w, s, 2), up[2:-2])
    assert np.array_equal(oracle.conv_transpose1d(x, w, s, 0, prologue=oracle.CONV_PRO_LEAKY, slope=0.1),
                          np.repeat(f16(oracle.leaky_relu(x, 0.1)), s, axis=0))
    w2 = rng.standard_normal((C, 4, 7)).astype(np.float32)
    assert np.array_equal(oracle.conv_transpose1d(x, w2, 3, 2), oracle.conv_transpose1d(x, w2.astype(np.float16), 3, 2))
