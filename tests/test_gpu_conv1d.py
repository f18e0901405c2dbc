"""cbx_conv1d (HiFT conv1d with the Snake / LeakyReLU prologue, bias and
residual fused) against the oracle's conv1d_CT restatement on the same
inputs: ResBlock convs at each stage's channel count, kernel size and
dilation (hift_vocoder.cpp:119-138), conv_pre, conv_post and the strided
source convs (:673, :713, :749).

Tolerance: both sides round the conv input and the weights to f16 and sum
exact products, the oracle in f64, the matrix cores in f32 in their own
order, so per output |got - ref| <= 2^-13 * sum_k |a_k b_k| (the sum of the
absolute products, computed by the oracle on |a|, |b|).  A Snake prologue
computed with the device's sinf can land on the other side of an f16
rounding boundary than glibc's for a few inputs; each such term moves by
2^-11 |a_k b_k|, inside the same bound."""
import ctypes

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def check(oracle, got, x, w, stride, pad, dil, pro, alpha, alpha_inv, slope, bias, res, what):
    ref = oracle.conv1d(x, w, stride, pad, dil, pro, alpha, alpha_inv, slope, bias, res, nth=8)
    if pro == oracle.CONV_PRO_SNAKE:
        h = oracle.snake(x, alpha, alpha_inv)
    elif pro == oracle.CONV_PRO_LEAKY:
        h = oracle.leaky_relu(x, slope)
    else:
        h = x
    mag = oracle.conv1d(np.abs(h), np.abs(w), stride, pad, dil, nth=8).astype(np.float64)
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = 2.0 ** -13 * mag + 2.0 ** -22 * np.abs(ref)
    bad = d > bound
    assert got.shape == ref.shape, what
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {got.size} outside the bound; worst excess "
                           f"{float((d - bound).max()):.3g} (d {float(d.max()):.3g})")


def check_sum(oracle, got, x, w, stride, pad, dil, pro, alpha, alpha_inv, slope, bias, res, acc, scale, what):
    """(acc + r) * scale against the oracle's conv r: the conv bound on r,
    scaled, plus the two f32 roundings of the sum and the scale
    (2^-22 |exp| covers both, one ulp of |exp| on each side)."""
    ref = oracle.conv1d(x, w, stride, pad, dil, pro, alpha, alpha_inv, slope, bias, res, nth=8)
    s = np.float32(scale)
    exp = oracle.add(acc, ref) * s if scale != 1.0 else oracle.add(acc, ref)
    if pro == oracle.CONV_PRO_SNAKE:
        h = oracle.snake(x, alpha, alpha_inv)
    elif pro == oracle.CONV_PRO_LEAKY:
        h = oracle.leaky_relu(x, slope)
    else:
        h = x
    mag = oracle.conv1d(np.abs(h), np.abs(w), stride, pad, dil, nth=8).astype(np.float64)
    d = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bound = abs(float(s)) * (2.0 ** -13 * mag + 2.0 ** -22 * np.abs(ref)) + 2.0 ** -22 * np.abs(exp)
    assert got.shape == exp.shape, what
    bad = d > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {got.size} outside the bound; worst excess "
                           f"{float((d - bound).max()):.3g}")


def case(oracle, C, T, C_out, K, stride, pad, dil, pro, with_bias=True, with_res=False, B=None, seed=0, w_f16=False,
         slope=0.1):
    sd = W.seed_of(11, seed)
    shape = (T, C) if B is None else (B, T, C)
    x = W.normal(sd, shape, 0.0, 1.0)
    w = W.normal(sd + 1, (C_out, C, K), 0.0, 1.0 / np.sqrt(C * K))
    if w_f16:
        w = w.astype(np.float16)
    alpha, alpha_inv = W.snake_alpha(C, seed + 2) if pro == oracle.CONV_PRO_SNAKE else (None, None)
    bias = W.normal(sd + 3, (C_out,), 0.0, 0.1) if with_bias else None
    T_out = (T + 2 * pad - dil * (K - 1) - 1) // stride + 1
    res = W.normal(sd + 4, shape[:-2] + (T_out, C_out), 0.0, 1.0) if with_res else None
    return x, w, alpha, alpha_inv, bias, res, slope


def run(cbx, x, w, stride, pad, dil, pro, alpha, alpha_inv, slope, bias, res, out=None):
    wts = cbx.Conv1dWeights(dev(w))
    opt = lambda a: dev(a) if a is not None else None  # noqa: E731
    y = cbx.conv1d(dev(x), wts, stride, pad, dil, pro, opt(alpha), opt(alpha_inv), slope, opt(bias), opt(res),
                   out=out)
    got = host(y)
    wts.close()
    return got


RESBLOCK = [  # (C, T, K, dilation): the three stages' channels with each kernel size
    (256, 300, 3, 1), (256, 301, 11, 5), (128, 800, 7, 3), (128, 777, 11, 1), (64, 2000, 11, 5), (64, 1500, 3, 3)]


@pytest.mark.parametrize("C,T,K,dil", RESBLOCK)
def test_resblock_snake_conv(cbx, oracle, C, T, K, dil):
    """snake -> conv (K, dilation, 'same' padding) + bias: a ResBlock's first conv."""
    pad = (K - 1) // 2 * dil
    x, w, al, ai, b, r, sl = case(oracle, C, T, C, K, 1, pad, dil, oracle.CONV_PRO_SNAKE, seed=C + K + dil)
    got = run(cbx, x, w, 1, pad, dil, cbx.CONV_PRO_SNAKE, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, pad, dil, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, f"C{C} T{T} K{K} d{dil}")


@pytest.mark.parametrize("C,T,K", [(256, 400, 11), (128, 640, 7), (64, 1000, 3)])
def test_resblock_second_conv_with_residual(cbx, oracle, C, T, K):
    """snake -> conv (K, dilation 1) + bias, then + x: the sublayer's output."""
    pad = (K - 1) // 2
    x, w, al, ai, b, r, sl = case(oracle, C, T, C, K, 1, pad, 1, oracle.CONV_PRO_SNAKE, with_res=True, seed=7 * K)
    got = run(cbx, x, w, 1, pad, 1, cbx.CONV_PRO_SNAKE, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, pad, 1, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, f"res C{C} K{K}")


def test_conv_pre_and_post(cbx, oracle):
    """conv_pre 80 -> 512 (k 7, p 3) and leaky_relu(0.01) -> conv_post 64 -> 18
    (hift_vocoder.cpp:673, :748-749): channel counts that are not multiples
    of the tiles."""
    x, w, al, ai, b, r, sl = case(oracle, 80, 250, 512, 7, 1, 3, 1, oracle.CONV_PRO_NONE, seed=31)
    got = run(cbx, x, w, 1, 3, 1, cbx.CONV_PRO_NONE, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, 3, 1, oracle.CONV_PRO_NONE, al, ai, sl, b, r, "conv_pre")
    x, w, al, ai, b, r, sl = case(oracle, 64, 3000, 18, 7, 1, 3, 1, oracle.CONV_PRO_LEAKY, seed=32, slope=0.01)
    got = run(cbx, x, w, 1, 3, 1, cbx.CONV_PRO_LEAKY_RELU, al, ai, 0.01, b, r)
    check(oracle, got, x, w, 1, 3, 1, oracle.CONV_PRO_LEAKY, al, ai, 0.01, b, r, "conv_post")


@pytest.mark.parametrize("stride,K,C_out", [(15, 7, 256), (3, 7, 128), (1, 11, 64)])
def test_source_down_convs(cbx, oracle, stride, K, C_out):
    """source_downs: 18 -> C_out with stride 15 / 3 / 1 (hift_vocoder.cpp:712-714)."""
    pad = 0 if stride == 1 else stride // 2
    x, w, al, ai, b, r, sl = case(oracle, 18, 1200, C_out, K, stride, pad, 1, oracle.CONV_PRO_NONE, seed=stride)
    got = run(cbx, x, w, stride, pad, 1, cbx.CONV_PRO_NONE, al, ai, sl, b, r)
    check(oracle, got, x, w, stride, pad, 1, oracle.CONV_PRO_NONE, al, ai, sl, b, r, f"src s{stride}")


def test_batch_f16_weights_no_bias_and_in_place_residual(cbx, oracle):
    x, w, al, ai, b, r, sl = case(oracle, 128, 333, 128, 7, 1, 9, 3, oracle.CONV_PRO_SNAKE, with_bias=False,
                                  with_res=True, B=3, seed=40, w_f16=True)
    wts = cbx.Conv1dWeights(dev(w))
    rd = dev(r)
    y = cbx.conv1d(dev(x), wts, 1, 9, 3, cbx.CONV_PRO_SNAKE, dev(al), dev(ai), sl, None, rd, out=rd)
    assert y is rd
    check(oracle, host(rd), x, w, 1, 9, 3, oracle.CONV_PRO_SNAKE, al, ai, sl, None, r, "batch 3, y == res")
    wts.close()


@pytest.mark.parametrize("C", [36, 34])
def test_strided_input_rows(cbx, oracle, C):
    """x rows read through a view with a larger row stride; 34 channels are
    not a multiple of 4, so the input is staged element by element."""
    big = W.normal(50, (400, 40))
    x = np.ascontiguousarray(big[:, :C])
    w = W.normal(51, (64, C, 3), 0.0, 0.1)
    b = W.normal(52, (64,), 0.0, 0.1)
    wts = cbx.Conv1dWeights(dev(w))
    y = cbx.conv1d(dev(big)[:, :C], wts, 1, 1, 1, cbx.CONV_PRO_LEAKY_RELU, None, None, 0.1, dev(b))
    check(oracle, host(y), x, w, 1, 1, 1, oracle.CONV_PRO_LEAKY, None, None, 0.1, b, None, f"strided rows C{C}")
    wts.close()


def test_hift_stage_shape(cbx, oracle):
    """A stage-2 ResBlock conv at full length: 64 channels, 24000 frames,
    K 11, dilation 5 (the oracle takes a few seconds)."""
    x, w, al, ai, b, r, sl = case(oracle, 64, 24000, 64, 11, 1, 25, 5, oracle.CONV_PRO_SNAKE, seed=60)
    got = run(cbx, x, w, 1, 25, 5, cbx.CONV_PRO_SNAKE, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, 25, 5, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, "64x24000 K11 d5")


@pytest.mark.parametrize("C,C_out,T,B", [(64, 64, 14362, 8), (64, 128, 3983, 16), (64, 128, 26196, 1),
                                         (64, 64, 8154, 4), (64, 512, 685, 16), (64, 64, 5050, 16),
                                         (64, 64, 3013, 16), (64, 64, 2000, 1)])
def test_tile_shapes(cbx, oracle, C, C_out, T, B):
    """Convs whose output counts pick each tile shape on a 256-CU device
    (256 x 64, 128 x 128, 64 x 128, 64 x 64 with KS 4, 96 x 128, 192 x 64,
    96 x 64 with KS 4, 32 x 64 with KS 4), Snake prologue, bias and
    residual."""
    x, w, al, ai, b, r, sl = case(oracle, C, T, C_out, 3, 1, 1, 1, oracle.CONV_PRO_SNAKE, with_res=True, B=B,
                                  seed=70 + C_out + T)
    got = run(cbx, x, w, 1, 1, 1, cbx.CONV_PRO_SNAKE, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, 1, 1, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, f"{B}x{C}x{T} -> {C_out}")


@pytest.mark.parametrize("C_in,C_out,T,B,with_mask", [(256, 256, 500, 1, True), (512, 256, 500, 1, True),
                                                      (80, 256, 377, 2, False), (256, 80, 500, 1, True)])
def test_cfm_causal_conv(cbx, oracle, C_in, C_out, T, B, with_mask):
    """CausalConv1d (cfm_decoder.cpp:89-120) after causal_block1d's pre-mask
    (:139): the oracle's conv1d of mask * x padded by K - 1 = 2 frames on
    both sides, first T outputs (output t reads inputs t - 2 .. t), within
    the conv tolerance."""
    K = 3
    sd = W.seed_of(15, C_in + C_out + T)
    shape = (T, C_in) if B == 1 else (B, T, C_in)
    x = W.normal(sd, shape)
    w = W.normal(sd + 1, (C_out, C_in, K), 0.0, 1.0 / np.sqrt(C_in * K))
    b = W.normal(sd + 2, (C_out,), 0.0, 0.1)
    mask = np.ones(T, dtype=np.float32)
    mask[T - T // 5:] = 0.0
    xm = (x * mask[:, None]).astype(np.float32) if with_mask else x
    ref = oracle.conv1d(xm, w, 1, K - 1, 1, oracle.CONV_PRO_NONE, None, None, 0.0, b, None, nth=8)[..., :T, :]
    mag = oracle.conv1d(np.abs(xm), np.abs(w), 1, K - 1, 1, nth=8)[..., :T, :].astype(np.float64)
    wts = cbx.Conv1dWeights(dev(w))
    got = host(cbx.causal_conv1d(dev(x), wts, dev(mask) if with_mask else None, dev(b)))
    wts.close()
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = 2.0 ** -13 * mag + 2.0 ** -22 * np.abs(ref)
    assert got.shape == ref.shape
    assert not (d > bound).any(), f"{int((d > bound).sum())} outside the bound"


def test_causal_conv_errors(cbx):
    L = cbx.load()
    d = lambda t: ctypes.byref(cbx.desc(t))  # noqa: E731
    wts = cbx.Conv1dWeights(torch.zeros((16, 32, 3), device="cuda"))
    x, y = torch.zeros((100, 32), device="cuda"), torch.zeros((100, 16), device="cuda")
    assert L.cbx_causal_conv1d(d(x), wts.handle, None, None, d(y), None) == cbx.OK, cbx.last_error()
    bad_mask = torch.ones(99, device="cuda")
    assert L.cbx_causal_conv1d(d(x), wts.handle, d(bad_mask), None, d(y), None) == cbx.ERR_INVALID_ARG
    assert "mask" in cbx.last_error()
    y_short = torch.zeros((98, 16), device="cuda")
    assert L.cbx_causal_conv1d(d(x), wts.handle, None, None, d(y_short), None) == cbx.ERR_INVALID_ARG
    buf = torch.zeros(1600, device="cuda")           # the mask is y's last 100 floats
    yv, mv = buf.view(100, 16), buf[1500:]
    assert L.cbx_causal_conv1d(d(x), wts.handle, d(mv), None, d(yv), None) == cbx.ERR_INVALID_ARG
    assert "overlap" in cbx.last_error()
    up = cbx.Conv1dWeights(torch.zeros((32, 16, 4), device="cuda"), transpose_stride=2)
    assert L.cbx_causal_conv1d(d(x), up.handle, None, None, d(y), None) == cbx.ERR_INVALID_ARG
    wts.close()
    up.close()


def test_errors(cbx):
    L = cbx.load()
    w = torch.zeros((16, 32, 3), device="cuda")
    wts = cbx.Conv1dWeights(w)
    d = lambda t: ctypes.byref(cbx.desc(t))  # noqa: E731
    x = torch.zeros((100, 32), device="cuda")
    y = torch.zeros((100, 16), device="cuda")
    ok = L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, 0, None, None, 0.0, None, None, d(y), None)
    assert ok == cbx.OK, cbx.last_error()
    bad_y = torch.zeros((99, 16), device="cuda")
    assert L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, 0, None, None, 0.0, None, None, d(bad_y), None) == \
        cbx.ERR_INVALID_ARG
    assert L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, cbx.CONV_PRO_SNAKE, None, None, 0.0, None, None, d(y), None) == \
        cbx.ERR_INVALID_ARG
    x16 = torch.zeros((100, 16), device="cuda")
    assert L.cbx_conv1d(d(x16), wts.handle, 1, 1, 1, 0, None, None, 0.0, None, None, d(y), None) == \
        cbx.ERR_INVALID_ARG
    # y overlapping x
    xy = torch.zeros((100, 32), device="cuda")
    assert L.cbx_conv1d(d(xy), wts.handle, 1, 1, 1, 0, None, None, 0.0, None, None, d(xy[:, :16]), None) == \
        cbx.ERR_INVALID_ARG
    assert L.cbx_conv1d(d(x), None, 1, 1, 1, 0, None, None, 0.0, None, None, d(y), None) == cbx.ERR_INVALID_ARG
    assert L.cbx_conv1d(d(x), wts.handle, 0, 1, 1, 0, None, None, 0.0, None, None, d(y), None) == \
        cbx.ERR_INVALID_ARG
    # bias, alpha, alpha_inv overlapping y; res overlapping y other than as y
    # itself (other workgroups' tile stores would race with their reads)
    buf = torch.zeros(1700, device="cuda")
    yb = buf[:1600].view(100, 16)
    assert L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, 0, None, None, 0.0, d(buf[1584:1600]), None, d(yb), None) == \
        cbx.ERR_INVALID_ARG
    assert "bias" in cbx.last_error()
    a32 = torch.ones(32, device="cuda")
    snake_y = torch.zeros(3300, device="cuda")
    ys = snake_y[:1600].view(100, 16)
    for al, ai in ((snake_y[:32], a32), (a32, snake_y[1590:1622])):
        assert L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, cbx.CONV_PRO_SNAKE, d(al), d(ai), 0.0, None, None, d(ys),
                            None) == cbx.ERR_INVALID_ARG
        assert "alpha" in cbx.last_error()
    shifted = buf[16:1616].view(100, 16)
    assert L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, 0, None, None, 0.0, None, d(shifted), d(yb), None) == \
        cbx.ERR_INVALID_ARG
    assert "res" in cbx.last_error()
    # res == y (same memory, same strides) is the documented in-place residual
    assert L.cbx_conv1d(d(x), wts.handle, 1, 1, 1, 0, None, None, 0.0, None, d(yb), d(yb), None) == cbx.OK
    torch.cuda.synchronize()
    wts.close()


def test_snake_large_arguments(cbx, oracle):
    """Arguments of sin at and past 2^16 (and just below) take the kernel's
    element-wise pass with the library sinf; all stay inside f16 after the
    prologue."""
    C, T, K = 64, 700, 3
    x = W.normal(70, (T, C), 0.0, 1.0)
    alpha = np.full(C, 5.0, np.float32)
    alpha[::3] = 0.5
    alpha_inv = (1.0 / alpha).astype(np.float32)
    x[::7, :] *= np.float32(3000.0)           # |x * alpha| ~ 1.5e4 .. 6e4
    x[5, :] = np.float32(13107.2)             # x * 5 = 65536 exactly
    x[6, :] = np.float32(13107.199)           # just below
    x[11, ::2] = np.float32(-20000.0)         # -1e5
    w = W.normal(71, (C, C, K), 0.0, 1.0 / np.sqrt(C * K))
    b = W.normal(72, (C,), 0.0, 0.1)
    got = run(cbx, x, w, 1, 1, 1, cbx.CONV_PRO_SNAKE, alpha, alpha_inv, 0.0, b, None)
    check(oracle, got, x, w, 1, 1, 1, oracle.CONV_PRO_SNAKE, alpha, alpha_inv, 0.0, b, None, "large sin arguments")


def test_snake_prologue_alone(cbx, oracle):
    """K = 1 with the identity weight: the conv returns the staged f16
    operand itself, f16(snake(x)), so this compares the kernel's snake
    (its own sin for |alpha x| < 2^16) with the oracle's glibc-sinf snake
    element by element.  Both round an f32 result to f16; they may differ
    by one f16 step where the f32 values straddle a rounding midpoint (the
    two sins differ by an f32 ulp or two): at most 1 in 10^4 elements, and
    never by more than one step."""
    C, T = 128, 4000
    x = W.normal(90, (T, C), 0.0, 2.0)
    alpha, alpha_inv = W.snake_alpha(C, 5)
    eye = np.eye(C, dtype=np.float32)[:, :, None]
    got = run(cbx, x, eye, 1, 0, 1, cbx.CONV_PRO_SNAKE, alpha, alpha_inv, 0.0, None, None)
    ref = oracle.snake(x, alpha, alpha_inv).astype(np.float16)
    g16 = got.astype(np.float16)
    assert np.array_equal(got, g16.astype(np.float32)), "identity conv output is not an f16 value"
    diff = g16 != ref
    d = np.abs(g16.astype(np.float64) - ref.astype(np.float64))
    step = np.spacing(np.maximum(np.abs(g16), np.abs(ref))).astype(np.float64)
    assert np.all(d[diff] <= step[diff]), "snake differs by more than one f16 step"
    assert diff.sum() <= x.size // 10000, f"{int(diff.sum())} of {x.size} f16 values differ"


def test_input_channels_in_chunks(cbx, oracle):
    """512 channels with K 11 dilation 15: the 64-frame tile's window (214
    rows) holds only 352 channels in 160 KiB of LDS, so the kernel runs two
    channel chunks (352 + 160), each staging its own snake alpha."""
    x, w, al, ai, b, r, sl = case(oracle, 512, 700, 512, 11, 1, 75, 15, oracle.CONV_PRO_SNAKE, with_res=True,
                                  seed=77)
    got = run(cbx, x, w, 1, 75, 15, cbx.CONV_PRO_SNAKE, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, 75, 15, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, "C512 K11 d15, two chunks")


def pipelined_tiles(C_in, C_out, T_out, B, K):
    """The launch runs k_conv1d_pipe when K >= 3, C_in % 64 == 0, C_out %
    64 == 0 and its tiles fill the CUs: C_out a multiple of 128 on 96 x 128
    tiles two a CU (a workgroup on every CU, 3/4 of every round's slots),
    else, with K >= 5, 192 x 128 tiles one a CU (at least half the CUs, 3/4
    of every round's slots), else 128 x 64 tiles two a CU when they give
    every CU a workgroup; other C_out on 128 x 64 tiles two a CU."""
    if not (K >= 3 and C_in % 64 == 0 and C_out % 64 == 0):
        return False
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    bc = 64 if C_out % 128 else 128

    def fills(bt, slots, need):
        items = -(-T_out // bt) * (C_out // bc) * (B or 1)
        return items >= need and 4 * items >= 3 * -(-items // slots) * slots

    if bc == 64:   # 128 x 64 tiles, two a CU, or k_conv1d
        return fills(128, 2 * n_cu, n_cu)
    if fills(96, 2 * n_cu, n_cu) or (K >= 5 and fills(192, n_cu, (n_cu + 1) // 2)):
        return True
    return -(-T_out // 128) * (C_out // 64) * (B or 1) >= n_cu   # 128 x 64 tiles on every CU


PIPE = [  # (C_in, C_out, T, B, K, dilation, prologue, residual)
    (128, 128, 48000, None, 11, 5, "SNAKE", False),   # the 128-channel stage's ResBlock conv 1, full length
    (128, 128, 48000, None, 11, 1, "SNAKE", True),    # a conv 2 with the residual, full length
    (64, 128, 300, 96, 11, 5, "LEAKY", False),        # one 64-channel chunk (the 4-deep ring), 96-row tiles
    (64, 128, 400, 64, 11, 5, "SNAKE", False),        # the same on 192-row tiles, a short last tile
    (256, 128, 400, 64, 7, 3, "NONE", True),          # four chunks, no prologue
    (64, 64, 120000, None, 11, 5, "SNAKE", False),    # the 64-channel stage's ResBlock conv 1, full length
    (64, 64, 120000, None, 11, 1, "SNAKE", True),     # its conv 2 with the residual
    (128, 128, 48000, None, 3, 1, "SNAKE", True),     # a K 3 conv with the residual, full length
    (64, 64, 120000, None, 3, 5, "LEAKY", False),     # a K 3 conv on the 128 x 64 tiles
    (128, 128, 400, 64, 5, 2, "SNAKE", False),        # the smallest K taken
    (128, 128, 20000, None, 11, 5, "SNAKE", False),   # 128 x 64 tiles for 128 channels (a 500-frame decode's stage)
    (128, 128, 20000, None, 3, 1, "SNAKE", True),     # the same at K 3 with the residual
]


@pytest.mark.parametrize("C,C_out,T,B,K,dil,pro,residual", PIPE)
def test_pipelined_kernel(cbx, oracle, C, C_out, T, B, K, dil, pro, residual):
    """Shapes that take the pipelined kernel (input channels staged in
    64-channel chunks by four waves while four others run the matrix
    cores): the ResBlock convs of the 48000-frame stage at full length,
    batches, one and four chunks, each prologue, bias and residual.  Snake
    inputs include arguments past 2^16 (the per-thread library-sinf pass)."""
    pad = (K - 1) // 2 * dil
    if not pipelined_tiles(C, C_out, T, B, K):
        pytest.skip("this device's CU count does not route the shape to the pipelined kernel")
    opro = getattr(oracle, f"CONV_PRO_{pro}")
    x, w, al, ai, b, r, sl = case(oracle, C, T, C_out, K, 1, pad, dil, opro, with_res=residual, B=B, seed=K + dil)
    if pro == "SNAKE":
        x[..., T // 3:T // 3 + 3, 5:9] = np.float32(30000.0)   # |x * alpha| in [15000, 45000]: the compact sin
        x[..., T // 2, :] = np.float32(-60000.0)              # past 2^16 where alpha > 1.09: the library sinf
    cpro = cbx.CONV_PRO_LEAKY_RELU if pro == "LEAKY" else getattr(cbx, f"CONV_PRO_{pro}")
    got = run(cbx, x, w, 1, pad, dil, cpro, al, ai, sl, b, r)
    check(oracle, got, x, w, 1, pad, dil, opro, al, ai, sl, b, r, f"pipelined C{C}->{C_out} T{T} B{B} K{K} d{dil}")


def test_pipelined_in_place_residual(cbx, oracle):
    """y == res on the pipelined kernel: each output is read and written by
    the thread that owns it."""
    C, T, B, K = 128, 400, 64, 7
    if not pipelined_tiles(C, C, T, B, K):
        pytest.skip("this device's CU count does not route the shape to the pipelined kernel")
    x, w, al, ai, b, r, sl = case(oracle, C, T, C, K, 1, 3, 1, oracle.CONV_PRO_SNAKE, with_res=True, B=B, seed=91)
    wts = cbx.Conv1dWeights(dev(w))
    rd = dev(r)
    y = cbx.conv1d(dev(x), wts, 1, 3, 1, cbx.CONV_PRO_SNAKE, dev(al), dev(ai), sl, dev(b), rd, out=rd)
    assert y is rd
    check(oracle, host(rd), x, w, 1, 3, 1, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, "pipelined y == res")
    wts.close()


SUM = [  # (C_in, C_out, T, B, K, dilation, scale): the conv kernels the sum rides on
    (256, 256, 400, None, 3, 1, 1.0 / 3.0),          # k_conv1d, float4 epilogue
    (128, 128, 48000, None, 11, 1, 1.0),             # k_conv1d_pipe (96 x 128 tiles), the sum alone
    (64, 128, 300, 96, 11, 5, 1.0 / 3.0),            # k_conv1d_pipe on a batch
    (64, 18, 500, None, 7, 1, 1.0 / 3.0),            # 18 channels out: the scalar epilogue
]


@pytest.mark.parametrize("C,C_out,T,B,K,dil,scale", SUM)
def test_conv1d_sum(cbx, oracle, C, C_out, T, B, K, dil, scale):
    """cbx_conv1d_sum: a ResBlock's last conv with the stage's sum and mean
    folded in, (acc + (res + conv)) * scale, against the oracle's conv, add
    and f32 scale."""
    pad = (K - 1) // 2 * dil
    x, w, al, ai, b, r, sl = case(oracle, C, T, C_out, K, 1, pad, dil, oracle.CONV_PRO_SNAKE, with_res=True, B=B,
                                  seed=K + 7)
    acc = W.normal(W.seed_of(12, K), r.shape, 0.0, 2.0)
    wts = cbx.Conv1dWeights(dev(w))
    got = host(cbx.conv1d_sum(dev(x), wts, 1, pad, dil, cbx.CONV_PRO_SNAKE, dev(al), dev(ai), 0.0, dev(b), dev(r),
                              dev(acc), scale))
    wts.close()
    check_sum(oracle, got, x, w, 1, pad, dil, oracle.CONV_PRO_SNAKE, al, ai, sl, b, r, acc, scale,
              f"sum C{C}->{C_out} T{T} B{B} K{K} d{dil} scale {scale}")


def test_conv1d_sum_refusals(cbx):
    x = dev(np.zeros((50, 16), np.float32))
    wts = cbx.Conv1dWeights(dev(np.zeros((16, 16, 3), np.float32)))
    y = torch.zeros((50, 16), device="cuda")
    with pytest.raises(cbx.CbxError, match="acc is NULL"):
        cbx.conv1d_sum(x, wts, 1, 1, 1, cbx.CONV_PRO_NONE, None, None, 0.0, None, None, None, 1.0, out=y)
    with pytest.raises(cbx.CbxError, match="acc must not overlap y"):
        cbx.conv1d_sum(x, wts, 1, 1, 1, cbx.CONV_PRO_NONE, None, None, 0.0, None, None, y, 1.0, out=y)
    with pytest.raises(cbx.CbxError, match="acc must be F32 with y's shape"):
        cbx.conv1d_sum(x, wts, 1, 1, 1, cbx.CONV_PRO_NONE, None, None, 0.0, None, None,
                       torch.zeros((49, 16), device="cuda"), 1.0, out=y)
    wts.close()
