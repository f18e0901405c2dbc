"""cbx_conv_transpose1d (the HiFT upsamplers: leaky_relu -> ConvTranspose1d
-> crop -> + bias, hift_vocoder.cpp:96-115, 680-687) against the oracle's
conv_transpose1d on the same inputs.

Tolerance: both sides round the input (after the prologue) and the weights
to f16 and sum exact products -- the oracle in f64, the matrix cores in f32
in their own order -- so per output |got - ref| <= 2^-13 * sum |a_k b_k|
(the oracle's conv_transpose1d of |h| and |w|) + 2^-22 |ref|."""
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


def check(oracle, got, x, w, stride, pad, pro, slope, bias, what):
    ref = oracle.conv_transpose1d(x, w, stride, pad, pro, slope=slope, bias=bias, nth=8)
    h = oracle.leaky_relu(x, slope) if pro == oracle.CONV_PRO_LEAKY else x
    mag = oracle.conv_transpose1d(np.abs(h), np.abs(w), stride, pad, nth=8).astype(np.float64)
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = 2.0 ** -13 * mag + 2.0 ** -22 * np.abs(ref)
    assert got.shape == ref.shape, what
    bad = d > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {got.size} outside the bound; worst excess "
                           f"{float((d - bound).max()):.3g}")


def run(cbx, x, w, stride, pad, pro, slope, bias):
    wts = cbx.Conv1dWeights(dev(w), transpose_stride=stride)
    y = cbx.conv_transpose1d(dev(x), wts, pad, pro, None, None, slope, dev(bias) if bias is not None else None)
    got = host(y)
    wts.close()
    return got


UPS = [  # (C_in, C_out, stride, K, T_in): the three HiFT stages, pad = (K - stride) / 2
    (512, 256, 8, 16, 60), (256, 128, 5, 11, 200), (128, 64, 3, 7, 700)]


@pytest.mark.parametrize("C_in,C_out,s,K,T", UPS)
def test_hift_upsample(cbx, oracle, C_in, C_out, s, K, T):
    pad = (K - s) // 2
    sd = W.seed_of(12, s)
    x = W.normal(sd, (T, C_in), 0.0, 1.0)
    w = W.normal(sd + 1, (C_in, C_out, K), 0.0, 1.0 / np.sqrt(C_in * K / s))
    b = W.normal(sd + 2, (C_out,), 0.0, 0.1)
    got = run(cbx, x, w, s, pad, cbx.CONV_PRO_LEAKY_RELU, 0.1, b)
    check(oracle, got, x, w, s, pad, oracle.CONV_PRO_LEAKY, 0.1, b, f"ups {C_in}->{C_out} s{s} K{K}")


@pytest.mark.parametrize("s,K,pad,C_in,C_out", [(1, 3, 1, 64, 64), (3, 2, 0, 32, 40), (4, 9, 0, 48, 96),
                                                (2, 5, 3, 96, 33), (7, 7, 0, 40, 128)])
def test_strides_kernels_and_crops(cbx, oracle, s, K, pad, C_in, C_out):
    """Stride 1 (one phase: the taps reversed), a kernel shorter than the
    stride (phases with no tap: bias only), a crop larger than the phase
    count, channel counts off the tile sizes."""
    sd = W.seed_of(13, s * 10 + K)
    x = W.normal(sd, (311, C_in), 0.0, 1.0)
    w = W.normal(sd + 1, (C_in, C_out, K), 0.0, 0.2)
    b = W.normal(sd + 2, (C_out,), 0.0, 0.1)
    got = run(cbx, x, w, s, pad, cbx.CONV_PRO_NONE, 0.0, b)
    check(oracle, got, x, w, s, pad, oracle.CONV_PRO_NONE, 0.0, b, f"s{s} K{K} pad{pad}")


def test_batch_f16_weights_no_bias(cbx, oracle):
    x = W.normal(80, (3, 97, 64), 0.0, 1.0)
    w = W.normal(81, (64, 32, 11), 0.0, 0.1).astype(np.float16)
    got = run(cbx, x, w, 5, 3, cbx.CONV_PRO_LEAKY_RELU, 0.01, None)
    check(oracle, got, x, w, 5, 3, oracle.CONV_PRO_LEAKY, 0.01, None, "batch 3, f16 weights")


@pytest.mark.parametrize("C", [36, 34])
def test_strided_input_rows(cbx, oracle, C):
    big = W.normal(82, (150, 40))
    x = np.ascontiguousarray(big[:, :C])
    w = W.normal(83, (C, 64, 6), 0.0, 0.1)
    wts = cbx.Conv1dWeights(dev(w), transpose_stride=3)
    y = cbx.conv_transpose1d(dev(big)[:, :C], wts, 1, cbx.CONV_PRO_LEAKY_RELU, None, None, 0.1, None)
    check(oracle, host(y), x, w, 3, 1, oracle.CONV_PRO_LEAKY, 0.1, None, f"strided rows C{C}")
    wts.close()


def test_errors(cbx):
    L = cbx.load()
    d = lambda t: ctypes.byref(cbx.desc(t))  # noqa: E731
    wt = torch.zeros((32, 16, 6), device="cuda")       # torch [C_in, C_out, K]
    wts = cbx.Conv1dWeights(wt, transpose_stride=3)
    plain = cbx.Conv1dWeights(torch.zeros((16, 32, 3), device="cuda"))
    x = torch.zeros((10, 32), device="cuda")
    y = torch.zeros((9 * 3 + 6 - 2, 16), device="cuda")
    assert L.cbx_conv_transpose1d(d(x), wts.handle, 1, 0, None, None, 0.0, None, d(y), None) == cbx.OK, \
        cbx.last_error()
    bad_y = torch.zeros((9 * 3 + 6, 16), device="cuda")
    assert L.cbx_conv_transpose1d(d(x), wts.handle, 1, 0, None, None, 0.0, None, d(bad_y), None) == \
        cbx.ERR_INVALID_ARG
    # each handle kind is refused by the other entry point
    assert L.cbx_conv_transpose1d(d(x), plain.handle, 1, 0, None, None, 0.0, None, d(y), None) == \
        cbx.ERR_INVALID_ARG
    y1 = torch.zeros((8, 16), device="cuda")
    assert L.cbx_conv1d(d(x), wts.handle, 1, 0, 1, 0, None, None, 0.0, None, None, d(y1), None) == \
        cbx.ERR_INVALID_ARG
    # a crop that leaves nothing, a negative crop, a bad stride
    assert L.cbx_conv_transpose1d(d(x), wts.handle, 17, 0, None, None, 0.0, None, d(y), None) == \
        cbx.ERR_INVALID_ARG
    assert L.cbx_conv_transpose1d(d(x), wts.handle, -1, 0, None, None, 0.0, None, d(y), None) == \
        cbx.ERR_INVALID_ARG
    h = ctypes.c_void_p()
    assert L.cbx_conv_transpose1d_weights_create(d(wt), 0, None, ctypes.byref(h)) == cbx.ERR_INVALID_ARG
    wts.close()
    plain.close()


def test_input_channels_in_chunks(cbx, oracle):
    """2048 input channels: a 65-row window of all of them needs 267 KB, so
    the phases run in channel chunks."""
    x = W.normal(84, (200, 2048), 0.0, 1.0)
    w = W.normal(85, (2048, 64, 4), 0.0, 0.02)
    b = W.normal(86, (64,), 0.0, 0.1)
    got = run(cbx, x, w, 2, 1, cbx.CONV_PRO_LEAKY_RELU, 0.1, b)
    check(oracle, got, x, w, 2, 1, oracle.CONV_PRO_LEAKY, 0.1, b, "C_in 2048, s2 K4, chunked")
