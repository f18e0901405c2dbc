"""cbx_scale_diag_mask_soft_max (scale -> diag_mask_inf -> soft_max over the
key axis) vs the oracle.  The exponentials come from the device libm, so
the bar is the f32 one (|d| <= 1e-5 |e|, plus a 1e-37 floor for outputs in
the f32 subnormal range); masked scores must come out exactly 0."""
import math

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def mask_of(shape, n_past):
    """True where diag_mask_inf hides key i from query j: i > n_past + j."""
    n_q, n_k = shape[-2], shape[-1]
    m = np.arange(n_k)[None, :] > n_past + np.arange(n_q)[:, None]
    return np.broadcast_to(m, shape) if n_past >= 0 else np.zeros(shape, dtype=bool)


def check(got, exp, what, masked=None):
    d = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = d > 1e-5 * np.abs(exp.astype(np.float64)) + 1e-37
    assert not bad.any(), f"{what}: {int(bad.sum())} of {got.size} off, max |d| {d.max():.3g}"
    if masked is not None:
        assert_bitexact(got[masked], np.zeros(int(masked.sum()), dtype=np.float32), f"{what}: masked")


def test_t3_prefill_causal(cbx, oracle):
    """[16 heads, 512 queries, 512 keys], scale 1/sqrt(64), causal (n_past 0)."""
    x = W.normal(130, (1, 16, 512, 512), 0.0, 8.0)
    got = host(cbx.scale_diag_mask_soft_max(dev(x), 1.0 / math.sqrt(64), 0))
    exp = oracle.scale_diag_mask_soft_max(x, 1.0 / math.sqrt(64), 0, nth=8)
    check(got, exp, "t3 prefill", mask_of(x.shape, 0))


@pytest.mark.parametrize("n_new,n_total", [(1, 777), (3, 100), (5, 4096), (2, 4097), (4, 9000)])
def test_t3_incremental(cbx, oracle, n_new, n_total):
    """New queries after n_past = n_total - n_new cached keys (t3.cpp:514-517)."""
    x = W.normal(131 + n_total, (16, n_new, n_total), 0.0, 6.0)
    n_past = n_total - n_new
    got = host(cbx.scale_diag_mask_soft_max(dev(x), 0.125, n_past))
    check(got, oracle.scale_diag_mask_soft_max(x, 0.125, n_past), f"t3 {n_new}x{n_total}",
          mask_of(x.shape, n_past))


def test_cfm_attention_no_mask(cbx, oracle):
    """CFM scores [2 (CFG pair), 8 heads, 500, 500], scale 1/8, no mask."""
    x = W.normal(132, (2, 8, 500, 500), 0.0, 4.0)
    got = host(cbx.scale_diag_mask_soft_max(dev(x), 0.125, -1))
    check(got, oracle.scale_diag_mask_soft_max(x, 0.125, -1, nth=8), "cfm")


@pytest.mark.parametrize("n", [1, 3, 4, 63, 64, 257, 1000, 4096])
def test_row_lengths_in_place_and_constant_rows(cbx, oracle, n):
    x = W.normal(133 + n, (7, n), 0.0, 10.0)
    x[0] = 1.5                     # constant row: exactly (float)(1/n)
    t = dev(x)
    cbx.scale_diag_mask_soft_max(t, 1.0, -1, out=t)
    got = host(t)
    check(got, oracle.scale_diag_mask_soft_max(x, 1.0, -1), f"n={n}")
    assert_bitexact(got[0], np.full(n, np.float32(1.0 / n)), "constant row")


@pytest.mark.parametrize("n", [300, 2000])
def test_few_rows_planes_not_at_one_stride(cbx, oracle, n):
    """Few rows whose planes are not one row stride apart (a slice of the
    rows and columns of a 3-D tensor): the decode kernels' row map, one wave
    a row up to 1024 columns and a workgroup a row past that."""
    base = W.normal(135 + n, (2, 5, n + 12), 0.0, 9.0)
    v = dev(base)[:, 1:4, 6:6 + n]
    exp = oracle.scale_diag_mask_soft_max(np.ascontiguousarray(base[:, 1:4, 6:6 + n]), 0.5, n - 3)
    got = host(cbx.scale_diag_mask_soft_max(v, 0.5, n - 3))
    check(got, exp, f"planes apart, n={n}", mask_of((2, 3, n), n - 3))


@pytest.mark.parametrize("shape,n_past", [((8, 250, 250), -1), ((20, 250, 250), 100), ((1500, 1023), 600),
                                          ((2, 700, 1021), 0), ((1100, 1025), 3), ((1100, 2046), 1000),
                                          ((1100, 2050), -1)])
def test_many_unaligned_rows(cbx, oracle, shape, n_past):
    """Many rows whose length is not a multiple of 4: a wave a row up to
    1024 columns (the 25 Hz conformer blocks' 250 keys), three passes past
    that."""
    x = W.normal(160 + shape[-1], shape, 0.0, 6.0)
    got = host(cbx.scale_diag_mask_soft_max(dev(x), 0.125, n_past))
    check(got, oracle.scale_diag_mask_soft_max(x, 0.125, n_past, nth=8), f"{shape}",
          mask_of(shape, n_past) if n_past >= 0 else None)


@pytest.mark.parametrize("c0", [2, 3])
def test_many_unaligned_rows_planes_apart(cbx, oracle, c0):
    """The same over a slice of a 3-D tensor (planes not one row stride
    apart): the row map, with rows at 8-byte steps (float2 loads, c0 2) or
    at 4-byte ones (c0 3)."""
    base = W.normal(170, (4, 300, 260), 0.0, 6.0)
    v = dev(base)[:, 10:290, c0:c0 + 250]
    exp = oracle.scale_diag_mask_soft_max(np.ascontiguousarray(base[:, 10:290, c0:c0 + 250]), 0.5, 7, nth=8)
    check(host(cbx.scale_diag_mask_soft_max(v, 0.5, 7)), exp, "planes apart", mask_of((4, 280, 250), 7))
    b = W.normal(171, (4, 280, 250), 0.0, 2.0)
    exp = oracle.scale_diag_mask_soft_max(oracle.add(np.ascontiguousarray(base[:, 10:290, c0:c0 + 250]), b), 0.5, -1,
                                          nth=8)
    check(host(cbx.add_scale_diag_mask_soft_max(v, dev(b), 0.5)), exp, "planes apart, with the added row")


def test_strided_rows_and_extremes(cbx, oracle):
    """A column-sliced view (rows at a stride, loop path) and large score gaps."""
    base = W.normal(134, (6, 300), 0.0, 30.0)
    v = dev(base)[:, 10:266]
    got = host(cbx.scale_diag_mask_soft_max(v, 2.0, 3))
    check(got, oracle.scale_diag_mask_soft_max(np.ascontiguousarray(base[:, 10:266]), 2.0, 3), "strided",
          mask_of((6, 256), 3))


@pytest.mark.parametrize("shape,n_past", [((8, 500, 500), -1), ((8, 250, 250), -1), ((8, 40, 40), -1),
                                          ((2, 3, 2000), 1990), ((6, 5000), 4000), ((1100, 37), 5),
                                          ((1, 8, 250, 252), -1)])
def test_add_scale_soft_max(cbx, oracle, shape, n_past):
    """cbx_add_scale_diag_mask_soft_max: the flow encoder's AC + BD scores
    ([8 heads, 2T, 2T] at T 250), few rows (one wave a row; a workgroup a
    row past 1024), rows past 4096 and rows of 37 (the three-pass kernel).
    The same bits as the plain epilogue over the sum rounded on the device,
    and within the f32 bar of the oracle's add -> scale -> soft_max."""
    a = W.normal(140 + shape[-1], shape, 0.0, 3.0)
    b = W.normal(141 + shape[-1], shape, 0.0, 3.0)
    ta, tb = dev(a), dev(b)
    got = host(cbx.add_scale_diag_mask_soft_max(ta, tb, 0.125, n_past))
    assert_bitexact(got, host(cbx.scale_diag_mask_soft_max(ta + tb, 0.125, n_past)), f"{shape}: fused vs sum")
    exp = oracle.scale_diag_mask_soft_max(oracle.add(a, b), 0.125, n_past, nth=8)
    check(got, exp, f"{shape}", mask_of(shape, n_past) if n_past >= 0 else None)


def test_add_scale_soft_max_in_place_and_strided(cbx, oracle):
    """y = a, y = b, and b a column slice of a wider tensor (rows at a
    stride, the row map)."""
    a = W.normal(150, (4, 64, 128), 0.0, 5.0)
    wide = W.normal(151, (4, 64, 160), 0.0, 5.0)
    b = np.ascontiguousarray(wide[..., 16:144])
    exp = oracle.scale_diag_mask_soft_max(oracle.add(a, b), 0.5, -1, nth=8)
    ta, tb = dev(a), dev(wide)[..., 16:144]
    check(host(cbx.add_scale_diag_mask_soft_max(ta, tb, 0.5)), exp, "strided b")
    cbx.add_scale_diag_mask_soft_max(ta, tb, 0.5, out=ta)
    check(host(ta), exp, "y = a")
    ta, tb = dev(a), dev(b)
    cbx.add_scale_diag_mask_soft_max(ta, tb, 0.5, out=tb)
    check(host(tb), exp, "y = b")


def test_add_scale_soft_max_refusals(cbx):
    a = torch.zeros(4, 64, device="cuda")
    with pytest.raises(cbx.CbxError, match="shapes differ"):
        cbx.add_scale_diag_mask_soft_max(a, torch.zeros(4, 32, device="cuda"))
    big = torch.zeros(5, 64, device="cuda")
    with pytest.raises(cbx.CbxError, match="overlap"):
        cbx.add_scale_diag_mask_soft_max(a, big[:4], out=big[1:])
