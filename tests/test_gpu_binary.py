"""cbx_binary (ggml_add / ggml_mul with the second operand repeated),
cbx_bias_residual (two ggml_adds in one pass), cbx_scale (ggml_scale) and
cbx_concat (ggml_concat)
against the oracle's add / mul (ggml's repeat by
index) and numpy's concatenate: one f32 rounding per element, so bit-exact;
a concat is a copy."""
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


# torch shapes (ggml ne reversed): a, then b repeating into it
SHAPES = [
    ((500, 256), (500, 256)),     # residual join, same shape
    ((500, 256), (256,)),         # a bias along the channels
    ((500, 256), (500, 1)),       # the per-frame mask of a (C, T) tensor
    ((500, 320), (500, 1)),
    ((3, 40, 12), (40, 1)),       # mask repeated over a batch
    ((2, 6, 10), (1, 3, 5)),      # repeats along every axis
    ((7, 13), (1, 13)),           # odd widths (the row path)
    ((5, 6, 7, 8), (1, 1, 7, 1)),
    ((1024,), (1024,)),           # vectors (the time embedding)
    ((250, 8, 64), (1, 8, 64)),   # pos_bias over the query heads (a flat period of 512)
    ((3, 5, 8, 12), (1, 1, 8, 12)),
    ((3, 5, 8, 12), (1, 5, 8, 12)),
    ((6, 8, 12), (1, 8, 1)),      # a leading-dim period with a 1 inside: the row map
]


@pytest.mark.parametrize("op", [0, 1])
@pytest.mark.parametrize("sa,sb", SHAPES)
def test_binary_repeat_shapes(cbx, oracle, op, sa, sb):
    a = W.normal(W.seed_of(40, len(sa)), sa, 0.0, 2.0)
    b = W.normal(W.seed_of(41, len(sb)), sb, 0.5, 1.5)
    got = host(cbx.binary(op, dev(a), dev(b)))
    exp = oracle.add(a, b) if op == cbx.BINARY_ADD else oracle.mul(a, b)
    assert_bitexact(got, exp, f"op {op} {sa} by {sb}")


@pytest.mark.parametrize("sx,sb,su", [
    ((250, 8, 64), (1, 8, 64), (1, 8, 64)),    # q's bias (re-described over the heads), pos_bias_u / v
    ((500, 8, 64), (1, 1, 64), (1, 8, 64)),
    ((7, 3, 10), (1, 3, 10), (1, 1, 10)),      # rows of 10: the row map
    ((4, 6, 8), (4, 1, 8), (1, 6, 1)),         # repeats inside: the row map
])
def test_bias_add_pair(cbx, oracle, sx, sb, su):
    """cbx_bias_add_pair: (x + bias) + u and (x + bias) + v, bit-exact to the
    oracle's two adds in ggml's order."""
    x = W.normal(W.seed_of(44, sx[0]), sx, 0.0, 2.0)
    b = W.normal(W.seed_of(45, sx[0]), sb, 0.0, 0.5)
    u = W.normal(W.seed_of(46, sx[0]), su, 0.0, 0.5)
    v = W.normal(W.seed_of(47, sx[0]), su, 0.0, 0.5)
    yu, yv = cbx.bias_add_pair(dev(x), dev(b), dev(u), dev(v))
    s = oracle.add(x, b)
    assert_bitexact(host(yu), oracle.add(s, u), f"{sx} + u")
    assert_bitexact(host(yv), oracle.add(s, v), f"{sx} + v")


def test_bias_add_pair_strided_and_refusals(cbx, oracle):
    """x a column slice of a wider buffer (the row map), and the refusals:
    outputs that overlap an input or each other, operands that do not
    repeat."""
    base = W.normal(W.seed_of(48, 0), (30, 80), 0.0, 1.0)
    b, u, v = (W.normal(W.seed_of(48, k), (64,), 0.0, 1.0) for k in (1, 2, 3))
    x = dev(base)[:, 8:72]
    yu, yv = cbx.bias_add_pair(x, dev(b), dev(u), dev(v))
    s = oracle.add(np.ascontiguousarray(base[:, 8:72]), b)
    assert_bitexact(host(yu), oracle.add(s, u), "strided + u")
    assert_bitexact(host(yv), oracle.add(s, v), "strided + v")
    xt, bt, ut, vt = dev(base[:, :64]), dev(b), dev(u), dev(v)
    with pytest.raises(cbx.CbxError, match="overlaps an input"):
        cbx.bias_add_pair(xt, bt, ut, vt, out_u=xt)
    y = torch.zeros(30, 64, device="cuda")
    with pytest.raises(cbx.CbxError, match="yu and yv overlap"):
        cbx.bias_add_pair(xt, bt, ut, vt, out_u=y, out_v=y)
    with pytest.raises(cbx.CbxError, match="repeat"):
        cbx.bias_add_pair(xt, dev(np.zeros(48, np.float32)), ut, vt)


def test_binary_views_and_in_place(cbx, oracle):
    """Strided a, b and y (column slices of wider buffers), and y == a."""
    base = W.normal(W.seed_of(42, 0), (60, 50), 0.0, 1.0)
    bb = W.normal(W.seed_of(42, 1), (60, 9), 0.0, 1.0)
    a = dev(base)[:, 3:43]
    m = dev(bb)[:, 2:3]                # (60, 1), rows 36 bytes apart
    yb = torch.full((60, 64), float("nan"), device="cuda")
    y = yb[:, 8:48]
    cbx.binary(cbx.BINARY_MUL, a, m, out=y)
    exp = oracle.mul(np.ascontiguousarray(base[:, 3:43]), np.ascontiguousarray(bb[:, 2:3]))
    assert_bitexact(host(y), exp, "strided mul")
    assert np.isnan(host(yb)[:, :8]).all() and np.isnan(host(yb)[:, 48:]).all(), "only y's columns written"
    t = dev(base)
    r = dev(W.normal(W.seed_of(42, 2), (60, 50), 0.0, 1.0))
    cbx.binary(cbx.BINARY_ADD, t, r, out=t)
    assert_bitexact(host(t), oracle.add(base, host(r)), "in place")


def test_binary_refusals(cbx):
    a = torch.zeros((6, 10), device="cuda")
    with pytest.raises(cbx.CbxError):
        cbx.binary(cbx.BINARY_ADD, a, torch.zeros((6, 3), device="cuda"))      # 10 % 3 != 0
    with pytest.raises(cbx.CbxError):
        cbx.binary(7, a, torch.zeros((10,), device="cuda"))                     # no such op
    with pytest.raises(cbx.CbxError):
        cbx.binary(cbx.BINARY_ADD, a, a[:, :5], out=a)                          # y overlaps b
    with pytest.raises(cbx.CbxError):
        cbx.binary(cbx.BINARY_ADD, a.half(), torch.zeros((10,), device="cuda").half())   # F32 only


# torch shapes: r, x repeating into r, bias repeating into x
BIAS_RESIDUAL = [
    ((500, 256), (500, 256), (256,)),     # a stack's last ff.2 output, its bias, the residual stream
    ((500, 256), (256,), (256,)),         # the time MLP's output broadcast over the frames
    ((500, 256), (1, 256), (256,)),
    ((2, 40, 12), (40, 12), (12,)),       # repeated over a batch
    ((7, 13), (7, 13), (1, 13)),          # odd widths (the row path)
    ((6, 12), (12,), (4,)),               # a bias shorter than x's row
    ((3, 8, 16), (1, 8, 1), (1, 1, 1)),
]


@pytest.mark.parametrize("sr,sx,sb", BIAS_RESIDUAL)
def test_bias_residual_shapes(cbx, oracle, sr, sx, sb):
    """r + (x + bias), the inner add rounded first: the two ggml adds the
    oracle runs one after the other."""
    r = W.normal(W.seed_of(46, len(sr)), sr, 0.0, 4.0)
    x = W.normal(W.seed_of(47, len(sx)), sx, 0.0, 3.0)
    b = W.normal(W.seed_of(48, len(sb)), sb, 0.5, 1.0)
    got = host(cbx.bias_residual(dev(x), dev(b), dev(r)))
    assert_bitexact(got, oracle.add(r, oracle.add(x, b)), f"{sr} {sx} {sb}")


def test_bias_residual_views_and_in_place(cbx, oracle):
    """Strided operands, y == r and y == x."""
    rb = W.normal(W.seed_of(49, 0), (60, 50), 0.0, 2.0)
    xb = W.normal(W.seed_of(49, 1), (60, 44), 0.0, 2.0)
    b = W.normal(W.seed_of(49, 2), (40,), 0.0, 1.0)
    yb = torch.full((60, 64), float("nan"), device="cuda")
    y = yb[:, 8:48]
    cbx.bias_residual(dev(xb)[:, 2:42], dev(b), dev(rb)[:, 5:45], out=y)
    exp = oracle.add(np.ascontiguousarray(rb[:, 5:45]), oracle.add(np.ascontiguousarray(xb[:, 2:42]), b))
    assert_bitexact(host(y), exp, "strided")
    assert np.isnan(host(yb)[:, :8]).all() and np.isnan(host(yb)[:, 48:]).all(), "only y's columns written"
    r = W.normal(W.seed_of(49, 3), (64, 40), 0.0, 2.0)
    x = W.normal(W.seed_of(49, 4), (64, 40), 0.0, 2.0)
    exp = oracle.add(r, oracle.add(x, b))
    t = dev(r)
    cbx.bias_residual(dev(x), dev(b), t, out=t)
    assert_bitexact(host(t), exp, "y is r")
    t = dev(x)
    cbx.bias_residual(t, dev(b), dev(r), out=t)
    assert_bitexact(host(t), exp, "y is x")


def test_bias_residual_refusals(cbx):
    r = torch.zeros((6, 12), device="cuda")
    b = torch.zeros((12,), device="cuda")
    with pytest.raises(cbx.CbxError):
        cbx.bias_residual(torch.zeros((6, 5), device="cuda"), torch.zeros((5,), device="cuda"), r)   # 12 % 5
    with pytest.raises(cbx.CbxError):
        cbx.bias_residual(torch.zeros((12,), device="cuda"), torch.zeros((6, 12), device="cuda"), r)  # bias into x
    with pytest.raises(cbx.CbxError):
        cbx.bias_residual(r, r[0], r, out=r)                                      # y overlaps bias
    x = torch.zeros((12,), device="cuda")
    with pytest.raises(cbx.CbxError):
        cbx.bias_residual(x, b, r, out=torch.zeros((6, 10), device="cuda"))       # y not r's shape
    with pytest.raises(cbx.CbxError):
        cbx.bias_residual(x.half(), b.half(), r.half())                           # F32 only


@pytest.mark.parametrize("shape", [(601, 64), (40, 256), (7, 13), (3, 5, 6, 2)])
def test_scale(cbx, shape):
    """ggml_scale: one f32 product per element, so numpy's f32 multiply is
    the whole reference; the resblock mean's 1/3 and a power of two."""
    x = W.normal(W.seed_of(50, len(shape)), shape, 0.0, 3.0)
    for s in (np.float32(1.0 / 3.0), np.float32(0.25), np.float32(-7.5)):
        assert_bitexact(host(cbx.scale(dev(x), float(s))), x * s, f"scale {shape} by {s}")


def test_scale_views_in_place_and_refusals(cbx):
    base = W.normal(W.seed_of(51, 0), (60, 50), 0.0, 1.0)
    yb = torch.full((60, 64), float("nan"), device="cuda")
    y = yb[:, 8:48]
    cbx.scale(dev(base)[:, 3:43], 1.0 / 3.0, out=y)
    assert_bitexact(host(y), base[:, 3:43] * np.float32(1.0 / 3.0), "strided")
    assert np.isnan(host(yb)[:, :8]).all() and np.isnan(host(yb)[:, 48:]).all(), "only y's columns written"
    t = dev(base)
    cbx.scale(t, 0.5, out=t)
    assert_bitexact(host(t), base * np.float32(0.5), "in place")
    with pytest.raises(cbx.CbxError):
        cbx.scale(t, 2.0, out=t[1:])                                          # y overlaps x otherwise
    with pytest.raises(cbx.CbxError):
        cbx.scale(t.half(), 2.0)                                              # F32 only


@pytest.mark.parametrize("dim", [0, 1, 2, 3])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_concat_dims(cbx, dim, dtype):
    sa = [2, 3, 4, 5]
    sb = list(sa)
    ax = 3 - dim
    sb[ax] = 2 + dim
    a = W.normal(W.seed_of(43, dim), tuple(sa), 0.0, 1.0).astype(dtype)
    b = W.normal(W.seed_of(44, dim), tuple(sb), 0.0, 1.0).astype(dtype)
    got = host(cbx.concat(dev(a), dev(b), dim))
    assert_bitexact(got, np.concatenate((a, b), axis=ax), f"concat dim {dim} {np.dtype(dtype).name}")


@pytest.mark.parametrize("sa,sb,dim", [((1, 64), (60000, 64), 1),      # the vocoder's one-frame pad
                                        ((500, 80), (500, 80), 0),      # the decoder's channel packing
                                        ((500, 256), (500, 256), 0),    # the skip join
                                        ((3, 7, 12), (3, 5, 12), 1),
                                        ((2, 3, 4, 8), (1, 3, 4, 8), 3)])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_concat_contiguous(cbx, sa, sb, dim, dtype):
    """Contiguous operands take the flat kernel, 16-byte vectors when every
    block is a multiple of 16 bytes, elements otherwise."""
    a = W.normal(W.seed_of(52, len(sa)), sa, 0.0, 1.0).astype(dtype)
    b = W.normal(W.seed_of(53, len(sb)), sb, 0.0, 1.0).astype(dtype)
    ax = a.ndim - 1 - dim
    got = host(cbx.concat(dev(a), dev(b), dim))
    assert_bitexact(got, np.concatenate((a, b), axis=ax), f"concat {sa} {sb} dim {dim} {np.dtype(dtype).name}")


def test_concat_channels_of_views(cbx):
    """The decoder's channel packing on (T, C) tensors, one operand a view."""
    x = W.normal(W.seed_of(45, 0), (500, 80), 0.0, 1.0)
    wide = W.normal(W.seed_of(45, 1), (500, 100), 0.0, 1.0)
    got = host(cbx.concat(dev(x), dev(wide)[:, 10:90], 0))
    assert_bitexact(got, np.concatenate((x, wide[:, 10:90]), axis=1), "pack")
    with pytest.raises(cbx.CbxError):
        cbx.concat(dev(x), dev(x[:10]), 0)                                      # other dims differ


@pytest.mark.parametrize("s0,s1,col", [((250, 512), (250, 512), False), ((500, 512), (37, 64), False),
                                       ((20, 30), (250, 512), False), ((40, 64), (12, 64), True)])
def test_bias_add_two(cbx, oracle, s0, s1, col):
    """cbx_bias_add_two: two independent bias adds in one launch, each
    bit-exact to the oracle's add; rows of 30 floats and a per-row bias
    (1, ne1) take the two-launch fallback."""
    x0 = W.normal(W.seed_of(50, s0[0]), s0, 0.0, 2.0)
    x1 = W.normal(W.seed_of(51, s1[0]), s1, 0.0, 2.0)
    b0 = W.normal(W.seed_of(52, s0[1]), (s0[1],), 0.0, 0.5)
    b1 = W.normal(W.seed_of(53, s1[1]), (s1[0], 1) if col else (s1[1],), 0.0, 0.5)
    y0, y1 = cbx.bias_add_two(dev(x0), dev(b0), dev(x1), dev(b1))
    assert_bitexact(host(y0), oracle.add(x0, b0), f"{s0}")
    assert_bitexact(host(y1), oracle.add(x1, b1), f"{s1}")


def test_bias_add_two_in_place_and_refusals(cbx, oracle):
    x0 = W.normal(W.seed_of(54, 0), (64, 128), 0.0, 1.0)
    x1 = W.normal(W.seed_of(54, 1), (64, 128), 0.0, 1.0)
    b = W.normal(W.seed_of(54, 2), (128,), 0.0, 1.0)
    t0, t1, tb = dev(x0), dev(x1), dev(b)
    cbx.bias_add_two(t0, tb, t1, tb, out0=t0, out1=t1)
    assert_bitexact(host(t0), oracle.add(x0, b), "y0 = x0")
    assert_bitexact(host(t1), oracle.add(x1, b), "y1 = x1")
    with pytest.raises(cbx.CbxError, match="overlaps the other"):
        cbx.bias_add_two(t0, tb, t1, tb, out0=t1)
    with pytest.raises(cbx.CbxError, match="ne = "):
        cbx.bias_add_two(t0, dev(np.zeros(64, np.float32)), t1, tb)
    wide = torch.zeros(65, 128, device="cuda")
    with pytest.raises(cbx.CbxError, match="its bias"):
        cbx.bias_add_two(t0, wide[63], t1, tb, out0=wide[:64])
