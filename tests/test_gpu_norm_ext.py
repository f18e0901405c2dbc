"""The LayerNorm's fused neighbours and the bias-add + activation entry
point, against the oracle evaluating the ggml nodes they replace one at a
time: cbx_add_layer_norm (residual join, t3.cpp:528-532), cbx_layer_norm_mask
(causal_block1d's LN -> Mish -> mask, cfm_decoder.cpp:143-148), cbx_bias_act
(t3.cpp:535-537, s3enc.cpp:176-177)."""
import ctypes

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ln_ref(oracle, s, w, b, eps):
    return oracle.add(oracle.mul(oracle.norm(s, eps), w), b)


@pytest.mark.parametrize("rows,D", [(1, 1024), (150, 1024), (37, 256), (9, 1000), (5, 4096), (3000, 512),
                                    (40, 64)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_add_layer_norm(cbx, oracle, rows, D, with_bias):
    """s = (a + bias) + r, y = LN(s)*w + b: both bit-exact.  3000 rows take
    the four-rows-per-workgroup launch."""
    sd = W.seed_of(20, rows * 7 + D)
    a = W.normal(sd, (rows, D), 0.0, 1.0)
    r = W.normal(sd + 1, (rows, D), 0.3, 2.0)
    ab = W.normal(sd + 2, (D,), 0.0, 0.1)
    w = W.normal(sd + 3, (D,), 1.0, 0.05)
    b = W.normal(sd + 4, (D,), 0.0, 0.05)
    s, y = cbx.add_layer_norm(dev(a), dev(r), dev(w), dev(b), 1e-5, a_bias=dev(ab) if with_bias else None)
    s_ref = oracle.add(oracle.add(a, ab) if with_bias else a, r)
    assert_bitexact(host(s), s_ref, f"sum {rows}x{D}")
    assert_bitexact(host(y), ln_ref(oracle, s_ref, w, b, 1e-5), f"LN(sum) {rows}x{D}")


@pytest.mark.parametrize("rows,D", [(250, 512), (500, 512), (7, 1024), (3000, 256)])
@pytest.mark.parametrize("store_sum", [True, False])
def test_bias_layer_norm(cbx, oracle, rows, D, store_sum):
    """r NULL: s = a + bias, y = LN(s)*w + b (the flow encoder's embed
    linears, flow_encoder.cpp:414-415), both bit-exact; r and a_bias both
    NULL is refused."""
    sd = W.seed_of(25, rows + D)
    a = W.normal(sd, (rows, D), 0.0, 1.0)
    ab = W.normal(sd + 1, (D,), 0.0, 0.1)
    w = W.normal(sd + 2, (D,), 1.0, 0.05)
    b = W.normal(sd + 3, (D,), 0.0, 0.05)
    s, y = cbx.add_layer_norm(dev(a), None, dev(w), dev(b), 1e-5, a_bias=dev(ab), store_sum=store_sum)
    s_ref = oracle.add(a, ab)
    if store_sum:
        assert_bitexact(host(s), s_ref, f"sum {rows}x{D}")
    assert_bitexact(host(y), ln_ref(oracle, s_ref, w, b, 1e-5), f"LN(a + bias) {rows}x{D}")
    with pytest.raises(cbx.CbxError, match="r may be NULL only"):
        cbx.add_layer_norm(dev(a), None, dev(w), dev(b), 1e-5)


@pytest.mark.parametrize("act", ["GELU", "MISH", "SILU"])
def test_add_layer_norm_activation(cbx, oracle, act):
    a = W.normal(21, (64, 512))
    r = W.normal(22, (64, 512))
    w = W.normal(23, (512,), 1.0, 0.1)
    b = W.normal(24, (512,), 0.0, 0.1)
    op = getattr(cbx, act)
    _, y = cbx.add_layer_norm(dev(a), dev(r), dev(w), dev(b), 1e-5, act=op, store_sum=False)
    ln = ln_ref(oracle, oracle.add(a, r), w, b, 1e-5)
    exp = oracle.unary(getattr(oracle, act), ln)
    if act == "GELU":
        assert_bitexact(host(y), exp, "add+LN+gelu")
    else:
        assert_close(host(y), exp, x=ln, what=f"add+LN+{act}")


def test_add_layer_norm_in_place_and_strided(cbx, oracle):
    """s written over r (the residual stream updated in place), rows of a
    read through a strided view."""
    D = 768
    big = W.normal(25, (30, 2 * D))
    r = W.normal(26, (30, D))
    w = W.normal(27, (D,), 1.0, 0.1)
    b = W.normal(28, (D,), 0.0, 0.1)
    a_dev = dev(big)[:, :D]                         # row stride 2*D floats
    r_dev = dev(r)
    s, y = cbx.add_layer_norm(a_dev, r_dev, dev(w), dev(b), 1e-5, s=r_dev)
    s_ref = oracle.add(np.ascontiguousarray(big[:, :D]), r)
    assert s is r_dev
    assert_bitexact(host(r_dev), s_ref, "sum in place over r")
    assert_bitexact(host(y), ln_ref(oracle, s_ref, w, b, 1e-5), "LN of strided a + r")
    # batch dims: (2, 5, D) rows enumerate ne1 then ne2
    a3 = W.normal(29, (2, 5, D))
    r3 = W.normal(30, (2, 5, D))
    _, y3 = cbx.add_layer_norm(dev(a3), dev(r3), None, None, 1e-6, store_sum=False)
    assert_bitexact(host(y3), oracle.norm(oracle.add(a3, r3), 1e-6), "3-D rows, no affine")


def test_add_layer_norm_errors(cbx):
    L = cbx.load()
    a = torch.zeros((4, 64), device="cuda")
    y = torch.zeros((4, 64), device="cuda")
    d = lambda t: ctypes.byref(cbx.desc(t))
    # s overlapping y
    rc = L.cbx_add_layer_norm(d(a), None, d(a), None, None, 1e-5, cbx.UNARY_NONE, d(y), d(y), None)
    assert rc == cbx.ERR_INVALID_ARG and "overlap" in cbx.last_error()
    # a row length the one-wave kernel does not take
    a2, y2 = torch.zeros((4, 66), device="cuda"), torch.zeros((4, 66), device="cuda")
    rc = L.cbx_add_layer_norm(d(a2), None, d(a2), None, None, 1e-5, cbx.UNARY_NONE, None, d(y2), None)
    assert rc == cbx.ERR_UNSUPPORTED
    # r with another shape
    rc = L.cbx_add_layer_norm(d(a), None, d(a2), None, None, 1e-5, cbx.UNARY_NONE, None, d(y), None)
    assert rc == cbx.ERR_INVALID_ARG
    # a bias that is not a row vector
    rc = L.cbx_add_layer_norm(d(a), d(a), d(a), None, None, 1e-5, cbx.UNARY_NONE, None, d(y), None)
    assert rc == cbx.ERR_UNSUPPORTED


@pytest.mark.parametrize("B,T,C", [(1, 500, 256), (2, 77, 512), (1, 3, 64)])
def test_layer_norm_mish_mask(cbx, oracle, B, T, C):
    x = W.normal(W.seed_of(31, T), (B, T, C), 0.1, 1.5)
    w = W.normal(W.seed_of(32, T), (C,), 1.0, 0.05)
    b = W.normal(W.seed_of(33, T), (C,), 0.0, 0.05)
    mask = (W.randint(W.seed_of(34, T), (T, 1), 0, 2)).astype(np.float32)
    mask[0, 0] = 0.5                                # not only 0/1
    ln = ln_ref(oracle, x, w, b, 1e-5)
    got = host(cbx.layer_norm_mask(dev(x), dev(w), dev(b), 1e-5, dev(mask), act=cbx.MISH))
    exp = oracle.mul(oracle.unary(oracle.MISH, ln), mask)
    assert_close(got, exp, x=ln, what=f"LN->mish->mask {B}x{T}x{C}")
    plain = host(cbx.layer_norm_mask(dev(x), dev(w), dev(b), 1e-5, dev(mask)))
    assert_bitexact(plain, oracle.mul(ln, mask), "LN->mask")


def test_layer_norm_mask_in_place(cbx, oracle):
    x = W.normal(35, (200, 256))
    w = W.normal(36, (256,), 1.0, 0.05)
    b = W.normal(37, (256,), 0.0, 0.05)
    mask = np.ones((200, 1), np.float32)
    xd = dev(x)
    cbx.layer_norm_mask(xd, dev(w), dev(b), 1e-5, dev(mask), out=xd)
    assert_bitexact(host(xd), ln_ref(oracle, x, w, b, 1e-5), "in place, mask of ones")


@pytest.mark.parametrize("act", ["UNARY_NONE", "GELU", "GELU_ERF", "SILU", "MISH"])
@pytest.mark.parametrize("shape", [(150, 4096), (3, 1024), (7, 75)])
def test_bias_act_inner(cbx, oracle, act, shape):
    """T3 fc (bias along ne0) with ggml_gelu; ragged rows take the row loop."""
    x = W.normal(W.seed_of(40, shape[1]), shape, 0.0, 2.0)
    bias = W.normal(W.seed_of(41, shape[1]), (shape[1],), 0.0, 0.5)
    got = host(cbx.bias_act(getattr(cbx, act), dev(x), dev(bias)))
    t = oracle.add(x, bias)
    if act == "UNARY_NONE":
        assert_bitexact(got, t, "bias add")
    elif act == "GELU":
        assert_bitexact(got, oracle.unary(oracle.GELU, t), "bias + gelu")
    else:
        assert_close(got, oracle.unary(getattr(oracle, act), t), x=t, what=f"bias + {act}")


@pytest.mark.parametrize("T", [75, 100])
def test_bias_act_outer(cbx, oracle, T):
    """s3enc's (1, C) bias on a time-major (T along ne0) tensor, then gelu_erf
    (s3enc.cpp:117-120,176-177); T = 75 is not a multiple of 4 (row loop)."""
    D = 1280
    x = W.normal(W.seed_of(42, T), (D, T), 0.0, 2.0)
    bias = W.normal(W.seed_of(43, T), (D, 1), 0.0, 0.5)
    got = host(cbx.bias_act(cbx.GELU_ERF, dev(x), dev(bias)))
    t = oracle.add(x, bias)
    assert_close(got, oracle.unary(oracle.GELU_ERF, t), x=t, what=f"outer bias + gelu_erf T={T}")
    # a strided x takes the row loop too
    big = W.normal(W.seed_of(44, T), (D, 2 * T), 0.0, 2.0)
    xs = dev(big)[:, :T]
    got = host(cbx.bias_act(cbx.UNARY_NONE, xs, dev(bias)))
    assert_bitexact(got, oracle.add(np.ascontiguousarray(big[:, :T]), bias), "strided bias add")


def test_t3_block_graph(cbx, oracle):
    """A T3 block's element-wise nodes around its matmuls (t3.cpp:526-546,
    the matmul outputs given): three launches, results as the nodes one at a
    time."""
    N, D, F = 40, 1024, 4096
    sd = W.seed_of(45, 0)
    mm_out, h = W.normal(sd, (N, D)), W.normal(sd + 1, (N, D))
    out_b, ln_w, ln_b = W.normal(sd + 2, (D,), 0, .1), W.normal(sd + 3, (D,), 1, .1), W.normal(sd + 4, (D,), 0, .1)
    fc_mm, fc_b = W.normal(sd + 5, (N, F)), W.normal(sd + 6, (F,), 0, .1)
    proj_mm, proj_b = W.normal(sd + 7, (N, D)), W.normal(sd + 8, (D,), 0, .1)
    n_w, n_b = W.normal(sd + 9, (D,), 1, .1), W.normal(sd + 10, (D,), 0, .1)
    g = cbx.Graph()
    T = {k: g.tensor(dev(v)) for k, v in dict(mm_out=mm_out, h=h, out_b=out_b, ln_w=ln_w, ln_b=ln_b, fc_mm=fc_mm,
                                                fc_b=fc_b, proj_mm=proj_mm, proj_b=proj_b, n_w=n_w, n_b=n_b).items()}
    bd = {k: torch.full((N, D), float("nan"), device="cuda") for k in ("cur", "res", "n", "m", "ln2", "pcur",
                                                                       "h2", "n2", "m2", "ln1")}
    bf = {k: torch.full((N, F), float("nan"), device="cuda") for k in ("fcb", "gelu")}
    t = {k: g.tensor(v) for k, v in {**bd, **bf}.items()}
    g.node(cbx.GOP_ADD, t["cur"], (T["mm_out"], T["out_b"]))
    g.node(cbx.GOP_ADD, t["res"], (t["cur"], T["h"]))
    g.node(cbx.GOP_NORM, t["n"], (t["res"],), fparam=1e-5)
    g.node(cbx.GOP_MUL, t["m"], (t["n"], T["ln_w"]))
    g.node(cbx.GOP_ADD, t["ln2"], (t["m"], T["ln_b"]))
    g.node(cbx.GOP_ADD, t["fcb"], (T["fc_mm"], T["fc_b"]))
    g.node(cbx.GOP_UNARY, t["gelu"], (t["fcb"],), iparam=cbx.GELU)
    g.node(cbx.GOP_ADD, t["pcur"], (T["proj_mm"], T["proj_b"]))
    g.node(cbx.GOP_ADD, t["h2"], (t["pcur"], t["res"]))
    g.node(cbx.GOP_NORM, t["n2"], (t["h2"],), fparam=1e-5)
    g.node(cbx.GOP_MUL, t["m2"], (t["n2"], T["n_w"]))
    g.node(cbx.GOP_ADD, t["ln1"], (t["m2"], T["n_b"]))
    keep = [t["ln2"], t["gelu"], t["h2"], t["ln1"]]
    assert [p[0] for p in g.plan(keep)] == [cbx.GL_ADD_LAYER_NORM, cbx.GL_BIAS_ACT, cbx.GL_ADD_LAYER_NORM]
    assert g.compute(keep) == 3

    res = oracle.add(oracle.add(mm_out, out_b), h)
    assert_bitexact(host(bd["res"]), res, "attn_residual")
    assert_bitexact(host(bd["ln2"]), ln_ref(oracle, res, ln_w, ln_b, 1e-5), "pre-FFN LN")
    assert_bitexact(host(bf["gelu"]), oracle.unary(oracle.GELU, oracle.add(fc_mm, fc_b)), "fc bias + gelu")
    h2 = oracle.add(oracle.add(proj_mm, proj_b), res)
    assert_bitexact(host(bd["h2"]), h2, "block output h")
    assert_bitexact(host(bd["ln1"]), ln_ref(oracle, h2, n_w, n_b, 1e-5), "next LN")
    for k in ("cur", "n", "m", "pcur", "n2", "m2"):
        assert np.isnan(host(bd[k])).all(), f"{k} is fused away"


def test_causal_block_tail_graph(cbx, oracle):
    T, C = 500, 256
    x = W.normal(46, (T, C), 0.1, 1.5)
    w, b = W.normal(47, (C,), 1.0, 0.05), W.normal(48, (C,), 0.0, 0.05)
    mask = np.ones((T, 1), np.float32)
    mask[-20:] = 0.0
    g = cbx.Graph()
    tx, tw, tb, tm = g.tensor(dev(x)), g.tensor(dev(w)), g.tensor(dev(b)), g.tensor(dev(mask))
    buf = [torch.full((T, C), float("nan"), device="cuda") for _ in range(7)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_NORM, t[0], (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, t[1], (t[0], tw))
    g.node(cbx.GOP_ADD, t[2], (t[1], tb))
    g.node(cbx.GOP_UNARY, t[3], (t[2],), iparam=cbx.SOFTPLUS)
    g.node(cbx.GOP_UNARY, t[4], (t[3],), iparam=cbx.TANH)
    g.node(cbx.GOP_MUL, t[5], (t[2], t[4]))
    g.node(cbx.GOP_MUL, t[6], (t[5], tm))
    assert g.compute() == 1
    ln = ln_ref(oracle, x, w, b, 1e-5)
    exp = oracle.mul(oracle.mul(ln, oracle.unary(oracle.TANH, oracle.unary(oracle.SOFTPLUS, ln))), mask)
    assert_close(host(buf[6]), exp, x=ln, what="causal_block1d tail nodes")
