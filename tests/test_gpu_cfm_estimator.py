"""One CFM estimator call's element-wise node list (cfm_decoder.cpp:395-558,
matmul outputs given; chatterbox_amdvulkan_amd/cfm_estimator.py) run launch
by launch, each launch checked against the oracle on the inputs it read
from the device: bit-exact for the adds, muls, concats and LayerNorms; the
f32 bar for the device-libm activations (SiLU, GELU-erf, Mish) and the
softmax; the conv bar for the causal convs (f16 operands, f32 sums).  Then
the whole list through cbx_graph_compute and a captured cbx_graph_exec:
the same output bits."""
import math

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.cfm_estimator import CFMEstimator
from tests._util import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def softmax_close(got, exp, what):
    d = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = d > 1e-5 * np.abs(exp.astype(np.float64)) + 1e-37
    assert not bad.any(), f"{what}: {int(bad.sum())} of {got.size} off, max |d| {d.max():.3g}"


def check_launch(e, oracle, launch, k):
    """Runs launch k and checks its output(s) against the oracle."""
    kind, f, n, flags = launch
    nd, at = e.graph.nodes, e.b.at
    H = lambda i: host(at(i))  # noqa: E731
    srcs = {s for j in range(f, f + n) for s in nd[j].src if s >= 0}
    made = {nd[j].dst for j in range(f, f + n)}
    for s in srcs - made:   # every input of the launch was written before it
        if s in e.given.values() or kind == C.GL_VIEW:
            continue
        v = H(s)
        assert np.isfinite(v).all(), f"launch {k} ({kind}) reads tensor {s} with non-finite values"
    T_, N_, K_ = e.graph._arrays(e.keep)
    rc = C.load().cbx_graph_launch(T_, len(e.graph._descs), N_, len(e.graph.nodes),
                                   C.ctypes.byref(C.GLaunch(kind, f, n, flags)), C._stream())
    assert rc == C.OK, C.last_error()
    y = nd[f + n - 1].dst
    what = f"launch {k} (kind {kind}, nodes {f}..{f + n - 1})"
    if kind == C.GL_VIEW:
        return
    if kind == C.GL_BINARY:
        a, b = H(nd[f].src[0]), H(nd[f].src[1])
        exp = oracle.mul(a, b) if flags == C.BINARY_MUL else oracle.add(a, b)
        assert_bitexact(H(y), exp, what)
    elif kind == C.GL_BIAS_RESIDUAL:
        last = nd[f + n - 1]
        s = nd[f + n - 2].dst                     # the bias sum, or its (C, 1) view
        r = last.src[1] if last.src[0] == s else last.src[0]
        exp = oracle.add(H(r), oracle.add(H(nd[f].src[0]), H(nd[f].src[1])))
        assert_bitexact(H(y), exp, what)
    elif kind == C.GL_CONCAT:
        a, b = H(nd[f].src[0]), H(nd[f].src[1])
        assert_bitexact(H(y), np.concatenate((a, b), axis=a.ndim - 1 - nd[f].iparam), what)
    elif kind == C.GL_BIAS_ACT:
        t = oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))
        if n == 1:
            assert_bitexact(H(y), t, what)
        else:
            assert n == 2
            assert_close(H(y), oracle.unary(nd[f + 1].iparam, t), x=t, what=what)
    elif kind == C.GL_UNARY:
        assert n == 3   # mish
        x = H(nd[f].src[0])
        exp = oracle.mul(x, oracle.unary(oracle.TANH, oracle.unary(oracle.SOFTPLUS, x)))
        assert_close(H(y), exp, x=x, what=what)
    elif kind == C.GL_SOFT_MAX:
        assert n == 2 and nd[f].op == C.GOP_SCALE
        softmax_close(H(y), oracle.scale_diag_mask_soft_max(H(nd[f].src[0]), nd[f].fparam, -1, nth=8), what)
    elif kind == C.GL_ADD_LAYER_NORM:
        assert n == 5   # add(a, bias) -> add(., r) -> norm -> mul -> add
        r_node = nd[f + 1]
        other = r_node.src[1] if r_node.src[0] == nd[f].dst else r_node.src[0]
        s = oracle.add(oracle.add(H(nd[f].src[0]), H(nd[f].src[1])), H(other))
        exp = oracle.add(oracle.mul(oracle.norm(s, nd[f + 2].fparam), H(nd[f + 3].src[1])), H(nd[f + 4].src[1]))
        assert_bitexact(H(y), exp, what)
        if not flags & 1:
            assert_bitexact(H(r_node.dst), s, what + " (the sum)")
    elif kind == C.GL_LAYER_NORM_MASK:
        assert n == 7
        ln = oracle.add(oracle.mul(oracle.norm(H(nd[f].src[0]), nd[f].fparam), H(nd[f + 1].src[1])),
                        H(nd[f + 2].src[1]))
        mish = oracle.mul(ln, oracle.unary(oracle.TANH, oracle.unary(oracle.SOFTPLUS, ln)))
        assert_close(H(y), oracle.mul(mish, H(nd[f + 6].src[1])), x=ln, what=what)
    elif kind == C.GL_CAUSAL_CONV1D:
        assert n == 15 and (flags & 3) == 3 and (flags & 4)
        x, mask = H(nd[f].src[0]), H(nd[f].src[1])
        w, bias = H(nd[f + 7].src[0]), H(nd[f + 11].src[0])
        K = w.shape[-1]
        T = x.shape[0]
        xm = oracle.mul(x, mask)
        ref = oracle.conv1d(xm, w, 1, K - 1, 1, oracle.CONV_PRO_NONE, None, None, 0.0, bias, None, nth=8)[:T]
        mag = oracle.conv1d(np.abs(xm), np.abs(w), 1, K - 1, 1, nth=8)[:T].astype(np.float64)
        d = np.abs(H(y).astype(np.float64) - ref.astype(np.float64))
        assert not (d > 2.0 ** -13 * mag + 2.0 ** -22 * np.abs(ref)).any(), what
    else:
        raise AssertionError(f"{what}: a launch kind the estimator list was not expected to hold")


@pytest.mark.parametrize("T,n_mid,n_tr,tail", [(72, 2, 2, 8), (130, 1, 1, 0)])
def test_estimator_launch_by_launch(cbx, oracle, T, n_mid, n_tr, tail):
    e = CFMEstimator(T, seed=T, n_mid=n_mid, n_tr=n_tr, mask_tail=tail)
    try:
        plan = e.plan()
        assert all(p[0] != C.GL_UNSUPPORTED for p in plan)
        for k, launch in enumerate(plan):
            check_launch(e, oracle, launch, k)
        out = host(e.b.at(e.out))
        assert np.isfinite(out).all()
        if tail:
            assert (out[T - tail:] == 0).all(), "masked frames come out zero"
        # the whole list again: the same bits
        e.b.at(e.out).fill_(float("nan"))
        assert e.graph.compute(e.keep) == sum(1 for p in plan if p[0] != C.GL_VIEW)
        assert_bitexact(host(e.b.at(e.out)), out, "cbx_graph_compute")
        ex = e.graph.capture(e.keep)
        try:
            e.b.at(e.out).fill_(float("nan"))
            ex.launch()
            assert_bitexact(host(e.b.at(e.out)), out, "cbx_graph_exec replay")
        finally:
            ex.close()
    finally:
        e.close()


def test_estimator_full_size_runs(cbx):
    """The reference's sizes (500 frames, 12 mid blocks, 4 transformers a
    stage: 352 launches) through one captured graph: finite output, masked
    frames zero."""
    e = CFMEstimator(500, seed=3, mask_tail=40)
    try:
        ex = e.graph.capture(e.keep)
        try:
            ex.launch()
            out = host(e.b.at(e.out))
        finally:
            ex.close()
        assert np.isfinite(out).all()
        assert (out[460:] == 0).all()
        assert math.isfinite(float(np.abs(out).max()))
    finally:
        e.close()
