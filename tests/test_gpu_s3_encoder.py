"""One S3 encoder call's element-wise node list (s3enc.cpp:124-290; matmul,
conv and FSMN outputs given; chatterbox_amdvulkan_amd/s3_encoder.py) run
launch by launch, each launch checked against the oracle on the inputs it
read from the device: bit-exact for the bias adds, the joins, the
LayerNorms and the RoPEs (q and k as 20 heads of 64, NEOX, base 10000); the
f32 bar for GELU-erf and the softmax.  Then the whole list through
cbx_graph_compute and a captured cbx_graph_exec: the same output bits."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.s3_encoder import HEAD_DIM, ROPE_BASE, ROPE_MAX, S3EncoderCall
from tests._util import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def softmax_close(got, exp, what):
    d = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = d > 1e-5 * np.abs(exp.astype(np.float64)) + 1e-37
    assert not bad.any(), f"{what}: {int(bad.sum())} of {got.size} off, max |d| {d.max():.3g}"


def ln_ref(oracle, nd, k, x, H):
    """norm -> mul -> add at nodes k..k+2 of x."""
    return oracle.add(oracle.mul(oracle.norm(x, nd[k].fparam), H(nd[k + 1].src[1])), H(nd[k + 2].src[1]))


def check_launch(e, oracle, launch, k):
    kind, f, n, flags = launch
    nd = e.graph.nodes
    H = lambda i: host(e.b.at(i))  # noqa: E731
    T_, N_, _ = e.graph._arrays(e.keep)
    rc = C.load().cbx_graph_launch(T_, len(e.graph._descs), N_, len(e.graph.nodes),
                                   C.ctypes.byref(C.GLaunch(kind, f, n, flags)), C._stream())
    assert rc == C.OK, C.last_error()
    y = nd[f + n - 1].dst
    what = f"launch {k} (kind {kind}, nodes {f}..{f + n - 1})"
    if kind == C.GL_VIEW:
        return
    got = H(y)
    if kind == C.GL_BIAS_ACT:
        t = oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))
        if n == 1:
            assert_bitexact(got, t, what)
        else:
            assert n == 2 and nd[f + 1].iparam == C.GELU_ERF
            assert_close(got, oracle.unary(nd[f + 1].iparam, t), x=t, what=what)
    elif kind == C.GL_LAYER_NORM:
        assert n == 3
        assert_bitexact(got, ln_ref(oracle, nd, f, H(nd[f].src[0]), H), what)
    elif kind == C.GL_ROPE:
        x = H(nd[f].src[0])
        pos = H(nd[f].src[1])
        exp = oracle.rope_ext(x, pos, HEAD_DIM, mode=2, n_ctx_orig=ROPE_MAX, freq_base=ROPE_BASE)
        assert_bitexact(got, exp, what)
    elif kind == C.GL_BINARY:
        assert flags == C.BINARY_ADD
        assert_bitexact(got, oracle.add(H(nd[f].src[0]), H(nd[f].src[1])), what)
    elif kind == C.GL_SOFT_MAX:
        assert n == 2 and nd[f].op == C.GOP_SCALE
        softmax_close(got, oracle.scale_diag_mask_soft_max(H(nd[f].src[0]), nd[f].fparam, -1, nth=8), what)
    elif kind == C.GL_BIAS_RESIDUAL:
        last = nd[f + n - 1]
        s = nd[f + n - 2].dst
        r = last.src[1] if last.src[0] == s else last.src[0]
        assert_bitexact(got, oracle.add(H(r), oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))), what)
    elif kind == C.GL_ADD_LAYER_NORM:
        if n == 4:      # add(x, attn) -> layer_norm
            s = oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))
            k_ln, r_node = f + 1, nd[f]
        else:           # add(mm, bias) -> add(x, .) -> layer_norm
            assert n == 5
            r_node = nd[f + 1]
            other = r_node.src[1] if r_node.src[0] == nd[f].dst else r_node.src[0]
            s = oracle.add(oracle.add(H(nd[f].src[0]), H(nd[f].src[1])), H(other))
            k_ln = f + 2
        assert_bitexact(got, ln_ref(oracle, nd, k_ln, s, H), what)
        if not flags & 1:
            assert_bitexact(H(r_node.dst), s, what + " (the sum)")
    else:
        raise AssertionError(f"{what}: a launch kind the encoder list was not expected to hold")


@pytest.mark.parametrize("T_mel,n_layer", [(64, 2), (150, 1)])
def test_encoder_launch_by_launch(cbx, oracle, T_mel, n_layer):
    e = S3EncoderCall(T_mel, seed=T_mel, n_layer=n_layer)
    try:
        plan = e.plan()
        assert all(p[0] != C.GL_UNSUPPORTED for p in plan)
        for k, launch in enumerate(plan):
            check_launch(e, oracle, launch, k)
        out = host(e.b.at(e.out))
        assert np.isfinite(out).all()
        e.b.at(e.out).fill_(float("nan"))
        assert e.graph.compute(e.keep) == sum(1 for q in plan if q[0] != C.GL_VIEW)
        assert_bitexact(host(e.b.at(e.out)), out, "cbx_graph_compute")
        ex = e.graph.capture(e.keep)
        try:
            for rep in range(2):
                e.b.at(e.out).fill_(float("nan"))
                ex.launch()
                assert_bitexact(host(e.b.at(e.out)), out, f"cbx_graph_exec replay {rep}")
        finally:
            ex.close()
    finally:
        e.close()


def test_encoder_full_size_runs(cbx):
    """10 s of audio (1000 mel frames, 250 tokens, 6 layers: 63 launches)
    through one captured graph: finite output."""
    e = S3EncoderCall(1000, seed=2)
    try:
        ex = e.graph.capture(e.keep)
        try:
            assert ex.n_launches == 63
            ex.launch()
            out = host(e.b.at(e.out))
        finally:
            ex.close()
        assert out.shape == (250, 1280) and np.isfinite(out).all()
    finally:
        e.close()
