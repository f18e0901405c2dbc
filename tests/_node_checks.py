"""Runs one planned launch of a node list through cbx_graph_launch and checks
what it wrote against the oracle, on the inputs it read from the device:
bit-exact for the gathers, adds, products, joins, scales, LayerNorms,
LeakyReLU and RoPE; the f32 bar of tests/_util.py for the device-libm
activations and the softmax.  Shared by the reference-sequence tests whose
lists hold only these launch kinds."""
import numpy as np
import torch

from chatterbox_amdvulkan_amd import cbxops as C
from tests._util import assert_bitexact, assert_close


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


def run_and_check(graph, at, keep, oracle, launch, k, rope=None):
    """graph: the cbxops.Graph; at(i): tensor i; rope: dict of oracle.rope_ext
    keyword arguments (with n_dims) for ROPE launches."""
    kind, f, n, flags = launch
    nd = graph.nodes
    H = lambda i: host(at(i))  # noqa: E731
    T_, N_, _ = graph._arrays(keep)
    rc = C.load().cbx_graph_launch(T_, len(graph._descs), N_, len(graph.nodes),
                                   C.ctypes.byref(C.GLaunch(kind, f, n, flags)), C._stream())
    assert rc == C.OK, C.last_error()
    y = nd[f + n - 1].dst
    what = f"launch {k} (kind {kind}, nodes {f}..{f + n - 1})"
    if kind == C.GL_VIEW:
        return
    got = H(y)
    if kind == C.GL_GET_ROWS:
        assert n == 1
        assert_bitexact(got, H(nd[f].src[0])[H(nd[f].src[1])], what)
    elif kind == C.GL_BIAS_ACT:
        t = oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))
        if n == 1:
            assert_bitexact(got, t, what)
        else:
            assert n == 2
            assert_close(got, oracle.unary(nd[f + 1].iparam, t), x=t, what=what)
    elif kind == C.GL_LAYER_NORM:
        assert n == 3
        assert_bitexact(got, ln_ref(oracle, nd, f, H(nd[f].src[0]), H), what)
    elif kind == C.GL_SCALE:
        assert_bitexact(got, H(nd[f].src[0]) * np.float32(nd[f].fparam), what)
    elif kind == C.GL_LEAKY_RELU:
        assert_bitexact(got, oracle.leaky_relu(H(nd[f].src[0]), nd[f].fparam), what)
    elif kind in (C.GL_ROPE, C.GL_ROPE_TWO):
        assert rope is not None, what
        for k in range(f, f + n):
            exp = oracle.rope_ext(H(nd[k].src[0]), H(nd[k].src[1]), **rope)
            assert_bitexact(H(nd[k].dst), exp, f"{what} (node {k})")
    elif kind == C.GL_BINARY:
        a, b = H(nd[f].src[0]), H(nd[f].src[1])
        assert_bitexact(got, oracle.mul(a, b) if flags == C.BINARY_MUL else oracle.add(a, b), what)
    elif kind == C.GL_SOFT_MAX:
        if nd[f].op == C.GOP_ADD:       # the score terms' sum in front
            assert n == 3 and nd[f + 1].op == C.GOP_SCALE
            x, sc = oracle.add(H(nd[f].src[0]), H(nd[f].src[1])), nd[f + 1].fparam
        else:
            assert n == 2 and nd[f].op == C.GOP_SCALE
            x, sc = H(nd[f].src[0]), nd[f].fparam
        softmax_close(got, oracle.scale_diag_mask_soft_max(x, sc, -1, nth=8), what)
    elif kind == C.GL_BIAS_ADD_TWO:
        for k in (f, f + 1):
            assert_bitexact(H(nd[k].dst), oracle.add(H(nd[k].src[0]), H(nd[k].src[1])), f"{what} (node {k})")
    elif kind == C.GL_BIAS_ADD_PAIR:     # add -> heads view -> [views] two adds
        s = oracle.add(H(nd[f].src[0]), H(nd[f].src[1])).reshape(at(nd[f + 1].dst).shape)
        adds = [k for k in range(f + 2, f + n) if nd[k].op == C.GOP_ADD]
        assert len(adds) == 2 and all(nd[k].src[0] == nd[f + 1].dst for k in adds), what
        for k in adds:
            assert_bitexact(H(nd[k].dst), oracle.add(s, H(nd[k].src[1])), f"{what} (node {k})")
    elif kind == C.GL_BIAS_RESIDUAL:
        last = nd[f + n - 1]
        s = nd[f + n - 2].dst
        r = last.src[1] if last.src[0] == s else last.src[0]
        assert_bitexact(got, oracle.add(H(r), oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))), what)
    elif kind == C.GL_ADD_LAYER_NORM:
        if n == 4:      # add(a, b) -> layer_norm
            s = oracle.add(H(nd[f].src[0]), H(nd[f].src[1]))
            k_ln, r_node = f + 1, nd[f]
        else:           # add(mm, bias) -> add(r, .) -> layer_norm
            assert n == 5
            r_node = nd[f + 1]
            other = r_node.src[1] if r_node.src[0] == nd[f].dst else r_node.src[0]
            s = oracle.add(oracle.add(H(nd[f].src[0]), H(nd[f].src[1])), H(other))
            k_ln = f + 2
        assert_bitexact(got, ln_ref(oracle, nd, k_ln, s, H), what)
        if not flags & 1:
            assert_bitexact(H(r_node.dst), s, what + " (the sum)")
    else:
        raise AssertionError(f"{what}: a launch kind this check does not cover")


def full_list_same_bits(graph, at, keep, out, plan):
    """The whole list through cbx_graph_compute and a captured, twice
    replayed cbx_graph_exec: the output's bits of the launch-by-launch run."""
    ref = host(at(out))
    at(out).fill_(float("nan"))
    assert graph.compute(keep) == sum(1 for q in plan if q[0] != C.GL_VIEW)
    assert_bitexact(host(at(out)), ref, "cbx_graph_compute")
    ex = graph.capture(keep)
    try:
        for rep in range(2):
            at(out).fill_(float("nan"))
            ex.launch()
            assert_bitexact(host(at(out)), ref, f"cbx_graph_exec replay {rep}")
    finally:
        ex.close()
