"""One HiFT vocoder decode's node list (hift_vocoder.cpp:613-749 between the
host STFT and iSTFT; chatterbox_amdvulkan_amd/hift_decode.py) run launch by
launch, each launch checked against the oracle on the inputs it read from
the device: the conv bar for the 77 conv1d_CT and 3 conv_transpose1d_CT
launches (f16 operands, f32 sums: |d| <= 2^-13 sum |a b| + 2^-22 |ref|;
with the resblock sum and mean folded into a conv, that bound scaled plus
the two f32 roundings), bit-exact for the source joins, the pad's copy and
its concat.  Then the whole list through cbx_graph_compute and a captured
cbx_graph_exec: the same output bits."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.hift_decode import HiFTDecode
from tests._util import assert_bitexact
from tests.test_gpu_conv1d import check as check_conv
from tests.test_gpu_conv1d import check_sum
from tests.test_gpu_conv_transpose1d import check as check_convt

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def check_launch(e, oracle, launch, k):
    kind, f, n, flags = launch
    nd = e.graph.nodes
    H = lambda i: host(e.b.at(i))  # noqa: E731
    H2 = lambda i: H(i).reshape(-1, e.b.shape(i)[-1])  # noqa: E731   (T, C) of a batch-1 (1, T, C)
    T_, N_, _ = e.graph._arrays(e.keep)
    rc = C.load().cbx_graph_launch(T_, len(e.graph._descs), N_, len(e.graph.nodes),
                                   C.ctypes.byref(C.GLaunch(kind, f, n, flags)), C._stream())
    assert rc == C.OK, C.last_error()
    y = nd[f + n - 1].dst
    what = f"launch {k} (kind {kind}, nodes {f}..{f + n - 1})"
    if kind == C.GL_VIEW:
        return
    got = H(y)
    assert np.isfinite(got).all(), what
    if kind == C.GL_CONV1D:
        extra = (1 if flags & C.GLF_SUM else 0) + (1 if flags & C.GLF_SCALE else 0)
        rout = nd[f + n - 1 - extra].dst           # the residual add's result: the recorded chain's end
        r = e.conv_ref[rout]
        x = H2(r["x"])
        pro = {"snake": oracle.CONV_PRO_SNAKE, "leaky": oracle.CONV_PRO_LEAKY, None: oracle.CONV_PRO_NONE}[r["pro"]]
        a, ai = (H(r["alpha"][0]), H(r["alpha"][1])) if r["pro"] == "snake" else (None, None)
        res = H2(r["res"]) if r["res"] is not None else None
        args = (x, H(r["w"]), r["stride"], r["pad"], r["dil"], pro, a, ai, r["slope"], H(r["bias"]), res)
        if not extra:
            check_conv(oracle, got.reshape(-1, got.shape[-1]), *args, what)
        else:
            sa = nd[f + n - extra]                 # add(sum so far, r)
            acc = H2(sa.src[0] if sa.src[1] == rout else sa.src[1])
            scale = nd[f + n - 1].fparam if flags & C.GLF_SCALE else 1.0
            check_sum(oracle, got.reshape(-1, got.shape[-1]), *args, acc, scale, what + " (with the resblock sum)")
    elif kind == C.GL_CONV_TRANSPOSE1D:
        r = e.conv_ref[y]
        check_convt(oracle, got.reshape(-1, got.shape[-1]), H2(r["x"]), H(r["w"]), r["stride"], r["pad"],
                    oracle.CONV_PRO_LEAKY, r["slope"], H(r["bias"]), what)
    elif kind == C.GL_BINARY:
        assert flags == C.BINARY_ADD
        assert_bitexact(got, oracle.add(H(nd[f].src[0]), H(nd[f].src[1])), what)
    elif kind == C.GL_SCALE:
        s = np.float32(nd[f].fparam)
        assert s == np.float32(1.0 / 3.0)
        assert_bitexact(got, H(nd[f].src[0]) * s, what)     # one f32 product per element
    elif kind == C.GL_CPY:
        assert_bitexact(got, H(nd[f].src[0]), what)
    elif kind == C.GL_CONCAT:
        a, b = H(nd[f].src[0]), H(nd[f].src[1])
        assert_bitexact(got, np.concatenate((a, b), axis=a.ndim - 1 - nd[f].iparam), what)
    else:
        raise AssertionError(f"{what}: a launch kind the decode list was not expected to hold")


@pytest.mark.parametrize("T_mel", [3, 8])
def test_decode_launch_by_launch(cbx, oracle, T_mel):
    e = HiFTDecode(T_mel, seed=T_mel)
    try:
        plan = e.plan()
        assert all(p[0] != C.GL_UNSUPPORTED for p in plan)
        for k, launch in enumerate(plan):
            check_launch(e, oracle, launch, k)
        out = host(e.b.at(e.out))
        # the reflection pad: frame 0 of stage 2 is a copy of frame 1
        p = host(e.b.at(e.padded))
        assert p.shape[0] == 120 * T_mel + 1 and np.array_equal(p[0], p[2])
        # the whole list again: the same bits
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


def test_decode_full_size_runs(cbx):
    """500 mel frames (10 s of audio; stages of 4000, 20000 and 60001
    frames) through one captured graph: finite output of 60001 x 18."""
    e = HiFTDecode(500, seed=1)
    try:
        ex = e.graph.capture(e.keep)
        try:
            ex.launch()
            out = host(e.b.at(e.out))
        finally:
            ex.close()
        assert out.shape == (1, 60001, 18)
        assert np.isfinite(out).all()
        assert float(np.abs(out).max()) > 0.0
    finally:
        e.close()
