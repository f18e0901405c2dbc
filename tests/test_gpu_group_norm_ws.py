"""cbx_group_norm_ws: GroupNorm with the statistics split over chunk
workgroups that meet in a workspace.  Same bits as cbx_group_norm and the
oracle for every chunk count, whether a workgroup waits for the others or
computes every chunk's partial itself (a wait of 0: forced from the host),
in place (with and without the wait), on consecutive calls over one
workspace (the words of earlier launches carry other tags), and when two
streams run calls over one workspace at the same time."""
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


def cfm(C):
    x = W.normal(W.seed_of(3, 0) + C, (2, C, 1, 500))
    w = W.normal(W.seed_of(3, 1) + C, (1, C, 1, 1), 1.0, 0.02)
    b = W.normal(W.seed_of(3, 2) + C, (1, C, 1, 1), 0.0, 0.02)
    return x, w, b


def no_device_errors(cbx):
    flags = ctypes.c_uint32(0)
    assert cbx.load().cbx_device_errors(0, ctypes.byref(flags), 1) == cbx.OK
    assert flags.value == 0, f"device error bits {flags.value:#x}"


@pytest.mark.parametrize("C", [256, 512])
def test_cfm_shapes(cbx, oracle, C):
    """[2 (CFG pair), C, 500], 8 groups, affine, with and without Mish:
    bit-exact against the oracle (GroupNorm) and against cbx_group_norm
    (Mish too)."""
    x, w, b = cfm(C)
    ws = cbx.GroupNormWorkspace()
    xd, wd, bd = dev(x), dev(w), dev(b)
    gn = oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)
    assert_bitexact(host(cbx.group_norm_ws(xd, 8, 1e-5, ws, wd, bd)), gn, "gn_ws+affine")
    got = host(cbx.group_norm_ws(xd, 8, 1e-5, ws, wd, bd, act=cbx.MISH))
    assert_bitexact(got, host(cbx.group_norm(xd, 8, 1e-5, wd, bd, act=cbx.MISH)), "gn_ws+mish vs gn+mish")
    assert_close(got, oracle.group_norm_affine(x, 8, 1e-5, w, b, True, nth=8), x=gn, what="gn_ws+mish")
    assert_bitexact(host(cbx.group_norm_ws(xd, 8, 1e-5, ws)), oracle.group_norm(x, 8, 1e-5, nth=8), "plain")
    no_device_errors(cbx)
    ws.close()


@pytest.mark.parametrize("n_chunks", [2, 3, 7, 16, 31, 32])
def test_every_chunk_count_same_bits(cbx, oracle, n_chunks):
    x, w, b = cfm(512)
    exp = oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)
    ws = cbx.GroupNormWorkspace(n_chunks=n_chunks)
    got = host(cbx.group_norm_ws(dev(x), 8, 1e-5, ws, dev(w), dev(b)))
    assert_bitexact(got, exp, f"{n_chunks} chunks")
    no_device_errors(cbx)
    ws.close()


@pytest.mark.parametrize("n_chunks", [0, 5, 32])
def test_no_wait_fallback_same_bits(cbx, oracle, n_chunks):
    """max_wait_us 0: no workgroup waits; each computes every chunk's
    partial from x itself -- the path a workgroup takes when the others do
    not arrive in time.  Same bits."""
    x, w, b = cfm(256)
    ws = cbx.GroupNormWorkspace(max_wait_us=0, n_chunks=n_chunks)
    gn = oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)
    assert_bitexact(host(cbx.group_norm_ws(dev(x), 8, 1e-5, ws, dev(w), dev(b))), gn, "no-wait")
    got = host(cbx.group_norm_ws(dev(x), 8, 1e-5, ws, dev(w), dev(b), act=cbx.MISH))
    assert_close(got, oracle.group_norm_affine(x, 8, 1e-5, w, b, True, nth=8), x=gn, what="no-wait mish")
    # and the workspace still serves waiting calls afterwards
    ws.tune(2000, n_chunks)
    assert_bitexact(host(cbx.group_norm_ws(dev(x), 8, 1e-5, ws, dev(w), dev(b))), gn, "wait after no-wait")
    no_device_errors(cbx)
    ws.close()


def test_consecutive_calls_reuse_the_workspace(cbx, oracle):
    """Many calls over one workspace on one stream, alternating shapes: the
    counters return to zero after every launch."""
    ws = cbx.GroupNormWorkspace()
    cases = []
    for C in (256, 512):
        x, w, b = cfm(C)
        cases.append((dev(x), dev(w), dev(b), oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)))
    outs = []
    for i in range(40):
        xd, wd, bd, _ = cases[i % 2]
        outs.append(cbx.group_norm_ws(xd, 8, 1e-5, ws, wd, bd))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert_bitexact(host(o), cases[i % 2][3], f"call {i}")
    no_device_errors(cbx)
    ws.close()


@pytest.mark.parametrize("max_wait_us", [None, 0, 1])
@pytest.mark.parametrize("C", [256, 512])
def test_in_place(cbx, oracle, C, max_wait_us):
    """y == x with the default wait, with no wait at all and with a 1 us
    wait (every or nearly every wave would stop waiting and re-read the
    group from x while other chunks store over it, if in-place calls took
    the split): the oracle's bits, with and without Mish, and no error bit."""
    x, w, b = cfm(C)
    ws = cbx.GroupNormWorkspace(max_wait_us=max_wait_us)
    gn = oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)
    t = dev(x)
    cbx.group_norm_ws(t, 8, 1e-5, ws, dev(w), dev(b), out=t)
    assert_bitexact(host(t), gn, f"in place, wait {max_wait_us}")
    t = dev(x)
    cbx.group_norm_ws(t, 8, 1e-5, ws, dev(w), dev(b), act=cbx.MISH, out=t)
    ref = cbx.group_norm_ws(dev(x), 8, 1e-5, ws, dev(w), dev(b), act=cbx.MISH)
    assert_bitexact(host(t), host(ref), f"in place + mish, wait {max_wait_us}")
    t = dev(x)
    cbx.group_norm_noalloc(t, 8, 1e-5, dev(w), dev(b), out=t)
    assert_bitexact(host(t), gn, "noalloc in place")
    t = dev(x)
    cbx.group_norm(t, 8, 1e-5, dev(w), dev(b), out=t)
    assert_bitexact(host(t), gn, "group_norm in place")
    no_device_errors(cbx)
    ws.close()


def test_split_enabled_on_this_device(cbx):
    """cbx_init's probe found workgroups with one index mod 8 on one XCD
    (MI355X deals them round-robin), so the split runs."""
    assert cbx.group_norm_split_enabled(0)


def test_two_streams_share_one_workspace(cbx, oracle):
    """Calls on two streams over one workspace, free to overlap in time
    (each writes partials the other's waves read past by tag): every result
    keeps the oracle's bits; a short wait keeps any stall brief."""
    ws = cbx.GroupNormWorkspace(max_wait_us=50)
    cases = []
    for C in (256, 512):
        x, w, b = cfm(C)
        cases.append((dev(x), dev(w), dev(b), oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    outs = []
    for i in range(24):
        k = i % 2
        with torch.cuda.stream(streams[k]):
            xd, wd, bd, _ = cases[k]
            outs.append((k, cbx.group_norm_ws(xd, 8, 1e-5, ws, wd, bd)))
    torch.cuda.synchronize()
    for i, (k, o) in enumerate(outs):
        assert_bitexact(host(o), cases[k][3], f"call {i} on stream {k}")
    no_device_errors(cbx)
    ws.close()


@pytest.mark.parametrize("shape,groups", [((2, 10, 1, 2048), 3), ((1, 6, 1, 1024), 4), ((3, 48, 2, 256), 2),
                                          ((1, 8, 1, 8192), 8), ((16, 64, 1, 100), 8), ((1, 7, 3, 5), 2),
                                          ((1, 32, 1, 4096), 1), ((4, 256, 1, 500), 32)])
def test_ragged_and_fallback_layouts(cbx, oracle, shape, groups):
    """Ragged last groups and an empty trailing group (ggml's ceil split),
    chunks of different lengths, batches, odd ne0 (not the split's layout:
    cbx_group_norm runs it), a group larger than 32 chunks of 2048 vectors
    would hold, and many groups."""
    x = W.normal(63 + shape[1] + shape[-1], shape, 0.5, 2.0)
    C = shape[1]
    w = W.normal(64, (1, C, 1, 1), 1.0, 0.1)
    b = W.normal(65, (1, C, 1, 1), 0.0, 0.1)
    ws = cbx.GroupNormWorkspace()
    gn = oracle.group_norm_affine(x, groups, 1e-5, w, b, False, nth=8)
    assert_bitexact(host(cbx.group_norm_ws(dev(x), groups, 1e-5, ws, dev(w), dev(b))), gn, f"{shape}/{groups}")
    got = host(cbx.group_norm_ws(dev(x), groups, 1e-5, ws, dev(w), dev(b), act=cbx.MISH))
    assert_close(got, oracle.group_norm_affine(x, groups, 1e-5, w, b, True, nth=8), x=gn, what="mish")
    no_device_errors(cbx)
    ws.close()


def test_errors(cbx):
    L = cbx.load()
    x = torch.zeros((2, 16, 1, 64), device="cuda")
    d = lambda t: ctypes.byref(cbx.desc(t))  # noqa: E731
    assert L.cbx_group_norm_ws(d(x), 8, 1e-5, None, None, -1, d(x), None, None) == cbx.ERR_INVALID_ARG
    ws = cbx.GroupNormWorkspace()
    # y overlapping x other than as x itself
    buf = torch.zeros(2 * 16 * 64 + 64, device="cuda")
    xs, ys = buf[:2048].view(2, 16, 1, 64), buf[64:2112].view(2, 16, 1, 64)
    assert L.cbx_group_norm_ws(d(xs), 8, 1e-5, None, None, -1, d(ys), ws.handle, None) == cbx.ERR_INVALID_ARG
    assert "overlap" in cbx.last_error()
    assert L.cbx_group_norm_workspace_tune(ws.handle, 10, 33) == cbx.ERR_INVALID_ARG
    ws.close()
