"""cbx_group_norm_noalloc: the split-reduction GroupNorm over the library's
static scratch, through the C ABI, against the existing entry point
cbx_group_norm (bit for bit: same statistics, same activation code) on two
calls in a row, the second with a smaller input, and against the oracle;
then its size limit."""
import ctypes

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def cfm(C):
    x = W.normal(W.seed_of(3, 0) + C, (2, C, 1, 500))
    w = W.normal(W.seed_of(3, 1) + C, (1, C, 1, 1), 1.0, 0.02)
    b = W.normal(W.seed_of(3, 2) + C, (1, C, 1, 1), 0.0, 0.02)
    return x, w, b


def test_two_calls_match_group_norm(cbx, oracle):
    L = cbx.load()
    d = lambda t: ctypes.byref(cbx.desc(t))  # noqa: E731
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for act in (cbx.UNARY_NONE, cbx.MISH):
        outs = []
        for C in (512, 256):                      # the second call is smaller
            x, w, b = cfm(C)
            xd, wd, bd = dev(x), dev(w), dev(b)
            y = torch.empty_like(xd)
            ref = torch.empty_like(xd)
            assert L.cbx_group_norm_noalloc(d(xd), 8, 1e-5, d(wd), d(bd), act, d(y), s) == cbx.OK, cbx.last_error()
            assert L.cbx_group_norm(d(xd), 8, 1e-5, d(wd), d(bd), act, d(ref), s) == cbx.OK, cbx.last_error()
            outs.append((C, x, w, b, y, ref))
        torch.cuda.synchronize()
        for C, x, w, b, y, ref in outs:
            assert_bitexact(y.cpu().numpy(), ref.cpu().numpy(), f"noalloc vs group_norm C={C} act={act}")
            if act == cbx.UNARY_NONE:
                assert_bitexact(y.cpu().numpy(), oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8),
                                f"noalloc vs oracle C={C}")
    flags = ctypes.c_uint32(0)
    assert L.cbx_device_errors(0, ctypes.byref(flags), 1) == cbx.OK and flags.value == 0


def test_size_limit(cbx):
    """More than 1024 group instances (n_groups x ne[3]) is refused with a
    clear error and launches nothing."""
    L = cbx.load()
    d = lambda t: ctypes.byref(cbx.desc(t))  # noqa: E731
    x = torch.zeros((129, 8, 1, 4), device="cuda")      # 129 x 8 = 1032 instances
    y = torch.empty_like(x)
    assert L.cbx_group_norm_noalloc(d(x), 8, 1e-5, None, None, -1, d(y), None) == cbx.ERR_UNSUPPORTED
    assert "1024" in cbx.last_error()
    x = torch.zeros((128, 8, 1, 4), device="cuda")      # exactly 1024: accepted
    y = torch.empty_like(x)
    assert L.cbx_group_norm_noalloc(d(x), 8, 1e-5, None, None, -1, d(y), None) == cbx.OK, cbx.last_error()
    torch.cuda.synchronize()
