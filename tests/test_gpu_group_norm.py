"""ggml_group_norm (+ per-channel affine, + Mish) through the C ABI vs the oracle."""
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


@pytest.mark.parametrize("C", [256, 512])
def test_cfm_group_norm_mish(cbx, oracle, C):
    """[2 (CFG pair), C, 500 frames], 8 groups, eps 1e-5, affine, Mish.
    ggml layout ne = (500, 1, C, 2): channels on ne[2]."""
    x = W.normal(W.seed_of(3, 0) + C, (2, C, 1, 500))
    w = W.normal(W.seed_of(3, 1) + C, (1, C, 1, 1), 1.0, 0.02)
    b = W.normal(W.seed_of(3, 2) + C, (1, C, 1, 1), 0.0, 0.02)
    gn = oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8)
    got_gn = host(cbx.group_norm(dev(x), 8, 1e-5, dev(w), dev(b)))
    assert_bitexact(got_gn, gn, "group_norm+affine")
    exp = oracle.group_norm_affine(x, 8, 1e-5, w, b, True, nth=8)
    got = host(cbx.group_norm(dev(x), 8, 1e-5, dev(w), dev(b), act=cbx.MISH))
    assert_close(got, exp, x=gn, what="group_norm+mish")
    assert_bitexact(host(cbx.group_norm(dev(x), 8, 1e-5)), oracle.group_norm(x, 8, 1e-5, nth=8), "plain")


@pytest.mark.parametrize("shape,groups", [((1, 10, 3, 7), 3), ((2, 6, 2, 13), 4), ((1, 32, 1, 4096), 1),
                                          ((1, 64, 4, 512), 2)])
def test_group_norm_ragged(cbx, oracle, shape, groups):
    """Channels not divisible by the group count (ggml's ceil split; empty
    trailing groups), odd ne0 (scalar path), and groups of 128K-256K
    elements (three-pass loop)."""
    x = W.normal(61 + shape[1], shape, 1.0, 3.0)
    got = host(cbx.group_norm(dev(x), groups, 1e-5))
    assert_bitexact(got, oracle.group_norm(x, groups, 1e-5), f"gn {shape}/{groups}")


def test_one_group_equals_layer_norm(cbx, oracle):
    """One group over (T, 1, C) is LayerNorm of the flattened group."""
    x = W.normal(62, (3, 16, 1, 64))
    got = host(cbx.group_norm(dev(x), 1, 1e-5)).reshape(3, -1)
    ln = oracle.norm(x.reshape(3, -1), 1e-5)
    assert_close(got, ln, what="gn(1) vs ln")


@pytest.mark.parametrize("shape,groups", [((2, 10, 1, 2048), 3), ((1, 6, 1, 1024), 4), ((3, 48, 2, 256), 2),
                                          ((1, 8, 1, 8192), 8), ((16, 64, 1, 100), 8)])
def test_group_norm_split_over_workgroups(cbx, oracle, shape, groups):
    """Contiguous groups few enough to be split over several workgroups:
    ragged last groups, an empty trailing group, batches, and the
    many-groups case that keeps one workgroup per group.  Affine + Mish."""
    x = W.normal(63 + shape[1] + shape[-1], shape, 0.5, 2.0)
    C = shape[1]
    w = W.normal(64, (1, C, 1, 1), 1.0, 0.1)
    b = W.normal(65, (1, C, 1, 1), 0.0, 0.1)
    gn = oracle.group_norm_affine(x, groups, 1e-5, w, b, False, nth=8)
    assert_bitexact(host(cbx.group_norm(dev(x), groups, 1e-5, dev(w), dev(b))), gn, f"gn {shape}/{groups}")
    got = host(cbx.group_norm(dev(x), groups, 1e-5, dev(w), dev(b), act=cbx.MISH))
    assert_close(got, oracle.group_norm_affine(x, groups, 1e-5, w, b, True, nth=8), x=gn, what="gn+mish")


def test_group_norm_in_place(cbx, oracle):
    """y == x: every group is read whole before any of it is written."""
    x = W.normal(W.seed_of(3, 0) + 512, (2, 512, 1, 500))
    w = W.normal(W.seed_of(3, 1) + 512, (1, 512, 1, 1), 1.0, 0.02)
    b = W.normal(W.seed_of(3, 2) + 512, (1, 512, 1, 1), 0.0, 0.02)
    t = dev(x)
    cbx.group_norm(t, 8, 1e-5, dev(w), dev(b), out=t)
    assert_bitexact(host(t), oracle.group_norm_affine(x, 8, 1e-5, w, b, False, nth=8), "in place")
