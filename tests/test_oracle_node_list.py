"""oracle.run_node_list -- the CPU restatement of a graph run node by node,
timed beside the GPU in bench.py's CPU leg -- against independent numpy on
the flow-encoder and S3-encoder lists at small sizes: every node's output
from the inputs the runner gave it, bit-exact for the gather, the adds,
the scales, LeakyReLU and the views; the f32 bar against float64 for the
LayerNorms, SiLU, GELU-erf and the softmax; the RoPE nodes as the oracle's
rope_ext, which tests/test_oracle_pins.py pins."""
import math

import numpy as np
import pytest

from chatterbox_amdvulkan_amd.flow_encoder import FlowEncoderCall
from chatterbox_amdvulkan_amd.s3_encoder import HEAD_DIM, ROPE_BASE, ROPE_MAX, S3EncoderCall
from chatterbox_amdvulkan_amd import cbxops as C


def f64_close(got, exp, what, rel=1e-5):
    d = np.abs(got.astype(np.float64) - exp)
    bad = d > rel * np.abs(exp) + 1e-6
    assert not bad.any(), f"{what}: {int(bad.sum())} of {got.size} off, max |d| {d.max():.3g}"


def check_all(O, e, rope=None):
    import bench

    nodes, shapes, leaves = bench.cpu_node_list(C, e)
    v = O.run_node_list(nodes, shapes, dict(leaves), rope=rope, nth=4)
    for k, (op, d, s0, s1, ip, fp) in enumerate(nodes):
        a, b, y = v.get(s0), v.get(s1), v[d]
        what = f"node {k} ({op})"
        assert y.shape == shapes[d], what
        if op == "view":
            np.testing.assert_array_equal(y, a.reshape(shapes[d]), what)
        elif op == "get_rows":
            np.testing.assert_array_equal(y, a[b], what)
        elif op == "add":
            np.testing.assert_array_equal(y, a + b, what)
        elif op == "mul":
            np.testing.assert_array_equal(y, a * b, what)
        elif op == "scale":
            np.testing.assert_array_equal(y, a * np.float32(fp), what)
        elif op == "leaky_relu":
            np.testing.assert_array_equal(y, np.where(a > 0, a, a * np.float32(fp)), what)
        elif op == "norm":
            x = a.astype(np.float64)
            mu = x.mean(-1, keepdims=True)
            f64_close(y, (x - mu) / np.sqrt(((x - mu) ** 2).mean(-1, keepdims=True) + fp), what)
        elif op == "soft_max":
            x = a.astype(np.float64) * fp
            ex = np.exp(x - x.max(-1, keepdims=True))
            f64_close(y, ex / ex.sum(-1, keepdims=True), what)
        elif op == "unary":
            x = a.astype(np.float64)
            exp = {C.SILU: x / (1.0 + np.exp(-x)),
                   C.GELU_ERF: 0.5 * x * (1.0 + np.vectorize(math.erf)(x / math.sqrt(2.0)))}[ip]
            d_ = np.abs(y - exp)
            assert (d_ <= 1e-5 * np.abs(exp) + 2.0 ** -22 * np.abs(x) + 1e-30).all(), what
        elif op == "rope":
            np.testing.assert_array_equal(y, O.rope_ext(a, b, **rope), what)
        else:
            raise AssertionError(what)


@pytest.mark.parametrize("T,n_blocks,n_up", [(7, 2, 1), (12, 1, 1)])
def test_flow_encoder_list(oracle, T, n_blocks, n_up):
    check_all(oracle, FlowEncoderCall(T, n_blocks=n_blocks, n_up_blocks=n_up, device=False))


def test_s3_encoder_list(oracle):
    e = S3EncoderCall(40, n_layer=2, device=False)
    check_all(oracle, e, rope=dict(n_dims=HEAD_DIM, mode=2, n_ctx_orig=ROPE_MAX, freq_base=ROPE_BASE))
