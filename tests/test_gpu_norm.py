"""LayerNorm / RMSNorm (+affine, +activation) through the C ABI vs the oracle.

The kernels reproduce ggml-cpu's arithmetic (f64 sums, same f32 rounding
sequence), so the f32 results are expected bit-identical; the gate is the
north-star bound (1e-5 relative), and the exact-match fraction is asserted
separately to be total."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import RTOL_F16, assert_bitexact, assert_close, exact_fraction

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_prefill_layer_norm(cbx, oracle):
    """T3 prefill LN: [512,1024], eps 1e-5, gamma ~N(1,.02), beta ~N(0,.02)."""
    inp = W.prefill_inputs()
    x = W.normal(W.seed_of(2, 6), (512, 1024))
    exp = oracle.layer_norm(x, inp["ln_w"], inp["ln_b"], 1e-5, nth=8)
    got = host(cbx.layer_norm(dev(x), dev(inp["ln_w"]), dev(inp["ln_b"]), 1e-5))
    assert_close(got, exp, what="layer_norm")
    assert exact_fraction(got, exp) == 1.0
    assert_bitexact(host(cbx.norm(dev(x), 1e-5)), oracle.norm(x, 1e-5, nth=8), "norm")


@pytest.mark.parametrize("shape", [(7, 80), (3, 1), (5, 1000), (2, 1027), (4, 256), (3, 1280), (2, 5120),
                                   (2, 8192), (2, 8196), (1, 20000)])
@pytest.mark.parametrize("eps", [1e-5, 1e-12])
def test_layer_norm_shapes(cbx, oracle, shape, eps):
    """Ragged rows (scalar path), the reference's widths (80..5120), and rows
    past the register budget (three-pass loop)."""
    x = W.normal(21 + shape[1], shape, 0.5, 2.0)
    w = W.normal(22, (shape[1],), 1.0, 0.02)
    b = W.normal(23, (shape[1],), 0.0, 0.02)
    got = host(cbx.layer_norm(dev(x), dev(w), dev(b), eps))
    exp = oracle.layer_norm(x, w, b, eps)
    assert_close(got, exp, what=f"layer_norm {shape}")
    assert_bitexact(got, exp, f"layer_norm {shape}")


def test_layer_norm_constant_row_and_views(cbx, oracle):
    """A constant row normalises to 0 (output = b); a row-strided view."""
    x = np.full((4, 512), 3.25, dtype=np.float32)
    w = W.normal(24, (512,), 1.0, 0.02)
    b = W.normal(25, (512,), 0.0, 0.02)
    got = host(cbx.layer_norm(dev(x), dev(w), dev(b), 1e-5))
    assert_bitexact(got, np.broadcast_to(b, x.shape).astype(np.float32), "constant row")
    big = W.normal(26, (6, 700))
    view = dev(big)[:, 16:528]                           # ne0 512, nb1 2800 bytes
    got = host(cbx.layer_norm(view, dev(w), dev(b), 1e-5))
    assert_bitexact(got, oracle.layer_norm(np.ascontiguousarray(big[:, 16:528]), w, b, 1e-5), "view")


def test_layer_norm_mish_epilogue(cbx, oracle):
    """causal_block1d's LN -> Mish in one pass (CFM, ne0 = 256 channels)."""
    x = W.normal(27, (500, 256))
    w = W.normal(28, (256,), 1.0, 0.02)
    b = W.normal(29, (256,), 0.0, 0.02)
    ln = oracle.layer_norm(x, w, b, 1e-5)
    exp = oracle.unary(oracle.MISH, ln)
    got = host(cbx.layer_norm(dev(x), dev(w), dev(b), 1e-5, act=cbx.MISH))
    assert_close(got, exp, x=ln, what="ln+mish")


def test_rms_norm_decode_step(cbx, oracle):
    """T3 decode step: RMSNorm eps 1e-5 with gamma on [1,1024]."""
    x = W.normal(W.seed_of(1, 0), (1, 1024))
    g = W.normal(W.seed_of(1, 1), (1024,), 1.0, 0.02)
    got = host(cbx.rms_norm_mul(dev(x), dev(g), 1e-5))
    exp = oracle.rms_norm_mul(x, g, 1e-5)
    assert_close(got, exp, what="rms_norm_mul")
    assert_bitexact(got, exp, "rms_norm_mul")
    assert_bitexact(host(cbx.rms_norm(dev(x), 1e-5)), oracle.rms_norm(x, 1e-5), "rms_norm")


@pytest.mark.parametrize("shape", [(64, 1024), (3, 77), (2, 12000)])
def test_rms_norm_f16_storage(cbx, oracle, shape):
    """64-stream decode: f16 storage, f32 arithmetic, one rounding at the store."""
    x = W.normal(W.seed_of(5, 2) + shape[1], shape).astype(np.float16)
    g = W.normal(W.seed_of(5, 3), (shape[1],), 1.0, 0.02)
    got = host(cbx.rms_norm_mul(dev(x), dev(g), 1e-5))
    exp = oracle.rms_norm_mul(x, g, 1e-5)
    assert_close(got.astype(np.float32), exp.astype(np.float32), rtol=RTOL_F16, what="rms f16")
    assert_bitexact(got, exp, "rms f16")


def test_layer_norm_f16_storage(cbx, oracle):
    x = W.normal(31, (40, 512)).astype(np.float16)
    w = W.normal(32, (512,), 1.0, 0.02)
    b = W.normal(33, (512,), 0.0, 0.02)
    got = host(cbx.layer_norm(dev(x), dev(w), dev(b), 1e-5))
    assert_bitexact(got, oracle.layer_norm(x, w, b, 1e-5), "ln f16")


@pytest.mark.parametrize("table", ["f32", "f16", "q8_0"])
def test_embed_then_layer_norm_fused(cbx, oracle, table):
    """T3 prefill: token + position rows, then LN-1 of layer 0, in one kernel;
    h (the residual stream) and y both bit-exact vs the unfused oracle chain."""
    inp = W.prefill_inputs()
    tab = inp["table"]
    q8 = table == "q8_0"
    if table == "f16":
        tab = tab.astype(np.float16)
    elif q8:
        tab = oracle.quantize_q8_0(tab)
    h_ref = oracle.get_rows_add(tab, inp["ids"], inp["pos_table"], inp["pos_ids"], q8_0=q8, nth=8)
    y_ref = oracle.layer_norm(h_ref, inp["ln_w"], inp["ln_b"], 1e-5, nth=8)
    h, y = cbx.get_rows_add_layer_norm(dev(tab), dev(inp["ids"]), dev(inp["pos_table"]), dev(inp["pos_ids"]),
                                       dev(inp["ln_w"]), dev(inp["ln_b"]), 1e-5, q8_0=q8)
    assert_bitexact(host(h), h_ref, "h")
    assert_bitexact(host(y), y_ref, "y")
    _, y2 = cbx.get_rows_add_layer_norm(dev(tab), dev(inp["ids"][:7]), dev(inp["pos_table"]),
                                        dev(inp["pos_ids"][:7]), dev(inp["ln_w"]), None, 1e-5, q8_0=q8,
                                        store_h=False)
    assert_bitexact(host(y2), oracle.layer_norm(h_ref[:7], inp["ln_w"], None, 1e-5), "no h, no bias")


def test_norm_rejects_bad_args(cbx):
    x = dev(W.normal(34, (4, 64)))
    with pytest.raises(cbx.CbxError):
        cbx.layer_norm(x, dev(W.normal(35, (32,))), None, 1e-5)      # w shape
    with pytest.raises(cbx.CbxError):
        cbx.norm(x, -1.0)                                            # eps < 0
    with pytest.raises(cbx.CbxError):
        cbx.norm(x, 1e-5, out=torch.empty((4, 63), device="cuda"))   # y shape
