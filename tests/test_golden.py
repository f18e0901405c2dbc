"""Committed golden vectors (tests/golden/ops_v1.npz, written by
tests/golden/make_golden.py after float64 cross-checks): the oracle must
reproduce them bit for bit (CPU), and the HIP library must match them to the
parity bar (GPU)."""
import os

import numpy as np
import pytest

from tests._util import assert_bitexact, assert_close

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ops_v1.npz")


@pytest.fixture(scope="module")
def G():
    with np.load(GOLD, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


UNARY = {"gelu_erf": "GELU_ERF", "silu": "SILU", "mish": "MISH", "tanh": "TANH", "softplus": "SOFTPLUS",
         "sin": "SIN", "gelu": "GELU"}


def test_oracle_reproduces_golden(oracle, G):
    assert_bitexact(oracle.get_rows_add(G["gather_table"], G["gather_ids"], G["gather_pos"], G["gather_pids"]),
                    G["gather_f32"], "gather")
    assert_bitexact(oracle.get_rows(G["gather_table"].astype(np.float16), G["gather_ids"]), G["gather_f16"], "f16")
    assert_bitexact(oracle.get_rows(G["gather_q8"], G["gather_ids"], q8_0=True), G["gather_q8_out"], "q8")
    assert np.array_equal(oracle.quantize_q8_0(G["gather_table"]), G["gather_q8"])
    assert_bitexact(oracle.layer_norm(G["ln_x"], G["ln_w"], G["ln_b"], 1e-5), G["ln_out"], "ln")
    assert_bitexact(oracle.rms_norm_mul(G["rms_x"], G["rms_g"], 1e-5), G["rms_out"], "rms")
    assert_bitexact(oracle.rope_ext(G["rope_x"], G["rope_pos"], 64, mode=2), G["rope_neox"], "neox")
    assert_bitexact(oracle.rope_ext(G["rope_x"], G["rope_pos"], 64, mode=0), G["rope_normal"], "normal")
    for name, op in UNARY.items():
        assert_bitexact(oracle.unary(getattr(oracle, op), G["act_x"]), G["act_" + name], name)
    assert_bitexact(oracle.leaky_relu(G["act_x"], 0.1), G["act_leaky"], "leaky")
    assert np.array_equal(oracle.gelu_table(0), G["gelu_table"])
    assert_bitexact(oracle.swiglu(G["swiglu_g"], G["swiglu_u"]), G["swiglu_out"], "swiglu")
    assert_bitexact(oracle.snake(G["snake_x"], G["snake_a"], G["snake_ai"]), G["snake_out"], "snake")
    assert_bitexact(oracle.group_norm_affine(G["gn_x"], 4, 1e-5, G["gn_w"], G["gn_b"], False), G["gn_out"], "gn")
    assert_bitexact(oracle.group_norm_affine(G["gn_x"], 4, 1e-5, G["gn_w"], G["gn_b"], True), G["gn_mish"], "gn mish")
    assert_bitexact(oracle.scale_diag_mask_soft_max(G["sm_x"], 0.125, 2), G["sm_out"], "softmax")
    ln = oracle.layer_norm(G["lnr_x"], G["lnr_w"], G["lnr_b"], 1e-5)
    assert_bitexact(oracle.rope_ext(ln.reshape(2, 6, 2, 64), G["lnr_pos"], 64, mode=2).reshape(ln.shape),
                    G["lnr_out"], "ln+rope")


@pytest.mark.gpu
def test_hip_matches_golden(cbx, G):
    import torch

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def host(t):
        torch.cuda.synchronize()
        return t.cpu().numpy()

    assert_bitexact(host(cbx.get_rows_add(dev(G["gather_table"]), dev(G["gather_ids"]), dev(G["gather_pos"]),
                                          dev(G["gather_pids"]))), G["gather_f32"], "gather")
    assert_bitexact(host(cbx.get_rows(dev(G["gather_table"].astype(np.float16)), dev(G["gather_ids"]))),
                    G["gather_f16"], "f16")
    assert_bitexact(host(cbx.get_rows(dev(G["gather_q8"]), dev(G["gather_ids"]), q8_0=True)), G["gather_q8_out"], "q8")
    assert_bitexact(host(cbx.layer_norm(dev(G["ln_x"]), dev(G["ln_w"]), dev(G["ln_b"]), 1e-5)), G["ln_out"], "ln")
    assert_bitexact(host(cbx.rms_norm_mul(dev(G["rms_x"]), dev(G["rms_g"]), 1e-5)), G["rms_out"], "rms")
    for mode, key in ((2, "rope_neox"), (0, "rope_normal")):
        c = cbx.RopeCache(64, mode=mode, n_pos=2048)
        assert_bitexact(host(cbx.rope_ext(dev(G["rope_x"]), dev(G["rope_pos"]), c)), G[key], key)
        c.close()
    for name, op in UNARY.items():
        got = host(cbx.unary(getattr(cbx, op), dev(G["act_x"])))
        if name == "gelu":
            assert_bitexact(got, G["act_gelu"], name)
        else:
            assert_close(got, G["act_" + name], x=G["act_x"], what=name)
    assert_bitexact(host(cbx.leaky_relu(dev(G["act_x"]), 0.1)), G["act_leaky"], "leaky")
    assert_close(host(cbx.swiglu(dev(G["swiglu_g"]), dev(G["swiglu_u"]))), G["swiglu_out"], what="swiglu")
    assert_close(host(cbx.snake(dev(G["snake_x"]), dev(G["snake_a"]), dev(G["snake_ai"]))), G["snake_out"],
                 x=G["snake_x"], what="snake")
    assert_bitexact(host(cbx.group_norm(dev(G["gn_x"]), 4, 1e-5, dev(G["gn_w"]), dev(G["gn_b"]))), G["gn_out"], "gn")
    assert_close(host(cbx.group_norm(dev(G["gn_x"]), 4, 1e-5, dev(G["gn_w"]), dev(G["gn_b"]), act=cbx.MISH)),
                 G["gn_mish"], x=G["gn_out"], what="gn mish")
    sm = host(cbx.scale_diag_mask_soft_max(dev(G["sm_x"]), 0.125, 2))
    assert np.all(np.abs(sm - G["sm_out"]) <= 1e-5 * np.abs(G["sm_out"]) + 1e-37), "softmax"
    assert_bitexact(sm[G["sm_out"] == 0], G["sm_out"][G["sm_out"] == 0], "softmax masked")
    c = cbx.RopeCache(64, mode=2, n_pos=2048)
    got = host(cbx.layer_norm_rope(dev(G["lnr_x"]), dev(G["lnr_w"]), dev(G["lnr_b"]), 1e-5, 64, dev(G["lnr_pos"]), c))
    c.close()
    assert_bitexact(got, G["lnr_out"], "ln+rope")
