"""The oracle's T3 decode-step composition (cbxo_t3_token_step: one token's
element-wise nodes in t3.cpp:446-546's order) against the same nodes
evaluated one at a time with the oracle's pinned ops, in the order and with
the operands the reference's builder gives them.  Planting a wrong operand
(the residual taken from h instead of the attention residual, LN-1's
parameters of the wrong block, the mask without n_past) fails it."""
import numpy as np
import pytest

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact

H = W.T3_HEADS


def small_inputs(L=3, max_ctx=64):
    inp = W.t3_token_inputs(L, max_ctx)
    return inp


def node_by_node(O, inp, token, position, n_past, eps=1e-5):
    """t3.cpp:446-546 at N_new = 1, node by node."""
    L, D = inp["ln1_w"].shape
    n_kv = n_past + 1
    tok = O.cpy(O.get_rows(inp["speech_emb"], np.array([token], np.int32)), np.float32)
    pos = O.cpy(O.get_rows(inp["pos_embd"], np.array([position], np.int32)), np.float32)
    h = O.add(tok, pos)
    out = {"h0": h, "blocks": []}
    scale = np.float32(1.0) / np.sqrt(np.float32(D // H))
    for il in range(L):
        ln1 = O.add(O.mul(O.norm(h, eps), inp["ln1_w"][il]), inp["ln1_b"][il])
        qkv = O.add(inp["qkv_mm"][il][None, :], inp["qkv_b"][il])
        kq = np.ascontiguousarray(inp["kq"][il, :H * n_kv].reshape(H, 1, n_kv))
        probs = O.soft_max(O.diag_mask_inf(O.scale(kq, float(scale)), n_past))
        attn_res = O.add(O.add(inp["out_mm"][il][None, :], inp["out_b"][il]), h)
        ln2 = O.add(O.mul(O.norm(attn_res, eps), inp["ln2_w"][il]), inp["ln2_b"][il])
        gelu = O.unary(O.GELU, O.add(inp["fc_mm"][il][None, :], inp["fc_b"][il]))
        h = O.add(O.add(inp["proj_mm"][il][None, :], inp["proj_b"][il]), attn_res)
        out["blocks"].append({"ln1": ln1, "qkv": qkv, "probs": probs.reshape(H, n_kv), "attn_res": attn_res,
                              "ln2": ln2, "gelu": gelu, "h": h})
    out["y"] = O.add(O.mul(O.norm(h, eps), inp["out_w"]), inp["out_b_final"])
    return out


@pytest.mark.parametrize("n_past,token,position", [(0, 0, 0), (5, 6562, 5), (63, 17, 8195)])
def test_composition_matches_nodes(oracle, n_past, token, position):
    inp = small_inputs()
    got = oracle.T3TokenStep(inp, n_past).run(token, position)
    exp = node_by_node(oracle, inp, token, position, n_past)
    assert_bitexact(got["h0"], exp["h0"], "h0")
    assert_bitexact(got["y"], exp["y"], "final LN")
    for il, e in enumerate(exp["blocks"]):
        for k, v in e.items():
            assert_bitexact(got[k][il].reshape(v.shape), v, f"block {il} {k}")


def test_scores_mask_nothing_at_n_kv(oracle):
    """With N_new = 1 the mask hides columns past n_past only, so the
    probabilities of a block sum to 1 over all n_past + 1 columns and none is
    zeroed (the n_kv columns are exactly the cache so far)."""
    inp = small_inputs(L=1)
    out = oracle.T3TokenStep(inp, 40).run(3, 40)
    p = out["probs"][0].astype(np.float64)
    assert p.shape == (H, 41)
    assert (p > 0).all()
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=1e-6)
