"""One T3 decode step's element-wise nodes (t3.cpp:446-546 at N_new = 1,
the 24 blocks of Chatterbox-Turbo's T3 with their matmul outputs given) run
through the node-list executor, token after token, checked node by node
against the oracle: the input embedding, every block's LN-1, qkv bias, score
probabilities, attention residual, LN-2, fc bias + GELU and output h, and
the final LayerNorm.  The list is captured once into a HIP graph and
re-pointed at each next token with cbx_graph_exec_update (new n_past: score
views one column longer, the mask's n_past), the token and position written
to their device tensors in between."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import t3_decode as T
from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact

pytestmark = pytest.mark.gpu

STEPS = [(0, 5, 0), (1, 6562, 1), (37, 100, 37), (511, 2, 8195), (1023, 77, 1023), (2, 0, 2)]


@pytest.fixture(scope="module")
def inputs():
    return W.t3_token_inputs()


def check_probs(got, exp, what):
    d = np.abs(got.astype(np.float64) - exp.astype(np.float64))
    bad = d > 1e-5 * np.abs(exp.astype(np.float64)) + 1e-37
    assert not bad.any(), f"{what}: {int(bad.sum())} of {got.size} off, max |d| {d.max():.3g}"


def compare(st, ref, what):
    out = {k: v.cpu().numpy() for k, v in st.out.items()}
    assert_bitexact(out["h0"], ref["h0"], f"{what}: embedding h")
    assert_bitexact(out["y"], ref["y"], f"{what}: final LayerNorm")
    for k in ("ln1", "qkv", "attn_res", "ln2", "gelu", "h"):
        assert_bitexact(out[k], ref[k], f"{what}: {k}")
    for il in range(st.n_blocks):
        check_probs(st.probs(il).cpu().numpy(), ref["probs"][il], f"{what}: block {il} probabilities")


def test_tokens_through_one_exec(cbx, oracle, inputs):
    dev = T.upload(inputs)
    st = T.T3DecodeStep(dev, STEPS[0][0])
    ex = st.graph.capture(st.keep)
    assert ex.n_launches == st.launches() == 121
    try:
        for k, (n_past, token, position) in enumerate(STEPS):
            if k:
                st.retarget(n_past)
                assert ex.update(st.graph, st.keep) is True, f"step {k}: not updated in place"
            for v in st.out.values():
                v.fill_(float("nan"))
            st.set_token(token, position)
            ex.launch()
            torch.cuda.synchronize()
            ref = oracle.T3TokenStep(inputs, n_past).run(token, position)
            compare(st, ref, f"n_past {n_past}, token {token} at {position}")
    finally:
        ex.close()


def test_compute_matches_exec_and_plan(cbx, inputs):
    """cbx_graph_compute on the same list gives the replay's bits, and the
    plan is the embedding + LN-1, then per block the qkv bias, the softmax,
    the residual join + LN-2, the fc bias + GELU and the residual join + the
    next LayerNorm."""
    dev = T.upload(inputs)
    st = T.T3DecodeStep(dev, 300)
    kinds = [p[0] for p in st.graph.plan(st.keep)]
    per_block = [cbx.GL_BIAS_ACT, cbx.GL_SOFT_MAX, cbx.GL_ADD_LAYER_NORM, cbx.GL_BIAS_ACT, cbx.GL_ADD_LAYER_NORM]
    assert kinds == [cbx.GL_GET_ROWS_ADD_LAYER_NORM] + per_block * st.n_blocks
    st.set_token(4000, 300)
    assert st.graph.compute(st.keep) == 121
    torch.cuda.synchronize()
    eager = {k: v.clone() for k, v in st.out.items()}
    ex = st.graph.capture(st.keep)
    try:
        for v in st.out.values():
            v.fill_(float("nan"))
        ex.launch()
        torch.cuda.synchronize()
        for k, v in st.out.items():
            a, b = v.view(torch.int32), eager[k].view(torch.int32)
            if k == "probs":
                a, b = a[:, : 16 * 301], b[:, : 16 * 301]
            assert torch.equal(a, b), k
    finally:
        ex.close()
