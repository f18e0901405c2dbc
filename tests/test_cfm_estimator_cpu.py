"""The CFM estimator's node list (cfm_decoder.cpp:395-558, matmul outputs
given) planned on the host: every node claimed, and the launches the
reference's structure implies for n_mid mid blocks and n_tr transformers a
stage."""
import collections

import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.cfm_estimator import CFMEstimator


@pytest.mark.parametrize("T,n_mid,n_tr", [(500, 12, 4), (37, 2, 3), (16, 0, 1)])
def test_plan_counts(T, n_mid, n_tr):
    e = CFMEstimator(T, n_mid=n_mid, n_tr=n_tr, device=False)
    plan = e.plan()
    names = {v: k for k, v in vars(C).items() if k.startswith("GL_") and isinstance(v, int)}
    got = collections.Counter(names[p[0]] for p in plan)
    n_res = n_mid + 2                      # down, mid blocks, up
    n_t = n_res * n_tr                     # transformer blocks
    exp = {
        "GL_CAUSAL_CONV1D": 2 * n_res + 3,      # two causal blocks a resnet, down and up convs, final block
        "GL_LAYER_NORM_MASK": 2 * n_res + 1,    # the causal blocks' LN -> Mish -> mask
        "GL_SOFT_MAX": n_t,                     # scale -> soft_max
        "GL_ADD_LAYER_NORM": 2 * n_t,           # every transformer LayerNorm, joined to its residual
        # gelu_erf per transformer; t and r time MLPs (bias + silu, bias);
        # final_proj's bias
        "GL_BIAS_ACT": n_t + 4 + 1,
        # mul(x, mask) before each res_conv; mul(h, mask) before final_proj
        # and after it
        "GL_BINARY": n_res + 2,
        # a resnet's mlp bias -> (C, 1) view -> add over the frames; a
        # stack's last ff.2 bias -> residual add (no norm follows)
        "GL_BIAS_RESIDUAL": 2 * n_res,
        "GL_UNARY": n_res,                      # mish(t_mix) in every resnet
        "GL_CONCAT": 5,                         # t|r, the three packing concats, the skip join
    }
    assert dict(got) == exp
    assert sum(p[2] for p in plan) == len(e.graph.nodes)
    for kind, first, n, flags in plan:
        if kind == C.GL_BINARY:
            op = e.graph.nodes[first].op
            assert flags == (C.BINARY_MUL if op == C.GOP_MUL else C.BINARY_ADD)
        if kind == C.GL_BIAS_RESIDUAL:
            assert n == (3 if e.graph.nodes[first + 1].op == C.GOP_VIEW else 2)
    # the kernel launches at the reference's sizes
    if (T, n_mid, n_tr) == (500, 12, 4):
        assert sum(1 for p in plan if p[0] != C.GL_VIEW) == 352
