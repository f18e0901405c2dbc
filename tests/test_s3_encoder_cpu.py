"""One S3 encoder call's node list (s3enc.cpp:124-290, matmul, conv and
FSMN outputs given) planned on the host: every node claimed, and the
launches the reference's structure implies for n_layer layers."""
import collections

import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.s3_encoder import S3EncoderCall


@pytest.mark.parametrize("T_mel,n_layer", [(1000, 6), (37, 2), (8, 1)])
def test_plan_counts(T_mel, n_layer):
    e = S3EncoderCall(T_mel, n_layer=n_layer, device=False)
    plan = e.plan()
    names = {v: k for k, v in vars(C).items() if k.startswith("GL_") and isinstance(v, int)}
    got = collections.Counter(names[p[0]] for p in plan)
    L = n_layer
    assert dict(got) == {
        # the two front convs' bias (as (1, C)) + gelu_erf; per layer the fc
        # bias + gelu_erf
        "GL_BIAS_ACT": 2 + L,
        "GL_BIAS_ADD_TWO": L,                 # the q and v bias adds side by side
        "GL_VIEW": 2 + 2 * L,                 # the front biases as (1, C); q and k as heads
        "GL_ROPE_TWO": L,                     # q and k side by side
        "GL_BINARY": L,                       # add(fsmn, v)
        "GL_SOFT_MAX": L,                     # scale -> soft_max
        # out bias + the FSMN join; the last layer's proj bias + residual
        "GL_BIAS_RESIDUAL": L + 1,
        # x + attn -> LN; proj bias + residual -> the next layer's LN
        "GL_ADD_LAYER_NORM": L + (L - 1),
        "GL_LAYER_NORM": 1,                   # the first layer's LN
    }
    assert sum(p[2] for p in plan) == len(e.graph.nodes)
    assert e.T_tok == ((T_mel - 1) // 2) // 2 + 1
