"""One flow-encoder call's node list (flow_encoder.cpp:537-700; matmul,
conv and layout outputs given) planned on the host: every node claimed,
and the launches the reference's structure implies for n_blocks blocks over
T tokens and n_up blocks over 2T frames."""
import collections

import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.flow_encoder import FlowEncoderCall


@pytest.mark.parametrize("T,n_blocks,n_up", [(250, 6, 4), (7, 2, 1), (2, 1, 1)])
def test_plan_counts(T, n_blocks, n_up):
    e = FlowEncoderCall(T, n_blocks=n_blocks, n_up_blocks=n_up, device=False)
    plan = e.plan()
    names = {v: k for k, v in vars(C).items() if k.startswith("GL_") and isinstance(v, int)}
    got = collections.Counter(names[p[0]] for p in plan)
    L = n_blocks + n_up
    assert dict(got) == {
        "GL_GET_ROWS": 1,                     # the speech-token embedding
        # per block the w1 bias + silu; the two pre-lookahead convs' and the
        # up conv's bias (as (1, C)), the encoder_proj bias
        "GL_BIAS_ACT": L + 4,
        "GL_BIAS_ADD_TWO": L,                 # per block the v and k bias adds side by side
        # per block q's bias, then q + pos_bias_u and q + pos_bias_v (with
        # q's view as heads and pos_bias_u, pos_bias_v's as (64, 8, 1))
        "GL_BIAS_ADD_PAIR": L,
        "GL_VIEW": 3,                         # the three conv biases as (1, C)
        "GL_SOFT_MAX": L,                     # AC + BD -> scale(1/8) -> soft_max
        # per block x + (out + b) -> LN; w2 bias + residual -> the next LN
        # (the up stack's last: after_norm); the pre-lookahead's residual ->
        # the first block's LN; the two embed linears' bias -> their LN
        "GL_ADD_LAYER_NORM": 2 * L + 2,
        "GL_BIAS_RESIDUAL": 1,                # the 25 Hz stack's last w2 bias + residual
        "GL_LAYER_NORM": 1,                   # the 50 Hz stack's first LN (after the scale)
        "GL_SCALE": 2,                        # x sqrt(512) after each embed LN
        "GL_LEAKY_RELU": 1,                   # the pre-lookahead's conv1
    }
    assert sum(p[2] for p in plan) == len(e.graph.nodes)
    assert all(p[2] == 3 for p in plan if p[0] == C.GL_SOFT_MAX)
    assert all(p[2] == 6 for p in plan if p[0] == C.GL_BIAS_ADD_PAIR)
    assert e.graph.nodes[-1].dst == e.out and tuple(e.b.shape(e.out)) == (2 * T, 80)
