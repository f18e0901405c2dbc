"""One flow-encoder call's element-wise node list (flow_encoder.cpp:537-700;
matmul, conv and layout outputs given; chatterbox_amdvulkan_amd/
flow_encoder.py) run launch by launch, each launch checked against the
oracle on the inputs it read from the device (tests/_node_checks.py):
bit-exact for the speech-token gather, the bias adds, the pos_bias adds,
the joins, the LayerNorms (eps 1e-5 and 1e-12), the sqrt(512) scales and
the pre-lookahead's LeakyReLU; the f32 bar for SiLU and the softmax.  Then
the whole list through cbx_graph_compute and a captured cbx_graph_exec:
the same output bits."""
import numpy as np
import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.flow_encoder import FlowEncoderCall
from tests._node_checks import full_list_same_bits, host, run_and_check

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,n_blocks,n_up", [(40, 2, 1), (97, 1, 2)])
def test_flow_encoder_launch_by_launch(cbx, oracle, T, n_blocks, n_up):
    e = FlowEncoderCall(T, seed=T, n_blocks=n_blocks, n_up_blocks=n_up)
    plan = e.plan()
    assert all(p[0] != C.GL_UNSUPPORTED for p in plan)
    for k, launch in enumerate(plan):
        run_and_check(e.graph, e.b.at, e.keep, oracle, launch, k)
    assert np.isfinite(host(e.b.at(e.out))).all()
    full_list_same_bits(e.graph, e.b.at, e.keep, e.out, plan)


def test_flow_encoder_full_size_runs(cbx):
    """10 s of audio (250 speech tokens; 6 blocks over 250, 4 over 500:
    72 launches) through one captured graph: finite (500, 80) output."""
    e = FlowEncoderCall(250, seed=2)
    ex = e.graph.capture(e.keep)
    try:
        assert ex.n_launches == 72
        ex.launch()
        out = host(e.b.at(e.out))
    finally:
        ex.close()
    assert out.shape == (500, 80) and np.isfinite(out).all()
