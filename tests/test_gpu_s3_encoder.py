"""One S3 encoder call's element-wise node list (s3enc.cpp:124-290; matmul,
conv and FSMN outputs given; chatterbox_amdvulkan_amd/s3_encoder.py) run
launch by launch, each launch checked against the oracle on the inputs it
read from the device (tests/_node_checks.py): bit-exact for the bias adds,
the joins, the LayerNorms and the RoPEs (q and k as 20 heads of 64, NEOX,
base 10000); the f32 bar for GELU-erf and the softmax.  Then the whole list
through cbx_graph_compute and a captured cbx_graph_exec: the same output
bits."""
import numpy as np
import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd.s3_encoder import HEAD_DIM, ROPE_BASE, ROPE_MAX, S3EncoderCall
from tests._node_checks import full_list_same_bits, host, run_and_check

pytestmark = pytest.mark.gpu

ROPE = dict(n_dims=HEAD_DIM, mode=2, n_ctx_orig=ROPE_MAX, freq_base=ROPE_BASE)


@pytest.mark.parametrize("T_mel,n_layer", [(64, 2), (150, 1)])
def test_encoder_launch_by_launch(cbx, oracle, T_mel, n_layer):
    e = S3EncoderCall(T_mel, seed=T_mel, n_layer=n_layer)
    try:
        plan = e.plan()
        assert all(p[0] != C.GL_UNSUPPORTED for p in plan)
        for k, launch in enumerate(plan):
            run_and_check(e.graph, e.b.at, e.keep, oracle, launch, k, rope=ROPE)
        assert np.isfinite(host(e.b.at(e.out))).all()
        full_list_same_bits(e.graph, e.b.at, e.keep, e.out, plan)
    finally:
        e.close()


def test_encoder_full_size_runs(cbx):
    """10 s of audio (1000 mel frames, 250 tokens, 6 layers: 51 launches)
    through one captured graph: finite output."""
    e = S3EncoderCall(1000, seed=2)
    try:
        ex = e.graph.capture(e.keep)
        try:
            assert ex.n_launches == 51
            ex.launch()
            out = host(e.b.at(e.out))
        finally:
            ex.close()
        assert out.shape == (250, 1280) and np.isfinite(out).all()
    finally:
        e.close()
