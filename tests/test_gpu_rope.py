"""ggml_rope_ext (NEOX and NORMAL) through the C ABI vs the oracle.

The cos/sin values come from the library's host-built table, formed with
ggml's recurrence and the host libm, the same values the oracle forms, so
results in range are bit-exact; positions outside the table use the
device's cosf/sinf and are held to the tolerance."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import RTOL_F16, assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.fixture(scope="module")
def cache64(cbx):
    c = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, freq_base=10000.0, n_pos=2048)
    yield c
    c.close()


def test_decode_steps_q_k(cbx, oracle, cache64):
    """T3 decode step: q, k [16 heads x 64] at positions 0..29 (one token per step)."""
    for step in range(30):
        for t in range(2):
            x = W.normal(W.seed_of(1, 2 + t) + 97 * step, (1, 16, 64))     # (n_tok, n_head, head_dim)
            pos = np.array([step], dtype=np.int32)
            got = host(cbx.rope_ext(dev(x), dev(pos), cache64))
            exp = oracle.rope_ext(x, pos, 64, mode=2)
            assert_bitexact(got, exp, f"step {step}")
            if step == 0:
                assert_bitexact(got, x, "position 0 is the identity")


def test_cfm_rope_batch(cbx, oracle, cache64):
    """[2, 500, 8 x 64] at positions 0..499 (ggml ne (64, 8, 500, 2))."""
    x = W.normal(W.seed_of(3, 4), (2, 500, 8, 64))
    pos = np.arange(500, dtype=np.int32)
    got = host(cbx.rope_ext(dev(x), dev(pos), cache64))
    exp = oracle.rope_ext(x, pos, 64, mode=2, nth=8)
    assert_close(got, exp, what="rope cfm")
    assert_bitexact(got, exp, "rope cfm")
    # rotation preserves each pair's norm
    xe, ge = x.astype(np.float64), got.astype(np.float64)
    n0 = xe[..., :32] ** 2 + xe[..., 32:] ** 2
    n1 = ge[..., :32] ** 2 + ge[..., 32:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


def test_serving_f16_positions(cbx, oracle, cache64):
    """64 streams, f16 storage, positions U[0,2048)."""
    x = W.normal(W.seed_of(5, 4), (64, 16, 64)).astype(np.float16)
    pos = W.randint(W.seed_of(5, 5), (64,), 0, 2048)
    got = host(cbx.rope_ext(dev(x), dev(pos), cache64))
    exp = oracle.rope_ext(x, pos, 64, mode=2)
    assert_close(got.astype(np.float32), exp.astype(np.float32), rtol=RTOL_F16, what="rope f16")
    assert_bitexact(got, exp, "rope f16")


def test_s3_encoder_shape_partial_dims_normal_mode(cbx, oracle):
    """The reference's real call: (64, 20 heads, T) NEOX; plus NORMAL mode and n_dims < head_dim."""
    x = W.normal(41, (37, 20, 64))
    pos = np.arange(37, dtype=np.int32)
    c = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=64)
    assert_bitexact(host(cbx.rope_ext(dev(x), dev(pos), c)), oracle.rope_ext(x, pos, 64, mode=2), "s3 shape")
    c.close()
    for mode in (0, 2):
        c = cbx.RopeCache(32, mode=mode, freq_base=500000.0, n_pos=100)
        got = host(cbx.rope_ext(dev(x), dev(pos), c))
        exp = oracle.rope_ext(x, pos, 32, mode=mode, freq_base=500000.0)
        assert_bitexact(got, exp, f"mode {mode} n_dims 32")
        assert_bitexact(got[..., 32:], x[..., 32:], "tail copied")
        c.close()


def test_yarn_and_freq_factors(cbx, oracle):
    x = W.normal(42, (50, 4, 128))
    pos = np.arange(50, dtype=np.int32) * 37
    ff = W.uniform_range(43, (64,), 1.0, 4.0)
    kw = dict(mode=2, n_ctx_orig=4096, freq_base=10000.0, freq_scale=0.25, ext_factor=1.0, attn_factor=1.0,
              beta_fast=32.0, beta_slow=1.0)
    c = cbx.RopeCache(128, n_pos=4096, freq_factors=ff, **kw)
    got = host(cbx.rope_ext(dev(x), dev(pos), c))
    exp = oracle.rope_ext(x, pos, 128, freq_factors=ff, **kw)
    assert_bitexact(got, exp, "yarn")
    c.close()


def test_positions_outside_table(cbx, oracle, cache64):
    """Out-of-table positions (negative, >= n_pos) are computed on the device."""
    x = W.normal(44, (6, 3, 64))
    pos = np.array([-5, 2047, 2048, 5000, 0, 70000], dtype=np.int32)
    got = host(cbx.rope_ext(dev(x), dev(pos), cache64))
    exp = oracle.rope_ext(x, pos, 64, mode=2)
    # device cosf/sinf may differ from glibc by an ulp or two: bound by the pair magnitude
    pair = np.concatenate([np.hypot(x[..., :32], x[..., 32:])] * 2, axis=-1)
    assert_close(got, exp, x=pair, atol_x=2.0 ** -20, what="rope out of table")
    assert_bitexact(got[[1, 4]], exp[[1, 4]], "in-table rows")


def test_in_place(cbx, oracle, cache64):
    x = W.normal(45, (9, 2, 64))
    pos = np.arange(9, dtype=np.int32)
    t = dev(x)
    cbx.rope_ext(t, dev(pos), cache64, out=t)
    assert_bitexact(host(t), oracle.rope_ext(x, pos, 64), "in place")


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("ne0,n_dims", [(64, 64), (66, 64), (64, 20), (128, 40)])
def test_vector_and_scalar_forms(cbx, oracle, dtype, mode, ne0, n_dims):
    """Four pairs a lane with vector loads (n_dims % 8 == 0, aligned head
    rows) and the pair-a-lane form (ne0 = 66: head rows off the vector
    alignment; n_dims 20 and 40: n_dims % 8 != 0), both pairings, f32 and
    f16, positions in and past the table: each as the oracle."""
    x = W.normal(46 + ne0 + n_dims, (19, 12, ne0)).astype(dtype)
    pos = np.concatenate([W.randint(47, (17,), 0, 200), [250, 400]]).astype(np.int32)
    c = cbx.RopeCache(n_dims, mode=mode, n_ctx_orig=2048, n_pos=200)
    got = host(cbx.rope_ext(dev(x), dev(pos), c))
    exp = oracle.rope_ext(x, pos, n_dims, mode=mode)
    assert_bitexact(got[:17], exp[:17], f"rope in table mode {mode} ne0 {ne0} n_dims {n_dims}")
    x32 = x.astype(np.float32)
    half = n_dims // 2
    if mode == 2:
        pr = np.hypot(x32[..., :half], x32[..., half:n_dims])
        pair = np.concatenate([pr, pr, np.abs(x32[..., n_dims:])], axis=-1)
    else:
        pr = np.repeat(np.hypot(x32[..., 0:n_dims:2], x32[..., 1:n_dims:2]), 2, axis=-1)
        pair = np.concatenate([pr, np.abs(x32[..., n_dims:])], axis=-1)
    rt = 2.0 ** -10 if dtype == np.float16 else 1e-5
    assert_close(got[17:].astype(np.float32), exp[17:].astype(np.float32), x=pair[17:], rtol=rt,
                 atol_x=2.0 ** -10 if dtype == np.float16 else 2.0 ** -20, what="rope past the table")
    c.close()
