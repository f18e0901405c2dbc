"""cbx_layer_norm_rope (LayerNorm+affine, then RoPE of the row viewed as
heads) vs the oracle's layer_norm followed by its rope_ext, and vs the two
standalone entry points."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact, assert_close

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_cfm_shape(cbx, oracle):
    """[2, 500, 8 heads x 64], positions 0..499, NEOX, theta 10000."""
    inp = W.cfm_inputs()
    x, w, b, pos = inp["xa"], inp["wa"], inp["ba"], inp["pos"]
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    got = host(cbx.layer_norm_rope(dev(x), dev(w), dev(b), 1e-5, 64, dev(pos), cache))
    ln = oracle.layer_norm(x, w, b, 1e-5, nth=8)
    exp = oracle.rope_ext(ln.reshape(2, W.CFM_T, 8, 64), pos, 64, mode=2, nth=8).reshape(x.shape)
    assert_bitexact(got, exp, "ln+rope")
    two = cbx.rope_ext(cbx.layer_norm(dev(x), dev(w), dev(b), 1e-5).view(2, W.CFM_T, 8, 64), dev(pos), cache)
    assert_bitexact(got, host(two).reshape(x.shape), "= layer_norm then rope_ext")
    cache.close()


@pytest.mark.parametrize("C,hd,n_dims,mode", [(256, 64, 64, 2), (1024, 128, 96, 2), (512, 64, 32, 0),
                                              (192, 64, 64, 0), (64, 32, 16, 2), (1000, 40, 40, 2),
                                              (1024, 256, 256, 2), (512, 128, 64, 2), (1024, 128, 128, 0),
                                              (96, 16, 8, 2), (48, 12, 12, 2), (96, 24, 20, 2),
                                              (240, 24, 20, 0)])
def test_shapes_modes_partial_dims(cbx, oracle, C, hd, n_dims, mode):
    """Row widths for every vector count, NORMAL and NEOX pairs, rotation of
    only the first n_dims of each head (the rest copied), ragged C; NEOX
    partners 2 to 32 lanes apart (taken from other lanes' registers) and
    heads that do not tile a wave (hd = 40) or whose half is not a power of
    two in vectors (n_dims = 96), which take the partners from LDS; NEOX
    with n_dims % 8 == 4 (half not a multiple of 4, so one 4-vector of each
    head straddles the half boundary and its cos/sin are read pair by
    pair)."""
    T, B = 37, 2
    x = W.normal(90 + C, (B, T, C), 0.3, 2.0)
    w = W.normal(91, (C,), 1.0, 0.05)
    b = W.normal(92, (C,), 0.0, 0.05)
    pos = W.randint(93, (T,), 0, 4096)
    cache = cbx.RopeCache(n_dims, mode=mode, n_ctx_orig=4096, freq_base=10000.0, n_pos=4096)
    got = host(cbx.layer_norm_rope(dev(x), dev(w), dev(b), 1e-5, hd, dev(pos), cache))
    ln = oracle.layer_norm(x, w, b, 1e-5)
    exp = oracle.rope_ext(ln.reshape(B, T, C // hd, hd), pos, n_dims, mode=mode, n_ctx_orig=4096).reshape(x.shape)
    assert_bitexact(got, exp, f"ln+rope C={C} hd={hd} n_dims={n_dims} mode={mode}")
    cache.close()


@pytest.mark.parametrize("C,hd,n_dims,mode", [(1024, 128, 96, 2), (1000, 40, 40, 2), (768, 64, 64, 0),
                                              (512, 128, 64, 2), (1024, 256, 256, 2)])
def test_many_rows_one_wave_a_row(cbx, oracle, C, hd, n_dims, mode):
    """600 rows: every width takes one wave a row (the launch holds at least
    two waves a CU), with partners from registers (hd = 64) or from LDS."""
    T, B = 300, 2
    x = W.normal(190 + C, (B, T, C), 0.1, 1.5)
    w = W.normal(191, (C,), 1.0, 0.05)
    b = W.normal(192, (C,), 0.0, 0.05)
    pos = W.randint(193, (T,), 0, 4096)
    cache = cbx.RopeCache(n_dims, mode=mode, n_ctx_orig=4096, freq_base=10000.0, n_pos=4096)
    got = host(cbx.layer_norm_rope(dev(x), dev(w), dev(b), 1e-5, hd, dev(pos), cache))
    ln = oracle.layer_norm(x, w, b, 1e-5, nth=8)
    exp = oracle.rope_ext(ln.reshape(B, T, C // hd, hd), pos, n_dims, mode=mode, n_ctx_orig=4096,
                          nth=8).reshape(x.shape)
    assert_bitexact(got, exp, f"ln+rope C={C} hd={hd} n_dims={n_dims} mode={mode}, 600 rows")
    cache.close()


def test_no_affine_in_place_and_positions_past_table(cbx, oracle):
    """w = b = NULL; y == x; positions beyond the table's rows use the device
    recurrence exactly as cbx_rope_ext does."""
    x = W.normal(94, (3, 20, 256))
    pos = np.arange(50, 70, dtype=np.int32)
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=60)
    t = dev(x)
    cbx.layer_norm_rope(t, None, None, 1e-12, 64, dev(pos), cache, out=t)
    two = cbx.rope_ext(cbx.layer_norm(dev(x), None, None, 1e-12).view(3, 20, 4, 64), dev(pos), cache)
    assert_bitexact(host(t), host(two).reshape(x.shape), "in place, fallback positions")
    ln = oracle.layer_norm(x, None, None, 1e-12)
    exp = oracle.rope_ext(ln.reshape(3, 20, 4, 64), pos, 64, mode=2).reshape(x.shape)
    assert_close(host(t), exp, x=ln, what="vs oracle")
    cache.close()


@pytest.mark.parametrize("n_pos", [0, 1, 45, 2048])
def test_positions_in_order_and_table_ends(cbx, oracle, n_pos):
    """Positions 0, 1, .. T-1 (the kernel reads the cos/sin row of position
    t for token t before the position itself arrives) against tables that
    end before, inside and after the sequence, and an empty one (no row to
    read ahead: every position takes the device recurrence); then the same
    tokens at positions 5, 6, .. (every speculative row is the wrong one)."""
    B, T = 2, 90
    x = W.normal(95, (B, T, 512))
    w = W.normal(96, (512,), 1.0, 0.02)
    b = W.normal(97, (512,), 0.0, 0.02)
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=n_pos)
    for off in (0, 5):
        pos = np.arange(off, off + T, dtype=np.int32)
        got = host(cbx.layer_norm_rope(dev(x), dev(w), dev(b), 1e-5, 64, dev(pos), cache))
        two = cbx.rope_ext(cbx.layer_norm(dev(x), dev(w), dev(b), 1e-5).view(B, T, 8, 64), dev(pos), cache)
        assert_bitexact(got, host(two).reshape(x.shape), f"n_pos {n_pos}, positions from {off}")
        ln = oracle.layer_norm(x, w, b, 1e-5)
        exp = oracle.rope_ext(ln.reshape(B, T, 8, 64), pos, 64, mode=2).reshape(x.shape)
        assert_close(got, exp, x=ln, what=f"n_pos {n_pos}, positions from {off} vs oracle")
    cache.close()


def test_rejects_bad_shapes(cbx):
    x = dev(W.normal(95, (2, 8, 256)))
    pos = dev(np.arange(8, dtype=np.int32))
    cache = cbx.RopeCache(64, mode=2, n_pos=64)
    with pytest.raises(cbx.CbxError, match="head_dim"):
        cbx.layer_norm_rope(x, None, None, 1e-5, 48, pos, cache)          # does not divide 256
    big = cbx.RopeCache(128, mode=2, n_pos=64)
    with pytest.raises(cbx.CbxError, match="n_dims"):
        cbx.layer_norm_rope(x, None, None, 1e-5, 64, pos, big)
    with pytest.raises(cbx.CbxError, match="pos"):
        cbx.layer_norm_rope(x, None, None, 1e-5, 64, dev(np.arange(7, dtype=np.int32)), cache)
    cache.close()
    big.close()
