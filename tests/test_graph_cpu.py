"""The node-list planner (cbx_graph_plan) on the host: which of the
reference's ggml op chains become one fused launch, when an intermediate
that someone else reads blocks the fusion, and how bad lists are refused.
Planning reads only shapes, types and addresses, so host tensors stand in
for device memory; nothing here launches a kernel."""
import ctypes

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import cbxops as C

from tests._hift_graph import HiftGraph


def f32(*shape):
    return torch.zeros(shape, dtype=torch.float32)


def t3_input(g: C.Graph, n_tok=6, D=64, residual_read=True):
    """t3.cpp:446-466: get_rows -> cast -> get_rows -> cast -> add -> norm -> mul -> add
    (+ the residual add that reads h again when residual_read)."""
    tok = g.tensor(f32(50, D))
    ids = g.tensor(torch.zeros(n_tok, dtype=torch.int32))
    pos = g.tensor(f32(40, D))
    pids = g.tensor(torch.zeros(n_tok, dtype=torch.int32))
    w, b = g.tensor(f32(D)), g.tensor(f32(D))
    t = [g.tensor(f32(n_tok, D)) for _ in range(9)]
    g.node(C.GOP_GET_ROWS, t[0], (tok, ids))
    g.node(C.GOP_CPY, t[1], (t[0],))
    g.node(C.GOP_GET_ROWS, t[2], (pos, pids))
    g.node(C.GOP_CPY, t[3], (t[2],))
    g.node(C.GOP_ADD, t[4], (t[1], t[3]))          # h
    g.node(C.GOP_NORM, t[5], (t[4],), fparam=1e-5)
    g.node(C.GOP_MUL, t[6], (t[5], w))
    g.node(C.GOP_ADD, t[7], (t[6], b))
    if residual_read:
        g.node(C.GOP_ADD, t[8], (t[7], t[4]))     # stands for attn_residual = add(cur, h)
    return t


def test_t3_input_chain_is_one_launch():
    g = C.Graph()
    t3_input(g)
    plan = g.plan()
    assert plan[0] == (C.GL_GET_ROWS_ADD_LAYER_NORM, 0, 8, 0)   # h is read again: stored
    assert plan[1] == (C.GL_BINARY, 8, 1, C.BINARY_ADD)         # a plain residual add: cbx_binary


def t3_input_concat(g: C.Graph, prompt=True, casts=True, D=64, n_pre=1, n_a=5, n_b=7, cast_type=torch.float32,
                    dim=1):
    """t3.cpp:432-466 with the conditioning prefix: [get_rows(speech, prompt)
    -> cast -> concat(prefix, ., 1) ->] get_rows(text, tokens) -> cast ->
    concat -> get_rows(pos) -> cast -> add -> norm -> mul -> add, then a
    node that reads h again (the block's residual).  Returns the tensors."""
    n = n_pre + (n_a if prompt else 0) + n_b
    pre = g.tensor(f32(n_pre, D))
    sp, tx, ps = g.tensor(f32(30, D)), g.tensor(f32(40, D)), g.tensor(f32(50, D))
    ia = g.tensor(torch.zeros(n_a, dtype=torch.int32))
    ib = g.tensor(torch.zeros(n_b, dtype=torch.int32))
    ip = g.tensor(torch.zeros(n, dtype=torch.int32))
    w, b = g.tensor(f32(D)), g.tensor(f32(D))

    def gather(table, ids, rows):
        v = g.tensor(f32(rows, D))
        g.node(C.GOP_GET_ROWS, v, (table, ids))
        if casts:
            c = g.tensor(torch.zeros(rows, D, dtype=cast_type))
            g.node(C.GOP_CPY, c, (v,))
            v = c
        return v

    seq, rows = pre, n_pre
    if prompt:
        v = gather(sp, ia, n_a)
        rows += n_a
        cat = g.tensor(f32(rows, D))
        g.node(C.GOP_CONCAT, cat, (seq, v), iparam=dim)
        seq = cat
    v = gather(tx, ib, n_b)
    rows += n_b
    cat = g.tensor(f32(rows, D))
    g.node(C.GOP_CONCAT, cat, (seq, v), iparam=dim)
    seq = cat
    pv = gather(ps, ip, n)
    t = [g.tensor(f32(n, D)) for _ in range(5)]
    g.node(C.GOP_ADD, t[0], (seq, pv))              # h
    g.node(C.GOP_NORM, t[1], (t[0],), fparam=1e-5)
    g.node(C.GOP_MUL, t[2], (t[1], w))
    g.node(C.GOP_ADD, t[3], (t[2], b))
    g.node(C.GOP_ADD, t[4], (t[3], t[0]))          # stands for the residual read of h
    return t


@pytest.mark.parametrize("prompt,casts,n_nodes", [(True, True, 12), (True, False, 9), (False, True, 9),
                                                  (False, False, 7)])
def test_t3_input_with_conditioning_prefix_is_one_launch(prompt, casts, n_nodes):
    g = C.Graph()
    t3_input_concat(g, prompt=prompt, casts=casts)
    plan = g.plan()
    assert plan[0] == (C.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM, 0, n_nodes, 0)   # h is read later: stored
    assert plan[1] == (C.GL_BINARY, n_nodes, 1, C.BINARY_ADD)                # the plain residual add


def test_t3_input_with_prefix_unread_sum_and_refusals():
    # h read only by the norm: not stored (flag 1)
    g = C.Graph()
    t = t3_input_concat(g)
    g.nodes.pop()
    assert g.plan() == [(C.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM, 0, 12, 1)]
    # a cast to F16 rounds: not this chain
    g = C.Graph()
    t3_input_concat(g, cast_type=torch.float16)
    assert g.plan()[0][0] != C.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM
    # concat along another dimension: not this chain
    g = C.Graph()
    t3_input_concat(g, dim=0)
    assert g.plan()[0][0] != C.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM
    # an intermediate kept by the caller: not fused
    g = C.Graph()
    t = t3_input_concat(g)
    concat_out = g.nodes[2].dst
    assert g.nodes[2].op == C.GOP_CONCAT
    assert g.plan(keep=[concat_out])[0][0] != C.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM


def test_t3_input_with_prefix_hand_made_launch_is_refused():
    """A launch of this kind whose node count does not match the chain is
    refused before anything runs (no device needed)."""
    g = C.Graph()
    t3_input_concat(g)
    Tn, Nn, _ = g._arrays([])
    bad = C.GLaunch(C.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM, 0, 11, 0)
    L = C.load()
    assert L.cbx_graph_launch(Tn, len(g._descs), Nn, len(g.nodes), ctypes.byref(bad), None) == C.ERR_INVALID_ARG
    assert "does not fit" in C.last_error()


def test_t3_input_unread_sum_is_not_stored():
    g = C.Graph()
    t3_input(g, residual_read=False)
    assert g.plan() == [(C.GL_GET_ROWS_ADD_LAYER_NORM, 0, 8, 1)]


def test_kept_intermediate_blocks_fusion():
    g = C.Graph()
    t = t3_input(g, residual_read=False)
    # the caller needs the position rows themselves: the gathers split
    plan = g.plan(keep=[t[3]])
    assert plan[0] == (C.GL_GET_ROWS, 0, 2, 0)
    assert plan[1] == (C.GL_GET_ROWS, 2, 2, 0)
    # the sum and its LayerNorm still fuse, as a residual join
    assert plan[2] == (C.GL_ADD_LAYER_NORM, 4, 4, 1)


def causal_block_tail(g: C.Graph, C_=32, T=20, extra_reader=False):
    """cfm_decoder.cpp:143-148: layer_norm -> mish -> mul(mask)."""
    x = g.tensor(f32(T, C_))
    w, b = g.tensor(f32(C_)), g.tensor(f32(C_))
    mask = g.tensor(f32(T, 1))
    t = [g.tensor(f32(T, C_)) for _ in range(7)]
    g.node(C.GOP_NORM, t[0], (x,), fparam=1e-5)
    g.node(C.GOP_MUL, t[1], (t[0], w))
    g.node(C.GOP_ADD, t[2], (t[1], b))
    g.node(C.GOP_UNARY, t[3], (t[2],), iparam=C.SOFTPLUS)
    g.node(C.GOP_UNARY, t[4], (t[3],), iparam=C.TANH)
    g.node(C.GOP_MUL, t[5], (t[2], t[4]))
    g.node(C.GOP_MUL, t[6], (t[5], mask))
    if extra_reader:
        g.node(C.GOP_UNARY, g.tensor(f32(T, C_)), (t[2],), iparam=C.GELU)
    return t


def test_layer_norm_mish_mask():
    g = C.Graph()
    causal_block_tail(g)
    assert g.plan() == [(C.GL_LAYER_NORM_MASK, 0, 7, 0)]
    # a mask that is not one value per frame is a plain multiply of its own
    g2 = C.Graph()
    t = causal_block_tail(g2)
    g2._descs[3] = C.desc(f32(20, 32))
    assert g2.plan() == [(C.GL_LAYER_NORM, 0, 6, 0), (C.GL_BINARY, 6, 1, C.BINARY_MUL)]


def t3_block_tail(g: C.Graph, N=5, D=64, F=256):
    """t3.cpp:526-541 around the matmuls (stood in by op 99, which the
    library does not run): bias add -> residual add -> layer_norm, bias add
    -> gelu, bias add -> residual add."""
    MM = 99
    attn_mm, h = g.tensor(f32(N, D)), g.tensor(f32(N, D))
    out_b, ln_w, ln_b = g.tensor(f32(D)), g.tensor(f32(D)), g.tensor(f32(D))
    fc_b, proj_b = g.tensor(f32(F)), g.tensor(f32(D))
    wd = [g.tensor(f32(N, D)) for _ in range(5)]
    wf = [g.tensor(f32(N, F)) for _ in range(3)]
    wp = [g.tensor(f32(N, D)) for _ in range(3)]
    g.node(C.GOP_ADD, wd[0], (attn_mm, out_b))      # cur = add(mm, out_b)
    g.node(C.GOP_ADD, wd[1], (wd[0], h))            # attn_residual = add(cur, h)
    g.node(C.GOP_NORM, wd[2], (wd[1],), fparam=1e-5)
    g.node(C.GOP_MUL, wd[3], (wd[2], ln_w))
    g.node(C.GOP_ADD, wd[4], (wd[3], ln_b))
    g.node(MM, wf[0], (wd[4],))                     # fc mul_mat
    g.node(C.GOP_ADD, wf[1], (wf[0], fc_b))
    g.node(C.GOP_UNARY, wf[2], (wf[1],), iparam=C.GELU)
    g.node(MM, wp[0], (wf[2],))                     # proj mul_mat
    g.node(C.GOP_ADD, wp[1], (wp[0], proj_b))
    g.node(C.GOP_ADD, wp[2], (wp[1], wd[1]))        # h = add(cur, attn_residual)
    return wd, wf, wp


def test_t3_block_tail():
    g = C.Graph()
    t3_block_tail(g)
    assert g.plan() == [(C.GL_ADD_LAYER_NORM, 0, 5, 0),   # attn_residual is read again: stored
                        (C.GL_UNSUPPORTED, 5, 1, 0),
                        (C.GL_BIAS_ACT, 6, 2, 0),
                        (C.GL_UNSUPPORTED, 8, 1, 0),
                        (C.GL_BIAS_RESIDUAL, 9, 2, 0)]    # proj bias add -> residual add, no norm after it


def test_residual_join_without_bias_and_unread_sum():
    g = C.Graph()
    a, r, w, b = g.tensor(f32(3, 32)), g.tensor(f32(3, 32)), g.tensor(f32(32)), g.tensor(f32(32))
    s = g.node(C.GOP_ADD, g.tensor(f32(3, 32)), (a, r))
    n = g.node(C.GOP_NORM, g.tensor(f32(3, 32)), (s,), fparam=1e-5)
    m = g.node(C.GOP_MUL, g.tensor(f32(3, 32)), (n, w))
    g.node(C.GOP_ADD, g.tensor(f32(3, 32)), (m, b))
    assert g.plan() == [(C.GL_ADD_LAYER_NORM, 0, 4, 1)]
    assert g.plan(keep=[s]) == [(C.GL_ADD_LAYER_NORM, 0, 4, 0)]


def test_bias_add_forms():
    """(C,) bias along ne0, (1, C) bias per row (s3enc.cpp:117-120), a mish
    chain after the bias, and a one-row tensor whose bias has its shape."""
    g = C.Graph()
    x = g.tensor(f32(6, 40))
    inner, outer = g.tensor(f32(40)), g.tensor(f32(6, 1))
    y1 = g.node(C.GOP_ADD, g.tensor(f32(6, 40)), (x, outer))
    g.node(C.GOP_UNARY, g.tensor(f32(6, 40)), (y1,), iparam=C.GELU_ERF)
    y2 = g.node(C.GOP_ADD, g.tensor(f32(6, 40)), (x, inner))
    sp = g.node(C.GOP_UNARY, g.tensor(f32(6, 40)), (y2,), iparam=C.SOFTPLUS)
    th = g.node(C.GOP_UNARY, g.tensor(f32(6, 40)), (sp,), iparam=C.TANH)
    g.node(C.GOP_MUL, g.tensor(f32(6, 40)), (y2, th))
    v, vb = g.tensor(f32(40)), g.tensor(f32(40))
    y3 = g.node(C.GOP_ADD, g.tensor(f32(40)), (v, vb))
    g.node(C.GOP_UNARY, g.tensor(f32(40)), (y3,), iparam=C.SILU)
    full = g.tensor(f32(6, 40))
    g.node(C.GOP_ADD, g.tensor(f32(6, 40)), (x, full))
    assert g.plan() == [(C.GL_BIAS_ACT, 0, 2, 0), (C.GL_BIAS_ACT, 2, 4, 0), (C.GL_BIAS_ACT, 6, 2, 0),
                        (C.GL_BINARY, 8, 1, C.BINARY_ADD)]   # the full-shape add


def test_layer_norm_output_read_elsewhere_keeps_mish_separate():
    g = C.Graph()
    causal_block_tail(g, extra_reader=True)
    assert g.plan() == [(C.GL_LAYER_NORM, 0, 3, 0), (C.GL_UNARY, 3, 3, 0), (C.GL_BINARY, 6, 1, C.BINARY_MUL),
                        (C.GL_UNARY, 7, 1, 0)]


def test_shape_mismatch_is_not_a_layer_norm():
    g = C.Graph()
    x = g.tensor(f32(4, 32))
    w = g.tensor(f32(4, 32))          # full-shape gain: not ggml's (ne0) broadcast of layer_norm
    b = g.tensor(f32(32))
    n, m, y = (g.tensor(f32(4, 32)) for _ in range(3))
    g.node(C.GOP_NORM, n, (x,), fparam=1e-5)
    g.node(C.GOP_MUL, m, (n, w))
    g.node(C.GOP_ADD, y, (m, b))
    # the norm alone, the full-shape multiply alone, the bias add alone
    assert [p[0] for p in g.plan()] == [C.GL_NORM, C.GL_BINARY, C.GL_BIAS_ACT]


def test_snake_chain():
    """hift_vocoder.cpp:64-73."""
    g = C.Graph()
    x = g.tensor(f32(30, 16))
    a, ai = g.tensor(f32(16)), g.tensor(f32(16))
    t = [g.tensor(f32(30, 16)) for _ in range(5)]
    g.node(C.GOP_MUL, t[0], (x, a))
    g.node(C.GOP_UNARY, t[1], (t[0],), iparam=C.SIN)
    g.node(C.GOP_UNARY, t[2], (t[1],), iparam=C.SQR)
    g.node(C.GOP_MUL, t[3], (t[2], ai))
    g.node(C.GOP_ADD, t[4], (x, t[3]))
    assert g.plan() == [(C.GL_SNAKE, 0, 5, 0)]
    # the same nodes with the sin result kept: five separate launches
    assert [p[0] for p in g.plan(keep=[t[1]])] == [C.GL_BINARY, C.GL_UNARY, C.GL_UNARY, C.GL_BINARY,
                                                    C.GL_BINARY]


@pytest.mark.parametrize("with_mask", [True, False])
def test_attention_scores(with_mask):
    """t3.cpp:513-518 (scale -> diag_mask_inf -> soft_max) and the unmasked
    form of cfm_decoder.cpp:218-220."""
    g = C.Graph()
    kq = g.tensor(f32(4, 7, 9))
    t = [g.tensor(f32(4, 7, 9)) for _ in range(3)]
    g.node(C.GOP_SCALE, t[0], (kq,), fparam=0.125)
    src = t[0]
    if with_mask:
        g.node(C.GOP_DIAG_MASK_INF, t[1], (t[0],), iparam=2)
        src = t[1]
    g.node(C.GOP_SOFT_MAX, t[2], (src,), fparam=1.0)
    assert g.plan() == [(C.GL_SOFT_MAX, 0, 3 if with_mask else 2, 0)]


@pytest.mark.parametrize("with_scale,with_mask", [(True, False), (True, True), (False, False)])
def test_score_terms_add_joins_the_soft_max(with_scale, with_mask):
    """flow_encoder.cpp:369-372: add(AC, BD_shift) -> scale -> soft_max is one
    launch; the sum kept by the caller, a broadcast or F16 operand, or a
    soft_max with its own scale leave the add a launch of its own."""
    def build(keep_sum=False, b_shape=(4, 7, 9), b_dtype=torch.float32, sm_scale=1.0):
        g = C.Graph()
        ac = g.tensor(f32(4, 7, 9))
        bd = g.tensor(torch.zeros(b_shape, dtype=b_dtype))
        t = [g.tensor(f32(4, 7, 9)) for _ in range(4)]
        g.node(C.GOP_ADD, t[0], (ac, bd))
        src = t[0]
        if with_scale:
            g.node(C.GOP_SCALE, t[1], (src,), fparam=0.125)
            src = t[1]
        if with_mask:
            g.node(C.GOP_DIAG_MASK_INF, t[2], (src,), iparam=2)
            src = t[2]
        g.node(C.GOP_SOFT_MAX, t[3], (src,), fparam=sm_scale)
        return g, g.plan(keep=[t[0]] if keep_sum else [])

    n = 2 + with_scale + with_mask
    g, plan = build()
    assert plan == [(C.GL_SOFT_MAX, 0, n, 0)]
    _, plan = build(keep_sum=True)
    assert plan == [(C.GL_BINARY, 0, 1, C.BINARY_ADD), (C.GL_SOFT_MAX, 1, n - 1, 0)]
    _, plan = build(b_shape=(1, 7, 9))
    assert plan[0] == (C.GL_BINARY, 0, 1, C.BINARY_ADD)
    _, plan = build(b_dtype=torch.float16)
    assert plan[0][0] != C.GL_SOFT_MAX
    _, plan = build(sm_scale=2.0)
    assert plan[0][0] != C.GL_SOFT_MAX and plan[-1] == (C.GL_SOFT_MAX, n - 1, 1, 0)


def test_bias_add_then_layer_norm():
    """flow_encoder.cpp:414-415: a linear's bias add, then its LayerNorm, is
    one launch when the fused kernel takes the layout (rows of 512); rows
    of 4100 floats or a kept sum that is not 16-byte stepped leave the two
    launches."""
    def build(D=512, keep_sum=False, mish=False):
        g = C.Graph()
        x, bias = g.tensor(f32(10, D)), g.tensor(f32(D))
        w, b = g.tensor(f32(D)), g.tensor(f32(D))
        s = g.tensor(f32(10, D))
        g.node(C.GOP_ADD, s, (x, bias))
        n, m, y = g.tensor(f32(10, D)), g.tensor(f32(10, D)), g.tensor(f32(10, D))
        g.node(C.GOP_NORM, n, (s,), fparam=1e-5)
        g.node(C.GOP_MUL, m, (n, w))
        g.node(C.GOP_ADD, y, (m, b))
        if mish:
            sp, th = g.tensor(f32(10, D)), g.tensor(f32(10, D))
            g.node(C.GOP_UNARY, sp, (y,), iparam=C.SOFTPLUS)
            g.node(C.GOP_UNARY, th, (sp,), iparam=C.TANH)
            g.node(C.GOP_MUL, g.tensor(f32(10, D)), (y, th))
        return g.plan(keep=[s] if keep_sum else [])

    assert build() == [(C.GL_ADD_LAYER_NORM, 0, 4, 1)]
    assert build(keep_sum=True) == [(C.GL_ADD_LAYER_NORM, 0, 4, 0)]
    assert build(mish=True) == [(C.GL_ADD_LAYER_NORM, 0, 7, 1)]
    assert build(D=4100) == [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_LAYER_NORM, 1, 3, 0)]
    assert build(D=510) == [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_LAYER_NORM, 1, 3, 0)]


def test_two_lone_bias_adds_share_a_launch():
    """Adjacent bias adds that neither read nor overlap each other's output
    (v's and k's projections) are one launch; an add reading the first's
    sum, one whose output overlaps the other's input, a column bias, or a
    bias add that starts a longer chain stay apart."""
    def build(dep=False, alias=False, col=False, act=False, rows=(10, 10)):
        g = C.Graph()
        v_mm, v_b = g.tensor(f32(rows[0], 64)), g.tensor(f32(64))
        k_mm = g.tensor(f32(rows[1], 64))
        k_b = g.tensor(f32(rows[1], 1) if col else f32(64))
        v_t = f32(rows[0], 64)
        v = g.tensor(v_t)
        g.node(C.GOP_ADD, v, (v_mm, v_b))
        k = g.tensor(v_t if alias else f32(rows[1], 64))
        g.node(C.GOP_ADD, k, (v if dep else k_mm, k_b))
        if act:
            g.node(C.GOP_UNARY, g.tensor(f32(rows[1], 64)), (k,), iparam=C.SILU)
        return g.plan(keep=[v] if act else [v, k])

    assert build() == [(C.GL_BIAS_ADD_TWO, 0, 2, 0)]
    assert build(rows=(10, 30)) == [(C.GL_BIAS_ADD_TWO, 0, 2, 0)]
    assert build(dep=True) == [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_BIAS_ACT, 1, 1, 0)]
    assert build(alias=True) == [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_BIAS_ACT, 1, 1, 0)]
    assert build(col=True) == [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_BIAS_ACT, 1, 1, 0)]
    assert build(act=True) == [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_BIAS_ACT, 1, 2, 0)]


def test_two_ropes_share_a_launch():
    """q's and k's RoPE in a row (s3enc.cpp:215-229) are one launch; a RoPE
    of the first's output, or one writing over the other's input, is not."""
    def build(chain=False, clobber=False, in_place=False):
        g = C.Graph()
        pos = g.tensor(torch.zeros(6, dtype=torch.int32))
        q, k = g.tensor(f32(6, 4, 64)), g.tensor(f32(6, 4, 64))
        qr_t = f32(6, 4, 64)
        qr = g.tensor(qr_t)
        g.node(C.GOP_ROPE, qr, (q, pos))
        kr = g.tensor(g._torch[q] if clobber else g._torch[k] if in_place else f32(6, 4, 64))
        g.node(C.GOP_ROPE, kr, (qr if chain else k, pos))
        return g.plan(keep=[qr, kr])

    assert build() == [(C.GL_ROPE_TWO, 0, 2, 0)]
    assert build(in_place=True) == [(C.GL_ROPE_TWO, 0, 2, 0)]     # k's RoPE over k itself
    assert build(chain=True) == [(C.GL_ROPE, 0, 1, 0), (C.GL_ROPE, 1, 1, 0)]
    assert build(clobber=True) == [(C.GL_ROPE, 0, 1, 0), (C.GL_ROPE, 1, 1, 0)]   # k's output over q


def test_query_bias_and_pos_bias_pair():
    """flow_encoder.cpp:320, 341-345: add(q_mm, q_b) -> reshape to (64, 8, T)
    heads -> add(., pos_bias_u), add(., pos_bias_v) is one launch; the sum
    or the heads read elsewhere, or a view that is not a contiguous reshape,
    leave the bias add and the two adds apart."""
    def build(T=10, keep_sum=False, keep_heads=False, sliced=False, third_reader=False):
        g = C.Graph()
        q_mm, q_b = g.tensor(f32(T, 512)), g.tensor(f32(512))
        s_t = f32(T, 512)
        s = g.tensor(s_t)
        g.node(C.GOP_ADD, s, (q_mm, q_b))
        heads = s_t[:, :256].view(T, 4, 64) if sliced else s_t.view(T, 8, 64)
        vw = g.tensor(heads)
        g.node(C.GOP_VIEW, vw, (s,))
        shp = tuple(heads.shape)
        u, v = g.tensor(f32(1, *shp[1:])), g.tensor(f32(1, *shp[1:]))
        g.node(C.GOP_ADD, g.tensor(f32(*shp)), (vw, u))
        g.node(C.GOP_ADD, g.tensor(f32(*shp)), (vw, v))
        if third_reader:
            g.node(C.GOP_ADD, g.tensor(f32(*shp)), (vw, u))
        keep = ([s] if keep_sum else []) + ([vw] if keep_heads else [])
        return g.plan(keep=keep)

    assert build() == [(C.GL_BIAS_ADD_PAIR, 0, 4, 0)]
    assert build(T=1) == [(C.GL_BIAS_ADD_PAIR, 0, 4, 0)]
    # the (8, 64) weights reshaped to (64, 8, 1) by views among the adds
    g = C.Graph()
    q_mm, q_b = g.tensor(f32(10, 512)), g.tensor(f32(512))
    s_t = f32(10, 512)
    s = g.tensor(s_t)
    g.node(C.GOP_ADD, s, (q_mm, q_b))
    vw = g.tensor(s_t.view(10, 8, 64))
    g.node(C.GOP_VIEW, vw, (s,))
    for _ in range(2):
        w = f32(8, 64)
        w3 = g.tensor(w.view(1, 8, 64))
        g.node(C.GOP_VIEW, w3, (g.tensor(w),))
        g.node(C.GOP_ADD, g.tensor(f32(10, 8, 64)), (vw, w3))
    assert g.plan() == [(C.GL_BIAS_ADD_PAIR, 0, 6, 0)]
    apart = [(C.GL_BIAS_ACT, 0, 1, 0), (C.GL_VIEW, 1, 1, 0), (C.GL_BINARY, 2, 1, C.BINARY_ADD),
             (C.GL_BINARY, 3, 1, C.BINARY_ADD)]
    assert build(keep_sum=True) == apart
    assert build(keep_heads=True) == apart
    assert build(third_reader=True)[:4] == apart
    assert build(sliced=True)[0] != (C.GL_BIAS_ADD_PAIR, 0, 4, 0)


def test_soft_max_with_own_scale_does_not_absorb_scale():
    g = C.Graph()
    kq = g.tensor(f32(4, 8))
    s, y = g.tensor(f32(4, 8)), g.tensor(f32(4, 8))
    g.node(C.GOP_SCALE, s, (kq,), fparam=0.5)
    g.node(C.GOP_SOFT_MAX, y, (s,), fparam=2.0)
    # the scale stays a launch of its own: folded in, it would round once
    # where ggml rounds twice
    assert g.plan() == [(C.GL_SCALE, 0, 1, 0), (C.GL_SOFT_MAX, 1, 1, 0)]


def test_lone_scale_and_mask():
    """A scale no soft_max follows is a cbx_scale launch; a lone
    diag_mask_inf is not a chain the library runs."""
    g = C.Graph()
    x = g.tensor(f32(4, 8))
    s = g.node(C.GOP_SCALE, g.tensor(f32(4, 8)), (x,), fparam=1.0 / 3.0)
    g.node(C.GOP_DIAG_MASK_INF, g.tensor(f32(4, 8)), (s,), iparam=1)
    assert g.plan() == [(C.GL_SCALE, 0, 1, 0), (C.GL_UNSUPPORTED, 1, 1, 0)]


def test_soft_max_with_mask_operand_is_unsupported():
    g = C.Graph()
    kq, m, y = g.tensor(f32(4, 8)), g.tensor(f32(4, 8)), g.tensor(f32(4, 8))
    g.node(C.GOP_SOFT_MAX, y, (kq, m), fparam=1.0)
    assert g.plan() == [(C.GL_UNSUPPORTED, 0, 1, 0)]


def test_layer_norm_view_rope():
    g = C.Graph()
    n_tok, H, hd = 10, 4, 16
    x = g.tensor(f32(n_tok, H * hd))
    w, b = g.tensor(f32(H * hd)), g.tensor(f32(H * hd))
    pos = g.tensor(torch.zeros(n_tok, dtype=torch.int32))
    n, m = g.tensor(f32(n_tok, H * hd)), g.tensor(f32(n_tok, H * hd))
    y_t = f32(n_tok, H * hd)
    y = g.tensor(y_t)
    v = g.tensor(y_t.view(n_tok, H, hd))
    r = g.tensor(f32(n_tok, H, hd))
    g.node(C.GOP_NORM, n, (x,), fparam=1e-5)
    g.node(C.GOP_MUL, m, (n, w))
    g.node(C.GOP_ADD, y, (m, b))
    g.node(C.GOP_VIEW, v, (y,))
    g.node(C.GOP_ROPE, r, (v, pos))
    assert g.plan() == [(C.GL_LAYER_NORM_ROPE, 0, 5, 0)]
    # a view of other memory is a different tensor: no fusion
    g.tensor(f32(n_tok, H, hd))
    g.nodes[3].dst = len(g._descs) - 1
    g.nodes[4].src[0] = len(g._descs) - 1
    assert [p[0] for p in g.plan()] == [C.GL_LAYER_NORM, C.GL_VIEW, C.GL_ROPE]


@pytest.mark.parametrize("affine,mish,want", [(True, True, 6), (True, False, 3), (False, True, 4), (False, False, 1)])
def test_group_norm_chains(affine, mish, want):
    g = C.Graph()
    Ch = 8
    x = g.tensor(f32(2, Ch, 5, 3))            # ggml ne = (3, 5, C, 2): channels on ne2
    w, b = g.tensor(f32(1, Ch, 1, 1)), g.tensor(f32(1, Ch, 1, 1))
    y = g.node(C.GOP_GROUP_NORM, g.tensor(f32(2, Ch, 5, 3)), (x,), iparam=4, fparam=1e-5)
    if affine:
        y = g.node(C.GOP_MUL, g.tensor(f32(2, Ch, 5, 3)), (y, w))
        y = g.node(C.GOP_ADD, g.tensor(f32(2, Ch, 5, 3)), (y, b))
    if mish:
        sp = g.node(C.GOP_UNARY, g.tensor(f32(2, Ch, 5, 3)), (y,), iparam=C.SOFTPLUS)
        th = g.node(C.GOP_UNARY, g.tensor(f32(2, Ch, 5, 3)), (sp,), iparam=C.TANH)
        g.node(C.GOP_MUL, g.tensor(f32(2, Ch, 5, 3)), (y, th))
    assert g.plan() == [(C.GL_GROUP_NORM, 0, want, 0)]


def test_silu_gate_and_singles():
    g = C.Graph()
    a, u = g.tensor(f32(3, 40)), g.tensor(f32(3, 40))
    s = g.node(C.GOP_UNARY, g.tensor(f32(3, 40)), (a,), iparam=C.SILU)
    y = g.node(C.GOP_MUL, g.tensor(f32(3, 40)), (s, u))
    g.node(C.GOP_UNARY, g.tensor(f32(3, 40)), (y,), iparam=C.GELU)
    g.node(C.GOP_LEAKY_RELU, g.tensor(f32(3, 40)), (y,), fparam=0.1)
    g.node(C.GOP_RMS_NORM, g.tensor(f32(3, 40)), (y,), fparam=1e-6)
    g.node(C.GOP_CPY, g.tensor(torch.zeros(3, 40, dtype=torch.float16)), (y,))
    g.node(C.GOP_UNARY, g.tensor(f32(3, 40)), (y,), iparam=42)   # no such activation
    assert [p[:3] for p in g.plan()] == [(C.GL_SWIGLU, 0, 2), (C.GL_UNARY, 2, 1), (C.GL_LEAKY_RELU, 3, 1),
                                         (C.GL_RMS_NORM, 4, 1), (C.GL_CPY, 5, 1), (C.GL_UNSUPPORTED, 6, 1)]


def _raw(g: C.Graph, keep=()):
    T, N, K = g._arrays(list(keep))
    return T, N, K


def test_bad_lists_are_refused():
    L = C.load()
    g = C.Graph()
    x, y = g.tensor(f32(2, 8)), g.tensor(f32(2, 8))
    g.node(C.GOP_NORM, y, (x,), fparam=1e-5)
    T, N, K = _raw(g)
    out = (C.GLaunch * 4)()
    n = ctypes.c_int32(-1)
    assert L.cbx_graph_plan(T, 2, N, 1, K, 0, out, 4, ctypes.byref(n)) == C.OK and n.value == 1
    # too little room: the count is still reported
    assert L.cbx_graph_plan(T, 2, N, 1, K, 0, out, 0, ctypes.byref(n)) == C.ERR_INVALID_ARG and n.value == 1
    # a node naming a tensor past the array
    g.nodes[0].src[0] = 7
    T, N, K = _raw(g)
    assert L.cbx_graph_plan(T, 2, N, 1, K, 0, out, 4, ctypes.byref(n)) == C.ERR_INVALID_ARG
    assert "out of range" in C.last_error()
    g.nodes[0].src[0] = x
    g.nodes[0].dst = -1
    T, N, K = _raw(g)
    assert L.cbx_graph_plan(T, 2, N, 1, K, 0, out, 4, ctypes.byref(n)) == C.ERR_INVALID_ARG
    g.nodes[0].dst = y
    # a keep index past the array
    T, N, K = _raw(g, keep=[5])
    assert L.cbx_graph_plan(T, 2, N, 1, K, 1, out, 4, ctypes.byref(n)) == C.ERR_INVALID_ARG
    # empty list: no launches
    assert L.cbx_graph_plan(None, 0, None, 0, None, 0, None, 0, ctypes.byref(n)) == C.OK and n.value == 0


def test_compute_refuses_unsupported_before_any_launch():
    """The whole list is planned first: an unsupported node anywhere stops
    the call before the device is touched (this runs without a GPU)."""
    L = C.load()
    g = C.Graph()
    t = t3_input(g)
    g.node(99, g.tensor(f32(6, 64)), (t[8],))     # a matmul (op 99 stands in): not this library's
    T, N, K = _raw(g)
    n = ctypes.c_int32(-1)
    rc = L.cbx_graph_compute(T, len(g._descs), N, len(g.nodes), K, 0, None, ctypes.byref(n))
    assert rc == C.ERR_UNSUPPORTED and n.value == 0
    assert "node 9 (unknown op)" in C.last_error()


def test_graph_exec_argument_errors():
    """cbx_graph_exec_*: a NULL out or exec is refused before the device is
    touched, and destroying NULL does nothing (this runs without a GPU)."""
    L = C.load()
    g = C.Graph()
    t3_input(g)
    T, N, K = _raw(g)
    n = ctypes.c_int32(-1)
    rc = L.cbx_graph_exec_create(T, len(g._descs), N, len(g.nodes), K, 0, None, ctypes.byref(n))
    assert rc == C.ERR_INVALID_ARG and n.value == 0
    assert "out is NULL" in C.last_error()
    assert L.cbx_graph_exec_launch(None, None) == C.ERR_INVALID_ARG
    assert "exec is NULL" in C.last_error()
    ip = ctypes.c_int32(-1)
    n = ctypes.c_int32(-1)
    rc = L.cbx_graph_exec_update(None, T, len(g._descs), N, len(g.nodes), K, 0, ctypes.byref(n), ctypes.byref(ip))
    assert rc == C.ERR_INVALID_ARG and n.value == 0 and ip.value == 0
    assert "cbx_graph_exec_update: exec is NULL" in C.last_error()
    L.cbx_graph_exec_destroy(None)


def test_hand_made_launches_stay_inside_the_list():
    L = C.load()
    g = C.Graph()
    x, y = g.tensor(f32(2, 8)), g.tensor(f32(2, 8))
    g.node(C.GOP_NORM, y, (x,), fparam=1e-5)
    g.node(C.GOP_VIEW, x, (y,))
    T, N, _ = _raw(g)
    bad = [C.GLaunch(C.GL_SNAKE, 0, 5, 0),         # runs past the two nodes
           C.GLaunch(C.GL_NORM, -1, 1, 0),
           C.GLaunch(C.GL_LAYER_NORM, 0, 4, 0),     # not a length a layer_norm chain has
           C.GLaunch(99, 0, 1, 0)]
    for l in bad:
        assert L.cbx_graph_launch(T, 2, N, 2, ctypes.byref(l), None) == C.ERR_INVALID_ARG, (l.kind, l.n_nodes)
    assert L.cbx_graph_launch(T, 2, N, 2, ctypes.byref(C.GLaunch(C.GL_UNSUPPORTED, 0, 1, 0)), None) == \
        C.ERR_UNSUPPORTED
    assert L.cbx_graph_launch(T, 2, N, 2, ctypes.byref(C.GLaunch(C.GL_VIEW, 1, 1, 0)), None) == C.OK


def test_hand_made_launches_of_the_paired_kinds_are_refused():
    """The two-output and paired launch kinds, and the softmax chain, on
    nodes that are not their chains: refused before any entry point runs."""
    L = C.load()
    g = C.Graph()
    ts = [g.tensor(f32(2, 8)) for _ in range(7)]
    for k in range(6):
        if k % 2:
            g.node(C.GOP_VIEW, ts[k + 1], (ts[k],))
        else:
            g.node(C.GOP_NORM, ts[k + 1], (ts[k],), fparam=1e-5)
    T, N, _ = _raw(g)
    for l in [C.GLaunch(C.GL_BIAS_ADD_PAIR, 0, 4, 0), C.GLaunch(C.GL_BIAS_ADD_PAIR, 0, 6, 0),
              C.GLaunch(C.GL_BIAS_ADD_TWO, 0, 2, 0), C.GLaunch(C.GL_ROPE_TWO, 0, 2, 0),
              C.GLaunch(C.GL_SOFT_MAX, 0, 1, 0), C.GLaunch(C.GL_SOFT_MAX, 0, 3, 0),
              C.GLaunch(C.GL_SOFT_MAX, 0, 4, 0), C.GLaunch(C.GL_BIAS_ADD_TWO, 0, 3, 0)]:
        assert L.cbx_graph_launch(T, 7, N, 6, ctypes.byref(l), None) == C.ERR_INVALID_ARG, (l.kind, l.n_nodes)
        assert "does not fit" in C.last_error()


def test_bias_residual_chains():
    """add(x, bias) [-> view] -> add(r, .) with no norm after it: one
    launch (cfm_decoder.cpp:162-165 the time MLP over the frames, :242-244 a
    stack's last ff.2); not when the sum is read again or kept, when the view
    is not the sum itself, or when a norm follows (that is the
    residual + LayerNorm launch)."""
    def time_mlp(view_of_other=False, keep_sum=False):
        g = C.Graph()
        h = g.tensor(f32(10, 16))
        mlp, b = g.tensor(f32(16)), g.tensor(f32(16))
        s_t = f32(16)
        s = g.tensor(s_t)
        v = g.tensor(f32(1, 16) if view_of_other else s_t.view(1, 16))
        g.node(C.GOP_ADD, s, (mlp, b))
        g.node(C.GOP_VIEW, v, (s,))
        g.node(C.GOP_ADD, g.tensor(f32(10, 16)), (h, v))
        return g.plan(keep=[s] if keep_sum else [])

    assert time_mlp() == [(C.GL_BIAS_RESIDUAL, 0, 3, 0)]
    assert [p[0] for p in time_mlp(view_of_other=True)] == [C.GL_BIAS_ACT, C.GL_VIEW, C.GL_BIAS_ACT]
    assert [p[0] for p in time_mlp(keep_sum=True)] == [C.GL_BIAS_ACT, C.GL_VIEW, C.GL_BIAS_ACT]

    def ff2(read_twice=False, norm_after=False):
        g = C.Graph()
        x, mm, b = g.tensor(f32(10, 16)), g.tensor(f32(10, 16)), g.tensor(f32(16))
        t = g.node(C.GOP_ADD, g.tensor(f32(10, 16)), (mm, b))
        y = g.node(C.GOP_ADD, g.tensor(f32(10, 16)), (x, t))
        if read_twice:
            g.node(C.GOP_UNARY, g.tensor(f32(10, 16)), (t,), iparam=C.SILU)
        if norm_after:
            n = g.node(C.GOP_NORM, g.tensor(f32(10, 16)), (y,), fparam=1e-5)
            m = g.node(C.GOP_MUL, g.tensor(f32(10, 16)), (n, g.tensor(f32(16))))
            g.node(C.GOP_ADD, g.tensor(f32(10, 16)), (m, g.tensor(f32(16))))
        return g.plan()

    assert ff2() == [(C.GL_BIAS_RESIDUAL, 0, 2, 0)]
    assert [p[0] for p in ff2(read_twice=True)] == [C.GL_BIAS_ACT, C.GL_BINARY, C.GL_UNARY]
    assert [p[0] for p in ff2(norm_after=True)] == [C.GL_ADD_LAYER_NORM]


def test_random_lists_plan_into_an_exact_cover():
    """Random node lists over random operands: the plan covers every node
    exactly once, in order, each launch within its kind's span."""
    rng = np.random.default_rng(5)
    spans = {C.GL_UNSUPPORTED: {1}, C.GL_VIEW: {1}, C.GL_GET_ROWS: {1, 2}, C.GL_GET_ROWS_ADD: {3, 4, 5},
             C.GL_GET_ROWS_ADD_LAYER_NORM: {6, 7, 8}, C.GL_NORM: {1}, C.GL_LAYER_NORM: {3, 6},
             C.GL_LAYER_NORM_ROPE: {5}, C.GL_RMS_NORM: {1, 2}, C.GL_GROUP_NORM: {1, 3, 4, 6},
             C.GL_SOFT_MAX: {1, 2, 3, 4}, C.GL_SNAKE: {5}, C.GL_UNARY: {1, 3}, C.GL_SWIGLU: {2},
             C.GL_LEAKY_RELU: {1}, C.GL_ROPE: {1}, C.GL_CPY: {1}, C.GL_ADD_LAYER_NORM: {4, 5, 7, 8},
             C.GL_LAYER_NORM_MASK: {4, 7}, C.GL_BIAS_ACT: {1, 2, 4}, C.GL_CONV1D: set(range(9, 18)),
             C.GL_CONV_TRANSPOSE1D: set(range(7, 15)), C.GL_CAUSAL_CONV1D: set(range(12, 16)),
             C.GL_BINARY: {1}, C.GL_CONCAT: {1}, C.GL_BIAS_RESIDUAL: {2, 3}, C.GL_SCALE: {1},
             C.GL_BIAS_ADD_PAIR: {4, 5, 6}, C.GL_BIAS_ADD_TWO: {2},
             C.GL_ROPE_TWO: {2}}
    shapes = [(4, 8), (8,), (1, 8, 1, 1), (4, 8), (4, 1)]
    for trial in range(200):
        g = C.Graph()
        n_t = int(rng.integers(3, 12))
        for k in range(n_t):
            g.tensor(f32(*shapes[int(rng.integers(0, len(shapes)))]))
        for k in range(int(rng.integers(1, 25))):
            op = int(rng.integers(0, 18))
            src = [int(rng.integers(-1, n_t)) for _ in range(2)]
            g.node(op, int(rng.integers(0, n_t)), src, iparam=int(rng.integers(-1, 9)),
                   fparam=float(rng.choice([1.0, 0.5, 1e-5])))
        keep = [int(v) for v in rng.integers(0, n_t, size=int(rng.integers(0, 3)))]
        plan = g.plan(keep)
        at = 0
        for kind, first, n, flags in plan:
            assert first == at and n in spans[kind], (trial, kind, n)
            at += n
        assert at == len(g.nodes)


# ---- HiFT conv chains (hift_vocoder.cpp) -----------------------------------------

def host_new(shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


DUMMY_W = 0x1000   # planning reads conv_w only for being non-null


def hift_params(h: HiftGraph, Ch=16, K=3):
    p = {}
    for s in ("1", "2"):
        p["a" + s], p["ai" + s] = h.t(f32(Ch)), h.t(f32(Ch))
        p["w" + s], p["b" + s] = h.t(torch.zeros(Ch, Ch, K, dtype=torch.float16)), h.t(f32(Ch))
    return p


def test_resblock_sublayer_is_two_conv_launches():
    """resblock_forward's layer (hift_vocoder.cpp:131-135): snake -> conv1d_CT
    -> snake -> conv1d_CT -> add(x, h): the first snake and conv1d_CT (its 9
    nodes and the 2 of the bias add) are one launch, the second adds the
    residual add."""
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    h.sublayer(x, hift_params(h), 3, DUMMY_W, DUMMY_W)
    assert h.g.plan() == [(C.GL_CONV1D, 0, 16, C.GLF_SNAKE | C.GLF_BIAS),
                          (C.GL_CONV1D, 16, 17, C.GLF_SNAKE | C.GLF_BIAS | C.GLF_RESIDUAL)]


def test_three_sublayers_chain():
    """resblock_forward runs its three layers in series (hift_vocoder.cpp:128-136)."""
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    for d in (1, 3, 5):
        x = h.sublayer(x, hift_params(h), d, DUMMY_W, DUMMY_W)
    plan = h.g.plan()
    assert [p[0] for p in plan] == [C.GL_CONV1D] * 6
    assert [p[3] & C.GLF_RESIDUAL for p in plan] == [0, 8] * 3
    assert sum(p[2] for p in plan) == len(h.g.nodes) == 99


def test_conv_post_and_plain_conv():
    """conv_post (hift_vocoder.cpp:748-749): leaky_relu -> conv1d_CT; a conv
    without prologue or bias (9 nodes) is a launch of its own."""
    h = HiftGraph(host_new)
    x = h.t(f32(30, 16))
    w, b = h.t(torch.zeros(18, 16, 7, dtype=torch.float16)), h.t(f32(18))
    y = h.conv1d(h.leaky(x, 0.01), w, b, 1, 3, 1, DUMMY_W)
    w2 = h.t(torch.zeros(8, 18, 3))
    h.conv1d(y, w2, None, 2, 1, 1, DUMMY_W)
    assert h.g.plan() == [(C.GL_CONV1D, 0, 12, C.GLF_LEAKY | C.GLF_BIAS), (C.GL_CONV1D, 12, 9, 0)]


@pytest.mark.parametrize("stride,K,pad", [(8, 16, 4), (5, 11, 3), (3, 7, 2), (1, 3, 1)])
def test_upsampler_is_one_transposed_conv_launch(stride, K, pad):
    """hift_vocoder.cpp:686-687: leaky_relu -> conv_transpose1d_CT (transpose,
    cont, conv_transpose_1d, the cropping view, cont, the bias add, transpose,
    cont)."""
    h = HiftGraph(host_new)
    x = h.t(f32(12, 32))
    w, b = h.t(torch.zeros(32, 16, K, dtype=torch.float16)), h.t(f32(16))
    h.conv_transpose1d(h.leaky(x, 0.1), w, b, stride, pad, DUMMY_W)
    assert h.g.plan() == [(C.GL_CONV_TRANSPOSE1D, 0, 10, C.GLF_LEAKY | C.GLF_BIAS)]


def test_conv_chains_that_do_not_fuse():
    def sublayer_graph():
        h = HiftGraph(host_new)
        x = h.t(f32(40, 16))
        return h, x, hift_params(h)

    # no prepared weights on the mul_mat: ggml's own mul_mat, not a conv launch
    h, x, p = sublayer_graph()
    h.sublayer(x, p, 1, None, DUMMY_W)
    plan = h.g.plan()
    assert plan[0] == (C.GL_SNAKE, 0, 5, 0)
    assert C.GL_UNSUPPORTED in [q[0] for q in plan]
    assert plan[-1] == (C.GL_CONV1D, 16, 17, C.GLF_SNAKE | C.GLF_BIAS | C.GLF_RESIDUAL)

    # the caller keeps the im2col columns: the chain stays apart
    h, x, p = sublayer_graph()
    h.sublayer(x, p, 1, DUMMY_W, DUMMY_W)
    col = h.g.nodes[7].dst
    assert h.g.nodes[7].op == C.GOP_IM2COL
    assert h.g.plan(keep=[col])[0] == (C.GL_SNAKE, 0, 5, 0)

    # the snake's result read elsewhere too: the snake runs alone, the conv
    # takes no prologue
    h, x, p = sublayer_graph()
    s = h.snake(x, p["a1"], p["ai1"])
    y = h.conv1d(s, p["w1"], p["b1"], 1, 1, 1, DUMMY_W)
    h.add(s, y)
    assert h.g.plan() == [(C.GL_SNAKE, 0, 5, 0), (C.GL_CONV1D, 5, 12, C.GLF_BIAS | C.GLF_RESIDUAL)]

    # alpha with one value per frame ((1, T), legal for a standalone snake)
    # is not the conv prologue's per-channel alpha, even when T == C_in: the
    # snake runs alone and the conv takes no prologue
    for T in (16, 40):
        h = HiftGraph(host_new)
        x = h.t(f32(T, 16))
        a, ai = h.t(f32(T, 1)), h.t(f32(T, 1))
        w, b = h.t(torch.zeros(16, 16, 3, dtype=torch.float16)), h.t(f32(16))
        h.conv1d(h.snake(x, a, ai), w, b, 1, 1, 1, DUMMY_W)
        assert h.g.plan() == [(C.GL_SNAKE, 0, 5, 0), (C.GL_CONV1D, 5, 11, C.GLF_BIAS)], T

    # a weight whose C_in is not x's
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    h.conv1d(x, h.t(torch.zeros(16, 8, 3)), None, 1, 1, 1, DUMMY_W)
    assert C.GL_CONV1D not in [q[0] for q in h.g.plan()]

    # conv1d_CT over two batch items: the graph's (OL*N, OC) -> (OL, OC, N)
    # reshape mixes the items, so the chain is not a batched conv
    h = HiftGraph(host_new)
    x = h.t(f32(2, 40, 16))
    h.conv1d(x, h.t(torch.zeros(16, 16, 3)), None, 1, 1, 1, DUMMY_W)
    assert C.GL_CONV1D not in [q[0] for q in h.g.plan()]

    # a transposed conv over two batch items: not the reference's shape
    h = HiftGraph(host_new)
    x = h.t(f32(2, 12, 32))
    w = h.t(torch.zeros(32, 16, 4))
    h.conv_transpose1d(x, w, None, 2, 1, DUMMY_W)
    assert C.GL_CONV_TRANSPOSE1D not in [q[0] for q in h.g.plan()]


def test_hand_made_conv_launches_are_refused():
    """A conv launch whose node count or flags do not fit the chain is
    refused before any weights or device are touched."""
    L = C.load()
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    h.sublayer(x, hift_params(h), 1, DUMMY_W, DUMMY_W)
    T, N, _ = _raw(h.g)
    nt, nn = len(h.g._descs), len(h.g.nodes)
    bad = [C.GLaunch(C.GL_CONV1D, 0, 16, C.GLF_SNAKE),                    # bias nodes not counted
           C.GLaunch(C.GL_CONV1D, 0, 16, C.GLF_SNAKE | C.GLF_LEAKY | C.GLF_BIAS),
           C.GLaunch(C.GL_CONV1D, 0, 8, 0),                               # shorter than any conv chain
           C.GLaunch(C.GL_CONV_TRANSPOSE1D, 16, 17, C.GLF_SNAKE | C.GLF_BIAS | C.GLF_RESIDUAL),
           C.GLaunch(C.GL_CONV1D, 20, 17, C.GLF_SNAKE | C.GLF_BIAS | C.GLF_RESIDUAL)]  # past the list
    for l in bad:
        assert L.cbx_graph_launch(T, nt, N, nn, ctypes.byref(l), None) == C.ERR_INVALID_ARG, \
            (l.kind, l.first_node, l.n_nodes, l.flags)


def test_cfm_causal_block():
    """causal_block1d (cfm_decoder.cpp:133-149): mul(x, mask) and the causal
    conv's 14 nodes (with its bias add) are one causal-conv launch, then
    layer_norm -> mish -> mul(mask) one more."""
    h = HiftGraph(host_new)
    x, mask = h.t(f32(50, 32)), h.t(f32(50, 1))
    w, b = h.t(torch.zeros(64, 32, 3, dtype=torch.float16)), h.t(f32(64))
    lw, lb = h.t(f32(64)), h.t(f32(64))
    h.causal_block(x, mask, w, b, lw, lb, DUMMY_W)
    assert h.g.plan() == [(C.GL_CAUSAL_CONV1D, 0, 15, C.GLF_MASK | C.GLF_BIAS), (C.GL_LAYER_NORM_MASK, 15, 7, 0)]
    # hand-made launches whose flags do not fit the 15 nodes are refused before any weights are read
    L = C.load()
    T_, N_, _ = _raw(h.g)
    for l in (C.GLaunch(C.GL_CAUSAL_CONV1D, 0, 15, C.GLF_BIAS), C.GLaunch(C.GL_CAUSAL_CONV1D, 0, 15, C.GLF_SNAKE),
              C.GLaunch(C.GL_CAUSAL_CONV1D, 0, 15, C.GLF_MASK | C.GLF_BIAS | C.GLF_RESIDUAL),
              C.GLaunch(C.GL_CAUSAL_CONV1D, 0, 11, 0)):
        assert L.cbx_graph_launch(T_, len(h.g._descs), N_, len(h.g.nodes), ctypes.byref(l), None) == C.ERR_INVALID_ARG


def test_causal_conv_forms():
    # no mask, no bias: 12 nodes
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    h.causal_conv1d(x, h.t(torch.zeros(24, 16, 4)), None, DUMMY_W)
    assert h.g.plan() == [(C.GL_CAUSAL_CONV1D, 0, 12, 0)]
    # the caller keeps the transposed copy: not fused
    x_tc = h.g.nodes[1].dst
    assert C.GL_CAUSAL_CONV1D not in [q[0] for q in h.g.plan(keep=[x_tc])]
    # a padding of K - 2 frames is not a causal conv of this weight
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    h.causal_conv1d(x, h.t(torch.zeros(24, 16, 4)), None, DUMMY_W)
    zv = h.g.nodes[2].dst
    h.g._descs[zv] = C.desc(h.at(h.g.nodes[1].dst)[:, :2])
    assert C.GL_CAUSAL_CONV1D not in [q[0] for q in h.g.plan()]
    # no prepared weights: the mul_mat stays the caller's
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    h.causal_conv1d(x, h.t(torch.zeros(24, 16, 3)), None, None)
    assert C.GL_CAUSAL_CONV1D not in [q[0] for q in h.g.plan()]
    # a mask that is not one value per frame is a plain multiply
    h = HiftGraph(host_new)
    x = h.t(f32(40, 16))
    m = h.t(f32(40, 16))
    h.causal_conv1d(h.mul(x, m), h.t(torch.zeros(24, 16, 3)), None, DUMMY_W)
    assert h.g.plan()[:2] == [(C.GL_BINARY, 0, 1, C.BINARY_MUL), (C.GL_CAUSAL_CONV1D, 1, 12, 0)]


def test_mutated_conv_chains_plan_into_an_exact_cover():
    """The reference's conv chains (a ResBlock layer, an upsampler, a causal
    block) with one node field changed at random -- an operand, the op, a
    parameter, the prepared weights -- still plan into an exact cover of the
    list, each launch within its kind's span (no chain is misread past its
    nodes, nothing runs off the list)."""
    spans = {C.GL_CONV1D: range(9, 18), C.GL_CONV_TRANSPOSE1D: range(7, 15), C.GL_CAUSAL_CONV1D: range(12, 16)}
    rng = np.random.default_rng(11)

    def lists():
        h = HiftGraph(host_new)
        h.sublayer(h.t(f32(40, 16)), hift_params(h), 3, DUMMY_W, DUMMY_W)
        yield h
        h = HiftGraph(host_new)
        h.conv_transpose1d(h.leaky(h.t(f32(12, 32)), 0.1), h.t(torch.zeros(32, 16, 8)), h.t(f32(16)), 4, 2, DUMMY_W)
        yield h
        h = HiftGraph(host_new)
        h.causal_block(h.t(f32(50, 32)), h.t(f32(50, 1)), h.t(torch.zeros(64, 32, 3)), h.t(f32(64)), h.t(f32(64)),
                       h.t(f32(64)), DUMMY_W)
        yield h

    for trial in range(300):
        for h in lists():
            g = h.g
            n = g.nodes[int(rng.integers(0, len(g.nodes)))]
            field = int(rng.integers(0, 6))
            if field == 0:
                n.src[0] = int(rng.integers(-1, len(g._descs)))
            elif field == 1:
                n.src[1] = int(rng.integers(-1, len(g._descs)))
            elif field == 2:
                n.op = int(rng.integers(0, 18))
            elif field == 3:
                n.dst = int(rng.integers(0, len(g._descs)))
            elif field == 4:
                n.conv[int(rng.integers(0, 3))] = int(rng.integers(-1, 4))
            else:
                n.conv_w = None if n.conv_w else DUMMY_W
            at = 0
            for kind, first, cnt, flags in g.plan():
                assert first == at, (trial, kind)
                if kind in spans:
                    assert cnt in spans[kind], (trial, kind, cnt)
                at += cnt
            assert at == len(g.nodes)
