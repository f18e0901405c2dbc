"""cbx_graph_compute on the reference's ggml node chains, checked against
the oracle evaluating the same nodes one at a time (ggml-cpu's order of
operations): T3 input embedding + first LayerNorm (t3.cpp:446-466),
causal_block1d's LayerNorm -> Mish (cfm_decoder.cpp:143-146), snake
(hift_vocoder.cpp:64-73), attention scores (t3.cpp:513-518), LayerNorm ->
view -> RoPE, GroupNorm + affine + Mish, and a list of single ops.  Also
checks how many kernel launches each list took.  The HiFT conv chains
(a ResBlock layer, an upsampler) are checked launch by launch against the
oracle's conv1d / conv_transpose1d."""
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


def empty(*shape, dtype=torch.float32):
    return torch.full(shape, float("nan"), dtype=dtype, device="cuda")


@pytest.mark.parametrize("keep_h", [True, False])
def test_t3_input_embedding(cbx, oracle, keep_h):
    n, D = 150, 1024
    tok_q = W.quantize_q8_0(W.normal(W.seed_of(7, 0), (704, D), 0.0, 0.02))
    pos_t = W.normal(W.seed_of(7, 1), (600, D), 0.0, 0.02)
    ids = W.randint(W.seed_of(7, 2), (n,), 0, 704)
    pids = np.arange(3, 3 + n, dtype=np.int32)
    w = W.normal(W.seed_of(7, 3), (D,), 1.0, 0.02)
    b = W.normal(W.seed_of(7, 4), (D,), 0.0, 0.02)

    g = cbx.Graph()
    tok = g.tensor(dev(tok_q), cbx.Q8_0)
    pos = g.tensor(dev(pos_t))
    ti, tp = g.tensor(dev(ids)), g.tensor(dev(pids))
    tw, tb = g.tensor(dev(w)), g.tensor(dev(b))
    buf = [empty(n, D) for _ in range(8)]
    t = [g.tensor(x) for x in buf]
    g.node(cbx.GOP_GET_ROWS, t[0], (tok, ti))
    g.node(cbx.GOP_CPY, t[1], (t[0],))
    g.node(cbx.GOP_GET_ROWS, t[2], (pos, tp))
    g.node(cbx.GOP_CPY, t[3], (t[2],))
    g.node(cbx.GOP_ADD, t[4], (t[1], t[3]))
    g.node(cbx.GOP_NORM, t[5], (t[4],), fparam=1e-5)
    g.node(cbx.GOP_MUL, t[6], (t[5], tw))
    g.node(cbx.GOP_ADD, t[7], (t[6], tb))
    keep = [t[4]] if keep_h else []
    assert g.compute(keep) == 1

    h = oracle.add(oracle.cpy(oracle.get_rows(tok_q, ids, q8_0=True), np.float32),
                   oracle.cpy(oracle.get_rows(pos_t, pids), np.float32))
    y = oracle.add(oracle.mul(oracle.norm(h, 1e-5), w), b)
    assert_bitexact(host(buf[7]), y, "LN(tok + pos)")
    if keep_h:
        assert_bitexact(host(buf[4]), h, "h kept")
    else:
        assert np.isnan(host(buf[4])).all(), "h was not asked for and stays unwritten"


@pytest.mark.parametrize("prompt,text_q8,keep_h", [(True, False, True), (True, True, False), (False, False, True)])
def test_t3_input_with_conditioning_prefix(cbx, oracle, prompt, text_q8, keep_h):
    """t3.cpp:432-466: the conditioning row (the encoder's output, given),
    the prompt's speech-token rows and the text-token rows concatenated,
    plus the position rows, then LN-1 -- the reference's node list, one
    launch, against the oracle evaluating every node (concat is a copy)."""
    D, Lp, Lt = 1024, 150, 40
    n = 1 + (Lp if prompt else 0) + Lt
    cond = W.normal(W.seed_of(7, 10), (1, D), 0.0, 0.5)
    speech = W.normal(W.seed_of(7, 11), (900, D), 0.0, 0.02).astype(np.float16)
    text = W.normal(W.seed_of(7, 12), (2000, D), 0.0, 0.02)
    text_dev = W.quantize_q8_0(text) if text_q8 else text.astype(np.float16)
    posT = W.normal(W.seed_of(7, 13), (600, D), 0.0, 0.02).astype(np.float16)
    prompt_ids = W.randint(W.seed_of(7, 14), (Lp,), 0, 900)
    toks = W.randint(W.seed_of(7, 15), (Lt,), 0, 2000)
    positions = np.arange(n, dtype=np.int32)
    w = W.normal(W.seed_of(7, 16), (D,), 1.0, 0.02)
    b = W.normal(W.seed_of(7, 17), (D,), 0.0, 0.02)

    g = cbx.Graph()
    tc = g.tensor(dev(cond))
    tsp, ttx = g.tensor(dev(speech)), g.tensor(dev(text_dev), cbx.Q8_0 if text_q8 else None)
    tps = g.tensor(dev(posT))
    tpi, ttk, tpo = g.tensor(dev(prompt_ids)), g.tensor(dev(toks)), g.tensor(dev(positions))
    tw, tb = g.tensor(dev(w)), g.tensor(dev(b))
    outs = {}

    def node(op, shape, src, **kw):
        buf = empty(*shape)
        t = g.tensor(buf)
        outs[t] = buf
        g.node(op, t, src, **kw)
        return t

    seq = tc
    if prompt:
        gp = node(cbx.GOP_GET_ROWS, (Lp, D), (tsp, tpi))
        cp = node(cbx.GOP_CPY, (Lp, D), (gp,))
        seq = node(cbx.GOP_CONCAT, (1 + Lp, D), (seq, cp), iparam=1)
    gt = node(cbx.GOP_GET_ROWS, (Lt, D), (ttx, ttk))
    ct = node(cbx.GOP_CPY, (Lt, D), (gt,))
    seq = node(cbx.GOP_CONCAT, (n, D), (seq, ct), iparam=1)
    gq = node(cbx.GOP_GET_ROWS, (n, D), (tps, tpo))
    cq = node(cbx.GOP_CPY, (n, D), (gq,))
    h = node(cbx.GOP_ADD, (n, D), (seq, cq))
    nn = node(cbx.GOP_NORM, (n, D), (h,), fparam=1e-5)
    mm = node(cbx.GOP_MUL, (n, D), (nn, tw))
    y = node(cbx.GOP_ADD, (n, D), (mm, tb))
    keep = [h, y] if keep_h else [y]
    assert g.compute(keep) == 1
    assert g.plan(keep)[0][0] == cbx.GL_GET_ROWS_CONCAT_ADD_LAYER_NORM

    parts = [cond]
    if prompt:
        parts.append(oracle.cpy(oracle.get_rows(speech, prompt_ids), np.float32))
    parts.append(oracle.cpy(oracle.get_rows(text_dev, toks, q8_0=text_q8), np.float32))
    h_ref = oracle.add(np.concatenate(parts, axis=0), oracle.cpy(oracle.get_rows(posT, positions), np.float32))
    y_ref = oracle.add(oracle.mul(oracle.norm(h_ref, 1e-5), w), b)
    assert_bitexact(host(outs[y]), y_ref, "LN(concat + pos)")
    if keep_h:
        assert_bitexact(host(outs[h]), h_ref, "h kept")
    else:
        assert np.isnan(host(outs[h])).all(), "h was not asked for and stays unwritten"


def test_t3_input_with_prefix_bad_id(cbx):
    """An out-of-range text id zeroes that row and raises the device error
    bit; the other rows are unaffected."""
    import ctypes
    D = 256
    cond = dev(W.normal(3, (2, D)))
    text = dev(W.normal(4, (50, D)))
    posT = dev(W.normal(5, (60, D)))
    toks = dev(np.array([1, 2, 77, 3], dtype=np.int32))
    pos = dev(np.arange(6, dtype=np.int32))
    h, y = cbx.get_rows_concat_add_layer_norm(cond, None, None, text, toks, posT, pos, None, None, 1e-5)
    flags = ctypes.c_uint32(0)
    assert cbx.load().cbx_device_errors(0, ctypes.byref(flags), 1) == cbx.OK
    assert flags.value & 1
    yh = host(y)
    assert not yh[4].any() and not host(h)[4].any()
    assert np.abs(yh[[0, 1, 2, 3, 5]]).sum() > 0


def test_causal_block_layer_norm_mish(cbx, oracle):
    T, Ch = 300, 256
    x = W.normal(W.seed_of(8, 0), (T, Ch), 0.1, 1.5)
    w = W.normal(W.seed_of(8, 1), (Ch,), 1.0, 0.05)
    b = W.normal(W.seed_of(8, 2), (Ch,), 0.0, 0.05)
    g = cbx.Graph()
    tx, tw, tb = g.tensor(dev(x)), g.tensor(dev(w)), g.tensor(dev(b))
    buf = [empty(T, Ch) for _ in range(6)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_NORM, t[0], (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, t[1], (t[0], tw))
    g.node(cbx.GOP_ADD, t[2], (t[1], tb))
    g.node(cbx.GOP_UNARY, t[3], (t[2],), iparam=cbx.SOFTPLUS)
    g.node(cbx.GOP_UNARY, t[4], (t[3],), iparam=cbx.TANH)
    g.node(cbx.GOP_MUL, t[5], (t[2], t[4]))
    assert g.compute() == 1
    ln = oracle.add(oracle.mul(oracle.norm(x, 1e-5), w), b)
    exp = oracle.mul(ln, oracle.unary(oracle.TANH, oracle.unary(oracle.SOFTPLUS, ln)))
    assert_close(host(buf[5]), exp, x=ln, what="layer_norm -> mish nodes")


def test_snake_nodes(cbx, oracle):
    T, Ch = 2000, 128
    x = W.normal(W.seed_of(9, 0), (T, Ch), 0.0, 2.0)
    alpha = np.abs(W.normal(W.seed_of(9, 1), (Ch,), 1.0, 0.3)).astype(np.float32)
    alpha_inv = (1.0 / (alpha + np.float32(1e-9))).astype(np.float32)
    g = cbx.Graph()
    tx, ta, tai = g.tensor(dev(x)), g.tensor(dev(alpha)), g.tensor(dev(alpha_inv))
    buf = [empty(T, Ch) for _ in range(5)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_MUL, t[0], (tx, ta))
    g.node(cbx.GOP_UNARY, t[1], (t[0],), iparam=cbx.SIN)
    g.node(cbx.GOP_UNARY, t[2], (t[1],), iparam=cbx.SQR)
    g.node(cbx.GOP_MUL, t[3], (t[2], tai))
    g.node(cbx.GOP_ADD, t[4], (tx, t[3]))
    assert g.compute() == 1
    xa = oracle.mul(x, alpha)
    exp = oracle.add(x, oracle.mul(oracle.unary(oracle.SQR, oracle.unary(oracle.SIN, xa)), alpha_inv))
    assert_close(host(buf[4]), exp, x=x, what="snake nodes")


@pytest.mark.parametrize("n_past", [-1, 0, 37])
def test_attention_score_nodes(cbx, oracle, n_past):
    H, nq = 8, 40
    nk = n_past + nq if n_past >= 0 else 40
    kq = W.normal(W.seed_of(10, n_past + 2), (H, nq, nk), 0.0, 3.0)
    s = np.float32(1.0 / np.sqrt(64.0))
    g = cbx.Graph()
    tkq = g.tensor(dev(kq))
    buf = [empty(H, nq, nk) for _ in range(3)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_SCALE, t[0], (tkq,), fparam=float(s))
    src = t[0]
    if n_past >= 0:
        g.node(cbx.GOP_DIAG_MASK_INF, t[1], (t[0],), iparam=n_past)
        src = t[1]
    g.node(cbx.GOP_SOFT_MAX, t[2], (src,), fparam=1.0)
    assert g.compute() == 1
    z = oracle.scale(kq, float(s))
    if n_past >= 0:
        z = oracle.diag_mask_inf(z, n_past)
    assert_close(host(buf[2]), oracle.soft_max(z), what=f"scores n_past={n_past}")


def test_layer_norm_view_rope(cbx, oracle):
    B, T, H, hd = 2, 100, 8, 64
    x = W.normal(W.seed_of(11, 0), (B, T, H * hd), 0.2, 1.0)
    w = W.normal(W.seed_of(11, 1), (H * hd,), 1.0, 0.02)
    b = W.normal(W.seed_of(11, 2), (H * hd,), 0.0, 0.02)
    pos = np.arange(T, dtype=np.int32)
    cache = cbx.RopeCache(hd, mode=2, n_ctx_orig=2048, n_pos=2048)
    g = cbx.Graph()
    tx, tw, tb, tp = g.tensor(dev(x)), g.tensor(dev(w)), g.tensor(dev(b)), g.tensor(dev(pos))
    n_, m_, y_ = (g.tensor(empty(B, T, H * hd)) for _ in range(3))
    y_buf = g._torch[y_]
    v_ = g.tensor(y_buf.view(B, T, H, hd))
    out = empty(B, T, H, hd)
    r_ = g.tensor(out)
    g.node(cbx.GOP_NORM, n_, (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, m_, (n_, tw))
    g.node(cbx.GOP_ADD, y_, (m_, tb))
    g.node(cbx.GOP_VIEW, v_, (y_,))
    g.node(cbx.GOP_ROPE, r_, (v_, tp), rope=cache)
    assert g.compute() == 1
    ln = oracle.add(oracle.mul(oracle.norm(x, 1e-5), w), b)
    exp = oracle.rope_ext(ln.reshape(B, T, H, hd), pos, hd, mode=2)
    assert_bitexact(host(out), exp, "layer_norm -> view -> rope")
    cache.close()


def test_group_norm_affine_mish_nodes(cbx, oracle):
    inp = W.cfm_inputs()
    x, w, b = inp["x256"], inp["w256"], inp["b256"]
    g = cbx.Graph()
    tx, tw, tb = g.tensor(dev(x)), g.tensor(dev(w)), g.tensor(dev(b))
    buf = [empty(*x.shape) for _ in range(6)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_GROUP_NORM, t[0], (tx,), iparam=8, fparam=1e-5)
    g.node(cbx.GOP_MUL, t[1], (t[0], tw))
    g.node(cbx.GOP_ADD, t[2], (t[1], tb))
    g.node(cbx.GOP_UNARY, t[3], (t[2],), iparam=cbx.SOFTPLUS)
    g.node(cbx.GOP_UNARY, t[4], (t[3],), iparam=cbx.TANH)
    g.node(cbx.GOP_MUL, t[5], (t[2], t[4]))
    assert g.compute() == 1
    gn = oracle.add(oracle.mul(oracle.group_norm(x, 8, 1e-5, nth=8), w), b)
    exp = oracle.mul(gn, oracle.unary(oracle.TANH, oracle.unary(oracle.SOFTPLUS, gn)))
    assert_close(host(buf[5]), exp, x=gn, what="group_norm -> mul -> add -> mish nodes")


def test_single_ops_and_views(cbx, oracle):
    R, Cc = 64, 1024
    a = W.normal(W.seed_of(12, 0), (R, Cc), 0.0, 3.0)
    u = W.normal(W.seed_of(12, 1), (R, Cc), 0.0, 1.0)
    gain = W.normal(W.seed_of(12, 2), (Cc,), 1.0, 0.1)
    g = cbx.Graph()
    ta, tu, tg = g.tensor(dev(a)), g.tensor(dev(u)), g.tensor(dev(gain))
    bufs = {k: empty(R, Cc) for k in ("s", "sw", "ge", "lr", "rn", "rm")}
    h16 = empty(R, Cc, dtype=torch.float16)
    t = {k: g.tensor(v) for k, v in bufs.items()}
    t16 = g.tensor(h16)
    sw_view = g.tensor(bufs["sw"].view(R * 4, Cc // 4))
    g.node(cbx.GOP_UNARY, t["s"], (ta,), iparam=cbx.SILU)
    g.node(cbx.GOP_MUL, t["sw"], (t["s"], tu))
    g.node(cbx.GOP_VIEW, sw_view, (t["sw"],))
    g.node(cbx.GOP_UNARY, t["ge"], (t["sw"],), iparam=cbx.GELU)
    g.node(cbx.GOP_LEAKY_RELU, t["lr"], (t["ge"],), fparam=0.1)
    g.node(cbx.GOP_RMS_NORM, t["rn"], (t["lr"],), fparam=1e-6)
    g.node(cbx.GOP_MUL, t["rm"], (t["rn"], tg))
    g.node(cbx.GOP_CPY, t16, (t["rm"],))
    assert g.compute() == 5            # swiglu, gelu, leaky_relu, rms_norm*g, cast
    sw = oracle.mul(oracle.unary(oracle.SILU, a), u)
    got_sw = host(bufs["sw"])
    assert_close(got_sw, sw, x=a, what="silu -> mul")
    # the remaining nodes are exact ops: feed them the device's own swiglu result
    ge = oracle.unary(oracle.GELU, got_sw)
    assert_bitexact(host(bufs["ge"]), ge, "gelu")
    lr = oracle.leaky_relu(ge, 0.1)
    assert_bitexact(host(bufs["lr"]), lr, "leaky_relu")
    rm = oracle.mul(oracle.rms_norm(lr, 1e-6), gain)
    assert_bitexact(host(bufs["rm"]), rm, "rms_norm -> mul")
    assert_bitexact(host(h16), oracle.cpy(rm, np.float16), "cast f16")
    assert np.isnan(host(bufs["rn"])).all(), "rms_norm's own output is fused away"


def test_plan_then_launch_one_by_one(cbx, oracle):
    """cbx_graph_plan + cbx_graph_launch, as a scheduler that interleaves
    its own kernels would use them: same results as compute."""
    import ctypes

    T, Ch = 64, 256
    x = W.normal(W.seed_of(13, 0), (T, Ch))
    w = W.normal(W.seed_of(13, 1), (Ch,), 1.0, 0.05)
    b = W.normal(W.seed_of(13, 2), (Ch,), 0.0, 0.05)
    g = cbx.Graph()
    tx, tw, tb = g.tensor(dev(x)), g.tensor(dev(w)), g.tensor(dev(b))
    buf = [empty(T, Ch) for _ in range(4)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_NORM, t[0], (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, t[1], (t[0], tw))
    g.node(cbx.GOP_ADD, t[2], (t[1], tb))
    g.node(cbx.GOP_UNARY, t[3], (t[2],), iparam=cbx.GELU)
    plan = g.plan()
    assert [p[0] for p in plan] == [cbx.GL_LAYER_NORM, cbx.GL_UNARY]
    T_, N_, _ = g._arrays([])
    L = cbx.load()
    for kind, first, n, flags in plan:
        rc = L.cbx_graph_launch(T_, len(g._descs), N_, len(g.nodes), ctypes.byref(cbx.GLaunch(kind, first, n, flags)),
                                cbx._stream())
        assert rc == cbx.OK, cbx.last_error()
    ln = oracle.add(oracle.mul(oracle.norm(x, 1e-5), w), b)
    assert_bitexact(host(buf[2]), ln, "planned layer_norm")
    assert_bitexact(host(buf[3]), oracle.unary(oracle.GELU, ln), "planned gelu")


def test_layout_error_names_the_nodes(cbx):
    """A chain that matches on structure but not on layout (a strided gain)
    fails in the entry point; the message names the node range."""
    g = cbx.Graph()
    x = g.tensor(empty(4, 2048))
    w_full = empty(2048 * 2)
    w = g.tensor(w_full[::2])                      # (2048,) with an 8-byte stride
    b = g.tensor(empty(2048))
    t = [g.tensor(empty(4, 2048)) for _ in range(3)]
    g.node(cbx.GOP_NORM, t[0], (x,), fparam=1e-5)
    g.node(cbx.GOP_MUL, t[1], (t[0], w))
    g.node(cbx.GOP_ADD, t[2], (t[1], b))
    with pytest.raises(cbx.CbxError) as e:
        g.compute()
    assert "nodes 0..2" in str(e.value)


# ---- HiFT conv chains --------------------------------------------------------------

def dev_new(shape, dtype=torch.float32):
    return torch.full(shape, float("nan"), dtype=dtype, device="cuda")


@pytest.mark.parametrize("Ch,T,K,d", [(128, 700, 11, 3), (64, 1500, 3, 5)])
def test_resblock_sublayer_nodes(cbx, oracle, Ch, T, K, d):
    """resblock_forward's layer as the reference's node list
    (hift_vocoder.cpp:131-135): two conv launches, the first writing the
    conv1d_CT result the second reads.  Each is checked against the oracle's
    conv1d on the same input it read, within the conv tolerance
    2^-13 sum |a b| + 2^-22 |ref| (f16 products summed in f32)."""
    from tests._hift_graph import HiftGraph
    from tests.test_gpu_conv1d import check

    sd = W.seed_of(13, K)
    x = W.normal(sd, (T, Ch), 0.0, 1.0)
    arrs, p, wts = {}, {}, []
    h = HiftGraph(dev_new)
    tx = h.t(dev(x))
    for k, s in enumerate(("1", "2")):
        a, ai = W.snake_alpha(Ch, 20 + k)
        w = W.normal(sd + 1 + k, (Ch, Ch, K), 0.0, 1.0 / np.sqrt(Ch * K))
        b = W.normal(sd + 3 + k, (Ch,), 0.0, 0.1)
        arrs.update({"a" + s: a, "ai" + s: ai, "w" + s: w, "b" + s: b})
        for name, v in (("a", a), ("ai", ai), ("w", w), ("b", b)):
            p[name + s] = h.t(dev(v))
        wts.append(cbx.Conv1dWeights(h.at(p["w" + s])))
    y = h.sublayer(tx, p, d, wts[0], wts[1])
    plan = h.g.plan()
    assert [q[0] for q in plan] == [cbx.GL_CONV1D] * 2
    assert h.g.compute() == 2
    mid = host(h.at(h.g.nodes[plan[0][2] - 1].dst)).reshape(T, Ch)   # the first conv1d_CT's result
    got = host(h.at(y))
    check(oracle, mid, x, arrs["w1"], 1, (K - 1) // 2 * d, d, oracle.CONV_PRO_SNAKE, arrs["a1"], arrs["ai1"], 0.0,
          arrs["b1"], None, "first conv of the layer")
    check(oracle, got, mid, arrs["w2"], 1, (K - 1) // 2, 1, oracle.CONV_PRO_SNAKE, arrs["a2"], arrs["ai2"], 0.0,
          arrs["b2"], x, "second conv + residual")
    for w_ in wts:
        w_.close()


def test_conv_pre_nodes(cbx, oracle):
    """conv_pre (hift_vocoder.cpp:673): conv1d_CT with no prologue, K 7,
    padding 3, bias, 80 mel channels in -> 512 out, as the reference's nine
    nodes plus the bias add: one conv launch, checked against the oracle's
    conv1d within the conv tolerance."""
    from tests._hift_graph import HiftGraph
    from tests.test_gpu_conv1d import check

    T, C_in, C_out, K = 300, 80, 512, 7
    sd = W.seed_of(17, 0)
    x = W.normal(sd, (T, C_in))
    w = W.normal(sd + 1, (C_out, C_in, K), 0.0, 1.0 / np.sqrt(C_in * K))
    b = W.normal(sd + 2, (C_out,), 0.0, 0.1)
    h = HiftGraph(dev_new)
    tx, tw, tb = h.t(dev(x)), h.t(dev(w)), h.t(dev(b))
    wts = cbx.Conv1dWeights(h.at(tw))
    y = h.conv1d(tx, tw, tb, 1, 3, 1, wts)
    assert h.g.plan() == [(cbx.GL_CONV1D, 0, 11, cbx.GLF_BIAS)]
    assert h.g.compute() == 1
    check(oracle, host(h.at(y)).reshape(T, C_out), x, w, 1, 3, 1, oracle.CONV_PRO_NONE, None, None, 0.0, b, None,
          "conv_pre nodes")
    wts.close()


@pytest.mark.parametrize("C_in,C_out,s,K,T", [(256, 128, 5, 11, 200), (128, 64, 3, 7, 500)])
def test_upsampler_nodes(cbx, oracle, C_in, C_out, s, K, T):
    """leaky_relu -> conv_transpose1d_CT (hift_vocoder.cpp:686-687) as the
    reference's node list: one transposed-conv launch, checked against the
    oracle's conv_transpose1d within the conv tolerance."""
    from tests._hift_graph import HiftGraph
    from tests.test_gpu_conv_transpose1d import check

    pad = (K - s) // 2
    sd = W.seed_of(14, s)
    x = W.normal(sd, (T, C_in), 0.0, 1.0)
    w = W.normal(sd + 1, (C_in, C_out, K), 0.0, 1.0 / np.sqrt(C_in * K / s))
    b = W.normal(sd + 2, (C_out,), 0.0, 0.1)
    h = HiftGraph(dev_new)
    tx, tw, tb = h.t(dev(x)), h.t(dev(w)), h.t(dev(b))
    wts = cbx.Conv1dWeights(h.at(tw), transpose_stride=s)
    y = h.conv_transpose1d(h.leaky(tx, 0.1), tw, tb, s, pad, wts)
    assert h.g.plan() == [(cbx.GL_CONV_TRANSPOSE1D, 0, 10, cbx.GLF_LEAKY | cbx.GLF_BIAS)]
    assert h.g.compute() == 1
    check(oracle, host(h.at(y)), x, w, s, pad, oracle.CONV_PRO_LEAKY, 0.1, b, "upsampler nodes")
    wts.close()


def test_conv_weights_of_another_shape_are_refused(cbx):
    """A conv launch whose prepared weights were made from another weight
    than the node's is refused before it runs."""
    from tests._hift_graph import HiftGraph

    h = HiftGraph(dev_new)
    x = h.t(dev_new((50, 16)).zero_())
    w = h.t(dev_new((16, 16, 3)).zero_())
    other = cbx.Conv1dWeights(dev_new((16, 16, 5)).zero_())
    h.conv1d(x, w, None, 1, 1, 1, other)
    assert h.g.plan() == [(cbx.GL_CONV1D, 0, 9, 0)]
    with pytest.raises(cbx.CbxError, match="conv_w was not made from the node's weight tensor"):
        h.g.compute()
    other.close()


def test_cfm_causal_block_nodes(cbx, oracle):
    """causal_block1d (cfm_decoder.cpp:133-149) as the reference's node list:
    mul(x, mask) -> causal_conv1d (+ bias) in one launch, layer_norm -> mish
    -> mul(mask) in another.  The conv output is checked against the oracle's
    conv of mask * x (K - 1 zero frames in front) within the conv
    tolerance; the tail against the oracle's nodes on that output."""
    from tests._hift_graph import HiftGraph

    T, C_in, C_out, K = 500, 256, 256, 3
    sd = W.seed_of(16, 0)
    x = W.normal(sd, (T, C_in))
    mask = np.ones((T, 1), dtype=np.float32)
    mask[T - 60:] = 0.0
    w = W.normal(sd + 1, (C_out, C_in, K), 0.0, 1.0 / np.sqrt(C_in * K))
    b = W.normal(sd + 2, (C_out,), 0.0, 0.1)
    lw = W.normal(sd + 3, (C_out,), 1.0, 0.02)
    lb = W.normal(sd + 4, (C_out,), 0.0, 0.02)
    h = HiftGraph(dev_new)
    tx, tm, tw, tb, tlw, tlb = (h.t(dev(v)) for v in (x, mask, w, b, lw, lb))
    wts = cbx.Conv1dWeights(h.at(tw))
    y = h.causal_block(tx, tm, tw, tb, tlw, tlb, wts)
    plan = h.g.plan()
    assert plan == [(cbx.GL_CAUSAL_CONV1D, 0, 15, cbx.GLF_MASK | cbx.GLF_BIAS), (cbx.GL_LAYER_NORM_MASK, 15, 7, 0)]
    assert h.g.compute() == 2
    conv = host(h.at(h.g.nodes[14].dst))
    xm = oracle.mul(x, mask)
    ref = oracle.conv1d(xm, w, 1, K - 1, 1, oracle.CONV_PRO_NONE, None, None, 0.0, b, None, nth=8)[:T]
    mag = oracle.conv1d(np.abs(xm), np.abs(w), 1, K - 1, 1, nth=8)[:T].astype(np.float64)
    d = np.abs(conv.astype(np.float64) - ref.astype(np.float64))
    assert not (d > 2.0 ** -13 * mag + 2.0 ** -22 * np.abs(ref)).any()
    ln = oracle.add(oracle.mul(oracle.norm(conv, 1e-5), lw), lb)
    exp = oracle.mul(oracle.mul(ln, oracle.unary(oracle.TANH, oracle.unary(oracle.SOFTPLUS, ln))), mask)
    assert_close(host(h.at(y)), exp, x=ln, what="causal block tail")
    wts.close()
