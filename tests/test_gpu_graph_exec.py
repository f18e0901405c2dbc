"""cbx_graph_exec: a node list planned once, recorded into a HIP graph and
replayed, as a decode or sampling loop would run the same list step after
step (t3.cpp:604, cfm_decoder.cpp:596, hift_vocoder.cpp:765 call
graph_compute on an identical node list every step).  Every replay must
give the bits cbx_graph_compute gives on the same buffers: replays are
interleaved with the program's own eager work (outputs overwritten with
NaN, inputs rewritten in place) and synchronisations, and each replay is
checked.  Node lists: one T3 block's element-wise nodes (three launches),
LayerNorm -> view -> RoPE, GroupNorm -> affine -> Mish, a HiFT ResBlock
layer (two conv launches), the CFM causal block (conv, then LayerNorm
-> Mish -> mask), and a decode step whose position changes between
replays; then cbx_graph_exec_update re-pointing an exec at other buffers,
other sequence lengths and other lists."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def empty(*shape, dtype=torch.float32):
    return torch.full(shape, float("nan"), dtype=dtype, device="cuda")


def new(shape, dtype=torch.float32):
    """HiftGraph's allocator: new(shape, dtype)."""
    return empty(*shape, dtype=dtype)


def bits(t):
    return t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16)


def check_replays(g, keep, outs, inputs, n_launches, replays=3):
    """Two rounds (the inputs as given, then rewritten in place): the eager
    result of the round, then `replays` replays each checked bit for bit
    against it, every replay after the outputs are overwritten with NaN."""
    ex = g.capture(keep)
    assert ex.n_launches == n_launches
    try:
        for rnd in range(2):
            if rnd:
                for t in inputs:
                    t.copy_(t * 0.75 + 0.125)     # new inputs in the same buffers
            for o in outs:
                o.fill_(float("nan"))
            assert g.compute(keep) == n_launches
            torch.cuda.synchronize()
            exp = [bits(o).clone() for o in outs]
            for o in exp:
                assert o.numel() > 0
            for r in range(replays):
                for o in outs:
                    o.fill_(float("nan"))
                torch.cuda.synchronize()
                ex.launch()
                torch.cuda.synchronize()
                for k, (o, e) in enumerate(zip(outs, exp)):
                    assert torch.equal(bits(o), e), f"round {rnd}, replay {r}: output {k} differs from eager"
        # many replays in flight back to back, then one check
        for o in outs:
            o.fill_(float("nan"))
        for _ in range(20):
            ex.launch()
        torch.cuda.synchronize()
        for k, (o, e) in enumerate(zip(outs, exp)):
            assert torch.equal(bits(o), e), f"after 20 replays: output {k} differs from eager"
    finally:
        ex.close()


def test_t3_block_elementwise(cbx):
    """The residual join + LN2, fc bias + GELU, and the projection's residual
    join + next LN1 (t3.cpp:526-546, matmul outputs given): 12 nodes, three
    launches, four kept outputs."""
    t = {k: dev(v) for k, v in W.t3_block_inputs().items()}
    N, D, F = W.N_PREFILL, W.D_MODEL, W.D_FF
    for k in ("cur", "res", "n", "m", "ln2", "pcur", "h2", "n2", "m2", "ln1"):
        t[k] = empty(N, D)
    for k in ("fcb", "gelu"):
        t[k] = empty(N, F)
    g = cbx.Graph()
    T = {k: g.tensor(v) for k, v in t.items()}
    g.node(cbx.GOP_ADD, T["cur"], (T["attn_mm"], T["out_b"]))
    g.node(cbx.GOP_ADD, T["res"], (T["cur"], T["h"]))
    g.node(cbx.GOP_NORM, T["n"], (T["res"],), fparam=1e-5)
    g.node(cbx.GOP_MUL, T["m"], (T["n"], T["ln2_w"]))
    g.node(cbx.GOP_ADD, T["ln2"], (T["m"], T["ln2_b"]))
    g.node(cbx.GOP_ADD, T["fcb"], (T["fc_mm"], T["fc_b"]))
    g.node(cbx.GOP_UNARY, T["gelu"], (T["fcb"],), iparam=cbx.GELU)
    g.node(cbx.GOP_ADD, T["pcur"], (T["proj_mm"], T["proj_b"]))
    g.node(cbx.GOP_ADD, T["h2"], (T["pcur"], T["res"]))
    g.node(cbx.GOP_NORM, T["n2"], (T["h2"],), fparam=1e-5)
    g.node(cbx.GOP_MUL, T["m2"], (T["n2"], T["ln1_w"]))
    g.node(cbx.GOP_ADD, T["ln1"], (T["m2"], T["ln1_b"]))
    keep = [T["ln2"], T["gelu"], T["h2"], T["ln1"]]
    check_replays(g, keep, [t["ln2"], t["gelu"], t["h2"], t["ln1"]],
                  [t["attn_mm"], t["h"], t["fc_mm"], t["proj_mm"]], 3)


def test_layer_norm_view_rope(cbx):
    B, T, H, hd = 2, 100, 8, 64
    x = dev(W.normal(W.seed_of(11, 0), (B, T, H * hd), 0.2, 1.0))
    w = W.normal(W.seed_of(11, 1), (H * hd,), 1.0, 0.02)
    b = W.normal(W.seed_of(11, 2), (H * hd,), 0.0, 0.02)
    pos = np.arange(T, dtype=np.int32)
    cache = cbx.RopeCache(hd, mode=2, n_ctx_orig=2048, n_pos=2048)
    g = cbx.Graph()
    tx, tw, tb, tp = g.tensor(x), g.tensor(dev(w)), g.tensor(dev(b)), g.tensor(dev(pos))
    n_, m_, y_ = (g.tensor(empty(B, T, H * hd)) for _ in range(3))
    v_ = g.tensor(g._torch[y_].view(B, T, H, hd))
    out = empty(B, T, H, hd)
    r_ = g.tensor(out)
    g.node(cbx.GOP_NORM, n_, (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, m_, (n_, tw))
    g.node(cbx.GOP_ADD, y_, (m_, tb))
    g.node(cbx.GOP_VIEW, v_, (y_,))
    g.node(cbx.GOP_ROPE, r_, (v_, tp), rope=cache)
    check_replays(g, [], [out], [x], 1)
    cache.close()


def test_group_norm_affine_mish(cbx):
    inp = W.cfm_inputs()
    x = dev(inp["x256"])
    g = cbx.Graph()
    tx, tw, tb = g.tensor(x), g.tensor(dev(inp["w256"])), g.tensor(dev(inp["b256"]))
    buf = [empty(*x.shape) for _ in range(6)]
    t = [g.tensor(v) for v in buf]
    g.node(cbx.GOP_GROUP_NORM, t[0], (tx,), iparam=8, fparam=1e-5)
    g.node(cbx.GOP_MUL, t[1], (t[0], tw))
    g.node(cbx.GOP_ADD, t[2], (t[1], tb))
    g.node(cbx.GOP_UNARY, t[3], (t[2],), iparam=cbx.SOFTPLUS)
    g.node(cbx.GOP_UNARY, t[4], (t[3],), iparam=cbx.TANH)
    g.node(cbx.GOP_MUL, t[5], (t[2], t[4]))
    check_replays(g, [], [buf[5]], [x], 1)


def test_resblock_layer(cbx):
    """resblock_forward's layer (hift_vocoder.cpp:131-135): two conv
    launches, the second reading what the first wrote."""
    from tests._hift_graph import HiftGraph

    Ch, T, K, d = 128, 700, 11, 3
    sd = W.seed_of(13, K)
    h = HiftGraph(new)
    x = dev(W.normal(sd, (T, Ch), 0.0, 1.0))
    tx = h.t(x)
    p, wts = {}, []
    for k, s in enumerate(("1", "2")):
        a, ai = W.snake_alpha(Ch, 20 + k)
        w = W.normal(sd + 1 + k, (Ch, Ch, K), 0.0, 1.0 / np.sqrt(Ch * K))
        b = W.normal(sd + 3 + k, (Ch,), 0.0, 0.1)
        for name, v in (("a", a), ("ai", ai), ("w", w), ("b", b)):
            p[name + s] = h.t(dev(v))
        wts.append(cbx.Conv1dWeights(h.at(p["w" + s])))
    y = h.sublayer(tx, p, d, wts[0], wts[1])
    plan = h.g.plan()
    assert [q[0] for q in plan] == [cbx.GL_CONV1D] * 2
    mid = h.at(h.g.nodes[plan[0][2] - 1].dst)
    check_replays(h.g, [], [mid, h.at(y)], [x], 2)
    for w_ in wts:
        w_.close()


def test_cfm_causal_block(cbx):
    """causal_block1d (cfm_decoder.cpp:133-149): mul(x, mask) -> causal
    conv + bias, then layer_norm -> mish -> mul(mask)."""
    from tests._hift_graph import HiftGraph

    T, C_in, C_out, K = 500, 256, 256, 3
    sd = W.seed_of(16, 0)
    mask = np.ones((T, 1), dtype=np.float32)
    mask[T - 60:] = 0.0
    h = HiftGraph(new)
    x = dev(W.normal(sd, (T, C_in)))
    w = W.normal(sd + 1, (C_out, C_in, K), 0.0, 1.0 / np.sqrt(C_in * K))
    vals = (mask, w, W.normal(sd + 2, (C_out,), 0.0, 0.1), W.normal(sd + 3, (C_out,), 1.0, 0.02),
            W.normal(sd + 4, (C_out,), 0.0, 0.02))
    tx = h.t(x)
    tm, tw, tb, tlw, tlb = (h.t(dev(v)) for v in vals)
    wts = cbx.Conv1dWeights(h.at(tw))
    y = h.causal_block(tx, tm, tw, tb, tlw, tlb, wts)
    assert [q[0] for q in h.g.plan()] == [cbx.GL_CAUSAL_CONV1D, cbx.GL_LAYER_NORM_MASK]
    check_replays(h.g, [], [h.at(h.g.nodes[14].dst), h.at(y)], [x], 2)
    wts.close()


def test_unsupported_node_is_refused(cbx):
    """A node that starts no chain the library runs: no exec is made."""
    n, D = 16, 64
    g = cbx.Graph()
    a, b, c = g.tensor(dev(np.ones((n, D), np.float32))), g.tensor(dev(np.ones((n, D), np.float32))), \
        g.tensor(empty(n, D))
    g.node(cbx.GOP_ADD, c, (a, b))         # a plain add of two activations: a binary launch
    g.node(cbx.GOP_UNARY, g.tensor(empty(n, D)), (c,), iparam=42)   # no such activation
    with pytest.raises(cbx.CbxError) as e:
        g.capture()
    assert e.value.status == cbx.ERR_UNSUPPORTED
    assert "node 1 (UNARY)" in str(e.value)


def test_views_only_list(cbx):
    """A list of VIEW nodes launches nothing: the exec holds an empty graph
    and its replays do nothing."""
    g = cbx.Graph()
    x = torch.arange(64, dtype=torch.float32, device="cuda")
    a = g.tensor(x)
    v = g.tensor(x.view(8, 8))
    g.node(cbx.GOP_VIEW, v, (a,))
    ex = g.capture()
    assert ex.n_launches == 0
    ex.launch()
    ex.launch()
    torch.cuda.synchronize()
    assert torch.equal(x, torch.arange(64, dtype=torch.float32, device="cuda"))
    ex.close()


def test_decode_step_with_new_positions(cbx):
    """A T3-style decode step (RMSNorm * gain, RoPE of q and k at the
    token's position in one launch, SiLU-gate: 3 launches) replayed as the position and the inputs
    change from step to step in the same buffers -- positions inside the
    cos/sin table, at its last row and past it (computed, not read): every
    replay matches cbx_graph_compute on the same buffers bit for bit."""
    D, H, hd, F = 1024, 16, 64, 4096
    x = dev(W.normal(W.seed_of(21, 0), (1, D)))
    gain = dev(W.normal(W.seed_of(21, 1), (D,), 1.0, 0.05))
    q = dev(W.normal(W.seed_of(21, 2), (1, H, hd)))
    k = dev(W.normal(W.seed_of(21, 3), (1, H, hd)))
    gt = dev(W.normal(W.seed_of(21, 4), (1, F)))
    up = dev(W.normal(W.seed_of(21, 5), (1, F)))
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    cache = cbx.RopeCache(hd, mode=2, n_ctx_orig=2048, n_pos=2048)
    g = cbx.Graph()
    tx, tg_, tq, tk, tgt, tup, tp = (g.tensor(v) for v in (x, gain, q, k, gt, up, pos))
    rn, y, qo, ko, s, o = empty(1, D), empty(1, D), empty(1, H, hd), empty(1, H, hd), empty(1, F), empty(1, F)
    trn, ty, tqo, tko, ts, to = (g.tensor(v) for v in (rn, y, qo, ko, s, o))
    g.node(cbx.GOP_RMS_NORM, trn, (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, ty, (trn, tg_))
    g.node(cbx.GOP_ROPE, tqo, (tq, tp), rope=cache)
    g.node(cbx.GOP_ROPE, tko, (tk, tp), rope=cache)
    g.node(cbx.GOP_UNARY, ts, (tgt,), iparam=cbx.SILU)
    g.node(cbx.GOP_MUL, to, (ts, tup))
    outs = [y, qo, ko, o]
    ex = g.capture()
    assert ex.n_launches == 3
    try:
        for step, p in enumerate((0, 1, 7, 29, 2047, 3000, 5)):
            pos.fill_(p)
            for t in (x, q, k, gt, up):
                t.copy_(t * 0.875 + 0.0625 * step)
            for t in outs:
                t.fill_(float("nan"))
            assert g.compute() == 3
            torch.cuda.synchronize()
            exp = [bits(t).clone() for t in outs]
            for t in outs:
                t.fill_(float("nan"))
            torch.cuda.synchronize()
            ex.launch()
            torch.cuda.synchronize()
            for n, (t, e) in enumerate(zip(outs, exp)):
                assert torch.equal(bits(t), e), f"position {p}: output {n} differs from eager"
    finally:
        ex.close()
        cache.close()


def decode_list(cbx, cache, bufs):
    """The decode step's six nodes over one buffer set (a dict of tensors)."""
    g = cbx.Graph()
    ids = {n: g.tensor(bufs[n]) for n in ("x", "gain", "q", "k", "gt", "up", "pos", "rn", "y", "qo", "ko", "s", "o")}
    g.node(cbx.GOP_RMS_NORM, ids["rn"], (ids["x"],), fparam=1e-5)
    g.node(cbx.GOP_MUL, ids["y"], (ids["rn"], ids["gain"]))
    g.node(cbx.GOP_ROPE, ids["qo"], (ids["q"], ids["pos"]), rope=cache)
    g.node(cbx.GOP_ROPE, ids["ko"], (ids["k"], ids["pos"]), rope=cache)
    g.node(cbx.GOP_UNARY, ids["s"], (ids["gt"],), iparam=cbx.SILU)
    g.node(cbx.GOP_MUL, ids["o"], (ids["s"], ids["up"]))
    return g, ids


def decode_bufs(seed, p):
    D, H, hd, F = 1024, 16, 64, 4096
    b = {"x": dev(W.normal(W.seed_of(seed, 0), (1, D))), "gain": dev(W.normal(W.seed_of(seed, 1), (D,), 1.0, 0.05)),
         "q": dev(W.normal(W.seed_of(seed, 2), (1, H, hd))), "k": dev(W.normal(W.seed_of(seed, 3), (1, H, hd))),
         "gt": dev(W.normal(W.seed_of(seed, 4), (1, F))), "up": dev(W.normal(W.seed_of(seed, 5), (1, F))),
         "pos": torch.full((1,), p, dtype=torch.int32, device="cuda")}
    for n, shape in (("rn", (1, D)), ("y", (1, D)), ("qo", (1, H, hd)), ("ko", (1, H, hd)), ("s", (1, F)),
                     ("o", (1, F))):
        b[n] = empty(*shape)
    return b


def test_update_to_other_buffers_in_place(cbx):
    """cbx_graph_exec_update: each step's decode list over its own buffer set
    and position (the same launches with other addresses and values) is taken
    by the instantiated graph in place; a replay queued before the update
    keeps its own arguments (replays and updates alternate with no
    synchronisation of the test's own before the end; every set is then
    checked against cbx_graph_compute)."""
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    sets = [decode_bufs(31 + i, p) for i, p in enumerate((3, 700, 2047, 2500))]
    outs = ("y", "qo", "ko", "o")
    exp = []
    for b in sets:
        g, _ = decode_list(cbx, cache, b)
        assert g.compute() == 3
        torch.cuda.synchronize()
        exp.append([bits(b[n]).clone() for n in outs])
        for n in outs:
            b[n].fill_(float("nan"))
    torch.cuda.synchronize()
    g, ids = decode_list(cbx, cache, sets[0])
    ex = g.capture()
    try:
        ex.launch()                                   # set 0, still queued
        for i in range(1, len(sets)):
            for n, t in ids.items():
                g.rebind(t, sets[i][n])
            assert ex.update() is True, f"set {i}: not updated in place"
            assert ex.n_launches == 3
            ex.launch()                               # no synchronisation in between
        torch.cuda.synchronize()
        for i, b in enumerate(sets):
            for n, e in zip(outs, exp[i]):
                assert torch.equal(bits(b[n]), e), f"set {i}: {n} differs from eager"
    finally:
        ex.close()
        cache.close()


def long_work_on(stream):
    """Enqueues ~0.05-1 s of bounded device work on `stream` (a spin kernel
    that ends after a fixed cycle count) and returns an event behind it."""
    done = torch.cuda.Event()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(120_000_000)
        done.record()
    return done


def test_update_leaves_other_streams_running(cbx):
    """An update waits for its own exec's replays only: work queued on
    another stream is still running when cbx_graph_exec_update returns (a
    device-wide wait would have waited for it), and the updated replay gives
    cbx_graph_compute's bits."""
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    sets = [decode_bufs(41 + i, p) for i, p in enumerate((5, 900, 17))]
    outs = ("y", "qo", "ko", "o")
    exp = []
    for b in sets:
        g, _ = decode_list(cbx, cache, b)
        assert g.compute() == 3
        torch.cuda.synchronize()
        exp.append([bits(b[n]).clone() for n in outs])
        for n in outs:
            b[n].fill_(float("nan"))
    torch.cuda.synchronize()
    g, ids = decode_list(cbx, cache, sets[0])
    ex = g.capture()
    other = torch.cuda.Stream()
    try:
        ex.launch()
        for i in (1, 2):
            done = long_work_on(other)
            for n, t in ids.items():
                g.rebind(t, sets[i][n])
            assert ex.update() is True
            running = not done.query()
            ex.launch()
            torch.cuda.synchronize()
            assert running, f"update {i} waited for another stream's work"
        for i, b in enumerate(sets):
            for n, e in zip(outs, exp[i]):
                assert torch.equal(bits(b[n]), e), f"set {i}: {n} differs from eager"
    finally:
        ex.close()
        cache.close()


def test_update_while_the_last_replay_runs(cbx):
    """A per-step loop: update, launch, update, launch ... with no
    synchronisation, each step over its own buffers and position, the
    replay before each update still queued behind long work on the same
    stream (the update must not change the arguments it was queued with):
    every step's outputs equal cbx_graph_compute's."""
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    sets = [decode_bufs(51 + i, p) for i, p in enumerate((0, 1, 2, 3, 2047, 2048, 9, 10))]
    outs = ("y", "qo", "ko", "o")
    exp = []
    for b in sets:
        g, _ = decode_list(cbx, cache, b)
        assert g.compute() == 3
        torch.cuda.synchronize()
        exp.append([bits(b[n]).clone() for n in outs])
        for n in outs:
            b[n].fill_(float("nan"))
    torch.cuda.synchronize()
    g, ids = decode_list(cbx, cache, sets[0])
    ex = g.capture()
    try:
        long_work_on(torch.cuda.current_stream())     # the replays queue behind it
        ex.launch()
        for i in range(1, len(sets)):
            for n, t in ids.items():
                g.rebind(t, sets[i][n])
            assert ex.update() is True
            ex.launch()
        torch.cuda.synchronize()
        for i, b in enumerate(sets):
            for n, e in zip(outs, exp[i]):
                assert torch.equal(bits(b[n]), e), f"step {i}: {n} differs from eager"
    finally:
        ex.close()
        cache.close()


def test_update_to_other_lengths(cbx):
    """LayerNorm -> view -> RoPE over views of T = 100, 37, 512 and 1 tokens of
    one buffer (a sequence whose length changes between steps, as the KV
    views of a decode loop do): every update is taken in place (new grids,
    and kernel variants where the row count picks another) and every replay
    after it matches cbx_graph_compute on the same views."""
    B, H, hd, Tmax = 1, 8, 64, 512
    xa = dev(W.normal(W.seed_of(33, 0), (B, Tmax, H * hd), 0.2, 1.0))
    w = dev(W.normal(W.seed_of(33, 1), (H * hd,), 1.0, 0.02))
    b = dev(W.normal(W.seed_of(33, 2), (H * hd,), 0.0, 0.02))
    posa = torch.arange(Tmax, dtype=torch.int32, device="cuda")
    bufs = [empty(B, Tmax, H * hd) for _ in range(3)]
    outa = empty(B, Tmax, H, hd)
    cache = cbx.RopeCache(hd, mode=2, n_ctx_orig=2048, n_pos=2048)

    def views(T):
        return ([xa[:, :T], w, b, posa[:T]] + [t[:, :T] for t in bufs] +
                [bufs[2][:, :T].view(B, T, H, hd), outa[:, :T]])

    g = cbx.Graph()
    tid = [g.tensor(v) for v in views(100)]
    tx, tw, tb, tp, n_, m_, y_, v_, r_ = tid
    g.node(cbx.GOP_NORM, n_, (tx,), fparam=1e-5)
    g.node(cbx.GOP_MUL, m_, (n_, tw))
    g.node(cbx.GOP_ADD, y_, (m_, tb))
    g.node(cbx.GOP_VIEW, v_, (y_,))
    g.node(cbx.GOP_ROPE, r_, (v_, tp), rope=cache)
    ex = g.capture()
    flags = []
    try:
        for T in (100, 37, 512, 1):
            for i, v in zip(tid, views(T)):
                g.rebind(i, v)
            outa.fill_(float("nan"))
            assert g.compute() == 1
            torch.cuda.synchronize()
            e = bits(outa).clone()
            outa.fill_(float("nan"))
            torch.cuda.synchronize()
            flags.append(ex.update())
            assert ex.n_launches == 1
            ex.launch()
            torch.cuda.synchronize()
            assert torch.equal(bits(outa), e), f"T = {T}: differs from eager"
            assert not torch.isnan(outa[:, :T]).any()
        assert flags == [True] * 4, f"in place per length: {flags}"
    finally:
        ex.close()
        cache.close()


def test_update_resblock_to_another_input(cbx):
    """The HiFT ResBlock layer's two conv launches re-pointed at another
    input buffer of the same shape (the next utterance's activations): the
    update goes in place and the replay matches cbx_graph_compute."""
    from tests._hift_graph import HiftGraph

    Ch, T, K, d = 128, 700, 11, 3
    sd = W.seed_of(14, K)
    h = HiftGraph(new)
    x0 = dev(W.normal(sd, (T, Ch), 0.0, 1.0))
    x1 = dev(W.normal(sd + 9, (T, Ch), 0.0, 1.0))
    tx = h.t(x0)
    p, wts = {}, []
    for k, s in enumerate(("1", "2")):
        a, ai = W.snake_alpha(Ch, 30 + k)
        w = W.normal(sd + 1 + k, (Ch, Ch, K), 0.0, 1.0 / np.sqrt(Ch * K))
        b = W.normal(sd + 3 + k, (Ch,), 0.0, 0.1)
        for name, v in (("a", a), ("ai", ai), ("w", w), ("b", b)):
            p[name + s] = h.t(dev(v))
        wts.append(cbx.Conv1dWeights(h.at(p["w" + s])))
    y = h.at(h.sublayer(tx, p, d, wts[0], wts[1]))
    ex = h.g.capture()
    try:
        h.g.rebind(tx, x1)
        y.fill_(float("nan"))
        assert h.g.compute() == 2
        torch.cuda.synchronize()
        e = bits(y).clone()
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        assert ex.update() is True
        ex.launch()
        torch.cuda.synchronize()
        assert torch.equal(bits(y), e)
    finally:
        ex.close()
        for w_ in wts:
            w_.close()


def test_update_to_another_list(cbx):
    """An update to a list with other launches (the decode step's four, then
    GroupNorm -> affine -> Mish's one) re-instantiates the graph; an update to
    a list with an unsupported node fails and leaves the exec as it was.
    The exec's two instantiations take turns, so going back to the decode
    list re-points the one that still holds it (in place), and a third list
    re-instantiates again."""
    cache = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    b0 = decode_bufs(41, 9)
    g, _ = decode_list(cbx, cache, b0)
    assert g.compute() == 3
    torch.cuda.synchronize()
    exp0 = [bits(b0[n]).clone() for n in ("y", "qo", "ko", "o")]
    inp = W.cfm_inputs()
    x = dev(inp["x256"])
    g2 = cbx.Graph()
    tx, tw, tb = g2.tensor(x), g2.tensor(dev(inp["w256"])), g2.tensor(dev(inp["b256"]))
    buf = [empty(*x.shape) for _ in range(6)]
    t = [g2.tensor(v) for v in buf]
    g2.node(cbx.GOP_GROUP_NORM, t[0], (tx,), iparam=8, fparam=1e-5)
    g2.node(cbx.GOP_MUL, t[1], (t[0], tw))
    g2.node(cbx.GOP_ADD, t[2], (t[1], tb))
    g2.node(cbx.GOP_UNARY, t[3], (t[2],), iparam=cbx.SOFTPLUS)
    g2.node(cbx.GOP_UNARY, t[4], (t[3],), iparam=cbx.TANH)
    g2.node(cbx.GOP_MUL, t[5], (t[2], t[4]))
    assert g2.compute() == 1
    torch.cuda.synchronize()
    exp2 = bits(buf[5]).clone()
    g3 = cbx.Graph()
    a3, b3, c3 = g3.tensor(dev(np.ones((4, 64), np.float32))), g3.tensor(dev(np.ones((4, 64), np.float32))), \
        g3.tensor(empty(4, 64))
    g3.node(cbx.GOP_ADD, c3, (a3, b3))
    g3.node(cbx.GOP_UNARY, g3.tensor(empty(4, 64)), (c3,), iparam=42)   # no such activation
    ex = g.capture()
    try:
        buf[5].fill_(float("nan"))
        torch.cuda.synchronize()
        assert ex.update(g2) is False
        assert ex.n_launches == 1
        ex.launch()
        torch.cuda.synchronize()
        assert torch.equal(bits(buf[5]), exp2)
        with pytest.raises(cbx.CbxError) as e:
            ex.update(g3)
        assert e.value.status == cbx.ERR_UNSUPPORTED
        buf[5].fill_(float("nan"))
        torch.cuda.synchronize()
        ex.launch()                                  # still the GroupNorm list
        torch.cuda.synchronize()
        assert torch.equal(bits(buf[5]), exp2)
        for n in ("y", "qo", "ko", "o"):
            b0[n].fill_(float("nan"))
        assert ex.update(g) is True                  # back to the decode list: the other instantiation
        assert ex.n_launches == 3
        ex.launch()
        torch.cuda.synchronize()
        for n, e0 in zip(("y", "qo", "ko", "o"), exp0):
            assert torch.equal(bits(b0[n]), e0), n
        buf[5].fill_(float("nan"))
        assert ex.update(g2) is True                 # and the GroupNorm list's is still there
        ex.launch()
        torch.cuda.synchronize()
        assert torch.equal(bits(buf[5]), exp2)
    finally:
        ex.close()
        cache.close()
