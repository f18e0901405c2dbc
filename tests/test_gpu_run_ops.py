"""cbx_run_ops: several independent ops in one launch must give exactly what
the single-op entry points give (and hence the oracle's results)."""
import ctypes

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
def rope64(cbx):
    c = cbx.RopeCache(64, mode=2, n_ctx_orig=2048, n_pos=2048)
    yield c
    c.close()


def test_decode_step_one_launch(cbx, oracle, rope64):
    """T3 decode step: RMSNorm+gamma, RoPE q, RoPE k, SiLU-gate in one launch."""
    x = W.normal(W.seed_of(1, 0), (1, 1024))
    g = W.normal(W.seed_of(1, 1), (1024,), 1.0, 0.02)
    q = W.normal(W.seed_of(1, 2), (1, 16, 64))
    k = W.normal(W.seed_of(1, 3), (1, 16, 64))
    pos = np.array([17], dtype=np.int32)
    gate = W.normal(W.seed_of(1, 5), (1, 4096))
    up = W.normal(W.seed_of(1, 6), (1, 4096))
    t = {n: dev(a) for n, a in dict(x=x, g=g, q=q, k=k, pos=pos, gate=gate, up=up).items()}
    y, qo, ko, h = (torch.empty_like(t["x"]), torch.empty_like(t["q"]), torch.empty_like(t["k"]),
                    torch.empty_like(t["gate"]))
    cbx.run_ops([
        cbx.Op(cbx.OP_RMS_NORM, [t["x"], t["g"]], [y], eps=1e-5),
        cbx.Op(cbx.OP_ROPE, [t["q"], t["pos"]], [qo], rope=rope64),
        cbx.Op(cbx.OP_ROPE, [t["k"], t["pos"]], [ko], rope=rope64),
        cbx.Op(cbx.OP_SWIGLU, [t["gate"], t["up"]], [h]),
    ])
    assert_bitexact(host(y), oracle.rms_norm_mul(x, g, 1e-5), "rms")
    assert_bitexact(host(qo), oracle.rope_ext(q, pos, 64), "rope q")
    assert_bitexact(host(ko), oracle.rope_ext(k, pos, 64), "rope k")
    assert_bitexact(host(h), host(cbx.swiglu(t["gate"], t["up"])), "swiglu = single op")
    assert_close(host(h), oracle.swiglu(gate, up), what="swiglu")


def test_serving_step_f16_and_q8(cbx, oracle, rope64):
    """64 streams, f16 storage: RMSNorm, RoPE q/k at per-stream positions,
    SiLU-gate, and a Q8_0 embedding gather, in one launch."""
    x = W.normal(W.seed_of(5, 2), (64, 1024)).astype(np.float16)
    g = W.normal(W.seed_of(5, 3), (1024,), 1.0, 0.02)
    q = W.normal(W.seed_of(5, 4), (64, 16, 64)).astype(np.float16)
    k = W.normal(W.seed_of(5, 6), (64, 16, 64)).astype(np.float16)
    pos = W.randint(W.seed_of(5, 5), (64,), 0, 2048)
    gate = W.normal(W.seed_of(5, 7), (64, 4096)).astype(np.float16)
    up = W.normal(W.seed_of(5, 8), (64, 4096)).astype(np.float16)
    tab = oracle.quantize_q8_0(W.normal(W.seed_of(5, 0), (W.VOCAB, 1024), 0.0, 0.02))
    ids = W.randint(W.seed_of(5, 1), (64,), 0, W.VOCAB)
    t = {n: dev(a) for n, a in dict(x=x, g=g, q=q, k=k, pos=pos, gate=gate, up=up, tab=tab, ids=ids).items()}
    y, qo, ko, h = (torch.empty_like(t["x"]), torch.empty_like(t["q"]), torch.empty_like(t["k"]),
                    torch.empty_like(t["gate"]))
    emb = torch.empty((64, 1024), dtype=torch.float32, device="cuda")
    cbx.run_ops([
        cbx.Op(cbx.OP_RMS_NORM, [t["x"], t["g"]], [y], eps=1e-5),
        cbx.Op(cbx.OP_ROPE, [t["q"], t["pos"]], [qo], rope=rope64),
        cbx.Op(cbx.OP_ROPE, [t["k"], t["pos"]], [ko], rope=rope64),
        cbx.Op(cbx.OP_SWIGLU, [t["gate"], t["up"]], [h]),
        cbx.Op(cbx.OP_GET_ROWS, [t["tab"], t["ids"]], [emb], q8=[0]),
    ])
    assert_bitexact(host(y), oracle.rms_norm_mul(x, g, 1e-5), "rms f16")
    assert_bitexact(host(qo), oracle.rope_ext(q, pos, 64), "rope q f16")
    assert_bitexact(host(ko), oracle.rope_ext(k, pos, 64), "rope k f16")
    assert_bitexact(host(h), host(cbx.swiglu(t["gate"], t["up"])), "swiglu f16 = single op")
    assert_bitexact(host(emb), oracle.get_rows(tab, ids, q8_0=True), "q8 gather")


def test_prefill_chain_one_launch(cbx, oracle):
    inp = W.prefill_inputs()
    t = {n: dev(inp[n]) for n in ("table", "ids", "pos_table", "pos_ids", "ln_w", "ln_b", "ffn")}
    h = torch.empty((512, 1024), dtype=torch.float32, device="cuda")
    y = torch.empty_like(h)
    g = torch.empty_like(t["ffn"])
    cbx.run_ops([
        cbx.Op(cbx.OP_GET_ROWS_ADD_LAYER_NORM, [t["table"], t["ids"], t["pos_table"], t["pos_ids"], t["ln_w"],
                                                t["ln_b"]], [h, y], eps=1e-5),
        cbx.Op(cbx.OP_UNARY, [t["ffn"]], [g], act=cbx.GELU),
    ])
    h_ref = oracle.get_rows_add(inp["table"], inp["ids"], inp["pos_table"], inp["pos_ids"], nth=8)
    assert_bitexact(host(h), h_ref, "h")
    assert_bitexact(host(y), oracle.layer_norm(h_ref, inp["ln_w"], inp["ln_b"], 1e-5, nth=8), "ln")
    assert_bitexact(host(g), oracle.unary(oracle.GELU, inp["ffn"], nth=8), "gelu")


@pytest.mark.parametrize("n", [2 * 1024 * 1024, 2 * 1024 * 1024 - 3, 1700001])
def test_large_launch_two_vectors_a_lane(cbx, oracle, n):
    """A launch of more workgroups than about 6 a CU gives its f32
    element-wise ops two vectors a lane: GELU and LeakyReLU over lengths
    with and without a tail (n % 4 != 0), next to a norm, match the
    single-op entry points bit for bit."""
    x = W.normal(140 + n % 7, (n,), 0.0, 3.0)
    xd = dev(x)
    g, lk = torch.empty_like(xd), torch.empty_like(xd)
    r = dev(W.normal(141, (64, 1024)))
    ry = torch.empty_like(r)
    cbx.run_ops([cbx.Op(cbx.OP_LAYER_NORM, [r], [ry], eps=1e-5),
                 cbx.Op(cbx.OP_UNARY, [xd], [g], act=cbx.GELU),
                 cbx.Op(cbx.OP_LEAKY_RELU, [xd], [lk], param=0.1)])
    assert_bitexact(host(g), oracle.unary(oracle.GELU, x, nth=8), "gelu")
    assert_bitexact(host(lk), oracle.leaky_relu(x, 0.1, nth=8), "leaky")
    assert_bitexact(host(ry), host(cbx.layer_norm(r, None, None, 1e-5)), "norm")


def test_vocoder_ops_and_tails(cbx, oracle):
    """Snake (both alpha layouts), LeakyReLU, LayerNorm+Mish, unary with a
    ragged length, gather + add -- together."""
    xs = W.normal(71, (300, 64))
    a = W.uniform_range(72, (64,), 0.5, 1.5)
    ai = (1.0 / (a + np.float32(1e-9))).astype(np.float32)
    xo = W.normal(73, (48, 1000))
    ao = W.uniform_range(74, (48, 1), 0.5, 1.5)
    aio = (1.0 / (ao + np.float32(1e-9))).astype(np.float32)
    xl = W.normal(75, (3, 1001))
    xn = W.normal(76, (40, 256))
    wn = W.normal(77, (256,), 1.0, 0.02)
    bn = W.normal(78, (256,), 0.0, 0.02)
    xu = W.normal(79, (1027,), 0.0, 3.0)
    tb = W.normal(80, (20, 32))
    tb2 = W.normal(81, (20, 32))
    ids = np.array([3, 19, 0], dtype=np.int32)
    ids2 = np.array([1, 2, 3], dtype=np.int32)
    T = {n: dev(v) for n, v in dict(xs=xs, a=a, ai=ai, xo=xo, ao=ao, aio=aio, xl=xl, xn=xn, wn=wn, bn=bn, xu=xu,
                                     tb=tb, tb2=tb2, ids=ids, ids2=ids2).items()}
    out = {n: torch.empty_like(T[s]) for n, s in (("s", "xs"), ("so", "xo"), ("l", "xl"), ("n", "xn"), ("u", "xu"))}
    out["g"] = torch.empty((3, 32), dtype=torch.float32, device="cuda")
    cbx.run_ops([
        cbx.Op(cbx.OP_SNAKE, [T["xs"], T["a"], T["ai"]], [out["s"]]),
        cbx.Op(cbx.OP_SNAKE, [T["xo"], T["ao"], T["aio"]], [out["so"]]),
        cbx.Op(cbx.OP_LEAKY_RELU, [T["xl"]], [out["l"]], param=0.1),
        cbx.Op(cbx.OP_LAYER_NORM, [T["xn"], T["wn"], T["bn"]], [out["n"]], eps=1e-5, act=cbx.MISH),
        cbx.Op(cbx.OP_UNARY, [T["xu"]], [out["u"]], act=cbx.SILU),
        cbx.Op(cbx.OP_GET_ROWS, [T["tb"], T["ids"], T["tb2"], T["ids2"]], [out["g"]]),
    ])
    assert_bitexact(host(out["s"]), host(cbx.snake(T["xs"], T["a"], T["ai"])), "snake inner = single op")
    assert_bitexact(host(out["so"]), host(cbx.snake(T["xo"], T["ao"], T["aio"])), "snake outer = single op")
    assert_close(host(out["s"]), oracle.snake(xs, a, ai), x=xs, what="snake")
    assert_bitexact(host(out["l"]), oracle.leaky_relu(xl, 0.1), "leaky")
    ln = oracle.layer_norm(xn, wn, bn, 1e-5)
    assert_bitexact(host(out["n"]), host(cbx.layer_norm(T["xn"], T["wn"], T["bn"], 1e-5, act=cbx.MISH)), "ln mish")
    assert_close(host(out["n"]), oracle.unary(oracle.MISH, ln), x=ln, what="ln mish")
    assert_bitexact(host(out["u"]), host(cbx.silu(T["xu"])), "silu = single op")
    assert_bitexact(host(out["g"]), oracle.get_rows_add(tb, ids, tb2, ids2), "gather add")


def test_rejects_dependent_or_bad_ops(cbx):
    x = dev(W.normal(82, (4, 256)))
    y = torch.empty_like(x)
    z = torch.empty_like(x)
    with pytest.raises(cbx.CbxError, match="writes memory"):
        cbx.run_ops([cbx.Op(cbx.OP_UNARY, [x], [y], act=cbx.SILU),
                     cbx.Op(cbx.OP_UNARY, [y], [z], act=cbx.SILU)])      # second reads what the first writes
    with pytest.raises(cbx.CbxError):
        cbx.run_ops([cbx.Op(cbx.OP_UNARY, [x], [y], act=42)])
    with pytest.raises(cbx.CbxError):
        cbx.run_ops([cbx.Op(99, [x], [y])])
    big = dev(W.normal(83, (2, 2048)))
    with pytest.raises(cbx.CbxError, match="1024"):
        cbx.run_ops([cbx.Op(cbx.OP_LAYER_NORM, [big], [torch.empty_like(big)], eps=1e-5)])
    # in place within one element-wise op is allowed
    x2 = dev(W.normal(84, (1000,)))
    ref = host(cbx.silu(x2))
    cbx.run_ops([cbx.Op(cbx.OP_UNARY, [x2], [x2], act=cbx.SILU)])
    assert_bitexact(host(x2), ref, "in place")


def test_gelu_all_codes_in_batch(cbx, oracle):
    """The batched GELU (f32 and f16) at every f16 code and the clamps."""
    codes = np.arange(65536, dtype=np.uint16).view(np.float16)
    x32 = codes.astype(np.float32)
    x32 = np.concatenate([x32[~np.isnan(x32)], np.array([-10.0, 10.0, np.nextafter(-10, 0), np.nextafter(10, 0)],
                                                        dtype=np.float32)])
    a, b = dev(x32), dev(codes)
    ya, yb = torch.empty_like(a), torch.empty_like(b)
    cbx.run_ops([cbx.Op(cbx.OP_UNARY, [a], [ya], act=cbx.GELU), cbx.Op(cbx.OP_UNARY, [b], [yb], act=cbx.GELU)])
    assert_bitexact(host(ya), oracle.unary(oracle.GELU, x32), "batched gelu f32")
    assert_bitexact(host(yb), oracle.unary(oracle.GELU, codes), "batched gelu f16")


@pytest.mark.parametrize("mode,n_dims", [(2, 64), (0, 64), (2, 32), (0, 32), (2, 20), (0, 20)])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_batched_rope_forms(cbx, oracle, mode, n_dims, dtype):
    """RoPE in the batch kernel, both pairings, full and partial rotation
    (n_dims % 8 != 0 takes the pair-a-lane form), positions inside and past
    the table (the device recurrence): the same bits as cbx_rope_ext, and the
    oracle's bits inside the table."""
    cache = cbx.RopeCache(n_dims, mode=mode, n_ctx_orig=2048, n_pos=48)
    x = W.normal(85 + n_dims + mode, (40, 12, 64)).astype(dtype)       # (n_tok, n_head, head_dim)
    pos = np.concatenate([np.arange(0, 40, 2), np.arange(44, 64)]).astype(np.int32)   # 20 past the table
    xd, pd = dev(x), dev(pos)
    y = torch.empty_like(xd)
    cbx.run_ops([cbx.Op(cbx.OP_ROPE, [xd, pd], [y], rope=cache)])
    single = host(cbx.rope_ext(xd, pd, cache))
    got = host(y)
    assert_bitexact(got, single, "batched rope = single op")
    inside = pos < 48
    exp = oracle.rope_ext(x, pos, n_dims, mode=mode)
    assert_bitexact(got[inside], exp[inside], "batched rope in the table")
    rtol = 1e-5 if dtype == np.float32 else RTOL_F16
    assert_close(got[~inside].astype(np.float32), exp[~inside].astype(np.float32), rtol=rtol, atol_x=2 ** -20,
                 x=x[~inside].astype(np.float32), what="batched rope past the table")
    cache.close()


@pytest.mark.parametrize("rows", [1, 64, 1500])
@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_batched_norm_row_forms(cbx, oracle, rows, dtype):
    """RMSNorm and LayerNorm of 1024-wide rows in the batch kernel: few rows
    (one row a workgroup over four waves) and many (four rows a workgroup):
    the same bits as the single-op entry points and the oracle."""
    x = W.normal(90 + rows, (rows, 1024)).astype(dtype)
    g = W.normal(91, (1024,), 1.0, 0.02)
    b = W.normal(92, (1024,), 0.0, 0.02)
    xd, gd, bd = dev(x), dev(g), dev(b)
    yr, yl = torch.empty_like(xd), torch.empty_like(xd)
    cbx.run_ops([cbx.Op(cbx.OP_RMS_NORM, [xd, gd], [yr], eps=1e-5),
                 cbx.Op(cbx.OP_LAYER_NORM, [xd, gd, bd], [yl], eps=1e-5)])
    assert_bitexact(host(yr), host(cbx.rms_norm_mul(xd, gd, 1e-5)), "batched rms = single op")
    assert_bitexact(host(yl), host(cbx.layer_norm(xd, gd, bd, 1e-5)), "batched ln = single op")
    if dtype == np.float32:
        assert_bitexact(host(yr), oracle.rms_norm_mul(x, g, 1e-5, nth=8), "batched rms")
        assert_bitexact(host(yl), oracle.layer_norm(x, g, b, 1e-5, nth=8), "batched ln")


@pytest.mark.parametrize("n,offset", [(4096 * 8, 0), (1003, 0), (4096, 4)])
def test_batched_f16_elementwise_forms(cbx, oracle, n, offset):
    """f16 element-wise ops in the batch over a long aligned run, a ragged
    length (the tail lane) and operands only 8-byte aligned (offset 4
    elements); each equals its single-op entry point and the oracle."""
    x = W.normal(90, (n + offset,), 0.0, 3.0).astype(np.float16)
    u = W.normal(91, (n + offset,), 0.0, 1.0).astype(np.float16)
    tx, tu = dev(x)[offset:], dev(u)[offset:]
    xs, us = x[offset:], u[offset:]
    ys = [torch.empty_like(tx) for _ in range(4)]
    cbx.run_ops([cbx.Op(cbx.OP_UNARY, [tx], [ys[0]], act=cbx.SILU),
                 cbx.Op(cbx.OP_LEAKY_RELU, [tx], [ys[1]], param=0.1),
                 cbx.Op(cbx.OP_SWIGLU, [tx, tu], [ys[2]]),
                 cbx.Op(cbx.OP_UNARY, [tu], [ys[3]], act=cbx.GELU)])
    assert_bitexact(host(ys[0]), host(cbx.silu(tx)), "silu = single op")
    assert_close(host(ys[0]), oracle.unary(oracle.SILU, xs), x=xs, what="silu f16", rtol=RTOL_F16)
    assert_bitexact(host(ys[1]), oracle.leaky_relu(xs, 0.1), "leaky f16")
    assert_bitexact(host(ys[2]), host(cbx.swiglu(tx, tu)), "swiglu = single op")
    assert_bitexact(host(ys[3]), oracle.unary(oracle.GELU, us), "gelu f16")


def cfm_flow_ops(cbx, rope64, order="gn_first", act=None):
    """The CFM flow step's three ops (GroupNorm(8)+affine+Mish on [2,256,500]
    and [2,512,500], LayerNorm+RoPE on [2,500,8x64]) as one op list."""
    act = cbx.MISH if act is None else act
    inp = W.cfm_inputs()
    t = {k: dev(v) for k, v in inp.items()}
    y256, y512, ya = (torch.full_like(t[k], float("nan")) for k in ("x256", "x512", "xa"))
    gn = [cbx.Op(cbx.OP_GROUP_NORM, [t["x256"], t["w256"], t["b256"]], [y256], act=act, eps=1e-5,
                 iparam=W.CFM_GROUPS),
          cbx.Op(cbx.OP_GROUP_NORM, [t["x512"], t["w512"], t["b512"]], [y512], act=act, eps=1e-5,
                 iparam=W.CFM_GROUPS)]
    lr = [cbx.Op(cbx.OP_LAYER_NORM_ROPE, [t["xa"], t["wa"], t["ba"], t["pos"]], [ya], eps=1e-5, rope=rope64,
                 iparam=W.HEAD_DIM)]
    ops = gn + lr if order == "gn_first" else lr + gn[::-1]
    return inp, t, (y256, y512, ya), ops


@pytest.mark.parametrize("order", ["gn_first", "ln_rope_first"])
@pytest.mark.parametrize("mish", [True, False])
def test_cfm_flow_step_one_launch(cbx, oracle, rope64, order, mish):
    """Both GroupNorms (split reduction) and LayerNorm+RoPE in one launch,
    listed in either order: the single-op entry points' bits (GroupNorm
    without Mish: the oracle's bits), LayerNorm+RoPE the oracle's bits."""
    act = cbx.MISH if mish else cbx.UNARY_NONE
    inp, t, (y256, y512, ya), ops = cfm_flow_ops(cbx, rope64, order, act)
    cbx.run_ops(ops)
    for x, w, b, y, C in ((t["x256"], t["w256"], t["b256"], y256, 256), (t["x512"], t["w512"], t["b512"], y512, 512)):
        ref = cbx.group_norm(x, W.CFM_GROUPS, 1e-5, w, b, act=act)
        assert_bitexact(host(y), host(ref), f"group norm {C} = cbx_group_norm")
        if not mish:
            exp = oracle.group_norm_affine(inp[f"x{C}"], W.CFM_GROUPS, 1e-5, inp[f"w{C}"], inp[f"b{C}"], False, nth=8)
            assert_bitexact(host(y), exp, f"group norm {C} vs oracle")
    ln = oracle.layer_norm(inp["xa"], inp["wa"], inp["ba"], 1e-5, nth=8)
    exp = oracle.rope_ext(ln.reshape(2, W.CFM_T, W.CFM_HEADS, W.HEAD_DIM), inp["pos"], W.HEAD_DIM, mode=2,
                          nth=8).reshape(inp["xa"].shape)
    assert_bitexact(host(ya), exp, "layer norm + rope vs oracle")
    f = ctypes.c_uint32(0)
    assert cbx.load().cbx_device_errors(0, ctypes.byref(f), 1) == cbx.OK and f.value == 0


def test_flow_step_repeated_and_with_other_ops(cbx, oracle, rope64):
    """The same list launched 20 times back to back (the exchange words of
    each launch carry its own tag) and once more beside a GELU op (the
    all-kinds kernel): same bits every time."""
    inp, t, outs, ops = cfm_flow_ops(cbx, rope64)
    batch = cbx.OpBatch(ops)
    batch.launch()
    ref = [host(o).copy() for o in outs]
    for o in outs:
        o.fill_(float("nan"))
    for _ in range(20):
        batch.launch()
    for o, r in zip(outs, ref):
        assert_bitexact(host(o), r, "after 20 launches")
    g = dev(W.normal(99, (4096,)))
    gy = torch.empty_like(g)
    for o in outs:
        o.fill_(float("nan"))
    cbx.run_ops(ops + [cbx.Op(cbx.OP_UNARY, [g], [gy], act=cbx.GELU)])
    for o, r in zip(outs, ref):
        assert_bitexact(host(o), r, "beside a GELU op")
    assert_bitexact(host(gy), host(cbx.gelu(g)), "gelu in the same launch")


def test_flow_ops_refused_layouts(cbx, rope64):
    """In-place GroupNorm (the split is out of place only), a GroupNorm of
    many small groups (no split), a head size whose partners span waves, and
    a non-zero reserved field are refused before anything launches."""
    x = dev(W.normal(5, (2, 256, 1, 500)))
    with pytest.raises(cbx.CbxError, match="in place"):
        cbx.run_ops([cbx.Op(cbx.OP_GROUP_NORM, [x], [x], eps=1e-5, iparam=8)])
    small = dev(W.normal(6, (64, 32, 1, 8)))
    with pytest.raises(cbx.CbxError, match="split"):
        cbx.run_ops([cbx.Op(cbx.OP_GROUP_NORM, [small], [torch.empty_like(small)], eps=1e-5, iparam=8)])
    xa = dev(W.normal(7, (2, 10, 320)))
    pos = dev(np.arange(10, dtype=np.int32))
    c40 = cbx.RopeCache(40, mode=2, n_pos=64)
    with pytest.raises(cbx.CbxError, match="partners"):
        cbx.run_ops([cbx.Op(cbx.OP_LAYER_NORM_ROPE, [xa, None, None, pos], [torch.empty_like(xa)], eps=1e-5,
                            rope=c40, iparam=40)])
    c40.close()
    op = cbx.Op(cbx.OP_LAYER_NORM_ROPE, [xa, None, None, pos], [torch.empty_like(xa)], eps=1e-5, rope=rope64,
                iparam=64)
    b = cbx.OpBatch([op])
    b.arr[0].reserved = 1
    with pytest.raises(cbx.CbxError, match="reserved"):
        b.launch()
