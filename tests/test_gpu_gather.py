"""Embedding gather (F32 / F16 / Q8_0 tables, fused position add) and f32/f16
casts through the C ABI, against the oracle: bit-exact."""
import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests._util import assert_bitexact

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_prefill_gather_pos(cbx, oracle, dtype):
    """T3 prefill embedding: 512 ids of an [8194,1024] table + position rows 0..511."""
    inp = W.prefill_inputs(f16_table=dtype == np.float16)
    exp = oracle.get_rows_add(inp["table"], inp["ids"], inp["pos_table"], inp["pos_ids"], nth=8)
    got = cbx.get_rows_add(dev(inp["table"]), dev(inp["ids"]), dev(inp["pos_table"]), dev(inp["pos_ids"]))
    assert_bitexact(host(got), exp, "get_rows_add")
    got1 = cbx.get_rows(dev(inp["table"]), dev(inp["ids"]))
    assert_bitexact(host(got1), oracle.get_rows(inp["table"], inp["ids"], nth=8), "get_rows")


def test_q8_0_gather_64_streams(cbx, oracle):
    """Q8_0 table [8194,1024] quantised with ggml's reference rule; 64 ids."""
    x = W.normal(W.seed_of(5, 0), (W.VOCAB, W.D_MODEL), 0.0, 0.02)
    q = oracle.quantize_q8_0(x)
    ids = W.randint(W.seed_of(5, 1), (64,), 0, W.VOCAB)
    exp = oracle.get_rows(q, ids, q8_0=True)
    got = cbx.get_rows(dev(q), dev(ids), q8_0=True)
    assert_bitexact(host(got), exp, "q8_0 gather")


def test_q8_0_special_scales(cbx, oracle):
    """Hand-built blocks: d in {1.0, 2^-10, smallest subnormal, -0.0, 65504}, qs -128..127."""
    scales = [0x3C00, 0x1400, 0x0001, 0x8000, 0x7BFF, 0x3555]
    rows = []
    for i, d in enumerate(scales):
        row = bytearray()
        for b in range(8):
            row += int(d).to_bytes(2, "little")
            qs = (np.arange(32) * 8 + b * 32 + i) % 256 - 128
            row += qs.astype(np.int8).tobytes()
        rows.append(np.frombuffer(bytes(row), dtype=np.uint8))
    q = np.stack(rows)
    ids = np.array([5, 0, 3, 1, 2, 4, 0], dtype=np.int32)
    exp = oracle.get_rows(q, ids, q8_0=True)
    got = cbx.get_rows(dev(q), dev(ids), q8_0=True)
    assert_bitexact(host(got), exp, "q8_0 special")


def test_q8_0_odd_address_and_added_q8_table(cbx, oracle):
    """A Q8_0 table at an odd byte address (read byte by byte) and a second
    Q8_0 table added in (16-bit quant loads): both as the oracle."""
    q = oracle.quantize_q8_0(W.normal(230, (40, 128), 0.0, 0.05))
    q2 = oracle.quantize_q8_0(W.normal(231, (40, 128), 0.0, 0.05))
    ids = W.randint(232, (33,), 0, 40)
    ids2 = W.randint(233, (33,), 0, 40)
    buf = torch.zeros(q.size + 1, dtype=torch.uint8, device="cuda")
    odd = buf[1:].view(q.shape)
    odd.copy_(dev(q))
    assert odd.data_ptr() % 2 == 1
    assert_bitexact(host(cbx.get_rows(odd, dev(ids), q8_0=True)), oracle.get_rows(q, ids, q8_0=True), "odd q8")
    got = cbx.get_rows_add(dev(q), dev(ids), dev(q2), dev(ids2), q8_0=True, q8_0_2=True)
    exp = oracle.add(oracle.get_rows(q, ids, q8_0=True), oracle.get_rows(q2, ids2, q8_0=True))
    assert_bitexact(host(got), exp, "q8 + q8")


def test_f16_table_all_codes(cbx, oracle):
    """All 65536 f16 codes as one table row each: widening is exact."""
    codes = np.arange(65536, dtype=np.uint16).view(np.float16).reshape(4096, 16)
    ids = np.arange(4096, dtype=np.int32)[::-1].copy()
    got = host(cbx.get_rows(dev(codes), dev(ids)))
    assert_bitexact(got, oracle.get_rows(codes, ids), "f16 codes")
    assert_bitexact(got, codes[ids].astype(np.float32), "numpy widening")


def test_gather_edges(cbx, oracle):
    """First/last row, repeats, ragged ne0 (scalar path), batched ids, empty ids."""
    tab = W.normal(11, (37, 10))
    ids = np.array([0, 36, 36, 0, 17], dtype=np.int32)
    assert_bitexact(host(cbx.get_rows(dev(tab), dev(ids))), oracle.get_rows(tab, ids), "ragged")
    tab3 = W.normal(12, (3, 9, 64))           # ggml ne (64, 9, 3)
    ids3 = W.randint(13, (3, 5), 0, 9)        # ggml ne (5, 3)
    assert_bitexact(host(cbx.get_rows(dev(tab3), dev(ids3))), oracle.get_rows(tab3, ids3), "batched")
    empty = cbx.get_rows(dev(tab), dev(np.zeros(0, dtype=np.int32)))
    assert tuple(empty.shape) == (0, 10)


def test_gather_out_of_range_sets_device_error(cbx):
    tab = W.normal(14, (8, 64))
    cbx.device_errors(clear=True)
    out = host(cbx.get_rows(dev(tab), dev(np.array([1, 8, -1, 2], dtype=np.int32))))
    assert cbx.device_errors(clear=True) & 1
    assert not out[1].any() and not out[2].any()
    assert np.array_equal(out[0], tab[1]) and np.array_equal(out[3], tab[2])
    assert cbx.device_errors(clear=True) == 0


@pytest.mark.parametrize("src_t,dst_t", [(np.float32, np.float16), (np.float16, np.float32),
                                         (np.float32, np.float32), (np.float16, np.float16)])
def test_cpy(cbx, oracle, src_t, dst_t):
    x = W.normal(15, (33, 1027), 0.0, 300.0).astype(src_t)    # spans f16 overflow and subnormals
    x.reshape(-1)[:8] = np.array([0.0, -0.0, 65504, 65520, 1e-8, -6e-8, 2.98e-8, 3e-8], dtype=src_t)
    out = torch.empty(x.shape, dtype=torch.from_numpy(np.zeros(1, dst_t)).dtype, device="cuda")
    got = host(cbx.cpy(dev(x), out))
    assert_bitexact(got, oracle.cpy(x, dst_t), "cpy")
    # a row-strided, unaligned source view goes through the row path
    xs = x[:, 3:1003]
    out2 = torch.empty(xs.shape, dtype=out.dtype, device="cuda")
    got2 = host(cbx.cpy(dev(x)[:, 3:1003], out2))
    assert_bitexact(got2, oracle.cpy(np.ascontiguousarray(xs), dst_t), "cpy strided")


@pytest.mark.parametrize("ne0", [256, 1024, 2560])
def test_q8_0_long_rows(cbx, oracle, ne0):
    """Q8_0 rows of 16-byte aligned length (ne0 % 256 == 0) over several
    workgroup passes (2560 = 2.5 x 1024 elements): alone, with a second
    Q8_0 table, with an f32 or f16 table added, first/last rows; bit-exact."""
    n_rows = 19
    q = oracle.quantize_q8_0(W.normal(240 + ne0, (n_rows, ne0), 0.0, 0.05))
    q2 = oracle.quantize_q8_0(W.normal(241 + ne0, (n_rows, ne0), 0.0, 0.05))
    f = W.normal(242 + ne0, (n_rows, ne0))
    h = W.normal(243 + ne0, (n_rows, ne0)).astype(np.float16)
    ids = np.concatenate([[0, n_rows - 1], W.randint(244, (21,), 0, n_rows)]).astype(np.int32)
    ids2 = W.randint(245, (ids.size,), 0, n_rows)
    gq = oracle.get_rows(q, ids, q8_0=True)
    assert_bitexact(host(cbx.get_rows(dev(q), dev(ids), q8_0=True)), gq, "q8 long rows")
    got = cbx.get_rows_add(dev(q), dev(ids), dev(q2), dev(ids2), q8_0=True, q8_0_2=True)
    assert_bitexact(host(got), oracle.add(gq, oracle.get_rows(q2, ids2, q8_0=True)), "q8 + q8")
    got = cbx.get_rows_add(dev(q), dev(ids), dev(f), dev(ids2), q8_0=True)
    assert_bitexact(host(got), oracle.add(gq, oracle.get_rows(f, ids2)), "q8 + f32")
    got = cbx.get_rows_add(dev(h), dev(ids2), dev(q), dev(ids), q8_0_2=True)
    assert_bitexact(host(got), oracle.add(oracle.get_rows(h, ids2), gq), "f16 + q8")


def test_q8_0_in_op_batch(cbx, oracle):
    """The one-launch gather with Q8_0 tables: ne0 = 2048 (two passes of the
    workgroup) and ne0 = 160 (a ragged pass), and an out-of-range id zeroing
    its row and raising the device error bit."""
    qa = oracle.quantize_q8_0(W.normal(250, (11, 2048), 0.0, 0.05))
    qb = oracle.quantize_q8_0(W.normal(251, (11, 160), 0.0, 0.05))
    ia = W.randint(252, (9,), 0, 11)
    ib = W.randint(253, (9,), 0, 11)
    ic = np.array([3, 11, 0], dtype=np.int32)
    ya = torch.empty((9, 2048), dtype=torch.float32, device="cuda")
    yb = torch.empty((9, 160), dtype=torch.float32, device="cuda")
    yc = torch.empty((3, 2048), dtype=torch.float32, device="cuda")
    ta, tb = dev(qa), dev(qb)
    cbx.device_errors(clear=True)
    cbx.run_ops([cbx.Op(cbx.OP_GET_ROWS, [ta, dev(ia)], [ya], q8=[0]),
                 cbx.Op(cbx.OP_GET_ROWS, [tb, dev(ib)], [yb], q8=[0]),
                 cbx.Op(cbx.OP_GET_ROWS, [ta, dev(ic)], [yc], q8=[0])])
    assert_bitexact(host(ya), oracle.get_rows(qa, ia, q8_0=True), "batch q8 2048")
    assert_bitexact(host(yb), oracle.get_rows(qb, ib, q8_0=True), "batch q8 160")
    out = host(yc)
    assert cbx.device_errors(clear=True) & 1
    assert not out[1].any()
    assert_bitexact(out[[0, 2]], oracle.get_rows(qa, ic[[0, 2]], q8_0=True), "batch q8 good rows")
