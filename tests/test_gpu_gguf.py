"""Tables uploaded from a GGUF file feed the gathers directly: the T3 input
embedding (Q8_0 token table + f32 position table + first LayerNorm) and an
f16 table, checked against the oracle on the same bytes."""
import ctypes

import numpy as np
import pytest
import torch

from chatterbox_amdvulkan_amd import workloads as W
from tests import gguf_file as G
from tests._util import assert_bitexact

pytestmark = pytest.mark.gpu


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_t3_embedding_from_gguf(cbx, oracle, tmp_path):
    D = 1024
    tok = W.quantize_q8_0(W.normal(W.seed_of(5, 0), (700, D), 0.0, 0.02))
    pos = W.normal(W.seed_of(2, 1), (600, D), 0.0, 0.02)
    sp = W.normal(210, (300, D), 0.0, 0.02).astype(np.float16)
    w = W.normal(W.seed_of(2, 3), (D,), 1.0, 0.02)
    b = W.normal(W.seed_of(2, 4), (D,), 0.0, 0.02)
    f = G.GgufFile()
    f.add_kv("general.architecture", G.STRING, "chatterbox")
    f.add_tensor("token_embd.text.weight", *G.table_q8_0(tok, D))
    f.add_tensor("token_embd.speech.weight", *G.table_f16(sp))
    f.add_tensor("position_embd.weight", *G.table_f32(pos))
    f.add_tensor("blk.0.attn_norm.weight", G.T_F32, [D], w.tobytes())
    f.add_tensor("blk.0.attn_norm.bias", G.T_F32, [D], b.tobytes())
    path = tmp_path / "t3.gguf"
    f.write(path)

    with cbx.Gguf(str(path)) as g:
        assert g.get_str("general.architecture") == "chatterbox"
        t = {name: g.upload(g.find(name)) for name in ("token_embd.text.weight", "token_embd.speech.weight",
                                                       "position_embd.weight", "blk.0.attn_norm.weight",
                                                       "blk.0.attn_norm.bias")}
        # the uploaded bytes are the file's
        assert np.array_equal(host(t["token_embd.text.weight"]), tok)
        assert_bitexact(host(t["position_embd.weight"]), pos, "f32 table")
        ids = W.randint(211, (333,), 0, 700)
        pids = np.arange(333, dtype=np.int32)
        di, dp = torch.from_numpy(ids).cuda(), torch.from_numpy(pids).cuda()
        d = {name: g.describe(g.find(name), v) for name, v in t.items()}
        h = torch.empty((333, D), dtype=torch.float32, device="cuda")
        y = torch.empty_like(h)
        L = cbx.load()
        rc = L.cbx_get_rows_add_layer_norm(ctypes.byref(d["token_embd.text.weight"]), ctypes.byref(cbx.desc(di)),
                                           ctypes.byref(d["position_embd.weight"]), ctypes.byref(cbx.desc(dp)),
                                           ctypes.byref(d["blk.0.attn_norm.weight"]),
                                           ctypes.byref(d["blk.0.attn_norm.bias"]), 1e-5, ctypes.byref(cbx.desc(h)),
                                           ctypes.byref(cbx.desc(y)), None)
        assert rc == cbx.OK, cbx.last_error()
        h_ref = oracle.get_rows_add(tok, ids, pos, pids, q8_0=True)
        assert_bitexact(host(h), h_ref, "h from gguf tables")
        assert_bitexact(host(y), oracle.layer_norm(h_ref, w, b, 1e-5), "LN(h) from gguf tables")
        # an f16 table straight from the file
        sid = W.randint(212, (77,), 0, 300)
        out = torch.empty((77, D), dtype=torch.float32, device="cuda")
        rc = L.cbx_get_rows(ctypes.byref(d["token_embd.speech.weight"]),
                            ctypes.byref(cbx.desc(torch.from_numpy(sid).cuda())), ctypes.byref(cbx.desc(out)), None)
        assert rc == cbx.OK, cbx.last_error()
        assert_bitexact(host(out), oracle.get_rows(sp, sid), "f16 gather from gguf")


def test_upload_rejects_small_destination(cbx, tmp_path):
    f = G.GgufFile()
    f.add_tensor("t", G.T_F32, [64], np.ones(64, np.float32).tobytes())
    path = tmp_path / "s.gguf"
    f.write(path)
    with cbx.Gguf(str(path)) as g:
        small = torch.empty(100, dtype=torch.uint8, device="cuda")
        rc = cbx.load().cbx_gguf_upload(g.handle, 0, ctypes.c_void_p(small.data_ptr()), 100, None)
        assert rc == cbx.ERR_INVALID_ARG and "smaller" in cbx.last_error()
