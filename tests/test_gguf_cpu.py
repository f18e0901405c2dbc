"""The GGUF reader (cbx_gguf_*) on the host: directory, keys, descriptors,
and rejection of malformed files.  No device is involved."""
import ctypes
import struct

import numpy as np
import pytest

from chatterbox_amdvulkan_amd import cbxops as C
from chatterbox_amdvulkan_amd import workloads as W
from tests import gguf_file as G


def _model(tmp_path, alignment=32, **kw):
    rng = np.random.default_rng(3)
    f = G.GgufFile(alignment=alignment)
    f.add_kv("general.architecture", G.STRING, "chatterbox")
    f.add_kv("general.name", G.STRING, "t3 test tables")
    f.add_kv("general.alignment", G.U32, alignment)
    f.add_kv("chatterbox.speech_vocab_size", G.U32, 6563)
    f.add_kv("chatterbox.layer_norm_eps", G.F32, 1e-5)
    f.add_kv("tokenizer.ggml.tokens", G.ARRAY, (G.STRING, ["a", "bb", "ccc"]))
    f.add_kv("tokenizer.ggml.scores", G.ARRAY, (G.F32, [0.5, 1.5, 2.5]))
    f.add_kv("some.flag", G.BOOL, True)
    f.add_kv("some.i64", G.I64, -7)
    q8 = W.quantize_q8_0(W.normal(200, (50, 64), 0.0, 0.02))
    f.add_tensor("token_embd.text.weight", *G.table_q8_0(q8, 64))
    f.add_tensor("position_embd.weight", *G.table_f32(rng.standard_normal((40, 64)).astype(np.float32)))
    f.add_tensor("token_embd.speech.weight", *G.table_f16(rng.standard_normal((30, 64)).astype(np.float16)))
    f.add_tensor("ln.bias", G.T_F32, [64], np.zeros(64, np.float32).tobytes())
    path = tmp_path / "m.gguf"
    f.write(path, **kw)
    return path, f


def test_directory_and_keys(tmp_path):
    path, f = _model(tmp_path)
    with C.Gguf(str(path)) as g:
        assert len(g) == 4
        assert g.get_str("general.architecture") == "chatterbox"
        assert g.get_str("general.name") == "t3 test tables"
        assert g.get_str("missing.key") is None
        i = g.find("token_embd.text.weight")
        assert i == 0 and g.find("nope") == -1
        inf = g.info(i)
        assert inf.name.decode() == "token_embd.text.weight" and inf.type == C.Q8_0 and inf.n_dims == 2
        assert list(inf.ne) == [64, 50, 1, 1] and inf.nbytes == 50 * 2 * 34
        raw = path.read_bytes()
        for k, (name, gtype, ne, data) in enumerate(f.tensors):
            inf = g.info(k)
            assert raw[inf.file_offset:inf.file_offset + inf.nbytes] == data, name
            assert inf.file_offset % 32 == 0


def test_descriptors(tmp_path):
    path, _ = _model(tmp_path)
    with C.Gguf(str(path)) as g:
        d = g.describe(g.find("token_embd.text.weight"), _FakePtr())
        assert d.type == C.Q8_0 and list(d.ne) == [64, 50, 1, 1] and list(d.nb) == [34, 68, 3400, 3400]
        d = g.describe(g.find("position_embd.weight"), _FakePtr())
        assert d.type == C.F32 and list(d.nb) == [4, 256, 10240, 10240]
        d = g.describe(g.find("token_embd.speech.weight"), _FakePtr())
        assert d.type == C.F16 and list(d.nb)[:2] == [2, 128]


class _FakePtr:
    """Stands in for a device tensor: describe only records the address."""

    def data_ptr(self):
        return 0x1000


def test_alignment_key_is_honoured(tmp_path):
    path, f = _model(tmp_path, alignment=64)
    with C.Gguf(str(path)) as g:
        raw = path.read_bytes()
        for k, (name, gtype, ne, data) in enumerate(f.tensors):
            inf = g.info(k)
            assert inf.file_offset % 64 == 0 and raw[inf.file_offset:inf.file_offset + inf.nbytes] == data


@pytest.mark.parametrize("case", ["magic", "version", "truncated", "past_end", "misaligned", "n_dims", "dup",
                                  "bad_type", "bad_value_type", "alignment"])
def test_rejects_malformed(tmp_path, case):
    path, f = _model(tmp_path)
    raw = bytearray(path.read_bytes())
    if case == "magic":
        raw[0:4] = b"GGML"
    elif case == "version":
        raw[4:8] = struct.pack("<I", 1)
    elif case == "truncated":
        raw = raw[: len(raw) // 3]
    elif case == "past_end":
        raw = raw[:-100]
    elif case == "misaligned":
        offs = [0, 3 * 32 + 1, 0, 0]
        raw = bytearray(f.bytes(offsets=offs))
    elif case == "n_dims":
        g = G.GgufFile()
        g.add_tensor("t", G.T_F32, [1, 1, 1, 1, 2], b"\0" * 8)
        raw = bytearray(g.bytes())
    elif case == "dup":
        g = G.GgufFile()
        g.add_tensor("t", G.T_F32, [2], b"\0" * 8)
        g.add_tensor("t", G.T_F32, [2], b"\0" * 8)
        raw = bytearray(g.bytes())
    elif case == "bad_type":
        g = G.GgufFile()
        g.add_tensor("t", 99, [32], b"\0" * 64)
        raw = bytearray(g.bytes())
    elif case == "bad_value_type":
        raw = bytearray(G.GGUF_MAGIC + struct.pack("<IQQ", 3, 0, 1) + G._str("k") + struct.pack("<I", 13))
    elif case == "alignment":
        g = G.GgufFile()
        g.add_kv("general.alignment", G.U32, 24)
        raw = bytearray(g.bytes())
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(bytes(raw))
    with pytest.raises(C.CbxError) as e:
        C.Gguf(str(bad))
    assert "cbx_gguf_open" in str(e.value)


def test_missing_file_and_bad_handles(tmp_path):
    with pytest.raises(C.CbxError):
        C.Gguf(str(tmp_path / "absent.gguf"))
    L = C.load()
    assert L.cbx_gguf_n_tensors(None) == -1
    assert L.cbx_gguf_find_tensor(None, b"x") == -1
    assert L.cbx_gguf_get_str(None, b"x") is None
    out = C.GgufTensorInfo()
    assert L.cbx_gguf_tensor(None, 0, ctypes.byref(out)) == C.ERR_INVALID_ARG
    path, _ = _model(tmp_path)
    with C.Gguf(str(path)) as g:
        assert L.cbx_gguf_tensor(g.handle, 9, ctypes.byref(out)) == C.ERR_INVALID_ARG
        assert L.cbx_gguf_upload(g.handle, 0, None, 0, None) == C.ERR_INVALID_ARG
        d = C.Tensor()
        assert L.cbx_gguf_describe(g.handle, 0, None, ctypes.byref(d)) == C.OK


def test_corrupted_files_never_crash(tmp_path):
    """Random byte flips and truncations of a valid file: each either opens
    with every tensor inside the file, or is rejected with an error."""
    path, _ = _model(tmp_path)
    good = path.read_bytes()
    rng = np.random.default_rng(11)
    head = 600                        # the header, keys and directory live in the first few hundred bytes
    bad = tmp_path / "fuzz.gguf"
    opened = 0
    for trial in range(300):
        raw = bytearray(good)
        if trial % 3 == 0:
            raw = raw[: int(rng.integers(0, len(raw)))]
        for _ in range(int(rng.integers(1, 4))):
            if raw:
                k = int(rng.integers(0, min(head, len(raw))))
                raw[k] = int(rng.integers(0, 256))
        bad.write_bytes(bytes(raw))
        try:
            g = C.Gguf(str(bad))
        except C.CbxError:
            continue
        opened += 1
        for i in range(len(g)):
            inf = g.info(i)
            assert inf.file_offset + inf.nbytes <= len(raw)
        g.close()
    assert opened < 300
