"""The C-ABI library without a GPU: it loads, exports every symbol the public
header declares, and reports errors without launching anything."""
import ctypes
import os

import pytest

from chatterbox_amdvulkan_amd import cbxops as C


def test_library_is_built_for_gfx950():
    assert os.path.exists(C.LIB_PATH), "run __graft_entry__.build() first"
    data = open(C.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_exports_every_header_symbol():
    lib = ctypes.CDLL(C.LIB_PATH)
    syms = C.header_symbols()
    assert len(syms) >= 20
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_descriptor_layout_matches_header():
    # struct cbx_tensor { void*; int32; int32; int64[4]; size_t[4]; }
    assert ctypes.sizeof(C.Tensor) == 8 + 4 + 4 + 32 + 32
    assert C.Tensor.ne.offset == 16 and C.Tensor.nb.offset == 48


def test_version_and_empty_error():
    L = C.load()
    assert L.cbx_version().decode().startswith("cbxops")
    assert isinstance(C.last_error(), str)


def test_ops_before_init_fail_cleanly():
    """No device (here) or no cbx_init: an error code and a message, never a crash."""
    L = C.load()
    t = C.Tensor()
    rc = L.cbx_norm(ctypes.byref(t), 1e-5, ctypes.byref(t), None)
    assert rc in (C.ERR_NOT_INITIALIZED, C.ERR_HIP)
    assert C.last_error()
    rc = L.cbx_unary(99, ctypes.byref(t), ctypes.byref(t), None)
    assert rc == C.ERR_INVALID_ARG
    assert "unknown op" in C.last_error()
    ops = (C.OpStruct * 1)()
    assert L.cbx_run_ops(ops, 1, None) in (C.ERR_NOT_INITIALIZED, C.ERR_HIP)
    assert C.last_error()


def test_op_struct_layout_matches_header():
    # struct cbx_op { int32 kind, act; float eps, param; cbx_tensor* src[6], dst[2]; void* rope;
    #                  int32 iparam, reserved; }
    assert C.OpStruct.src.offset == 16 and C.OpStruct.dst.offset == 64 and C.OpStruct.rope.offset == 80
    assert C.OpStruct.iparam.offset == 88 and ctypes.sizeof(C.OpStruct) == 96
    with pytest.raises(C.CbxError):
        C.OpBatch([C.Op(C.OP_UNARY)] * (C.MAX_OPS + 1))


def test_init_without_gpu_reports_hip_error():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = C.load()
    assert L.cbx_init(0) == C.ERR_HIP
    assert "device" in C.last_error()
    assert L.cbx_rope_cache_create(63, 2, 2048, 1e4, 1.0, 0.0, 1.0, 0.0, 0.0, None, 16,
                                   ctypes.byref(ctypes.c_void_p())) == C.ERR_INVALID_ARG


def test_descriptor_from_torch_cpu_tensor():
    import torch

    x = torch.zeros((3, 5, 7), dtype=torch.float16)
    d = C.desc(x)
    assert list(d.ne) == [7, 5, 3, 1]
    assert list(d.nb) == [2, 14, 70, 210]
    assert d.type == C.F16
    q = torch.zeros((4, 34 * 3), dtype=torch.uint8)
    dq = C.desc(q, C.Q8_0)
    assert list(dq.ne) == [96, 4, 1, 1] and list(dq.nb)[:2] == [34, 102]
    v = torch.zeros((6, 10))[:, 2:8]
    dv = C.desc(v)
    assert list(dv.ne)[:2] == [6, 6] and list(dv.nb)[:2] == [4, 40]


def test_descriptor_of_extent_one_dims():
    """Dimensions of extent 1 get contiguous strides whatever torch reports
    for them (0 after None-indexing or expand): they are never stepped over,
    and the library checks nb[0] against the element size."""
    import torch

    w = torch.eye(4)[:, :, None]              # torch strides (4, 1, 0)
    d = C.desc(w)
    assert list(d.ne) == [1, 4, 4, 1] and list(d.nb) == [4, 4, 16, 64]
    b = torch.zeros(5).expand(1, 5)          # stride 0 on the leading extent-1 dim
    db = C.desc(b)
    assert list(db.ne) == [5, 1, 1, 1] and list(db.nb) == [4, 20, 20, 20]


def test_graph_node_layout_matches_header():
    # struct cbx_gnode { int32 op, dst, src[2], iparam; float fparam; const void* rope;
    #                    int32 conv[3]; const void* conv_w; }
    assert C.GNode.rope.offset == 24 and C.GNode.conv.offset == 32 and C.GNode.conv_w.offset == 48
    assert ctypes.sizeof(C.GNode) == 56
