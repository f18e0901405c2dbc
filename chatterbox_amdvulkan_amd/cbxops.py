"""Python front end of libcbxops (the gfx950 fused layer-op library).

Functions carry the names of the ggml ops they replace on chatterbox-cpp's
layer-op path and take torch tensors that live on a ROCm device; every call
goes through the library's C ABI (include/cbxops.h) on torch's current
stream.  Shapes are torch order (outermost first); the descriptor passed to
the library reverses them into ggml's ne[] (innermost first), with byte
strides as nb[].

There is no fallback: if libcbxops.so is missing or a call fails, a
CbxError is raised.
"""
from __future__ import annotations

import ctypes
import os
import re
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcbxops.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "cbxops.h")

# ggml_type numbering
F32, F16, Q8_0, I32 = 0, 1, 8, 26
QK8_0, Q8_0_BLOCK = 32, 34

# cbx_unary_op
UNARY_NONE, GELU, GELU_ERF, SILU, TANH, SOFTPLUS, SIN, SQR, MISH = -1, 0, 1, 2, 3, 4, 5, 6, 7

# cbx_status
OK, ERR_INVALID_ARG, ERR_UNSUPPORTED, ERR_NOT_INITIALIZED, ERR_HIP = 0, -1, -2, -3, -4


class CbxError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"cbxops error {status}: {message}")
        self.status = status


class Tensor(ctypes.Structure):
    """cbx_tensor"""

    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


class OpStruct(ctypes.Structure):
    """cbx_op"""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("act", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("param", ctypes.c_float),
        ("src", ctypes.POINTER(Tensor) * 6),
        ("dst", ctypes.POINTER(Tensor) * 2),
        ("rope", ctypes.c_void_p),
        ("iparam", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class GgufTensorInfo(ctypes.Structure):
    """cbx_gguf_tensor_info"""

    _fields_ = [
        ("name", ctypes.c_char_p),
        ("type", ctypes.c_int32),
        ("n_dims", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nbytes", ctypes.c_size_t),
        ("file_offset", ctypes.c_size_t),
    ]


class GNode(ctypes.Structure):
    """cbx_gnode"""

    _fields_ = [
        ("op", ctypes.c_int32),
        ("dst", ctypes.c_int32),
        ("src", ctypes.c_int32 * 2),
        ("iparam", ctypes.c_int32),
        ("fparam", ctypes.c_float),
        ("rope", ctypes.c_void_p),
        ("conv", ctypes.c_int32 * 3),
        ("conv_w", ctypes.c_void_p),
    ]


class GLaunch(ctypes.Structure):
    """cbx_glaunch"""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("first_node", ctypes.c_int32),
        ("n_nodes", ctypes.c_int32),
        ("flags", ctypes.c_int32),
    ]


# cbx_gop
GOP_VIEW, GOP_GET_ROWS, GOP_ADD, GOP_MUL, GOP_SCALE, GOP_NORM, GOP_RMS_NORM, GOP_GROUP_NORM, GOP_ROPE, \
    GOP_SOFT_MAX, GOP_DIAG_MASK_INF, GOP_UNARY, GOP_LEAKY_RELU, GOP_CPY, GOP_IM2COL, GOP_MUL_MAT, \
    GOP_CONV_TRANSPOSE_1D, GOP_CONCAT = range(18)
# cbx_glaunch_kind
GL_UNSUPPORTED, GL_VIEW, GL_GET_ROWS, GL_GET_ROWS_ADD, GL_GET_ROWS_ADD_LAYER_NORM, GL_NORM, GL_LAYER_NORM, \
    GL_LAYER_NORM_ROPE, GL_RMS_NORM, GL_GROUP_NORM, GL_SOFT_MAX, GL_SNAKE, GL_UNARY, GL_SWIGLU, GL_LEAKY_RELU, \
    GL_ROPE, GL_CPY, GL_ADD_LAYER_NORM, GL_LAYER_NORM_MASK, GL_BIAS_ACT, GL_CONV1D, GL_CONV_TRANSPOSE1D, \
    GL_CAUSAL_CONV1D, GL_GET_ROWS_CONCAT_ADD_LAYER_NORM, GL_BINARY, GL_CONCAT, \
    GL_BIAS_RESIDUAL, GL_SCALE, GL_BIAS_ADD_PAIR, GL_BIAS_ADD_TWO, GL_ROPE_TWO = range(31)
# conv launch flags: the prologue (bits 0-1), a bias add, the residual add
GLF_SNAKE, GLF_LEAKY, GLF_MASK, GLF_BIAS, GLF_RESIDUAL, GLF_SUM, GLF_SCALE = 1, 2, 3, 4, 8, 16, 32

# cbx_op_kind
OP_LAYER_NORM, OP_RMS_NORM, OP_UNARY, OP_LEAKY_RELU, OP_SWIGLU, OP_ROPE, OP_GET_ROWS, \
    OP_GET_ROWS_ADD_LAYER_NORM, OP_SNAKE, OP_GROUP_NORM, OP_LAYER_NORM_ROPE = range(1, 12)
MAX_OPS = 12

_lib = None
_initialised: set[int] = set()


def header_symbols() -> list[str]:
    """Every function the public header declares."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cbx_[a-z0-9_]+)\s*\(", text)))


def load() -> ctypes.CDLL:
    """Loads libcbxops.so (no GPU needed) and declares its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise CbxError(ERR_UNSUPPORTED, f"{LIB_PATH} is not built; run python -m chatterbox_amdvulkan_amd.build")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER(Tensor)
    i, f, vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
    sigs = {
        "cbx_init": (i, [i]),
        "cbx_shutdown": (None, []),
        "cbx_last_error": (ctypes.c_char_p, []),
        "cbx_version": (ctypes.c_char_p, []),
        "cbx_device_errors": (i, [i, ctypes.POINTER(ctypes.c_uint32), i]),
        "cbx_get_rows": (i, [P, P, P, vp]),
        "cbx_get_rows_add": (i, [P, P, P, P, P, vp]),
        "cbx_get_rows_add_layer_norm": (i, [P, P, P, P, P, P, f, P, P, vp]),
        "cbx_get_rows_concat_add_layer_norm": (i, [P, P, P, P, P, P, P, P, P, f, P, P, vp]),
        "cbx_cpy": (i, [P, P, vp]),
        "cbx_norm": (i, [P, f, P, vp]),
        "cbx_layer_norm": (i, [P, P, P, f, i, P, vp]),
        "cbx_rms_norm": (i, [P, f, P, vp]),
        "cbx_rms_norm_mul": (i, [P, P, f, P, vp]),
        "cbx_group_norm": (i, [P, i, f, P, P, i, P, vp]),
        "cbx_group_norm_workspace_create": (i, [ctypes.POINTER(vp)]),
        "cbx_group_norm_workspace_destroy": (None, [vp]),
        "cbx_group_norm_workspace_tune": (i, [vp, ctypes.c_uint32, ctypes.c_int32]),
        "cbx_group_norm_ws": (i, [P, i, f, P, P, i, P, vp, vp]),
        "cbx_group_norm_noalloc": (i, [P, i, f, P, P, i, P, vp]),
        "cbx_group_norm_split_enabled": (i, [i]),
        "cbx_rope_cache_create": (i, [i, i, i, f, f, f, f, f, f, vp, ctypes.c_int32, ctypes.POINTER(vp)]),
        "cbx_rope_cache_destroy": (None, [vp]),
        "cbx_rope_ext": (i, [P, P, vp, P, vp]),
        "cbx_layer_norm_rope": (i, [P, P, P, f, ctypes.c_int64, P, vp, P, vp]),
        "cbx_scale_diag_mask_soft_max": (i, [P, f, ctypes.c_int32, P, vp]),
        "cbx_add_scale_diag_mask_soft_max": (i, [P, P, f, ctypes.c_int32, P, vp]),
        "cbx_unary": (i, [i, P, P, vp]),
        "cbx_gelu": (i, [P, P, vp]),
        "cbx_gelu_erf": (i, [P, P, vp]),
        "cbx_silu": (i, [P, P, vp]),
        "cbx_mish": (i, [P, P, vp]),
        "cbx_leaky_relu": (i, [P, f, P, vp]),
        "cbx_swiglu": (i, [P, P, P, vp]),
        "cbx_snake": (i, [P, P, P, P, vp]),
        "cbx_add_layer_norm": (i, [P, P, P, P, P, f, i, P, P, vp]),
        "cbx_layer_norm_mask": (i, [P, P, P, f, i, P, P, vp]),
        "cbx_bias_act": (i, [i, P, P, P, vp]),
        "cbx_binary": (i, [i, P, P, P, vp]),
        "cbx_concat": (i, [P, P, i, P, vp]),
        "cbx_bias_residual": (i, [P, P, P, P, vp]),
        "cbx_bias_add_pair": (i, [P, P, P, P, P, P, vp]),
        "cbx_bias_add_two": (i, [P, P, P, P, P, P, vp]),
        "cbx_scale": (i, [P, f, P, vp]),
        "cbx_conv1d_weights_create": (i, [P, vp, ctypes.POINTER(vp)]),
        "cbx_conv1d_weights_destroy": (None, [vp]),
        "cbx_conv1d": (i, [P, vp, i, i, i, i, P, P, f, P, P, P, vp]),
        "cbx_conv1d_sum": (i, [P, vp, i, i, i, i, P, P, f, P, P, P, f, P, vp]),
        "cbx_conv_transpose1d_weights_create": (i, [P, i, vp, ctypes.POINTER(vp)]),
        "cbx_conv_transpose1d": (i, [P, vp, i, i, P, P, f, P, P, vp]),
        "cbx_causal_conv1d": (i, [P, vp, P, P, P, vp]),
        "cbx_run_ops": (i, [ctypes.POINTER(OpStruct), i, vp]),
        "cbx_gguf_open": (i, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "cbx_gguf_close": (None, [vp]),
        "cbx_gguf_n_tensors": (ctypes.c_int64, [vp]),
        "cbx_gguf_find_tensor": (ctypes.c_int64, [vp, ctypes.c_char_p]),
        "cbx_gguf_get_str": (ctypes.c_char_p, [vp, ctypes.c_char_p]),
        "cbx_gguf_tensor": (i, [vp, ctypes.c_int64, ctypes.POINTER(GgufTensorInfo)]),
        "cbx_gguf_describe": (i, [vp, ctypes.c_int64, vp, P]),
        "cbx_gguf_upload": (i, [vp, ctypes.c_int64, vp, ctypes.c_size_t, vp]),
        "cbx_graph_plan": (i, [P, ctypes.c_int32, ctypes.POINTER(GNode), ctypes.c_int32,
                               ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, ctypes.POINTER(GLaunch),
                               ctypes.c_int32, ctypes.POINTER(ctypes.c_int32)]),
        "cbx_graph_launch": (i, [P, ctypes.c_int32, ctypes.POINTER(GNode), ctypes.c_int32,
                                 ctypes.POINTER(GLaunch), vp]),
        "cbx_graph_compute": (i, [P, ctypes.c_int32, ctypes.POINTER(GNode), ctypes.c_int32,
                                  ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, vp,
                                  ctypes.POINTER(ctypes.c_int32)]),
        "cbx_graph_exec_create": (i, [P, ctypes.c_int32, ctypes.POINTER(GNode), ctypes.c_int32,
                                      ctypes.POINTER(ctypes.c_int32), ctypes.c_int32, ctypes.POINTER(vp),
                                      ctypes.POINTER(ctypes.c_int32)]),
        "cbx_graph_exec_launch": (i, [vp, vp]),
        "cbx_graph_exec_update": (i, [vp, P, ctypes.c_int32, ctypes.POINTER(GNode), ctypes.c_int32,
                                      ctypes.POINTER(ctypes.c_int32), ctypes.c_int32,
                                      ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]),
        "cbx_graph_exec_destroy": (None, [vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def last_error() -> str:
    # messages can quote names read from files: never fail on their bytes
    return (load().cbx_last_error() or b"").decode("utf-8", errors="replace")


def _check(rc: int):
    if rc != OK:
        raise CbxError(rc, last_error())


def init(device: Optional[int] = None) -> None:
    """cbx_init for `device` (default: torch's current device); idempotent."""
    dev = torch.cuda.current_device() if device is None else int(device)
    if dev in _initialised:
        return
    _check(load().cbx_init(dev))
    _initialised.add(dev)


def device_errors(device: Optional[int] = None, clear: bool = True) -> int:
    dev = torch.cuda.current_device() if device is None else int(device)
    out = ctypes.c_uint32(0)
    _check(load().cbx_device_errors(dev, ctypes.byref(out), 1 if clear else 0))
    return out.value


def _ready(t: torch.Tensor):
    if not t.is_cuda:
        raise CbxError(ERR_INVALID_ARG, "tensor is not on a ROCm device")
    init(t.device.index)


_DTYPES = {torch.float32: F32, torch.float16: F16, torch.int32: I32}


def desc(t: torch.Tensor, ggml_type: Optional[int] = None) -> Tensor:
    """cbx_tensor for a torch tensor (up to 4 dims, any strides)."""
    if t.dim() > 4:
        raise CbxError(ERR_INVALID_ARG, "more than 4 dims")
    d = Tensor()
    d.data = t.data_ptr()
    es = t.element_size()
    shape = list(t.shape[::-1]) or [1]
    if t.numel() == 0:
        t = t.contiguous()
    strides = [s * es for s in t.stride()[::-1]] or [es]
    # a dimension of extent 1 is never stepped over: give it the stride a
    # contiguous tensor would have (torch leaves 0 there after indexing with
    # None or expand), as ggml does for its trivial dimensions
    for k in range(len(shape)):
        if shape[k] == 1:
            strides[k] = es if k == 0 else strides[k - 1] * shape[k - 1]
    row_bytes = strides[-1] * shape[-1]
    if ggml_type == Q8_0:
        if t.dtype != torch.uint8 or t.shape[-1] % Q8_0_BLOCK or t.stride(-1) != 1:
            raise CbxError(ERR_INVALID_ARG, "Q8_0 tables are uint8 [..., n_blocks * 34] with unit inner stride")
        shape[0] = shape[0] // Q8_0_BLOCK * QK8_0
        strides[0] = Q8_0_BLOCK
        d.type = Q8_0
    else:
        if t.dtype not in _DTYPES:
            raise CbxError(ERR_INVALID_ARG, f"unsupported dtype {t.dtype}")
        d.type = _DTYPES[t.dtype] if ggml_type is None else ggml_type
    while len(shape) < 4:
        shape.append(1)
        strides.append(row_bytes)
    for k in range(4):
        d.ne[k] = shape[k]
        d.nb[k] = strides[k]
    return d


def _ref(d: Optional[Tensor]):
    return ctypes.byref(d) if d is not None else None


def _stream() -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


# ---- gather / conversion ----------------------------------------------------

def get_rows(table: torch.Tensor, ids: torch.Tensor, out: Optional[torch.Tensor] = None,
             q8_0: bool = False) -> torch.Tensor:
    """ggml_get_rows + ggml_cast(F32).  table [.., n_rows, ne0] (f32/f16, or
    uint8 Q8_0 blocks with q8_0=True); ids int32; out f32 ids.shape + (ne0,)."""
    _ready(table)
    ne0 = table.shape[-1] // Q8_0_BLOCK * QK8_0 if q8_0 else table.shape[-1]
    if out is None:
        out = torch.empty(tuple(ids.shape) + (ne0,), dtype=torch.float32, device=table.device)
    _check(load().cbx_get_rows(_ref(desc(table, Q8_0 if q8_0 else None)), _ref(desc(ids)), _ref(desc(out)),
                               _stream()))
    return out


def get_rows_add(table, ids, table2, ids2, out=None, q8_0=False, q8_0_2=False):
    """ggml_add(get_rows(table, ids), get_rows(table2, ids2)) in one pass."""
    _ready(table)
    ne0 = table.shape[-1] // Q8_0_BLOCK * QK8_0 if q8_0 else table.shape[-1]
    if out is None:
        out = torch.empty(tuple(ids.shape) + (ne0,), dtype=torch.float32, device=table.device)
    _check(load().cbx_get_rows_add(_ref(desc(table, Q8_0 if q8_0 else None)), _ref(desc(ids)),
                                   _ref(desc(table2, Q8_0 if q8_0_2 else None)), _ref(desc(ids2)),
                                   _ref(desc(out)), _stream()))
    return out


def get_rows_concat_add_layer_norm(prefix, table_a, ids_a, table_b, ids_b, table2, ids2, w, b, eps, h=None,
                                   out=None, store_h=True, q8=()):
    """The T3 input with the conditioning prefix (t3.cpp:432-466): rows of
    concat(prefix, get_rows(table_a, ids_a), get_rows(table_b, ids_b)) plus
    get_rows(table2, ids2), then LayerNorm; returns (h, y).  prefix and
    table_a/ids_a may be None; q8 names the tables ("a", "b", "2") stored as Q8_0."""
    _ready(table_b)
    ne0 = table_b.shape[-1] // Q8_0_BLOCK * QK8_0 if "b" in q8 else table_b.shape[-1]
    n = (prefix.shape[0] if prefix is not None else 0) + (ids_a.numel() if ids_a is not None else 0) + ids_b.numel()
    if out is None:
        out = torch.empty((n, ne0), dtype=torch.float32, device=table_b.device)
    if h is None and store_h:
        h = torch.empty((n, ne0), dtype=torch.float32, device=table_b.device)
    opt = lambda t, k=None: _ref(desc(t, Q8_0 if k in q8 else None)) if t is not None else None  # noqa: E731
    _check(load().cbx_get_rows_concat_add_layer_norm(
        opt(prefix), opt(table_a, "a"), opt(ids_a), opt(table_b, "b"), opt(ids_b), opt(table2, "2"), opt(ids2),
        opt(w), opt(b), eps, opt(h), _ref(desc(out)), _stream()))
    return h, out


def get_rows_add_layer_norm(table, ids, table2, ids2, w, b, eps, h=None, out=None, q8_0=False, q8_0_2=False,
                            store_h=True):
    """T3 embedding + first LayerNorm in one pass; returns (h, y) (h None when
    store_h is False and no h buffer is given)."""
    _ready(table)
    ne0 = table.shape[-1] // Q8_0_BLOCK * QK8_0 if q8_0 else table.shape[-1]
    shape = tuple(ids.shape) + (ne0,)
    if out is None:
        out = torch.empty(shape, dtype=torch.float32, device=table.device)
    if h is None and store_h:
        h = torch.empty(shape, dtype=torch.float32, device=table.device)
    _check(load().cbx_get_rows_add_layer_norm(
        _ref(desc(table, Q8_0 if q8_0 else None)), _ref(desc(ids)), _ref(desc(table2, Q8_0 if q8_0_2 else None)),
        _ref(desc(ids2)), _ref(desc(w)) if w is not None else None, _ref(desc(b)) if b is not None else None, eps,
        _ref(desc(h)) if h is not None else None, _ref(desc(out)), _stream()))
    return h, out


def cpy(src: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """ggml_cpy / ggml_cast between f32 and f16."""
    _ready(src)
    _check(load().cbx_cpy(_ref(desc(src)), _ref(desc(out)), _stream()))
    return out


# ---- norms --------------------------------------------------------------------

def _out_like(x, out):
    return torch.empty_like(x) if out is None else out


def norm(x, eps, out=None):
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_norm(_ref(desc(x)), eps, _ref(desc(out)), _stream()))
    return out


def layer_norm(x, w, b, eps, act=UNARY_NONE, out=None):
    """layer_norm() helper: add(mul(norm(x), w), b) [-> act] in one pass."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_layer_norm(_ref(desc(x)), _ref(desc(w)) if w is not None else None,
                                 _ref(desc(b)) if b is not None else None, eps, act, _ref(desc(out)), _stream()))
    return out


def rms_norm(x, eps, out=None):
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_rms_norm(_ref(desc(x)), eps, _ref(desc(out)), _stream()))
    return out


def rms_norm_mul(x, g, eps, out=None):
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_rms_norm_mul(_ref(desc(x)), _ref(desc(g)) if g is not None else None, eps,
                                   _ref(desc(out)), _stream()))
    return out


def group_norm(x, n_groups, eps, w=None, b=None, act=UNARY_NONE, out=None):
    """ggml_group_norm (channels = ggml ne[2], i.e. torch dim -3) [+ affine] [+ act]."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_group_norm(_ref(desc(x)), n_groups, eps, _ref(desc(w)) if w is not None else None,
                                 _ref(desc(b)) if b is not None else None, act, _ref(desc(out)), _stream()))
    return out


GN_WAIT_AUTO = 0xFFFFFFFF   # CBX_GN_WAIT_AUTO


def group_norm_split_enabled(device: Optional[int] = None) -> bool:
    """cbx_group_norm_split_enabled: whether cbx_init's probe let the split
    reduction run on the device."""
    dev = torch.cuda.current_device() if device is None else int(device)
    init(dev)
    r = load().cbx_group_norm_split_enabled(dev)
    _check(min(r, 0))
    return r == 1


class GroupNormWorkspace:
    """cbx_group_norm_workspace: the tagged partial sums of the
    split-reduction GroupNorm (one call at a time per workspace)."""

    def __init__(self, device: Optional[int] = None, max_wait_us: Optional[int] = None, n_chunks: int = 0):
        dev = torch.cuda.current_device() if device is None else int(device)
        init(dev)
        h = ctypes.c_void_p()
        with torch.cuda.device(dev):
            _check(load().cbx_group_norm_workspace_create(ctypes.byref(h)))
        self.handle = h
        if max_wait_us is not None or n_chunks:
            self.tune(GN_WAIT_AUTO if max_wait_us is None else max_wait_us, n_chunks)

    def tune(self, max_wait_us: int, n_chunks: int = 0):
        _check(load().cbx_group_norm_workspace_tune(self.handle, max_wait_us, n_chunks))

    def close(self):
        if self.handle:
            load().cbx_group_norm_workspace_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def group_norm_ws(x, n_groups, eps, ws: GroupNormWorkspace, w=None, b=None, act=UNARY_NONE, out=None):
    """group_norm with the statistics split over many workgroups (same results)."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_group_norm_ws(_ref(desc(x)), n_groups, eps, _ref(desc(w)) if w is not None else None,
                                    _ref(desc(b)) if b is not None else None, act, _ref(desc(out)), ws.handle,
                                    _stream()))
    return out


def group_norm_noalloc(x, n_groups, eps, w=None, b=None, act=UNARY_NONE, out=None):
    """group_norm_ws over the library's static scratch (allocates nothing)."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_group_norm_noalloc(_ref(desc(x)), n_groups, eps, _ref(desc(w)) if w is not None else None,
                                         _ref(desc(b)) if b is not None else None, act, _ref(desc(out)), _stream()))
    return out


# ---- rope -----------------------------------------------------------------------

class RopeCache:
    """cbx_rope_cache: cos/sin table for ggml_rope_ext's parameters."""

    def __init__(self, n_dims: int, mode: int = 2, n_ctx_orig: int = 2048, freq_base: float = 10000.0,
                 freq_scale: float = 1.0, ext_factor: float = 0.0, attn_factor: float = 1.0,
                 beta_fast: float = 0.0, beta_slow: float = 0.0, freq_factors=None, n_pos: int = 2048,
                 device: Optional[int] = None):
        dev = torch.cuda.current_device() if device is None else int(device)
        init(dev)
        self.n_dims, self.mode, self.n_pos = n_dims, mode, n_pos
        ff = None
        if freq_factors is not None:
            ff = (ctypes.c_float * len(freq_factors))(*[float(v) for v in freq_factors])
        h = ctypes.c_void_p()
        with torch.cuda.device(dev):
            _check(load().cbx_rope_cache_create(n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor,
                                                attn_factor, beta_fast, beta_slow,
                                                ctypes.cast(ff, ctypes.c_void_p) if ff is not None else None,
                                                n_pos, ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            load().cbx_rope_cache_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def rope_ext(x, pos, cache: RopeCache, out=None):
    """ggml_rope_ext.  x [batch, n_tok, n_head, head_dim] (ggml (head_dim, n_head, n_tok, batch))."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_rope_ext(_ref(desc(x)), _ref(desc(pos)), cache.handle, _ref(desc(out)), _stream()))
    return out


def layer_norm_rope(x, w, b, eps, head_dim, pos, cache: RopeCache, out=None):
    """LayerNorm+affine of each row of x [batch, n_tok, C], then RoPE of the
    row viewed as [C/head_dim, head_dim] heads at position pos[token]."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_layer_norm_rope(_ref(desc(x)), _ref(desc(w)) if w is not None else None,
                                      _ref(desc(b)) if b is not None else None, eps, head_dim, _ref(desc(pos)),
                                      cache.handle, _ref(desc(out)), _stream()))
    return out


# ---- attention-score epilogue ---------------------------------------------------

def scale_diag_mask_soft_max(x, scale=1.0, n_past=-1, out=None):
    """soft_max(diag_mask_inf(scale(x), n_past)) over the last dim of x
    [.., n_queries, n_keys]; n_past < 0: no mask."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_scale_diag_mask_soft_max(_ref(desc(x)), scale, n_past, _ref(desc(out)), _stream()))
    return out


def add_scale_diag_mask_soft_max(a, b, scale=1.0, n_past=-1, out=None):
    """soft_max(diag_mask_inf(scale(a + b), n_past)) over the last dim, a and b
    of one shape (the relative-position attention's content and shifted
    position scores); n_past < 0: no mask."""
    _ready(a)
    _ready(b)
    out = _out_like(a, out)
    _check(load().cbx_add_scale_diag_mask_soft_max(_ref(desc(a)), _ref(desc(b)), scale, n_past, _ref(desc(out)),
                                                    _stream()))
    return out


# ---- activations ----------------------------------------------------------------

def unary(op, x, out=None):
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_unary(op, _ref(desc(x)), _ref(desc(out)), _stream()))
    return out


def gelu(x, out=None):
    return unary(GELU, x, out)


def gelu_erf(x, out=None):
    return unary(GELU_ERF, x, out)


def silu(x, out=None):
    return unary(SILU, x, out)


def tanh(x, out=None):
    return unary(TANH, x, out)


def softplus(x, out=None):
    return unary(SOFTPLUS, x, out)


def sin(x, out=None):
    return unary(SIN, x, out)


def sqr(x, out=None):
    return unary(SQR, x, out)


def mish(x, out=None):
    return unary(MISH, x, out)


def leaky_relu(x, slope, out=None):
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_leaky_relu(_ref(desc(x)), slope, _ref(desc(out)), _stream()))
    return out


def swiglu(g, u, out=None):
    """ggml_swiglu_split(g, u) = silu(g) * u."""
    _ready(g)
    out = _out_like(g, out)
    _check(load().cbx_swiglu(_ref(desc(g)), _ref(desc(u)), _ref(desc(out)), _stream()))
    return out


def add_layer_norm(a, r, w, b, eps, a_bias=None, act=UNARY_NONE, s=None, out=None, store_sum=True):
    """Residual join + LayerNorm: s = (a [+ a_bias]) [+ r], y = act(LN(s)*w + b)
    (r None: a linear's bias, then its LayerNorm; a_bias required).
    Returns (s, y); s is None when store_sum is False."""
    _ready(a)
    out = _out_like(a, out)
    if store_sum and s is None:
        s = torch.empty_like(a)
    if not store_sum:
        s = None
    _check(load().cbx_add_layer_norm(_ref(desc(a)), _ref(desc(a_bias) if a_bias is not None else None),
                                     _ref(desc(r) if r is not None else None), _ref(desc(w) if w is not None else None),
                                     _ref(desc(b) if b is not None else None), eps, act,
                                     _ref(desc(s) if s is not None else None), _ref(desc(out)), _stream()))
    return s, out


def layer_norm_mask(x, w, b, eps, mask, act=UNARY_NONE, out=None):
    """act(LN(x)*w + b) * mask, mask with one value per row index i1."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_layer_norm_mask(_ref(desc(x)), _ref(desc(w) if w is not None else None),
                                      _ref(desc(b) if b is not None else None), eps, act, _ref(desc(mask)),
                                      _ref(desc(out)), _stream()))
    return out


def bias_act(act, x, bias, out=None):
    """act(x + bias); bias shaped (C,) along the last dim, or (C, 1) per row."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_bias_act(act, _ref(desc(x)), _ref(desc(bias)), _ref(desc(out)), _stream()))
    return out


# cbx_binary_op
BINARY_ADD, BINARY_MUL = 0, 1


def binary(op, a, b, out=None):
    """ggml_add / ggml_mul(a, b) with b repeated to a's shape (torch shapes are
    ggml's ne reversed: a mask of one value per frame of a (T, C) tensor is
    (T, 1))."""
    _ready(a)
    out = _out_like(a, out)
    _check(load().cbx_binary(op, _ref(desc(a)), _ref(desc(b)), _ref(desc(out)), _stream()))
    return out


def bias_residual(x, bias, r, out=None):
    """ggml_add(r, ggml_add(x, bias)) in one pass: bias repeats to x's shape
    and x to r's; the inner add is rounded first."""
    _ready(r)
    out = _out_like(r, out)
    _check(load().cbx_bias_residual(_ref(desc(x)), _ref(desc(bias)), _ref(desc(r)), _ref(desc(out)), _stream()))
    return out


def bias_add_pair(x, bias, u, v, out_u=None, out_v=None):
    """(x + bias) + u and (x + bias) + v in one pass, the sum not stored:
    bias, u and v repeat to x's shape; each add one f32 rounding."""
    _ready(x)
    out_u = _out_like(x, out_u)
    out_v = _out_like(x, out_v)
    _check(load().cbx_bias_add_pair(_ref(desc(x)), _ref(desc(bias)), _ref(desc(u)), _ref(desc(v)), _ref(desc(out_u)),
                                    _ref(desc(out_v)), _stream()))
    return out_u, out_v


def bias_add_two(x0, b0, x1, b1, out0=None, out1=None):
    """x0 + b0 and x1 + b1, two independent bias adds in one launch."""
    _ready(x0)
    _ready(x1)
    out0 = _out_like(x0, out0)
    out1 = _out_like(x1, out1)
    _check(load().cbx_bias_add_two(_ref(desc(x0)), _ref(desc(b0)), _ref(desc(out0)), _ref(desc(x1)), _ref(desc(b1)),
                                   _ref(desc(out1)), _stream()))
    return out0, out1


def scale(x, s, out=None):
    """ggml_scale(x, s): x * s, one f32 rounding."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_scale(_ref(desc(x)), float(s), _ref(desc(out)), _stream()))
    return out


def concat(a, b, dim, out=None):
    """ggml_concat(a, b, dim), dim a ggml axis (0: the last torch axis)."""
    _ready(a)
    if out is None:
        shape = list(a.shape)
        ax = a.dim() - 1 - dim
        shape[ax] = a.shape[ax] + b.shape[ax]
        out = torch.empty(shape, dtype=a.dtype, device=a.device)
    _check(load().cbx_concat(_ref(desc(a)), _ref(desc(b)), dim, _ref(desc(out)), _stream()))
    return out


# cbx_conv_prologue
CONV_PRO_NONE, CONV_PRO_SNAKE, CONV_PRO_LEAKY_RELU = 0, 1, 2


class Conv1dWeights:
    """cbx_conv1d_weights: the f16 copy of a conv1d weight, torch [C_out,
    C_in, K] (ggml ne (K, C_in, C_out)), F32 or F16.  With transpose_stride
    set: a transposed conv's weight, torch [C_in, C_out, K] (ggml ne (K,
    C_out, C_in)), split into that many phases."""

    def __init__(self, w: torch.Tensor, transpose_stride=None):
        _ready(w)
        h = ctypes.c_void_p()
        if transpose_stride is None:
            _check(load().cbx_conv1d_weights_create(_ref(desc(w)), _stream(), ctypes.byref(h)))
            self.c_out, self.c_in, self.k = w.shape
        else:
            _check(load().cbx_conv_transpose1d_weights_create(_ref(desc(w)), transpose_stride, _stream(),
                                                               ctypes.byref(h)))
            self.c_in, self.c_out, self.k = w.shape
        self.handle = h
        self.stride = transpose_stride

    def close(self):
        if self.handle:
            load().cbx_conv1d_weights_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def conv1d(x, weights: Conv1dWeights, stride=1, pad=0, dilation=1, prologue=CONV_PRO_NONE, alpha=None,
           alpha_inv=None, slope=0.0, bias=None, res=None, out=None):
    """conv1d_CT(pro(x)) (+ bias) (+ res): x torch [B, T_in, C_in] or [T_in,
    C_in] (channel innermost, the reference's (C, T)); returns [.., T_out, C_out]."""
    _ready(x)
    t_in = x.shape[-2]
    t_out = (t_in + 2 * pad - dilation * (weights.k - 1) - 1) // stride + 1
    if out is None:
        out = torch.empty(tuple(x.shape[:-2]) + (t_out, weights.c_out), dtype=torch.float32, device=x.device)
    opt = lambda t: _ref(desc(t)) if t is not None else None  # noqa: E731
    _check(load().cbx_conv1d(_ref(desc(x)), weights.handle, stride, pad, dilation, prologue, opt(alpha),
                             opt(alpha_inv), slope, opt(bias), opt(res), _ref(desc(out)), _stream()))
    return out


def conv1d_sum(x, weights: Conv1dWeights, stride, pad, dilation, prologue, alpha, alpha_inv, slope, bias, res, acc,
               scale=1.0, out=None):
    """(acc + conv1d(...)) * scale in one kernel: a HiFT stage's ResBlock sum
    and mean folded into the resblock's last conv."""
    _ready(x)
    t_out = (x.shape[-2] + 2 * pad - dilation * (weights.k - 1) - 1) // stride + 1
    if out is None:
        out = torch.empty(tuple(x.shape[:-2]) + (t_out, weights.c_out), dtype=torch.float32, device=x.device)
    opt = lambda t: _ref(desc(t)) if t is not None else None  # noqa: E731
    _check(load().cbx_conv1d_sum(_ref(desc(x)), weights.handle, stride, pad, dilation, prologue, opt(alpha),
                                 opt(alpha_inv), slope, opt(bias), opt(res), opt(acc), float(scale),
                                 _ref(desc(out)), _stream()))
    return out


def conv_transpose1d(x, weights: Conv1dWeights, pad=0, prologue=CONV_PRO_NONE, alpha=None, alpha_inv=None, slope=0.0,
                     bias=None, out=None):
    """conv_transpose1d_CT(pro(x)) (+ bias) with `pad` cropped from both
    ends: x torch [B, T_in, C_in] or [T_in, C_in]; weights made with
    transpose_stride; returns [.., (T_in - 1) * stride + K - 2 pad, C_out]."""
    _ready(x)
    t_out = (x.shape[-2] - 1) * weights.stride + weights.k - 2 * pad
    if out is None:
        out = torch.empty(tuple(x.shape[:-2]) + (t_out, weights.c_out), dtype=torch.float32, device=x.device)
    opt = lambda t: _ref(desc(t)) if t is not None else None  # noqa: E731
    _check(load().cbx_conv_transpose1d(_ref(desc(x)), weights.handle, pad, prologue, opt(alpha), opt(alpha_inv), slope,
                                       opt(bias), _ref(desc(out)), _stream()))
    return out


def causal_conv1d(x, weights: Conv1dWeights, mask=None, bias=None, out=None):
    """CausalConv1d(mask * x) (+ bias): K - 1 zero frames on the left, stride
    1, T_out = T_in.  x torch [B, T, C_in] or [T, C_in]; mask T floats (the
    reference's (1, T)) or None; returns [.., T, C_out]."""
    _ready(x)
    if out is None:
        out = torch.empty(tuple(x.shape[:-1]) + (weights.c_out,), dtype=torch.float32, device=x.device)
    opt = lambda t: _ref(desc(t)) if t is not None else None  # noqa: E731
    _check(load().cbx_causal_conv1d(_ref(desc(x)), weights.handle, opt(mask), opt(bias), _ref(desc(out)), _stream()))
    return out


def snake(x, alpha, alpha_inv, out=None):
    """snake() helper: x + sin^2(x*alpha) * alpha_inv.  alpha shaped (C,) for
    channel-innermost x [.., T, C], or (C, 1) for x [.., C, T]."""
    _ready(x)
    out = _out_like(x, out)
    _check(load().cbx_snake(_ref(desc(x)), _ref(desc(alpha)), _ref(desc(alpha_inv)), _ref(desc(out)), _stream()))
    return out


# ---- one launch for several independent ops -----------------------------------

class Op:
    """One entry of run_ops: kind (OP_*), source and destination tensors
    (None for absent optional operands), activation, eps, param, rope table,
    iparam (GroupNorm's n_groups, LayerNorm+RoPE's head_dim).  q8 lists the
    source indices that are Q8_0 tables (uint8 blocks)."""

    def __init__(self, kind, src=(), dst=(), act=UNARY_NONE, eps=0.0, param=0.0, rope: Optional[RopeCache] = None,
                 q8=(), iparam=0):
        self.kind, self.act, self.eps, self.param, self.rope = kind, act, eps, param, rope
        self.iparam = iparam
        self.src = list(src) + [None] * (6 - len(src))
        self.dst = list(dst) + [None] * (2 - len(dst))
        self.q8 = set(q8)

    def struct(self, keep: list) -> OpStruct:
        o = OpStruct()
        o.kind, o.act, o.eps, o.param = self.kind, self.act, self.eps, self.param
        for k, t in enumerate(self.src):
            if t is not None:
                d = desc(t, Q8_0 if k in self.q8 else None)
                keep.append(d)
                o.src[k] = ctypes.pointer(d)
        for k, t in enumerate(self.dst):
            if t is not None:
                d = desc(t)
                keep.append(d)
                o.dst[k] = ctypes.pointer(d)
        o.rope = self.rope.handle.value if self.rope is not None else None
        o.iparam = self.iparam
        return o


class OpBatch:
    """Prebuilt argument array for cbx_run_ops (build once, launch often)."""

    def __init__(self, ops):
        if not ops or len(ops) > MAX_OPS:
            raise CbxError(ERR_INVALID_ARG, f"1..{MAX_OPS} ops per launch")
        self._keep: list = []
        self.ops = list(ops)
        self.n = len(ops)
        self.arr = (OpStruct * self.n)(*[op.struct(self._keep) for op in ops])

    def launch(self, stream=None) -> None:
        _check(load().cbx_run_ops(self.arr, self.n, stream if stream is not None else _stream()))


def run_ops(ops) -> None:
    """Runs independent ops in one kernel launch (cbx_run_ops)."""
    for op in ops:
        for t in op.src + op.dst:
            if t is not None:
                _ready(t)
                break
    OpBatch(ops).launch()


# ---- GGUF tables ------------------------------------------------------------------

class Gguf:
    """cbx_gguf: a GGUF file's directory; tensors upload into torch device tensors."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _check(load().cbx_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            load().cbx_gguf_close(self.handle)
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __len__(self) -> int:
        return int(load().cbx_gguf_n_tensors(self.handle))

    def find(self, name: str) -> int:
        return int(load().cbx_gguf_find_tensor(self.handle, name.encode()))

    def get_str(self, key: str) -> Optional[str]:
        v = load().cbx_gguf_get_str(self.handle, key.encode())
        return v.decode() if v is not None else None

    def info(self, index: int) -> GgufTensorInfo:
        out = GgufTensorInfo()
        _check(load().cbx_gguf_tensor(self.handle, index, ctypes.byref(out)))
        return out

    def upload(self, index: int, device: Optional[int] = None) -> torch.Tensor:
        """The tensor's bytes as a uint8 device tensor (viewed as float32 /
        float16 / int32 for those types, Q8_0 blocks stay uint8 [rows, n*34])."""
        inf = self.info(index)
        dev = torch.cuda.current_device() if device is None else int(device)
        raw = torch.empty(inf.nbytes, dtype=torch.uint8, device=f"cuda:{dev}")
        with torch.cuda.device(dev):
            _check(load().cbx_gguf_upload(self.handle, index, ctypes.c_void_p(raw.data_ptr()), inf.nbytes,
                                          _stream()))
        ne = [inf.ne[k] for k in range(inf.n_dims)][::-1]
        if inf.type == Q8_0:
            return raw.view(*ne[:-1], ne[-1] // QK8_0 * Q8_0_BLOCK)
        dt = {F32: torch.float32, F16: torch.float16, I32: torch.int32}.get(inf.type)
        return raw.view(dt).view(*ne) if dt is not None else raw

    def describe(self, index: int, data: torch.Tensor) -> Tensor:
        d = Tensor()
        _check(load().cbx_gguf_describe(self.handle, index, ctypes.c_void_p(data.data_ptr()), ctypes.byref(d)))
        return d

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- ggml-style node lists -------------------------------------------------------

class Graph:
    """A node list for cbx_graph_*: tensors are registered once (torch
    tensors, device or host -- planning reads only shapes, types and
    addresses) and nodes name them by index, as a ggml graph names its
    tensors.  plan() shows how the nodes group into launches; compute() runs
    them on torch's current stream."""

    def __init__(self):
        self._descs: list = []
        self._torch: list = []
        self.nodes: list = []
        self._bound = None

    def tensor(self, t: torch.Tensor, ggml_type: Optional[int] = None) -> int:
        self._bound = None
        self._descs.append(desc(t, ggml_type))
        self._torch.append(t)
        return len(self._descs) - 1

    def rebind(self, i: int, t: torch.Tensor, ggml_type: Optional[int] = None) -> None:
        """Tensor i of the list becomes t (another buffer, or a view of
        another length: the next step of a loop)."""
        if self._bound is not None:
            self._bound[0][i] = desc(t, ggml_type)   # copied into the array _descs[i] views
        else:
            self._descs[i] = desc(t, ggml_type)
        self._torch[i] = t

    def bind_arrays(self, keep=()):
        """Builds the arrays the C calls take once and makes the list's
        descriptors and nodes views of them, so a loop that changes a few
        descriptors (rebind, or their fields set in place) or node
        parameters between calls passes the same arrays again without
        rebuilding them.  Adding a tensor or a node unbinds."""
        T, N, K = self._arrays(keep)
        self._descs = [T[i] for i in range(len(self._descs))]
        self.nodes = [N[i] for i in range(len(self.nodes))]
        self._bound = (T, N, K, tuple(keep))
        return T, N, K

    def node(self, op: int, dst: int, src=(), iparam: int = 0, fparam: float = 0.0,
             rope: Optional[RopeCache] = None, conv=(0, 0, 0), conv_w=None) -> int:
        """conv: (stride, padding, dilation) of an IM2COL node, (stride,) of a
        CONV_TRANSPOSE_1D node; conv_w: Conv1dWeights on the MUL_MAT /
        CONV_TRANSPOSE_1D node, or any non-null address when only planning."""
        s = list(src) + [-1] * (2 - len(src))
        n = GNode()
        n.op, n.dst, n.iparam, n.fparam = op, dst, iparam, fparam
        n.src[0], n.src[1] = s[0], s[1]
        n.rope = rope.handle.value if rope is not None else None
        cv = list(conv) + [0] * (3 - len(conv))
        n.conv[0], n.conv[1], n.conv[2] = cv[0], cv[1], cv[2]
        n.conv_w = conv_w.handle.value if isinstance(conv_w, Conv1dWeights) else conv_w
        self._bound = None
        self.nodes.append(n)
        return dst

    def _arrays(self, keep):
        if self._bound is not None and self._bound[3] == tuple(keep):
            return self._bound[:3]
        T = (Tensor * max(1, len(self._descs)))(*self._descs)
        N = (GNode * max(1, len(self.nodes)))(*self.nodes)
        K = (ctypes.c_int32 * max(1, len(keep)))(*keep)
        return T, N, K

    def plan(self, keep=()) -> list:
        """[(kind, first_node, n_nodes, flags)] from cbx_graph_plan."""
        T, N, K = self._arrays(keep)
        cap = max(1, len(self.nodes))
        out = (GLaunch * cap)()
        n = ctypes.c_int32(0)
        _check(load().cbx_graph_plan(T, len(self._descs), N, len(self.nodes), K, len(keep), out, cap,
                                     ctypes.byref(n)))
        return [(out[k].kind, out[k].first_node, out[k].n_nodes, out[k].flags) for k in range(n.value)]

    def compute(self, keep=()) -> int:
        """Runs the nodes (cbx_graph_compute); returns the number of launches."""
        for t in self._torch:
            if t.is_cuda:
                _ready(t)
                break
        T, N, K = self._arrays(keep)
        n = ctypes.c_int32(0)
        _check(load().cbx_graph_compute(T, len(self._descs), N, len(self.nodes), K, len(keep), _stream(),
                                        ctypes.byref(n)))
        return n.value

    def capture(self, keep=()) -> "GraphExec":
        """The node list recorded once into a HIP graph (cbx_graph_exec_create)
        for replays over the same buffers."""
        return GraphExec(self, keep)


class GraphExec:
    """cbx_graph_exec: a Graph's launches captured into a HIP graph; launch()
    replays them on torch's current stream.  The graph holds the tensors'
    addresses: keep the Graph (and its tensors) alive while this is used."""

    def __init__(self, g: Graph, keep=()):
        for t in g._torch:
            if t.is_cuda:
                _ready(t)
                break
        T, N, K = g._arrays(keep)
        h = ctypes.c_void_p()
        n = ctypes.c_int32(0)
        _check(load().cbx_graph_exec_create(T, len(g._descs), N, len(g.nodes), K, len(keep), ctypes.byref(h),
                                            ctypes.byref(n)))
        self.handle = h
        self.n_launches = n.value
        self._graph = g

    def launch(self, stream=None):
        _check(load().cbx_graph_exec_launch(self.handle, _stream() if stream is None else stream))

    def update(self, g: Graph = None, keep=()) -> bool:
        """cbx_graph_exec_update: the exec re-pointed at `g` (default: the
        Graph it was captured from, as it is now -- its tensors re-bound or its
        nodes' parameters changed).  True when the instantiated graph took the
        new arguments in place, False when it was re-instantiated."""
        g = self._graph if g is None else g
        for t in g._torch:
            if t.is_cuda:
                _ready(t)
                break
        T, N, K = g._arrays(keep)
        n = ctypes.c_int32(0)
        ip = ctypes.c_int32(0)
        _check(load().cbx_graph_exec_update(self.handle, T, len(g._descs), N, len(g.nodes), K, len(keep),
                                            ctypes.byref(n), ctypes.byref(ip)))
        self.n_launches = n.value
        self._graph = g
        return bool(ip.value)

    def close(self):
        if self.handle:
            load().cbx_graph_exec_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
