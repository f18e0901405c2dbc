"""ctypes front end of the CPU oracle (liboracle_cbx.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Arrays are numpy,
host memory; shapes follow numpy order (outermost first) and are mapped to
ggml's ne[] (innermost first) by reversing them.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_cbx.so")

F32, F16, Q8_0, I32 = 0, 1, 8, 26
GELU, GELU_ERF, SILU, TANH, SOFTPLUS, SIN, SQR, MISH = range(8)
QK8_0 = 32
Q8_0_BLOCK = 34


class Tensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
    ]


_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(Tensor)
        i, f, vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
        sig = {
            "cbxo_fp16_to_fp32": (f, [ctypes.c_uint16]),
            "cbxo_fp32_to_fp16": (ctypes.c_uint16, [f]),
            "cbxo_quantize_row_q8_0": (None, [vp, vp, ctypes.c_int64]),
            "cbxo_dequantize_row_q8_0": (None, [vp, vp, ctypes.c_int64]),
            "cbxo_gelu_table": (None, [vp, i]),
            "cbxo_gelu_f32": (f, [f, i]),
            "cbxo_get_rows": (i, [P, P, P, i]),
            "cbxo_add": (i, [P, P, P, i]),
            "cbxo_mul": (i, [P, P, P, i]),
            "cbxo_norm": (i, [P, f, P, i]),
            "cbxo_rms_norm": (i, [P, f, P, i]),
            "cbxo_group_norm": (i, [P, i, f, P, i]),
            "cbxo_unary": (i, [i, P, P, i]),
            "cbxo_leaky_relu": (i, [P, f, P, i]),
            "cbxo_swiglu": (i, [P, P, P, i]),
            "cbxo_cpy": (i, [P, P, i]),
            "cbxo_rope_yarn_corr_dims": (None, [i, i, f, f, f, vp]),
            "cbxo_rope_cache_init": (None, [f, f, vp, vp, ctypes.c_int64, f, f, vp, f, f]),
            "cbxo_rope_ext": (i, [P, P, vp, i, i, i, f, f, f, f, f, f, P, i]),
            "cbxo_layer_norm": (i, [P, P, P, f, P, i]),
            "cbxo_rms_norm_mul": (i, [P, P, f, P, i]),
            "cbxo_group_norm_affine": (i, [P, i, f, P, P, i, P, i]),
            "cbxo_snake": (i, [P, P, P, P, i]),
            "cbxo_get_rows_add": (i, [P, P, P, P, P, i]),
            "cbxo_scale": (i, [P, f, P, i]),
            "cbxo_diag_mask_inf": (i, [P, i, P, i]),
            "cbxo_soft_max": (i, [P, P, i]),
            "cbxo_scale_diag_mask_soft_max": (i, [P, f, i, P, i]),
            "cbxo_conv1d": (i, [P, P, i, i, i, i, P, P, f, P, P, P, i]),
            "cbxo_conv_transpose1d": (i, [P, P, i, i, i, P, P, f, P, P, i]),
            "cbxo_t3_token_step": (i, [P, ctypes.c_int32, P, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64,
                                       ctypes.c_int32, f, ctypes.POINTER(T3Block), ctypes.c_int32, vp, vp, vp,
                                       vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ggml_type(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.int32:
        return I32
    raise TypeError(f"unsupported dtype {a.dtype}")


def desc(a: np.ndarray, ggml_type: int | None = None) -> Tensor:
    """Descriptor of a numpy array (any strides, up to 4 dims)."""
    t = Tensor()
    t.data = a.ctypes.data
    assert 1 <= a.ndim <= 4
    shape = list(a.shape[::-1])
    strides = list(a.strides[::-1])
    # size in bytes of one step of the last listed dim, used to pad to 4 dims
    row_bytes = strides[-1] * shape[-1]
    if ggml_type == Q8_0:
        # a: uint8 [..., n_blocks * 34]; ne0 counts elements, nb0 is the block size
        assert a.dtype == np.uint8 and a.shape[-1] % Q8_0_BLOCK == 0 and a.strides[-1] == 1
        shape[0] = shape[0] // Q8_0_BLOCK * QK8_0
        strides[0] = Q8_0_BLOCK
        t.type = Q8_0
    else:
        t.type = _ggml_type(a) if ggml_type is None else ggml_type
    while len(shape) < 4:
        shape.append(1)
        strides.append(row_bytes)
    for k in range(4):
        t.ne[k] = shape[k]
        t.nb[k] = strides[k]
    return t


def _ref(t: Tensor):
    return ctypes.byref(t)


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with {rc}")


# ---- scalar helpers -------------------------------------------------------

def fp16_to_fp32(h: int) -> float:
    return lib().cbxo_fp16_to_fp32(h)


def fp32_to_fp16(x: float) -> int:
    return lib().cbxo_fp32_to_fp16(x)


def gelu_table(fma_variant: int = 0) -> np.ndarray:
    out = np.empty(65536, dtype=np.uint16)
    lib().cbxo_gelu_table(out.ctypes.data, fma_variant)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """x float32 [rows, k] -> uint8 [rows, k/32*34] (ggml block_q8_0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    out = np.empty((rows, k // QK8_0 * Q8_0_BLOCK), dtype=np.uint8)
    for r in range(rows):
        lib().cbxo_quantize_row_q8_0(x[r].ctypes.data, out[r].ctypes.data, k)
    return out


def dequantize_q8_0(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q)
    rows = q.shape[0]
    k = q.shape[1] // Q8_0_BLOCK * QK8_0
    out = np.empty((rows, k), dtype=np.float32)
    for r in range(rows):
        lib().cbxo_dequantize_row_q8_0(q[r].ctypes.data, out[r].ctypes.data, k)
    return out


# ---- ops ------------------------------------------------------------------

def get_rows(table: np.ndarray, ids: np.ndarray, q8_0: bool = False, nth: int = 1) -> np.ndarray:
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    ne0 = table.shape[-1] // Q8_0_BLOCK * QK8_0 if q8_0 else table.shape[-1]
    out = np.empty(ids.shape + (ne0,), dtype=np.float32)
    td = desc(table, Q8_0 if q8_0 else None)
    _check(lib().cbxo_get_rows(_ref(td), _ref(desc(ids)), _ref(desc(out)), nth), "get_rows")
    return out


def get_rows_add(table, ids, table2, ids2, q8_0=False, nth=1):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    ids2 = np.ascontiguousarray(ids2, dtype=np.int32)
    ne0 = table.shape[-1] // Q8_0_BLOCK * QK8_0 if q8_0 else table.shape[-1]
    out = np.empty(ids.shape + (ne0,), dtype=np.float32)
    td = desc(table, Q8_0 if q8_0 else None)
    _check(lib().cbxo_get_rows_add(_ref(td), _ref(desc(ids)), _ref(desc(table2)), _ref(desc(ids2)),
                                   _ref(desc(out)), nth), "get_rows_add")
    return out


def add(a, b, nth=1):
    out = np.empty_like(a)
    _check(lib().cbxo_add(_ref(desc(a)), _ref(desc(b)), _ref(desc(out)), nth), "add")
    return out


def mul(a, b, nth=1):
    out = np.empty_like(a)
    _check(lib().cbxo_mul(_ref(desc(a)), _ref(desc(b)), _ref(desc(out)), nth), "mul")
    return out


def norm(x, eps, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_norm(_ref(desc(x)), eps, _ref(desc(out)), nth), "norm")
    return out


def rms_norm(x, eps, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_rms_norm(_ref(desc(x)), eps, _ref(desc(out)), nth), "rms_norm")
    return out


def group_norm(x, n_groups, eps, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_group_norm(_ref(desc(x)), n_groups, eps, _ref(desc(out)), nth), "group_norm")
    return out


def unary(op, x, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_unary(op, _ref(desc(x)), _ref(desc(out)), nth), "unary")
    return out


def leaky_relu(x, slope, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_leaky_relu(_ref(desc(x)), slope, _ref(desc(out)), nth), "leaky_relu")
    return out


def swiglu(g, u, nth=1):
    out = np.empty_like(g)
    _check(lib().cbxo_swiglu(_ref(desc(g)), _ref(desc(u)), _ref(desc(out)), nth), "swiglu")
    return out


def cpy(src, dtype, nth=1):
    out = np.empty(src.shape, dtype=dtype)
    _check(lib().cbxo_cpy(_ref(desc(src)), _ref(desc(out)), nth), "cpy")
    return out


def rope_ext(x, pos, n_dims, mode=2, n_ctx_orig=2048, freq_base=10000.0, freq_scale=1.0,
             ext_factor=0.0, attn_factor=1.0, beta_fast=0.0, beta_slow=0.0,
             freq_factors=None, nth=1):
    """x: numpy [.., n_tok, n_head, head_dim] (ggml ne = (head_dim, n_head, n_tok, b))."""
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    out = np.empty_like(x)
    ff = None
    if freq_factors is not None:
        ff = np.ascontiguousarray(freq_factors, dtype=np.float32)
    _check(lib().cbxo_rope_ext(_ref(desc(x)), _ref(desc(pos)), ff.ctypes.data if ff is not None else None,
                               n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor,
                               beta_fast, beta_slow, _ref(desc(out)), nth), "rope_ext")
    return out


_libm = None


def theta_scale_f32(freq_base: float, n_dims: int) -> float:
    """powf(freq_base, -2.0f/n_dims) from the C library, as ggml forms it
    (numpy's float32 power can differ by an ulp, which moves theta by up to
    ~1e-3 rad at position 2047)."""
    global _libm
    if _libm is None:
        _libm = ctypes.CDLL("libm.so.6")
        _libm.powf.restype = ctypes.c_float
        _libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return float(_libm.powf(freq_base, float(np.float32(-2.0) / np.float32(n_dims))))


def rope_cache(pos, n_dims, freq_base=10000.0, freq_scale=1.0, ext_factor=0.0, attn_factor=1.0,
               n_ctx_orig=2048, beta_fast=0.0, beta_slow=0.0, freq_factors=None):
    """cos/sin cache of one position, ggml_rope_cache_init layout [cos0, sin0, cos1, ...]."""
    L = lib()
    dims = np.zeros(2, dtype=np.float32)
    L.cbxo_rope_yarn_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, dims.ctypes.data)
    cache = np.zeros(n_dims, dtype=np.float32)
    theta_scale = theta_scale_f32(freq_base, n_dims)
    ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
    L.cbxo_rope_cache_init(float(pos), freq_scale, ff.ctypes.data if ff is not None else None,
                           dims.ctypes.data, n_dims, ext_factor, attn_factor, cache.ctypes.data, 1.0,
                           float(theta_scale))
    return cache


def layer_norm(x, w, b, eps, out_dtype=None, nth=1):
    out = np.empty(x.shape, dtype=out_dtype or x.dtype)
    _check(lib().cbxo_layer_norm(_ref(desc(x)), _ref(desc(w)) if w is not None else None,
                                 _ref(desc(b)) if b is not None else None, eps, _ref(desc(out)), nth),
           "layer_norm")
    return out


def rms_norm_mul(x, g, eps, out_dtype=None, nth=1):
    out = np.empty(x.shape, dtype=out_dtype or x.dtype)
    _check(lib().cbxo_rms_norm_mul(_ref(desc(x)), _ref(desc(g)) if g is not None else None, eps,
                                   _ref(desc(out)), nth), "rms_norm_mul")
    return out


def group_norm_affine(x, n_groups, eps, w, b, fuse_mish, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_group_norm_affine(_ref(desc(x)), n_groups, eps,
                                        _ref(desc(w)) if w is not None else None,
                                        _ref(desc(b)) if b is not None else None,
                                        1 if fuse_mish else 0, _ref(desc(out)), nth), "group_norm_affine")
    return out


def scale(x, s, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_scale(_ref(desc(x)), s, _ref(desc(out)), nth), "scale")
    return out


def diag_mask_inf(x, n_past, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_diag_mask_inf(_ref(desc(x)), n_past, _ref(desc(out)), nth), "diag_mask_inf")
    return out


def soft_max(x, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_soft_max(_ref(desc(x)), _ref(desc(out)), nth), "soft_max")
    return out


def scale_diag_mask_soft_max(x, s, n_past=-1, nth=1):
    """soft_max(diag_mask_inf(scale(x, s), n_past)); n_past < 0: no mask."""
    out = np.empty_like(x)
    _check(lib().cbxo_scale_diag_mask_soft_max(_ref(desc(x)), s, n_past, _ref(desc(out)), nth),
           "scale_diag_mask_soft_max")
    return out


def snake(x, alpha, alpha_inv, nth=1):
    out = np.empty_like(x)
    _check(lib().cbxo_snake(_ref(desc(x)), _ref(desc(alpha)), _ref(desc(alpha_inv)), _ref(desc(out)), nth),
           "snake")
    return out


CONV_PRO_NONE, CONV_PRO_SNAKE, CONV_PRO_LEAKY = 0, 1, 2


def conv1d(x, w, stride=1, pad=0, dilation=1, prologue=0, alpha=None, alpha_inv=None, slope=0.0, bias=None,
           res=None, nth=1):
    """conv1d_CT(pro(x)) (+ bias) (+ res).  x: numpy [B, T_in, C_in] or
    [T_in, C_in] (ggml ne = (C_in, T_in, B)); w: [C_out, C_in, K] (ggml ne =
    (K, C_in, C_out), the PyTorch layout); returns [.., T_out, C_out]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    C_out, C_in, K = w.shape
    T_in = x.shape[-2]
    T_out = (T_in + 2 * pad - dilation * (K - 1) - 1) // stride + 1
    out = np.empty(x.shape[:-2] + (T_out, C_out), dtype=np.float32)
    opt = lambda a: _ref(desc(np.ascontiguousarray(a, dtype=np.float32))) if a is not None else None  # noqa: E731
    keep = [np.ascontiguousarray(a, dtype=np.float32) if a is not None else None for a in (alpha, alpha_inv, bias, res)]
    _check(lib().cbxo_conv1d(_ref(desc(x)), _ref(desc(np.ascontiguousarray(w))), stride, pad, dilation, prologue,
                             opt(keep[0]), opt(keep[1]), slope, opt(keep[2]), opt(keep[3]), _ref(desc(out)), nth),
           "conv1d")
    return out


def conv_transpose1d(x, w, stride, pad=0, prologue=0, alpha=None, alpha_inv=None, slope=0.0, bias=None, nth=1):
    """conv_transpose1d_CT(pro(x)) (+ bias), pad cropped from both ends.  x:
    numpy [B, T_in, C_in] or [T_in, C_in]; w: [C_in, C_out, K] (ggml ne (K,
    C_out, C_in), the PyTorch ConvTranspose1d layout); returns [.., T_out,
    C_out], T_out = (T_in - 1) * stride + K - 2 * pad."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    C_in, C_out, K = w.shape
    T_out = (x.shape[-2] - 1) * stride + K - 2 * pad
    out = np.empty(x.shape[:-2] + (T_out, C_out), dtype=np.float32)
    opt = lambda a: _ref(desc(np.ascontiguousarray(a, dtype=np.float32))) if a is not None else None  # noqa: E731
    keep = [np.ascontiguousarray(a, dtype=np.float32) if a is not None else None for a in (alpha, alpha_inv, bias)]
    _check(lib().cbxo_conv_transpose1d(_ref(desc(x)), _ref(desc(np.ascontiguousarray(w))), stride, pad, prologue,
                                       opt(keep[0]), opt(keep[1]), slope, opt(keep[2]), _ref(desc(out)), nth),
           "conv_transpose1d")
    return out


# ---- the T3 decode step's element-wise nodes (t3.cpp:446-546, N_new = 1) ----

T3_BLOCK_IN = ("ln1_w", "ln1_b", "qkv_b", "out_b", "ln2_w", "ln2_b", "fc_b", "proj_b",
               "qkv_mm", "kq", "out_mm", "fc_mm", "proj_mm")
T3_BLOCK_OUT = ("ln1", "qkv", "probs", "attn_res", "ln2", "gelu", "h")


class T3Block(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in T3_BLOCK_IN + T3_BLOCK_OUT]


class T3TokenStep:
    """cbxo_t3_token_step over the arrays of workloads.t3_token_inputs: one
    token's element-wise nodes in the reference's order, one thread.  The
    block table is built once per n_past, so run() is one C call (the CPU
    baseline times it).  Outputs: h0, y and per block the T3_BLOCK_OUT
    arrays (probs as (H, n_past + 1))."""

    def __init__(self, inp: dict, n_past: int, n_head: int = 16, eps: float = 1e-5):
        self.inp, self.n_past, self.n_head, self.eps = inp, int(n_past), int(n_head), float(eps)
        L, D = inp["ln1_w"].shape
        F = inp["fc_b"].shape[1]
        n_kv = self.n_past + 1
        self.d_ff = F
        self.kq = [np.ascontiguousarray(inp["kq"][il, :n_head * n_kv].reshape(n_head, n_kv)) for il in range(L)]
        self.out = {"h0": np.empty((1, D), np.float32), "y": np.empty((1, D), np.float32)}
        shapes = {"ln1": (L, D), "qkv": (L, 3 * D), "probs": (L, n_head, n_kv), "attn_res": (L, D),
                  "ln2": (L, D), "gelu": (L, F), "h": (L, D)}
        for k, shp in shapes.items():
            self.out[k] = np.full(shp, np.nan, np.float32)
        self.blocks = (T3Block * L)()
        for il in range(L):
            b = self.blocks[il]
            for k in T3_BLOCK_IN:
                a = self.kq[il] if k == "kq" else inp[k][il]
                assert a.dtype == np.float32 and a.flags.c_contiguous
                setattr(b, k, a.ctypes.data)
            for k in T3_BLOCK_OUT:
                setattr(b, k, self.out[k][il].ctypes.data)
        self._tok = desc(inp["speech_emb"])
        self._pos = desc(inp["pos_embd"])

    def run(self, token: int, position: int) -> dict:
        _check(lib().cbxo_t3_token_step(_ref(self._tok), int(token), _ref(self._pos), int(position), self.d_ff,
                                         self.n_head, self.n_past, self.eps, self.blocks, len(self.blocks),
                                         self.inp["out_w"].ctypes.data, self.inp["out_b_final"].ctypes.data,
                                         self.out["h0"].ctypes.data, self.out["y"].ctypes.data), "t3_token_step")
        return self.out


def run_node_list(nodes, shapes, values, rope=None, nth=1):
    """Runs a ggml-style node list node by node, as ggml-cpu's graph compute
    does (chatterbox-cpp/src/backend.cpp:108-122 on the CPU backend).

    nodes: (op, dst, src0, src1, iparam, fparam) tuples, op one of "view",
    "get_rows", "add", "mul", "scale", "norm", "soft_max", "unary",
    "leaky_relu", "rope"; shapes[i]: the numpy shape of tensor i; values: a
    dict holding the leaf arrays by index, filled with every node's output.
    A view is a reshape of its contiguous source.  rope: rope_ext's keyword
    arguments (n_dims first) for the rope nodes.  Returns values."""
    for op, d, s0, s1, ip, fp in nodes:
        a = values[s0] if s0 >= 0 else None
        b = values[s1] if s1 >= 0 else None
        if op == "view":
            out = a.reshape(shapes[d])
        elif op == "get_rows":
            out = get_rows(a, b, nth=nth)
        elif op == "add":
            out = add(a, b, nth=nth)
        elif op == "mul":
            out = mul(a, b, nth=nth)
        elif op == "scale":
            out = scale(a, fp, nth=nth)
        elif op == "norm":
            out = norm(a, fp, nth=nth)
        elif op == "soft_max":
            out = scale_diag_mask_soft_max(a, fp, -1, nth=nth)
        elif op == "unary":
            out = unary(ip, a, nth=nth)
        elif op == "leaky_relu":
            out = leaky_relu(a, fp, nth=nth)
        elif op == "rope":
            out = rope_ext(a, b, **rope, nth=nth)
        else:
            raise ValueError(f"run_node_list: no oracle op for {op!r}")
        values[d] = out
    return values
