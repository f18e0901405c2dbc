"""Synthetic inputs and the workload shapes used by bench.py and the tests.

Inputs come from a counter-based generator: splitmix64 of (seed, index)
gives uniform 53-bit doubles, Box-Muller turns pairs of them into normals.
Every tensor has its own seed, 0x5EED0000 + 16 * workload + tensor, so the
CPU and GPU legs of a run consume identical bits.

Workloads (torch shape order; ggml's ne[] is the reverse):
  1  T3 decode step, f32: RMSNorm+gamma [1,1024]; NEOX RoPE q,k [1,16,64]
     at positions 0..29; SiLU(gate)*up [1,4096]; 30 steps.
  2  T3 prefill: gather 512 ids of [8194,1024] (f32 and f16 tables) plus
     position rows 0..511; LayerNorm+affine [512,1024]; tanh-GELU [512,4096].
  3  CFM estimator: GroupNorm(8)+affine+Mish on [2,256,500] and [2,512,500]
     (ggml ne (500,1,C,2)); LayerNorm+RoPE on [2,500,8,64]; 10 flow steps.
  4  HiFT vocoder: Snake (per-channel alpha) and LeakyReLU(0.1) on
     [1,256,6000], [1,128,48000], [1,64,120000], [16,64,120000].
  5  64-stream decode, f16 storage: RMSNorm+gamma [64,1024]; RoPE q,k
     [64,16,64] at positions U[0,2048); SiLU-gate [64,4096]; Q8_0 gather of
     64 rows of [8194,1024].
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def seed_of(workload: int, tensor: int) -> int:
    return 0x5EED0000 + 16 * workload + tensor


def splitmix64(seed: int, n: int, offset: int = 0) -> np.ndarray:
    """n successive splitmix64 outputs of the stream `seed`."""
    with np.errstate(over="ignore"):
        i = np.arange(offset + 1, offset + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int) -> np.ndarray:
    """float64 in [0, 1)."""
    return (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    m = (n + 1) // 2
    u = uniform(seed, 2 * m)
    r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
    th = 2.0 * np.pi * u[1::2]
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(th)
    z[1::2] = r * np.sin(th)
    return (mean + std * z[:n]).astype(np.float32).reshape(shape)


def uniform_range(seed: int, shape, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape))
    return (lo + (hi - lo) * uniform(seed, n)).astype(np.float32).reshape(shape)


def randint(seed: int, shape, lo: int, hi: int) -> np.ndarray:
    """int32 uniform in [lo, hi)."""
    n = int(np.prod(shape))
    z = splitmix64(seed, n)
    return (lo + (z % np.uint64(hi - lo)).astype(np.int64)).astype(np.int32).reshape(shape)


# ---- workload 2 (T3 prefill), the default bench workload -----------------------
VOCAB = 8194
D_MODEL = 1024
D_FF = 4096
N_PREFILL = 512
LN_EPS = 1e-5


def prefill_inputs(f16_table: bool = False) -> dict:
    w = 2
    tab = normal(seed_of(w, 0), (VOCAB, D_MODEL), 0.0, 0.02)
    pos_tab = normal(seed_of(w, 1), (VOCAB, D_MODEL), 0.0, 0.02)
    if f16_table:
        tab = tab.astype(np.float16)
    return {
        "table": tab,
        "ids": randint(seed_of(w, 2), (N_PREFILL,), 0, VOCAB),
        "pos_table": pos_tab,
        "pos_ids": np.arange(N_PREFILL, dtype=np.int32),
        "ln_w": normal(seed_of(w, 3), (D_MODEL,), 1.0, 0.02),
        "ln_b": normal(seed_of(w, 4), (D_MODEL,), 0.0, 0.02),
        "ffn": normal(seed_of(w, 5), (N_PREFILL, D_FF)),
    }


def prefill_bytes(f16_table: bool = False, fused: bool = True) -> dict:
    """Algorithmic bytes of one prefill step: each input read once, each
    output written once.  fused: token+position gather and LayerNorm are one
    kernel that writes both h (the residual stream) and LN(h); unfused: the
    gather writes h and the LayerNorm reads it back."""
    es = 2 if f16_table else 4
    row = D_MODEL * es
    rows_in = N_PREFILL * (row + 4 * D_MODEL) + N_PREFILL * 4 * 2      # table + pos rows, both id vectors
    act = N_PREFILL * D_MODEL * 4                                        # one [512,1024] f32 tensor
    affine = 2 * D_MODEL * 4
    gelu = 2 * N_PREFILL * D_FF * 4
    if fused:
        return {"embed_layer_norm": rows_in + affine + 2 * act, "gelu": gelu}
    return {"gather_pos": rows_in + act, "layer_norm": 2 * act + affine, "gelu": gelu}


QK8_0, Q8_0_BLOCK = 32, 34


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    """float32 [rows, k] -> uint8 [rows, k/32*34] Q8_0 blocks (f16 scale
    d = amax/127, then q = round(x/d) half away from zero).  Builds synthetic
    tables only; what the kernels must reproduce exactly is the dequant."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    b = x.reshape(rows, k // QK8_0, QK8_0)
    d = (np.abs(b).max(axis=2) / np.float32(127.0)).astype(np.float32)
    inv = np.divide(np.float32(1.0), d, out=np.zeros_like(d), where=d != 0)
    v = b * inv[:, :, None]
    q = np.clip(np.trunc(v + np.copysign(np.float32(0.5), v)), -128, 127).astype(np.int8)
    out = np.empty((rows, k // QK8_0, Q8_0_BLOCK), dtype=np.uint8)
    out[:, :, :2] = d.astype(np.float16).view(np.uint8).reshape(rows, k // QK8_0, 2)
    out[:, :, 2:] = q.view(np.uint8)
    return out.reshape(rows, k // QK8_0 * Q8_0_BLOCK)


# ---- workload 1: T3 decode step ------------------------------------------------

DECODE_STEPS, N_HEAD, HEAD_DIM = 30, 16, 64


def decode_inputs(step: int) -> dict:
    """Inputs of decode step `step` (RoPE position = step)."""
    w = 1
    return {
        "x": normal(seed_of(w, 0) + step, (1, D_MODEL)),
        "g": normal(seed_of(w, 1), (D_MODEL,), 1.0, 0.02),
        "q": normal(seed_of(w, 2) + 97 * step, (1, N_HEAD, HEAD_DIM)),
        "k": normal(seed_of(w, 3) + 97 * step, (1, N_HEAD, HEAD_DIM)),
        "pos": np.array([step], dtype=np.int32),
        "gate": normal(seed_of(w, 5) + step, (1, D_FF)),
        "up": normal(seed_of(w, 6) + step, (1, D_FF)),
    }


def decode_bytes() -> dict:
    return {"rms_norm_mul": 3 * D_MODEL * 4, "rope_qk": 4 * N_HEAD * HEAD_DIM * 4, "swiglu": 3 * D_FF * 4}


# ---- workload 5: 64-stream decode, f16 storage -------------------------------

N_STREAMS = 64


def serving_inputs() -> dict:
    w = 5
    return {
        "tab": quantize_q8_0(normal(seed_of(w, 0), (VOCAB, D_MODEL), 0.0, 0.02)),
        "ids": randint(seed_of(w, 1), (N_STREAMS,), 0, VOCAB),
        "x": normal(seed_of(w, 2), (N_STREAMS, D_MODEL)).astype(np.float16),
        "g": normal(seed_of(w, 3), (D_MODEL,), 1.0, 0.02),
        "q": normal(seed_of(w, 4), (N_STREAMS, N_HEAD, HEAD_DIM)).astype(np.float16),
        "pos": randint(seed_of(w, 5), (N_STREAMS,), 0, 2048),
        "k": normal(seed_of(w, 6), (N_STREAMS, N_HEAD, HEAD_DIM)).astype(np.float16),
        "gate": normal(seed_of(w, 7), (N_STREAMS, D_FF)).astype(np.float16),
        "up": normal(seed_of(w, 8), (N_STREAMS, D_FF)).astype(np.float16),
    }


def serving_bytes() -> dict:
    act = N_STREAMS * D_MODEL * 2
    qk = N_STREAMS * N_HEAD * HEAD_DIM * 2
    return {"rms_norm_mul": 2 * act + D_MODEL * 4,
            "rope_qk": 4 * qk + N_STREAMS * 4,
            "swiglu": 3 * N_STREAMS * D_FF * 2,
            "get_rows_q8_0": N_STREAMS * (D_MODEL // QK8_0 * Q8_0_BLOCK) + N_STREAMS * 4 + N_STREAMS * D_MODEL * 4}


# ---- workload 3: CFM estimator ops ----------------------------------------------

CFM_GROUPS, CFM_T, CFM_HEADS = 8, 500, 8


def cfm_inputs() -> dict:
    """GroupNorm inputs in torch order [2, C, 1, T] (ggml ne (T, 1, C, 2)):
    the group statistics run over C/8 channels x T frames of one batch item."""
    w = 3
    return {
        "x256": normal(seed_of(w, 0), (2, 256, 1, CFM_T)),
        "w256": normal(seed_of(w, 1), (1, 256, 1, 1), 1.0, 0.02),
        "b256": normal(seed_of(w, 2), (1, 256, 1, 1), 0.0, 0.02),
        "x512": normal(seed_of(w, 3), (2, 512, 1, CFM_T)),
        "w512": normal(seed_of(w, 4), (1, 512, 1, 1), 1.0, 0.02),
        "b512": normal(seed_of(w, 5), (1, 512, 1, 1), 0.0, 0.02),
        "xa": normal(seed_of(w, 6), (2, CFM_T, CFM_HEADS * HEAD_DIM)),
        "wa": normal(seed_of(w, 7), (CFM_HEADS * HEAD_DIM,), 1.0, 0.02),
        "ba": normal(seed_of(w, 8), (CFM_HEADS * HEAD_DIM,), 0.0, 0.02),
        "pos": np.arange(CFM_T, dtype=np.int32),
    }


def cfm_bytes() -> dict:
    return {"group_norm_mish_256": 2 * 2 * 256 * CFM_T * 4 + 2 * 256 * 4,
            "group_norm_mish_512": 2 * 2 * 512 * CFM_T * 4 + 2 * 512 * 4,
            "layer_norm_rope": 2 * 2 * CFM_T * CFM_HEADS * HEAD_DIM * 4 + 2 * CFM_HEADS * HEAD_DIM * 4}


# ---- workload 4: HiFT activations -----------------------------------------------

HIFT_SHAPES = ((1, 256, 6000), (1, 128, 48000), (1, 64, 120000), (16, 64, 120000))   # (B, C, T)


def snake_alpha(C: int, tensor: int = 1):
    a = uniform_range(seed_of(4, tensor), (C,), 0.5, 1.5)
    return a, (np.float32(1.0) / (a + np.float32(1e-9))).astype(np.float32)


# ---- workload 5: one T3 block's element-wise nodes around its matmuls --------------

def t3_block_inputs() -> dict:
    """The matmul outputs and parameters of one T3 block at prefill size
    (t3.cpp:526-546): attention output projection [512,1024] + out_b, the
    residual h, LN2 w/b, fc output [512,4096] + fc_b, projection output
    [512,1024] + proj_b, the next block's LN1 w/b."""
    w = 7
    N, D, F = N_PREFILL, D_MODEL, D_FF
    return {
        "attn_mm": normal(seed_of(w, 0), (N, D)), "h": normal(seed_of(w, 1), (N, D)),
        "out_b": normal(seed_of(w, 2), (D,), 0.0, 0.02),
        "ln2_w": normal(seed_of(w, 3), (D,), 1.0, 0.02), "ln2_b": normal(seed_of(w, 4), (D,), 0.0, 0.02),
        "fc_mm": normal(seed_of(w, 5), (N, F)), "fc_b": normal(seed_of(w, 6), (F,), 0.0, 0.02),
        "proj_mm": normal(seed_of(w, 7), (N, D)), "proj_b": normal(seed_of(w, 8), (D,), 0.0, 0.02),
        "ln1_w": normal(seed_of(w, 9), (D,), 1.0, 0.02), "ln1_b": normal(seed_of(w, 10), (D,), 0.0, 0.02),
    }


def t3_block_bytes() -> dict:
    """Algorithmic bytes of the three fused launches (each input read once,
    each output written once), and what the ggml nodes they replace move
    when each node reads its inputs and writes its output (vectors aside):
    add-bias, add-residual, norm, mul, add = 11 [N,D] rows per residual
    join; add-bias, gelu = 4 [N,F] rows."""
    N, D, F = N_PREFILL, D_MODEL, D_FF
    act = N * D * 4
    join = 4 * act + 3 * D * 4                 # read a, r; write s, y; out_b/proj_b, w, b
    bias_gelu = 2 * N * F * 4 + F * 4
    return {"residual_ln2": join, "fc_bias_gelu": bias_gelu, "residual_next_ln1": join,
            "ggml_nodes": 2 * 11 * act + 4 * N * F * 4}


# ---- workload 6: the T3 decode step's element-wise nodes, one token -------------
# Chatterbox-Turbo's T3 (t3.h): 24 blocks, width 1024, 16 heads of 64, FFN
# 4096; the speech-token table (6563 rows) and the learned position table
# (8196 rows) are F16 in the shipped GGUF (convert_chatterbox_to_gguf.py:277-290).
T3_LAYERS = 24
T3_HEADS = 16
T3_SPEECH_VOCAB = 6563
T3_POS_ROWS = 8196
T3_MAX_CTX = 1024


def t3_token_inputs(n_layers: int = T3_LAYERS, max_ctx: int = T3_MAX_CTX) -> dict:
    """Tables, per-block parameters and per-block matmul outputs of one T3
    decode step at N_new = 1 (t3.cpp:446-546); per-block arrays are stacked
    [n_layers, width].  kq holds H x max_ctx scores a block: the step with
    n_past uses its first H x (n_past + 1) floats as (H, 1, n_past + 1), the
    contiguous output of mul_mat(K, Q)."""
    w = 6
    L, D, F, H = n_layers, D_MODEL, D_FF, T3_HEADS
    return {
        "speech_emb": normal(seed_of(w, 0), (T3_SPEECH_VOCAB, D), 0.0, 0.02).astype(np.float16),
        "pos_embd": normal(seed_of(w, 1), (T3_POS_ROWS, D), 0.0, 0.02).astype(np.float16),
        "ln1_w": normal(seed_of(w, 2), (L, D), 1.0, 0.02), "ln1_b": normal(seed_of(w, 3), (L, D), 0.0, 0.02),
        "qkv_b": normal(seed_of(w, 4), (L, 3 * D), 0.0, 0.02), "out_b": normal(seed_of(w, 5), (L, D), 0.0, 0.02),
        "ln2_w": normal(seed_of(w, 6), (L, D), 1.0, 0.02), "ln2_b": normal(seed_of(w, 7), (L, D), 0.0, 0.02),
        "fc_b": normal(seed_of(w, 8), (L, F), 0.0, 0.02), "proj_b": normal(seed_of(w, 9), (L, D), 0.0, 0.02),
        "qkv_mm": normal(seed_of(w, 10), (L, 3 * D)), "kq": normal(seed_of(w, 11), (L, H * max_ctx), 0.0, 3.0),
        "out_mm": normal(seed_of(w, 12), (L, D), 0.0, 0.5), "fc_mm": normal(seed_of(w, 13), (L, F)),
        "proj_mm": normal(seed_of(w, 14), (L, D), 0.0, 0.5),
        "out_w": normal(seed_of(w, 15), (D,), 1.0, 0.02), "out_b_final": normal(seed_of(9, 0), (D,), 0.0, 0.02),
    }


def t3_token_bytes(n_layers: int = T3_LAYERS, n_past: int = 0) -> int:
    """Algorithmic bytes of one token's element-wise launches: every input
    read once and every output written once (embedding: two F16 rows in, h
    and LN-1 out; per block: the qkv bias add, the scores, the residual
    joins with their LayerNorms, the fc bias + GELU; vectors counted once)."""
    D, F, H = D_MODEL, D_FF, T3_HEADS
    n_kv = n_past + 1
    emb = 2 * D * 2 + 2 * D * 4 + 2 * D * 4
    per = (3 * D * 4 * 3                      # qkv_mm + qkv_b in, qkv out
           + 2 * H * n_kv * 4                 # scores in, probabilities out
           + (3 * D * 4 + 3 * D * 4 + 2 * D * 4)   # out_mm, h in, out_b; attn_res, ln2 out; ln2 w, b
           + 3 * F * 4                        # fc_mm + fc_b in, gelu out
           + (3 * D * 4 + 3 * D * 4 + 2 * D * 4))  # proj_mm, attn_res, proj_b; h, ln out; ln w, b
    return emb + n_layers * per
