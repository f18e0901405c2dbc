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
