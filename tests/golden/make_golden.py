"""Writes tests/golden/ops_v1.npz: small seeded inputs for every op on the
fused layer-op path with the oracle's outputs, after checking each output
against a float64 closed form (so a fixture cannot silently record an oracle
mistake).  Run from the repository root:

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from chatterbox_amdvulkan_amd import workloads as W  # noqa: E402
from oracle import oracle as O  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ops_v1.npz")


def close64(got, ref, x=None, rtol=1e-6, atol_x=2.0 ** -22, what=""):
    g = np.asarray(got, np.float64)
    r = np.asarray(ref, np.float64)
    bound = rtol * np.abs(r) + (atol_x * np.abs(np.asarray(x, np.float64)) if x is not None else 1e-7)
    assert np.all(np.abs(g - r) <= bound), what


def main():
    f = {}
    # gather: f32, f16 and Q8_0 tables, token + position rows
    tab = W.normal(101, (40, 64), 0.0, 0.02)
    pos = W.normal(102, (40, 64), 0.0, 0.02)
    ids = np.array([0, 39, 7, 7, 21, 3], dtype=np.int32)
    pids = np.arange(6, dtype=np.int32)
    q8 = O.quantize_q8_0(tab)
    f.update(gather_table=tab, gather_pos=pos, gather_ids=ids, gather_pids=pids, gather_q8=q8,
             gather_f32=O.get_rows_add(tab, ids, pos, pids),
             gather_f16=O.get_rows(tab.astype(np.float16), ids),
             gather_q8_out=O.get_rows(q8, ids, q8_0=True))
    assert np.array_equal(f["gather_f32"], tab[ids] + pos[pids])
    blocks = q8.reshape(-1, 34)
    deq = (blocks[:, 2:].view(np.int8).astype(np.float32) *
           blocks[:, :2].copy().view(np.float16).astype(np.float32)).reshape(40, 64)
    assert np.array_equal(f["gather_q8_out"], deq[ids])

    # layer norm + affine, rms norm + gamma
    x = W.normal(103, (8, 256), 0.3, 1.5)
    w = W.normal(104, (256,), 1.0, 0.02)
    b = W.normal(105, (256,), 0.0, 0.02)
    ln = O.layer_norm(x, w, b, 1e-5)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * w + b
    close64(ln, ref, rtol=2e-6, what="ln")
    xr = W.normal(106, (4, 1024))
    g = W.normal(107, (1024,), 1.0, 0.02)
    rms = O.rms_norm_mul(xr, g, 1e-5)
    xrd = xr.astype(np.float64)
    close64(rms, xrd / np.sqrt((xrd ** 2).mean(1, keepdims=True) + 1e-5) * g, rtol=2e-6, what="rms")
    f.update(ln_x=x, ln_w=w, ln_b=b, ln_out=ln, rms_x=xr, rms_g=g, rms_out=rms)

    # rope NEOX and NORMAL
    xq = W.normal(108, (6, 2, 64))
    pq = np.array([0, 1, 5, 100, 1000, 2047], dtype=np.int32)
    f.update(rope_x=xq, rope_pos=pq, rope_neox=O.rope_ext(xq, pq, 64, mode=2), rope_normal=O.rope_ext(xq, pq, 64, mode=0))
    assert np.array_equal(f["rope_neox"][0], xq[0])

    # activations
    xa = np.concatenate([W.normal(109, (997,), 0.0, 3.0),
                         np.array([0.0, -0.0, 10.0, -10.0, 20.0, 21.0, -30.0], dtype=np.float32)])
    f["act_x"] = xa
    xd = xa.astype(np.float64)
    closed = {
        "gelu_erf": (O.GELU_ERF, 0.5 * xd * (1 + np.vectorize(math.erf)(xd / math.sqrt(2)))),
        "silu": (O.SILU, xd / (1 + np.exp(-xd))),
        "mish": (O.MISH, xd * np.tanh(np.where(xd > 20, xd, np.log1p(np.exp(np.minimum(xd, 20)))))),
        "tanh": (O.TANH, np.tanh(xd)),
        "softplus": (O.SOFTPLUS, np.where(xd > 20, xd, np.log1p(np.exp(np.minimum(xd, 20))))),
        "sin": (O.SIN, np.sin(xd)),
    }
    for name, (op, ref) in closed.items():
        out = O.unary(op, xa)
        close64(out, ref, x=xa, rtol=1e-6, what=name)
        f["act_" + name] = out
    f["act_gelu"] = O.unary(O.GELU, xa)
    f["act_leaky"] = O.leaky_relu(xa, 0.1)
    assert np.array_equal(f["act_leaky"], (np.where(xa > 0, xa, 0) + np.float32(0.1) * np.where(xa < 0, xa, 0)).astype(np.float32))
    f["gelu_table"] = O.gelu_table(0)

    # swiglu, snake
    gg, uu = W.normal(110, (2, 512)), W.normal(111, (2, 512))
    f.update(swiglu_g=gg, swiglu_u=uu, swiglu_out=O.swiglu(gg, uu))
    close64(f["swiglu_out"], gg.astype(np.float64) / (1 + np.exp(-gg.astype(np.float64))) * uu, rtol=1e-6, what="swiglu")
    xs = W.normal(112, (50, 16), 0.0, 2.0)
    a = W.uniform_range(113, (16,), 0.5, 1.5)
    ai = (1.0 / (a + np.float32(1e-9))).astype(np.float32)
    sn = O.snake(xs, a, ai)
    close64(sn, xs + (1 / (a.astype(np.float64) + 1e-9)) * np.sin(xs.astype(np.float64) * a) ** 2, x=xs, what="snake")
    f.update(snake_x=xs, snake_a=a, snake_ai=ai, snake_out=sn)

    # group norm + affine (+ mish)
    xg = W.normal(114, (2, 8, 1, 50), 0.5, 2.0)
    wg = W.normal(115, (1, 8, 1, 1), 1.0, 0.05)
    bg = W.normal(116, (1, 8, 1, 1), 0.0, 0.05)
    gn = O.group_norm_affine(xg, 4, 1e-5, wg, bg, False)
    xgd = xg.astype(np.float64).reshape(2, 4, -1)
    ref = ((xgd - xgd.mean(-1, keepdims=True)) / np.sqrt(xgd.var(-1, keepdims=True) + 1e-5)).reshape(xg.shape) * wg + bg
    close64(gn, ref, rtol=3e-6, what="gn")
    f.update(gn_x=xg, gn_w=wg, gn_b=bg, gn_out=gn, gn_mish=O.group_norm_affine(xg, 4, 1e-5, wg, bg, True))

    # attention-score epilogue: scale -> diag_mask_inf(n_past) -> soft_max
    xs = W.normal(117, (3, 5, 40), 0.0, 6.0)
    sm = O.scale_diag_mask_soft_max(xs, 0.125, 2)
    t = xs.astype(np.float64) * 0.125
    t = np.where(np.arange(40)[None, None, :] > 2 + np.arange(5)[None, :, None], -np.inf, t)
    e = np.exp(t - t.max(-1, keepdims=True))
    close64(sm, e / e.sum(-1, keepdims=True), rtol=1e-6, what="softmax")
    f.update(sm_x=xs, sm_out=sm)

    # LayerNorm + affine, then NEOX RoPE of the normalised row viewed as heads
    xl = W.normal(118, (2, 6, 128), 0.2, 1.5)
    wl = W.normal(119, (128,), 1.0, 0.05)
    bl = W.normal(120, (128,), 0.0, 0.05)
    pl = np.array([0, 1, 2, 3, 5, 8], dtype=np.int32)
    lr = O.rope_ext(O.layer_norm(xl, wl, bl, 1e-5).reshape(2, 6, 2, 64), pl, 64, mode=2).reshape(xl.shape)
    xd = xl.astype(np.float64)
    n64 = ((xd - xd.mean(-1, keepdims=True)) / np.sqrt(xd.var(-1, keepdims=True) + 1e-5) * wl + bl).reshape(2, 6, 2, 64)
    th = pl[None, :, None, None].astype(np.float64) * 10000.0 ** (-np.arange(32) / 32.0)
    a0, a1 = n64[..., :32], n64[..., 32:]
    ref = np.concatenate([a0 * np.cos(th) - a1 * np.sin(th), a0 * np.sin(th) + a1 * np.cos(th)], -1).reshape(xl.shape)
    close64(lr, ref, rtol=3e-6, what="ln+rope")
    f.update(lnr_x=xl, lnr_w=wl, lnr_b=bl, lnr_pos=pl, lnr_out=lr)

    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT}: {len(f)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
