"""The element-wise nodes of one S3 speech-tokenizer encoder call --
S3Encoder::forward (chatterbox-cpp/src/s3enc.cpp:124-290) -- as that
builder emits them, with each matmul's output, the two front-end convs'
outputs, the FSMN branch's depthwise conv (with its transposes) and the
layout copies around the attention given as device tensors: the
caller-side list that libcbxops' node-list executor (cbx_graph_*) plans and
runs once per call.

Per call the reference builds (ggml node order; [..] the given outputs):
  front: [conv1, stride 2] add_bias_td -> gelu_erf, [conv2, stride 2]
    add_bias_td -> gelu_erf, on the convs' time-major (T, C) layout, the
    bias viewed as (1, C)                                     (:170-178)
  [transposed to (D, T_tok)]                                  (:184)
  per layer (6 of them; D 1280, 20 heads of 64):              (:193-275)
    layer_norm(x) -> [q] add(q_b), [k], [v] add(v_b); q and k viewed as
    (64, 20, T_tok) -> rope_ext (NEOX, base 10000) each
    [FSMN: depthwise conv of v] add(fsmn, v)
    [scores] scale(1/8) -> soft_max
    [out] add(out_b) -> add(., fsmn + v) -> add(x, .)
    layer_norm -> [fc] add(fc_b) -> gelu_erf -> [proj] add(proj_b) ->
    add(x, .)
Over T_mel mel frames the layers run T_tok = T_mel / 4 tokens (25 a
second of audio at T_mel = 100 a second).  With the reference's sizes a
call holds 13 LayerNorms, 12 RoPEs, 6 softmaxes and 8 GELU-erfs.

Tensors are torch tensors laid out as ggml's (torch shape = reversed ne):
a (D, T) activation is torch (T, D), the front convs' (T, C) outputs torch
(C, T), the scores (T_k, T_q, H) torch (H, T, T).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import cbxops as C
from . import workloads as W
from .ggml_nodes import NodeList

N_STATE, N_HEAD, HEAD_DIM, N_LAYER, EPS = 1280, 20, 64, 6, 1e-5
ROPE_BASE, ROPE_MAX = 10000.0, 2048


class S3EncoderCall:
    """One encoder call's node list over T_mel mel frames (T_tok = T_mel / 4
    tokens).  device=True: every tensor on the GPU, weights and given
    outputs random (seeded), the RoPE table built (close() releases it);
    device=False: host tensors for planning only."""

    def __init__(self, T_mel: int, seed: int = 0, n_layer: int = N_LAYER, device: bool = True):
        self.T_mel, self.n_layer, self.device = int(T_mel), int(n_layer), bool(device)
        self.T1 = (self.T_mel - 1) // 2 + 1            # conv1: K 3, stride 2, padding 1
        self.T_tok = (self.T1 - 1) // 2 + 1            # conv2: the same
        self._seed = int(seed) * 1000
        dev = "cuda" if device else "cpu"
        nan = float("nan")
        self.b = NodeList(lambda shape, dtype: torch.full(shape, nan, dtype=dtype, device=dev))
        self.keep: list[int] = []      # read by a given op, or the output
        self.given: dict[str, int] = {}
        self.rope = C.RopeCache(HEAD_DIM, mode=2, n_ctx_orig=ROPE_MAX, freq_base=ROPE_BASE,
                                n_pos=ROPE_MAX) if device else None
        self._build()

    # ---- tensors ----------------------------------------------------------------

    def _next(self) -> int:
        self._seed += 1
        return self._seed

    def _t(self, arr: np.ndarray) -> int:
        if not self.device:
            return self.b.t(torch.empty(arr.shape, dtype=torch.from_numpy(arr[:0]).dtype))
        return self.b.t(torch.from_numpy(np.ascontiguousarray(arr)).cuda())

    def _rand(self, shape, mean=0.0, std=1.0) -> int:
        if not self.device:
            return self.b.t(torch.empty(shape, dtype=torch.float32))
        return self._t(W.normal(self._next(), shape, mean, std))

    def _given(self, name, shape, std=1.0) -> int:
        i = self._rand(shape, 0.0, std)
        self.given[name] = i
        return i

    def _keep(self, i: int) -> int:
        self.keep.append(i)
        return i

    def _ln(self):
        return self._rand((N_STATE,), 1.0, 0.05), self._rand((N_STATE,), 0.0, 0.05)

    def _bias(self, n):
        return self._rand((n,), 0.0, 0.1)

    # ---- blocks -----------------------------------------------------------------

    def _front(self, name, T):
        """[conv] add_bias_td -> gelu_erf on the (T, C) layout (torch (C, T))."""
        b = self.b
        y = self._given(name, (N_STATE, T))
        bias = self._bias(N_STATE)
        bv = b.node_view(b.at(bias).reshape(N_STATE, 1), bias)
        return self._keep(b.unary(b.add(y, bv), C.GELU_ERF))

    def _layer(self, x, il, ln_in):
        b, T = self.b, self.T_tok
        if ln_in is None:           # the first layer's LayerNorm stands alone
            w1, b1 = self._ln()
            x_n = self._keep(b.layer_norm(x, w1, b1, EPS))
        else:
            x_n = ln_in
        q = b.add(self._given(f"l{il}.q", (T, N_STATE)), self._bias(N_STATE))
        k = self._given(f"l{il}.k", (T, N_STATE))
        v = self._keep(b.add(self._given(f"l{il}.v", (T, N_STATE)), self._bias(N_STATE)))
        qh = b.node_view(b.at(q).view(T, N_HEAD, HEAD_DIM), q)
        kh = b.node_view(b.at(k).view(T, N_HEAD, HEAD_DIM), k)
        qr = self._keep(b.node_new(C.GOP_ROPE, (T, N_HEAD, HEAD_DIM), (qh, self.pos), rope=self.rope))
        kr = self._keep(b.node_new(C.GOP_ROPE, (T, N_HEAD, HEAD_DIM), (kh, self.pos), rope=self.rope))
        fsmn = b.add(self._given(f"l{il}.fsmn", (T, N_STATE)), v)
        scores = self._given(f"l{il}.scores", (N_HEAD, T, T), std=3.0)
        self._keep(b.soft_max(b.scale(scores, 1.0 / math.sqrt(HEAD_DIM))))
        attn = b.add(b.add(self._given(f"l{il}.out", (T, N_STATE)), self._bias(N_STATE)), fsmn)
        x = b.add(x, attn)
        w2, b2 = self._ln()
        x_n2 = self._keep(b.layer_norm(x, w2, b2, EPS))
        self._keep(b.unary(b.add(self._given(f"l{il}.fc", (T, 4 * N_STATE)), self._bias(4 * N_STATE)), C.GELU_ERF))
        h = b.add(self._given(f"l{il}.proj", (T, N_STATE)), self._bias(N_STATE))
        return b.add(x, h), (qr, kr, x_n2)

    def _build(self):
        self._front("conv1", self.T1)
        self._front("conv2", self.T_tok)
        x = self._given("x", (self.T_tok, N_STATE))    # conv2's output transposed to (D, T_tok)
        self.pos = self._t(np.arange(self.T_tok, dtype=np.int32))
        ln_next = None
        for il in range(self.n_layer):
            x, _ = self._layer(x, il, ln_next)
            if il + 1 < self.n_layer:
                w1, b1 = self._ln()
                ln_next = self._keep(self.b.layer_norm(x, w1, b1, EPS))
        self.out = self._keep(x)

    # ---- running ----------------------------------------------------------------

    @property
    def graph(self) -> C.Graph:
        return self.b.g

    def plan(self):
        return self.graph.plan(self.keep)

    def close(self):
        if self.rope is not None:
            self.rope.close()
            self.rope = None
