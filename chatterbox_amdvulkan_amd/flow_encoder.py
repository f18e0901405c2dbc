"""The element-wise nodes of one flow-encoder call --
FlowEncoder::forward_with_stages (chatterbox-cpp/src/flow_encoder.cpp:
537-700) -- as that builder emits them, with each matmul's output, the
pre-lookahead and up-layer convs' outputs (with their pads) and the layout
copies around the attention (permutes, the relative-position shift) given as
device tensors: the caller-side list that libcbxops' node-list executor
(cbx_graph_*) plans and runs once per call.

Per call the reference builds (ggml node order; [..] the given outputs):
  the speech-token embedding: get_rows of the (512, 6561) table  (:588-590)
  linear_no_subsample: [lin] add(b) -> layer_norm (eps 1e-5) -> scale(sqrt 512)
                                                                 (:409-418)
  pre_lookahead (:435-477): [conv1] add(b as (1, C)) -> leaky_relu(0.01),
    [pad, conv2] add(b as (1, C)), [transposed] add(., x)
  6 conformer blocks over T tokens (:306-406): layer_norm (eps 1e-12) ->
    [v] add(b), [k] add(b), [q] add(b) -> viewed as (64, 8, T) -> add(.,
    pos_bias_u as (64, 8, 1)), add(., pos_bias_v); [AC, BD shifted] add ->
    scale(1/8) -> soft_max; [attn, out] add(b) -> add(x, .) -> layer_norm ->
    [w1] add(b) -> silu -> [w2] add(b) -> add(x, .)
    (v, k, q: the order ggml's depth-first graph build visits them in, from
    the attention product V_trans x scores, whose scores read k's and q's
    products)
  up_layer (:487-535): [nearest x2, pad, conv] add(b as (1, C)) [transposed]
  linear_no_subsample again, 4 conformer blocks over 2T, layer_norm
  (after_norm, eps 1e-5), [encoder_proj] add(b)                 (:632-660)
Over T speech tokens (25 a second) the up blocks run 2T frames, the CFM
decoder's T_mel.

Tensors are torch tensors laid out as ggml's (torch shape = reversed ne):
a (D, T) activation is torch (T, D), the convs' time-major (T, C) outputs
torch (C, T), the scores (T_k, T_q, H) torch (H, T, T).
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import cbxops as C
from . import workloads as W
from .ggml_nodes import NodeList

VOCAB, D, N_HEAD, HEAD_DIM, FF = 6561, 512, 8, 64, 2048
N_BLOCKS, N_UP_BLOCKS, D_OUT = 6, 4, 80
LN_EPS, LN_EPS_ATTN = 1e-5, 1e-12


class FlowEncoderCall:
    """One flow-encoder call's node list over T speech tokens.  device=True:
    every tensor on the GPU, the table, weights and given outputs random
    (seeded); device=False: host tensors for planning only."""

    def __init__(self, T: int, seed: int = 0, n_blocks: int = N_BLOCKS, n_up_blocks: int = N_UP_BLOCKS,
                 device: bool = True):
        self.T, self.device = int(T), bool(device)
        self.n_blocks, self.n_up_blocks = int(n_blocks), int(n_up_blocks)
        self._seed = int(seed) * 1000
        dev = "cuda" if device else "cpu"
        nan = float("nan")
        self.b = NodeList(lambda shape, dtype: torch.full(shape, nan, dtype=dtype, device=dev))
        self.keep: list[int] = []      # read by a given op, or the output
        self.given: dict[str, int] = {}
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

    def _ln(self, x, eps):
        w, bb = self._rand((D,), 1.0, 0.05), self._rand((D,), 0.0, 0.05)
        return self.b.layer_norm(x, w, bb, eps)

    def _bias(self, n):
        return self._rand((n,), 0.0, 0.1)

    def _bias_tc(self, y):
        """add(y, b viewed as (1, C)) on a conv's time-major (T, C) output."""
        b = self.b
        bias = self._bias(D)
        return b.add(y, b.node_view(b.at(bias).reshape(D, 1), bias))

    # ---- blocks -----------------------------------------------------------------

    def _linear_no_subsample(self, x, name, T):
        """[lin] add(b) -> layer_norm -> scale(sqrt D) (flow_encoder.cpp:409-418)."""
        b = self.b
        y = b.add(self._given(name, (T, D)), self._bias(D))
        return self._keep(b.scale(self._ln(y, LN_EPS), math.sqrt(D)))

    def _block(self, x, name, T):
        """conformer_block_forward (flow_encoder.cpp:306-406) after its first
        LayerNorm, which the caller adds to the list (after the add before
        it, so the two join)."""
        b = self.b
        self._keep(b.add(self._given(f"{name}.v", (T, D)), self._bias(D)))
        self._keep(b.add(self._given(f"{name}.k", (T, D)), self._bias(D)))
        q = b.add(self._given(f"{name}.q", (T, D)), self._bias(D))
        qh = b.node_view(b.at(q).view(T, N_HEAD, HEAD_DIM), q)
        for pb in ("u", "v"):
            bias = self._rand((N_HEAD, HEAD_DIM), 0.0, 0.1)
            bv = b.node_view(b.at(bias).reshape(1, N_HEAD, HEAD_DIM), bias)
            self._keep(b.add(qh, bv))
        ac = self._given(f"{name}.ac", (N_HEAD, T, T), std=3.0)
        bd = self._given(f"{name}.bd_shifted", (N_HEAD, T, T), std=3.0)
        self._keep(b.soft_max(b.scale(b.add(ac, bd), 1.0 / math.sqrt(HEAD_DIM))))
        x = b.add(x, b.add(self._given(f"{name}.out", (T, D)), self._bias(D)))
        self._keep(self._ln(x, LN_EPS_ATTN))
        self._keep(b.unary(b.add(self._given(f"{name}.w1", (T, FF)), self._bias(FF)), C.SILU))
        return b.add(x, b.add(self._given(f"{name}.w2", (T, D)), self._bias(D)))

    def _stack(self, x, prefix, n, T, last_eps):
        """n conformer blocks; each block's first LayerNorm follows the add
        before it, and the stack's last add is followed by a LayerNorm of
        eps last_eps (the next stack's first, or after_norm)."""
        for i in range(n):
            self._keep(self._ln(x, LN_EPS_ATTN))
            x = self._block(x, f"{prefix}{i}", T)
        if last_eps:
            self._keep(self._ln(x, last_eps))
        return x

    def _build(self):
        b, T = self.b, self.T
        table = self._rand((VOCAB, D), 0.0, 1.0)
        ids = self._t(W.randint(self._next(), (T,), 0, VOCAB).astype(np.int32))
        x = self._keep(b.node_new(C.GOP_GET_ROWS, (T, D), (table, ids)))
        x = self._linear_no_subsample(x, "embed_lin", T)
        # pre_lookahead
        self._keep(b.leaky(self._bias_tc(self._given("prelook.conv1", (D, T))), 0.01))
        self._keep(self._bias_tc(self._given("prelook.conv2", (D, T))))
        x = b.add(self._given("prelook.out_transposed", (T, D)), x)
        x = self._stack(x, "enc", self.n_blocks, T, None)
        self.x_enc = self._keep(x)
        # up_layer, up_embed, the up blocks, after_norm, encoder_proj
        self._keep(self._bias_tc(self._given("up.conv", (D, 2 * T))))
        x = self._linear_no_subsample(self._given("up.out_transposed", (2 * T, D)), "up_embed_lin", 2 * T)
        self._stack(x, "up_enc", self.n_up_blocks, 2 * T, LN_EPS)
        self.out = self._keep(b.add(self._given("encoder_proj", (2 * T, D_OUT)), self._bias(D_OUT)))

    # ---- running ----------------------------------------------------------------

    @property
    def graph(self) -> C.Graph:
        return self.b.g

    def plan(self):
        return self.graph.plan(self.keep)

    def close(self):
        pass
