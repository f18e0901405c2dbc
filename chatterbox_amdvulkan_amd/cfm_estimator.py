"""The element-wise nodes of one CFM estimator call -- the flow decoder's
U-Net, CFMDecoder::estimator_forward_with_stages
(chatterbox-cpp/src/cfm_decoder.cpp:395-558) -- as that builder emits them,
each matmul's output given as a device tensor and the causal convs run by
the library: the caller-side list that libcbxops' node-list executor
(cbx_graph_*) plans and runs, once per flow step.

Per call the reference builds (ggml node order; matmuls left out, [..] the
given outputs):
  time embedding, for t and r: [l1] add(b) -> silu, [l2] add(b); concat
    (the mixer's input)                                        (:463-477)
  pack: concat(x, mu), concat(., spks), concat(., cond)        (:480-491)
  down: resnet 320 -> 256, n_tr transformers, mul(h, mask) -> causal conv
                                                               (:494-513)
  mid, n_mid times: resnet 256 -> 256, n_tr transformers       (:515-526)
  up: concat(h, skip), resnet 512 -> 256, n_tr transformers, mul(h, mask)
    -> causal conv                                             (:528-544)
  final: causal_block1d, mul(h, mask) -> [final_proj] add(b) -> mul(mask)
                                                               (:546-557)
  resnet (causal_resnet_block1d, :152-179): causal_block1d, mish(t_mix) ->
    [mlp] add(b) -> add(h, .), causal_block1d, mul(x, mask) -> [res_conv]
    add(b) -> add(h, .)
  transformer (basic_transformer_block, :190-245): layer_norm -> [q, k, v,
    scores] scale -> soft_max -> [attn, to_out] add(b) -> add(x, .) ->
    layer_norm -> [ff.0] add(b) -> gelu_erf -> [ff.2] add(b) -> add(x, .)
  causal_block1d (:133-149): mul(x, mask) -> causal conv (+ bias) ->
    layer_norm -> mish -> mul(mask)

The repeat of spks over the frames (ggml_repeat, :482-485) is given: the
library has no repeat.  With the reference's sizes (n_mid 12, n_tr 4) a
call holds 14 resnet blocks (29 causal_block1d with the final block) and 56
transformer blocks (112 LayerNorms, 56 bias + gelu_erf).

Tensors are torch tensors laid out as ggml's (torch shape = reversed ne): a
(C, T) activation is torch (T, C), the (1, T) mask torch (T, 1), the
scores (T_k, T_q, H) torch (H, T, T).
"""
from __future__ import annotations

import math

import torch

from . import cbxops as C
from .ggml_nodes import NodeList

C_IN, C_MID, C_OUT, T_EMB_IN, D_T, SKIP_IN = 320, 256, 80, 320, 1024, 512
N_HEADS, HEAD_DIM, FF_HIDDEN = 8, 64, 1024
N_MID, N_TR, EPS = 12, 4, 1e-5

PLAN_W = 0x1000   # the conv weights' stand-in when the list is only planned (non-null)


class CFMEstimator:
    """One estimator call's node list over T frames.  device=True: every
    tensor on the GPU, weights and given matmul outputs random (seeded),
    conv weights prepared (close() releases them); device=False: host
    tensors for planning only."""

    def __init__(self, T: int, seed: int = 0, n_mid: int = N_MID, n_tr: int = N_TR, device: bool = True,
                 mask_tail: int = 0):
        self.T, self.n_mid, self.n_tr, self.device = int(T), int(n_mid), int(n_tr), bool(device)
        self._gen = torch.Generator(device="cuda" if device else "cpu")
        self._gen.manual_seed(int(seed))
        dev = "cuda" if device else "cpu"
        nan = float("nan")
        self.b = NodeList(lambda shape, dtype: torch.full(shape, nan, dtype=dtype, device=dev))
        self.keep: list[int] = []      # read by a given matmul, or the output
        self.given: dict[str, int] = {}
        self.convs: list = []
        self._build(int(mask_tail))

    # ---- tensors ----------------------------------------------------------------

    def _rand(self, shape, mean=0.0, std=1.0) -> torch.Tensor:
        if not self.device:
            return torch.empty(shape, dtype=torch.float32)
        return torch.randn(shape, generator=self._gen, device="cuda", dtype=torch.float32) * std + mean

    def _w(self, shape, mean=0.0, std=1.0) -> int:
        return self.b.t(self._rand(shape, mean, std))

    def _given(self, name, shape, std=1.0) -> int:
        i = self._w(shape, 0.0, std)
        self.given[name] = i
        return i

    def _conv(self, c_out, c_in, k=3):
        w = self._w((c_out, c_in, k), 0.0, 1.0 / math.sqrt(c_in * k))
        bias = self._w((c_out,), 0.0, 0.1)
        if self.device:
            cw = C.Conv1dWeights(self.b.at(w))
            self.convs.append(cw)
        else:
            cw = PLAN_W
        return w, bias, cw

    def _ln(self, c):
        return self._w((c,), 1.0, 0.05), self._w((c,), 0.0, 0.05)

    def _keep(self, i: int) -> int:
        self.keep.append(i)
        return i

    # ---- blocks -----------------------------------------------------------------

    def _causal_block(self, x, c_in, c_out):
        w, bias, cw = self._conv(c_out, c_in)
        lw, lb = self._ln(c_out)
        return self.b.causal_block(x, self.mask, w, bias, lw, lb, cw, EPS)

    def _resnet(self, x, c_in, c_out, name):
        b = self.b
        h = self._causal_block(x, c_in, c_out)
        tm = self._keep(b.mish(self.t_mix))
        mlp = self._given(f"{name}.mlp", (c_out,))
        tmb = b.add(mlp, self._w((c_out,), 0.0, 0.1))
        tmv = b.node_view(b.at(tmb).reshape(1, c_out), tmb)
        h = b.add(h, tmv)
        h = self._causal_block(h, c_out, c_out)
        self._keep(b.mul(x, self.mask))
        res = self._given(f"{name}.res", (self.T, c_out))
        sc = b.add(res, self._w((c_out,), 0.0, 0.1))
        return b.add(h, sc)

    def _transformer(self, x, name):
        b, T = self.b, self.T
        w1, b1 = self._ln(C_MID)
        self._keep(b.layer_norm(x, w1, b1, EPS))
        scores = self._given(f"{name}.scores", (N_HEADS, T, T), std=3.0)
        self._keep(b.soft_max(b.scale(scores, 1.0 / math.sqrt(HEAD_DIM))))
        a_out = self._given(f"{name}.to_out", (T, C_MID))
        x = b.add(x, b.add(a_out, self._w((C_MID,), 0.0, 0.1)))
        w3, b3 = self._ln(C_MID)
        self._keep(b.layer_norm(x, w3, b3, EPS))
        ffp = self._given(f"{name}.ff0", (T, FF_HIDDEN))
        self._keep(b.unary(b.add(ffp, self._w((FF_HIDDEN,), 0.0, 0.1)), C.GELU_ERF))
        ff2 = self._given(f"{name}.ff2", (T, C_MID))
        return b.add(x, b.add(ff2, self._w((C_MID,), 0.0, 0.1)))

    def _stack(self, h, name):
        for i in range(self.n_tr):
            h = self._transformer(h, f"{name}.tr{i}")
        return h

    def _time_mlp(self, name):
        b = self.b
        l1 = self._given(f"{name}.l1", (D_T,))
        self._keep(b.unary(b.add(l1, self._w((D_T,), 0.0, 0.1)), C.SILU))
        l2 = self._given(f"{name}.l2", (D_T,))
        return b.add(l2, self._w((D_T,), 0.0, 0.1))

    def _build(self, mask_tail):
        b, T = self.b, self.T
        m = self._rand((T, 1))
        if self.device:
            m.fill_(1.0)
            if mask_tail:
                m[T - mask_tail:] = 0.0
        self.mask = b.t(m)
        # time embedding (the mixer's matmul output t_mix is given)
        t_emb, r_emb = self._time_mlp("t"), self._time_mlp("r")
        self._keep(b.concat(t_emb, r_emb, 0))
        self.t_mix = self._given("t_mix", (D_T,))
        # pack [x, mu, spks over the frames, cond] along the channels
        x_in, mu_in = self._given("x", (T, C_OUT)), self._given("mu", (T, C_OUT))
        spks, cond = self._given("spks_repeated", (T, C_OUT)), self._given("cond", (T, C_OUT))
        packed = b.concat(b.concat(b.concat(x_in, mu_in, 0), spks, 0), cond, 0)
        # down
        h = self._stack(self._resnet(packed, C_IN, C_MID, "down"), "down")
        skip = h
        w, bias, cw = self._conv(C_MID, C_MID)
        h = b.causal_conv1d(b.mul(h, self.mask), w, bias, cw)
        # mid
        for i in range(self.n_mid):
            h = self._stack(self._resnet(h, C_MID, C_MID, f"mid{i}"), f"mid{i}")
        # up
        h = self._resnet(b.concat(h, skip, 0), SKIP_IN, C_MID, "up")
        h = self._stack(h, "up")
        w, bias, cw = self._conv(C_MID, C_MID)
        h = b.causal_conv1d(b.mul(h, self.mask), w, bias, cw)
        # final_block, final_proj
        h = self._causal_block(h, C_MID, C_MID)
        self._keep(b.mul(h, self.mask))
        fp = self._given("final_proj", (T, C_OUT))
        self.out = self._keep(b.mul(b.add(fp, self._w((C_OUT,), 0.0, 0.1)), self.mask))

    # ---- running ----------------------------------------------------------------

    @property
    def graph(self) -> C.Graph:
        return self.b.g

    def plan(self):
        return self.graph.plan(self.keep)

    def close(self):
        for cw in self.convs:
            cw.close()
        self.convs = []
