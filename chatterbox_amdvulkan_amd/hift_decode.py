"""The nodes of one HiFT vocoder decode -- HiFTVocoder::decode_with_stages
(chatterbox-cpp/src/hift_vocoder.cpp:613-749), the graph between the host
STFT of the source and the host iSTFT -- as that builder emits them, the mel
spectrogram and the source STFT given as device tensors: the caller-side
list that libcbxops' node-list executor (cbx_graph_*) plans and runs once
per decode.

Per decode the reference builds (ggml node order):
  conv_pre: conv1d_CT 80 -> 512, K 7, padding 3, + bias          (:673)
  stage i = 0, 1, 2 (C = 256, 128, 64; upsampling u = 8, 5, 3; K 16, 11, 7):
    leaky_relu(0.1) -> conv_transpose1d_CT, padding (K - u) / 2, + bias
                                                                 (:686-687)
    stage 2 only: the reflection pad of one frame on the left -- a view of
      frame 1 -> cont -> concat(frame, x) along the frames       (:694-707)
    source_downs[i]: conv1d_CT of the source STFT, 18 -> C, stride 15, 3, 1
      (K 30, 6, 1 and padding 7, 1, 0: the sizes that give the stage's
      frame count), + bias                                       (:710-714)
    source_resblocks[i] (kernel 7, 7, 11)                        (:716-717)
    add(x, source)                                               (:723)
    the three resblocks (kernels 3, 7, 11) on x, added in order, then
      scale(1/3)                                                 (:731-736)
  resblock (resblock_forward, :119-138): three layers at dilation 1, 3, 5:
    snake -> conv1d_CT (K, dilation d) + bias -> snake -> conv1d_CT (K) +
    bias -> add(x, .)
  conv_post: leaky_relu(0.01) -> conv1d_CT 64 -> 18, K 7, padding 3, + bias
                                                                 (:748-749)
Over T_mel mel frames the stages run 8, 40 and 120 T_mel frames (one more
after the pad), the source STFT has 120 T_mel + 1 frames (a hop of 4 on
480 T_mel samples, :478), and a decode holds 77 conv1d_CT (72 with a Snake
prologue: the 72 snakes of a decode) and 3 conv_transpose1d_CT.

Each conv chain's parameters are recorded in `conv_ref`, keyed by the
tensor the chain's launch writes last (for a layer's second conv, the
residual add), so a test can recompute every launch from its inputs.

Tensors are torch tensors laid out as ggml's (torch shape = reversed ne): a
(C, T) activation is torch (T, C); conv1d weights torch [C_out, C_in, K],
conv_transpose1d weights torch [C_in, C_out, K].
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import cbxops as C
from . import workloads as W
from .ggml_nodes import NodeList

MEL, BASE, STFT_CH = 80, 512, 18
UP_STRIDES, UP_KERNELS = (8, 5, 3), (16, 11, 7)
RESBLOCK_KERNELS = (3, 7, 11)
SRC_STRIDES, SRC_KERNELS = (15, 3, 1), (7, 7, 11)
DILATIONS = (1, 3, 5)
LRELU, LRELU_POST = 0.1, 0.01
HOP, UPSAMPLE = 4, 480

PLAN_W = 0x1000   # the conv weights' stand-in when the list is only planned (non-null)


def src_down_shape(stride: int) -> tuple:
    """(K, padding) of source_downs for a stride: K 2s, padding s / 2; a 1x1
    conv at stride 1."""
    return (1, 0) if stride == 1 else (2 * stride, stride // 2)


class HiFTDecode:
    """One decode's node list over T_mel mel frames.  device=True: every
    tensor on the GPU, inputs and weights random (seeded), conv weights
    prepared (close() releases them); device=False: host tensors for
    planning only."""

    def __init__(self, T_mel: int, seed: int = 0, device: bool = True):
        self.T_mel, self.device = int(T_mel), bool(device)
        self._seed = int(seed) * 1000
        dev = "cuda" if device else "cpu"
        nan = float("nan")
        self.b = NodeList(lambda shape, dtype: torch.full(shape, nan, dtype=dtype, device=dev))
        self.keep: list[int] = []       # stage outputs the reference marks, and the output
        self.convs: list = []
        self.stage_frames: list[int] = []
        self.conv_ref: dict[int, dict] = {}
        self._build()

    # ---- tensors ----------------------------------------------------------------

    def _next(self) -> int:
        self._seed += 1
        return self._seed

    def _host(self, arr: np.ndarray) -> int:
        if not self.device:
            return self.b.t(torch.empty(arr.shape, dtype=torch.float32))
        return self.b.t(torch.from_numpy(np.ascontiguousarray(arr)).cuda())

    def _rand(self, shape, mean=0.0, std=1.0) -> int:
        if not self.device:
            return self.b.t(torch.empty(shape, dtype=torch.float32))
        return self._host(W.normal(self._next(), shape, mean, std))

    def _conv(self, c_out, c_in, k, transposed_stride=0):
        fan = c_in * k / (transposed_stride or 1)
        shape = (c_in, c_out, k) if transposed_stride else (c_out, c_in, k)
        w = self._rand(shape, 0.0, 1.0 / math.sqrt(fan))
        bias = self._rand((c_out,), 0.0, 0.1)
        if self.device:
            cw = C.Conv1dWeights(self.b.at(w), transpose_stride=transposed_stride or None)
            self.convs.append(cw)
        else:
            cw = PLAN_W
        return w, bias, cw

    def _alpha(self, c):
        if not self.device:
            return self._rand((c,)), self._rand((c,))
        a, ai = W.snake_alpha(c, self._next())
        return self._host(a), self._host(ai)

    def _keep(self, i: int) -> int:
        self.keep.append(i)
        return i

    # ---- blocks -----------------------------------------------------------------

    def _conv1d(self, x, w, bias, cw, stride, pad, dil, pro=None, alpha=None, slope=0.0, res=None):
        """conv1d_CT of x with an optional snake / leaky_relu before it and
        a residual add after it, recorded in conv_ref."""
        b = self.b
        h = b.snake(x, *alpha) if pro == "snake" else b.leaky(x, slope) if pro == "leaky" else x
        y = b.conv1d(h, w, bias, stride, pad, dil, cw)
        if res is not None:
            y = b.add(res, y)
        self.conv_ref[y] = dict(x=x, w=w, bias=bias, stride=stride, pad=pad, dil=dil, pro=pro, alpha=alpha,
                                slope=slope, res=res)
        return y

    def _resblock(self, x: int, c: int, k: int) -> int:
        """resblock_forward: per layer snake -> conv (dilation d) -> snake ->
        conv -> add(x, .)"""
        for d in DILATIONS:
            a1 = self._alpha(c)
            w1, b1, cw1 = self._conv(c, c, k)
            a2 = self._alpha(c)
            w2, b2, cw2 = self._conv(c, c, k)
            h = self._conv1d(x, w1, b1, cw1, 1, (k - 1) // 2 * d, d, "snake", a1)
            x = self._conv1d(h, w2, b2, cw2, 1, (k - 1) // 2, 1, "snake", a2, res=x)
        return x

    def _build(self):
        b, T = self.b, self.T_mel
        self.mel = self._rand((T, MEL))
        self.stft = self._rand((UPSAMPLE * T // HOP + 1, STFT_CH))
        w, bias, cw = self._conv(BASE, MEL, 7)
        x = self._keep(self._conv1d(self.mel, w, bias, cw, 1, 3, 1))              # after_conv_pre
        for i in range(3):
            c_out, u, k = BASE >> (i + 1), UP_STRIDES[i], UP_KERNELS[i]
            w, bias, cw = self._conv(c_out, BASE >> i, k, transposed_stride=u)
            y = b.conv_transpose1d(b.leaky(x, LRELU), w, bias, u, (k - u) // 2, cw)
            self.conv_ref[y] = dict(x=x, w=w, bias=bias, stride=u, pad=(k - u) // 2, slope=LRELU, transposed=True)
            x = self._keep(y)                                                     # after_ups
            if i == 2:
                col1 = b.node_view(b.at(x)[1:2], x)
                col1c = b.node_new(C.GOP_CPY, b.shape(col1), (col1,))
                x = self.padded = self._keep(b.concat(col1c, x, 1))               # after_refl_pad
            ks, pad = src_down_shape(SRC_STRIDES[i])
            w, bias, cw = self._conv(c_out, STFT_CH, ks)
            si = self._conv1d(self.stft, w, bias, cw, SRC_STRIDES[i], pad, 1)
            si = self._keep(self._resblock(si, c_out, SRC_KERNELS[i]))            # after_src_rb
            x = self._keep(b.add(x, si))                                          # after_src_add
            total = None
            for j in range(3):
                r = self._resblock(x, c_out, RESBLOCK_KERNELS[j])
                total = r if total is None else b.add(total, r)
            x = self._keep(b.scale(total, 1.0 / 3.0))                            # after_rb_avg
            self.stage_frames.append(b.shape(x)[0])
        w, bias, cw = self._conv(STFT_CH, BASE >> 3, 7)
        self.out = self._keep(self._conv1d(x, w, bias, cw, 1, 3, 1, "leaky", slope=LRELU_POST))   # after_conv_post

    # ---- running ----------------------------------------------------------------

    @property
    def graph(self) -> C.Graph:
        return self.b.g

    def plan(self):
        return self.graph.plan(self.keep)

    def flops(self) -> int:
        """Multiply-adds x 2 of the decode's convs (the arithmetic that
        dominates it)."""
        total = 0
        for node in self.graph.nodes:
            if node.op == C.GOP_MUL_MAT:
                m, n = self.b.shape(node.dst)
                total += 2 * m * n * self.b.shape(node.src[0])[-1]
            elif node.op == C.GOP_CONV_TRANSPOSE_1D:
                c_in, c_out, k = self.b.shape(node.src[0])
                total += 2 * c_in * c_out * k * self.b.shape(node.src[1])[-1]
        return total

    def close(self):
        for cw in self.convs:
            cw.close()
        self.convs = []
