"""Node lists as the reference's graph builders emit them, for the node-list
planner (cbx_graph_*).

HiFT (chatterbox-cpp/src/hift_vocoder.cpp): snake() (:64-73), conv1d_CT
(:77-93: im2col to F16, mul_mat and a reshape, the bias add, between two
transposes; conv_1d_f32 at :46-58), conv_transpose1d_CT (:96-116:
conv_transpose_1d, a cropping view and cont, the bias add, between two
transposes), composed as resblock_forward's sublayer (:119-138), conv_post
(:748-749) and an upsampler (:685-687).

CFM decoder (chatterbox-cpp/src/cfm_decoder.cpp): layer_norm (:29-33), mish
(:36-38), causal_conv1d (:89-120, its left padding from left_pad_TC at
:66-77), causal_block1d (:133-149), and the add / mul / concat / scale /
soft_max nodes the estimator's builders emit around the matmuls.

Tensors are torch tensors laid out as ggml's (torch shape = reversed ne);
views share their source's storage, so the planner sees what the ggml graph
holds.  `new(shape, dtype)` makes every tensor that is not a view: host
memory for planning, device memory for running."""
from __future__ import annotations

import torch

from . import cbxops as C


class NodeList:
    def __init__(self, new):
        self.g = C.Graph()
        self.new = new

    def t(self, x: torch.Tensor) -> int:
        return self.g.tensor(x)

    def at(self, i: int) -> torch.Tensor:
        return self.g._torch[i]

    def shape(self, i: int) -> tuple:
        return tuple(self.at(i).shape)

    def node_new(self, op, shape, src, dtype=torch.float32, **kw) -> int:
        """A node whose result is a new tensor of `shape`."""
        d = self.t(self.new(shape, dtype))
        self.g.node(op, d, src, **kw)
        return d

    def node_view(self, view: torch.Tensor, src: int) -> int:
        """A VIEW node (reshape / transpose / view in ggml) of tensor src."""
        d = self.t(view)
        self.g.node(C.GOP_VIEW, d, (src,))
        return d

    # ---- element-wise nodes ---------------------------------------------------

    def add(self, a: int, b: int) -> int:
        return self.node_new(C.GOP_ADD, self.shape(a), (a, b))

    def mul(self, a: int, b: int) -> int:
        return self.node_new(C.GOP_MUL, self.shape(a), (a, b))

    def unary(self, x: int, op: int) -> int:
        return self.node_new(C.GOP_UNARY, self.shape(x), (x,), iparam=op)

    def mish(self, x: int) -> int:
        """mul(x, tanh(softplus(x))) (cfm_decoder.cpp:36-38)."""
        sp = self.unary(x, C.SOFTPLUS)
        th = self.unary(sp, C.TANH)
        return self.node_new(C.GOP_MUL, self.shape(x), (x, th))

    def layer_norm(self, x: int, w: int, b: int, eps: float = 1e-5) -> int:
        """add(mul(norm(x), w), b) (cfm_decoder.cpp:29-33)."""
        n = self.node_new(C.GOP_NORM, self.shape(x), (x,), fparam=eps)
        m = self.node_new(C.GOP_MUL, self.shape(x), (n, w))
        return self.node_new(C.GOP_ADD, self.shape(x), (m, b))

    def scale(self, x: int, s: float) -> int:
        return self.node_new(C.GOP_SCALE, self.shape(x), (x,), fparam=s)

    def soft_max(self, x: int) -> int:
        return self.node_new(C.GOP_SOFT_MAX, self.shape(x), (x,), fparam=1.0)

    def concat(self, a: int, b: int, dim: int) -> int:
        """ggml_concat(a, b, dim), dim a ggml axis."""
        sa, sb = self.shape(a), self.shape(b)
        ax = len(sa) - 1 - dim
        out = list(sa)
        out[ax] = sa[ax] + sb[ax]
        return self.node_new(C.GOP_CONCAT, tuple(out), (a, b), iparam=dim)

    # ---- HiFT ------------------------------------------------------------------

    def snake(self, x: int, a: int, ai: int) -> int:
        """mul(x, a) -> sin -> sqr -> mul(., a_inv) -> add(x, .); a, ai (C,)."""
        sh = self.shape(x)
        m1 = self.node_new(C.GOP_MUL, sh, (x, a))
        sn = self.node_new(C.GOP_UNARY, sh, (m1,), iparam=C.SIN)
        sq = self.node_new(C.GOP_UNARY, sh, (sn,), iparam=C.SQR)
        m2 = self.node_new(C.GOP_MUL, sh, (sq, ai))
        return self.node_new(C.GOP_ADD, sh, (x, m2))

    def leaky(self, x: int, slope: float) -> int:
        return self.node_new(C.GOP_LEAKY_RELU, self.shape(x), (x,), fparam=slope)

    def transposed_copy(self, x: int) -> int:
        """cont(transpose(x))."""
        v = self.node_view(self.at(x).transpose(-1, -2), x)
        return self.node_new(C.GOP_CPY, self.shape(v), (v,))

    def tail(self, y: int, b) -> int:
        """[add(y, reshape_2d(b, 1, C))] -> cont(transpose(.))."""
        if b is not None:
            bv = self.node_view(self.at(b).reshape(-1, 1), b)
            y = self.node_new(C.GOP_ADD, self.shape(y), (y, bv))
        return self.transposed_copy(y)

    def conv1d(self, x: int, w: int, b, stride: int, pad: int, dil: int, conv_w) -> int:
        """conv1d_CT of x (ggml (C_in, T)); w torch [C_out, C_in, K]."""
        C_out, C_in, K = self.at(w).shape
        T_in = self.at(x).shape[-2]
        B = self.at(x).shape[0] if self.at(x).dim() == 3 else 1
        T_out = (T_in + 2 * pad - dil * (K - 1) - 1) // stride + 1
        xt = self.transposed_copy(x)
        col = self.node_new(C.GOP_IM2COL, (B, T_out, C_in * K), (w, xt), dtype=torch.float16,
                            conv=(stride, pad, dil))
        col2 = self.node_view(self.at(col).reshape(B * T_out, C_in * K), col)
        w2 = self.node_view(self.at(w).reshape(C_out, C_in * K), w)
        mm = self.node_new(C.GOP_MUL_MAT, (C_out, B * T_out), (col2, w2), conv_w=conv_w)
        y3 = self.node_view(self.at(mm).reshape(B, C_out, T_out), mm)
        return self.tail(y3, b)

    def conv_transpose1d(self, x: int, w: int, b, stride: int, pad: int, conv_w) -> int:
        """conv_transpose1d_CT of x (ggml (C_in, T)); w torch [C_in, C_out, K]."""
        C_in, C_out, K = self.at(w).shape
        T_full = (self.at(x).shape[-2] - 1) * stride + K
        xt = self.transposed_copy(x)
        full = self.node_new(C.GOP_CONV_TRANSPOSE_1D, (C_out, T_full), (w, xt), conv=(stride,), conv_w=conv_w)
        crop = self.node_view(self.at(full)[:, pad:T_full - pad], full)
        cc = self.node_new(C.GOP_CPY, (C_out, T_full - 2 * pad), (crop,))
        return self.tail(cc, b)

    def sublayer(self, x: int, p: dict, d: int, conv_w1, conv_w2) -> int:
        """One resblock_forward layer: x + conv2(snake2(conv1(snake1(x))))
        with "same" padding; p holds the tensor indices a1, ai1, w1, b1,
        a2, ai2, w2, b2."""
        K = self.at(p["w1"]).shape[-1]
        h = self.snake(x, p["a1"], p["ai1"])
        h = self.conv1d(h, p["w1"], p["b1"], 1, (K - 1) // 2 * d, d, conv_w1)
        h = self.snake(h, p["a2"], p["ai2"])
        h = self.conv1d(h, p["w2"], p["b2"], 1, (K - 1) // 2, 1, conv_w2)
        return self.add(x, h)

    # ---- CFM decoder -------------------------------------------------------------

    def causal_conv1d(self, x: int, w: int, b, conv_w) -> int:
        """causal_conv1d of x (ggml (C_in, T)); w torch [C_out, C_in, K]: K - 1
        zero frames from a zero-scaled view of the first frames, concatenated
        in front, then im2col (stride 1, no padding) and mul_mat."""
        C_out, C_in, K = self.at(w).shape
        T = self.at(x).shape[-2]
        xt = self.transposed_copy(x)
        zv = self.node_view(self.at(xt)[:, :K - 1], xt)
        zc = self.node_new(C.GOP_CPY, (C_in, K - 1), (zv,))
        zs = self.node_new(C.GOP_SCALE, (C_in, K - 1), (zc,), fparam=0.0)
        pd = self.node_new(C.GOP_CONCAT, (C_in, T + K - 1), (zs, xt), iparam=0)
        col = self.node_new(C.GOP_IM2COL, (1, T, C_in * K), (w, pd), dtype=torch.float16, conv=(1, 0, 1))
        col2 = self.node_view(self.at(col).reshape(T, C_in * K), col)
        w2 = self.node_view(self.at(w).reshape(C_out, C_in * K), w)
        mm = self.node_new(C.GOP_MUL_MAT, (C_out, T), (col2, w2), conv_w=conv_w)
        return self.tail(mm, b)

    def causal_block(self, x: int, mask: int, w: int, b: int, ln_w: int, ln_b: int, conv_w, eps=1e-5) -> int:
        """causal_block1d (cfm_decoder.cpp:133-149): mul(x, mask) -> causal
        conv (+ bias) -> layer_norm -> mish -> mul(., mask)."""
        h = self.causal_conv1d(self.mul(x, mask), w, b, conv_w)
        return self.mul(self.mish(self.layer_norm(h, ln_w, ln_b, eps)), mask)
