"""The element-wise nodes of one T3 decode step, built as the reference's
T3::forward_impl builds them (chatterbox-cpp/src/t3.cpp:446-546) for one new
token (N_new = 1), with each matmul's output given as a device tensor: the
caller-side list that libcbxops' node-list executor (cbx_graph_*) plans and
runs, one token after another.

Per token the reference builds (ggml node order, matmuls left out):
  get_rows(speech_emb, token) -> cast, get_rows(pos_embd, position) -> cast,
  add                                                        (t3.cpp:446-455)
  per block:
    norm -> mul(ln1_w) -> add(ln1_b)                          (t3.cpp:465-466)
    add(qkv_mm, qkv_b)                                        (t3.cpp:470)
    scale(kq, 1/sqrt(64)) -> diag_mask_inf(n_past) -> soft_max (t3.cpp:513-518)
    add(out_mm, out_b) -> add(., h) -> norm -> mul -> add     (t3.cpp:525-532)
    add(fc_mm, fc_b) -> gelu                                  (t3.cpp:535-537)
    add(proj_mm, proj_b) -> add(., attn_residual)             (t3.cpp:539-541)
  norm -> mul(out_norm_w) -> add(out_norm_b)                  (t3.cpp:545-546)

The planner turns this into 1 + 5 x n_blocks launches: the embedding with
block 0's LN-1, then per block the qkv bias add, the score softmax, the
residual join with LN-2, the fc bias with GELU, and the projection's
residual join with the next block's LN-1 (the last block's: the final LN).

The scores of the step with n_past have n_past + 1 columns a head, the
contiguous (n_kv, 1, H) output of mul_mat(K, Q); retarget(n_past) re-points
those views and the mask for the next token, and the token and its position
live in device int32 tensors the caller writes.
"""
from __future__ import annotations

import numpy as np
import torch

from . import cbxops as C

BLOCK_IN = ("ln1_w", "ln1_b", "qkv_b", "out_b", "ln2_w", "ln2_b", "fc_b", "proj_b",
            "qkv_mm", "kq", "out_mm", "fc_mm", "proj_mm")
BLOCK_OUT = ("ln1", "qkv", "probs", "attn_res", "ln2", "gelu", "h")


def upload(inp: dict, device: str = "cuda") -> dict:
    """workloads.t3_token_inputs arrays as device tensors, plus the token and
    position tensors (int32, one element each)."""
    d = {k: torch.from_numpy(np.ascontiguousarray(v)).to(device) for k, v in inp.items()}
    d["token"] = torch.zeros(1, dtype=torch.int32, device=device)
    d["position"] = torch.zeros(1, dtype=torch.int32, device=device)
    return d


class T3DecodeStep:
    """One token's element-wise node list over device buffers `dev` (from
    upload()), for n_past tokens already in the cache."""

    def __init__(self, dev: dict, n_past: int, n_head: int = 16, eps: float = 1e-5):
        self.dev, self.n_head, self.eps = dev, int(n_head), float(eps)
        L, D = dev["ln1_w"].shape
        F = dev["fc_b"].shape[1]
        self.n_blocks, self.D, self.F = L, D, F
        self.max_ctx = dev["kq"].shape[1] // n_head
        dv = dev["kq"].device
        nan = lambda *s: torch.full(s, float("nan"), dtype=torch.float32, device=dv)  # noqa: E731
        # outputs (what the matmuls that follow read, and the residual stream)
        self.out = {"h0": nan(1, D), "y": nan(1, D), "ln1": nan(L, D), "qkv": nan(L, 3 * D),
                    "probs": nan(L, n_head * self.max_ctx), "attn_res": nan(L, D), "ln2": nan(L, D),
                    "gelu": nan(L, F), "h": nan(L, D)}
        # the chains' intermediates (registered like any ggml tensor; the
        # fused launches never write them)
        self._mid = {"e0": nan(1, D), "c0": nan(1, D), "e1": nan(1, D), "c1": nan(1, D),
                     "n": nan(L + 1, D), "m": nan(L + 1, D), "n2": nan(L, D), "m2": nan(L, D),
                     "cur": nan(L, D), "fcb": nan(L, F), "pc": nan(L, D),
                     "s": nan(L, n_head * self.max_ctx), "mk": nan(L, n_head * self.max_ctx)}
        self.kq_scale = float(np.float32(1.0) / np.sqrt(np.float32(D // n_head)))
        self.n_past = -1
        self._build(int(n_past))

    def _scores(self, t: torch.Tensor, il: int, n_kv: int) -> torch.Tensor:
        return t[il, : self.n_head * n_kv].view(self.n_head, 1, n_kv)

    def _build(self, n_past: int) -> None:
        if not 0 <= n_past < self.max_ctx:
            raise ValueError(f"n_past {n_past} outside [0, {self.max_ctx})")
        dev, out, mid, L = self.dev, self.out, self._mid, self.n_blocks
        n_kv = n_past + 1
        g = C.Graph()
        T = g.tensor
        tok, pos = T(dev["speech_emb"]), T(dev["pos_embd"])
        tid, pid = T(dev["token"]), T(dev["position"])
        e0, c0, e1, c1 = (T(mid[k]) for k in ("e0", "c0", "e1", "c1"))
        h = h0 = T(out["h0"])
        g.node(C.GOP_GET_ROWS, e0, (tok, tid))
        g.node(C.GOP_CPY, c0, (e0,))
        g.node(C.GOP_GET_ROWS, e1, (pos, pid))
        g.node(C.GOP_CPY, c1, (e1,))
        g.node(C.GOP_ADD, h, (c0, c1))
        keep = []
        self._kq_ids, self._mask_nodes = [], []
        for il in range(L):
            p = {k: T(dev[k][il]) for k in BLOCK_IN if k != "kq"}
            o = {k: T(out[k][il]) for k in BLOCK_OUT if k != "probs"}
            n, m = T(mid["n"][il]), T(mid["m"][il])
            g.node(C.GOP_NORM, n, (h,), fparam=self.eps)
            g.node(C.GOP_MUL, m, (n, p["ln1_w"]))
            g.node(C.GOP_ADD, o["ln1"], (m, p["ln1_b"]))
            g.node(C.GOP_ADD, o["qkv"], (p["qkv_mm"], p["qkv_b"]))
            kq = T(self._scores(dev["kq"], il, n_kv))
            s, mk = T(self._scores(mid["s"], il, n_kv)), T(self._scores(mid["mk"], il, n_kv))
            probs = T(self._scores(out["probs"], il, n_kv))
            self._kq_ids.append((kq, s, mk, probs))
            g.node(C.GOP_SCALE, s, (kq,), fparam=self.kq_scale)
            self._mask_nodes.append(len(g.nodes))
            g.node(C.GOP_DIAG_MASK_INF, mk, (s,), iparam=n_past)
            g.node(C.GOP_SOFT_MAX, probs, (mk,), fparam=1.0)
            cur = T(mid["cur"][il])
            g.node(C.GOP_ADD, cur, (p["out_mm"], p["out_b"]))
            g.node(C.GOP_ADD, o["attn_res"], (cur, h))
            n2, m2 = T(mid["n2"][il]), T(mid["m2"][il])
            g.node(C.GOP_NORM, n2, (o["attn_res"],), fparam=self.eps)
            g.node(C.GOP_MUL, m2, (n2, p["ln2_w"]))
            g.node(C.GOP_ADD, o["ln2"], (m2, p["ln2_b"]))
            fcb = T(mid["fcb"][il])
            g.node(C.GOP_ADD, fcb, (p["fc_mm"], p["fc_b"]))
            g.node(C.GOP_UNARY, o["gelu"], (fcb,), iparam=C.GELU)
            pc = T(mid["pc"][il])
            g.node(C.GOP_ADD, pc, (p["proj_mm"], p["proj_b"]))
            g.node(C.GOP_ADD, o["h"], (pc, o["attn_res"]))
            keep += [o["ln1"], o["qkv"], probs, o["ln2"], o["gelu"], o["h"]]
            h = o["h"]
        n, m = T(mid["n"][L]), T(mid["m"][L])
        y = T(out["y"])
        g.node(C.GOP_NORM, n, (h,), fparam=self.eps)
        g.node(C.GOP_MUL, m, (n, T(dev["out_w"])))
        g.node(C.GOP_ADD, y, (m, T(dev["out_b_final"])))
        keep += [h0, y]
        g.bind_arrays(keep)
        self.graph, self.keep, self.n_past = g, keep, n_past

    def retarget(self, n_past: int) -> None:
        """The list of the token after n_past cached ones: the score views
        (n_past + 1 columns a head, same first element) and the mask's n_past
        change; the graph's tensor indices and launches stay the same.  The
        descriptors are patched in place (the graph's arrays are bound)."""
        if not 0 <= n_past < self.max_ctx:
            raise ValueError(f"n_past {n_past} outside [0, {self.max_ctx})")
        n_kv = n_past + 1
        g = self.graph
        row, plane = 4 * n_kv, 4 * n_kv * self.n_head
        for ids in self._kq_ids:
            for i in ids:
                d = g._descs[i]
                d.ne[0] = n_kv
                d.nb[1] = row
                d.nb[2] = row
                d.nb[3] = plane
        for k in self._mask_nodes:
            g.nodes[k].iparam = n_past
        self.n_past = n_past

    def set_token(self, token: int, position: int) -> None:
        """Writes the token id and its position into their device tensors
        (stream-ordered on torch's current stream)."""
        self.dev["token"].fill_(int(token))
        self.dev["position"].fill_(int(position))

    def probs(self, il: int) -> torch.Tensor:
        """Block il's probabilities of the current step, (H, n_past + 1)."""
        return self._scores(self.out["probs"], il, self.n_past + 1).view(self.n_head, self.n_past + 1)

    def launches(self) -> int:
        return 1 + 5 * self.n_blocks
