// cbx_graph.cpp -- runs a list of ggml-style op nodes by mapping the
// reference's op compositions onto the fused entry points.
//
// The reference reaches its layer ops through ggml graphs that the backend
// scheduler runs node by node (chatterbox-cpp/src/backend.cpp:108-122); its
// helpers emit the same short node chains every time: layer_norm() is
// norm -> mul -> add (cfm_decoder.cpp:29-33), mish() is softplus -> tanh ->
// mul (cfm_decoder.cpp:36-38) and follows a layer_norm in causal_block1d
// (cfm_decoder.cpp:143-146), snake() is mul -> sin -> sqr -> mul -> add
// (hift_vocoder.cpp:64-73), the T3 input is get_rows -> cast -> get_rows ->
// cast -> add -> norm -> mul -> add (t3.cpp:446-466), attention scores are
// scale -> diag_mask_inf -> soft_max (t3.cpp:513-518), a block's residual
// join is add(add(mul_mat, bias), h) -> layer_norm (t3.cpp:528-532), its
// feed-forward input add(mul_mat, bias) -> gelu (t3.cpp:535-537), and
// causal_block1d ends layer_norm -> mish -> mul(mask) (cfm_decoder.cpp:
// 143-148), and HiFT's convolutions are transpose -> cont -> im2col ->
// mul_mat -> bias add -> transpose -> cont (conv1d_CT, hift_vocoder.cpp:
// 77-93) or the same around conv_transpose_1d and a cropping view
// (conv_transpose1d_CT, :96-115), after snake() or leaky_relu and, in a
// ResBlock, before the residual add (:128-135); the CFM decoder's
// causal_conv1d pads K-1 zero frames on the left with a zero-scaled view
// and a concat before its im2col (cfm_decoder.cpp:66-120), after
// causal_block1d's mul(x, mask) (:139).  The planner walks
// the nodes in order and, at each node, takes the longest such chain whose
// intermediate results no other node reads and the caller does not keep;
// the chain then runs as one library call.  Because a chain is a run of
// consecutive nodes of a topologically ordered list, every value it reads
// from outside is ready when its first node's turn comes.  Host code only:
// every launch goes through the public entry points, which check operand
// layouts as they do for any caller.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "cbx_internal.h"

using namespace cbx;

namespace {

// The T3 input chain with the conditioning prefix, as t3.cpp:432-466 builds
// it (in graph order):
//   [get_rows(src_a, ids_a) [-> cast] -> concat(prefix, ., 1) ->]
//   get_rows(src_b, ids_b) [-> cast] -> concat(seq, ., 1) ->
//   get_rows(src2, ids2) [-> cast] -> add(seq, .) -> norm -> mul -> add
// where the first concat's src0 is the prefix rows (the conditioning
// encoder's output).  Without the prompt segment the text gather's concat
// is the first one.  Parsed from node i on structure alone (ops, operand
// links, concat along dim 1).
struct ConcatT3 {
    int32_t g_a = -1, g_b = -1, g_pos = -1;   // gather nodes (g_a -1: no prompt segment)
    int32_t prefix = -1;                      // tensor holding the prefix rows
    int32_t add = -1;                         // seq + positions; the LayerNorm is add + 1 .. add + 3
    int32_t n_nodes = 0;
    int32_t inner[8];                         // intermediates: each has exactly one reader in the chain
    int32_t n_inner = 0;
    int32_t cast[3];                          // the cast nodes (each must make F32)
    int32_t n_cast = 0;
};

bool parse_concat_t3(const cbx_gnode* nd, int32_t n, int32_t i, ConcatT3* c) {
    auto is = [&](int32_t k, int op) { return k >= 0 && k < n && nd[k].op == op; };
    // a gather at k with an optional cast: the node after it, its value in *v
    auto gather = [&](int32_t k, int32_t* v) -> int32_t {
        if (!is(k, CBX_GOP_GET_ROWS)) return -1;
        *v = nd[k].dst;
        if (is(k + 1, CBX_GOP_CPY) && nd[k + 1].src[0] == *v) {
            c->inner[c->n_inner++] = *v;
            c->cast[c->n_cast++] = k + 1;
            *v = nd[k + 1].dst;
            return k + 2;
        }
        return k + 1;
    };
    auto concat_of = [&](int32_t k, int32_t src1) {
        return is(k, CBX_GOP_CONCAT) && nd[k].src[1] == src1 && nd[k].iparam == 1;
    };
    c->n_inner = 0;
    c->n_cast = 0;
    int32_t v1 = -1;
    const int32_t k1 = gather(i, &v1);
    if (k1 < 0 || !concat_of(k1, v1)) return false;
    c->prefix = nd[k1].src[0];
    c->inner[c->n_inner++] = v1;
    int32_t seq = nd[k1].dst;
    int32_t v2 = -1;
    const int32_t k2 = gather(k1 + 1, &v2);
    if (k2 < 0) return false;
    int32_t add, vpos;
    if (concat_of(k2, v2) && nd[k2].src[0] == seq) {   // prompt, then text
        c->g_a = i;
        c->g_b = k1 + 1;
        c->inner[c->n_inner++] = seq;
        c->inner[c->n_inner++] = v2;
        seq = nd[k2].dst;
        c->g_pos = k2 + 1;
        add = gather(k2 + 1, &vpos);
    } else {                                          // text only
        c->g_a = -1;
        c->g_b = i;
        c->g_pos = k1 + 1;
        vpos = v2;
        add = k2;
    }
    if (add < 0 || !is(add, CBX_GOP_ADD) || nd[add].src[0] != seq || nd[add].src[1] != vpos) return false;
    c->inner[c->n_inner++] = seq;
    c->inner[c->n_inner++] = vpos;
    const int32_t h = nd[add].dst;
    if (!is(add + 1, CBX_GOP_NORM) || nd[add + 1].src[0] != h || !is(add + 2, CBX_GOP_MUL) ||
        nd[add + 2].src[0] != nd[add + 1].dst || !is(add + 3, CBX_GOP_ADD) || nd[add + 3].src[0] != nd[add + 2].dst) {
        return false;
    }
    c->add = add;
    c->n_nodes = add + 4 - i;
    return true;
}

// The number of leading dims of v whose sizes multiply to n (a vector of n
// values re-described as one period of v's shape), or -1
int lead_dims(const cbx_tensor& v, int64_t n) {
    int64_t p = 1;
    for (int k = 0; k < 4; k++) {
        p *= v.ne[k];
        if (p == n) return k + 1;
        if (p > n) return -1;
    }
    return -1;
}

struct Planner {
    const cbx_tensor* t;
    int32_t n_t;
    const cbx_gnode* nd;
    int32_t n;
    std::vector<int32_t> uses;   // how many node operands name each tensor
    std::vector<char> keep;

    bool valid_t(int32_t i) const { return i >= 0 && i < n_t; }
    bool is(int32_t i, int op) const { return i < n && nd[i].op == op; }
    bool is_unary(int32_t i, int u) const { return is(i, CBX_GOP_UNARY) && nd[i].iparam == u; }
    // An intermediate may stay unstored: the caller does not keep it and the
    // `inside` operands that read it within the chain are all its readers.
    bool internal(int32_t tensor, int inside) const {
        return valid_t(tensor) && !keep[static_cast<size_t>(tensor)] && uses[static_cast<size_t>(tensor)] == inside;
    }
    bool dims(int32_t p, int64_t a, int64_t b, int64_t c, int64_t d) const {
        return valid_t(p) && t[p].ne[0] == a && t[p].ne[1] == b && t[p].ne[2] == c && t[p].ne[3] == d;
    }
    bool row_vec(int32_t p, int32_t x) const { return valid_t(x) && dims(p, t[x].ne[0], 1, 1, 1); }
    bool chan_vec(int32_t p, int32_t x) const { return valid_t(x) && dims(p, 1, 1, t[x].ne[2], 1); }
    bool same_dims(int32_t a, int32_t b) const {
        return valid_t(a) && valid_t(b) && dims(a, t[b].ne[0], t[b].ne[1], t[b].ne[2], t[b].ne[3]);
    }

    // mish(x) = mul(x, tanh(softplus(x))) at node i
    bool mish_at(int32_t i, int32_t x) const {
        return is_unary(i, CBX_UNARY_SOFTPLUS) && nd[i].src[0] == x && is_unary(i + 1, CBX_UNARY_TANH) &&
               nd[i + 1].src[0] == nd[i].dst && is(i + 2, CBX_GOP_MUL) && nd[i + 2].src[0] == x &&
               nd[i + 2].src[1] == nd[i + 1].dst && internal(nd[i].dst, 1) && internal(nd[i + 1].dst, 1);
    }

    // layer_norm(x) = add(mul(norm(x), w), b) at node i, w and b (x.ne0)
    bool layer_norm_at(int32_t i) const {
        if (!is(i, CBX_GOP_NORM)) return false;
        const int32_t x = nd[i].src[0];
        return is(i + 1, CBX_GOP_MUL) && nd[i + 1].src[0] == nd[i].dst && row_vec(nd[i + 1].src[1], x) &&
               is(i + 2, CBX_GOP_ADD) && nd[i + 2].src[0] == nd[i + 1].dst && row_vec(nd[i + 2].src[1], x) &&
               internal(nd[i].dst, 1) && internal(nd[i + 1].dst, 1);
    }

    // a cast right after a gather takes over its result: 1 node, or 0
    int32_t cast_after(int32_t i, int32_t* value) const {
        if (is(i, CBX_GOP_CPY) && nd[i].src[0] == *value && internal(*value, 1) && valid_t(nd[i].dst) &&
            t[nd[i].dst].type == CBX_TYPE_F32) {
            *value = nd[i].dst;
            return 1;
        }
        return 0;
    }

    bool col_vec(int32_t p, int32_t x) const { return valid_t(x) && dims(p, 1, t[x].ne[1], 1, 1); }
    // b repeats to x's shape (ggml_can_repeat): every x.ne[k] a multiple of b.ne[k]
    bool repeats(int32_t b, int32_t x) const {
        if (!valid_t(b) || !valid_t(x)) return false;
        for (int k = 0; k < 4; k++) {
            if (t[b].ne[k] < 1 || t[x].ne[k] % t[b].ne[k] != 0) return false;
        }
        return true;
    }

    // v views the whole of p unchanged: same data, dims and (contiguous) layout
    bool alias(int32_t v, int32_t p) const {
        return same_dims(v, p) && t[v].data == t[p].data && t[v].type == t[p].type && is_contiguous(&t[v]) &&
               is_contiguous(&t[p]);
    }

    // add(a, b) of two F32 tensors of one shape at node i, then [scale ->]
    // [diag_mask_inf ->] soft_max reading the sum alone: the node count, or 0
    int32_t add_soft_max_at(int32_t i) const {
        const cbx_gnode& a = nd[i];
        const int32_t x = a.src[0];
        if (!same_dims(a.src[1], x) || !same_dims(a.dst, x) || t[x].type != CBX_TYPE_F32 ||
            t[a.src[1]].type != CBX_TYPE_F32) {
            return 0;
        }
        int32_t j = i + 1, prev = a.dst;
        if (is(j, CBX_GOP_SCALE) && nd[j].src[0] == prev && internal(prev, 1)) prev = nd[j++].dst;
        if (is(j, CBX_GOP_DIAG_MASK_INF) && nd[j].src[0] == prev && internal(prev, 1)) {
            if (nd[j].iparam < 0) return 0;
            prev = nd[j++].dst;
        }
        const bool sm = is(j, CBX_GOP_SOFT_MAX) && nd[j].src[0] == prev && internal(prev, 1) && nd[j].src[1] < 0 &&
                        nd[j].fparam == 1.0f;
        return sm ? j + 1 - i : 0;
    }

    // add(x, bias) -> view (a contiguous reshape of the sum) -> add(view, u),
    // add(view, v) at node i, the sum and the view read by nothing else
    // (flow_encoder.cpp:320, 341-345: q's bias, then pos_bias_u and
    // pos_bias_v over the query heads); up to two views of other tensors
    // (u's and v's reshapes) may stand among the adds, a view running
    // nothing: the node count (4 to 6), or 0
    int32_t bias_pair_at(int32_t i) const {
        const cbx_gnode& a = nd[i];
        const int32_t x = a.src[0], bias = a.src[1], s = a.dst;
        if (!row_vec(bias, x) || !same_dims(s, x) || !is(i + 1, CBX_GOP_VIEW) || nd[i + 1].src[0] != s ||
            !internal(s, 1)) {
            return 0;
        }
        const int32_t vw = nd[i + 1].dst;
        if (!valid_t(vw) || !internal(vw, 2)) return 0;
        const cbx_tensor &X = t[x], &B = t[bias], &S = t[s], &V = t[vw];
        if (X.type != CBX_TYPE_F32 || B.type != CBX_TYPE_F32 || S.type != CBX_TYPE_F32 || V.type != CBX_TYPE_F32 ||
            !is_contiguous(&X) || !is_contiguous(&B) || !is_contiguous(&S) || !is_contiguous(&V) ||
            V.data != S.data || nelements(&V) != nelements(&S) || lead_dims(V, X.ne[0]) < 0) {
            return 0;
        }
        int32_t j = i + 2, n_add = 0;
        for (; n_add < 2 && j < i + 6; j++) {
            if (is(j, CBX_GOP_VIEW) && nd[j].src[0] != s && nd[j].src[0] != vw) continue;
            if (!is(j, CBX_GOP_ADD) || nd[j].src[0] != vw || !repeats(nd[j].src[1], vw) ||
                t[nd[j].src[1]].type != CBX_TYPE_F32 || !same_dims(nd[j].dst, vw)) {
                return 0;
            }
            n_add++;
        }
        return n_add == 2 ? j - i : 0;
    }

    // add(x, bias) [-> view (an alias of the sum)] -> add(r, .) at node i,
    // bias repeating to x and x to r: the node count (2 or 3), or 0
    int32_t bias_residual_at(int32_t i) const {
        if (!is(i, CBX_GOP_ADD)) return 0;
        const int32_t x = nd[i].src[0], t1 = nd[i].dst;
        if (!repeats(nd[i].src[1], x) || !same_dims(t1, x) || !internal(t1, 1)) return 0;
        int32_t k = i + 1, sum = t1;
        if (is(k, CBX_GOP_VIEW) && nd[k].src[0] == t1) {
            if (!alias(nd[k].dst, t1) || !internal(nd[k].dst, 1)) return 0;
            sum = nd[k++].dst;
        }
        if (!is(k, CBX_GOP_ADD)) return 0;
        const int32_t r = nd[k].src[0] == sum ? nd[k].src[1] : nd[k].src[1] == sum ? nd[k].src[0] : -1;
        return r >= 0 && r != sum && repeats(sum, r) && same_dims(nd[k].dst, r) ? k + 1 - i : 0;
    }

    // layer_norm at node i reading `in`, optionally followed by a mish
    // chain: the node count (3 or 6), or 0
    // a tensor in a layout the fused LayerNorm kernel takes: ne0 % 4 == 0,
    // ne0 <= 4096, 16-byte aligned data and row steps
    bool ln_ext_fits(int32_t p) const {
        if (!valid_t(p) || t[p].ne[0] % 4 != 0 || t[p].ne[0] > 4096 || reinterpret_cast<uintptr_t>(t[p].data) % 16) {
            return false;
        }
        for (int k = 1; k < 4; k++) {
            if (t[p].nb[k] % 16) return false;
        }
        return true;
    }

    int32_t layer_norm_mish_at(int32_t i, int32_t in) const {
        if (!layer_norm_at(i) || nd[i].src[0] != in) return 0;
        const int32_t y = nd[i + 2].dst;
        return mish_at(i + 3, y) && internal(y, 2) ? 6 : 3;
    }

    // norm -> mul -> add -> view -> rope, the view splitting rows into heads
    bool layer_norm_rope_at(int32_t i) const {
        if (!layer_norm_at(i) || !is(i + 3, CBX_GOP_VIEW) || !is(i + 4, CBX_GOP_ROPE)) return false;
        const int32_t x = nd[i].src[0], y = nd[i + 2].dst, v = nd[i + 3].dst, r = nd[i + 4].dst;
        if (nd[i + 3].src[0] != y || nd[i + 4].src[0] != v || !internal(y, 1) || !internal(v, 1) || !valid_t(x)) {
            return false;
        }
        const cbx_tensor &X = t[x], &Y = t[y], &V = t[v], &R = t[r];
        return X.ne[3] == 1 && V.ne[0] > 0 && V.ne[0] * V.ne[1] == X.ne[0] && V.ne[2] == X.ne[1] &&
               V.ne[3] == X.ne[2] && V.data == Y.data && V.type == CBX_TYPE_F32 && R.type == CBX_TYPE_F32 &&
               is_contiguous(&Y) && is_contiguous(&V) && is_contiguous(&R) && same_dims(r, v);
    }

    // transpose (view) -> cont of x (C, T, B) at node i: the contiguous
    // (T, C, B) copy, or -1
    int32_t transposed_copy_at(int32_t i, int32_t x) const {
        if (!valid_t(x) || !is(i, CBX_GOP_VIEW) || nd[i].src[0] != x || !is(i + 1, CBX_GOP_CPY)) return -1;
        const cbx_tensor& X = t[x];
        const int32_t v = nd[i].dst, c = nd[i + 1].dst;
        if (!dims(v, X.ne[1], X.ne[0], X.ne[2], X.ne[3]) || t[v].data != X.data || !internal(v, 1) ||
            nd[i + 1].src[0] != v || !same_dims(c, v) || !internal(c, 1)) {
            return -1;
        }
        return c;
    }

    // [view (bias as (1, C)) -> add(y, view)] -> transpose (view) -> cont,
    // from y (T, C, B) at node j: the node count, or 0; *fl gets bit 2 for
    // the bias add and *out the (C, T, B) result
    int32_t conv_tail_at(int32_t j, int32_t y, int32_t* fl, int32_t* out) const {
        const int32_t j0 = j;
        int32_t cur = y;
        const int64_t C = valid_t(y) ? t[y].ne[1] : -1;
        if (is(j, CBX_GOP_VIEW) && is(j + 1, CBX_GOP_ADD) && nd[j + 1].src[0] == cur && nd[j + 1].src[1] == nd[j].dst &&
            valid_t(nd[j].src[0]) && nelements(&t[nd[j].src[0]]) == C && dims(nd[j].dst, 1, C, 1, 1) &&
            internal(cur, 1) && internal(nd[j].dst, 1) && same_dims(nd[j + 1].dst, cur)) {
            *fl |= 4;
            cur = nd[j + 1].dst;
            j += 2;
        }
        if (!valid_t(cur) || !is(j, CBX_GOP_VIEW) || nd[j].src[0] != cur || !internal(cur, 1) ||
            !is(j + 1, CBX_GOP_CPY)) {
            return 0;
        }
        const cbx_tensor& Y = t[cur];
        const int32_t v = nd[j].dst, o = nd[j + 1].dst;
        if (!dims(v, Y.ne[1], Y.ne[0], Y.ne[2], Y.ne[3]) || t[v].data != Y.data || !internal(v, 1) ||
            nd[j + 1].src[0] != v || !same_dims(o, v)) {
            return 0;
        }
        *out = o;
        return j + 2 - j0;
    }

    // conv1d_CT of x (C_in, T_in, B) at node i: transpose -> cont ->
    // im2col -> view (2-D) -> view (weight 2-D) -> mul_mat (with prepared
    // weights) -> view (3-D) -> conv_tail [-> add(., residual)].  The node
    // count, or 0; *fl gets bits 2 (bias) and 3 (residual).
    int32_t conv1d_at(int32_t i, int32_t x, int32_t* fl) const {
        const int32_t c = transposed_copy_at(i, x);
        if (c < 0 || !is(i + 2, CBX_GOP_IM2COL) || nd[i + 2].src[1] != c) return 0;
        const int32_t wk = nd[i + 2].src[0], col = nd[i + 2].dst;
        if (!valid_t(wk) || !valid_t(col) || !internal(col, 1)) return 0;
        const cbx_tensor &X = t[x], &Wk = t[wk], &Col = t[col];
        // one batch item only: for N > 1 the graph's reshape of the (OL*N,
        // OC) product to (OL, OC, N) does not separate the items, so the
        // nodes would not compute a batched conv
        const int64_t K = Wk.ne[0], C_in = Wk.ne[1], C_out = Wk.ne[2], B = X.ne[2], T_out = Col.ne[1];
        if (C_in != X.ne[0] || Wk.ne[3] != 1 || Col.ne[0] != C_in * K || Col.ne[2] != B || B != 1 || X.ne[3] != 1) {
            return 0;
        }
        if (!is(i + 3, CBX_GOP_VIEW) || nd[i + 3].src[0] != col || !is(i + 4, CBX_GOP_VIEW) ||
            nd[i + 4].src[0] != wk || !is(i + 5, CBX_GOP_MUL_MAT)) {
            return 0;
        }
        const int32_t col2 = nd[i + 3].dst, w2 = nd[i + 4].dst, mm = nd[i + 5].dst;
        if (!dims(col2, C_in * K, T_out * B, 1, 1) || !internal(col2, 1) || !dims(w2, K * C_in, C_out, 1, 1) ||
            !internal(w2, 1) || nd[i + 5].src[0] != col2 || nd[i + 5].src[1] != w2 || !nd[i + 5].conv_w ||
            !dims(mm, T_out * B, C_out, 1, 1) || !internal(mm, 1) || !is(i + 6, CBX_GOP_VIEW) ||
            nd[i + 6].src[0] != mm || !dims(nd[i + 6].dst, T_out, C_out, B, 1)) {
            return 0;
        }
        int32_t out = -1;
        const int32_t tail = conv_tail_at(i + 7, nd[i + 6].dst, fl, &out);
        if (!tail) return 0;
        int32_t j = i + 7 + tail;
        if (is(j, CBX_GOP_ADD) && internal(out, 1)) {
            const int32_t other = nd[j].src[0] == out ? nd[j].src[1] : nd[j].src[1] == out ? nd[j].src[0] : -1;
            if (same_dims(other, out) && same_dims(nd[j].dst, out)) {
                *fl |= 8;
                j++;
                // the ResBlock sum: add(sum, r) of the residual's result r,
                // then [scale] (hift_vocoder.cpp:731-736)
                const int32_t r = nd[j - 1].dst;
                if (is(j, CBX_GOP_ADD) && internal(r, 1)) {
                    const int32_t acc = nd[j].src[0] == r ? nd[j].src[1] : nd[j].src[1] == r ? nd[j].src[0] : -1;
                    if (acc != r && same_dims(acc, r) && same_dims(nd[j].dst, r)) {
                        *fl |= 16;
                        j++;
                        const int32_t sum = nd[j - 1].dst;
                        if (is(j, CBX_GOP_SCALE) && nd[j].src[0] == sum && internal(sum, 1) && same_dims(nd[j].dst, r)) {
                            *fl |= 32;
                            j++;
                        }
                    }
                }
            }
        }
        return j - i;
    }

    // conv_transpose1d_CT of x (C_in, T_in, 1) at node i: transpose ->
    // cont -> conv_transpose_1d (with prepared weights) -> view cropping
    // pad frames at both ends -> cont -> conv_tail.  The node count, or 0.
    int32_t convt_at(int32_t i, int32_t x, int32_t* fl) const {
        const int32_t c = transposed_copy_at(i, x);
        if (c < 0 || !is(i + 2, CBX_GOP_CONV_TRANSPOSE_1D) || nd[i + 2].src[1] != c || !nd[i + 2].conv_w) return 0;
        const int32_t wk = nd[i + 2].src[0], full = nd[i + 2].dst;
        if (!valid_t(wk) || !valid_t(full) || !internal(full, 1)) return 0;
        const cbx_tensor &X = t[x], &Wk = t[wk], &F = t[full];
        const int64_t K = Wk.ne[0], C_out = Wk.ne[1], s0 = nd[i + 2].conv[0];
        if (Wk.ne[2] != X.ne[0] || X.ne[2] != 1 || X.ne[3] != 1 || s0 < 1 ||
            !dims(full, (X.ne[1] - 1) * s0 + K, C_out, 1, 1) || F.type != CBX_TYPE_F32) {
            return 0;
        }
        if (!is(i + 3, CBX_GOP_VIEW) || nd[i + 3].src[0] != full || !is(i + 4, CBX_GOP_CPY)) return 0;
        const int32_t crop = nd[i + 3].dst, cc = nd[i + 4].dst;
        const char* d0 = static_cast<const char*>(F.data);
        const char* d1 = valid_t(crop) ? static_cast<const char*>(t[crop].data) : nullptr;
        const int64_t off = d1 ? d1 - d0 : -1;
        if (off < 0 || off % 4 || t[crop].nb[1] != F.nb[1] || !internal(crop, 1) || nd[i + 4].src[0] != crop ||
            !same_dims(cc, crop) || !internal(cc, 1) || !dims(crop, F.ne[0] - 2 * (off / 4), C_out, 1, 1)) {
            return 0;
        }
        int32_t out = -1;
        const int32_t tail = conv_tail_at(i + 5, cc, fl, &out);
        return tail ? 5 + tail : 0;
    }

    // causal_conv1d of x (C_in, T, 1) at node i (cfm_decoder.cpp:89-120):
    // transpose -> cont (read twice) -> view of its first K-1 frames ->
    // cont -> scale(0) -> concat(zeros, cont, dim 0) -> im2col (stride 1,
    // padding 0, dilation 1) -> view (2-D) -> view (weight 2-D) -> mul_mat
    // (with prepared weights) -> conv_tail.  The node count, or 0; *fl gets
    // bit 2 for the bias add.
    int32_t causal_at(int32_t i, int32_t x, int32_t* fl) const {
        if (!valid_t(x) || !is(i, CBX_GOP_VIEW) || nd[i].src[0] != x || !is(i + 1, CBX_GOP_CPY)) return 0;
        const cbx_tensor& X = t[x];
        const int32_t v = nd[i].dst, c = nd[i + 1].dst;
        if (X.ne[2] != 1 || X.ne[3] != 1 || !dims(v, X.ne[1], X.ne[0], 1, 1) || t[v].data != X.data ||
            !internal(v, 1) || nd[i + 1].src[0] != v || !same_dims(c, v) || !internal(c, 2)) {
            return 0;
        }
        if (!is(i + 2, CBX_GOP_VIEW) || nd[i + 2].src[0] != c || !is(i + 3, CBX_GOP_CPY) ||
            !is(i + 4, CBX_GOP_SCALE) || !is(i + 5, CBX_GOP_CONCAT)) {
            return 0;
        }
        const int32_t zv = nd[i + 2].dst, zc = nd[i + 3].dst, zs = nd[i + 4].dst, pd = nd[i + 5].dst;
        if (!valid_t(zv)) return 0;
        const int64_t pad = t[zv].ne[0];
        if (pad < 1 || !dims(zv, pad, X.ne[0], 1, 1) || t[zv].data != t[c].data || t[zv].nb[1] != t[c].nb[1] ||
            !internal(zv, 1) || nd[i + 3].src[0] != zv || !same_dims(zc, zv) || !internal(zc, 1) ||
            nd[i + 4].src[0] != zc || nd[i + 4].fparam != 0.0f || !same_dims(zs, zv) || !internal(zs, 1) ||
            nd[i + 5].src[0] != zs || nd[i + 5].src[1] != c || nd[i + 5].iparam != 0 ||
            !dims(pd, X.ne[1] + pad, X.ne[0], 1, 1) || !internal(pd, 1)) {
            return 0;
        }
        if (!is(i + 6, CBX_GOP_IM2COL) || nd[i + 6].src[1] != pd) return 0;
        const cbx_gnode& ic = nd[i + 6];
        const int32_t wk = ic.src[0], col = ic.dst;
        if (!valid_t(wk) || !valid_t(col) || !internal(col, 1)) return 0;
        const cbx_tensor& Wk = t[wk];
        const int64_t K = Wk.ne[0], C_in = Wk.ne[1], C_out = Wk.ne[2], T = X.ne[1];
        if (C_in != X.ne[0] || Wk.ne[3] != 1 || K - 1 != pad || ic.conv[0] != 1 || ic.conv[1] != 0 ||
            ic.conv[2] != 1 || !dims(col, C_in * K, T, 1, 1)) {
            return 0;
        }
        if (!is(i + 7, CBX_GOP_VIEW) || nd[i + 7].src[0] != col || !is(i + 8, CBX_GOP_VIEW) ||
            nd[i + 8].src[0] != wk || !is(i + 9, CBX_GOP_MUL_MAT)) {
            return 0;
        }
        const int32_t col2 = nd[i + 7].dst, w2 = nd[i + 8].dst, mm = nd[i + 9].dst;
        if (!dims(col2, C_in * K, T, 1, 1) || !internal(col2, 1) || !dims(w2, K * C_in, C_out, 1, 1) ||
            !internal(w2, 1) || nd[i + 9].src[0] != col2 || nd[i + 9].src[1] != w2 || !nd[i + 9].conv_w ||
            !dims(mm, T, C_out, 1, 1) || !internal(mm, 1)) {
            return 0;
        }
        int32_t out = -1;
        const int32_t tail = conv_tail_at(i + 10, mm, fl, &out);
        return tail ? 10 + tail : 0;
    }

    // A conv chain starting at node i whose input is x (the prologue's
    // output, or the chain's own input): CONV1D / CONV_TRANSPOSE1D and its
    // node count, or UNSUPPORTED.
    int32_t conv_chain_at(int32_t i, int32_t x, int32_t* n, int32_t* fl) const {
        if ((*n = conv1d_at(i, x, fl))) return CBX_GL_CONV1D;
        if ((*n = convt_at(i, x, fl))) return CBX_GL_CONV_TRANSPOSE1D;
        return CBX_GL_UNSUPPORTED;
    }

    // The longest chain at node i: its kind, *len nodes, *flags.
    int32_t match(int32_t i, int32_t* len, int32_t* flags) const {
        const cbx_gnode& a = nd[i];
        *len = 1;
        *flags = 0;
        switch (a.op) {
            case CBX_GOP_VIEW: {
                int32_t n = 0, fl = 0;
                const int32_t k = conv_chain_at(i, a.src[0], &n, &fl);
                if (k != CBX_GL_UNSUPPORTED) {
                    *len = n;
                    *flags = fl;
                    return k;
                }
                if ((n = causal_at(i, a.src[0], &fl))) {
                    *len = n;
                    *flags = fl;
                    return CBX_GL_CAUSAL_CONV1D;
                }
                return CBX_GL_VIEW;
            }
            case CBX_GOP_GET_ROWS: {
                ConcatT3 c;
                if (parse_concat_t3(nd, n, i, &c)) {
                    bool ok = true;
                    for (int32_t q = 0; q < c.n_inner; q++) ok = ok && internal(c.inner[q], 1);
                    for (int32_t q = 0; q < c.n_cast; q++) ok = ok && t[nd[c.cast[q]].dst].type == CBX_TYPE_F32;
                    const int32_t h = nd[c.add].dst, nn = nd[c.add + 1].dst, mm = nd[c.add + 2].dst;
                    const int32_t P = c.prefix;
                    ok = ok && internal(nn, 1) && internal(mm, 1) && valid_t(P) && valid_t(h) &&
                         t[P].type == CBX_TYPE_F32 && t[P].ne[0] == t[h].ne[0] && t[P].ne[2] == 1 && t[P].ne[3] == 1 &&
                         row_vec(nd[c.add + 2].src[1], h) && row_vec(nd[c.add + 3].src[1], h);
                    if (ok) {
                        if (internal(h, 1)) *flags = 1;   // h read only by the norm: not stored
                        *len = c.n_nodes;
                        return CBX_GL_GET_ROWS_CONCAT_ADD_LAYER_NORM;
                    }
                }
                int32_t g1 = a.dst;
                const int32_t j = i + 1 + cast_after(i + 1, &g1);
                if (is(j, CBX_GOP_GET_ROWS)) {
                    int32_t g2 = nd[j].dst;
                    const int32_t k = j + 1 + cast_after(j + 1, &g2);
                    if (is(k, CBX_GOP_ADD) && nd[k].src[0] == g1 && nd[k].src[1] == g2 && same_dims(g1, g2) &&
                        internal(g1, 1) && internal(g2, 1)) {
                        const int32_t h = nd[k].dst;
                        if (layer_norm_at(k + 1) && nd[k + 1].src[0] == h) {
                            // h is the residual stream: stored unless only the norm reads it
                            if (internal(h, 1)) *flags = 1;
                            *len = k + 4 - i;
                            return CBX_GL_GET_ROWS_ADD_LAYER_NORM;
                        }
                        *len = k + 1 - i;
                        return CBX_GL_GET_ROWS_ADD;
                    }
                }
                *len = j - i;
                return CBX_GL_GET_ROWS;
            }
            case CBX_GOP_NORM: {
                if (layer_norm_rope_at(i)) {
                    *len = 5;
                    return CBX_GL_LAYER_NORM_ROPE;
                }
                const int32_t l = layer_norm_mish_at(i, a.src[0]);
                if (!l) return CBX_GL_NORM;
                *len = l;
                // causal_block1d's post-mask: mul(., mask) with one value per frame
                const int32_t z = nd[i + l - 1].dst;
                if (is(i + l, CBX_GOP_MUL) && nd[i + l].src[0] == z && internal(z, 1) &&
                    col_vec(nd[i + l].src[1], a.src[0])) {
                    *len = l + 1;
                    return CBX_GL_LAYER_NORM_MASK;
                }
                return CBX_GL_LAYER_NORM;
            }
            case CBX_GOP_ADD: {
                const int32_t x = a.src[0], t1 = a.dst;
                const bool bias = row_vec(a.src[1], x);
                // bias add -> residual add -> layer_norm [-> mish]
                if (bias && is(i + 1, CBX_GOP_ADD) && internal(t1, 1)) {
                    const cbx_gnode& r = nd[i + 1];
                    const int32_t other = r.src[0] == t1 ? r.src[1] : r.src[1] == t1 ? r.src[0] : -1;
                    const int32_t l = same_dims(other, x) ? layer_norm_mish_at(i + 2, r.dst) : 0;
                    if (l) {
                        if (internal(r.dst, 1)) *flags = 1;
                        *len = 2 + l;
                        return CBX_GL_ADD_LAYER_NORM;
                    }
                }
                // bias add -> heads view -> two broadcast adds
                if (const int32_t l = bias_pair_at(i)) {
                    *len = l;
                    return CBX_GL_BIAS_ADD_PAIR;
                }
                // bias add [-> view] -> residual add with no norm after it
                if (const int32_t l = bias_residual_at(i)) {
                    *len = l;
                    return CBX_GL_BIAS_RESIDUAL;
                }
                // score terms' add -> [scale] [mask] -> soft_max
                if (const int32_t l = add_soft_max_at(i)) {
                    *len = l;
                    return CBX_GL_SOFT_MAX;
                }
                // residual add -> layer_norm [-> mish]
                if (same_dims(a.src[1], x)) {
                    const int32_t l = layer_norm_mish_at(i + 1, t1);
                    if (l) {
                        if (internal(t1, 1)) *flags = 1;
                        *len = 1 + l;
                        return CBX_GL_ADD_LAYER_NORM;
                    }
                    if (!bias) {   // (a one-row x is also a bias add)
                        *flags = CBX_BINARY_ADD;
                        return CBX_GL_BINARY;
                    }
                }
                // bias add [-> activation]
                if (!bias && !col_vec(a.src[1], x)) {
                    *flags = CBX_BINARY_ADD;
                    return repeats(a.src[1], x) ? CBX_GL_BINARY : CBX_GL_UNSUPPORTED;
                }
                // bias add -> layer_norm [-> mish] (a linear's bias, then its
                // LayerNorm: flow_encoder.cpp:414-415), in the layouts the
                // fused kernel takes (else the two launches as before)
                if (const int32_t l = bias ? layer_norm_mish_at(i + 1, t1) : 0) {
                    const bool fits = ln_ext_fits(x) && ln_ext_fits(a.src[1]) && ln_ext_fits(nd[i + 2].src[1]) &&
                                      ln_ext_fits(nd[i + 3].src[1]) && ln_ext_fits(nd[i + l].dst) &&
                                      (internal(t1, 1) || ln_ext_fits(t1));
                    if (fits) {
                        if (internal(t1, 1)) *flags = 1;
                        *len = 1 + l;
                        return CBX_GL_ADD_LAYER_NORM;
                    }
                }
                if (is_unary(i + 1, CBX_UNARY_SOFTPLUS) && mish_at(i + 1, t1) && internal(t1, 2)) {
                    *len = 4;
                } else if (is(i + 1, CBX_GOP_UNARY) && nd[i + 1].src[0] == t1 && internal(t1, 1) &&
                           nd[i + 1].iparam >= CBX_UNARY_GELU && nd[i + 1].iparam <= CBX_UNARY_MISH) {
                    *len = 2;
                }
                return CBX_GL_BIAS_ACT;
            }
            case CBX_GOP_RMS_NORM:
                if (is(i + 1, CBX_GOP_MUL) && nd[i + 1].src[0] == a.dst && row_vec(nd[i + 1].src[1], a.src[0]) &&
                    internal(a.dst, 1)) {
                    *len = 2;
                }
                return CBX_GL_RMS_NORM;
            case CBX_GOP_GROUP_NORM: {
                int32_t y = a.dst;
                if (is(i + 1, CBX_GOP_MUL) && nd[i + 1].src[0] == a.dst && chan_vec(nd[i + 1].src[1], a.src[0]) &&
                    is(i + 2, CBX_GOP_ADD) && nd[i + 2].src[0] == nd[i + 1].dst &&
                    chan_vec(nd[i + 2].src[1], a.src[0]) && internal(a.dst, 1) && internal(nd[i + 1].dst, 1)) {
                    y = nd[i + 2].dst;
                    *len = 3;
                }
                if (mish_at(i + *len, y) && internal(y, 2)) *len += 3;
                return CBX_GL_GROUP_NORM;
            }
            case CBX_GOP_SCALE:
            case CBX_GOP_DIAG_MASK_INF: {
                // scale and the mask only fuse into a plain soft_max: a
                // soft_max with its own scale would round twice
                int32_t j = i, prev = a.src[0];
                bool chain = true;
                if (is(j, CBX_GOP_SCALE)) prev = nd[j++].dst;
                if (is(j, CBX_GOP_DIAG_MASK_INF) && (j == i || (nd[j].src[0] == prev && internal(prev, 1)))) {
                    if (nd[j].iparam < 0) chain = false;
                    else prev = nd[j++].dst;
                }
                if (chain && is(j, CBX_GOP_SOFT_MAX) && nd[j].src[0] == prev && internal(prev, 1) &&
                    nd[j].src[1] < 0 && nd[j].fparam == 1.0f) {
                    *len = j + 1 - i;
                    return CBX_GL_SOFT_MAX;
                }
                // a scale on its own (the mean of a HiFT stage's resblocks)
                return a.op == CBX_GOP_SCALE ? CBX_GL_SCALE : CBX_GL_UNSUPPORTED;
            }
            case CBX_GOP_SOFT_MAX:
                return a.src[1] < 0 ? CBX_GL_SOFT_MAX : CBX_GL_UNSUPPORTED;
            case CBX_GOP_MUL: {
                const int32_t x = a.src[0], al = a.src[1];
                const bool bcast = row_vec(al, x) || (valid_t(x) && dims(al, 1, t[x].ne[1], 1, 1));
                if (bcast && is_unary(i + 1, CBX_UNARY_SIN) && nd[i + 1].src[0] == a.dst &&
                    is_unary(i + 2, CBX_UNARY_SQR) && nd[i + 2].src[0] == nd[i + 1].dst && is(i + 3, CBX_GOP_MUL) &&
                    nd[i + 3].src[0] == nd[i + 2].dst && same_dims(nd[i + 3].src[1], al) && is(i + 4, CBX_GOP_ADD) &&
                    nd[i + 4].src[0] == x && nd[i + 4].src[1] == nd[i + 3].dst && internal(a.dst, 1) &&
                    internal(nd[i + 1].dst, 1) && internal(nd[i + 2].dst, 1) && internal(nd[i + 3].dst, 1)) {
                    // snake() as the prologue of a conv: one conv launch.
                    // The conv's prologue reads alpha per input channel,
                    // i.e. along ne0 of the (C, T) input: a (1, T) alpha
                    // (one value per frame) is a snake of its own.
                    const int32_t h = nd[i + 4].dst;
                    const bool per_channel = row_vec(al, x) && row_vec(nd[i + 3].src[1], x);
                    int32_t n = 0, fl = 1;
                    const int32_t k = per_channel && internal(h, 1) ? conv_chain_at(i + 5, h, &n, &fl)
                                                                    : CBX_GL_UNSUPPORTED;
                    if (k != CBX_GL_UNSUPPORTED) {
                        *len = 5 + n;
                        *flags = fl;
                        return k;
                    }
                    *len = 5;
                    return CBX_GL_SNAKE;
                }
                // causal_block1d's mul(x, mask (1, T)) before a causal conv
                if (valid_t(x) && dims(al, 1, t[x].ne[1], 1, 1) && internal(a.dst, 1)) {
                    int32_t fl = 3;
                    const int32_t n = causal_at(i + 1, a.dst, &fl);
                    if (n) {
                        *len = 1 + n;
                        *flags = fl;
                        return CBX_GL_CAUSAL_CONV1D;
                    }
                }
                *flags = CBX_BINARY_MUL;
                return repeats(al, x) ? CBX_GL_BINARY : CBX_GL_UNSUPPORTED;
            }
            case CBX_GOP_UNARY: {
                const int32_t x = a.src[0];
                if (a.iparam == CBX_UNARY_SOFTPLUS && mish_at(i, x)) {
                    *len = 3;
                    return CBX_GL_UNARY;
                }
                if (a.iparam == CBX_UNARY_SILU && is(i + 1, CBX_GOP_MUL) && nd[i + 1].src[0] == a.dst &&
                    same_dims(nd[i + 1].src[1], x) && internal(a.dst, 1)) {
                    *len = 2;
                    return CBX_GL_SWIGLU;
                }
                return a.iparam >= CBX_UNARY_GELU && a.iparam <= CBX_UNARY_MISH ? CBX_GL_UNARY : CBX_GL_UNSUPPORTED;
            }
            case CBX_GOP_LEAKY_RELU: {
                int32_t n = 0, fl = 2;
                const int32_t k = internal(a.dst, 1) ? conv_chain_at(i + 1, a.dst, &n, &fl) : CBX_GL_UNSUPPORTED;
                if (k != CBX_GL_UNSUPPORTED) {
                    *len = 1 + n;
                    *flags = fl;
                    return k;
                }
                return CBX_GL_LEAKY_RELU;
            }
            case CBX_GOP_ROPE:
                return CBX_GL_ROPE;
            case CBX_GOP_CPY:
                return CBX_GL_CPY;
            case CBX_GOP_CONCAT:
                return CBX_GL_CONCAT;
            default:
                return CBX_GL_UNSUPPORTED;
        }
    }
};

const char* op_name(int op) {
    switch (op) {
        case CBX_GOP_VIEW: return "VIEW";
        case CBX_GOP_GET_ROWS: return "GET_ROWS";
        case CBX_GOP_ADD: return "ADD";
        case CBX_GOP_MUL: return "MUL";
        case CBX_GOP_SCALE: return "SCALE";
        case CBX_GOP_NORM: return "NORM";
        case CBX_GOP_RMS_NORM: return "RMS_NORM";
        case CBX_GOP_GROUP_NORM: return "GROUP_NORM";
        case CBX_GOP_ROPE: return "ROPE";
        case CBX_GOP_SOFT_MAX: return "SOFT_MAX";
        case CBX_GOP_DIAG_MASK_INF: return "DIAG_MASK_INF";
        case CBX_GOP_UNARY: return "UNARY";
        case CBX_GOP_LEAKY_RELU: return "LEAKY_RELU";
        case CBX_GOP_CPY: return "CPY";
        case CBX_GOP_IM2COL: return "IM2COL";
        case CBX_GOP_MUL_MAT: return "MUL_MAT";
        case CBX_GOP_CONV_TRANSPOSE_1D: return "CONV_TRANSPOSE_1D";
        case CBX_GOP_CONCAT: return "CONCAT";
        default: return "unknown op";
    }
}

// The bias adds at nodes i and i + 1 neither read nor write what the other
// writes (by bytes), neither output meets its own bias, and each bias is a
// row of its x: the two may run side by side in one launch.
bool independent_adds(const cbx_tensor* t, const cbx_gnode* nd, int32_t i) {
    const cbx_gnode &a = nd[i], &b = nd[i + 1];
    if (a.op != CBX_GOP_ADD || b.op != CBX_GOP_ADD) return false;
    for (const cbx_gnode* g : {&a, &b}) {
        if (g->src[0] < 0 || g->src[1] < 0) return false;
        const cbx_tensor &x = t[g->src[0]], &bias = t[g->src[1]], &y = t[g->dst];
        if (x.type != CBX_TYPE_F32 || bias.type != CBX_TYPE_F32 || y.type != CBX_TYPE_F32 || !same_shape(&x, &y) ||
            !is_contiguous(&bias) || bias.ne[0] != x.ne[0] || nelements(&bias) != bias.ne[0]) {
            return false;
        }
    }
    const cbx_tensor *ya = &t[a.dst], *yb = &t[b.dst];
    return !bytes_overlap(ya, &t[b.src[0]]) && !bytes_overlap(ya, &t[b.src[1]]) && !bytes_overlap(ya, yb) &&
           !bytes_overlap(yb, &t[a.src[0]]) && !bytes_overlap(yb, &t[a.src[1]]) && !bytes_overlap(ya, &t[a.src[1]]) &&
           !bytes_overlap(yb, &t[b.src[1]]);
}

// Nodes i and i + 1 neither read nor write what the other writes, by
// tensor bytes: they may run side by side in one launch.
bool independent_nodes(const cbx_tensor* t, const cbx_gnode* nd, int32_t i) {
    const cbx_gnode &a = nd[i], &b = nd[i + 1];
    const cbx_tensor *ya = &t[a.dst], *yb = &t[b.dst];
    if (bytes_overlap(ya, yb)) return false;
    for (int32_t s : b.src) {
        if (s >= 0 && bytes_overlap(ya, &t[s])) return false;
    }
    for (int32_t s : a.src) {
        if (s >= 0 && bytes_overlap(yb, &t[s])) return false;
    }
    return true;
}

int check_lists(const cbx_tensor* tensors, int32_t n_tensors, const cbx_gnode* nodes, int32_t n_nodes,
                const char* what) {
    if ((!tensors && n_tensors) || n_tensors < 0 || (!nodes && n_nodes) || n_nodes < 0) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": bad tensor or node array");
    }
    for (int32_t i = 0; i < n_nodes; i++) {
        bool ok = nodes[i].dst >= 0 && nodes[i].dst < n_tensors;
        for (int32_t s : nodes[i].src) ok = ok && s >= -1 && s < n_tensors;
        if (!ok) {
            return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": node " + std::to_string(i) +
                                                      " names a tensor index out of range");
        }
    }
    return CBX_OK;
}

int plan(const cbx_tensor* tensors, int32_t n_tensors, const cbx_gnode* nodes, int32_t n_nodes, const int32_t* keep,
         int32_t n_keep, std::vector<cbx_glaunch>* out, const char* what) {
    int rc = check_lists(tensors, n_tensors, nodes, n_nodes, what);
    if (rc) return rc;
    if ((!keep && n_keep) || n_keep < 0) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": bad keep array");
    Planner p{tensors, n_tensors, nodes, n_nodes, std::vector<int32_t>(static_cast<size_t>(n_tensors), 0),
              std::vector<char>(static_cast<size_t>(n_tensors), 0)};
    for (int32_t k = 0; k < n_keep; k++) {
        if (!p.valid_t(keep[k])) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": keep index out of range");
        p.keep[static_cast<size_t>(keep[k])] = 1;
    }
    for (int32_t i = 0; i < n_nodes; i++) {
        for (int32_t s : nodes[i].src) {
            if (s >= 0) p.uses[static_cast<size_t>(s)]++;
        }
    }
    for (int32_t i = 0; i < n_nodes;) {
        int32_t len = 1, flags = 0;
        const int32_t kind = p.match(i, &len, &flags);
        // two lone bias adds in a row that do not read each other (the
        // projections of v and k, flow_encoder.cpp:320-322): one launch
        if (kind == CBX_GL_BIAS_ACT && len == 1 && !out->empty() && out->back().kind == CBX_GL_BIAS_ACT &&
            out->back().n_nodes == 1 && out->back().first_node == i - 1 && independent_adds(tensors, nodes, i - 1)) {
            out->back() = cbx_glaunch{CBX_GL_BIAS_ADD_TWO, i - 1, 2, 0};
            i += 1;
            continue;
        }
        // two RoPEs in a row on separate tensors (q and k, s3enc.cpp:215-229)
        if (kind == CBX_GL_ROPE && !out->empty() && out->back().kind == CBX_GL_ROPE &&
            out->back().first_node == i - 1 && independent_nodes(tensors, nodes, i - 1)) {
            out->back() = cbx_glaunch{CBX_GL_ROPE_TWO, i - 1, 2, 0};
            i += 1;
            continue;
        }
        out->push_back(cbx_glaunch{kind, i, kind == CBX_GL_UNSUPPORTED ? 1 : len, flags});
        i += out->back().n_nodes;
    }
    return CBX_OK;
}

const cbx_tensor* T(const cbx_tensor* t, int32_t i) { return i >= 0 ? &t[i] : nullptr; }

// Node counts a launch of each kind may span.
constexpr int32_t kSpan[][2] = {
    {1, 1},  // UNSUPPORTED
    {1, 1},  // VIEW
    {1, 2},  // GET_ROWS [cast]
    {3, 5},  // GET_ROWS_ADD
    {6, 8},  // GET_ROWS_ADD_LAYER_NORM
    {1, 1},  // NORM
    {3, 6},  // LAYER_NORM [mish]
    {5, 5},  // LAYER_NORM_ROPE
    {1, 2},  // RMS_NORM [mul]
    {1, 6},  // GROUP_NORM [affine] [mish]
    {1, 4},  // SOFT_MAX [add] [scale] [mask]
    {5, 5},  // SNAKE
    {1, 3},  // UNARY / mish
    {2, 2},  // SWIGLU
    {1, 1},  // LEAKY_RELU
    {1, 1},  // ROPE
    {1, 1},  // CPY
    {4, 8},  // ADD_LAYER_NORM [bias] [mish]
    {4, 7},  // LAYER_NORM_MASK [mish]
    {1, 4},  // BIAS_ACT [act | mish]
    {9, 19}, // CONV1D [snake | leaky] [bias] [residual [sum [scale]]]
    {7, 14}, // CONV_TRANSPOSE1D [snake | leaky] [bias]
    {12, 15}, // CAUSAL_CONV1D [mask] [bias]
    {7, 12},  // GET_ROWS_CONCAT_ADD_LAYER_NORM [prompt gather, concat] [casts]
    {1, 1},  // BINARY
    {1, 1},  // CONCAT
    {2, 3},  // BIAS_RESIDUAL [view]
    {1, 1},  // SCALE
    {4, 6},  // BIAS_ADD_PAIR [views of u, v]
    {2, 2},  // BIAS_ADD_TWO
    {2, 2},  // ROPE_TWO
};
constexpr int32_t kLastKind = CBX_GL_ROPE_TWO;
static_assert(sizeof(kSpan) / sizeof(kSpan[0]) == kLastKind + 1, "one span per launch kind");

// Issues the entry point a launch maps to.  A launch is only read within
// the node list, so one not made by the planner cannot read past it.
int run(const cbx_tensor* t, const cbx_gnode* nd, int32_t n_nodes, const cbx_glaunch& l, cbx_stream s) {
    if (l.kind < CBX_GL_UNSUPPORTED || l.kind > kLastKind || l.first_node < 0 || l.n_nodes < kSpan[l.kind][0] ||
        l.n_nodes > kSpan[l.kind][1] || l.first_node > n_nodes - l.n_nodes) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: launch does not fit the node list");
    }
    const int32_t f = l.first_node;
    const cbx_gnode& a = nd[f];
    cbx_tensor* y = const_cast<cbx_tensor*>(&t[nd[f + l.n_nodes - 1].dst]);
    switch (l.kind) {
        case CBX_GL_UNSUPPORTED:
            return set_error(CBX_ERR_UNSUPPORTED, std::string("cbx_graph_launch: node ") + std::to_string(f) + " (" +
                                                      op_name(a.op) + ") starts no chain the library runs");
        case CBX_GL_VIEW:
            return CBX_OK;
        case CBX_GL_GET_ROWS:
            return cbx_get_rows(T(t, a.src[0]), T(t, a.src[1]), y, s);
        case CBX_GL_GET_ROWS_ADD:
        case CBX_GL_GET_ROWS_ADD_LAYER_NORM: {
            const int32_t k_add = l.kind == CBX_GL_GET_ROWS_ADD ? f + l.n_nodes - 1 : f + l.n_nodes - 4;
            const int32_t j = nd[f + 1].op == CBX_GOP_CPY ? f + 2 : f + 1;   // the second gather
            const cbx_gnode& b = nd[j];
            if (l.kind == CBX_GL_GET_ROWS_ADD) {
                return cbx_get_rows_add(T(t, a.src[0]), T(t, a.src[1]), T(t, b.src[0]), T(t, b.src[1]), y, s);
            }
            cbx_tensor* h = (l.flags & 1) ? nullptr : const_cast<cbx_tensor*>(&t[nd[k_add].dst]);
            return cbx_get_rows_add_layer_norm(T(t, a.src[0]), T(t, a.src[1]), T(t, b.src[0]), T(t, b.src[1]),
                                               T(t, nd[k_add + 2].src[1]), T(t, nd[k_add + 3].src[1]),
                                               nd[k_add + 1].fparam, h, y, s);
        }
        case CBX_GL_GET_ROWS_CONCAT_ADD_LAYER_NORM: {
            ConcatT3 c;
            if (!parse_concat_t3(nd, n_nodes, f, &c) || c.n_nodes != l.n_nodes) break;
            bool f32_casts = true;
            for (int32_t q = 0; q < c.n_cast; q++) f32_casts = f32_casts && t[nd[c.cast[q]].dst].type == CBX_TYPE_F32;
            if (!f32_casts) break;
            const cbx_gnode &ga = nd[c.g_a < 0 ? c.g_b : c.g_a], &gb = nd[c.g_b], &gp = nd[c.g_pos];
            cbx_tensor* h = (l.flags & 1) ? nullptr : const_cast<cbx_tensor*>(&t[nd[c.add].dst]);
            return cbx_get_rows_concat_add_layer_norm(
                T(t, c.prefix), c.g_a < 0 ? nullptr : T(t, ga.src[0]), c.g_a < 0 ? nullptr : T(t, ga.src[1]),
                T(t, gb.src[0]), T(t, gb.src[1]), T(t, gp.src[0]), T(t, gp.src[1]), T(t, nd[c.add + 2].src[1]),
                T(t, nd[c.add + 3].src[1]), nd[c.add + 1].fparam, h, y, s);
        }
        case CBX_GL_NORM:
            return cbx_norm(T(t, a.src[0]), a.fparam, y, s);
        case CBX_GL_LAYER_NORM:
            if (l.n_nodes != 3 && l.n_nodes != 6) break;
            return cbx_layer_norm(T(t, a.src[0]), T(t, nd[f + 1].src[1]), T(t, nd[f + 2].src[1]), a.fparam,
                                  l.n_nodes == 6 ? CBX_UNARY_MISH : CBX_UNARY_NONE, y, s);
        case CBX_GL_LAYER_NORM_ROPE: {
            const cbx_tensor* x = T(t, a.src[0]);
            if (!x) break;
            // the rope output re-described with the rows' shape (C, n_tok, batch)
            cbx_tensor out = *y;
            out.ne[0] = x->ne[0];
            out.ne[1] = x->ne[1];
            out.ne[2] = x->ne[2];
            out.ne[3] = 1;
            out.nb[0] = sizeof(float);
            for (int k = 1; k < 4; k++) out.nb[k] = out.nb[k - 1] * static_cast<size_t>(out.ne[k - 1]);
            const cbx_gnode& r = nd[f + 4];
            return cbx_layer_norm_rope(x, T(t, nd[f + 1].src[1]), T(t, nd[f + 2].src[1]), a.fparam,
                                       t[nd[f + 3].dst].ne[0], T(t, r.src[1]), r.rope, &out, s);
        }
        case CBX_GL_RMS_NORM:
            if (l.n_nodes == 2) return cbx_rms_norm_mul(T(t, a.src[0]), T(t, nd[f + 1].src[1]), a.fparam, y, s);
            return cbx_rms_norm(T(t, a.src[0]), a.fparam, y, s);
        case CBX_GL_GROUP_NORM: {
            if (l.n_nodes == 2 || l.n_nodes == 5) break;
            const bool affine = l.n_nodes == 3 || l.n_nodes == 6;
            const bool mish = l.n_nodes == 4 || l.n_nodes == 6;
            return cbx_group_norm(T(t, a.src[0]), a.iparam, a.fparam, affine ? T(t, nd[f + 1].src[1]) : nullptr,
                                  affine ? T(t, nd[f + 2].src[1]) : nullptr, mish ? CBX_UNARY_MISH : CBX_UNARY_NONE, y,
                                  s);
        }
        case CBX_GL_SOFT_MAX: {
            if (l.n_nodes == 1) {
                if (a.op != CBX_GOP_SOFT_MAX) break;
                return cbx_scale_diag_mask_soft_max(T(t, a.src[0]), a.fparam, -1, y, s);
            }
            const bool add = a.op == CBX_GOP_ADD;
            float scale = 1.0f;
            int32_t n_past = -1;
            bool chain = nd[f + l.n_nodes - 1].op == CBX_GOP_SOFT_MAX;
            for (int32_t k = add ? f + 1 : f; k < f + l.n_nodes - 1; k++) {
                chain = chain && (nd[k].op == CBX_GOP_SCALE || nd[k].op == CBX_GOP_DIAG_MASK_INF);
            }
            if (!chain) break;
            for (int32_t k = add ? f + 1 : f; k < f + l.n_nodes - 1; k++) {
                if (nd[k].op == CBX_GOP_SCALE) scale = nd[k].fparam;
                if (nd[k].op == CBX_GOP_DIAG_MASK_INF) {
                    if (nd[k].iparam < 0) {
                        return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: DIAG_MASK_INF needs n_past >= 0");
                    }
                    n_past = nd[k].iparam;
                }
            }
            if (add) return cbx_add_scale_diag_mask_soft_max(T(t, a.src[0]), T(t, a.src[1]), scale, n_past, y, s);
            return cbx_scale_diag_mask_soft_max(T(t, a.src[0]), scale, n_past, y, s);
        }
        case CBX_GL_SNAKE:
            return cbx_snake(T(t, a.src[0]), T(t, a.src[1]), T(t, nd[f + 3].src[1]), y, s);
        case CBX_GL_UNARY:
            if (l.n_nodes == 3) return cbx_unary(CBX_UNARY_MISH, T(t, a.src[0]), y, s);
            if (l.n_nodes != 1) break;
            return cbx_unary(a.iparam, T(t, a.src[0]), y, s);
        case CBX_GL_SWIGLU:
            return cbx_swiglu(T(t, a.src[0]), T(t, nd[f + 1].src[1]), y, s);
        case CBX_GL_LEAKY_RELU:
            return cbx_leaky_relu(T(t, a.src[0]), a.fparam, y, s);
        case CBX_GL_ROPE:
            return cbx_rope_ext(T(t, a.src[0]), T(t, a.src[1]), a.rope, y, s);
        case CBX_GL_ROPE_TWO: {
            const cbx_gnode& b = nd[f + 1];
            if (a.op != CBX_GOP_ROPE || b.op != CBX_GOP_ROPE) break;
            cbx_op ops[2] = {};
            for (int k = 0; k < 2; k++) {
                const cbx_gnode& g = nd[f + k];
                ops[k].kind = CBX_OP_ROPE;
                ops[k].src[0] = T(t, g.src[0]);
                ops[k].src[1] = T(t, g.src[1]);
                ops[k].dst[0] = const_cast<cbx_tensor*>(&t[g.dst]);
                ops[k].rope = g.rope;
            }
            const int rc = cbx_run_ops(ops, 2, s);
            if (rc != CBX_ERR_UNSUPPORTED) return rc;
            // a layout the one-launch kernel does not take (nothing was
            // launched): the two RoPEs one after the other
            const int r0 = cbx_rope_ext(T(t, a.src[0]), T(t, a.src[1]), a.rope, const_cast<cbx_tensor*>(&t[a.dst]), s);
            return r0 ? r0 : cbx_rope_ext(T(t, b.src[0]), T(t, b.src[1]), b.rope, y, s);
        }
        case CBX_GL_CPY:
            return cbx_cpy(T(t, a.src[0]), y, s);
        case CBX_GL_BINARY:
            if (a.op != (l.flags == CBX_BINARY_MUL ? CBX_GOP_MUL : CBX_GOP_ADD)) break;
            return cbx_binary(l.flags, T(t, a.src[0]), T(t, a.src[1]), y, s);
        case CBX_GL_BIAS_ADD_TWO: {
            const cbx_gnode& b = nd[f + 1];
            if (a.op != CBX_GOP_ADD || b.op != CBX_GOP_ADD) break;
            return cbx_bias_add_two(T(t, a.src[0]), T(t, a.src[1]), const_cast<cbx_tensor*>(&t[a.dst]),
                                    T(t, b.src[0]), T(t, b.src[1]), y, s);
        }
        case CBX_GL_BIAS_ADD_PAIR: {
            // the heads view, then views of other tensors and the two adds
            const cbx_gnode& v = nd[f + 1];
            if (a.op != CBX_GOP_ADD || v.op != CBX_GOP_VIEW || v.src[0] != a.dst) break;
            int32_t k_add[2], n_add = 0;
            for (int32_t k = f + 2; k < f + l.n_nodes; k++) {
                if (nd[k].op == CBX_GOP_ADD && nd[k].src[0] == v.dst && n_add < 2) k_add[n_add++] = k;
                else if (nd[k].op != CBX_GOP_VIEW || nd[k].src[0] == a.dst || nd[k].src[0] == v.dst) n_add = 3;
            }
            if (n_add != 2 || k_add[1] != f + l.n_nodes - 1) break;
            const cbx_gnode &pu = nd[k_add[0]], &pv = nd[k_add[1]];
            const cbx_tensor *X = T(t, a.src[0]), *B = T(t, a.src[1]), *S = T(t, a.dst), *V = T(t, v.dst);
            if (!X || !B || !S || !V) break;
            const int kb = lead_dims(*V, X->ne[0]);
            if (!is_contiguous(X) || !is_contiguous(B) || !is_contiguous(S) || !is_contiguous(V) || V->data != S->data ||
                nelements(V) != nelements(X) || !same_shape(S, X) || B->ne[0] != X->ne[0] ||
                nelements(B) != B->ne[0] || kb < 0) {
                return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: node " + std::to_string(f + 1) +
                                                          ": the view is not a contiguous reshape of the biased sum");
            }
            // x and the bias re-described over the view's dims (the sum is
            // never stored, the two adds read it through the view)
            cbx_tensor xv = *V, bv = *V;
            xv.data = X->data;
            bv.data = B->data;
            for (int k = kb; k < 4; k++) bv.ne[k] = 1;
            for (int k = 1; k < 4; k++) bv.nb[k] = bv.nb[k - 1] * static_cast<size_t>(bv.ne[k - 1]);
            return cbx_bias_add_pair(&xv, &bv, T(t, pu.src[1]), T(t, pv.src[1]),
                                     const_cast<cbx_tensor*>(&t[pu.dst]), y, s);
        }
        case CBX_GL_BIAS_RESIDUAL: {
            const cbx_gnode& last = nd[f + l.n_nodes - 1];
            int32_t sum = a.dst;
            if (l.n_nodes == 3) {
                const cbx_gnode& v = nd[f + 1];
                if (v.op != CBX_GOP_VIEW || v.src[0] != a.dst || v.dst < 0 || a.dst < 0 ||
                    t[v.dst].data != t[a.dst].data || !same_shape(&t[v.dst], &t[a.dst]) ||
                    !is_contiguous(&t[v.dst]) || !is_contiguous(&t[a.dst])) {
                    break;
                }
                sum = v.dst;
            }
            const int32_t r = last.src[0] == sum ? last.src[1] : last.src[1] == sum ? last.src[0] : -1;
            if (a.op != CBX_GOP_ADD || last.op != CBX_GOP_ADD || r < 0) break;
            return cbx_bias_residual(T(t, a.src[0]), T(t, a.src[1]), T(t, r), y, s);
        }
        case CBX_GL_SCALE:
            if (a.op != CBX_GOP_SCALE) break;
            return cbx_scale(T(t, a.src[0]), a.fparam, y, s);
        case CBX_GL_CONCAT:
            return cbx_concat(T(t, a.src[0]), T(t, a.src[1]), a.iparam, y, s);
        case CBX_GL_ADD_LAYER_NORM: {
            if (l.n_nodes == 6) break;
            const bool bias = l.n_nodes == 5 || l.n_nodes == 8;
            // 4 or 7 nodes: add(a, r) of one shape, or add(a, bias) with no
            // residual (bias a row of a)
            const cbx_tensor *a0 = T(t, a.src[0]), *a1 = T(t, a.src[1]);
            if (!bias && a0 && a1 && !same_shape(a0, a1) && a1->ne[0] == a0->ne[0] && nelements(a1) == a1->ne[0]) {
                const int32_t ln = f + 1;
                cbx_tensor* sum = (l.flags & 1) ? nullptr : const_cast<cbx_tensor*>(&t[a.dst]);
                return cbx_add_layer_norm(a0, a1, nullptr, T(t, nd[ln + 1].src[1]), T(t, nd[ln + 2].src[1]),
                                          nd[ln].fparam, l.n_nodes == 7 ? CBX_UNARY_MISH : CBX_UNARY_NONE, sum, y, s);
            }
            const int32_t k = bias ? f + 1 : f;        // the residual add
            const int32_t ln = k + 1;                  // the norm
            const cbx_gnode& r = nd[k];
            const int32_t other = !bias ? r.src[1] : r.src[0] == a.dst ? r.src[1] : r.src[0];
            cbx_tensor* sum = (l.flags & 1) ? nullptr : const_cast<cbx_tensor*>(&t[r.dst]);
            return cbx_add_layer_norm(T(t, a.src[0]), bias ? T(t, a.src[1]) : nullptr, T(t, other),
                                      T(t, nd[ln + 1].src[1]), T(t, nd[ln + 2].src[1]), nd[ln].fparam,
                                      l.n_nodes >= 7 ? CBX_UNARY_MISH : CBX_UNARY_NONE, sum, y, s);
        }
        case CBX_GL_LAYER_NORM_MASK:
            if (l.n_nodes != 4 && l.n_nodes != 7) break;
            return cbx_layer_norm_mask(T(t, a.src[0]), T(t, nd[f + 1].src[1]), T(t, nd[f + 2].src[1]), a.fparam,
                                       l.n_nodes == 7 ? CBX_UNARY_MISH : CBX_UNARY_NONE,
                                       T(t, nd[f + l.n_nodes - 1].src[1]), y, s);
        case CBX_GL_BIAS_ACT: {
            if (l.n_nodes == 3) break;
            const int act = l.n_nodes == 1 ? CBX_UNARY_NONE : l.n_nodes == 4 ? CBX_UNARY_MISH : nd[f + 1].iparam;
            return cbx_bias_act(act, T(t, a.src[0]), T(t, a.src[1]), y, s);
        }
        case CBX_GL_CONV1D:
        case CBX_GL_CONV_TRANSPOSE1D: {
            // the layout the flags describe: prologue, body, bias, residual
            // [, the sum [, its scale]]
            const int pro = l.flags & 3;
            const bool bias = (l.flags & 4) != 0, res = (l.flags & 8) != 0;
            const bool sum = (l.flags & 16) != 0, scl = (l.flags & 32) != 0;
            const bool tr = l.kind == CBX_GL_CONV_TRANSPOSE1D;
            const int32_t p = pro == 1 ? 5 : pro == 2 ? 1 : 0;
            const int32_t n_res = p + (tr ? 7 : 9) + (bias ? 2 : 0) + (res ? 1 : 0);   // nodes up to the residual add
            if (pro == 3 || (tr && (res || sum)) || (sum && !res) || (scl && !sum) ||
                l.n_nodes != n_res + (sum ? 1 : 0) + (scl ? 1 : 0)) {
                break;
            }
            const int32_t b0 = f + p;   // the transpose view
            const cbx_tensor* x = T(t, a.src[0]);
            const cbx_tensor* al = pro == 1 ? T(t, a.src[1]) : nullptr;
            const cbx_tensor* ai = pro == 1 ? T(t, nd[f + 3].src[1]) : nullptr;
            const float slope = pro == 2 ? a.fparam : 0.0f;
            const int cp = pro == 1 ? CBX_CONV_PRO_SNAKE : pro == 2 ? CBX_CONV_PRO_LEAKY_RELU : CBX_CONV_PRO_NONE;
            const int32_t bview = b0 + (tr ? 5 : 7);   // the bias view, when there is one
            const cbx_tensor* bt = bias ? T(t, nd[bview].src[0]) : nullptr;
            // the prepared weights must be the node's weight tensor's
            const cbx_gnode& wn = nd[b0 + (tr ? 2 : 5)];
            const cbx_tensor* wk = T(t, nd[b0 + 2].src[0]);
            if (!wk || !conv1d_weights_match(wn.conv_w, tr ? wn.conv[0] : 0, wk->ne[0], tr ? wk->ne[2] : wk->ne[1],
                                             tr ? wk->ne[1] : wk->ne[2])) {
                return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: node " + std::to_string(b0 + (tr ? 2 : 5)) +
                                                          ": conv_w was not made from the node's weight tensor");
            }
            if (!tr) {
                const cbx_gnode& ic = nd[b0 + 2];
                const cbx_tensor* r = nullptr;
                if (res) {
                    const cbx_gnode& ra = nd[f + n_res - 1];   // add(residual, conv out)
                    const int32_t out = nd[f + n_res - 2].dst;
                    r = T(t, ra.src[0] == out ? ra.src[1] : ra.src[0]);
                }
                if (!sum) {
                    return cbx_conv1d(x, nd[b0 + 5].conv_w, ic.conv[0], ic.conv[1], ic.conv[2], cp, al, ai, slope, bt,
                                      r, y, s);
                }
                const cbx_gnode& sa = nd[f + n_res];          // add(acc, residual's result)
                const int32_t rr = nd[f + n_res - 1].dst;
                if (sa.op != CBX_GOP_ADD || (sa.src[0] != rr && sa.src[1] != rr)) break;
                const cbx_tensor* acc = T(t, sa.src[0] == rr ? sa.src[1] : sa.src[0]);
                float sc = 1.0f;
                if (scl) {
                    const cbx_gnode& sn = nd[f + n_res + 1];
                    if (sn.op != CBX_GOP_SCALE || sn.src[0] != sa.dst) break;
                    sc = sn.fparam;
                }
                return cbx_conv1d_sum(x, nd[b0 + 5].conv_w, ic.conv[0], ic.conv[1], ic.conv[2], cp, al, ai, slope, bt,
                                      r, acc, sc, y, s);
            }
            // the crop: the view's offset into the full output, in frames
            const cbx_tensor* full = T(t, nd[b0 + 2].dst);
            const cbx_tensor* crop = T(t, nd[b0 + 3].dst);
            if (!full || !crop) break;
            const int64_t off = static_cast<const char*>(crop->data) - static_cast<const char*>(full->data);
            if (off < 0 || off % 4 || off / 4 > (int64_t{1} << 30)) break;
            return cbx_conv_transpose1d(x, nd[b0 + 2].conv_w, static_cast<int>(off / 4), cp, al, ai, slope, bt, y, s);
        }
        case CBX_GL_CAUSAL_CONV1D: {
            // [mask ->] 12 nodes [+ bias 2]
            const bool masked = (l.flags & 3) == 3, bias = (l.flags & 4) != 0;
            if (((l.flags & 3) != 0 && !masked) || (l.flags & 8) ||
                l.n_nodes != (masked ? 1 : 0) + 12 + (bias ? 2 : 0)) {
                break;
            }
            const int32_t b0 = f + (masked ? 1 : 0);   // the transpose view
            const cbx_gnode& wn = nd[b0 + 9];
            const cbx_tensor* wk = T(t, nd[b0 + 6].src[0]);
            if (!wk || !conv1d_weights_match(wn.conv_w, 0, wk->ne[0], wk->ne[1], wk->ne[2])) {
                return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: node " + std::to_string(b0 + 9) +
                                                          ": conv_w was not made from the node's weight tensor");
            }
            return cbx_causal_conv1d(T(t, a.src[0]), wn.conv_w, masked ? T(t, a.src[1]) : nullptr,
                                     bias ? T(t, nd[b0 + 10].src[0]) : nullptr, y, s);
        }
        default:
            break;
    }
    return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: launch does not fit the node list");
}

}  // namespace

extern "C" {

int cbx_graph_plan(const cbx_tensor* tensors, int32_t n_tensors, const cbx_gnode* nodes, int32_t n_nodes,
                   const int32_t* keep, int32_t n_keep, cbx_glaunch* launches, int32_t max_launches,
                   int32_t* n_launches) {
    clear_error();
    std::vector<cbx_glaunch> ls;
    const int rc = plan(tensors, n_tensors, nodes, n_nodes, keep, n_keep, &ls, "cbx_graph_plan");
    if (n_launches) *n_launches = static_cast<int32_t>(ls.size());
    if (rc) return rc;
    if (static_cast<int64_t>(ls.size()) > max_launches || (!launches && !ls.empty())) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_plan: " + std::to_string(ls.size()) +
                                                  " launches do not fit max_launches");
    }
    for (size_t k = 0; k < ls.size(); k++) launches[k] = ls[k];
    return CBX_OK;
}

int cbx_graph_launch(const cbx_tensor* tensors, int32_t n_tensors, const cbx_gnode* nodes, int32_t n_nodes,
                     const cbx_glaunch* launch, cbx_stream stream) {
    clear_error();
    int rc = check_lists(tensors, n_tensors, nodes, n_nodes, "cbx_graph_launch");
    if (rc) return rc;
    if (!launch) return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_launch: launch is NULL");
    return run(tensors, nodes, n_nodes, *launch, stream);
}

// A planned node list recorded into a HIP graph.  The graph holds the
// kernels' arguments as they were when it was captured (the tensors'
// addresses and shapes, the nodes' parameters); a replay runs the same
// launches on whatever those buffers hold then.
//
// Two instantiations of it take turns: launches replay inst[cur]; an update
// re-points the other one, inst[1 - cur], and makes it current.  So an
// update never changes the arguments of the instantiation whose replays may
// still be queued: it waits only for the other one's replays, all issued
// before the previous update.  Events recorded by each update, on every
// stream the exec was launched on since the one before, mark them (one
// event a stream per update, none per replay).
//
// Each instantiation remembers the plan it holds, each launch's signature
// (every value its kernels are built from) and which of its graph's kernel
// nodes each launch issued.  An update whose plan has the same launches
// re-records only the launches whose signature changed and sets their
// kernel nodes' arguments in the instantiated graph (a decode loop's next
// token changes a few launches of many); anything else records the whole
// list and updates or re-instantiates the graph.
struct GraphInst {
    hipGraph_t graph = nullptr;            // the graph `exec` was instantiated from
    hipGraphExec_t exec = nullptr;
    int32_t n_launches = 0;                // kernel launches of one replay
    bool indexed = false;                  // the fields below describe `exec`
    std::vector<hipGraphNode_t> knodes;    // graph's kernel nodes in launch order
    std::vector<cbx_glaunch> ls;           // the plan it holds
    std::vector<int32_t> k0, kn;           // per launch: first kernel node, kernel count
    std::vector<uint64_t> sig;             // the launches' signatures, back to back
    std::vector<size_t> sig_at;            // launch i's signature: [sig_at[i], sig_at[i + 1])
};

struct cbx_graph_exec {
    int device;
    hipStream_t cs;                       // the stream its captures are recorded on
    GraphInst inst[2];
    int cur;                              // the instantiation launches replay
    std::vector<hipStream_t> launched;    // streams launched on since the last update
    std::vector<hipEvent_t> marks;        // recorded at the last update: inst[1 - cur]'s replays
    std::vector<hipEvent_t> spare;        // events free for reuse
};

// Waits for the events of the last update (the replays of inst[1 - cur]).
static int wait_marks(cbx_graph_exec* x, const char* f) {
    bool ok = true;
    for (hipEvent_t e : x->marks) {
        ok = hipEventSynchronize(e) == hipSuccess && ok;
        x->spare.push_back(e);
    }
    x->marks.clear();
    return ok ? CBX_OK : set_error(CBX_ERR_HIP, std::string(f) + ": waiting for earlier replays failed");
}

// Records an event on every stream launched on since the last update (they
// follow every replay of inst[cur] issued so far) into x->marks.
static int mark_launches(cbx_graph_exec* x, const char* f) {
    for (hipStream_t st : x->launched) {
        hipEvent_t e = nullptr;
        if (!x->spare.empty()) {
            e = x->spare.back();
            x->spare.pop_back();
        } else if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            return set_error(CBX_ERR_HIP, std::string(f) + ": event creation failed");
        }
        if (hipEventRecord(e, st) != hipSuccess) {
            x->spare.push_back(e);
            return set_error(CBX_ERR_HIP, std::string(f) + ": recording an event behind the replays failed");
        }
        x->marks.push_back(e);
    }
    x->launched.clear();
    return CBX_OK;
}

// Every value a launch's kernels are built from: its place and kind, every
// field of its nodes, every field of the tensors they name, and the serial
// numbers of the RoPE cache and conv weights they use (a new handle at a
// freed one's address differs).  Equal signatures issue equal kernels with
// equal arguments.
static void launch_signature(const cbx_tensor* t, const cbx_gnode* nd, const cbx_glaunch& l,
                             std::vector<uint64_t>* sig) {
    auto u = [](auto v) { return static_cast<uint64_t>(v); };
    sig->insert(sig->end(), {u(l.kind), u(l.first_node), u(l.n_nodes), u(l.flags)});
    for (int32_t i = l.first_node; i < l.first_node + l.n_nodes; i++) {
        const cbx_gnode& n = nd[i];
        uint32_t fb;
        std::memcpy(&fb, &n.fparam, 4);
        sig->insert(sig->end(), {u(n.op), u(n.dst), u(n.src[0]), u(n.src[1]), u(n.iparam), u(fb),
                                 u(reinterpret_cast<uintptr_t>(n.rope)), rope_cache_serial(n.rope), u(n.conv[0]),
                                 u(n.conv[1]), u(n.conv[2]), u(reinterpret_cast<uintptr_t>(n.conv_w)),
                                 conv1d_weights_serial(n.conv_w)});
        for (int32_t k : {n.dst, n.src[0], n.src[1]}) {
            if (k < 0) {
                sig->push_back(~uint64_t{0});
                continue;
            }
            const cbx_tensor& x = t[k];
            sig->insert(sig->end(), {u(reinterpret_cast<uintptr_t>(x.data)), u(x.type), u(x.reserved), u(x.ne[0]),
                                     u(x.ne[1]), u(x.ne[2]), u(x.ne[3]), u(x.nb[0]), u(x.nb[1]), u(x.nb[2]),
                                     u(x.nb[3])});
        }
    }
}

static void signatures(const cbx_tensor* t, const cbx_gnode* nd, const std::vector<cbx_glaunch>& ls,
                       std::vector<uint64_t>* sig, std::vector<size_t>* at) {
    sig->clear();
    at->assign(1, 0);
    for (const cbx_glaunch& l : ls) {
        launch_signature(t, nd, l, sig);
        at->push_back(sig->size());
    }
}

// The kernel nodes of a graph recorded from one stream, in order: a chain
// from its one root.  False when the graph is not such a chain of kernel
// nodes.
static bool kernel_chain(hipGraph_t g, std::vector<hipGraphNode_t>* out) {
    out->clear();
    size_t n = 0;
    if (hipGraphGetNodes(g, nullptr, &n) != hipSuccess) return false;
    if (n == 0) return true;
    size_t nr = 1;
    hipGraphNode_t node = nullptr;
    if (hipGraphGetRootNodes(g, &node, &nr) != hipSuccess || nr != 1) return false;
    out->reserve(n);
    while (node) {
        hipGraphNodeType ty;
        if (hipGraphNodeGetType(node, &ty) != hipSuccess || ty != hipGraphNodeTypeKernel) return false;
        out->push_back(node);
        size_t nd = 0;
        if (hipGraphNodeGetDependentNodes(node, nullptr, &nd) != hipSuccess || nd > 1) return false;
        hipGraphNode_t next = nullptr;
        if (nd == 1 && hipGraphNodeGetDependentNodes(node, &next, &nd) != hipSuccess) return false;
        node = nd == 1 ? next : nullptr;
    }
    return out->size() == n;
}

// The unsupported-node check every recording makes first.
static int refuse_unsupported(const cbx_gnode* nodes, const std::vector<cbx_glaunch>& ls, const char* f) {
    for (const cbx_glaunch& l : ls) {
        if (l.kind == CBX_GL_UNSUPPORTED) {
            return set_error(CBX_ERR_UNSUPPORTED, std::string(f) + ": node " + std::to_string(l.first_node) + " (" +
                                                      op_name(nodes[l.first_node].op) +
                                                      ") starts no chain the library runs");
        }
    }
    return CBX_OK;
}

// Records launches ls[which[0]], ls[which[1]], .. (every launch when which
// is NULL) on cs (a stream of the exec's own, so nothing else the caller has
// queued ends up in the graph) into a new HIP graph (*out); kcount[j] gets
// the kernel nodes launch j of the recording added (-1 when that could not
// be read) and *issued the kernel launch count.  f names the caller in
// errors.
static int record(const cbx_tensor* tensors, const cbx_gnode* nodes, int32_t n_nodes,
                  const std::vector<cbx_glaunch>& ls, const std::vector<int32_t>* which, hipStream_t cs,
                  hipGraph_t* out, std::vector<int32_t>* kcount, int32_t* issued, const char* f) {
    *out = nullptr;
    *issued = 0;
    kcount->clear();
    if (hipStreamBeginCapture(cs, hipStreamCaptureModeRelaxed) != hipSuccess) {
        return set_error(CBX_ERR_HIP, std::string(f) + ": stream capture failed to start");
    }
    int rc = CBX_OK;
    int32_t n = 0;
    size_t before = 0;
    std::string inner;
    const size_t count = which ? which->size() : ls.size();
    for (size_t j = 0; j < count; j++) {
        const cbx_glaunch& l = ls[which ? static_cast<size_t>((*which)[j]) : j];
        rc = run(tensors, nodes, n_nodes, l, cs);
        if (rc) {
            inner = "nodes " + std::to_string(l.first_node) + ".." + std::to_string(l.first_node + l.n_nodes - 1) +
                    ": " + cbx_last_error();
            break;
        }
        if (l.kind != CBX_GL_VIEW) n++;
        // the nodes the capture holds now, less those before this launch
        hipStreamCaptureStatus cst;
        hipGraph_t cg = nullptr;
        size_t now = 0;
        if (hipStreamGetCaptureInfo_v2(cs, &cst, nullptr, &cg, nullptr, nullptr) == hipSuccess && cg &&
            hipGraphGetNodes(cg, nullptr, &now) == hipSuccess && now >= before) {
            kcount->push_back(static_cast<int32_t>(now - before));
            before = now;
        } else {
            kcount->push_back(-1);
        }
    }
    hipGraph_t g = nullptr;
    const hipError_t ec = hipStreamEndCapture(cs, &g);
    if (rc || ec != hipSuccess || !g) {
        if (g) (void)hipGraphDestroy(g);
        if (rc) return set_error(rc, std::string(f) + ": " + inner);
        return set_error(CBX_ERR_HIP, std::string(f) + ": stream capture failed: " + hipGetErrorString(ec));
    }
    *out = g;
    *issued = n;
    return CBX_OK;
}

// Fills an instantiation's bookkeeping for the plan it now holds, recorded
// with per-launch kernel counts kcount; indexed stays false when the
// graph's kernel nodes cannot be matched to the launches.
static void index_inst(GraphInst* t, const cbx_tensor* tensors, const cbx_gnode* nodes,
                       const std::vector<cbx_glaunch>& ls, const std::vector<int32_t>& kcount, bool keep_nodes) {
    t->indexed = false;
    t->ls = ls;
    signatures(tensors, nodes, ls, &t->sig, &t->sig_at);
    t->k0.assign(ls.size(), 0);
    t->kn.assign(ls.size(), 0);
    int32_t at = 0;
    for (size_t i = 0; i < ls.size(); i++) {
        if (i >= kcount.size() || kcount[i] < 0) return;
        t->k0[i] = at;
        t->kn[i] = kcount[i];
        at += kcount[i];
    }
    if (!keep_nodes && !kernel_chain(t->graph, &t->knodes)) return;
    t->indexed = static_cast<int32_t>(t->knodes.size()) == at;
}

int cbx_graph_exec_create(const cbx_tensor* tensors, int32_t n_tensors, const cbx_gnode* nodes, int32_t n_nodes,
                          const int32_t* keep, int32_t n_keep, cbx_graph_exec** out, int32_t* n_launches) {
    clear_error();
    static const char* f = "cbx_graph_exec_create";
    if (n_launches) *n_launches = 0;
    if (!out) return set_error(CBX_ERR_INVALID_ARG, std::string(f) + ": out is NULL");
    *out = nullptr;
    int rc = CBX_OK;
    if (!current_state(&rc)) return rc;
    std::vector<cbx_glaunch> ls;
    if ((rc = plan(tensors, n_tensors, nodes, n_nodes, keep, n_keep, &ls, f)) ||
        (rc = refuse_unsupported(nodes, ls, f))) {
        return rc;
    }
    hipStream_t cs = nullptr;
    if (hipStreamCreateWithFlags(&cs, hipStreamNonBlocking) != hipSuccess) {
        return set_error(CBX_ERR_HIP, std::string(f) + ": stream creation failed");
    }
    hipGraph_t g[2] = {nullptr, nullptr};
    int32_t issued = 0;
    std::vector<int32_t> kcount;
    rc = record(tensors, nodes, n_nodes, ls, nullptr, cs, &g[0], &kcount, &issued, f);
    if (rc == CBX_OK && hipGraphClone(&g[1], g[0]) != hipSuccess) {
        rc = set_error(CBX_ERR_HIP, std::string(f) + ": graph clone failed");
    }
    hipGraphExec_t ge[2] = {nullptr, nullptr};
    for (int k = 0; k < 2 && rc == CBX_OK; k++) {
        if (hipGraphInstantiate(&ge[k], g[k], nullptr, nullptr, 0) != hipSuccess || !ge[k]) {
            rc = set_error(CBX_ERR_HIP, std::string(f) + ": graph instantiation failed");
        }
    }
    auto* x = rc == CBX_OK ? new (std::nothrow) cbx_graph_exec() : nullptr;
    if (rc == CBX_OK && !x) rc = set_error(CBX_ERR_HIP, std::string(f) + ": out of host memory");
    if (rc != CBX_OK) {
        for (int k = 0; k < 2; k++) {
            if (ge[k]) (void)hipGraphExecDestroy(ge[k]);
            if (g[k]) (void)hipGraphDestroy(g[k]);
        }
        (void)hipStreamDestroy(cs);
        return rc;
    }
    (void)hipGetDevice(&x->device);
    x->cs = cs;
    for (int k = 0; k < 2; k++) {
        GraphInst& t = x->inst[k];
        t.graph = g[k];
        t.exec = ge[k];
        t.n_launches = issued;
        index_inst(&t, tensors, nodes, ls, kcount, false);
    }
    x->cur = 0;
    *out = x;
    if (n_launches) *n_launches = issued;
    return CBX_OK;
}

// The targeted update: the launches whose signature changed, recorded
// alone, their kernels' arguments set on t's kernel nodes.  *done = false
// (and nothing fatal) when the update has to take the whole-list path.
static int update_changed(cbx_graph_exec* x, GraphInst& t, const cbx_tensor* tensors, const cbx_gnode* nodes,
                          int32_t n_nodes, const std::vector<cbx_glaunch>& ls, const std::vector<uint64_t>& sig,
                          const std::vector<size_t>& sig_at, bool* done, const char* f) {
    *done = false;
    std::vector<int32_t> changed;
    for (size_t i = 0; i < ls.size(); i++) {
        const size_t a = sig_at[i], b = sig_at[i + 1];
        if (b - a != t.sig_at[i + 1] - t.sig_at[i] ||
            !std::equal(sig.begin() + static_cast<std::ptrdiff_t>(a), sig.begin() + static_cast<std::ptrdiff_t>(b),
                        t.sig.begin() + static_cast<std::ptrdiff_t>(t.sig_at[i]))) {
            changed.push_back(static_cast<int32_t>(i));
        }
    }
    if (!changed.empty()) {
        hipGraph_t g = nullptr;
        std::vector<int32_t> kcount;
        int32_t issued = 0;
        int rc = record(tensors, nodes, n_nodes, ls, &changed, x->cs, &g, &kcount, &issued, f);
        if (rc) return rc;   // t untouched
        std::vector<hipGraphNode_t> gn;
        bool ok = kernel_chain(g, &gn);
        size_t want = 0;
        for (size_t j = 0; ok && j < changed.size(); j++) {
            ok = kcount[j] == t.kn[static_cast<size_t>(changed[j])];
            want += static_cast<size_t>(kcount[j] > 0 ? kcount[j] : 0);
        }
        ok = ok && gn.size() == want;
        // each changed launch's kernels, in order, onto the nodes it issued
        size_t p = 0;
        for (size_t j = 0; ok && j < changed.size(); j++) {
            const size_t i = static_cast<size_t>(changed[j]);
            for (int32_t q = 0; ok && q < t.kn[i]; q++, p++) {
                hipKernelNodeParams kp;
                ok = hipGraphKernelNodeGetParams(gn[p], &kp) == hipSuccess &&
                     hipGraphExecKernelNodeSetParams(t.exec, t.knodes[static_cast<size_t>(t.k0[i] + q)], &kp) ==
                         hipSuccess;
            }
        }
        (void)hipGraphDestroy(g);
        if (!ok) {
            (void)hipGetLastError();
            t.indexed = false;   // possibly half set: the whole-list path rewrites every node
            return CBX_OK;
        }
    }
    t.ls = ls;
    t.sig = sig;
    t.sig_at = sig_at;
    *done = true;
    return CBX_OK;
}

int cbx_graph_exec_update(cbx_graph_exec* exec, const cbx_tensor* tensors, int32_t n_tensors,
                          const cbx_gnode* nodes, int32_t n_nodes, const int32_t* keep, int32_t n_keep,
                          int32_t* n_launches, int32_t* in_place) {
    clear_error();
    static const char* f = "cbx_graph_exec_update";
    if (n_launches) *n_launches = 0;
    if (in_place) *in_place = 0;
    if (!exec) return set_error(CBX_ERR_INVALID_ARG, std::string(f) + ": exec is NULL");
    int dev = -1;
    (void)hipGetDevice(&dev);
    if (dev != exec->device) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(f) + ": the graph was captured on device " +
                                                  std::to_string(exec->device) + ", the current device is " +
                                                  std::to_string(dev));
    }
    int rc = CBX_OK;
    if (!current_state(&rc)) return rc;
    std::vector<cbx_glaunch> ls;
    if ((rc = plan(tensors, n_tensors, nodes, n_nodes, keep, n_keep, &ls, f)) ||
        (rc = refuse_unsupported(nodes, ls, f))) {
        return rc;   // exec is left as it was
    }
    GraphInst& t = exec->inst[1 - exec->cur];
    bool same_plan = t.indexed && ls.size() == t.ls.size();
    for (size_t i = 0; same_plan && i < ls.size(); i++) {
        same_plan = ls[i].kind == t.ls[i].kind && ls[i].first_node == t.ls[i].first_node &&
                    ls[i].n_nodes == t.ls[i].n_nodes && ls[i].flags == t.ls[i].flags;
    }
    if (same_plan) {
        std::vector<uint64_t> sig;
        std::vector<size_t> sig_at;
        signatures(tensors, nodes, ls, &sig, &sig_at);
        // the instantiation to re-point is the one not replayed since the
        // last update: wait for its replays (issued before that update),
        // then mark the current one's
        if ((rc = wait_marks(exec, f)) || (rc = mark_launches(exec, f))) return rc;
        bool done = false;
        if ((rc = update_changed(exec, t, tensors, nodes, n_nodes, ls, sig, sig_at, &done, f))) return rc;
        if (done) {
            exec->cur = 1 - exec->cur;
            if (n_launches) *n_launches = t.n_launches;
            if (in_place) *in_place = 1;
            return CBX_OK;
        }
    }
    hipGraph_t g = nullptr;
    int32_t issued = 0;
    std::vector<int32_t> kcount;
    rc = record(tensors, nodes, n_nodes, ls, nullptr, exec->cs, &g, &kcount, &issued, f);
    if (rc) return rc;   // exec is left as it was
    if (!same_plan && ((rc = wait_marks(exec, f)) || (rc = mark_launches(exec, f)))) {
        (void)hipGraphDestroy(g);
        return rc;
    }
    // the same launches with other arguments: the instantiated graph takes
    // the new arguments in place (its kernel nodes stay those of t.graph)
    hipGraphNode_t bad_node = nullptr;
    hipGraphExecUpdateResult res = hipGraphExecUpdateError;
    if (issued == t.n_launches && hipGraphExecUpdate(t.exec, g, &bad_node, &res) == hipSuccess &&
        res == hipGraphExecUpdateSuccess) {
        (void)hipGraphDestroy(g);
        index_inst(&t, tensors, nodes, ls, kcount, true);
        exec->cur = 1 - exec->cur;
        if (n_launches) *n_launches = issued;
        if (in_place) *in_place = 1;
        return CBX_OK;
    }
    (void)hipGetLastError();   // a refused update leaves nothing to report
    // another set of launches: a new instantiation replaces the old one
    hipGraphExec_t ge = nullptr;
    if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess || !ge) {
        (void)hipGraphDestroy(g);
        return set_error(CBX_ERR_HIP, std::string(f) + ": graph instantiation failed");
    }
    (void)hipGraphExecDestroy(t.exec);
    (void)hipGraphDestroy(t.graph);
    t.graph = g;
    t.exec = ge;
    t.n_launches = issued;
    index_inst(&t, tensors, nodes, ls, kcount, false);
    exec->cur = 1 - exec->cur;
    if (n_launches) *n_launches = issued;
    return CBX_OK;
}

int cbx_graph_exec_launch(cbx_graph_exec* exec, cbx_stream stream) {
    clear_error();
    if (!exec) return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_exec_launch: exec is NULL");
    int dev = -1;
    (void)hipGetDevice(&dev);
    if (dev != exec->device) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_graph_exec_launch: the graph was captured on device " +
                                                  std::to_string(exec->device) + ", the current device is " +
                                                  std::to_string(dev));
    }
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const hipError_t e = hipGraphLaunch(exec->inst[exec->cur].exec, s);
    if (e != hipSuccess) {
        return set_error(CBX_ERR_HIP, std::string("cbx_graph_exec_launch: ") + hipGetErrorString(e));
    }
    bool seen = false;
    for (hipStream_t t : exec->launched) seen = seen || t == s;
    if (!seen) exec->launched.push_back(s);
    return CBX_OK;
}

void cbx_graph_exec_destroy(cbx_graph_exec* exec) {
    if (!exec) return;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(exec->device);
    // no replay of either instantiation still in flight
    static const char* f = "cbx_graph_exec_destroy";
    if (wait_marks(exec, f) != CBX_OK || mark_launches(exec, f) != CBX_OK || wait_marks(exec, f) != CBX_OK) {
        (void)hipDeviceSynchronize();
    }
    for (hipEvent_t e : exec->spare) (void)hipEventDestroy(e);
    for (GraphInst& t : exec->inst) {
        (void)hipGraphExecDestroy(t.exec);
        (void)hipGraphDestroy(t.graph);
    }
    (void)hipStreamDestroy(exec->cs);
    (void)hipSetDevice(prev);
    delete exec;
}

int cbx_graph_compute(const cbx_tensor* tensors, int32_t n_tensors, const cbx_gnode* nodes, int32_t n_nodes,
                      const int32_t* keep, int32_t n_keep, cbx_stream stream, int32_t* n_launches) {
    clear_error();
    if (n_launches) *n_launches = 0;
    std::vector<cbx_glaunch> ls;
    int rc = plan(tensors, n_tensors, nodes, n_nodes, keep, n_keep, &ls, "cbx_graph_compute");
    if (rc) return rc;
    for (const cbx_glaunch& l : ls) {
        if (l.kind == CBX_GL_UNSUPPORTED) {
            return set_error(CBX_ERR_UNSUPPORTED, "cbx_graph_compute: node " + std::to_string(l.first_node) + " (" +
                                                      op_name(nodes[l.first_node].op) +
                                                      ") starts no chain the library runs");
        }
    }
    int32_t issued = 0;
    for (const cbx_glaunch& l : ls) {
        rc = run(tensors, nodes, n_nodes, l, stream);
        if (rc) {
            const std::string inner = cbx_last_error();
            return set_error(rc, "cbx_graph_compute: nodes " + std::to_string(l.first_node) + ".." +
                                     std::to_string(l.first_node + l.n_nodes - 1) + ": " + inner);
        }
        if (l.kind != CBX_GL_VIEW) issued++;
        if (n_launches) *n_launches = issued;
    }
    return CBX_OK;
}

}  // extern "C"
