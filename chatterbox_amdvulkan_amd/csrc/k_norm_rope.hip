// k_norm_rope.hip -- LayerNorm (+ affine) of each token row followed by
// RoPE of the row viewed as heads, in one read and one write:
//
//   t = ggml_add(ggml_mul(ggml_norm(x, eps), w), b)          x ne = (C, T, B)
//   y = ggml_rope_ext(ggml_reshape_4d(t, hd, C/hd, T, B), pos, ...)
//
// the norm -> attention-input chain of a CFM/S3 transformer block when the
// rotary embedding is applied to the normalised stream (ggml composition of
// cfm_decoder.cpp:29-33 and s3enc.cpp:215-229).
//
// One wave per token row (C <= 1024): the row is normalised in registers
// exactly as the standalone LayerNorm does (same lanes, same f64 wave
// reductions, same rounding order), the normalised row goes to LDS, and
// each lane then rotates its own 4-element vectors, reading the partner
// elements from there and the cos/sin of its elements from the table row of
// the token's position.  Rotation arithmetic is the standalone RoPE's.
#include "cbx_normrope.h"

namespace cbx {
namespace {

template <int NV, int MODE, bool FLAT, int W = 1, bool XS = false>
__global__ __launch_bounds__(64 * W) void k_layer_norm_rope(NormRopeArgs a) {
    __shared__ float row[kRowMax];
    __shared__ double lds[2 * W];
    ln_rope_row<NV, MODE, FLAT, W, XS>(a, blockIdx.x, (threadIdx.x >> 6) * 64 * NV + (threadIdx.x & 63), row, lds);
}

template <int MODE, bool FLAT, bool XS>
void go(const NormRopeArgs& a, int nv, int w, dim3 grid, hipStream_t s) {
    if (FLAT && w > 1) {
        const dim3 block(64 * w);
        switch (nv * 8 + w) {
            case 2 * 8 + 2: hipLaunchKernelGGL((k_layer_norm_rope<1, MODE, FLAT, 2, XS>), grid, block, 0, s, a); break;
            case 4 * 8 + 2: hipLaunchKernelGGL((k_layer_norm_rope<2, MODE, FLAT, 2, XS>), grid, block, 0, s, a); break;
            default: hipLaunchKernelGGL((k_layer_norm_rope<1, MODE, FLAT, 4, XS>), grid, block, 0, s, a); break;   // 4, 4
        }
        return;
    }
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_layer_norm_rope<1, MODE, FLAT, 1, XS>), grid, dim3(64), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_layer_norm_rope<2, MODE, FLAT, 1, XS>), grid, dim3(64), 0, s, a); break;
        default: hipLaunchKernelGGL((k_layer_norm_rope<4, MODE, FLAT, 1, XS>), grid, dim3(64), 0, s, a); break;
    }
}

}  // namespace

int launch_layer_norm_rope(const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int64_t head_dim,
                           const cbx_tensor* pos, const RopeParams& p, const float2* table, int32_t n_pos,
                           const float* ff, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    NormRopeArgs a;
    a.x = static_cast<const char*>(x->data);
    a.y = static_cast<char*>(y->data);
    a.w = w ? static_cast<const float*>(w->data) : nullptr;
    a.b = b ? static_cast<const float*>(b->data) : nullptr;
    a.pos = static_cast<const char*>(pos->data);
    a.table = table;
    a.ff = ff;
    a.mx = row_map(x);
    a.my = row_map(y);
    a.pos_nb0 = static_cast<int64_t>(pos->nb[0]);
    a.ne0 = static_cast<int32_t>(x->ne[0]);
    a.hd = static_cast<int32_t>(head_dim);
    a.n_tok = static_cast<uint32_t>(x->ne[1]);
    a.n_pos = n_pos;
    a.eps = eps;
    a.rp = p;
    const int64_t rows = x->ne[1] * x->ne[2] * x->ne[3];
    if (rows >= (int64_t{1} << 31)) return set_error(CBX_ERR_UNSUPPORTED, "layer_norm_rope: too many rows");
    // 16-byte cos/sin loads: NORMAL needs n_dims % 4 == 0 (a vector's two
    // pairs are one float4 of the row); NEOX needs n_dims % 8 == 0, so that
    // half % 4 == 0 and no vector straddles the half boundary (with
    // n_dims % 8 == 4 a vector at i0 < half < i0 + 4 would take pairs
    // half, half + 1 of the next table row for its upper elements)
    const int vec_mod = p.mode == 2 ? 8 : 4;
    a.vec_cs = (reinterpret_cast<uintptr_t>(table) % 16 == 0 && p.n_dims % vec_mod == 0) ? 1 : 0;
    const int nv = x->ne[0] <= 256 ? 1 : x->ne[0] <= 512 ? 2 : 4;
    // waves a row: one, unless the launch would have fewer than about two
    // waves a CU; then up to 4, at most one per vector a lane (the rotation
    // reads partners from the LDS row after a workgroup barrier, so a wave's
    // share need not be whole heads).  [2,500,512]: one wave a row, 3.30
    // against 3.41 us with two (the second reduction's barrier)
    int wr = 1;
    while (wr < 4 && wr < nv && rows * wr < int64_t{2} * st->n_cu) wr *= 2;
    const dim3 grid(static_cast<unsigned>(rows));
    const bool flat = a.mx.flat && a.my.flat;
    // partners in registers: the head's vectors on consecutive lanes of one
    // wave (hd/4 divides 64), whole 4-vectors rotated or copied (n_dims % 4
    // == 0; NEOX: half/4 a power of two, so the partner is lane ^ (half/4))
    const int64_t hq = head_dim / 4, dq = p.n_dims / 8;
    const bool xs = flat && a.vec_cs && 64 % hq == 0 && p.n_dims % 4 == 0 &&
                    (p.mode != 2 || (p.n_dims % 8 == 0 && dq > 0 && (dq & (dq - 1)) == 0));
    if (p.mode == 2) {
        if (xs) go<2, true, true>(a, nv, wr, grid, s);
        else if (flat) go<2, true, false>(a, nv, wr, grid, s);
        else go<2, false, false>(a, nv, 1, grid, s);
    } else {
        if (xs) go<0, true, true>(a, nv, wr, grid, s);
        else if (flat) go<0, true, false>(a, nv, wr, grid, s);
        else go<0, false, false>(a, nv, 1, grid, s);
    }
    return check_launch("layer_norm_rope");
}

}  // namespace cbx
