// k_rope.hip -- ggml_rope_ext (forward, NORMAL and NEOX modes) from a
// host-built cos/sin table.
//
// Layout as ggml: x ne = (head_dim, n_head, n_tok, batch); pos[i2] is the
// position of token i2.  One workgroup per token: the token's row of the
// cos/sin table (n_dims/2 float2) is staged in LDS once and shared by all
// heads.  Pairs: NEOX (i, i + n_dims/2), NORMAL (2i, 2i+1); dims past n_dims
// are copied.  y0 = x0*c - x1*s, y1 = x0*s + x1*c, each product and sum
// rounded to f32 (built with -ffp-contract=off), as ggml-cpu's rotate_pairs.
//
// A position outside the table's range is computed on the device with the
// same recurrence (theta <- theta * theta_scale, one f32 multiply per pair)
// and the device's cosf/sinf.
#include "cbx_rowops.h"

namespace cbx {
namespace {

constexpr int kRopeThreads = 256;

// One workgroup per token (exactly ne2*ne3 workgroups of a fixed size: no
// grid-stride loop bound or block-size read to wait for before the loads).
template <typename T, int MODE>
__global__ __launch_bounds__(kRopeThreads) void k_rope(View x, View y, const char* __restrict__ pos, int64_t pos_nb0,
                                                       RopeParams rp, const float2* __restrict__ table, int32_t n_pos,
                                                       const float* __restrict__ ff) {
    extern __shared__ float2 cs[];
    const uint32_t ne1 = static_cast<uint32_t>(x.ne[1]), ne2 = static_cast<uint32_t>(x.ne[2]);
    const uint32_t half = static_cast<uint32_t>(rp.n_dims / 2);
    const uint32_t n_tail = static_cast<uint32_t>(x.ne[0] - rp.n_dims);
    const uint32_t t = blockIdx.x;
    const uint32_t i2 = t % ne2, i3 = t / ne2;
    const int32_t p = *reinterpret_cast<const int32_t*>(pos + i2 * pos_nb0);
    for (uint32_t k = threadIdx.x; k < half; k += kRopeThreads) {
        if (p >= 0 && p < n_pos) {
            cs[k] = table[static_cast<int64_t>(p) * half + k];
        } else {
            float c, s;
            rope_cos_sin_dev(p, static_cast<int>(k), rp, ff, &c, &s);
            cs[k] = make_float2(c, s);
        }
    }
    __syncthreads();
    const char* xt = x.data + i2 * x.nb[2] + i3 * x.nb[3];
    char* yt = y.data + i2 * y.nb[2] + i3 * y.nb[3];
    for (uint32_t q = threadIdx.x; q < ne1 * half; q += kRopeThreads) {
        const uint32_t h = q / half;
        const uint32_t k = q - h * half;
        const char* xr = xt + h * x.nb[1];
        char* yr = yt + h * y.nb[1];
        const uint32_t ia = MODE == 2 ? k : 2 * k;
        const uint32_t ib = MODE == 2 ? k + half : 2 * k + 1;
        const float x0 = Elt<T>::load1(xr + ia * Elt<T>::size);
        const float x1 = Elt<T>::load1(xr + ib * Elt<T>::size);
        const float2 c = cs[k];
        Elt<T>::store1(yr + ia * Elt<T>::size, x0 * c.x - x1 * c.y);
        Elt<T>::store1(yr + ib * Elt<T>::size, x0 * c.y + x1 * c.x);
    }
    for (uint32_t q = threadIdx.x; q < ne1 * n_tail; q += kRopeThreads) {
        const uint32_t h = q / n_tail;
        const uint32_t j = static_cast<uint32_t>(rp.n_dims) + (q - h * n_tail);
        *reinterpret_cast<T*>(yt + h * y.nb[1] + j * Elt<T>::size) =
            *reinterpret_cast<const T*>(xt + h * x.nb[1] + j * Elt<T>::size);
    }
}

}  // namespace

int launch_rope(const cbx_tensor* x, const cbx_tensor* pos, const RopeParams& p, const float2* table, int32_t n_pos,
                const float* ff, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    (void)st;
    const int64_t ntok = x->ne[2] * x->ne[3];
    if (ntok >= (int64_t{1} << 31) || x->ne[1] * (x->ne[0] + p.n_dims) >= (int64_t{1} << 31)) {
        return set_error(CBX_ERR_UNSUPPORTED, "rope_ext: too many tokens or heads");
    }
    const dim3 grid(static_cast<unsigned>(ntok)), block(kRopeThreads);
    const size_t lds = static_cast<size_t>(p.n_dims / 2) * sizeof(float2);
    const char* pp = static_cast<const char*>(pos->data);
    const int64_t pnb = static_cast<int64_t>(pos->nb[0]);
    if (x->type == CBX_TYPE_F32) {
        if (p.mode == 2) hipLaunchKernelGGL((k_rope<float, 2>), grid, block, lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
        else hipLaunchKernelGGL((k_rope<float, 0>), grid, block, lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
    } else {
        if (p.mode == 2) hipLaunchKernelGGL((k_rope<uint16_t, 2>), grid, block, lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
        else hipLaunchKernelGGL((k_rope<uint16_t, 0>), grid, block, lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
    }
    return check_launch("rope_ext");
}

}  // namespace cbx
