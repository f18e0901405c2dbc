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

template <typename T, int MODE>
__global__ __launch_bounds__(256) void k_rope(View x, View y, const char* __restrict__ pos, int64_t pos_nb0,
                                              RopeParams rp, const float2* __restrict__ table, int32_t n_pos,
                                              const float* __restrict__ ff) {
    extern __shared__ float2 cs[];
    const int64_t ne0 = x.ne[0], ne1 = x.ne[1], ne2 = x.ne[2], ne3 = x.ne[3];
    const int half = rp.n_dims / 2;
    const int64_t n_tail = ne0 - rp.n_dims;
    for (int64_t t = blockIdx.x; t < ne2 * ne3; t += gridDim.x) {
        const int64_t i2 = t % ne2, i3 = t / ne2;
        const int32_t p = *reinterpret_cast<const int32_t*>(pos + i2 * pos_nb0);
        for (int k = threadIdx.x; k < half; k += blockDim.x) {
            if (p >= 0 && p < n_pos) {
                cs[k] = table[static_cast<int64_t>(p) * half + k];
            } else {
                float c, s;
                rope_cos_sin_dev(p, k, rp, ff, &c, &s);
                cs[k] = make_float2(c, s);
            }
        }
        __syncthreads();
        for (int64_t q = threadIdx.x; q < ne1 * half; q += blockDim.x) {
            const int64_t h = q / half;
            const int k = static_cast<int>(q - h * half);
            const char* xr = x.data + h * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
            char* yr = y.data + h * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
            const int64_t ia = MODE == 2 ? k : 2 * k;
            const int64_t ib = MODE == 2 ? k + half : 2 * k + 1;
            const float x0 = Elt<T>::load1(xr + ia * Elt<T>::size);
            const float x1 = Elt<T>::load1(xr + ib * Elt<T>::size);
            const float2 c = cs[k];
            Elt<T>::store1(yr + ia * Elt<T>::size, x0 * c.x - x1 * c.y);
            Elt<T>::store1(yr + ib * Elt<T>::size, x0 * c.y + x1 * c.x);
        }
        if (n_tail > 0) {
            for (int64_t q = threadIdx.x; q < ne1 * n_tail; q += blockDim.x) {
                const int64_t h = q / n_tail;
                const int64_t j = rp.n_dims + (q - h * n_tail);
                const char* xr = x.data + h * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
                char* yr = y.data + h * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
                *reinterpret_cast<T*>(yr + j * Elt<T>::size) = *reinterpret_cast<const T*>(xr + j * Elt<T>::size);
            }
        }
        __syncthreads();
    }
}

}  // namespace

int launch_rope(const cbx_tensor* x, const cbx_tensor* pos, const RopeParams& p, const float2* table, int32_t n_pos,
                const float* ff, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    (void)st;
    const int64_t ntok = x->ne[2] * x->ne[3];
    const int64_t pairs = x->ne[1] * (p.n_dims / 2);
    const int threads = static_cast<int>(std::min<int64_t>(256, std::max<int64_t>(64, cdiv(pairs, 64) * 64)));
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ntok, int64_t{1} << 20)));
    const size_t lds = static_cast<size_t>(p.n_dims / 2) * sizeof(float2);
    const char* pp = static_cast<const char*>(pos->data);
    const int64_t pnb = static_cast<int64_t>(pos->nb[0]);
    if (x->type == CBX_TYPE_F32) {
        if (p.mode == 2) hipLaunchKernelGGL((k_rope<float, 2>), grid, dim3(threads), lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
        else hipLaunchKernelGGL((k_rope<float, 0>), grid, dim3(threads), lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
    } else {
        if (p.mode == 2) hipLaunchKernelGGL((k_rope<uint16_t, 2>), grid, dim3(threads), lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
        else hipLaunchKernelGGL((k_rope<uint16_t, 0>), grid, dim3(threads), lds, s, view_of(x), view_of(y), pp, pnb, p, table, n_pos, ff);
    }
    return check_launch("rope_ext");
}

}  // namespace cbx
