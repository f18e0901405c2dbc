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
struct RopeArgs {
    const char* x;
    char* y;
    const char* pos;
    const float2* table;
    const float* ff;
    int64_t xnb1, xnb2, xnb3, ynb1, ynb2, ynb3, pos_nb0;
    uint32_t ne1, ne2, n_tail;
    int32_t n_pos;
    RopeParams rp;
};

// IT > 0: every pair of the token is one of the lane's first IT (ne1 *
// n_dims/2 <= IT * 256), and the lane's x values are loaded before the
// position and table reads, so the row's HBM latency overlaps theirs.
// IT == 0: any head count, pairs loaded after the table is staged.
template <typename T, int MODE, int IT>
__global__ __launch_bounds__(kRopeThreads) void k_rope(RopeArgs a) {
    extern __shared__ float2 cs[];
    const RopeParams& rp = a.rp;
    const float2* __restrict__ table = a.table;
    const uint32_t ne1 = a.ne1, ne2 = a.ne2;
    const uint32_t half = static_cast<uint32_t>(rp.n_dims / 2);
    const uint32_t n_tail = a.n_tail;
    const int32_t n_pos = a.n_pos;
    const uint32_t t = blockIdx.x;
    const uint32_t i2 = t % ne2, i3 = t / ne2;
    const int32_t p = *reinterpret_cast<const int32_t*>(a.pos + i2 * a.pos_nb0);
    const char* xt = a.x + i2 * a.xnb2 + i3 * a.xnb3;
    char* yt = a.y + i2 * a.ynb2 + i3 * a.ynb3;
    const uint32_t n_pairs = ne1 * half;
    constexpr int NI = IT > 0 ? IT : 1;
    float x0[NI], x1[NI];
    uint32_t qh[NI], qk[NI];
    if constexpr (IT > 0) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const uint32_t q = threadIdx.x + it * kRopeThreads;
            const uint32_t qc = q < n_pairs ? q : 0;
            qh[it] = qc / half;
            qk[it] = qc - qh[it] * half;
            const char* xr = xt + qh[it] * a.xnb1;
            const uint32_t ia = MODE == 2 ? qk[it] : 2 * qk[it];
            const uint32_t ib = MODE == 2 ? qk[it] + half : 2 * qk[it] + 1;
            x0[it] = Elt<T>::load1(xr + ia * Elt<T>::size);
            x1[it] = Elt<T>::load1(xr + ib * Elt<T>::size);
        }
    }
    for (uint32_t k = threadIdx.x; k < half; k += kRopeThreads) {
        if (p >= 0 && p < n_pos) {
            cs[k] = table[static_cast<int64_t>(p) * half + k];
        } else {
            float c, s;
            rope_cos_sin_dev(p, static_cast<int>(k), rp, a.ff, &c, &s);
            cs[k] = make_float2(c, s);
        }
    }
    __syncthreads();
    if constexpr (IT > 0) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const uint32_t q = threadIdx.x + it * kRopeThreads;
            if (q >= n_pairs) continue;
            char* yr = yt + qh[it] * a.ynb1;
            const uint32_t k = qk[it];
            const uint32_t ia = MODE == 2 ? k : 2 * k;
            const uint32_t ib = MODE == 2 ? k + half : 2 * k + 1;
            const float2 c = cs[k];
            Elt<T>::store1(yr + ia * Elt<T>::size, x0[it] * c.x - x1[it] * c.y);
            Elt<T>::store1(yr + ib * Elt<T>::size, x0[it] * c.y + x1[it] * c.x);
        }
    } else {
        for (uint32_t q = threadIdx.x; q < n_pairs; q += kRopeThreads) {
            const uint32_t h = q / half;
            const uint32_t k = q - h * half;
            const char* xr = xt + h * a.xnb1;
            char* yr = yt + h * a.ynb1;
            const uint32_t ia = MODE == 2 ? k : 2 * k;
            const uint32_t ib = MODE == 2 ? k + half : 2 * k + 1;
            const float v0 = Elt<T>::load1(xr + ia * Elt<T>::size);
            const float v1 = Elt<T>::load1(xr + ib * Elt<T>::size);
            const float2 c = cs[k];
            Elt<T>::store1(yr + ia * Elt<T>::size, v0 * c.x - v1 * c.y);
            Elt<T>::store1(yr + ib * Elt<T>::size, v0 * c.y + v1 * c.x);
        }
    }
    for (uint32_t q = threadIdx.x; q < ne1 * n_tail; q += kRopeThreads) {
        const uint32_t h = q / n_tail;
        const uint32_t j = static_cast<uint32_t>(rp.n_dims) + (q - h * n_tail);
        *reinterpret_cast<T*>(yt + h * a.ynb1 + j * Elt<T>::size) =
            *reinterpret_cast<const T*>(xt + h * a.xnb1 + j * Elt<T>::size);
    }
}

template <typename T, int MODE>
void rope_it(int it, dim3 grid, dim3 block, size_t lds, hipStream_t s, const RopeArgs& a) {
    switch (it) {
        case 1: hipLaunchKernelGGL((k_rope<T, MODE, 1>), grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL((k_rope<T, MODE, 2>), grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL((k_rope<T, MODE, 4>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((k_rope<T, MODE, 0>), grid, block, lds, s, a); break;
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
    RopeArgs a;
    a.x = static_cast<const char*>(x->data);
    a.y = static_cast<char*>(y->data);
    a.pos = static_cast<const char*>(pos->data);
    a.table = table;
    a.ff = ff;
    a.xnb1 = static_cast<int64_t>(x->nb[1]);
    a.xnb2 = static_cast<int64_t>(x->nb[2]);
    a.xnb3 = static_cast<int64_t>(x->nb[3]);
    a.ynb1 = static_cast<int64_t>(y->nb[1]);
    a.ynb2 = static_cast<int64_t>(y->nb[2]);
    a.ynb3 = static_cast<int64_t>(y->nb[3]);
    a.pos_nb0 = static_cast<int64_t>(pos->nb[0]);
    a.ne1 = static_cast<uint32_t>(x->ne[1]);
    a.ne2 = static_cast<uint32_t>(x->ne[2]);
    a.n_tail = static_cast<uint32_t>(x->ne[0] - p.n_dims);
    a.n_pos = n_pos;
    a.rp = p;
    // pairs per token over the workgroup: 1, 2 or 4 per lane preload their x
    const int64_t per_lane = cdiv(x->ne[1] * (p.n_dims / 2), kRopeThreads);
    const int it = per_lane <= 1 ? 1 : per_lane <= 2 ? 2 : per_lane <= 4 ? 4 : 0;
    if (x->type == CBX_TYPE_F32) {
        if (p.mode == 2) rope_it<float, 2>(it, grid, block, lds, s, a);
        else rope_it<float, 0>(it, grid, block, lds, s, a);
    } else {
        if (p.mode == 2) rope_it<uint16_t, 2>(it, grid, block, lds, s, a);
        else rope_it<uint16_t, 0>(it, grid, block, lds, s, a);
    }
    return check_launch("rope_ext");
}

}  // namespace cbx
