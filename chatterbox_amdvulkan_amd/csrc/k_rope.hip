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

#include <algorithm>

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
    uint32_t nth;   // k_rope_vec: its block size (a multiple of 64 up to kRopeThreads)
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

// Four pairs a lane, no LDS: NEOX pairs m..m+3 of a head are two 4-element
// vectors (at m and m + n_dims/2), NORMAL pairs m..m+3 the 8 elements from
// 2m; their cos/sin are two 16-byte loads from the table row of the token's
// position.  One workgroup per token, the token's ne1 * n_dims/8 pair
// groups over its lanes (a loop past the block).  Needs n_dims % 8 == 0, a
// 16-byte aligned table, and x / y head rows aligned for 4-element loads.
// The products and roundings are those of k_rope.
template <typename T, int MODE>
__global__ __launch_bounds__(kRopeThreads) void k_rope_vec(RopeArgs a) {
    const RopeParams& rp = a.rp;
    const uint32_t half = static_cast<uint32_t>(rp.n_dims / 2);
    const uint32_t per_head = half / 4;
    const uint32_t t = blockIdx.x;
    const uint32_t i2 = t % a.ne2, i3 = t / a.ne2;
    const int32_t p = *reinterpret_cast<const int32_t*>(a.pos + i2 * a.pos_nb0);
    // the fields used once the position is known, in the argument loads that
    // go out with the position's (left alone, the compiler loads some of them
    // only after the position has arrived: one more scalar round trip before
    // the table and row loads); after the position load, which stays scalar
    arg_now(a.x); arg_now(a.y); arg_now(a.table);
    arg_now(reinterpret_cast<const void*>(a.xnb1)); arg_now(reinterpret_cast<const void*>(a.xnb2));
    arg_now(reinterpret_cast<const void*>(a.xnb3)); arg_now(reinterpret_cast<const void*>(a.ynb1));
    arg_now(reinterpret_cast<const void*>(a.ynb2)); arg_now(reinterpret_cast<const void*>(a.ynb3));
    arg_now(a.ne1); arg_now(static_cast<uint32_t>(a.n_pos)); arg_now(static_cast<uint32_t>(rp.n_dims));
    arg_now(a.nth);
    const uint32_t nth = a.nth;   // the block size (read with the other fields, not from the dispatch packet)
    const bool in_tab = p >= 0 && p < a.n_pos;
    const float2* tr = a.table + static_cast<int64_t>(in_tab ? p : 0) * half;
    constexpr int es = Elt<T>::size;
    const char* xt = a.x + i2 * a.xnb2 + i3 * a.xnb3;
    char* yt = a.y + i2 * a.ynb2 + i3 * a.ynb3;
    for (uint32_t q = threadIdx.x; q < a.ne1 * per_head; q += nth) {
        const uint32_t h = q / per_head;
        const uint32_t m = (q - h * per_head) * 4;
        const char* xr = xt + h * a.xnb1;
        char* yr = yt + h * a.ynb1;
        const uint32_t ia = MODE == 2 ? m : 2 * m, ib = MODE == 2 ? m + half : 2 * m + 4;
        const float4 xa = Elt<T>::load4(xr + ia * es);
        const float4 xb = Elt<T>::load4(xr + ib * es);
        float2 c[4];
        if (in_tab) {
            const float4 c01 = *reinterpret_cast<const float4*>(tr + m);
            const float4 c23 = *reinterpret_cast<const float4*>(tr + m + 2);
            c[0] = make_float2(c01.x, c01.y);
            c[1] = make_float2(c01.z, c01.w);
            c[2] = make_float2(c23.x, c23.y);
            c[3] = make_float2(c23.z, c23.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) rope_cos_sin_dev(p, static_cast<int>(m) + e, rp, a.ff, &c[e].x, &c[e].y);
        }
        float4 ya, yb;
        if constexpr (MODE == 2) {   // y[i] = x0 cos - x1 sin, y[i + half] = x0 sin + x1 cos
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x0 = get(xa, e), x1 = get(xb, e);
                set(ya, e, x0 * c[e].x - x1 * c[e].y);
                set(yb, e, x0 * c[e].y + x1 * c[e].x);
            }
        } else {                     // pairs (2k, 2k + 1)
            ya = make_float4(xa.x * c[0].x - xa.y * c[0].y, xa.x * c[0].y + xa.y * c[0].x,
                             xa.z * c[1].x - xa.w * c[1].y, xa.z * c[1].y + xa.w * c[1].x);
            yb = make_float4(xb.x * c[2].x - xb.y * c[2].y, xb.x * c[2].y + xb.y * c[2].x,
                             xb.z * c[3].x - xb.w * c[3].y, xb.z * c[3].y + xb.w * c[3].x);
        }
        Elt<T>::store4(yr + ia * es, ya);
        Elt<T>::store4(yr + ib * es, yb);
    }
    for (uint32_t q = threadIdx.x; q < a.ne1 * a.n_tail; q += nth) {
        const uint32_t h = q / a.n_tail;
        const uint32_t j = static_cast<uint32_t>(rp.n_dims) + (q - h * a.n_tail);
        *reinterpret_cast<T*>(yt + h * a.ynb1 + j * es) = *reinterpret_cast<const T*>(xt + h * a.xnb1 + j * es);
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
    a.nth = kRopeThreads;
    // four pairs a lane with vector loads: the block just covers the
    // token's pair groups (a multiple of 64 lanes, at most kRopeThreads)
    const int64_t al = x->type == CBX_TYPE_F32 ? 16 : 8;
    bool vec = p.n_dims % 8 == 0 && p.n_dims > 0 && reinterpret_cast<uintptr_t>(table) % 16 == 0;
    for (const cbx_tensor* t : {x, static_cast<const cbx_tensor*>(y)}) {
        if (reinterpret_cast<uintptr_t>(t->data) % al) vec = false;
        for (int k = 1; k < 4; k++) if (t->ne[k] > 1 && static_cast<int64_t>(t->nb[k]) % al) vec = false;
    }
    if (vec) {
        const int64_t groups = x->ne[1] * (p.n_dims / 8);
        const dim3 vblock(static_cast<unsigned>(std::min<int64_t>(kRopeThreads, cdiv(groups, 64) * 64)));
        a.nth = vblock.x;
        if (x->type == CBX_TYPE_F32) {
            if (p.mode == 2) hipLaunchKernelGGL((k_rope_vec<float, 2>), grid, vblock, 0, s, a);
            else hipLaunchKernelGGL((k_rope_vec<float, 0>), grid, vblock, 0, s, a);
        } else {
            if (p.mode == 2) hipLaunchKernelGGL((k_rope_vec<uint16_t, 2>), grid, vblock, 0, s, a);
            else hipLaunchKernelGGL((k_rope_vec<uint16_t, 0>), grid, vblock, 0, s, a);
        }
        return check_launch("rope_ext");
    }
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
