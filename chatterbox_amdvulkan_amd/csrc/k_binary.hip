// k_binary.hip -- ggml_add / ggml_mul with the second operand repeated to
// the first's shape, and ggml_concat.
//
// Binary: y[i0,i1,i2,i3] = a[i0,i1,i2,i3] op b[i0 % b.ne0, i1 % b.ne1,
// i2 % b.ne2, i3 % b.ne3] (ggml_can_repeat(b, a)), one f32 rounding -- the
// CFM decoder's mul(x, mask) of a (C, T) tensor by its per-frame mask
// before the 1x1 convs and around final_proj (cfm_decoder.cpp:176,553,555)
// and the residual join that ends a transformer stack (:244).  Contiguous tensors with b
// the same shape, a repeated row of ne0 values, or one value per row take
// one 4-element vector per lane over a grid that covers a once; other
// layouts take a workgroup per row.
//
// Bias + residual: y = r + (x + bias), the inner add rounded first -- a
// projection's bias add joined to the residual it feeds when no norm
// follows (cfm_decoder.cpp:162-165 the time MLP broadcast over the frames,
// :242-244 a stack's last ff.2).  Same two forms as the binary ops.
//
// Scale: y = x * s (ggml_scale) -- the mean of a HiFT stage's three
// resblocks (hift_vocoder.cpp:736), the same two forms.
//
// Concat: y = ggml_concat(a, b, dim) -- the decoder's channel packing and
// skip join (cfm_decoder.cpp:489-491,530), the time embeddings (:476), the
// HiFT vocoder's one-frame reflection pad (hift_vocoder.cpp:694-707).
// Contiguous tensors take one vector a lane over a grid that covers y once
// (each of y's blocks a's block then b's); other layouts a workgroup per
// output row.
#include <type_traits>

#include "cbx_internal.h"
#include "cbx_device.h"

namespace cbx {
namespace {

constexpr int kThreads = 256;

enum { BIN_SAME = 0, BIN_ROW = 1, BIN_COL = 2 };

template <int OP>
__device__ __forceinline__ float bin(float x, float y) {
    if constexpr (OP == CBX_BINARY_ADD) return x + y;
    else return x * y;
}

// MODE BIN_SAME: b[i]; BIN_ROW: b[i % (4 ne0_4)], b one period of a's
// leading dims (a row, or a (ne0, ne1) plane repeated over ne2: the flow
// encoder's (64, 8, 1) pos_bias over (64, 8, T) query heads); BIN_COL:
// b[row % nbr], one value a row of ne0 elements.
template <int OP, int MODE>
__global__ __launch_bounds__(kThreads) void k_binary_flat(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ y, uint32_t n4, uint32_t ne0_4,
                                                          uint32_t nbr) {
    arg_now(a);
    arg_now(b);
    arg_now(y);
    // lanes past the end load the last vector and store nothing (n4 >= 1)
    const uint32_t iu = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i = iu < n4 ? iu : n4 - 1;
    float4 bv;
    if constexpr (MODE == BIN_SAME) {
        bv = *reinterpret_cast<const float4*>(b + 4ull * i);
    } else if constexpr (MODE == BIN_ROW) {
        bv = *reinterpret_cast<const float4*>(b + 4u * (i % ne0_4));
    } else {
        const float s = b[(i / ne0_4) % nbr];
        bv = make_float4(s, s, s, s);
    }
    const float4 v = *reinterpret_cast<const float4*>(a + 4ull * i);
    const float4 o = make_float4(bin<OP>(v.x, bv.x), bin<OP>(v.y, bv.y), bin<OP>(v.z, bv.z), bin<OP>(v.w, bv.w));
    if (iu < n4) *reinterpret_cast<float4*>(y + 4ull * i) = o;
}

// Any strides: rows of a (and y) enumerate ne1, ne2, ne3; b's row is the
// repeat of the same indices.
template <int OP>
__global__ __launch_bounds__(kThreads) void k_binary_rows(View a, View b, View y, int64_t nr) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const int64_t i1 = r % a.ne[1], q = r / a.ne[1];
        const int64_t i2 = q % a.ne[2], i3 = q / a.ne[2];
        const char* ar = a.data + i1 * a.nb[1] + i2 * a.nb[2] + i3 * a.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
        const char* br = b.data + (i1 % b.ne[1]) * b.nb[1] + (i2 % b.ne[2]) * b.nb[2] + (i3 % b.ne[3]) * b.nb[3];
        for (int64_t j = threadIdx.x; j < a.ne[0]; j += kThreads) {
            const float x = *reinterpret_cast<const float*>(ar + j * a.nb[0]);
            const float v = *reinterpret_cast<const float*>(br + (j % b.ne[0]) * b.nb[0]);
            *reinterpret_cast<float*>(yr + j * y.nb[0]) = bin<OP>(x, v);
        }
    }
}

// one 4-element vector of an operand with r's shape (BIN_SAME) or of one
// repeated row of ne0 values (BIN_ROW)
template <int MODE>
__device__ __forceinline__ float4 load_rep(const float* __restrict__ p, uint32_t i, uint32_t ne0_4) {
    if constexpr (MODE == BIN_SAME) return *reinterpret_cast<const float4*>(p + 4ull * i);
    else return *reinterpret_cast<const float4*>(p + 4u * (i % ne0_4));
}

// y = r + (x + bias) over contiguous r and y; XM, BM: the modes of x and bias
template <int XM, int BM>
__global__ __launch_bounds__(kThreads) void k_bias_residual_flat(const float* __restrict__ x,
                                                                 const float* __restrict__ b,
                                                                 const float* __restrict__ r, float* __restrict__ y,
                                                                 uint32_t n4, uint32_t ne0_4) {
    arg_now(x);
    arg_now(b);
    arg_now(r);
    arg_now(y);
    const uint32_t iu = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i = iu < n4 ? iu : n4 - 1;
    const float4 xv = load_rep<XM>(x, i, ne0_4), bv = load_rep<BM>(b, i, ne0_4);
    const float4 rv = *reinterpret_cast<const float4*>(r + 4ull * i);
    const float4 o = make_float4(rv.x + (xv.x + bv.x), rv.y + (xv.y + bv.y), rv.z + (xv.z + bv.z),
                                 rv.w + (xv.w + bv.w));
    if (iu < n4) *reinterpret_cast<float4*>(y + 4ull * i) = o;
}

// yu = (x + bias) + u, yv = (x + bias) + v over contiguous x, yu, yv;
// bias, u and v each one period of x's leading dims (pb, pu, pv float4s)
__global__ __launch_bounds__(kThreads) void k_bias_add_pair_flat(const float* __restrict__ x,
                                                                 const float* __restrict__ b,
                                                                 const float* __restrict__ u,
                                                                 const float* __restrict__ v, float* __restrict__ yu,
                                                                 float* __restrict__ yv, uint32_t n4, uint32_t pb,
                                                                 uint32_t pu, uint32_t pv) {
    arg_now(x);
    arg_now(b);
    arg_now(u);
    arg_now(v);
    arg_now(yu);
    arg_now(yv);
    const uint32_t iu = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i = iu < n4 ? iu : n4 - 1;
    const float4 xv = *reinterpret_cast<const float4*>(x + 4ull * i);
    const float4 bv = *reinterpret_cast<const float4*>(b + 4u * (i % pb));
    const float4 uv = *reinterpret_cast<const float4*>(u + 4u * (i % pu));
    const float4 vv = *reinterpret_cast<const float4*>(v + 4u * (i % pv));
    const float4 sv = make_float4(xv.x + bv.x, xv.y + bv.y, xv.z + bv.z, xv.w + bv.w);
    if (iu < n4) {
        *reinterpret_cast<float4*>(yu + 4ull * i) = make_float4(sv.x + uv.x, sv.y + uv.y, sv.z + uv.z, sv.w + uv.w);
        *reinterpret_cast<float4*>(yv + 4ull * i) = make_float4(sv.x + vv.x, sv.y + vv.y, sv.z + vv.z, sv.w + vv.w);
    }
}

// y0 = x0 + b0 and y1 = x1 + b1, two independent bias adds over contiguous
// tensors, each bias one period of its x's leading dims (p0, p1 float4s):
// the first g0 workgroups take the first add's n0 float4s, the rest the
// second's n1 (which add is uniform per workgroup)
__global__ __launch_bounds__(kThreads) void k_bias_add_two_flat(const float* __restrict__ x0,
                                                                const float* __restrict__ b0, float* __restrict__ y0,
                                                                uint32_t n0, uint32_t p0, uint32_t g0,
                                                                const float* __restrict__ x1,
                                                                const float* __restrict__ b1, float* __restrict__ y1,
                                                                uint32_t n1, uint32_t p1) {
    const bool second = blockIdx.x >= g0;
    const uint32_t i = (second ? blockIdx.x - g0 : blockIdx.x) * kThreads + threadIdx.x;
    const float* x = second ? x1 : x0;
    const float* b = second ? b1 : b0;
    float* y = second ? y1 : y0;
    const uint32_t n = second ? n1 : n0, p = second ? p1 : p0;
    if (i >= n) return;
    const float4 xv = *reinterpret_cast<const float4*>(x + 4ull * i);
    const float4 bv = *reinterpret_cast<const float4*>(b + 4u * (i % p));
    *reinterpret_cast<float4*>(y + 4ull * i) = make_float4(xv.x + bv.x, xv.y + bv.y, xv.z + bv.z, xv.w + bv.w);
}

__device__ __forceinline__ const char* rep_row(const View& p, int64_t i1, int64_t i2, int64_t i3) {
    return p.data + (i1 % p.ne[1]) * p.nb[1] + (i2 % p.ne[2]) * p.nb[2] + (i3 % p.ne[3]) * p.nb[3];
}

__device__ __forceinline__ float rep_at(const char* row, const View& p, int64_t j) {
    return *reinterpret_cast<const float*>(row + (j % p.ne[0]) * p.nb[0]);
}

// Any strides: rows of x (and yu, yv) enumerate ne1, ne2, ne3; bias, u and
// v repeat to x by index
__global__ __launch_bounds__(kThreads) void k_bias_add_pair_rows(View x, View b, View u, View v, View yu, View yv,
                                                                 int64_t nr) {
    for (int64_t q = blockIdx.x; q < nr; q += gridDim.x) {
        const int64_t i1 = q % x.ne[1], w = q / x.ne[1];
        const int64_t i2 = w % x.ne[2], i3 = w / x.ne[2];
        const char* xr = x.data + i1 * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
        char* ur = yu.data + i1 * yu.nb[1] + i2 * yu.nb[2] + i3 * yu.nb[3];
        char* vr = yv.data + i1 * yv.nb[1] + i2 * yv.nb[2] + i3 * yv.nb[3];
        const char *br = rep_row(b, i1, i2, i3), *pur = rep_row(u, i1, i2, i3), *pvr = rep_row(v, i1, i2, i3);
        for (int64_t j = threadIdx.x; j < x.ne[0]; j += kThreads) {
            const float sv = *reinterpret_cast<const float*>(xr + j * x.nb[0]) + rep_at(br, b, j);
            *reinterpret_cast<float*>(ur + j * yu.nb[0]) = sv + rep_at(pur, u, j);
            *reinterpret_cast<float*>(vr + j * yv.nb[0]) = sv + rep_at(pvr, v, j);
        }
    }
}

// Any strides: rows of r (and y) enumerate ne1, ne2, ne3; x's and bias's
// rows are the repeats of the same indices (bias repeats to x and x to r,
// so i mod bias.ne = (i mod x.ne) mod bias.ne)
__global__ __launch_bounds__(kThreads) void k_bias_residual_rows(View x, View b, View r, View y, int64_t nr) {
    for (int64_t q = blockIdx.x; q < nr; q += gridDim.x) {
        const int64_t i1 = q % r.ne[1], u = q / r.ne[1];
        const int64_t i2 = u % r.ne[2], i3 = u / r.ne[2];
        const char* rr = r.data + i1 * r.nb[1] + i2 * r.nb[2] + i3 * r.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
        const char* xr = x.data + (i1 % x.ne[1]) * x.nb[1] + (i2 % x.ne[2]) * x.nb[2] + (i3 % x.ne[3]) * x.nb[3];
        const char* br = b.data + (i1 % b.ne[1]) * b.nb[1] + (i2 % b.ne[2]) * b.nb[2] + (i3 % b.ne[3]) * b.nb[3];
        for (int64_t j = threadIdx.x; j < r.ne[0]; j += kThreads) {
            const float xv = *reinterpret_cast<const float*>(xr + (j % x.ne[0]) * x.nb[0]);
            const float bv = *reinterpret_cast<const float*>(br + (j % b.ne[0]) * b.nb[0]);
            const float rv = *reinterpret_cast<const float*>(rr + j * r.nb[0]);
            *reinterpret_cast<float*>(yr + j * y.nb[0]) = rv + (xv + bv);
        }
    }
}

// y = x * s over contiguous x and y
__global__ __launch_bounds__(kThreads) void k_scale_flat(const float* __restrict__ x, float* __restrict__ y, float s,
                                                         uint32_t n4) {
    arg_now(x);
    arg_now(y);
    const uint32_t iu = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i = iu < n4 ? iu : n4 - 1;
    const float4 v = *reinterpret_cast<const float4*>(x + 4ull * i);
    if (iu < n4) *reinterpret_cast<float4*>(y + 4ull * i) = make_float4(v.x * s, v.y * s, v.z * s, v.w * s);
}

// any strides: a workgroup per row
__global__ __launch_bounds__(kThreads) void k_scale_rows(View x, View y, float s, int64_t nr) {
    for (int64_t q = blockIdx.x; q < nr; q += gridDim.x) {
        const int64_t i1 = q % x.ne[1], u = q / x.ne[1];
        const int64_t i2 = u % x.ne[2], i3 = u / x.ne[2];
        const char* xr = x.data + i1 * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
        for (int64_t j = threadIdx.x; j < x.ne[0]; j += kThreads) {
            *reinterpret_cast<float*>(yr + j * y.nb[0]) = *reinterpret_cast<const float*>(xr + j * x.nb[0]) * s;
        }
    }
}

// A workgroup per row of y: along dim 0 the row is a's row then b's; along
// dim d > 0 the row is a's when its index along d is below a.ne[d], else
// b's at that index minus a.ne[d].  ES: the element size (4 or 2).
template <int ES>
__global__ __launch_bounds__(kThreads) void k_concat(View a, View b, View y, int dim, int64_t nr) {
    using E = typename std::conditional<ES == 4, uint32_t, uint16_t>::type;
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        int64_t idx[4];
        idx[1] = r % y.ne[1];
        const int64_t q = r / y.ne[1];
        idx[2] = q % y.ne[2];
        idx[3] = q / y.ne[2];
        char* yr = y.data + idx[1] * y.nb[1] + idx[2] * y.nb[2] + idx[3] * y.nb[3];
        if (dim == 0) {
            const char* ar = a.data + idx[1] * a.nb[1] + idx[2] * a.nb[2] + idx[3] * a.nb[3];
            const char* br = b.data + idx[1] * b.nb[1] + idx[2] * b.nb[2] + idx[3] * b.nb[3];
            for (int64_t j = threadIdx.x; j < y.ne[0]; j += kThreads) {
                const E v = j < a.ne[0] ? *reinterpret_cast<const E*>(ar + j * a.nb[0])
                                        : *reinterpret_cast<const E*>(br + (j - a.ne[0]) * b.nb[0]);
                *reinterpret_cast<E*>(yr + j * y.nb[0]) = v;
            }
        } else {
            // the source's fields by value (a reference to a kernel argument
            // would put the argument block in scratch)
            const bool from_a = idx[dim] < a.ne[dim];
            if (!from_a) idx[dim] -= a.ne[dim];
            const char* sd = from_a ? a.data : b.data;
            const int64_t s0 = from_a ? a.nb[0] : b.nb[0], s1 = from_a ? a.nb[1] : b.nb[1];
            const int64_t s2 = from_a ? a.nb[2] : b.nb[2], s3 = from_a ? a.nb[3] : b.nb[3];
            const char* sr = sd + idx[1] * s1 + idx[2] * s2 + idx[3] * s3;
            for (int64_t j = threadIdx.x; j < y.ne[0]; j += kThreads) {
                *reinterpret_cast<E*>(yr + j * y.nb[0]) = *reinterpret_cast<const E*>(sr + j * s0);
            }
        }
    }
}

// Contiguous a, b and y: y is `outer` blocks, each a's block of na vectors
// then b's of nb (na, nb: the elements up to and including the concat dim,
// in units of V).  One vector a lane over a grid that covers y once.
template <typename V>
__global__ __launch_bounds__(kThreads) void k_concat_flat(const V* __restrict__ a, const V* __restrict__ b,
                                                          V* __restrict__ y, uint32_t na, uint32_t nb, uint32_t n) {
    arg_now(a);
    arg_now(b);
    arg_now(y);
    const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const uint32_t blk = i / (na + nb), r = i - blk * (na + nb);
    y[i] = r < na ? a[blk * na + r] : b[blk * nb + (r - na)];
}

bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// An operand p of r's leading dims (p.ne[k] == r.ne[k] below some k >= 1,
// 1 from k on), contiguous and 16-byte aligned: the float4s of one period
// of it in r's elements, or 0 when p is not such an operand.
uint32_t period4(const cbx_tensor* p, const cbx_tensor* r) {
    if (!is_contiguous(p) || !al16(p->data)) return 0;
    int k = 0;
    int64_t per = 1;
    while (k < 4 && p->ne[k] == r->ne[k]) per *= r->ne[k++];
    for (int j = k; j < 4; j++) {
        if (p->ne[j] != 1) return 0;
    }
    return k >= 1 && per % 4 == 0 && per / 4 < (int64_t{1} << 31) ? static_cast<uint32_t>(per / 4) : 0;
}

template <int OP>
void binary_go(const cbx_tensor* a, const cbx_tensor* b, cbx_tensor* y, hipStream_t s) {
    const int64_t n = nelements(a);
    const bool same = same_shape(a, b) && is_contiguous(b) && al16(b->data);
    const uint32_t per4 = period4(b, a);
    const bool row = !same && per4 > 0;
    const bool col = b->ne[0] == 1 && b->ne[1] == a->ne[1] && b->ne[2] == 1 && b->ne[3] == 1 &&
                     (b->ne[1] == 1 || b->nb[1] == sizeof(float));
    const bool flat = is_contiguous(a) && is_contiguous(y) && al16(a->data) && al16(y->data) && a->ne[0] % 4 == 0 &&
                      n / 4 < (int64_t{1} << 31) && (same || row || col);
    if (flat) {
        const uint32_t n4 = static_cast<uint32_t>(n / 4);
        const uint32_t ne0_4 = row ? per4 : static_cast<uint32_t>(a->ne[0] / 4);
        const uint32_t nbr = static_cast<uint32_t>(b->ne[1]);
        const dim3 grid(static_cast<unsigned>(cdiv(n4, kThreads)));
        const float* ap = static_cast<const float*>(a->data);
        const float* bp = static_cast<const float*>(b->data);
        float* yp = static_cast<float*>(y->data);
        if (same) hipLaunchKernelGGL((k_binary_flat<OP, BIN_SAME>), grid, dim3(kThreads), 0, s, ap, bp, yp, n4, ne0_4, nbr);
        else if (row) hipLaunchKernelGGL((k_binary_flat<OP, BIN_ROW>), grid, dim3(kThreads), 0, s, ap, bp, yp, n4, ne0_4, nbr);
        else hipLaunchKernelGGL((k_binary_flat<OP, BIN_COL>), grid, dim3(kThreads), 0, s, ap, bp, yp, n4, ne0_4, nbr);
        return;
    }
    const int64_t nr = nrows(a);
    hipLaunchKernelGGL((k_binary_rows<OP>), dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20))),
                       dim3(kThreads), 0, s, view_of(a), view_of(b), view_of(y), nr);
}

// x or bias as a flat operand of r's shape: 0 the same shape, 1 one row, -1 neither
int flat_mode(const cbx_tensor* p, const cbx_tensor* r) {
    if (!is_contiguous(p) || !al16(p->data)) return -1;
    if (same_shape(p, r)) return BIN_SAME;
    if (p->ne[0] == r->ne[0] && p->ne[1] == 1 && p->ne[2] == 1 && p->ne[3] == 1) return BIN_ROW;
    return -1;
}

}  // namespace

int launch_bias_residual(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* r, cbx_tensor* y,
                         hipStream_t s) {
    const int64_t n = nelements(r);
    const int xm = flat_mode(x, r), bm = flat_mode(bias, r);
    if (xm >= 0 && bm >= 0 && is_contiguous(r) && is_contiguous(y) && al16(r->data) && al16(y->data) &&
        r->ne[0] % 4 == 0 && n / 4 < (int64_t{1} << 31)) {
        const uint32_t n4 = static_cast<uint32_t>(n / 4), ne0_4 = static_cast<uint32_t>(r->ne[0] / 4);
        const dim3 grid(static_cast<unsigned>(cdiv(n4, kThreads)));
        const float* xp = static_cast<const float*>(x->data);
        const float* bp = static_cast<const float*>(bias->data);
        const float* rp = static_cast<const float*>(r->data);
        float* yp = static_cast<float*>(y->data);
        if (xm == BIN_SAME && bm == BIN_SAME) {
            hipLaunchKernelGGL((k_bias_residual_flat<BIN_SAME, BIN_SAME>), grid, dim3(kThreads), 0, s, xp, bp, rp, yp,
                               n4, ne0_4);
        } else if (xm == BIN_SAME) {
            hipLaunchKernelGGL((k_bias_residual_flat<BIN_SAME, BIN_ROW>), grid, dim3(kThreads), 0, s, xp, bp, rp, yp,
                               n4, ne0_4);
        } else {   // x one row: bias, repeating to it, is one row too
            hipLaunchKernelGGL((k_bias_residual_flat<BIN_ROW, BIN_ROW>), grid, dim3(kThreads), 0, s, xp, bp, rp, yp,
                               n4, ne0_4);
        }
    } else {
        const int64_t nr = nrows(r);
        hipLaunchKernelGGL(k_bias_residual_rows, dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20))),
                           dim3(kThreads), 0, s, view_of(x), view_of(bias), view_of(r), view_of(y), nr);
    }
    return check_launch("bias residual");
}

int launch_bias_add_two(const cbx_tensor* x0, const cbx_tensor* b0, cbx_tensor* y0, const cbx_tensor* x1,
                        const cbx_tensor* b1, cbx_tensor* y1, DeviceState* st, hipStream_t s) {
    const int64_t m0 = nelements(x0), m1 = nelements(x1);
    auto flat = [](const cbx_tensor* x, const cbx_tensor* b, const cbx_tensor* y) {
        return period4(b, x) > 0 && is_contiguous(x) && is_contiguous(y) && al16(x->data) && al16(y->data);
    };
    const int64_t g0 = cdiv(m0 / 4, kThreads), g1 = cdiv(m1 / 4, kThreads);
    if (m0 > 0 && m1 > 0 && flat(x0, b0, y0) && flat(x1, b1, y1) && g0 + g1 < (int64_t{1} << 31)) {
        hipLaunchKernelGGL(k_bias_add_two_flat, dim3(static_cast<unsigned>(g0 + g1)), dim3(kThreads), 0, s,
                           static_cast<const float*>(x0->data), static_cast<const float*>(b0->data),
                           static_cast<float*>(y0->data), static_cast<uint32_t>(m0 / 4), period4(b0, x0),
                           static_cast<uint32_t>(g0), static_cast<const float*>(x1->data),
                           static_cast<const float*>(b1->data), static_cast<float*>(y1->data),
                           static_cast<uint32_t>(m1 / 4), period4(b1, x1));
        return check_launch("bias add two");
    }
    // other layouts: the two bias adds one after the other
    int rc = m0 > 0 ? launch_bias_act(CBX_UNARY_NONE, x0, b0, y0, st, s) : CBX_OK;
    if (rc == CBX_OK && m1 > 0) rc = launch_bias_act(CBX_UNARY_NONE, x1, b1, y1, st, s);
    return rc;
}

int launch_bias_add_pair(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* u, const cbx_tensor* v,
                         cbx_tensor* yu, cbx_tensor* yv, hipStream_t s) {
    const int64_t n = nelements(x);
    const uint32_t pb = period4(bias, x), pu = period4(u, x), pv = period4(v, x);
    if (pb && pu && pv && is_contiguous(x) && is_contiguous(yu) && is_contiguous(yv) && al16(x->data) &&
        al16(yu->data) && al16(yv->data) && n / 4 < (int64_t{1} << 31)) {   // pb > 0: n a multiple of 4
        const uint32_t n4 = static_cast<uint32_t>(n / 4);
        hipLaunchKernelGGL(k_bias_add_pair_flat, dim3(static_cast<unsigned>(cdiv(n4, kThreads))), dim3(kThreads), 0, s,
                           static_cast<const float*>(x->data), static_cast<const float*>(bias->data),
                           static_cast<const float*>(u->data), static_cast<const float*>(v->data),
                           static_cast<float*>(yu->data), static_cast<float*>(yv->data), n4, pb, pu, pv);
    } else {
        const int64_t nr = nrows(x);
        hipLaunchKernelGGL(k_bias_add_pair_rows, dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20))),
                           dim3(kThreads), 0, s, view_of(x), view_of(bias), view_of(u), view_of(v), view_of(yu),
                           view_of(yv), nr);
    }
    return check_launch("bias add pair");
}

int launch_scale(const cbx_tensor* x, float s, cbx_tensor* y, hipStream_t strm) {
    const int64_t n = nelements(x);
    if (is_contiguous(x) && is_contiguous(y) && al16(x->data) && al16(y->data) && n % 4 == 0 &&
        n / 4 < (int64_t{1} << 31)) {
        const uint32_t n4 = static_cast<uint32_t>(n / 4);
        hipLaunchKernelGGL(k_scale_flat, dim3(static_cast<unsigned>(cdiv(n4, kThreads))), dim3(kThreads), 0, strm,
                           static_cast<const float*>(x->data), static_cast<float*>(y->data), s, n4);
    } else {
        const int64_t nr = nrows(x);
        hipLaunchKernelGGL(k_scale_rows, dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20))),
                           dim3(kThreads), 0, strm, view_of(x), view_of(y), s, nr);
    }
    return check_launch("scale");
}

int launch_binary(int op, const cbx_tensor* a, const cbx_tensor* b, cbx_tensor* y, hipStream_t s) {
    if (op == CBX_BINARY_ADD) binary_go<CBX_BINARY_ADD>(a, b, y, s);
    else binary_go<CBX_BINARY_MUL>(a, b, y, s);
    return check_launch(op == CBX_BINARY_ADD ? "binary add" : "binary mul");
}

int launch_concat(const cbx_tensor* a, const cbx_tensor* b, int dim, cbx_tensor* y, hipStream_t s) {
    if (is_contiguous(a) && is_contiguous(b) && is_contiguous(y) && nelements(y) < (int64_t{1} << 32)) {
        int64_t ia = 1, ib = 1;
        for (int k = 0; k <= dim; k++) {
            ia *= a->ne[k];
            ib *= b->ne[k];
        }
        const int64_t es = y->type == CBX_TYPE_F32 ? 4 : 2;
        const bool v16 = (ia * es) % 16 == 0 && (ib * es) % 16 == 0 && al16(a->data) && al16(b->data) && al16(y->data);
        const int64_t vb = v16 ? 16 : es;
        const uint32_t na = static_cast<uint32_t>(ia * es / vb), nb = static_cast<uint32_t>(ib * es / vb);
        const uint32_t n = static_cast<uint32_t>(nelements(y) * es / vb);
        const dim3 grid(static_cast<unsigned>(cdiv(n, kThreads)));
        if (v16) {
            hipLaunchKernelGGL(k_concat_flat<uint4>, grid, dim3(kThreads), 0, s, static_cast<const uint4*>(a->data),
                               static_cast<const uint4*>(b->data), static_cast<uint4*>(y->data), na, nb, n);
        } else if (es == 4) {
            hipLaunchKernelGGL(k_concat_flat<uint32_t>, grid, dim3(kThreads), 0, s,
                               static_cast<const uint32_t*>(a->data), static_cast<const uint32_t*>(b->data),
                               static_cast<uint32_t*>(y->data), na, nb, n);
        } else {
            hipLaunchKernelGGL(k_concat_flat<uint16_t>, grid, dim3(kThreads), 0, s,
                               static_cast<const uint16_t*>(a->data), static_cast<const uint16_t*>(b->data),
                               static_cast<uint16_t*>(y->data), na, nb, n);
        }
        return check_launch("concat");
    }
    const int64_t nr = nrows(y);
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20)));
    if (y->type == CBX_TYPE_F32) {
        hipLaunchKernelGGL((k_concat<4>), grid, dim3(kThreads), 0, s, view_of(a), view_of(b), view_of(y), dim, nr);
    } else {
        hipLaunchKernelGGL((k_concat<2>), grid, dim3(kThreads), 0, s, view_of(a), view_of(b), view_of(y), dim, nr);
    }
    return check_launch("concat");
}

}  // namespace cbx
