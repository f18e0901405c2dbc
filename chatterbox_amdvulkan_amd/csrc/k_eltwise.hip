// k_eltwise.hip -- element-wise activations: the ggml unary ops, leaky_relu,
// swiglu (silu(g) * u), bias add + activation and the fused Snake chain.
//
// Contiguous tensors take the streaming path: one 4-element vector per lane
// over a grid that covers the tensor once (no grid-stride loop), with
// nontemporal 16-byte loads and stores for f32 (8-byte for f16); the lane
// just past the last full vector also does the n % 4 tail.  On MI355X this
// shape sustains the highest bandwidth at every size measured (4 MiB to
// 1 GiB).  Non-contiguous tensors (rows with nb[0] == element size) take a
// row loop.
//
// Each op body is ggml-cpu's scalar expression, compiled without FMA
// contraction.  GELU reproduces the fp16 table exactly (act_gelu_fast).
// Other transcendentals (expf, logf, tanhf, erff, sinf) are the device's
// libm and may differ from the CPU result in the last bit; Snake's sin^2 is
// the compact sin_sq_small below 2^16 (an ulp or two from the CPU's).
#include "cbx_device.h"

namespace cbx {
namespace {

constexpr int kThreads = 256;

template <int OP>
__device__ __forceinline__ float unary_op(float x, const uint16_t* __restrict__ tab, float param) {
    if constexpr (OP == CBX_UNARY_GELU) return act_gelu_fast(tab, x);
    else if constexpr (OP == CBX_UNARY_GELU_ERF) return act_gelu_erf(x);
    else if constexpr (OP == CBX_UNARY_SILU) return act_silu(x);
    else if constexpr (OP == CBX_UNARY_TANH) return tanhf(x);
    else if constexpr (OP == CBX_UNARY_SOFTPLUS) return act_softplus(x);
    else if constexpr (OP == CBX_UNARY_SIN) return sinf(x);
    else if constexpr (OP == CBX_UNARY_SQR) return x * x;
    else if constexpr (OP == CBX_UNARY_MISH) return act_mish(x);
    else return act_leaky(x, param);
}

// ggml_vec_gelu_f16: the f16 path indexes the table with the input's code.
template <int OP>
__device__ __forceinline__ uint16_t unary_f16_code(uint16_t h, const uint16_t* __restrict__ tab, float param) {
    if constexpr (OP == CBX_UNARY_GELU) return tab[h];
    else return f2h(unary_op<OP>(h2f(h), tab, param));
}

template <typename T, int OP>
__device__ __forceinline__ void unary_scalar(const char* x, char* y, int64_t i, const uint16_t* tab, float param) {
    if constexpr (std::is_same<T, uint16_t>::value) {
        *reinterpret_cast<uint16_t*>(y + i * 2) = unary_f16_code<OP>(*reinterpret_cast<const uint16_t*>(x + i * 2), tab, param);
    } else {
        reinterpret_cast<float*>(y)[i] = unary_op<OP>(reinterpret_cast<const float*>(x)[i], tab, param);
    }
}

template <typename T, int OP>
__global__ __launch_bounds__(kThreads) void k_unary(const char* __restrict__ x, char* __restrict__ y, int64_t n,
                                                    float param, const uint16_t* __restrict__ tab) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t n4 = n >> 2;
    if (i < n4) {
        if constexpr (std::is_same<T, uint16_t>::value && OP == CBX_UNARY_GELU) {
            const cbx_u2v raw = __builtin_nontemporal_load(reinterpret_cast<const cbx_u2v*>(x + i * 8));
            cbx_u2v o;
            o.x = tab[raw.x & 0xffffu] | (static_cast<uint32_t>(tab[raw.x >> 16]) << 16);
            o.y = tab[raw.y & 0xffffu] | (static_cast<uint32_t>(tab[raw.y >> 16]) << 16);
            __builtin_nontemporal_store(o, reinterpret_cast<cbx_u2v*>(y + i * 8));
        } else {
            const float4 v = Stream<T>::load4(x + i * 4 * Elt<T>::size);
            float4 o;
            if constexpr (OP == CBX_UNARY_GELU) {
                o = act_gelu_fast4(tab, v);
            } else {
                o.x = unary_op<OP>(v.x, tab, param);
                o.y = unary_op<OP>(v.y, tab, param);
                o.z = unary_op<OP>(v.z, tab, param);
                o.w = unary_op<OP>(v.w, tab, param);
            }
            Stream<T>::store4(y + i * 4 * Elt<T>::size, o);
        }
    } else if (i == n4) {
        for (int64_t j = n4 * 4; j < n; j++) unary_scalar<T, OP>(x, y, j, tab, param);
    }
}

template <typename T, int OP>
__global__ __launch_bounds__(kThreads) void k_unary_rows(View x, View y, int64_t nr, float param,
                                                         const uint16_t* __restrict__ tab, bool fx, bool fy) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const char* xr = x.data + row_offset(x, r, fx);
        char* yr = y.data + row_offset(y, r, fy);
        for (int64_t j = threadIdx.x; j < x.ne[0]; j += kThreads) unary_scalar<T, OP>(xr, yr, j, tab, param);
    }
}

// ---- swiglu -------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(kThreads) void k_swiglu(const char* __restrict__ g, const char* __restrict__ u,
                                                     char* __restrict__ y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t n4 = n >> 2;
    constexpr int es = Elt<T>::size;
    if (i < n4) {
        const float4 vg = Stream<T>::load4(g + i * 4 * es);
        const float4 vu = Stream<T>::load4(u + i * 4 * es);
        float4 o;
        o.x = act_silu(vg.x) * vu.x;
        o.y = act_silu(vg.y) * vu.y;
        o.z = act_silu(vg.z) * vu.z;
        o.w = act_silu(vg.w) * vu.w;
        Stream<T>::store4(y + i * 4 * es, o);
    } else if (i == n4) {
        for (int64_t j = n4 * 4; j < n; j++) {
            Elt<T>::store1(y + j * es, act_silu(Elt<T>::load1(g + j * es)) * Elt<T>::load1(u + j * es));
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void k_swiglu_rows(View g, View u, View y, int64_t nr) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const char* gr = g.data + row_offset(g, r, false);
        const char* ur = u.data + row_offset(u, r, false);
        char* yr = y.data + row_offset(y, r, false);
        for (int64_t j = threadIdx.x; j < g.ne[0]; j += kThreads) {
            const float gv = Elt<T>::load1(gr + j * Elt<T>::size), uv = Elt<T>::load1(ur + j * Elt<T>::size);
            Elt<T>::store1(yr + j * Elt<T>::size, act_silu(gv) * uv);
        }
    }
}

// ---- snake --------------------------------------------------------------------
// y = x + sin(x*a)^2 * ainv (snake_elem: the five ggml ops of snake() in
// their order).

__device__ __forceinline__ float snake1(float xv, float a, float ai) { return snake_elem(xv, a, ai); }

// Contiguous x/y.  INNER: alpha per element of ne[0] (the reference's (C, T)
// layout, C % 4 == 0), channel = element % C.  Otherwise alpha per row of
// ne[0] (ne0 % 4 == 0), channel = (element / ne0) % ne1.  Indices use 32-bit
// arithmetic (the launcher guarantees n < 2^32); cmask = C - 1 when C is a
// power of two.
template <bool INNER>
__global__ __launch_bounds__(kThreads) void k_snake(const float* __restrict__ x, float* __restrict__ y,
                                                    const float* __restrict__ a, const float* __restrict__ ai,
                                                    uint32_t n4, uint32_t C, uint32_t cmask, uint32_t ne0_4) {
    // lanes past the end load the last vector and store nothing: no early
    // exit stands before the loads (n4 >= 1)
    arg_now(x);
    arg_now(y);
    arg_now(a);
    arg_now(ai);
    const uint32_t iu = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i = iu < n4 ? iu : n4 - 1;
    uint32_t c;
    if constexpr (INNER) {
        c = cmask ? (4u * i) & cmask : (4u * i) % C;
    } else {
        const uint32_t row = i / ne0_4;
        c = cmask ? row & cmask : row % C;
    }
    const float4 v = Stream<float>::load4(reinterpret_cast<const char*>(x + 4ull * i));
    float4 o;
    if constexpr (INNER) {
        const float4 av = *reinterpret_cast<const float4*>(a + c);
        const float4 iv = *reinterpret_cast<const float4*>(ai + c);
        o.x = snake1(v.x, av.x, iv.x);
        o.y = snake1(v.y, av.y, iv.y);
        o.z = snake1(v.z, av.z, iv.z);
        o.w = snake1(v.w, av.w, iv.w);
    } else {
        const float av = a[c], iv = ai[c];
        o.x = snake1(v.x, av, iv);
        o.y = snake1(v.y, av, iv);
        o.z = snake1(v.z, av, iv);
        o.w = snake1(v.w, av, iv);
    }
    if (iu < n4) Stream<float>::store4(reinterpret_cast<char*>(y + 4ull * i), o);
}

// General rows: alpha either per element of ne[0] (inner) or per row i1 (outer).
template <bool INNER>
__global__ __launch_bounds__(kThreads) void k_snake_rows(View x, View y, const float* __restrict__ a,
                                                         const float* __restrict__ ai, int64_t nr,
                                                         int64_t chunks_per_row, bool fx, bool fy) {
    const int64_t ne0 = x.ne[0];
    const int64_t total = nr * chunks_per_row;
    for (int64_t bidx = blockIdx.x; bidx < total; bidx += gridDim.x) {
        const int64_t r = bidx / chunks_per_row;
        const int64_t chunk = bidx - r * chunks_per_row;
        const int64_t i1 = r % x.ne[1];
        const float* xr = reinterpret_cast<const float*>(x.data + row_offset(x, r, fx));
        float* yr = reinterpret_cast<float*>(y.data + row_offset(y, r, fy));
        const float ar = INNER ? 0.0f : a[i1];
        const float ir = INNER ? 0.0f : ai[i1];
        const int64_t j0 = chunk * kThreads * 4;
        const int64_t j1 = j0 + kThreads * 4 < ne0 ? j0 + kThreads * 4 : ne0;
        for (int64_t j = j0 + threadIdx.x; j < j1; j += kThreads) {
            yr[j] = INNER ? snake1(xr[j], a[j], ai[j]) : snake1(xr[j], ar, ir);
        }
    }
}

// ---- bias add + activation -------------------------------------------------------
// y = act(x + bias): the ggml_add of a bias vector rounded to f32, then the
// activation node reading it (t3.cpp:535-537, cfm_decoder.cpp:237-239,
// flow_encoder.cpp:401-402, s3enc.cpp:176-177).  INNER: the bias runs along
// ne[0] (ne0 % 4 == 0), element c = element % ne0; otherwise one bias value
// per row index i1 (the (1, C) bias of a time-major tensor,
// s3enc.cpp:117-120), c = (element / ne0) % ne1.

template <int OP>
__device__ __forceinline__ float4 act4(float4 t, const uint16_t* __restrict__ tab) {
    if constexpr (OP == CBX_UNARY_NONE) {
        return t;
    } else if constexpr (OP == CBX_UNARY_GELU) {
        return act_gelu_fast4(tab, t);
    } else {
        return make_float4(unary_op<OP>(t.x, tab, 0.0f), unary_op<OP>(t.y, tab, 0.0f), unary_op<OP>(t.z, tab, 0.0f),
                           unary_op<OP>(t.w, tab, 0.0f));
    }
}

template <int OP, bool INNER>
__global__ __launch_bounds__(kThreads) void k_bias_act(const float* __restrict__ x, float* __restrict__ y,
                                                       const float* __restrict__ bias, uint32_t n4, uint32_t C,
                                                       uint32_t cmask, uint32_t ne0_4, const uint16_t* __restrict__ tab) {
    // lanes past the end load the last vector and store nothing (n4 >= 1)
    arg_now(x);
    arg_now(y);
    arg_now(bias);
    const uint32_t iu = blockIdx.x * kThreads + threadIdx.x;
    const uint32_t i = iu < n4 ? iu : n4 - 1;
    float4 bv;
    if constexpr (INNER) {
        const uint32_t c = cmask ? (4u * i) & cmask : (4u * i) % C;
        bv = *reinterpret_cast<const float4*>(bias + c);
    } else {
        const uint32_t row = i / ne0_4;
        const float bb = bias[cmask ? row & cmask : row % C];
        bv = make_float4(bb, bb, bb, bb);
    }
    const float4 v = Stream<float>::load4(reinterpret_cast<const char*>(x + 4ull * i));
    const float4 t = make_float4(v.x + bv.x, v.y + bv.y, v.z + bv.z, v.w + bv.w);
    const float4 o = act4<OP>(t, tab);
    if (iu < n4) Stream<float>::store4(reinterpret_cast<char*>(y + 4ull * i), o);
}

template <int OP>
__global__ __launch_bounds__(kThreads) void k_bias_act_rows(View x, View y, const float* __restrict__ bias, int64_t nr,
                                                            bool inner, bool fx, bool fy,
                                                            const uint16_t* __restrict__ tab) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const float* xr = reinterpret_cast<const float*>(x.data + row_offset(x, r, fx));
        float* yr = reinterpret_cast<float*>(y.data + row_offset(y, r, fy));
        const float br = inner ? 0.0f : bias[r % x.ne[1]];
        for (int64_t j = threadIdx.x; j < x.ne[0]; j += kThreads) {
            const float t = xr[j] + (inner ? bias[j] : br);
            if constexpr (OP == CBX_UNARY_NONE) yr[j] = t;
            else yr[j] = unary_op<OP>(t, tab, 0.0f);
        }
    }
}

// ---- launch helpers -------------------------------------------------------------

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// grid covering n4 vectors plus the tail lane
dim3 full_grid(int64_t n4) { return dim3(static_cast<unsigned>(cdiv(n4 + 1, kThreads))); }

template <typename T, int OP>
void unary_go(const cbx_tensor* x, cbx_tensor* y, float param, DeviceState* st, hipStream_t s, bool flat) {
    if (flat) {
        const int64_t n = nelements(x);
        hipLaunchKernelGGL((k_unary<T, OP>), full_grid(n >> 2), dim3(kThreads), 0, s,
                           static_cast<const char*>(x->data), static_cast<char*>(y->data), n, param, st->gelu_table);
    } else {
        const int64_t nr = nrows(x);
        hipLaunchKernelGGL((k_unary_rows<T, OP>), dim3(std::min<int64_t>(nr, int64_t{1} << 20)), dim3(kThreads), 0,
                           s, view_of(x), view_of(y), nr, param, st->gelu_table, flat_rows(x), flat_rows(y));
    }
}

template <typename T>
void unary_dispatch(int op, const cbx_tensor* x, cbx_tensor* y, float param, DeviceState* st, hipStream_t s,
                    bool flat) {
    switch (op) {
        case CBX_UNARY_GELU: unary_go<T, CBX_UNARY_GELU>(x, y, param, st, s, flat); break;
        case CBX_UNARY_GELU_ERF: unary_go<T, CBX_UNARY_GELU_ERF>(x, y, param, st, s, flat); break;
        case CBX_UNARY_SILU: unary_go<T, CBX_UNARY_SILU>(x, y, param, st, s, flat); break;
        case CBX_UNARY_TANH: unary_go<T, CBX_UNARY_TANH>(x, y, param, st, s, flat); break;
        case CBX_UNARY_SOFTPLUS: unary_go<T, CBX_UNARY_SOFTPLUS>(x, y, param, st, s, flat); break;
        case CBX_UNARY_SIN: unary_go<T, CBX_UNARY_SIN>(x, y, param, st, s, flat); break;
        case CBX_UNARY_SQR: unary_go<T, CBX_UNARY_SQR>(x, y, param, st, s, flat); break;
        case CBX_UNARY_MISH: unary_go<T, CBX_UNARY_MISH>(x, y, param, st, s, flat); break;
        default: unary_go<T, UNARY_LEAKY>(x, y, param, st, s, flat); break;
    }
}

template <int OP>
void bias_act_go(const cbx_tensor* x, const cbx_tensor* bias, bool inner, cbx_tensor* y, DeviceState* st,
                 hipStream_t s) {
    const int64_t n = nelements(x);
    const int64_t C = inner ? x->ne[0] : x->ne[1];
    const bool flat = is_contiguous(x) && is_contiguous(y) && aligned(x->data, 16) && aligned(y->data, 16) &&
                      aligned(bias->data, 16) && x->ne[0] % 4 == 0 && n / 4 < (int64_t{1} << 32);
    if (flat) {
        const uint32_t n4 = static_cast<uint32_t>(n / 4);
        const uint32_t cmask = (C & (C - 1)) == 0 ? static_cast<uint32_t>(C - 1) : 0u;
        const uint32_t ne0_4 = static_cast<uint32_t>(x->ne[0] / 4);
        const dim3 grid(static_cast<unsigned>(cdiv(n4, kThreads)));
        const float* xp = static_cast<const float*>(x->data);
        float* yp = static_cast<float*>(y->data);
        const float* bp = static_cast<const float*>(bias->data);
        if (inner) {
            hipLaunchKernelGGL((k_bias_act<OP, true>), grid, dim3(kThreads), 0, s, xp, yp, bp, n4,
                               static_cast<uint32_t>(C), cmask, ne0_4, st->gelu_table);
        } else {
            hipLaunchKernelGGL((k_bias_act<OP, false>), grid, dim3(kThreads), 0, s, xp, yp, bp, n4,
                               static_cast<uint32_t>(C), cmask, ne0_4, st->gelu_table);
        }
    } else {
        const int64_t nr = nrows(x);
        hipLaunchKernelGGL((k_bias_act_rows<OP>), dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20))),
                           dim3(kThreads), 0, s, view_of(x), view_of(y), static_cast<const float*>(bias->data), nr,
                           inner, flat_rows(x), flat_rows(y), st->gelu_table);
    }
}

}  // namespace

int launch_bias_act(int op, const cbx_tensor* x, const cbx_tensor* bias, cbx_tensor* y, DeviceState* st,
                    hipStream_t s) {
    const bool inner = bias->ne[0] == x->ne[0] && bias->ne[1] == 1;
    switch (op) {
        case CBX_UNARY_NONE: bias_act_go<CBX_UNARY_NONE>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_GELU: bias_act_go<CBX_UNARY_GELU>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_GELU_ERF: bias_act_go<CBX_UNARY_GELU_ERF>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_SILU: bias_act_go<CBX_UNARY_SILU>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_TANH: bias_act_go<CBX_UNARY_TANH>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_SOFTPLUS: bias_act_go<CBX_UNARY_SOFTPLUS>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_SIN: bias_act_go<CBX_UNARY_SIN>(x, bias, inner, y, st, s); break;
        case CBX_UNARY_SQR: bias_act_go<CBX_UNARY_SQR>(x, bias, inner, y, st, s); break;
        default: bias_act_go<CBX_UNARY_MISH>(x, bias, inner, y, st, s); break;
    }
    return check_launch("bias_act");
}

int launch_unary(int op, float param, const cbx_tensor* x, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    const size_t a = x->type == CBX_TYPE_F32 ? 16 : 8;
    const bool flat = is_contiguous(x) && is_contiguous(y) && aligned(x->data, a) && aligned(y->data, a) &&
                      nelements(x) / 4 + 1 < (int64_t{1} << 39);
    if (x->type == CBX_TYPE_F32) unary_dispatch<float>(op, x, y, param, st, s, flat);
    else unary_dispatch<uint16_t>(op, x, y, param, st, s, flat);
    return check_launch("unary");
}

int launch_swiglu(const cbx_tensor* g, const cbx_tensor* u, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    (void)st;
    const size_t a = g->type == CBX_TYPE_F32 ? 16 : 8;
    const int64_t n = nelements(y);
    const bool flat = is_contiguous(g) && is_contiguous(u) && is_contiguous(y) && aligned(g->data, a) &&
                      aligned(u->data, a) && aligned(y->data, a) && n / 4 + 1 < (int64_t{1} << 39);
    if (flat) {
        const char* gp = static_cast<const char*>(g->data);
        const char* up = static_cast<const char*>(u->data);
        char* yp = static_cast<char*>(y->data);
        if (g->type == CBX_TYPE_F32) hipLaunchKernelGGL((k_swiglu<float>), full_grid(n >> 2), dim3(kThreads), 0, s, gp, up, yp, n);
        else hipLaunchKernelGGL((k_swiglu<uint16_t>), full_grid(n >> 2), dim3(kThreads), 0, s, gp, up, yp, n);
    } else {
        const int64_t nr = nrows(y);
        const dim3 grid(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20)));
        if (g->type == CBX_TYPE_F32) {
            hipLaunchKernelGGL((k_swiglu_rows<float>), grid, dim3(kThreads), 0, s, view_of(g), view_of(u), view_of(y), nr);
        } else {
            hipLaunchKernelGGL((k_swiglu_rows<uint16_t>), grid, dim3(kThreads), 0, s, view_of(g), view_of(u), view_of(y), nr);
        }
    }
    return check_launch("swiglu");
}

int launch_snake(const cbx_tensor* x, const cbx_tensor* a, const cbx_tensor* ai, cbx_tensor* y, DeviceState* st,
                 hipStream_t s) {
    (void)st;
    const bool inner = a->ne[0] == x->ne[0] && x->ne[0] > 1;
    const int64_t n = nelements(x);
    const int64_t C = inner ? x->ne[0] : x->ne[1];
    const bool flat = is_contiguous(x) && is_contiguous(y) && aligned(x->data, 16) && aligned(y->data, 16) &&
                      aligned(a->data, 16) && aligned(ai->data, 16) && x->ne[0] % 4 == 0 &&
                      n < (int64_t{1} << 32);
    if (flat) {
        const uint32_t n4 = static_cast<uint32_t>(n / 4);
        const uint32_t cmask = (C & (C - 1)) == 0 ? static_cast<uint32_t>(C - 1) : 0u;
        const uint32_t ne0_4 = static_cast<uint32_t>(x->ne[0] / 4);
        const dim3 grid(static_cast<unsigned>(cdiv(n4, kThreads)));
        const float* xp = static_cast<const float*>(x->data);
        float* yp = static_cast<float*>(y->data);
        const float* ap = static_cast<const float*>(a->data);
        const float* ip = static_cast<const float*>(ai->data);
        if (inner) hipLaunchKernelGGL((k_snake<true>), grid, dim3(kThreads), 0, s, xp, yp, ap, ip, n4, static_cast<uint32_t>(C), cmask, ne0_4);
        else hipLaunchKernelGGL((k_snake<false>), grid, dim3(kThreads), 0, s, xp, yp, ap, ip, n4, static_cast<uint32_t>(C), cmask, ne0_4);
    } else {
        const int64_t nr = nrows(x);
        const int64_t cpr = cdiv(x->ne[0], int64_t{kThreads} * 4);
        const int64_t total = nr * cpr;
        const dim3 grid(static_cast<unsigned>(std::min<int64_t>(total, int64_t{1} << 20)));
        if (inner) {
            hipLaunchKernelGGL((k_snake_rows<true>), grid, dim3(kThreads), 0, s, view_of(x), view_of(y),
                               static_cast<const float*>(a->data), static_cast<const float*>(ai->data), nr, cpr,
                               flat_rows(x), flat_rows(y));
        } else {
            hipLaunchKernelGGL((k_snake_rows<false>), grid, dim3(kThreads), 0, s, view_of(x), view_of(y),
                               static_cast<const float*>(a->data), static_cast<const float*>(ai->data), nr, cpr,
                               flat_rows(x), flat_rows(y));
        }
    }
    return check_launch("snake");
}

}  // namespace cbx
