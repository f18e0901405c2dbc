// k_eltwise.hip -- element-wise activations: the ggml unary ops, leaky_relu,
// swiglu (silu(g) * u) and the fused Snake chain.
//
// Contiguous tensors take the streaming path: a grid-stride loop in which
// each lane keeps U independent 4-element vectors in flight (16-byte loads
// and stores for f32), so a wave moves U KiB per iteration.  Non-contiguous
// tensors (rows with nb[0] == element size) take a row loop.
//
// Each op body is ggml-cpu's scalar expression, compiled without FMA
// contraction; GELU uses the fp16 table uploaded by cbx_init, so it is
// exact.  Transcendentals (expf, logf, tanhf, erff, sinf) are the device's
// libm, not glibc's, and may differ from the CPU result in the last bit.
#include "cbx_device.h"

namespace cbx {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

template <int OP>
__device__ __forceinline__ float unary_op(float x, const uint16_t* __restrict__ tab, float param) {
    if constexpr (OP == CBX_UNARY_GELU) return act_gelu_tab(tab, x);
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
template <typename T, int OP>
__device__ __forceinline__ uint16_t unary_f16_code(uint16_t h, const uint16_t* __restrict__ tab, float param) {
    if constexpr (OP == CBX_UNARY_GELU) return tab[h];
    else return f2h(unary_op<OP>(h2f(h), tab, param));
}

template <typename T, int OP>
__global__ __launch_bounds__(kThreads) void k_unary_flat(const char* __restrict__ x, char* __restrict__ y, int64_t n,
                                                         float param, const uint16_t* __restrict__ tab) {
    const int64_t n4 = n / 4;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x; base < n4; base += step) {
        constexpr bool kF16Table = std::is_same<T, uint16_t>::value && OP == CBX_UNARY_GELU;
        float4 v[kUnroll];
        uint2 raw[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t i = base + u * kThreads;
            if (i < n4) {
                if constexpr (kF16Table) raw[u] = *reinterpret_cast<const uint2*>(x + i * 8);
                else v[u] = Elt<T>::load4(x + i * 4 * Elt<T>::size);
            }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int64_t i = base + u * kThreads;
            if (i < n4) {
                if constexpr (kF16Table) {
                    uint2 o;
                    o.x = tab[raw[u].x & 0xffffu] | (static_cast<uint32_t>(tab[raw[u].x >> 16]) << 16);
                    o.y = tab[raw[u].y & 0xffffu] | (static_cast<uint32_t>(tab[raw[u].y >> 16]) << 16);
                    *reinterpret_cast<uint2*>(y + i * 8) = o;
                } else {
                    float4 o;
                    o.x = unary_op<OP>(v[u].x, tab, param);
                    o.y = unary_op<OP>(v[u].y, tab, param);
                    o.z = unary_op<OP>(v[u].z, tab, param);
                    o.w = unary_op<OP>(v[u].w, tab, param);
                    Elt<T>::store4(y + i * 4 * Elt<T>::size, o);
                }
            }
        }
    }
    if (blockIdx.x == 0) {
        for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += kThreads) {
            if constexpr (std::is_same<T, uint16_t>::value) {
                const uint16_t h = *reinterpret_cast<const uint16_t*>(x + i * 2);
                *reinterpret_cast<uint16_t*>(y + i * 2) = unary_f16_code<T, OP>(h, tab, param);
            } else {
                Elt<T>::store1(y + i * 4, unary_op<OP>(Elt<T>::load1(x + i * 4), tab, param));
            }
        }
    }
}

template <typename T, int OP>
__global__ __launch_bounds__(kThreads) void k_unary_rows(View x, View y, int64_t nr, float param,
                                                         const uint16_t* __restrict__ tab) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const int64_t i3 = r / (x.ne[2] * x.ne[1]);
        const int64_t i2 = (r - i3 * x.ne[2] * x.ne[1]) / x.ne[1];
        const int64_t i1 = r - i3 * x.ne[2] * x.ne[1] - i2 * x.ne[1];
        const char* xr = x.data + i1 * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
        for (int64_t j = threadIdx.x; j < x.ne[0]; j += kThreads) {
            if constexpr (std::is_same<T, uint16_t>::value) {
                const uint16_t h = *reinterpret_cast<const uint16_t*>(xr + j * 2);
                *reinterpret_cast<uint16_t*>(yr + j * 2) = unary_f16_code<T, OP>(h, tab, param);
            } else {
                Elt<T>::store1(yr + j * 4, unary_op<OP>(Elt<T>::load1(xr + j * 4), tab, param));
            }
        }
    }
}

// ---- swiglu -------------------------------------------------------------------

template <typename T>
__global__ __launch_bounds__(kThreads) void k_swiglu_flat(const char* __restrict__ g, const char* __restrict__ u,
                                                          char* __restrict__ y, int64_t n) {
    const int64_t n4 = n / 4;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
    for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x; base < n4; base += step) {
        float4 vg[kUnroll], vu[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const int64_t i = base + k * kThreads;
            if (i < n4) {
                vg[k] = Elt<T>::load4(g + i * 4 * Elt<T>::size);
                vu[k] = Elt<T>::load4(u + i * 4 * Elt<T>::size);
            }
        }
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const int64_t i = base + k * kThreads;
            if (i < n4) {
                float4 o;
                o.x = act_silu(vg[k].x) * vu[k].x;
                o.y = act_silu(vg[k].y) * vu[k].y;
                o.z = act_silu(vg[k].z) * vu[k].z;
                o.w = act_silu(vg[k].w) * vu[k].w;
                Elt<T>::store4(y + i * 4 * Elt<T>::size, o);
            }
        }
    }
    if (blockIdx.x == 0) {
        for (int64_t i = n4 * 4 + threadIdx.x; i < n; i += kThreads) {
            const float gv = Elt<T>::load1(g + i * Elt<T>::size), uv = Elt<T>::load1(u + i * Elt<T>::size);
            Elt<T>::store1(y + i * Elt<T>::size, act_silu(gv) * uv);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kThreads) void k_swiglu_rows(View g, View u, View y, int64_t nr) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const int64_t i3 = r / (g.ne[2] * g.ne[1]);
        const int64_t i2 = (r - i3 * g.ne[2] * g.ne[1]) / g.ne[1];
        const int64_t i1 = r - i3 * g.ne[2] * g.ne[1] - i2 * g.ne[1];
        const char* gr = g.data + i1 * g.nb[1] + i2 * g.nb[2] + i3 * g.nb[3];
        const char* ur = u.data + i1 * u.nb[1] + i2 * u.nb[2] + i3 * u.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
        for (int64_t j = threadIdx.x; j < g.ne[0]; j += kThreads) {
            const float gv = Elt<T>::load1(gr + j * Elt<T>::size), uv = Elt<T>::load1(ur + j * Elt<T>::size);
            Elt<T>::store1(yr + j * Elt<T>::size, act_silu(gv) * uv);
        }
    }
}

// ---- snake --------------------------------------------------------------------
// y = x + sin(x*a)^2 * ainv, each step rounded to f32 as the five ggml ops
// of snake() (mul, sin, sqr, mul, add) round it.

__device__ __forceinline__ float snake1(float xv, float a, float ai) {
    const float xa = xv * a;
    const float sn = sinf(xa);
    const float s2 = sn * sn;
    const float m = s2 * ai;
    return xv + m;
}

// Channel innermost, contiguous x/y and C % 4 == 0: the channel of a vector
// advances by a fixed amount per step, tracked without division.
__global__ __launch_bounds__(kThreads) void k_snake_inner(const float* __restrict__ x, float* __restrict__ y,
                                                          const float* __restrict__ a, const float* __restrict__ ai,
                                                          int64_t n, int64_t C, int64_t c_step, int64_t c_lane) {
    const int64_t n4 = n / 4;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
    int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x;
    int64_t cb = (base * 4) % C;
    for (; base < n4; base += step) {
        float4 v[kUnroll];
        int64_t cc[kUnroll];
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const int64_t i = base + k * kThreads;
            int64_t c = cb + k * c_lane;
            while (c >= C) c -= C;
            cc[k] = c;
            if (i < n4) v[k] = *reinterpret_cast<const float4*>(x + i * 4);
        }
#pragma unroll
        for (int k = 0; k < kUnroll; k++) {
            const int64_t i = base + k * kThreads;
            if (i < n4) {
                const float4 av = *reinterpret_cast<const float4*>(a + cc[k]);
                const float4 iv = *reinterpret_cast<const float4*>(ai + cc[k]);
                float4 o;
                o.x = snake1(v[k].x, av.x, iv.x);
                o.y = snake1(v[k].y, av.y, iv.y);
                o.z = snake1(v[k].z, av.z, iv.z);
                o.w = snake1(v[k].w, av.w, iv.w);
                *reinterpret_cast<float4*>(y + i * 4) = o;
            }
        }
        cb += c_step;
        while (cb >= C) cb -= C;
    }
}

// General rows: alpha either per element of ne[0] (inner) or per row i1 (outer).
template <bool INNER>
__global__ __launch_bounds__(kThreads) void k_snake_rows(View x, View y, const float* __restrict__ a,
                                                         const float* __restrict__ ai, int64_t nr,
                                                         int64_t chunks_per_row) {
    const int64_t ne0 = x.ne[0];
    const int64_t total = nr * chunks_per_row;
    for (int64_t bidx = blockIdx.x; bidx < total; bidx += gridDim.x) {
        const int64_t r = bidx / chunks_per_row;
        const int64_t chunk = bidx - r * chunks_per_row;
        const int64_t i3 = r / (x.ne[2] * x.ne[1]);
        const int64_t i2 = (r - i3 * x.ne[2] * x.ne[1]) / x.ne[1];
        const int64_t i1 = r - i3 * x.ne[2] * x.ne[1] - i2 * x.ne[1];
        const float* xr = reinterpret_cast<const float*>(x.data + i1 * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3]);
        float* yr = reinterpret_cast<float*>(y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3]);
        const float ar = INNER ? 0.0f : a[i1];
        const float ir = INNER ? 0.0f : ai[i1];
        const int64_t j0 = chunk * kThreads * kUnroll;
        const int64_t j1 = j0 + kThreads * kUnroll < ne0 ? j0 + kThreads * kUnroll : ne0;
        for (int64_t j = j0 + threadIdx.x; j < j1; j += kThreads) {
            yr[j] = INNER ? snake1(xr[j], a[j], ai[j]) : snake1(xr[j], ar, ir);
        }
    }
}

// ---- launch helpers -------------------------------------------------------------

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int64_t flat_blocks(int64_t n4, const DeviceState* st) {
    return std::max<int64_t>(1, std::min<int64_t>(cdiv(n4, int64_t{kThreads} * kUnroll), int64_t{st->n_cu} * 16));
}

template <typename T, int OP>
void unary_go(const cbx_tensor* x, cbx_tensor* y, float param, DeviceState* st, hipStream_t s, bool flat) {
    if (flat) {
        const int64_t n = nelements(x);
        hipLaunchKernelGGL((k_unary_flat<T, OP>), dim3(flat_blocks(n / 4, st)), dim3(kThreads), 0, s,
                           static_cast<const char*>(x->data), static_cast<char*>(y->data), n, param, st->gelu_table);
    } else {
        const int64_t nr = nrows(x);
        hipLaunchKernelGGL((k_unary_rows<T, OP>), dim3(std::min<int64_t>(nr, int64_t{1} << 20)), dim3(kThreads), 0,
                           s, view_of(x), view_of(y), nr, param, st->gelu_table);
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

}  // namespace

int launch_unary(int op, float param, const cbx_tensor* x, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    const size_t a = x->type == CBX_TYPE_F32 ? 16 : 8;
    const bool flat = is_contiguous(x) && is_contiguous(y) && aligned(x->data, a) && aligned(y->data, a);
    if (x->type == CBX_TYPE_F32) unary_dispatch<float>(op, x, y, param, st, s, flat);
    else unary_dispatch<uint16_t>(op, x, y, param, st, s, flat);
    return check_launch("unary");
}

int launch_swiglu(const cbx_tensor* g, const cbx_tensor* u, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    const size_t a = g->type == CBX_TYPE_F32 ? 16 : 8;
    const bool flat = is_contiguous(g) && is_contiguous(u) && is_contiguous(y) && aligned(g->data, a) &&
                      aligned(u->data, a) && aligned(y->data, a);
    const int64_t n = nelements(y);
    if (flat) {
        const dim3 grid(static_cast<unsigned>(flat_blocks(n / 4, st)));
        if (g->type == CBX_TYPE_F32) {
            hipLaunchKernelGGL((k_swiglu_flat<float>), grid, dim3(kThreads), 0, s, static_cast<const char*>(g->data),
                               static_cast<const char*>(u->data), static_cast<char*>(y->data), n);
        } else {
            hipLaunchKernelGGL((k_swiglu_flat<uint16_t>), grid, dim3(kThreads), 0, s,
                               static_cast<const char*>(g->data), static_cast<const char*>(u->data),
                               static_cast<char*>(y->data), n);
        }
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
    const bool inner = a->ne[0] == x->ne[0] && x->ne[0] > 1;
    const int64_t n = nelements(x);
    const int64_t C = x->ne[0];
    const bool flat = inner && C % 4 == 0 && is_contiguous(x) && is_contiguous(y) && aligned(x->data, 16) &&
                      aligned(y->data, 16) && aligned(a->data, 16) && aligned(ai->data, 16);
    if (flat) {
        const int64_t blocks = flat_blocks(n / 4, st);
        const int64_t c_step = (blocks * kThreads * kUnroll * 4) % C;
        const int64_t c_lane = (int64_t{kThreads} * 4) % C;
        hipLaunchKernelGGL(k_snake_inner, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, s,
                           static_cast<const float*>(x->data), static_cast<float*>(y->data),
                           static_cast<const float*>(a->data), static_cast<const float*>(ai->data), n, C, c_step,
                           c_lane);
    } else {
        const int64_t nr = nrows(x);
        const int64_t cpr = cdiv(x->ne[0], int64_t{kThreads} * kUnroll);
        const int64_t total = nr * cpr;
        const dim3 grid(static_cast<unsigned>(std::min<int64_t>(total, int64_t{1} << 20)));
        if (inner) {
            hipLaunchKernelGGL((k_snake_rows<true>), grid, dim3(kThreads), 0, s, view_of(x), view_of(y),
                               static_cast<const float*>(a->data), static_cast<const float*>(ai->data), nr, cpr);
        } else {
            hipLaunchKernelGGL((k_snake_rows<false>), grid, dim3(kThreads), 0, s, view_of(x), view_of(y),
                               static_cast<const float*>(a->data), static_cast<const float*>(ai->data), nr, cpr);
        }
    }
    return check_launch("snake");
}

}  // namespace cbx
