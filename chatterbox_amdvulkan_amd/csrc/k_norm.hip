// k_norm.hip -- LayerNorm / RMSNorm over ne[0] with the affine multiply/add
// and an optional activation fused into the same pass: one HBM read of x,
// one write of y, per row.
//
// Arithmetic follows ggml-cpu exactly:
//   LN : mean = (float)(sum_f64 x) / n;  v = x - mean;
//        var = (float)(sum_f64 (v*v) / n);  y = v * (1/sqrtf(var + eps))
//   RMS: ms = (float)(sum_f64 (x*x) / n);   y = x * (1/sqrtf(ms + eps))
//   then y*w, then +b, each rounded to f32 (ggml_mul, ggml_add).
// The f64 sums use a fixed butterfly + per-wave order rather than ggml's
// sequential order; the f32 values derived from them agree unless an f64
// sum falls within ~2^-29 relative of an f32 rounding boundary.
//
// One workgroup per row; each lane keeps its share of the row in registers
// (NV 4-element vectors), so x is read from HBM once.  Rows longer than
// 8 * 4 * 256 = 8192 elements use a three-pass loop instead.
// x and y share one storage type (F32, or F16 with f32 arithmetic).
#include "cbx_device.h"

namespace cbx {
namespace {

constexpr int kMaxThreads = 256;

template <typename T, int NV, int KIND, bool ACT, bool VEC>
__global__ __launch_bounds__(kMaxThreads) void k_row_norm(View x, View y, const float* __restrict__ w,
                                                           const float* __restrict__ b, float eps, int act,
                                                           const uint16_t* __restrict__ tab, int64_t nr) {
    __shared__ double red[kMaxThreads / WAVE];
    const int64_t ne0 = x.ne[0];
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const int64_t i3 = r / (x.ne[2] * x.ne[1]);
        const int64_t i2 = (r - i3 * x.ne[2] * x.ne[1]) / x.ne[1];
        const int64_t i1 = r - i3 * x.ne[2] * x.ne[1] - i2 * x.ne[1];
        const char* xr = x.data + i1 * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];

        // element index of component e of vector k held by this lane
        auto idx = [&](int k, int e) -> int64_t {
            return VEC ? (threadIdx.x + static_cast<int64_t>(k) * blockDim.x) * 4 + e
                       : threadIdx.x + (static_cast<int64_t>(k) * 4 + e) * blockDim.x;
        };

        float4 v[NV];
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            if constexpr (VEC) {
                const int64_t j = idx(k, 0);
                v[k] = j < ne0 ? Elt<T>::load4(xr + j * Elt<T>::size) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int64_t j = idx(k, e);
                    set(v[k], e, j < ne0 ? Elt<T>::load1(xr + j * Elt<T>::size) : 0.0f);
                }
            }
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = get(v[k], e);
                if constexpr (KIND == NORM_LN) s += static_cast<double>(t);
                else s += static_cast<double>(t * t);
            }
        }
        s = block_sum(s, red);

        float scale;
        if constexpr (KIND == NORM_LN) {
            const float mean = static_cast<float>(s) / static_cast<float>(ne0);
            double s2 = 0.0;
#pragma unroll
            for (int k = 0; k < NV; k++) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    if (idx(k, e) < ne0) {
                        const float d = get(v[k], e) - mean;
                        set(v[k], e, d);
                        s2 += static_cast<double>(d * d);
                    }
                }
            }
            s2 = block_sum(s2, red);
            const float var = static_cast<float>(s2 / static_cast<double>(ne0));
            scale = 1.0f / sqrtf(var + eps);
        } else {
            const float ms = static_cast<float>(s / static_cast<double>(ne0));
            scale = 1.0f / sqrtf(ms + eps);
        }

#pragma unroll
        for (int k = 0; k < NV; k++) {
            float4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int64_t j = idx(k, e) < ne0 ? idx(k, e) : 0;
                float t = get(v[k], e) * scale;
                if (w) t = t * w[j];
                if (b) t = t + b[j];
                if constexpr (ACT) t = apply_act(act, t, tab, 0.0f);
                set(o, e, t);
            }
            if constexpr (VEC) {
                const int64_t j = idx(k, 0);
                if (j < ne0) Elt<T>::store4(yr + j * Elt<T>::size, o);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int64_t j = idx(k, e);
                    if (j < ne0) Elt<T>::store1(yr + j * Elt<T>::size, get(o, e));
                }
            }
        }
    }
}

// Long rows: three passes over global memory (one row stays in L2).
template <typename T, int KIND, bool ACT>
__global__ __launch_bounds__(kMaxThreads) void k_row_norm_loop(View x, View y, const float* __restrict__ w,
                                                                const float* __restrict__ b, float eps, int act,
                                                                const uint16_t* __restrict__ tab, int64_t nr) {
    __shared__ double red[kMaxThreads / WAVE];
    const int64_t ne0 = x.ne[0];
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const int64_t i3 = r / (x.ne[2] * x.ne[1]);
        const int64_t i2 = (r - i3 * x.ne[2] * x.ne[1]) / x.ne[1];
        const int64_t i1 = r - i3 * x.ne[2] * x.ne[1] - i2 * x.ne[1];
        const char* xr = x.data + i1 * x.nb[1] + i2 * x.nb[2] + i3 * x.nb[3];
        char* yr = y.data + i1 * y.nb[1] + i2 * y.nb[2] + i3 * y.nb[3];
        double s = 0.0;
        for (int64_t j = threadIdx.x; j < ne0; j += blockDim.x) {
            const float t = Elt<T>::load1(xr + j * Elt<T>::size);
            if constexpr (KIND == NORM_LN) s += static_cast<double>(t);
            else s += static_cast<double>(t * t);
        }
        s = block_sum(s, red);
        float scale, mean = 0.0f;
        if constexpr (KIND == NORM_LN) {
            mean = static_cast<float>(s) / static_cast<float>(ne0);
            double s2 = 0.0;
            for (int64_t j = threadIdx.x; j < ne0; j += blockDim.x) {
                const float d = Elt<T>::load1(xr + j * Elt<T>::size) - mean;
                s2 += static_cast<double>(d * d);
            }
            s2 = block_sum(s2, red);
            scale = 1.0f / sqrtf(static_cast<float>(s2 / static_cast<double>(ne0)) + eps);
        } else {
            scale = 1.0f / sqrtf(static_cast<float>(s / static_cast<double>(ne0)) + eps);
        }
        for (int64_t j = threadIdx.x; j < ne0; j += blockDim.x) {
            float t = Elt<T>::load1(xr + j * Elt<T>::size);
            if constexpr (KIND == NORM_LN) t = t - mean;
            t = t * scale;
            if (w) t = t * w[j];
            if (b) t = t + b[j];
            if constexpr (ACT) t = apply_act(act, t, tab, 0.0f);
            Elt<T>::store1(yr + j * Elt<T>::size, t);
        }
    }
}

struct NormLaunch {
    View x, y;
    const float* w;
    const float* b;
    float eps;
    int act;
    const uint16_t* tab;
    int64_t nr;
    dim3 grid, block;
    hipStream_t s;
};

template <typename T, int KIND, bool ACT, bool VEC>
void go_nv(const NormLaunch& L, int nv) {
#define CBX_NORM_CASE(N)                                                                                         \
    case N:                                                                                                     \
        hipLaunchKernelGGL((k_row_norm<T, N, KIND, ACT, VEC>), L.grid, L.block, 0, L.s, L.x, L.y, L.w, L.b,     \
                           L.eps, L.act, L.tab, L.nr);                                                          \
        break;
    switch (nv) {
        CBX_NORM_CASE(1)
        CBX_NORM_CASE(2)
        CBX_NORM_CASE(4)
        CBX_NORM_CASE(8)
        default:
            hipLaunchKernelGGL((k_row_norm_loop<T, KIND, ACT>), L.grid, L.block, 0, L.s, L.x, L.y, L.w, L.b, L.eps,
                               L.act, L.tab, L.nr);
    }
#undef CBX_NORM_CASE
}

template <typename T, int KIND>
void go(const NormLaunch& L, int nv, bool vec) {
    const bool act = L.act != CBX_UNARY_NONE;
    if (act) {
        if (vec) go_nv<T, KIND, true, true>(L, nv);
        else go_nv<T, KIND, true, false>(L, nv);
    } else {
        if (vec) go_nv<T, KIND, false, true>(L, nv);
        else go_nv<T, KIND, false, false>(L, nv);
    }
}

bool rows_aligned(const cbx_tensor* t, size_t a) {
    if (reinterpret_cast<uintptr_t>(t->data) % a) return false;
    for (int i = 1; i < 4; i++) if (t->nb[i] % a) return false;
    return true;
}

}  // namespace

int launch_row_norm(int kind, const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int act,
                    cbx_tensor* y, DeviceState* st, hipStream_t s) {
    if (x->type != y->type) return set_error(CBX_ERR_UNSUPPORTED, "norm: x and y must have the same type");
    const int64_t ne0 = x->ne[0];
    const int64_t nr = nrows(x);
    const size_t a = x->type == CBX_TYPE_F32 ? 16 : 8;
    const bool vec = ne0 % 4 == 0 && rows_aligned(x, a) && rows_aligned(y, a);
    const int64_t quads = cdiv(ne0, 4);
    const int threads = static_cast<int>(std::min<int64_t>(kMaxThreads, std::max<int64_t>(WAVE, cdiv(quads, WAVE) * WAVE)));
    const int64_t need = cdiv(quads, threads);
    const int nv = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 0;
    NormLaunch L;
    L.x = view_of(x);
    L.y = view_of(y);
    L.w = w ? static_cast<const float*>(w->data) : nullptr;
    L.b = b ? static_cast<const float*>(b->data) : nullptr;
    L.eps = eps;
    L.act = act;
    L.tab = st->gelu_table;
    L.nr = nr;
    L.grid = dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20)));
    L.block = dim3(threads);
    L.s = s;
    if (x->type == CBX_TYPE_F32) {
        if (kind == NORM_LN) go<float, NORM_LN>(L, nv, vec);
        else go<float, NORM_RMS>(L, nv, vec);
    } else {
        if (kind == NORM_LN) go<uint16_t, NORM_LN>(L, nv, vec);
        else go<uint16_t, NORM_RMS>(L, nv, vec);
    }
    return check_launch(kind == NORM_LN ? "layer_norm" : "rms_norm");
}

}  // namespace cbx
