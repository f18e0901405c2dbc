// k_group_norm.hip -- ggml_group_norm with the per-channel affine and an
// optional activation (Mish for the CFM blocks) fused: one read, one write.
//
// ggml's convention: channels are ne[2]; group g holds channels
// [g*cpg, min((g+1)*cpg, C)), cpg = ceil(C / n_groups), over all of ne[0] x
// ne[1], separately per ne[3] (batch).  Arithmetic as ggml-cpu:
//   mean = (float)(sum_f64 x / count); v = x - mean;
//   var = (float)(sum_f64 (v*v) / count); y = v * (1/sqrtf(var + eps)),
// then y*w[c], +b[c], activation -- each rounded to f32.
//
// One 1024-lane workgroup per (batch, group); the group (up to 64K
// elements) stays in registers between the two reductions and the store.
#include "cbx_device.h"

namespace cbx {
namespace {

constexpr int kThreads = 1024;

struct GnArgs {
    View x, y;
    const float* w;
    const float* b;
    int n_groups;
    int64_t cpg;
    float eps;
    int act;
    const uint16_t* tab;
};

// Byte offset of element e (0 <= e < count) of the group starting at channel c0.
__device__ __forceinline__ int64_t gn_offset(const View& t, int64_t e, int64_t c0, int64_t i3, int64_t* ch) {
    const int64_t per_ch = t.ne[0] * t.ne[1];
    const int64_t c = e / per_ch;
    const int64_t rem = e - c * per_ch;
    const int64_t i1 = rem / t.ne[0];
    const int64_t i0 = rem - i1 * t.ne[0];
    *ch = c0 + c;
    return i0 * 4 + i1 * t.nb[1] + (c0 + c) * t.nb[2] + i3 * t.nb[3];
}

template <int NV, bool ACT, bool VEC>
__global__ __launch_bounds__(kThreads) void k_group_norm(GnArgs a) {
    __shared__ double red[kThreads / WAVE];
    const int64_t C = a.x.ne[2];
    const int64_t g = blockIdx.x % a.n_groups;
    const int64_t i3 = blockIdx.x / a.n_groups;
    const int64_t c0 = g * a.cpg;
    const int64_t c1 = c0 + a.cpg < C ? c0 + a.cpg : C;
    if (c0 >= c1) return;   // uniform across the workgroup
    const int64_t count = a.x.ne[0] * a.x.ne[1] * (c1 - c0);

    // VEC: the group is one contiguous run of count floats (x and y), read
    // with unconditional 16-byte loads (clamped addresses) so all NV are in
    // flight together; per_ch floats per channel.
    const char* xg = a.x.data + c0 * a.x.nb[2] + i3 * a.x.nb[3];
    char* yg = a.y.data + c0 * a.y.nb[2] + i3 * a.y.nb[3];
    const uint32_t per_ch = static_cast<uint32_t>(a.x.ne[0] * a.x.ne[1]);
    float4 v[NV];
    int64_t ch[NV];
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t e = (threadIdx.x + static_cast<int64_t>(k) * blockDim.x) * 4;
        if constexpr (VEC) {
            v[k] = *reinterpret_cast<const float4*>(xg + 4 * (e < count ? e : 0));
        } else {
            if (e < count) {
                for (int q = 0; q < 4; q++) {
                    int64_t chq;
                    const int64_t oq = gn_offset(a.x, e + q, c0, i3, &chq);
                    set(v[k], q, e + q < count ? *reinterpret_cast<const float*>(a.x.data + oq) : 0.0f);
                }
            } else {
                v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t e = (threadIdx.x + static_cast<int64_t>(k) * blockDim.x) * 4;
        if constexpr (VEC) {
            if (e >= count) v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
            ch[k] = c0 + static_cast<uint32_t>(e < count ? e : 0) / per_ch;
        } else {
            ch[k] = 0;
        }
#pragma unroll
        for (int q = 0; q < 4; q++) s += static_cast<double>(get(v[k], q));
    }
    s = block_sum(s, red);
    const float mean = static_cast<float>(s / static_cast<double>(count));
    double s2 = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t e = (threadIdx.x + static_cast<int64_t>(k) * blockDim.x) * 4;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (e + q < count) {
                const float d = get(v[k], q) - mean;
                set(v[k], q, d);
                s2 += static_cast<double>(d * d);
            }
        }
    }
    s2 = block_sum(s2, red);
    const float var = static_cast<float>(s2 / static_cast<double>(count));
    const float scale = 1.0f / sqrtf(var + a.eps);

#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t e = (threadIdx.x + static_cast<int64_t>(k) * blockDim.x) * 4;
        if (e >= count) continue;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (e + q >= count) continue;   // scalar tail of the last vector
            int64_t c = ch[k];
            if constexpr (!VEC) gn_offset(a.y, e + q, c0, i3, &c);
            float t = get(v[k], q) * scale;
            if (a.w) t = t * a.w[c];
            if (a.b) t = t + a.b[c];
            if constexpr (ACT) t = apply_act(a.act, t, a.tab, 0.0f);
            set(o, q, t);
        }
        if constexpr (VEC) {
            *reinterpret_cast<float4*>(yg + 4 * e) = o;
        } else {
            for (int q = 0; q < 4; q++) {
                if (e + q < count) {
                    int64_t cy;
                    *reinterpret_cast<float*>(a.y.data + gn_offset(a.y, e + q, c0, i3, &cy)) = get(o, q);
                }
            }
        }
    }
}

// Groups larger than the register budget: three passes over global memory.
template <bool ACT>
__global__ __launch_bounds__(kThreads) void k_group_norm_loop(GnArgs a) {
    __shared__ double red[kThreads / WAVE];
    const int64_t C = a.x.ne[2];
    const int64_t g = blockIdx.x % a.n_groups;
    const int64_t i3 = blockIdx.x / a.n_groups;
    const int64_t c0 = g * a.cpg;
    const int64_t c1 = c0 + a.cpg < C ? c0 + a.cpg : C;
    if (c0 >= c1) return;
    const int64_t count = a.x.ne[0] * a.x.ne[1] * (c1 - c0);
    double s = 0.0;
    for (int64_t e = threadIdx.x; e < count; e += blockDim.x) {
        int64_t c;
        s += static_cast<double>(*reinterpret_cast<const float*>(a.x.data + gn_offset(a.x, e, c0, i3, &c)));
    }
    s = block_sum(s, red);
    const float mean = static_cast<float>(s / static_cast<double>(count));
    double s2 = 0.0;
    for (int64_t e = threadIdx.x; e < count; e += blockDim.x) {
        int64_t c;
        const float d = *reinterpret_cast<const float*>(a.x.data + gn_offset(a.x, e, c0, i3, &c)) - mean;
        s2 += static_cast<double>(d * d);
    }
    s2 = block_sum(s2, red);
    const float scale = 1.0f / sqrtf(static_cast<float>(s2 / static_cast<double>(count)) + a.eps);
    for (int64_t e = threadIdx.x; e < count; e += blockDim.x) {
        int64_t c;
        float t = *reinterpret_cast<const float*>(a.x.data + gn_offset(a.x, e, c0, i3, &c)) - mean;
        t = t * scale;
        if (a.w) t = t * a.w[c];
        if (a.b) t = t + a.b[c];
        if constexpr (ACT) t = apply_act(a.act, t, a.tab, 0.0f);
        *reinterpret_cast<float*>(a.y.data + gn_offset(a.y, e, c0, i3, &c)) = t;
    }
}

template <bool ACT, bool VEC>
void gn_nv(const GnArgs& a, int nv, dim3 grid, hipStream_t s) {
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_group_norm<1, ACT, VEC>), grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_group_norm<2, ACT, VEC>), grid, dim3(kThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_group_norm<4, ACT, VEC>), grid, dim3(kThreads), 0, s, a); break;
        case 8: hipLaunchKernelGGL((k_group_norm<8, ACT, VEC>), grid, dim3(kThreads), 0, s, a); break;
        case 16: hipLaunchKernelGGL((k_group_norm<16, ACT, VEC>), grid, dim3(kThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((k_group_norm_loop<ACT>), grid, dim3(kThreads), 0, s, a); break;
    }
}

}  // namespace

int launch_group_norm(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                      int act, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    GnArgs a;
    a.x = view_of(x);
    a.y = view_of(y);
    a.w = w ? static_cast<const float*>(w->data) : nullptr;
    a.b = b ? static_cast<const float*>(b->data) : nullptr;
    a.n_groups = n_groups;
    a.cpg = cdiv(x->ne[2], n_groups);
    a.eps = eps;
    a.act = act;
    a.tab = st->gelu_table;
    // VEC: every group is a contiguous run of floats (ne0, ne1 dense within a
    // channel, channels adjacent), 16-byte aligned, ne0 % 4 == 0.
    bool vec = x->ne[0] % 4 == 0;
    for (const cbx_tensor* t : {x, static_cast<const cbx_tensor*>(y)}) {
        const size_t row = 4 * static_cast<size_t>(t->ne[0]);
        if (t->ne[1] > 1 && t->nb[1] != row) vec = false;
        if (t->ne[2] > 1 && t->nb[2] != row * static_cast<size_t>(t->ne[1])) vec = false;
        if (reinterpret_cast<uintptr_t>(t->data) % 16 || t->nb[2] % 16 || t->nb[3] % 16) vec = false;
    }
    const int64_t count = x->ne[0] * x->ne[1] * std::min<int64_t>(a.cpg, x->ne[2]);
    const int64_t need = cdiv(count, int64_t{kThreads} * 4);
    const int nv = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : need <= 16 ? 16 : 0;
    const int64_t nblocks = int64_t{n_groups} * x->ne[3];
    if (nblocks > (int64_t{1} << 30)) return set_error(CBX_ERR_UNSUPPORTED, "group_norm: too many groups");
    const dim3 grid(static_cast<unsigned>(nblocks));
    const bool act_on = a.act != CBX_UNARY_NONE;
    if (act_on && vec) gn_nv<true, true>(a, nv, grid, s);
    else if (act_on) gn_nv<true, false>(a, nv, grid, s);
    else if (vec) gn_nv<false, true>(a, nv, grid, s);
    else gn_nv<false, false>(a, nv, grid, s);
    return check_launch("group_norm");
}

}  // namespace cbx
