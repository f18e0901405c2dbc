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
// Groups of up to 64K elements stay in registers between the two
// reductions; larger ones take three passes over memory.
#include <algorithm>

#include "cbx_device.h"

namespace cbx {
namespace {

constexpr int kThreads = 1024;
constexpr uint32_t kXcds = 8;   // gfx950: workgroups go to XCD (index % 8)

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

// Strided layouts: each lane gathers its 4 elements one by one.
template <int NV, bool ACT>
__global__ __launch_bounds__(kThreads) void k_group_norm(GnArgs a) {
    __shared__ double red[kThreads / WAVE];
    const int64_t C = a.x.ne[2];
    const int64_t g = blockIdx.x % a.n_groups;
    const int64_t i3 = blockIdx.x / a.n_groups;
    const int64_t c0 = g * a.cpg;
    const int64_t c1 = c0 + a.cpg < C ? c0 + a.cpg : C;
    if (c0 >= c1) return;   // uniform across the workgroup
    const int64_t count = a.x.ne[0] * a.x.ne[1] * (c1 - c0);

    float4 v[NV];
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t e = (threadIdx.x + static_cast<int64_t>(k) * blockDim.x) * 4;
        v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (e < count) {
            for (int q = 0; q < 4; q++) {
                int64_t chq;
                const int64_t oq = gn_offset(a.x, e + q, c0, i3, &chq);
                set(v[k], q, e + q < count ? *reinterpret_cast<const float*>(a.x.data + oq) : 0.0f);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NV; k++) {
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
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (e + q >= count) continue;
            int64_t c;
            const int64_t oy = gn_offset(a.y, e + q, c0, i3, &c);
            float t = get(v[k], q) * scale;
            if (a.w) t = t * a.w[c];
            if (a.b) t = t + a.b[c];
            if constexpr (ACT) t = apply_act(a.act, t, a.tab, 0.0f);
            *reinterpret_cast<float*>(a.y.data + oy) = t;
        }
    }
}

// y of 4 elements of channel c, given d = x - mean.
template <bool ACT>
__device__ __forceinline__ float4 gn_apply4(const GnArgs& a, float4 d, float scale, int64_t c) {
    float4 o;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float t = get(d, q) * scale;
        if (a.w) t = t * a.w[c];
        if (a.b) t = t + a.b[c];
        if constexpr (ACT) t = apply_act(a.act, t, a.tab, 0.0f);
        set(o, q, t);
    }
    return o;
}

// f64 sum of a thread's NV partials (each the sum of one float4's four
// terms) as a tree: log-depth instead of a chain of 4*NV dependent adds.
template <int NV>
__device__ __forceinline__ double thread_tree_sum(double (&p)[NV]) {
#pragma unroll
    for (int w = 1; w < NV; w *= 2) {
#pragma unroll
        for (int i = 0; i + w < NV; i += 2 * w) p[i] += p[i + w];
    }
    return p[0];
}

// Sum over the kThreads threads: each wave's total (DPP butterfly), then
// wave 0 adds the kThreads/64 totals with the same butterfly and leaves the
// result in scratch[slot] for everyone.  Fixed order: every workgroup that
// reduces the same values gets the same bits.  Two barriers; a second call
// with another slot needs none before it.
__device__ __forceinline__ double block_sum_tree(double v, double* scratch, int slot) {
    constexpr int NW = kThreads / WAVE;
    static_assert(NW <= 16, "one DPP row of wave totals");
    v = wave_sum(v);
    const int lane = threadIdx.x % WAVE, wid = threadIdx.x / WAVE;
    if (lane == 0) scratch[wid] = v;
    __syncthreads();
    if (wid == 0) {
        double t = lane < NW ? scratch[lane] : 0.0;
        t += dpp_f64<0xB1>(t);
        t += dpp_f64<0x4E>(t);
        t += dpp_f64<0x141>(t);
        t += dpp_f64<0x140>(t);
        if (lane == 0) scratch[slot] = t;
    }
    __syncthreads();
    return scratch[slot];
}

// Contiguous groups (ne0 % 4 == 0, ne0 x ne1 dense per channel, channels
// adjacent, 16-byte aligned), split over n_chunks workgroups per group so a
// few large groups still fill the chip.  Every workgroup of a group reads
// the whole group into registers and computes the same statistics (same
// lanes, same order: bit-identical mean and scale), then writes only its
// chunk, from the registers that hold it.  Workgroups are dealt to the 8
// XCDs round-robin by index, so the chunks of one group are given indices
// that land on one XCD: its L2 serves the repeated reads of the group and
// HBM sees it once.
template <int NV, bool ACT>
__global__ __launch_bounds__(kThreads) void k_group_norm_vec(GnArgs a, uint32_t n_chunks, uint32_t n_gi) {
    __shared__ double red[kThreads / WAVE + 2];
    const uint32_t b = blockIdx.x;
    const uint32_t j = b / kXcds;
    const uint32_t m = j / n_chunks;
    const uint32_t ci = j - m * n_chunks;
    const uint32_t gi = b % kXcds + kXcds * m;
    const int64_t C = a.x.ne[2];
    int64_t g = gi % a.n_groups;
    int64_t i3 = gi / a.n_groups;
    int64_t c0 = g * a.cpg;
    // a workgroup past the last group, or of an empty group (past C), reads
    // group 0 and stores nothing: no early exit stands before the loads
    const bool live = gi < n_gi && c0 < C;
    if (!live) g = i3 = c0 = 0;
    const int64_t c1 = c0 + a.cpg < C ? c0 + a.cpg : C;
    const int64_t count = a.x.ne[0] * a.x.ne[1] * (c1 - c0);
    const char* xg = a.x.data + c0 * a.x.nb[2] + i3 * a.x.nb[3];
    char* yg = a.y.data + c0 * a.y.nb[2] + i3 * a.y.nb[3];
    const uint32_t per_ch = static_cast<uint32_t>(a.x.ne[0] * a.x.ne[1]);

    // this workgroup's chunk: float4 indices [q0, q1) of the group
    const int64_t n4 = count / 4;
    const int64_t per = (n4 + n_chunks - 1) / n_chunks;
    const int64_t q0 = ci * per;
    const int64_t q1 = q0 + per < n4 ? q0 + per : n4;
    // unconditional 16-byte loads (clamped addresses) keep all NV in flight;
    // up to NV = 8 the affine values of the channel of each vector this
    // workgroup stores are loaded with them (a vector lies in one channel:
    // ne0 % 4 == 0), past that (128 registers a thread) when it is stored
    constexpr bool kEarly = NV <= 8;
    float4 v[NV];
    float wv[kEarly ? NV : 1], bv[kEarly ? NV : 1];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t qi = threadIdx.x + static_cast<int64_t>(k) * kThreads;
        v[k] = *reinterpret_cast<const float4*>(xg + 16 * (qi < n4 ? qi : 0));
        if constexpr (kEarly) {
            wv[k] = 1.0f;
            bv[k] = 0.0f;
            if (qi >= q0 && qi < q1) {   // only the vectors this workgroup stores
                const int64_t c = c0 + static_cast<uint32_t>(4 * qi) / per_ch;
                if (a.w) wv[k] = a.w[c];
                if (a.b) bv[k] = a.b[c];
            }
        }
    }
    double p[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t qi = threadIdx.x + static_cast<int64_t>(k) * kThreads;
        if (qi >= n4) v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        p[k] = (static_cast<double>(v[k].x) + static_cast<double>(v[k].y)) +
               (static_cast<double>(v[k].z) + static_cast<double>(v[k].w));
    }
    const double s = block_sum_tree(thread_tree_sum<NV>(p), red, kThreads / WAVE);
    const float mean = static_cast<float>(s / static_cast<double>(count));
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t qi = threadIdx.x + static_cast<int64_t>(k) * kThreads;
        const bool in = qi < n4;   // count % 4 == 0: a vector is all in or all out
#pragma unroll
        for (int e = 0; e < 4; e++) set(v[k], e, in ? get(v[k], e) - mean : 0.0f);
        p[k] = (static_cast<double>(v[k].x * v[k].x) + static_cast<double>(v[k].y * v[k].y)) +
               (static_cast<double>(v[k].z * v[k].z) + static_cast<double>(v[k].w * v[k].w));
    }
    const double s2 = block_sum_tree(thread_tree_sum<NV>(p), red, kThreads / WAVE + 1);
    const float var = static_cast<float>(s2 / static_cast<double>(count));
    const float scale = 1.0f / sqrtf(var + a.eps);
    if (!live) return;   // uniform across the workgroup
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t qi = threadIdx.x + static_cast<int64_t>(k) * kThreads;
        if (qi < q0 || qi >= q1) continue;
        const int64_t c = c0 + static_cast<uint32_t>(4 * qi) / per_ch;
        const float wk = kEarly ? wv[kEarly ? k : 0] : (a.w ? a.w[c] : 1.0f);
        const float bk = kEarly ? bv[kEarly ? k : 0] : (a.b ? a.b[c] : 0.0f);
        float4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float t = get(v[k], e) * scale;
            if (a.w) t = t * wk;
            if (a.b) t = t + bk;
            if constexpr (ACT) t = apply_act(a.act, t, a.tab, 0.0f);
            set(o, e, t);
        }
        if (n_chunks == 1) *reinterpret_cast<float4*>(yg + 16 * qi) = o;
        else Stream<float>::store4(yg + 16 * qi, o);
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

template <bool ACT>
void gn_nv(const GnArgs& a, int nv, dim3 grid, hipStream_t s) {
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_group_norm<1, ACT>), grid, dim3(kThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_group_norm<2, ACT>), grid, dim3(kThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_group_norm<4, ACT>), grid, dim3(kThreads), 0, s, a); break;
        case 8: hipLaunchKernelGGL((k_group_norm<8, ACT>), grid, dim3(kThreads), 0, s, a); break;
        case 16: hipLaunchKernelGGL((k_group_norm<16, ACT>), grid, dim3(kThreads), 0, s, a); break;
        default: hipLaunchKernelGGL((k_group_norm_loop<ACT>), grid, dim3(kThreads), 0, s, a); break;
    }
}

template <bool ACT>
void gn_vec(const GnArgs& a, int nv, uint32_t n_chunks, uint32_t n_gi, hipStream_t s) {
    const dim3 grid(kXcds * ((n_gi + kXcds - 1) / kXcds) * n_chunks);
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_group_norm_vec<1, ACT>), grid, dim3(kThreads), 0, s, a, n_chunks, n_gi); break;
        case 2: hipLaunchKernelGGL((k_group_norm_vec<2, ACT>), grid, dim3(kThreads), 0, s, a, n_chunks, n_gi); break;
        case 4: hipLaunchKernelGGL((k_group_norm_vec<4, ACT>), grid, dim3(kThreads), 0, s, a, n_chunks, n_gi); break;
        case 8: hipLaunchKernelGGL((k_group_norm_vec<8, ACT>), grid, dim3(kThreads), 0, s, a, n_chunks, n_gi); break;
        default: hipLaunchKernelGGL((k_group_norm_vec<16, ACT>), grid, dim3(kThreads), 0, s, a, n_chunks, n_gi); break;
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
    const bool act_on = a.act != CBX_UNARY_NONE;
    if (vec && nv != 0) {
        // chunks per group: about two workgroups per CU in all, each chunk
        // at least 1024 elements, at most 16 (each chunk re-reads the
        // group).  In place, one chunk: a group is read whole before any of
        // it is written only when one workgroup owns it.
        const int64_t want = cdiv(int64_t{2} * st->n_cu, nblocks);
        int64_t n_chunks = std::max<int64_t>(1, std::min<int64_t>({want, cdiv(count, 1024), int64_t{16}}));
        const uintptr_t xl = reinterpret_cast<uintptr_t>(x->data), yl = reinterpret_cast<uintptr_t>(y->data);
        const size_t span = static_cast<size_t>(x->ne[3]) * x->nb[3];
        if (xl < yl + span && yl < xl + span) n_chunks = 1;
        if (act_on) gn_vec<true>(a, nv, static_cast<uint32_t>(n_chunks), static_cast<uint32_t>(nblocks), s);
        else gn_vec<false>(a, nv, static_cast<uint32_t>(n_chunks), static_cast<uint32_t>(nblocks), s);
        return check_launch("group_norm");
    }
    const dim3 grid(static_cast<unsigned>(nblocks));
    if (act_on) gn_nv<true>(a, nv, grid, s);
    else gn_nv<false>(a, nv, grid, s);
    return check_launch("group_norm");
}

}  // namespace cbx
