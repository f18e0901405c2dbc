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
#include <string>

#include "cbx_gnsplit.h"

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

// Sum over the kThreads threads: each wave's total (DPP butterfly), then
// wave 0 adds the kThreads/64 totals with the same butterfly and leaves the
// result in lds[slot] for everyone.  Fixed order: every workgroup that
// reduces the same values gets the same bits.  Two barriers; a second call
// with another slot needs none before it.
template <int THREADS = kThreads>
__device__ __forceinline__ double block_sum_tree(double v, double* lds, int slot) {
    constexpr int NW = THREADS / WAVE;
    static_assert(NW <= 16, "one DPP row of wave totals");
    v = wave_sum(v);
    const int lane = threadIdx.x % WAVE, wid = threadIdx.x / WAVE;
    if (lane == 0) lds[wid] = v;
    __syncthreads();
    if (wid == 0) {
        double t = lane < NW ? lds[lane] : 0.0;
        t += dpp_f64<0xB1>(t);
        t += dpp_f64<0x4E>(t);
        t += dpp_f64<0x141>(t);
        t += dpp_f64<0x140>(t);
        if (lane == 0) lds[slot] = t;
    }
    __syncthreads();
    return lds[slot];
}

// The same sum with one barrier: each wave's total (DPP butterfly) to LDS,
// then every thread adds the wave totals in index order (the same bits in
// every thread and every workgroup that reduces the same values).  Calls
// alternate between two LDS areas by the parity of `slot`; a call may reuse
// an area once a barrier has passed since its last reads (every caller
// here has one in between).
template <int THREADS>
__device__ __forceinline__ double block_sum_1b(double v, double* lds, int slot) {
    constexpr int NW = THREADS / WAVE;
    v = wave_sum(v);
    double* sc = lds + NW * (slot & 1);
    if (threadIdx.x % WAVE == 0) sc[threadIdx.x / WAVE] = v;
    __syncthreads();
    double t = sc[0];
#pragma unroll
    for (int i = 1; i < NW; i++) t += sc[i];
    return t;
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
    __shared__ double red[2 * (kThreads / WAVE)];
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
    const double s = block_sum_1b<kThreads>(thread_tree_sum<NV>(p), red, 0);
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
    const double s2 = block_sum_1b<kThreads>(thread_tree_sum<NV>(p), red, 1);
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
        float4 o[1];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float t = get(v[k], e) * scale;
            if (a.w) t = t * wk;
            if (a.b) t = t + bk;
            set(o[0], e, t);
        }
        // a thread stores only the vectors of its workgroup's chunk (one or
        // two of the NV it holds): the activation's switch once per vector
        if constexpr (ACT) apply_act_vec<1>(a.act, o, a.tab, 0.0f);
        if (n_chunks == 1) *reinterpret_cast<float4*>(yg + 16 * qi) = o[0];
        else Stream<float>::store4(yg + 16 * qi, o[0]);
    }
}

// ACT: 0 none, 1 the activation chosen at run time, 2 Mish compiled in.
template <int NV, int ACT>
__global__ __launch_bounds__(kSplitThreads) void k_group_norm_split(GnSplit a) {
    gn_split_body<NV, ACT>(a, blockIdx.x);
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

template <int ACT>
void gn_split(const GnSplit& sp, uint32_t n_slots, int nv, hipStream_t s) {
    const dim3 grid(n_slots);
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_group_norm_split<1, ACT>), grid, dim3(kSplitThreads), 0, s, sp); break;
        case 2: hipLaunchKernelGGL((k_group_norm_split<2, ACT>), grid, dim3(kSplitThreads), 0, s, sp); break;
        case 4: hipLaunchKernelGGL((k_group_norm_split<4, ACT>), grid, dim3(kSplitThreads), 0, s, sp); break;
        default: hipLaunchKernelGGL((k_group_norm_split<8, ACT>), grid, dim3(kSplitThreads), 0, s, sp); break;
    }
}

// The vectorised layout: every group a contiguous run of floats (ne0, ne1
// dense within a channel, channels adjacent), 16-byte aligned, ne0 % 4 == 0.
bool gn_vec_layout(const cbx_tensor* x, const cbx_tensor* y) {
    bool vec = x->ne[0] % 4 == 0;
    for (const cbx_tensor* t : {x, y}) {
        const size_t row = 4 * static_cast<size_t>(t->ne[0]);
        if (t->ne[1] > 1 && t->nb[1] != row) vec = false;
        if (t->ne[2] > 1 && t->nb[2] != row * static_cast<size_t>(t->ne[1])) vec = false;
        if (reinterpret_cast<uintptr_t>(t->data) % 16 || t->nb[2] % 16 || t->nb[3] % 16) vec = false;
    }
    return vec;
}

GnArgs gn_args(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b, int act,
               cbx_tensor* y, DeviceState* st) {
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
    return a;
}

// Scratch of cbx_group_norm_noalloc and cbx_group_norm, for callers that
// cannot allocate: kScratchSets sets of the split reduction's exchange
// words, each for kSplitMaxSlots chunk slots (128 KiB a set, 1 MiB in all),
// in the library's own device memory, one copy per GPU, held until the
// process ends.  A call takes the set its stream hashes to, so calls on
// different streams rarely share one (and when they do, the launch tags
// keep the results exact; only the waits run out).  Zero at load; the launch
// tags mean nothing in it ever needs clearing.  Host code must not pass
// `scratch` itself to a kernel (on the host it names a stand-in, not device
// memory): group_norm_scratch_setup looks up each device's address once, at
// cbx_init, and launches use that.
constexpr uint32_t kScratchSets = 8;
static __device__ __align__(256) uint64_t scratch[kScratchSets * 2 * kSplitStageWords];

// Which XCD (its XCC_ID hardware register) runs each workgroup.
__global__ __launch_bounds__(kSplitThreads) void k_xcc_probe(uint32_t* out) {
    if (threadIdx.x == 0) {
        uint32_t id;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(id));
        out[blockIdx.x] = id;
    }
}

}  // namespace

int group_norm_scratch_setup(void** out) {
    *out = nullptr;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        return set_error(CBX_ERR_HIP, std::string("cbx_init: hipGetSymbolAddress of the group norm scratch failed: ") +
                                          hipGetErrorString(e));
    }
    *out = p;
    return CBX_OK;
}

size_t group_norm_scratch_slots() { return kSplitMaxSlots; }

void* group_norm_scratch_for(const DeviceState* st, hipStream_t s) {
    const uint64_t h = (static_cast<uint64_t>(reinterpret_cast<uintptr_t>(s)) >> 4) * 0x9E3779B97F4A7C15ull;
    const uint32_t set = static_cast<uint32_t>(h >> 61) % kScratchSets;
    return static_cast<char*>(st->gn_scratch) + set * group_norm_workspace_bytes();
}

size_t group_norm_workspace_bytes() {
    return 2 * static_cast<size_t>(kSplitStageWords) * sizeof(uint64_t);
}

int group_norm_probe_xcd(bool* ok) {
    *ok = false;
    constexpr uint32_t kBlocks = 2048;
    uint32_t* d = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&d), kBlocks * sizeof(uint32_t)) != hipSuccess) {
        return set_error(CBX_ERR_HIP, "cbx_init: hipMalloc of the XCD probe failed");
    }
    hipLaunchKernelGGL(k_xcc_probe, dim3(kBlocks), dim3(kSplitThreads), 0, nullptr, d);
    uint32_t h[kBlocks];
    const bool good = hipGetLastError() == hipSuccess &&
                      hipMemcpy(h, d, sizeof(h), hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(d);
    if (!good) return set_error(CBX_ERR_HIP, "cbx_init: the XCD probe failed");
    // the split's chunks of one group are workgroups b with one b % 8: they
    // must share an XCD (and so an L2)
    bool same = true;
    for (uint32_t b = kXcds; b < kBlocks; b++) same = same && h[b] == h[b % kXcds];
    *ok = same;
    return CBX_OK;
}

bool group_norm_split_args(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                           int act, const cbx_tensor* y, void* workspace, uint32_t first_slot, uint64_t wait_ticks,
                           int n_chunks_req, const DeviceState* st, GnSplit* sp, uint32_t* n_slots, int* nv,
                           uint32_t* slots_used, const char** why) {
    const int64_t cpg = cdiv(x->ne[2], n_groups);
    const int64_t count = x->ne[0] * x->ne[1] * std::min<int64_t>(cpg, x->ne[2]);
    const int64_t n_gi = int64_t{n_groups} * x->ne[3];
    const int64_t n4 = count / 4;
    // one 256-lane workgroup per CU (measured best on the CFM shapes against
    // 8 to 32 chunks of 256 to 1024 lanes: more chunks add participants and
    // dispatch skew to every exchange, fewer leave the activation and stores
    // to too few SIMDs); at most 8 vectors a lane
    int64_t n_chunks = n_chunks_req > 0 ? n_chunks_req : cdiv(st->n_cu, n_gi);
    n_chunks = std::min<int64_t>({n_chunks, kSplitMaxChunks, n4});
    n_chunks = std::max<int64_t>(n_chunks, cdiv(n4, 8 * kSplitThreads));
    const int64_t padded_gi = int64_t{kXcds} * cdiv(n_gi, kXcds);
    // the split applies out of place (a wave that stops waiting re-reads x),
    // on a device whose dispatch was seen to deal workgroups to XCDs by
    // index mod 8, when the groups are few (n_chunks >= 2) and the whole
    // grid is resident at once (at most 2 workgroups a CU)
    const uintptr_t xl = reinterpret_cast<uintptr_t>(x->data), yl = reinterpret_cast<uintptr_t>(y->data);
    const size_t span = static_cast<size_t>(x->ne[3]) * x->nb[3];
    *why = nullptr;
    if (xl < yl + span && yl < xl + span) *why = "in place";
    else if (!st->gn_split_ok) *why = "the device's dispatch does not place workgroups by index mod 8";
    else if (!gn_vec_layout(x, y)) *why = "groups are not contiguous, 16-byte aligned runs";
    else if (n_chunks < 2 || n_chunks > kSplitMaxChunks) *why = "groups too many or too small to split";
    else if (int64_t{first_slot} + n_gi * n_chunks > kSplitMaxSlots) *why = "more than 1024 chunk slots";
    else if (padded_gi * n_chunks > int64_t{2} * st->n_cu) *why = "the grid is not resident at once";
    else if (x->ne[0] * x->ne[1] * cpg >= (int64_t{1} << 30)) *why = "groups too large";
    if (*why) return false;
    if (wait_ticks == kGnWaitAuto) {
        // ten times what the launch should take (a few microseconds plus its
        // bytes at 2 TB/s), at least 20 us: long past a resident grid's
        // arrival skew, short against the fallback's cost of a stall
        const double bytes = 8.0 * static_cast<double>(count) * static_cast<double>(n_gi);
        const double us = std::max(20.0, 10.0 * (3.0 + bytes / 2.0e6));
        wait_ticks = static_cast<uint64_t>(us * 100.0);
    }
    const int64_t per = cdiv(n4, n_chunks);
    *nv = per <= kSplitThreads ? 1 : per <= 2 * kSplitThreads ? 2 : per <= 4 * kSplitThreads ? 4 : 8;
    sp->x = static_cast<const char*>(x->data);
    sp->y = static_cast<char*>(y->data);
    sp->w = w ? static_cast<const float*>(w->data) : nullptr;
    sp->b = b ? static_cast<const float*>(b->data) : nullptr;
    sp->word = static_cast<uint64_t*>(workspace) + 2 * static_cast<size_t>(first_slot) * kSplitWaves;
    sp->tab = st->gelu_table;
    sp->x_nb3 = static_cast<int64_t>(x->nb[3]);
    sp->y_nb3 = static_cast<int64_t>(y->nb[3]);
    sp->wait_ticks = wait_ticks;
    sp->n_chunks = static_cast<uint32_t>(n_chunks);
    sp->n_gi = static_cast<uint32_t>(n_gi);
    sp->n_groups = static_cast<uint32_t>(n_groups);
    sp->per_ch = static_cast<uint32_t>(x->ne[0] * x->ne[1]);
    sp->cpg = static_cast<uint32_t>(cpg);
    sp->C = static_cast<uint32_t>(x->ne[2]);
    sp->eps = eps;
    sp->act = act;
    *n_slots = static_cast<uint32_t>(padded_gi * n_chunks);
    *slots_used = static_cast<uint32_t>(n_gi * n_chunks);
    return true;
}

int launch_group_norm_split(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                            int act, cbx_tensor* y, void* workspace, uint64_t wait_ticks, int n_chunks_req,
                            DeviceState* st, hipStream_t s) {
    GnSplit sp;
    uint32_t n_slots = 0, used = 0;
    int nv = 1;
    const char* why = nullptr;
    if (!group_norm_split_args(x, n_groups, eps, w, b, act, y, workspace, 0, wait_ticks, n_chunks_req, st, &sp,
                               &n_slots, &nv, &used, &why)) {
        return launch_group_norm(x, n_groups, eps, w, b, act, y, st, s);
    }
    if (act == CBX_UNARY_MISH) gn_split<2>(sp, n_slots, nv, s);
    else if (act != CBX_UNARY_NONE) gn_split<1>(sp, n_slots, nv, s);
    else gn_split<0>(sp, n_slots, nv, s);
    return check_launch("group_norm");
}

int launch_group_norm(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                      int act, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    GnArgs a = gn_args(x, n_groups, eps, w, b, act, y, st);
    const bool vec = gn_vec_layout(x, y);
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
