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

// ---- split reduction --------------------------------------------------------
// A few large groups (the CFM's 2 x 8) spread over many workgroups: each
// chunk workgroup holds only its chunk of the group in registers, and the
// f64 partial sums of its waves meet those of the group's other chunks in a
// workspace, once for the mean and once for the variance.  Each element is
// read once and every workgroup's VALU work is its own chunk.  Out of place
// only: the host sends a y that overlaps x to the one-workgroup-per-group
// kernels, because a wave that stops waiting (below) re-reads the whole
// group from x, which must then still hold the input.
//
// Every wave publishes its own partial and every wave collects the group's
// partials itself: no barrier and no LDS anywhere, so a wave goes from its
// loads to its exchange and from the exchange to its stores without waiting
// for the other waves of its workgroup.  The group's P = n_chunks x 4
// partials (slot ci * 4 + wave) are added in slot order -- lane l adds
// slots l, l + 64, .. starting from +0, then the lanes by the DPP
// butterfly -- the same bits in every wave of the group.
//
// A partial travels as two 64-bit words (its low and high halves); the
// upper 32 bits of the first carry the low half of the launch's 64-bit tag,
// those of the second its high half.  The tag is an odd multiple of the
// dispatch's 64-bit packet index on its queue plus a hash of the queue and
// kernel-argument addresses (a bijection of the packet index: launches on
// one queue never share a tag), never 0 (fresh memory).  A word is written
// whole and read whole, so a reader that finds all 64 tag bits in a slot has
// that wave's partial; words left by earlier launches, or by a launch on
// another stream that shares the workspace, carry other tags, and nothing
// is ever cleared.  The words are written with plain stores, which reach
// the L2 that the workgroups of one group share (their indices put them on
// one XCD: dispatch deals workgroups to the 8 XCDs round-robin, which the
// host checks once per device before it uses this kernel), and read with
// agent-scope loads.
//
// Waits are bounded: after GnSplit::wait_ticks of the 100 MHz real-time
// counter a wave stops waiting and computes every slot's partial itself
// from x, with the same lanes and order as the wave that owns the slot, so
// the statistics are the same bits either way, and a workgroup that never
// gets a CU while the others run (another stream's kernel holding the CUs,
// or a launch on another stream writing the same workspace) delays them by
// the wait, never changes a result.  wait_ticks == 0: never wait.
constexpr int kSplitThreads = 256;
constexpr int kSplitWaves = kSplitThreads / WAVE;
constexpr int kSplitMaxChunks = 32;
constexpr int kSplitLaneSlots = kSplitMaxChunks * kSplitWaves / WAVE;   // partial slots a lane collects
constexpr uint32_t kSplitMaxSlots = 1024;   // group instances x chunks per launch
constexpr uint32_t kSplitStageWords = 2 * kSplitMaxSlots * kSplitWaves;

// Compact arguments: every field arrives in the kernel's first round of
// scalar loads, and the index arithmetic before the first load is 32-bit.
struct GnSplit {
    const char* x;
    char* y;
    const float* w;
    const float* b;
    uint64_t* word;          // [2 stages][kSplitMaxSlots * kSplitWaves][2 words]
    const uint16_t* tab;
    int64_t x_nb3, y_nb3;    // batch strides (bytes)
    uint64_t wait_ticks;
    uint32_t n_chunks, n_gi, n_groups, per_ch, cpg, C;   // per_ch = ne0 * ne1
    float eps;
    int32_t act;
};

// The dispatch's 64-bit packet index on its queue (llvm.amdgcn.dispatch.id;
// clang has no builtin for it).
extern "C" __device__ uint64_t cbx_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

__device__ __forceinline__ uint64_t launch_tag() {
    const uint64_t id = cbx_dispatch_id();
    const uint64_t q = reinterpret_cast<uintptr_t>(__builtin_amdgcn_queue_ptr());
    const uint64_t ka = reinterpret_cast<uintptr_t>(__builtin_amdgcn_kernarg_segment_ptr());
    const uint64_t mix = ((q >> 6) * 0xC2B2AE3D27D4EB4Full) ^ ((ka >> 4) * 0x165667B19E3779F9ull);
    const uint64_t t = id * 0x9E3779B97F4A7C15ull + mix;   // odd multiplier: one tag per packet index
    return t ? t : 1;
}

// A lane's partial of stage 0 (Σx) or 1 (Σ(x - mean)^2, the f32
// difference and square summed in f64) over its NV vectors.
template <int NV>
__device__ __forceinline__ double lane_partial(const float4 (&v)[NV], const bool (&ok)[NV], int stage, float mean) {
    double p[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if (stage == 0) {
            p[k] = ok[k] ? (static_cast<double>(v[k].x) + static_cast<double>(v[k].y)) +
                               (static_cast<double>(v[k].z) + static_cast<double>(v[k].w))
                         : 0.0;
        } else {
            const float d0 = v[k].x - mean, d1 = v[k].y - mean, d2 = v[k].z - mean, d3 = v[k].w - mean;
            p[k] = ok[k] ? (static_cast<double>(d0 * d0) + static_cast<double>(d1 * d1)) +
                               (static_cast<double>(d2 * d2) + static_cast<double>(d3 * d3))
                         : 0.0;
        }
    }
    return thread_tree_sum<NV>(p);
}

// The NV vectors that wave `wv` of the chunk [q0, q1) holds in lane `lane`
// (float4 indices q0 + wv*64 + lane + k*kSplitThreads); lanes past the chunk
// (a chunk may be empty) load the group's first vector, an address inside
// the group.
template <int NV>
__device__ __forceinline__ void wave_chunk_load(const char* xg, uint32_t q0, uint32_t q1, uint32_t wv, uint32_t lane,
                                                float4 (&v)[NV], bool (&ok)[NV]) {
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const uint32_t qi = q0 + wv * WAVE + lane + static_cast<uint32_t>(k) * kSplitThreads;
        ok[k] = qi < q1;
        v[k] = *reinterpret_cast<const float4*>(xg + 16 * static_cast<uint64_t>(ok[k] ? qi : 0));
    }
}

// Publishes this wave's partial of `stage`, waits (bounded) for the group's
// other partials and returns the group's sum (the same bits in every wave
// of the group), or computes every slot's partial itself when the wait
// runs out.
template <int NV>
__device__ __forceinline__ double split_exchange(const GnSplit& a, uint64_t tag, uint32_t gi, uint32_t ci, int stage,
                                                 double mine, float mean, const char* xg, uint32_t n4, uint32_t per) {
    const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
    const uint32_t P = a.n_chunks * kSplitWaves;
    uint64_t* wd = a.word + static_cast<uint64_t>(stage) * kSplitStageWords + 2 * static_cast<uint64_t>(gi) * P;
    const uint64_t bits = __builtin_bit_cast(uint64_t, mine);
    const uint64_t tag_lo = tag << 32, tag_hi = tag & 0xffffffff00000000ull;
    const uint32_t own = ci * kSplitWaves + wave;
    if (lane < 2) {
        // lanes 0 and 1 publish the low and high halves
        const uint64_t word = lane == 0 ? tag_lo | (bits & 0xffffffffu) : tag_hi | (bits >> 32);
        __hip_atomic_store(&wd[2 * own + lane], word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    double val[kSplitLaneSlots];
    bool ok = false;
    if (a.wait_ticks) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (true) {
            bool have = true;
#pragma unroll
            for (int r = 0; r < kSplitLaneSlots; r++) {
                const uint32_t sl = lane + WAVE * r;
                val[r] = 0.0;
                if (sl < P) {
                    if (sl == own) {
                        val[r] = mine;
                    } else {
                        const uint64_t lo = __hip_atomic_load(&wd[2 * sl], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const uint64_t hi =
                            __hip_atomic_load(&wd[2 * sl + 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        have = have && (lo & 0xffffffff00000000ull) == tag_lo &&
                               (hi & 0xffffffff00000000ull) == tag_hi;
                        val[r] = __builtin_bit_cast(double, (lo & 0xffffffffu) | (hi << 32));
                    }
                }
            }
            if (__all(have)) {
                ok = true;
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > a.wait_ticks) break;
        }
    }
    if (!ok) {
        // every slot's partial, as the wave that owns it computes it (x is
        // still the input: the split runs out of place only)
#pragma unroll
        for (int r = 0; r < kSplitLaneSlots; r++) val[r] = 0.0;
        for (uint32_t sl = 0; sl < P; sl++) {
            const uint32_t c = sl / kSplitWaves, wv = sl - c * kSplitWaves;
            const uint32_t q0 = c * per, q1 = q0 + per < n4 ? q0 + per : n4;
            float4 v[NV];
            bool okv[NV];
            wave_chunk_load<NV>(xg, q0, q1, wv, lane, v, okv);
            const double ps = wave_sum(lane_partial<NV>(v, okv, stage, mean));
#pragma unroll
            for (int r = 0; r < kSplitLaneSlots; r++) {
                if (sl == lane + WAVE * r) val[r] = ps;
            }
        }
    }
    double t = 0.0;
#pragma unroll
    for (int r = 0; r < kSplitLaneSlots; r++) t += val[r];
    return wave_sum(t);
}

// ACT: 0 none, 1 the activation chosen at run time, 2 Mish (the CFM
// decoder's GroupNorm -> Mish) compiled in, without the switch's branches.
template <int NV, int ACT>
__global__ __launch_bounds__(kSplitThreads) void k_group_norm_split(GnSplit a) {
    arg_now(a.x);
    arg_now(a.y);
    arg_now(a.w);
    arg_now(a.b);
    arg_now(a.word);
    arg_now(reinterpret_cast<const void*>(a.x_nb3));
    arg_now(reinterpret_cast<const void*>(a.y_nb3));
    arg_now(a.per_ch);
    arg_now(a.cpg);
    arg_now(a.C);
    // workgroup b: XCD b % 8, and its chunks on that XCD
    const uint32_t b = blockIdx.x, j = b / kXcds;
    const uint32_t m = j / a.n_chunks, ci = j - m * a.n_chunks;
    const uint32_t gi = b % kXcds + kXcds * m;
    const uint32_t i3 = gi / a.n_groups, g = gi - i3 * a.n_groups;
    const uint32_t c0 = g * a.cpg;
    // past the last group, or an empty group (past C): every workgroup of it
    // leaves here, so nobody counts on its partials
    if (gi >= a.n_gi || c0 >= a.C) return;
    const uint32_t c1 = c0 + a.cpg < a.C ? c0 + a.cpg : a.C;
    const uint32_t n4 = (a.per_ch * (c1 - c0)) / 4;
    const uint32_t per = (n4 + a.n_chunks - 1) / a.n_chunks;
    const uint32_t q0 = ci * per, q1 = q0 + per < n4 ? q0 + per : n4;
    const uint64_t gofs = static_cast<uint64_t>(c0) * a.per_ch * 4;
    const char* xg = a.x + gofs + static_cast<int64_t>(i3) * a.x_nb3;
    char* yg = a.y + gofs + static_cast<int64_t>(i3) * a.y_nb3;
    const uint32_t lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;

    float4 v[NV];
    bool ok[NV];
    wave_chunk_load<NV>(xg, q0, q1, wave, lane, v, ok);
    // the affine values of each vector's channel (a vector lies in one
    // channel: ne0 % 4 == 0), read from x where there are none
    float wv[NV], bv[NV];
    const float* wq = a.w ? a.w : reinterpret_cast<const float*>(xg);
    const float* bq = a.b ? a.b : reinterpret_cast<const float*>(xg);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const uint32_t qi = q0 + threadIdx.x + static_cast<uint32_t>(k) * kSplitThreads;
        const uint32_t c = c0 + (4 * (ok[k] ? qi : q0)) / a.per_ch;
        wv[k] = wq[a.w ? c : 0];
        bv[k] = bq[a.b ? c : 0];
    }
    const uint64_t tag = launch_tag();
    const double count = static_cast<double>(4 * n4);
    const double s =
        split_exchange<NV>(a, tag, gi, ci, 0, wave_sum(lane_partial<NV>(v, ok, 0, 0.0f)), 0.0f, xg, n4, per);
    const float mean = static_cast<float>(s / count);
    const double s2 =
        split_exchange<NV>(a, tag, gi, ci, 1, wave_sum(lane_partial<NV>(v, ok, 1, mean)), mean, xg, n4, per);
    const float var = static_cast<float>(s2 / count);
    const float scale = 1.0f / sqrtf(var + a.eps);
#pragma unroll
    for (int k = 0; k < NV; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float t = (get(v[k], e) - mean) * scale;
            if (a.w) t = t * wv[k];
            if (a.b) t = t + bv[k];
            if constexpr (ACT == 2) t = act_mish(t);
            set(v[k], e, t);
        }
    }
    if constexpr (ACT == 1) apply_act_vec<NV>(a.act, v, a.tab, 0.0f);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const uint32_t qi = q0 + threadIdx.x + static_cast<uint32_t>(k) * kSplitThreads;
        if (ok[k]) Stream<float>::store4(yg + 16 * static_cast<uint64_t>(qi), v[k]);
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

int launch_group_norm_split(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                            int act, cbx_tensor* y, void* workspace, uint64_t wait_ticks, int n_chunks_req,
                            DeviceState* st, hipStream_t s) {
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
    const bool overlap = xl < yl + span && yl < xl + span;
    if (overlap || !st->gn_split_ok || !gn_vec_layout(x, y) || n_chunks < 2 || n_chunks > kSplitMaxChunks ||
        n_gi * n_chunks > kSplitMaxSlots || padded_gi * n_chunks > int64_t{2} * st->n_cu ||
        x->ne[0] * x->ne[1] * cpg >= (int64_t{1} << 30)) {
        return launch_group_norm(x, n_groups, eps, w, b, act, y, st, s);
    }
    if (wait_ticks == kGnWaitAuto) {
        // ten times what the launch should take (a few microseconds plus its
        // bytes at 2 TB/s), at least 20 us: long past a resident grid's
        // arrival skew, short against the fallback's cost of a stall
        const double bytes = 8.0 * static_cast<double>(count) * static_cast<double>(n_gi);
        const double us = std::max(20.0, 10.0 * (3.0 + bytes / 2.0e6));
        wait_ticks = static_cast<uint64_t>(us * 100.0);
    }
    const int64_t per = cdiv(n4, n_chunks);
    const int nv = per <= kSplitThreads ? 1 : per <= 2 * kSplitThreads ? 2 : per <= 4 * kSplitThreads ? 4 : 8;
    GnSplit sp;
    sp.x = static_cast<const char*>(x->data);
    sp.y = static_cast<char*>(y->data);
    sp.w = w ? static_cast<const float*>(w->data) : nullptr;
    sp.b = b ? static_cast<const float*>(b->data) : nullptr;
    sp.word = static_cast<uint64_t*>(workspace);
    sp.tab = st->gelu_table;
    sp.x_nb3 = static_cast<int64_t>(x->nb[3]);
    sp.y_nb3 = static_cast<int64_t>(y->nb[3]);
    sp.wait_ticks = wait_ticks;
    sp.n_chunks = static_cast<uint32_t>(n_chunks);
    sp.n_gi = static_cast<uint32_t>(n_gi);
    sp.n_groups = static_cast<uint32_t>(n_groups);
    sp.per_ch = static_cast<uint32_t>(x->ne[0] * x->ne[1]);
    sp.cpg = static_cast<uint32_t>(cpg);
    sp.C = static_cast<uint32_t>(x->ne[2]);
    sp.eps = eps;
    sp.act = act;
    const uint32_t n_slots = static_cast<uint32_t>(padded_gi * n_chunks);
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
