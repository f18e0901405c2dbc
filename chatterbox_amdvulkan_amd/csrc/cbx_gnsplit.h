// cbx_gnsplit.h -- the split-reduction GroupNorm body (each chunk workgroup
// of a group reduces its chunk; the chunks' partial sums meet in a
// workspace), shared by the standalone kernel (k_group_norm.hip) and the
// op batch (k_batch.hip).  Device code only.
#pragma once

#include "cbx_device.h"

namespace cbx {
namespace {

constexpr uint32_t kXcds = 8;   // gfx950: workgroups go to XCD (index % 8)

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

// GnSplit (cbx_internal.h) carries the arguments: every field arrives in
// the kernel's first round of scalar loads, and the index arithmetic
// before the first load is 32-bit.

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
__device__ __forceinline__ void gn_split_body(const GnSplit& a, uint32_t b) {
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
    // workgroup b: XCD b % 8 (b counts from a multiple of 8), and its
    // chunks on that XCD
    const uint32_t j = b / kXcds;
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

}  // namespace
}  // namespace cbx
