// cbx_rowops.h -- device building blocks shared by the standalone kernels and
// the one-launch op batch (k_batch.hip): wave-per-row normalisation, table
// row loads, and the RoPE angle recurrence.
#pragma once

#include "cbx_device.h"

namespace cbx {

// ---------------------------------------------------------------------------
// argument and row addressing for the row kernels
// ---------------------------------------------------------------------------

// Byte offset of row r of a tensor whose rows enumerate ne1, ne2, ne3
// (fewer than 2^31 rows), with 32-bit index arithmetic.
struct RowMap {
    int64_t nb1, nb2, nb3;
    uint32_t ne1, ne2;
    uint32_t flat;   // rows at one uniform step nb1: no index split
};

inline RowMap row_map(const cbx_tensor* t) {
    RowMap m;
    m.flat = flat_rows(t) ? 1u : 0u;
    m.nb1 = static_cast<int64_t>(t->nb[1]);
    m.nb2 = static_cast<int64_t>(t->nb[2]);
    m.nb3 = static_cast<int64_t>(t->nb[3]);
    m.ne1 = static_cast<uint32_t>(t->ne[1] > 0 ? t->ne[1] : 1);
    m.ne2 = static_cast<uint32_t>(t->ne[2] > 0 ? t->ne[2] : 1);
    return m;
}

__device__ __forceinline__ int64_t row_at(const RowMap& m, uint32_t r) {
    if (m.flat) return r * m.nb1;
    const uint32_t i1 = r % m.ne1, q = r / m.ne1;
    const uint32_t i2 = q % m.ne2, i3 = q / m.ne2;
    return i1 * m.nb1 + i2 * m.nb2 + i3 * m.nb3;
}

// ---------------------------------------------------------------------------
// wave-per-row building blocks
// ---------------------------------------------------------------------------

// Normalisation scale of the row held in v (lane owns elements
// (lane + 64k)*4 .. +3); for LN, v is replaced by v - mean.
template <int NV, int KIND>
__device__ __forceinline__ float wave_row_scale(float4 (&v)[NV], int lane, int64_t ne0, float eps) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float t = get(v[k], e);
            if constexpr (KIND == NORM_LN) s += static_cast<double>(t);
            else s += static_cast<double>(t * t);
        }
    }
    s = wave_sum(s);
    if constexpr (KIND == NORM_LN) {
        const float mean = static_cast<float>(s) / static_cast<float>(ne0);
        double s2 = 0.0;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            if ((lane + 64 * k) * 4 < ne0) {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float d = get(v[k], e) - mean;
                    set(v[k], e, d);
                    s2 += static_cast<double>(d * d);
                }
            }
        }
        s2 = wave_sum(s2);
        const float var = static_cast<float>(s2 / static_cast<double>(ne0));
        return 1.0f / sqrtf(var + eps);
    } else {
        const float ms = static_cast<float>(s / static_cast<double>(ne0));
        return 1.0f / sqrtf(ms + eps);
    }
}

// W waves of one workgroup cooperating on one row: wave w holds float4s
// [w*64*NV, (w+1)*64*NV) of it, so the helpers here, written for a lane's
// vectors lane4 + 64k, take lane4 = w*64*NV + lane (lane4 = lane for one
// wave a row).  Each reduction: the wave's total by the DPP butterfly, the
// W totals through LDS (one barrier), added in wave order by every thread
// -- a fixed order, like the one-wave form.  lds: 2*W doubles.
template <int NV, int KIND, int W>
__device__ __forceinline__ float row_scale_w(float4 (&v)[NV], int lane4, int64_t ne0, float eps, double* lds) {
    if constexpr (W == 1) {
        return wave_row_scale<NV, KIND>(v, lane4, ne0, eps);
    } else {
        const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < NV; k++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = get(v[k], e);
                if constexpr (KIND == NORM_LN) s += static_cast<double>(t);
                else s += static_cast<double>(t * t);
            }
        }
        s = wave_sum(s);
        if (lane == 0) lds[wid] = s;
        __syncthreads();
        s = lds[0];
#pragma unroll
        for (int i = 1; i < W; i++) s += lds[i];
        if constexpr (KIND == NORM_LN) {
            const float mean = static_cast<float>(s) / static_cast<float>(ne0);
            double s2 = 0.0;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                if ((lane4 + 64 * k) * 4 < ne0) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float d = get(v[k], e) - mean;
                        set(v[k], e, d);
                        s2 += static_cast<double>(d * d);
                    }
                }
            }
            s2 = wave_sum(s2);
            if (lane == 0) lds[W + wid] = s2;
            __syncthreads();
            s2 = lds[W];
#pragma unroll
            for (int i = 1; i < W; i++) s2 += lds[W + i];
            const float var = static_cast<float>(s2 / static_cast<double>(ne0));
            return 1.0f / sqrtf(var + eps);
        } else {
            const float ms = static_cast<float>(s / static_cast<double>(ne0));
            return 1.0f / sqrtf(ms + eps);
        }
    }
}

// Affine vectors for the lane's elements, loaded up front (uniform branches:
// the loads overlap the row loads instead of stalling the epilogue).
template <int NV>
struct Affine {
    float4 w[NV], b[NV];
    // Branch-free form: a null wp/bp reads its vectors from `safe` (a
    // 16-byte aligned address of at least ne0 floats) instead, and the
    // caller ignores them.  A pointer select rather than a branch, so the
    // compiler has no conditional block to sink argument loads into: every
    // argument arrives in the kernel's first round of scalar loads.
    __device__ __forceinline__ void load_sel(const float* wp, const float* bp, const float* safe, int lane,
                                             int64_t ne0) {
        const float* wq = wp ? wp : safe;
        const float* bq = bp ? bp : safe;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int64_t j = (lane + 64 * k) * 4;
            const int64_t jc = j < ne0 ? j : 0;
            w[k] = *reinterpret_cast<const float4*>(wq + jc);
            b[k] = *reinterpret_cast<const float4*>(bq + jc);
        }
    }
    __device__ __forceinline__ void load(const float* __restrict__ wp, const float* __restrict__ bp, int lane,
                                         int64_t ne0) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int64_t j = (lane + 64 * k) * 4;
            const int64_t jc = j < ne0 ? j : 0;
            if (wp) w[k] = *reinterpret_cast<const float4*>(wp + jc);
            if (bp) b[k] = *reinterpret_cast<const float4*>(bp + jc);
        }
    }
};

// Output rows are written with streaming (nontemporal) stores: left dirty
// in the L2 instead, the rows were written back at the kernel's end, which
// measured 0.2 us longer per launch for the 8 MB of the T3 prefill's
// embedding + LayerNorm.
template <typename TO, int NV, bool ACT>
__device__ __forceinline__ void wave_row_store(const float4 (&v)[NV], int lane, int64_t ne0, float scale,
                                               const Affine<NV>& af, bool hw, bool hb, int act,
                                               const uint16_t* __restrict__ tab, char* yr) {
    float4 o[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float t = get(v[k], e) * scale;
            if (hw) t = t * get(af.w[k], e);
            if (hb) t = t + get(af.b[k], e);
            set(o[k], e, t);
        }
    }
    // the activation's switch once for all of the lane's elements
    if constexpr (ACT) apply_act_vec<NV>(act, o, tab, 0.0f);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        if (j < ne0) Stream<TO>::store4(yr + j * Elt<TO>::size, o[k]);
    }
}

template <int TYPE>
__device__ __forceinline__ float4 load_table4(const char* row, int64_t j) {
    if constexpr (TYPE == CBX_TYPE_F32) {
        return *reinterpret_cast<const float4*>(row + j * 4);
    } else if constexpr (TYPE == CBX_TYPE_F16) {
        return Elt<uint16_t>::load4(row + j * 2);
    } else {
        // block: f16 scale d, then 32 int8 quants; the 4 quants of a
        // 4-aligned j sit at an even offset, read as two 16-bit words
        const char* blk = row + (j >> 5) * 34;
        const float d = h2f(*reinterpret_cast<const uint16_t*>(blk));
        const uint16_t* q = reinterpret_cast<const uint16_t*>(blk + 2 + (j & 31));
        const uint32_t q01 = q[0], q23 = q[1];
        return make_float4(static_cast<float>(static_cast<int8_t>(q01 & 0xffu)) * d,
                           static_cast<float>(static_cast<int8_t>(q01 >> 8)) * d,
                           static_cast<float>(static_cast<int8_t>(q23 & 0xffu)) * d,
                           static_cast<float>(static_cast<int8_t>(q23 >> 8)) * d);
    }
}

// An out-of-range id: ggml aborts; here the row's outputs are zeroed and
// the sticky device error bit is raised.
__device__ __forceinline__ void embed_bad_row(char* hr, char* yr, int64_t ne0, int lane, uint32_t* err) {
    for (int64_t j = lane; j < ne0; j += 64) {
        reinterpret_cast<float*>(yr)[j] = 0.0f;
        if (hr) reinterpret_cast<float*>(hr)[j] = 0.0f;
    }
    if (lane == 0) atomicOr(err, static_cast<uint32_t>(DEV_ERR_ROW_INDEX));
}

// The T3 embedding row: h = f32(table row) + f32(position row), stored when
// hr is non-null, then y = LN(h)*w + b.  Row loads are unconditional
// (clamped addresses) so all 2*NV are in flight together.  `bad` (uniform):
// an id was out of range -- the caller passed row 0 in its place, and the
// row's outputs are zeroed instead, after the loads, so no branch precedes
// them.
template <int TYPE, int TYPE2, int NV, int W = 1>
__device__ __forceinline__ void embed_ln_row(const char* s1, const char* s2, const Affine<NV>& af, bool hw, bool hb,
                                             char* hr, char* yr, int64_t ne0, float eps, int lane, bool bad,
                                             uint32_t* err, double* lds = nullptr) {
    // several waves a row: the caller's w and b loads stay ahead of the row
    // loads (the standalone [512,1024] kernel, four waves a token: 3.85
    // against 3.99 us with the rows first); one wave a row: the compiler's
    // order (the op batch's prefill launch: 6.00 against 6.14 us)
    if constexpr (W > 1) __builtin_amdgcn_sched_barrier(0);
    float4 p[NV], q[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        p[k] = load_table4<TYPE>(s1, j < ne0 ? j : 0);
        q[k] = load_table4<TYPE2>(s2, j < ne0 ? j : 0);
    }
    if (bad) {   // uniform over the workgroup: every wave of the row leaves
        if (lane < 64) embed_bad_row(hr, yr, ne0, lane, err);
        return;
    }
    // h by a select, not a branch (a branch would take the row loads into
    // its block), then h stored with nothing else pending: the prefill
    // launch's embedding + LayerNorm beside GELU, 6.00 against 6.47 us
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const bool in = (lane + 64 * k) * 4 < ne0;
        v[k] = make_float4(in ? p[k].x + q[k].x : 0.f, in ? p[k].y + q[k].y : 0.f, in ? p[k].z + q[k].z : 0.f,
                           in ? p[k].w + q[k].w : 0.f);
    }
    wait_vector_memory();
    if (hr) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int64_t j = (lane + 64 * k) * 4;
            if (j < ne0) Stream<float>::store4(hr + j * 4, v[k]);
        }
    }
    const float scale = row_scale_w<NV, NORM_LN, W>(v, lane, ne0, eps, lds);
    wave_row_store<float, NV, false>(v, lane, ne0, scale, af, hw, hb, CBX_UNARY_NONE, nullptr, yr);
}

// cos/sin of pair k for position p: theta = p * theta_scale^k as an iterated
// f32 product (ggml's rope cache), then ggml's YaRN correction.
__device__ inline void rope_cos_sin_dev(int32_t p, int k, const RopeParams& rp, const float* __restrict__ ff, float* c,
                                 float* s) {
    float theta = static_cast<float>(p);
    for (int i = 0; i < k; i++) theta = theta * rp.theta_scale;
    const float theta_extrap = ff ? theta / ff[k] : theta;
    const float theta_interp = rp.freq_scale * theta_extrap;
    float th = theta_interp;
    float mscale = rp.attn_factor;
    if (rp.ext_factor != 0.0f) {
        const float d = rp.corr_dims[1] - rp.corr_dims[0];
        const float y = (static_cast<float>(k) - rp.corr_dims[0]) / (d > 0.001f ? d : 0.001f);
        const float cl = y < 0.0f ? 0.0f : y;
        const float ramp_mix = (1.0f - (cl < 1.0f ? cl : 1.0f)) * rp.ext_factor;
        th = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
        mscale = mscale * (1.0f + 0.1f * logf(1.0f / rp.freq_scale));
    }
    *c = cosf(th) * mscale;
    *s = sinf(th) * mscale;
}

}  // namespace cbx
