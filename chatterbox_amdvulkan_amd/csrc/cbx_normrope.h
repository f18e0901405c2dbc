// cbx_normrope.h -- LayerNorm (+ affine) of a token row followed by RoPE of
// the row viewed as heads: the row body shared by the standalone kernel
// (k_norm_rope.hip) and the op batch (k_batch.hip).  Device code only.
#pragma once

#include "cbx_rowops.h"

namespace cbx {
namespace {

constexpr int kRowMax = 1024;

struct NormRopeArgs {
    const char* x;
    char* y;
    const float* w;
    const float* b;
    const char* pos;
    const float2* table;
    const float* ff;
    RowMap mx, my;
    int64_t pos_nb0;
    int32_t ne0, hd;       // row length, head size (rotation row length)
    uint32_t n_tok;        // x.ne1: tokens per batch item (the position index)
    int32_t n_pos;
    float eps;
    int32_t vec_cs;        // 16-byte cos/sin loads: table 16-byte aligned, n_dims % 4 (NEOX: % 8) == 0
    RopeParams rp;
};

// Table slot (pair index) of head-local element i, or -1 past n_dims.
template <int MODE>
__device__ __forceinline__ int pair_of(int i, int nd, int half) {
    if (i >= nd) return -1;
    if constexpr (MODE == 2) return i < half ? i : i - half;
    return i >> 1;
}

// cos/sin of the 4 elements of a vector starting at head-local element i0
// (a multiple of 4) from the table row tr, when all 4 are rotated: NEOX's
// pairs are i0 .. i0 + 3 (or those less half), four consecutive float2 --
// two 16-byte loads; NORMAL's are i0/2, i0/2 (+1 twice) -- one.
template <int MODE>
__device__ __forceinline__ void cos_sin4(const float2* tr, int i0, int half, float2 (&cs)[4]) {
    if constexpr (MODE == 2) {
        const int m = i0 < half ? i0 : i0 - half;
        const float4 a = *reinterpret_cast<const float4*>(tr + m);
        const float4 b = *reinterpret_cast<const float4*>(tr + m + 2);
        cs[0] = make_float2(a.x, a.y);
        cs[1] = make_float2(a.z, a.w);
        cs[2] = make_float2(b.x, b.y);
        cs[3] = make_float2(b.z, b.w);
    } else {
        const float4 a = *reinterpret_cast<const float4*>(tr + (i0 >> 1));
        cs[0] = cs[1] = make_float2(a.x, a.y);
        cs[2] = cs[3] = make_float2(a.z, a.w);
    }
}

// FLAT: x and y rows at one stride each (no test of the row map before the
// loads are issued).  W waves share a row (wave w holds float4s
// [w*64*NV, (w+1)*64*NV) of it) when the rows are few.  XS: the rotation
// partners come from other lanes' registers instead of the LDS row: NORMAL
// pairs (2k, 2k+1) lie in one 4-vector; a NEOX pair is half/4 vectors
// apart, which is lane ^ (half/4) when hd/4 divides 64 and half/4 is a
// power of two (the head's vectors sit on consecutive lanes of one wave).
//
// The body of one token row r: `lane` is the row lane's first float4 (wave
// w of the row's W holds float4s [w*64*NV, (w+1)*64*NV)); `row` (kRowMax
// floats) and `lds` (2W doubles) are the workgroup's shared arrays, unused
// when XS and W == 1.
template <int NV, int MODE, bool FLAT, int W, bool XS>
__device__ __forceinline__ void ln_rope_row(const NormRopeArgs& a, uint32_t r, int lane, float* row, double* lds) {
    const int64_t ne0 = a.ne0;
    const char* xr = a.x + (FLAT ? static_cast<int64_t>(r) * a.mx.nb1 : row_at(a.mx, r));
    char* yr = a.y + (FLAT ? static_cast<int64_t>(r) * a.my.nb1 : row_at(a.my, r));
    const int nd = a.rp.n_dims, half = nd / 2;

    // position of the token (ne1 index of x); the row and affine loads go
    // out first, then the cos/sin of each of the lane's elements (table rows
    // are L2-resident), so the table latency hides under the row loads.  The
    // cos/sin are read for the position the token would have in a sequence
    // numbered 0, 1, 2, .. (the CFM and S3 transformers' positions) while
    // its position is still being read, and read again only when it
    // differs: no second round trip in the common case.
    const uint32_t tok = r % a.n_tok;
    const int32_t ps = static_cast<int32_t>(tok);
    const int32_t p = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int32_t*>(a.pos + tok * a.pos_nb0));
    Affine<NV> af;
    af.load_sel(a.w, a.b, reinterpret_cast<const float*>(yr), lane, ne0);
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        v[k] = Elt<float>::load4(xr + (j < ne0 ? j : 0) * 4);
    }
    float2 cs[NV][4];
    int i0[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        const int64_t jc = j < ne0 ? j : 0;
        // hd % 4 == 0: the vector sits in one head (32-bit: jc < 1024)
        i0[k] = static_cast<int>(static_cast<uint32_t>(jc) % static_cast<uint32_t>(a.hd));
    }
    auto table_row = [&](int32_t q) {
        const float2* tr = a.table + static_cast<int64_t>(q) * half;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            if (a.vec_cs && i0[k] + 4 <= nd) {
                cos_sin4<MODE>(tr, i0[k], half, cs[k]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int m = pair_of<MODE>(i0[k] + e, nd, half);
                    cs[k][e] = m >= 0 ? tr[m] : make_float2(0.f, 0.f);
                }
            }
        }
    };
    if (a.n_pos > 0) table_row(ps < a.n_pos ? ps : 0);   // speculative: row ps (row 0 past the table)
    if (p == ps && p < a.n_pos) {                         // uniform: the speculative row is the token's
    } else if (p >= 0 && p < a.n_pos) {
        table_row(p);
    } else {   // positions past the table: the device recurrence
#pragma unroll
        for (int k = 0; k < NV; k++) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int m = pair_of<MODE>(i0[k] + e, nd, half);
                cs[k][e] = make_float2(0.f, 0.f);
                if (m >= 0) rope_cos_sin_dev(p, m, a.rp, a.ff, &cs[k][e].x, &cs[k][e].y);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if ((lane + 64 * k) * 4 >= ne0) v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float scale = row_scale_w<NV, NORM_LN, W>(v, lane, ne0, a.eps, lds);
    const bool hw = a.w != nullptr, hb = a.b != nullptr;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        if (j < ne0) {
            float4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float t = get(v[k], e) * scale;
                if (hw) t = t * get(af.w[k], e);
                if (hb) t = t + get(af.b[k], e);
                set(o, e, t);
            }
            v[k] = o;
            if constexpr (!XS) *reinterpret_cast<float4*>(&row[j]) = o;
        }
    }
    if constexpr (XS) {
        const int dq = half >> 2;   // partner distance in vectors (NEOX)
#pragma unroll
        for (int k = 0; k < NV; k++) {
            float4 pv = v[k];
            if constexpr (MODE == 2) {   // every lane takes part in the shuffles
                pv.x = __shfl_xor(v[k].x, dq);
                pv.y = __shfl_xor(v[k].y, dq);
                pv.z = __shfl_xor(v[k].z, dq);
                pv.w = __shfl_xor(v[k].w, dq);
            }
            const int64_t j = (lane + 64 * k) * 4;
            if (j >= ne0) continue;
            float4 o = v[k];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int i = i0[k] + e;
                if (i >= nd) continue;            // past n_dims: copied
                const float2 c = cs[k][e];
                if constexpr (MODE == 2) {
                    if (i < half) set(o, e, get(v[k], e) * c.x - get(pv, e) * c.y);
                    else set(o, e, get(pv, e) * c.y + get(v[k], e) * c.x);
                } else {
                    if ((i & 1) == 0) set(o, e, get(v[k], e) * c.x - get(v[k], e + 1) * c.y);
                    else set(o, e, get(v[k], e - 1) * c.y + get(v[k], e) * c.x);
                }
            }
            Stream<float>::store4(yr + j * 4, o);
        }
        return;
    }
    __syncthreads();

#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        if (j >= ne0) continue;
        const int64_t h0 = j - i0[k];             // first element of the head
        float4 o = v[k];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int i = i0[k] + e;
            if (i >= nd) continue;                // past n_dims: copied
            const float2 c = cs[k][e];
            if constexpr (MODE == 2) {
                if (i < half) {
                    const float x0 = get(v[k], e), x1 = row[h0 + i + half];
                    set(o, e, x0 * c.x - x1 * c.y);
                } else {
                    const float x0 = row[h0 + i - half], x1 = get(v[k], e);
                    set(o, e, x0 * c.y + x1 * c.x);
                }
            } else {
                if ((i & 1) == 0) {
                    const float x0 = get(v[k], e), x1 = row[h0 + i + 1];
                    set(o, e, x0 * c.x - x1 * c.y);
                } else {
                    const float x0 = row[h0 + i - 1], x1 = get(v[k], e);
                    set(o, e, x0 * c.y + x1 * c.x);
                }
            }
        }
        Stream<float>::store4(yr + j * 4, o);
    }
}

}  // namespace
}  // namespace cbx
