// k_batch.hip -- several independent ops in one kernel launch.
//
// Every workgroup (256 lanes) finds its op by scanning the ops' first-block
// offsets (scalar, in kernel-argument memory) and runs that op's body on
// its local block index.  The bodies are the standalone kernels' bodies
// (same arithmetic, bit-identical results): wave-per-row norms (4 rows per
// workgroup), full-grid element-wise ops (256 vectors per workgroup), RoPE
// with the token's cos/sin row in LDS (one token per workgroup), row gathers
// (one row per workgroup) and the fused embedding + LayerNorm (4 tokens per
// workgroup).  Launching them together pays the fixed dispatch cost once.
#include "cbx_gnsplit.h"
#include "cbx_normrope.h"
#include "cbx_rowops.h"

namespace cbx {
namespace {

constexpr int kThreads = 256;
constexpr int kRopeMaxHalf = 256;

// ---- norms: wave per row ----------------------------------------------------
template <typename T, int NV, int KIND, bool ACT>
__device__ __forceinline__ void b_norm_row(const BOp& op, int64_t row, int lane, const uint16_t* tab) {
    const int64_t ne0 = op.ne0;
    const char* xr = op.t[0].p + row * op.t[0].nb1;
    char* yr = op.t[6].p + row * op.t[6].nb1;
    const float* w = reinterpret_cast<const float*>(op.t[1].p);
    const float* b = reinterpret_cast<const float*>(op.t[2].p);
    // branch-free affine loads (a missing w or b reads the GELU table, 64K
    // floats, instead): with `if (w)` the compiler sinks them past the
    // reduction, adding their latency to the row's chain
    Affine<NV> af;
    af.load_sel(w, b, reinterpret_cast<const float*>(tab), lane, ne0);
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        v[k] = Elt<T>::load4(xr + (j < ne0 ? j : 0) * Elt<T>::size);
    }
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if ((lane + 64 * k) * 4 >= ne0) v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float scale = wave_row_scale<NV, KIND>(v, lane, ne0, op.eps);
    if (ACT && op.act != CBX_UNARY_NONE) {
        wave_row_store<T, NV, true>(v, lane, ne0, scale, af, w != nullptr, b != nullptr, op.act, tab, yr);
    } else {
        wave_row_store<T, NV, false>(v, lane, ne0, scale, af, w != nullptr, b != nullptr, op.act, tab, yr);
    }
}

template <typename T, int KIND, bool ACT>
__device__ __forceinline__ void b_norm_nv(const BOp& op, int64_t row, int lane, const uint16_t* tab) {
    switch (op.nv) {
        case 1: b_norm_row<T, 1, KIND, ACT>(op, row, lane, tab); break;
        case 2: b_norm_row<T, 2, KIND, ACT>(op, row, lane, tab); break;
        default: b_norm_row<T, 4, KIND, ACT>(op, row, lane, tab); break;
    }
}

// One row a workgroup, its 4 waves holding a quarter of it each (rows of
// 1024 = 4 x 64 lanes x one float4): few rows then still give the SIMDs
// work, where one wave a row left a 64-row step on 16 workgroups.
template <typename T, int KIND, bool ACT>
__device__ __forceinline__ void b_norm_row4(const BOp& op, int64_t row, const uint16_t* tab, double* lds) {
    const int64_t ne0 = op.ne0;
    const int lane4 = threadIdx.x;   // wave w: float4s [64w, 64w + 64)
    const char* xr = op.t[0].p + row * op.t[0].nb1;
    char* yr = op.t[6].p + row * op.t[6].nb1;
    const float* w = reinterpret_cast<const float*>(op.t[1].p);
    const float* b = reinterpret_cast<const float*>(op.t[2].p);
    Affine<1> af;
    af.load_sel(w, b, reinterpret_cast<const float*>(tab), lane4, ne0);
    float4 v[1];
    const int64_t j = lane4 * 4;
    v[0] = Elt<T>::load4(xr + (j < ne0 ? j : 0) * Elt<T>::size);
    if (j >= ne0) v[0] = make_float4(0.f, 0.f, 0.f, 0.f);
    const float scale = row_scale_w<1, KIND, 4>(v, lane4, ne0, op.eps, lds);
    if (ACT && op.act != CBX_UNARY_NONE) {
        wave_row_store<T, 1, true>(v, lane4, ne0, scale, af, w != nullptr, b != nullptr, op.act, tab, yr);
    } else {
        wave_row_store<T, 1, false>(v, lane4, ne0, scale, af, w != nullptr, b != nullptr, op.act, tab, yr);
    }
}

// T: the element type of a norm body (one of the two when the kernel has
// only that one compiled in, else chosen by the op).
template <bool F32, bool F16, typename Body>
__device__ __forceinline__ void by_type(bool f16, Body body) {
    if constexpr (F16) {
        if (f16 || !F32) {
            body(uint16_t{});
            return;
        }
    }
    if constexpr (F32) body(float{});
}

// NB: which of the f32 (bit 0) and f16 (bit 1) norms, and (bit 2) the
// activation epilogue (without it the kernel holds no activation code and
// the host sends no norm with an activation)
template <uint32_t NB>
__device__ __forceinline__ void b_norm(const BOp& op, uint32_t lb, const uint16_t* tab, double* lds) {
    constexpr bool F32 = (NB & 1u) != 0, F16 = (NB & 2u) != 0, ACT = (NB & 4u) != 0;
    const bool f16 = op.t_x == CBX_TYPE_F16;
    const bool ln = op.kind == CBX_OP_LAYER_NORM;
    if (op.aux3 == 4) {   // one row a workgroup (rows <= 1024 elements, nv == 4)
        const int64_t row = lb;
        by_type<F32, F16>(f16, [&](auto t) {
            using T = decltype(t);
            if (ln) b_norm_row4<T, NORM_LN, ACT>(op, row, tab, lds);
            else b_norm_row4<T, NORM_RMS, ACT>(op, row, tab, lds);
        });
        return;
    }
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(lb) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= op.rows) return;   // uniform per wave
    by_type<F32, F16>(f16, [&](auto t) {
        using T = decltype(t);
        if (ln) b_norm_nv<T, NORM_LN, ACT>(op, row, lane, tab);
        else b_norm_nv<T, NORM_RMS, ACT>(op, row, lane, tab);
    });
}

// ---- element-wise: one 4-vector per lane --------------------------------------
__device__ __forceinline__ float b_unary1(int op, float x, const uint16_t* tab, float param) {
    if (op == CBX_UNARY_GELU) return act_gelu_fast(tab, x);
    return apply_act(op, x, tab, param);
}

// Two 4-vectors a lane (aux3 == 2; f32, not the f16 table path): half the
// workgroups, so that a large element-wise op fits the CUs in one round
// beside the other ops of its launch.  Both loads issue first; the same
// arithmetic per element as one vector a lane.
__device__ __forceinline__ void b_unary_f32_x2(const BOp& op, uint32_t lb, const uint16_t* tab) {
    const int64_t i0 = static_cast<int64_t>(lb) * (2 * kThreads) + threadIdx.x;
    const int64_t i1 = i0 + kThreads;
    const int64_t n = op.rows, n4 = n >> 2;
    const int fn = op.kind == CBX_OP_LEAKY_RELU ? UNARY_LEAKY : op.act;
    const char* x = op.t[0].p;
    char* y = op.t[6].p;
    const float4 v0 = Stream<float>::load4(x + (i0 < n4 ? i0 : 0) * 16);
    const float4 v1 = Stream<float>::load4(x + (i1 < n4 ? i1 : 0) * 16);
    float4 o0, o1;
    if (fn == CBX_UNARY_GELU) {
        o0 = act_gelu_fast4(tab, v0);
        o1 = act_gelu_fast4(tab, v1);
    } else {
        o0 = make_float4(b_unary1(fn, v0.x, tab, op.param), b_unary1(fn, v0.y, tab, op.param),
                         b_unary1(fn, v0.z, tab, op.param), b_unary1(fn, v0.w, tab, op.param));
        o1 = make_float4(b_unary1(fn, v1.x, tab, op.param), b_unary1(fn, v1.y, tab, op.param),
                         b_unary1(fn, v1.z, tab, op.param), b_unary1(fn, v1.w, tab, op.param));
    }
    if (i0 < n4) Stream<float>::store4(y + i0 * 16, o0);
    if (i1 < n4) Stream<float>::store4(y + i1 * 16, o1);
    for (int64_t i : {i0, i1}) {
        if (i == n4) {
            for (int64_t j = n4 * 4; j < n; j++) {
                Elt<float>::store1(y + j * 4, b_unary1(fn, Elt<float>::load1(x + j * 4), tab, op.param));
            }
        }
    }
}

template <typename T>
__device__ __forceinline__ void b_unary_t(const BOp& op, uint32_t lb, const uint16_t* tab) {
    if constexpr (std::is_same<T, float>::value) {
        if (op.aux3 == 2) {
            b_unary_f32_x2(op, lb, tab);
            return;
        }
    }
    const int64_t i = static_cast<int64_t>(lb) * kThreads + threadIdx.x;
    const int64_t n = op.rows, n4 = n >> 2;
    const int fn = op.kind == CBX_OP_LEAKY_RELU ? UNARY_LEAKY : op.act;
    const char* x = op.t[0].p;
    char* y = op.t[6].p;
    constexpr int es = Elt<T>::size;
    if (i < n4) {
        if (std::is_same<T, uint16_t>::value && fn == CBX_UNARY_GELU) {
            const cbx_u2v raw = __builtin_nontemporal_load(reinterpret_cast<const cbx_u2v*>(x + i * 8));
            cbx_u2v o;
            o.x = tab[raw.x & 0xffffu] | (static_cast<uint32_t>(tab[raw.x >> 16]) << 16);
            o.y = tab[raw.y & 0xffffu] | (static_cast<uint32_t>(tab[raw.y >> 16]) << 16);
            __builtin_nontemporal_store(o, reinterpret_cast<cbx_u2v*>(y + i * 8));
        } else {
            const float4 v = Stream<T>::load4(x + i * 4 * es);
            float4 o;
            if (fn == CBX_UNARY_GELU) {
                o = act_gelu_fast4(tab, v);
            } else {
                o.x = b_unary1(fn, v.x, tab, op.param);
                o.y = b_unary1(fn, v.y, tab, op.param);
                o.z = b_unary1(fn, v.z, tab, op.param);
                o.w = b_unary1(fn, v.w, tab, op.param);
            }
            Stream<T>::store4(y + i * 4 * es, o);
        }
    } else if (i == n4) {
        for (int64_t j = n4 * 4; j < n; j++) {
            if (std::is_same<T, uint16_t>::value && fn == CBX_UNARY_GELU) {
                *reinterpret_cast<uint16_t*>(y + j * 2) = tab[*reinterpret_cast<const uint16_t*>(x + j * 2)];
            } else {
                Elt<T>::store1(y + j * es, b_unary1(fn, Elt<T>::load1(x + j * es), tab, op.param));
            }
        }
    }
}

template <typename T>
__device__ __forceinline__ void b_swiglu_t(const BOp& op, uint32_t lb) {
    const int64_t i = static_cast<int64_t>(lb) * kThreads + threadIdx.x;
    const int64_t n = op.rows, n4 = n >> 2;
    const char* g = op.t[0].p;
    const char* u = op.t[1].p;
    char* y = op.t[6].p;
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

__device__ __forceinline__ float b_snake1(float xv, float a, float ai) { return snake_elem(xv, a, ai); }

__device__ __forceinline__ void b_snake(const BOp& op, uint32_t lb) {
    const uint32_t i = lb * kThreads + threadIdx.x;
    const uint32_t n4 = static_cast<uint32_t>(op.rows >> 2);
    if (i >= n4) return;
    const uint32_t C = static_cast<uint32_t>(op.aux), cmask = static_cast<uint32_t>(op.aux2);
    const float* a = reinterpret_cast<const float*>(op.t[1].p);
    const float* ai = reinterpret_cast<const float*>(op.t[2].p);
    const float4 v = Stream<float>::load4(op.t[0].p + 16ull * i);
    float4 o;
    if (op.act) {   // alpha along ne0
        const uint32_t c = cmask ? (4u * i) & cmask : (4u * i) % C;
        const float4 av = *reinterpret_cast<const float4*>(a + c);
        const float4 iv = *reinterpret_cast<const float4*>(ai + c);
        o.x = b_snake1(v.x, av.x, iv.x);
        o.y = b_snake1(v.y, av.y, iv.y);
        o.z = b_snake1(v.z, av.z, iv.z);
        o.w = b_snake1(v.w, av.w, iv.w);
    } else {        // alpha per row
        const uint32_t row = i / static_cast<uint32_t>(op.aux3);
        const uint32_t c = cmask ? row & cmask : row % C;
        const float av = a[c], iv = ai[c];
        o.x = b_snake1(v.x, av, iv);
        o.y = b_snake1(v.y, av, iv);
        o.z = b_snake1(v.z, av, iv);
        o.w = b_snake1(v.w, av, iv);
    }
    Stream<float>::store4(op.t[6].p + 16ull * i, o);
}

// ---- rope: one token per workgroup ------------------------------------------------
// Four rotation pairs a lane: NEOX pairs m..m+3 are two 4-element vectors of
// the head (at m and m + n_dims/2), NORMAL pairs m..m+3 the 8 elements from
// 2m; their cos/sin are two 16-byte loads from the table row of the
// token's position (no staging: the row is in L2 after the first lane).
// Same products and roundings as the one-pair-a-lane form below.
template <typename T>
__device__ __forceinline__ void b_rope_vec(const BOp& op, uint32_t t) {
    const uint32_t half = static_cast<uint32_t>(op.rp.n_dims / 2);
    const uint32_t heads = static_cast<uint32_t>(op.aux), ne2 = static_cast<uint32_t>(op.aux2);
    const uint32_t n_tail = static_cast<uint32_t>(op.ne0 - op.rp.n_dims);
    const int32_t p = *reinterpret_cast<const int32_t*>(op.t[1].p + (t % ne2) * op.t[1].nb1);
    const bool in_tab = p >= 0 && p < op.n_pos;
    const float2* tr = reinterpret_cast<const float2*>(op.table) + static_cast<int64_t>(in_tab ? p : 0) * half;
    constexpr int es = Elt<T>::size;
    const char* xt = op.t[0].p + static_cast<int64_t>(t) * heads * op.t[0].nb1;
    char* yt = op.t[6].p + static_cast<int64_t>(t) * heads * op.t[6].nb1;
    const uint32_t per_head = half / 4;
    const bool neox = op.rp.mode == 2;
    for (uint32_t q = threadIdx.x; q < heads * per_head; q += kThreads) {
        const uint32_t h = q / per_head;
        const uint32_t m = (q - h * per_head) * 4;
        const char* xr = xt + h * op.t[0].nb1;
        char* yr = yt + h * op.t[6].nb1;
        const uint32_t ia = neox ? m : 2 * m, ib = neox ? m + half : 2 * m + 4;
        const float4 xa = Elt<T>::load4(xr + ia * es);
        const float4 xb = Elt<T>::load4(xr + ib * es);
        float2 c[4];
        if (in_tab) {
            const float4 c01 = *reinterpret_cast<const float4*>(tr + m);
            const float4 c23 = *reinterpret_cast<const float4*>(tr + m + 2);
            c[0] = make_float2(c01.x, c01.y);
            c[1] = make_float2(c01.z, c01.w);
            c[2] = make_float2(c23.x, c23.y);
            c[3] = make_float2(c23.z, c23.w);
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) rope_cos_sin_dev(p, static_cast<int>(m) + e, op.rp, op.ff, &c[e].x, &c[e].y);
        }
        float4 ya, yb;
        if (neox) {   // y[i] = x0 cos - x1 sin, y[i + half] = x0 sin + x1 cos
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x0 = get(xa, e), x1 = get(xb, e);
                set(ya, e, x0 * c[e].x - x1 * c[e].y);
                set(yb, e, x0 * c[e].y + x1 * c[e].x);
            }
        } else {      // pairs (2k, 2k + 1)
            ya = make_float4(xa.x * c[0].x - xa.y * c[0].y, xa.x * c[0].y + xa.y * c[0].x,
                             xa.z * c[1].x - xa.w * c[1].y, xa.z * c[1].y + xa.w * c[1].x);
            yb = make_float4(xb.x * c[2].x - xb.y * c[2].y, xb.x * c[2].y + xb.y * c[2].x,
                             xb.z * c[3].x - xb.w * c[3].y, xb.z * c[3].y + xb.w * c[3].x);
        }
        Elt<T>::store4(yr + ia * es, ya);
        Elt<T>::store4(yr + ib * es, yb);
    }
    for (uint32_t q = threadIdx.x; q < heads * n_tail; q += kThreads) {
        const uint32_t h = q / n_tail;
        const uint32_t j = static_cast<uint32_t>(op.rp.n_dims) + (q - h * n_tail);
        *reinterpret_cast<T*>(yt + h * op.t[6].nb1 + j * es) = *reinterpret_cast<const T*>(xt + h * op.t[0].nb1 + j * es);
    }
}

template <typename T>
__device__ __forceinline__ void b_rope_t(const BOp& op, uint32_t lb, float2* cs) {
    if (op.nv == 1) {
        b_rope_vec<T>(op, lb);
        return;
    }
    const uint32_t t = lb;                        // token index over ne2 * ne3
    const uint32_t half = static_cast<uint32_t>(op.rp.n_dims / 2);
    const uint32_t heads = static_cast<uint32_t>(op.aux), ne2 = static_cast<uint32_t>(op.aux2);
    const uint32_t n_tail = static_cast<uint32_t>(op.ne0 - op.rp.n_dims);
    const int32_t p = *reinterpret_cast<const int32_t*>(op.t[1].p + (t % ne2) * op.t[1].nb1);
    const float2* table = reinterpret_cast<const float2*>(op.table);
    for (uint32_t k = threadIdx.x; k < half; k += kThreads) {
        if (p >= 0 && p < op.n_pos) {
            cs[k] = table[static_cast<int64_t>(p) * half + k];
        } else {
            float c, s;
            rope_cos_sin_dev(p, static_cast<int>(k), op.rp, op.ff, &c, &s);
            cs[k] = make_float2(c, s);
        }
    }
    __syncthreads();
    constexpr int es = Elt<T>::size;
    const char* xt = op.t[0].p + static_cast<int64_t>(t) * heads * op.t[0].nb1;
    char* yt = op.t[6].p + static_cast<int64_t>(t) * heads * op.t[6].nb1;
    for (uint32_t q = threadIdx.x; q < heads * half; q += kThreads) {
        const uint32_t h = q / half;
        const uint32_t k = q - h * half;
        const char* xr = xt + h * op.t[0].nb1;
        char* yr = yt + h * op.t[6].nb1;
        const uint32_t ia = op.rp.mode == 2 ? k : 2 * k;
        const uint32_t ib = op.rp.mode == 2 ? k + half : 2 * k + 1;
        const float x0 = Elt<T>::load1(xr + ia * es);
        const float x1 = Elt<T>::load1(xr + ib * es);
        const float2 c = cs[k];
        Elt<T>::store1(yr + ia * es, x0 * c.x - x1 * c.y);
        Elt<T>::store1(yr + ib * es, x0 * c.y + x1 * c.x);
    }
    for (uint32_t q = threadIdx.x; q < heads * n_tail; q += kThreads) {
        const uint32_t h = q / n_tail;
        const uint32_t j = static_cast<uint32_t>(op.rp.n_dims) + (q - h * n_tail);
        *reinterpret_cast<T*>(yt + h * op.t[6].nb1 + j * es) = *reinterpret_cast<const T*>(xt + h * op.t[0].nb1 + j * es);
    }
}

// ---- gathers -------------------------------------------------------------------------
template <int TYPE>
__device__ __forceinline__ float4 b_load_row4(const BOp& op, const char* row, int64_t j) {
    return load_table4<TYPE>(row, j);
}

template <int TYPE, int TYPE2>
__device__ __forceinline__ void b_gather_t(const BOp& op, uint32_t lb, uint32_t* err) {
    const int64_t r = lb;
    const int32_t id = *reinterpret_cast<const int32_t*>(op.t[1].p + r * op.t[1].nb1);
    int32_t id2 = 0;
    bool ok = id >= 0 && id < op.aux;
    if constexpr (TYPE2 >= 0) {
        id2 = *reinterpret_cast<const int32_t*>(op.t[3].p + r * op.t[3].nb1);
        ok = ok && id2 >= 0 && id2 < op.aux2;
    }
    float* d = reinterpret_cast<float*>(op.t[6].p + r * op.t[6].nb1);
    if (!ok) {
        for (int64_t j = threadIdx.x; j < op.ne0; j += kThreads) d[j] = 0.0f;
        if (threadIdx.x == 0) atomicOr(err, static_cast<uint32_t>(DEV_ERR_ROW_INDEX));
        return;
    }
    const char* s1 = op.t[0].p + id * op.t[0].nb1;
    const char* s2 = TYPE2 >= 0 ? op.t[2].p + id2 * op.t[2].nb1 : nullptr;
    for (int64_t j = threadIdx.x * 4; j < op.ne0; j += kThreads * 4) {
        float4 v = load_table4<TYPE>(s1, j);
        if constexpr (TYPE2 >= 0) {
            const float4 q = load_table4<TYPE2>(s2, j);
            v = make_float4(v.x + q.x, v.y + q.y, v.z + q.z, v.w + q.w);
        }
        *reinterpret_cast<float4*>(d + j) = v;
    }
}

template <int TYPE, int TYPE2, int NV>
__device__ __forceinline__ void b_embed_ln_t(const BOp& op, uint32_t lb, uint32_t* err) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(lb) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (t >= op.rows) return;   // uniform per wave
    const int64_t ne0 = op.ne0;
    const int32_t id = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int32_t*>(op.t[1].p + t * op.t[1].nb1));
    const int32_t id2 = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int32_t*>(op.t[3].p + t * op.t[3].nb1));
    char* yr = op.t[7].p + t * op.t[7].nb1;
    char* hr = op.t[6].p ? op.t[6].p + t * op.t[6].nb1 : nullptr;
    const float* w = reinterpret_cast<const float*>(op.t[4].p);
    const float* b = reinterpret_cast<const float*>(op.t[5].p);
    Affine<NV> af;
    af.load_sel(w, b, reinterpret_cast<const float*>(op.table), lane, ne0);
    const bool bad = id < 0 || id >= op.aux || id2 < 0 || id2 >= op.aux2;
    const int64_t r1 = bad ? 0 : id, r2 = bad ? 0 : id2;
    embed_ln_row<TYPE, TYPE2, NV>(op.t[0].p + r1 * op.t[0].nb1, op.t[2].p + r2 * op.t[2].nb1, af, w != nullptr,
                                  b != nullptr, hr, yr, ne0, op.eps, lane, bad, err);
}

template <int TYPE>
__device__ __forceinline__ void b_gather_1(const BOp& op, uint32_t lb, uint32_t* err) {
    if (op.t[2].p == nullptr) b_gather_t<TYPE, -1>(op, lb, err);
    else if (op.t_x2 == CBX_TYPE_F32) b_gather_t<TYPE, CBX_TYPE_F32>(op, lb, err);
    else if (op.t_x2 == CBX_TYPE_F16) b_gather_t<TYPE, CBX_TYPE_F16>(op, lb, err);
    else b_gather_t<TYPE, CBX_TYPE_Q8_0>(op, lb, err);
}

// One token a workgroup, its 4 waves holding a quarter of the row each
// (rows of 513..1024 elements, aux3 == 4): the standalone kernel's few-row
// form, for launches whose tokens are few against the CUs (a 512-token
// prefill), where one wave a token walks the whole row's chain alone.
template <int TYPE, int TYPE2>
__device__ __forceinline__ void b_embed_ln_w4(const BOp& op, uint32_t lb, uint32_t* err, double* lds) {
    const int lane = threadIdx.x;   // wave w: float4s [64w, 64w + 64)
    const int64_t t = lb;
    const int64_t ne0 = op.ne0;
    const int32_t id = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int32_t*>(op.t[1].p + t * op.t[1].nb1));
    const int32_t id2 = __builtin_amdgcn_readfirstlane(*reinterpret_cast<const int32_t*>(op.t[3].p + t * op.t[3].nb1));
    char* yr = op.t[7].p + t * op.t[7].nb1;
    char* hr = op.t[6].p ? op.t[6].p + t * op.t[6].nb1 : nullptr;
    const float* w = reinterpret_cast<const float*>(op.t[4].p);
    const float* b = reinterpret_cast<const float*>(op.t[5].p);
    Affine<1> af;
    af.load_sel(w, b, reinterpret_cast<const float*>(op.table), lane, ne0);
    const bool bad = id < 0 || id >= op.aux || id2 < 0 || id2 >= op.aux2;
    const int64_t r1 = bad ? 0 : id, r2 = bad ? 0 : id2;
    embed_ln_row<TYPE, TYPE2, 1, 4>(op.t[0].p + r1 * op.t[0].nb1, op.t[2].p + r2 * op.t[2].nb1, af, w != nullptr,
                                    b != nullptr, hr, yr, ne0, op.eps, lane, bad, err, lds);
}

template <int TYPE, int TYPE2>
__device__ __forceinline__ void b_embed_nv(const BOp& op, uint32_t lb, uint32_t* err, double* lds) {
    if (op.aux3 == 4) {
        b_embed_ln_w4<TYPE, TYPE2>(op, lb, err, lds);
        return;
    }
    switch (op.nv) {
        case 1: b_embed_ln_t<TYPE, TYPE2, 1>(op, lb, err); break;
        case 2: b_embed_ln_t<TYPE, TYPE2, 2>(op, lb, err); break;
        default: b_embed_ln_t<TYPE, TYPE2, 4>(op, lb, err); break;
    }
}

template <int TYPE>
__device__ __forceinline__ void b_embed_1(const BOp& op, uint32_t lb, uint32_t* err, double* lds) {
    if (op.t_x2 == CBX_TYPE_F32) b_embed_nv<TYPE, CBX_TYPE_F32>(op, lb, err, lds);
    else if (op.t_x2 == CBX_TYPE_F16) b_embed_nv<TYPE, CBX_TYPE_F16>(op, lb, err, lds);
    else b_embed_nv<TYPE, CBX_TYPE_Q8_0>(op, lb, err, lds);
}

// ---- GroupNorm (split reduction): one chunk a workgroup -------------------------------
// The op's block range starts at a multiple of 8 (GroupNorm ops come first in
// a launch), so the body's index mod 8 is the XCD's, as in its own kernel.
// gn is read where it lies in the argument segment: it shares its bytes with
// the tensor slots of the workgroup's copy of the op, and reading one copy
// through both views would keep that copy in memory.
__device__ __forceinline__ void b_group_norm(const GnSplit& gn, int nv, int64_t act, uint32_t lb) {
    if (act == 2) {   // Mish
        switch (nv) {
            case 1: gn_split_body<1, 2>(gn, lb); break;
            case 2: gn_split_body<2, 2>(gn, lb); break;
            default: gn_split_body<4, 2>(gn, lb); break;
        }
    } else {
        switch (nv) {
            case 1: gn_split_body<1, 0>(gn, lb); break;
            case 2: gn_split_body<2, 0>(gn, lb); break;
            default: gn_split_body<4, 0>(gn, lb); break;
        }
    }
}

// ---- LayerNorm + RoPE: one wave a token row, four rows a workgroup --------------------
// The rotation partners come from other lanes of the row's wave (the host
// admits only such layouts), so no LDS and no barrier.
template <int MODE, int NV>
__device__ __forceinline__ void b_ln_rope_nv(const BOp& op, uint32_t lb) {
    const uint32_t r = lb * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (r >= static_cast<uint32_t>(op.rows)) return;   // uniform per wave
    NormRopeArgs a;
    a.x = op.t[0].p;
    a.y = op.t[6].p;
    a.w = reinterpret_cast<const float*>(op.t[2].p);
    a.b = reinterpret_cast<const float*>(op.t[3].p);
    a.pos = op.t[1].p;
    a.pos_nb0 = op.t[1].nb1;
    a.table = reinterpret_cast<const float2*>(op.table);
    a.ff = op.ff;
    a.mx.nb1 = op.t[0].nb1;
    a.mx.flat = 1;
    a.my.nb1 = op.t[6].nb1;
    a.my.flat = 1;
    a.ne0 = static_cast<int32_t>(op.ne0);
    a.hd = static_cast<int32_t>(op.aux);
    a.n_tok = static_cast<uint32_t>(op.aux2);
    a.n_pos = op.n_pos;
    a.eps = op.eps;
    a.vec_cs = 1;
    a.rp = op.rp;
    ln_rope_row<NV, MODE, true, 1, true>(a, r, static_cast<int>(threadIdx.x & 63), nullptr, nullptr);
}

__device__ __forceinline__ void b_ln_rope(const BOp& op, uint32_t lb) {
    if (op.rp.mode == 2) {
        switch (op.nv) {
            case 1: b_ln_rope_nv<2, 1>(op, lb); break;
            case 2: b_ln_rope_nv<2, 2>(op, lb); break;
            default: b_ln_rope_nv<2, 4>(op, lb); break;
        }
    } else {
        switch (op.nv) {
            case 1: b_ln_rope_nv<0, 1>(op, lb); break;
            case 2: b_ln_rope_nv<0, 2>(op, lb); break;
            default: b_ln_rope_nv<0, 4>(op, lb); break;
        }
    }
}

// ---- the batch kernel ------------------------------------------------------------------
// Which op bodies a kernel compiles in (by kind and element type): the
// kernel's registers are those of its heaviest body, so each launch takes
// the smallest instantiation that covers its ops (a decode step's norms,
// RoPE, SiLU-gate and gathers fit in far fewer than the fused embedding +
// LayerNorm with its three table types).
enum : uint32_t {
    KB_NORM_F32 = 1u << 0,
    KB_NORM_F16 = 1u << 1,
    KB_UNARY_F32 = 1u << 2,
    KB_UNARY_F16 = 1u << 3,
    KB_SWIGLU_F32 = 1u << 4,
    KB_SWIGLU_F16 = 1u << 5,
    KB_ROPE_F32 = 1u << 6,
    KB_ROPE_F16 = 1u << 7,
    KB_GATHER = 1u << 8,
    KB_EMBED = 1u << 9,
    KB_SNAKE = 1u << 10,
    KB_NORM_ACT = 1u << 11,   // a norm with an activation epilogue
    KB_GROUP_NORM = 1u << 12,
    KB_LN_ROPE = 1u << 13,
    KB_ALL = (1u << 14) - 1,
};

// The op list is read in place from the kernel-argument segment (the
// pointer's origin lets the compiler use scalar constant loads); indexing the
// by-value parameter with a run-time index would copy all of it to scratch.
template <uint32_t KS>
__global__ __launch_bounds__(kThreads) void k_batch(BatchArgs args) {
    (void)args;
    __shared__ float2 cs[(KS & (KB_ROPE_F32 | KB_ROPE_F16)) ? kRopeMaxHalf : 1];
    __shared__ double lds[8];
    const BatchArgs* a = (const BatchArgs*)(const void*)__builtin_amdgcn_kernarg_segment_ptr();
    const uint32_t b = blockIdx.x;
    // the op owning this workgroup: every first-block offset is read, in one
    // round of scalar loads (the host fills the entries past the last op
    // with UINT32_MAX, so no test of the op count stands between them: with
    // one, the compiler loaded the offsets one dependent round at a time)
    uint32_t blk[kBatchMaxOps];
#pragma unroll
    for (int k = 0; k < kBatchMaxOps; k++) blk[k] = a->blk0[k];
    int i = 0;
    uint32_t base = 0;   // blk0[0] == 0
#pragma unroll
    for (int k = 1; k < kBatchMaxOps; k++) {
        const bool in = b >= blk[k];
        i = in ? k : i;
        base = in ? blk[k] : base;
    }
    // the op's fields, copied before any branch on them: the copy's scalar
    // loads issue together, where reads under each branch (kind, layout,
    // type) came as dependent rounds of argument loads before the first
    // load of data
    const BOp op = a->op[i];
    const uint32_t lb = b - base;
    uint32_t* err = a->err;
    const uint16_t* tab = reinterpret_cast<const uint16_t*>(op.table);
    const bool f16 = op.t_x == CBX_TYPE_F16;
    switch (op.kind) {
        case CBX_OP_LAYER_NORM:
        case CBX_OP_RMS_NORM:
            if constexpr ((KS & (KB_NORM_F32 | KB_NORM_F16)) != 0) {
                b_norm<(KS & (KB_NORM_F32 | KB_NORM_F16)) | ((KS & KB_NORM_ACT) ? 4u : 0u)>(op, lb, tab, lds);
            }
            break;
        case CBX_OP_UNARY:
        case CBX_OP_LEAKY_RELU:
            if constexpr ((KS & KB_UNARY_F16) != 0) {
                if (f16) {
                    b_unary_t<uint16_t>(op, lb, tab);
                    break;
                }
            }
            if constexpr ((KS & KB_UNARY_F32) != 0) {
                if (!f16) b_unary_t<float>(op, lb, tab);
            }
            break;
        case CBX_OP_SWIGLU:
            if constexpr ((KS & KB_SWIGLU_F16) != 0) {
                if (f16) {
                    b_swiglu_t<uint16_t>(op, lb);
                    break;
                }
            }
            if constexpr ((KS & KB_SWIGLU_F32) != 0) {
                if (!f16) b_swiglu_t<float>(op, lb);
            }
            break;
        case CBX_OP_ROPE:
            if constexpr ((KS & KB_ROPE_F16) != 0) {
                if (f16) {
                    b_rope_t<uint16_t>(op, lb, cs);
                    break;
                }
            }
            if constexpr ((KS & KB_ROPE_F32) != 0) {
                if (!f16) b_rope_t<float>(op, lb, cs);
            }
            break;
        case CBX_OP_GET_ROWS:
            if constexpr ((KS & KB_GATHER) != 0) {
                if (op.t_x == CBX_TYPE_F32) b_gather_1<CBX_TYPE_F32>(op, lb, err);
                else if (op.t_x == CBX_TYPE_F16) b_gather_1<CBX_TYPE_F16>(op, lb, err);
                else b_gather_1<CBX_TYPE_Q8_0>(op, lb, err);
            }
            break;
        case CBX_OP_GET_ROWS_ADD_LAYER_NORM:
            if constexpr ((KS & KB_EMBED) != 0) {
                if (op.t_x == CBX_TYPE_F32) b_embed_1<CBX_TYPE_F32>(op, lb, err, lds);
                else if (op.t_x == CBX_TYPE_F16) b_embed_1<CBX_TYPE_F16>(op, lb, err, lds);
                else b_embed_1<CBX_TYPE_Q8_0>(op, lb, err, lds);
            }
            break;
        case CBX_OP_SNAKE:
            if constexpr ((KS & KB_SNAKE) != 0) b_snake(op, lb);
            break;
        case CBX_OP_GROUP_NORM:
            if constexpr ((KS & KB_GROUP_NORM) != 0) b_group_norm(a->op[i].gn, op.nv, op.aux, lb);
            break;
        case CBX_OP_LAYER_NORM_ROPE:
            if constexpr ((KS & KB_LN_ROPE) != 0) b_ln_rope(op, lb);
            break;
        default:
            break;
    }
}

// The bodies an op needs.
uint32_t op_bits(const BOp& op) {
    const bool f16 = op.t_x == CBX_TYPE_F16;
    switch (op.kind) {
        case CBX_OP_LAYER_NORM:
        case CBX_OP_RMS_NORM: return (f16 ? KB_NORM_F16 : KB_NORM_F32) | (op.act != CBX_UNARY_NONE ? KB_NORM_ACT : 0u);
        case CBX_OP_UNARY:
        case CBX_OP_LEAKY_RELU: return f16 ? KB_UNARY_F16 : KB_UNARY_F32;
        case CBX_OP_SWIGLU: return f16 ? KB_SWIGLU_F16 : KB_SWIGLU_F32;
        case CBX_OP_ROPE: return f16 ? KB_ROPE_F16 : KB_ROPE_F32;
        case CBX_OP_GET_ROWS: return KB_GATHER;
        case CBX_OP_GET_ROWS_ADD_LAYER_NORM: return KB_EMBED;
        case CBX_OP_SNAKE: return KB_SNAKE;
        case CBX_OP_GROUP_NORM: return KB_GROUP_NORM;
        case CBX_OP_LAYER_NORM_ROPE: return KB_LN_ROPE;
        default: return KB_ALL;
    }
}

// The instantiations, smallest first: the decode step in f32 (norm, RoPE,
// SiLU-gate, gather), the 64-stream f16 step (the same in f16 with the Q8_0
// gather), the prefill's embedding + LayerNorm with GELU, the CFM flow
// step's GroupNorms with LayerNorm + RoPE, the element-wise ops, snake, and
// everything.
template <uint32_t KS>
void go(const BatchArgs& a, uint32_t total_blocks, hipStream_t s) {
    hipLaunchKernelGGL(k_batch<KS>, dim3(total_blocks), dim3(kThreads), 0, s, a);
}

constexpr uint32_t kDecodeF32 = KB_NORM_F32 | KB_ROPE_F32 | KB_SWIGLU_F32 | KB_GATHER;
constexpr uint32_t kDecodeF16 = KB_NORM_F16 | KB_ROPE_F16 | KB_SWIGLU_F16 | KB_GATHER;
constexpr uint32_t kPrefill = KB_EMBED | KB_UNARY_F32;
constexpr uint32_t kFlow = KB_GROUP_NORM | KB_LN_ROPE;

}  // namespace

int launch_batch(const BatchArgs& a, uint32_t total_blocks, hipStream_t s) {
    uint32_t need = 0;
    for (int i = 0; i < a.n; i++) need |= op_bits(a.op[i]);
    auto covers = [need](uint32_t ks) { return (need & ~ks) == 0; };
    if (covers(kDecodeF32)) go<kDecodeF32>(a, total_blocks, s);
    else if (covers(kDecodeF16)) go<kDecodeF16>(a, total_blocks, s);
    else if (covers(kPrefill)) go<kPrefill>(a, total_blocks, s);
    else if (covers(KB_GROUP_NORM)) go<KB_GROUP_NORM>(a, total_blocks, s);
    else if (covers(KB_LN_ROPE)) go<KB_LN_ROPE>(a, total_blocks, s);
    else if (covers(kFlow)) go<kFlow>(a, total_blocks, s);
    else if (covers(KB_UNARY_F32 | KB_UNARY_F16)) go<KB_UNARY_F32 | KB_UNARY_F16>(a, total_blocks, s);
    else if (covers(KB_SNAKE)) go<KB_SNAKE>(a, total_blocks, s);
    else go<KB_ALL>(a, total_blocks, s);
    return check_launch("run_ops");
}

}  // namespace cbx
