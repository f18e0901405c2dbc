// k_norm.hip -- LayerNorm / RMSNorm over ne[0] with the affine multiply/add
// and an optional activation fused into the same pass: one HBM read of x,
// one write of y, per row.  Also the T3 embedding chain: token row + learned
// position row, then the first LayerNorm, in one pass.
//
// Arithmetic follows ggml-cpu exactly:
//   LN : mean = (float)(sum_f64 x) / n;  v = x - mean;
//        var = (float)(sum_f64 (v*v) / n);  y = v * (1/sqrtf(var + eps))
//   RMS: ms = (float)(sum_f64 (x*x) / n);   y = x * (1/sqrtf(ms + eps))
//   then y*w, then +b, each rounded to f32 (ggml_mul, ggml_add).
// The f64 sums use a fixed butterfly order rather than ggml's sequential
// order; the f32 values derived from them agree unless an f64 sum falls
// within ~2^-29 relative of an f32 rounding boundary.
//
// Rows of up to 4096 elements (ne0 % 4 == 0, 16-byte aligned) take one
// wave per row: each lane holds NV 4-element vectors in registers and the
// two reductions are wave-local (DPP), with no LDS or barrier.  Other rows
// take one workgroup per row (LDS combine), and rows past 8192 elements a
// three-pass loop.
#include "cbx_rowops.h"

namespace cbx {
namespace {

constexpr int kMaxThreads = 256;

// Compact arguments of the wave-per-row norm (a small argument block: its
// loads are on the path to the first row load).
struct WaveNormArgs {
    const char* x;
    char* y;
    const float* w;
    const float* b;
    const uint16_t* tab;
    RowMap mx, my;
    int32_t ne0, nr;
    float eps;
    int32_t act;
};

// WPB waves (rows) per workgroup.  With WPB == 1 the grid has exactly one
// workgroup per row, so there is no bounds check and no read of the block
// size before the loads.
// FLAT: x and y rows at one stride each, so a row's address is one multiply
// and nothing tests an argument before the loads are issued.
template <typename T, int NV, int KIND, bool ACT, int WPB, bool FLAT>
__global__ __launch_bounds__(64 * WPB) void k_row_norm_wave(WaveNormArgs a) {
    // every field the loads need in the first batch of argument loads (left
    // alone, the compiler loads the row count first and the rest after the
    // bounds test, or the row maps after the affine pointers)
    arg_now(a.x); arg_now(a.y); arg_now(a.w); arg_now(a.b); arg_now(a.tab);
    arg_now(reinterpret_cast<const void*>(a.mx.nb1)); arg_now(reinterpret_cast<const void*>(a.my.nb1));
    arg_now(static_cast<uint32_t>(a.ne0)); arg_now(static_cast<uint32_t>(a.nr));
    if constexpr (!FLAT) {
        arg_now(reinterpret_cast<const void*>(a.mx.nb2)); arg_now(reinterpret_cast<const void*>(a.mx.nb3));
        arg_now(reinterpret_cast<const void*>(a.my.nb2)); arg_now(reinterpret_cast<const void*>(a.my.nb3));
        arg_now(a.mx.ne1); arg_now(a.mx.ne2); arg_now(a.my.ne1); arg_now(a.my.ne2); arg_now(a.mx.flat); arg_now(a.my.flat);
    }
    const int lane = threadIdx.x & 63;
    uint32_t r = blockIdx.x;
    if constexpr (WPB > 1) {
        r = r * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (r >= static_cast<uint32_t>(a.nr)) return;   // uniform per wave
    }
    const int64_t ne0 = a.ne0;
    const char* xr = a.x + (FLAT ? static_cast<int64_t>(r) * a.mx.nb1 : row_at(a.mx, r));
    char* yr = a.y + (FLAT ? static_cast<int64_t>(r) * a.my.nb1 : row_at(a.my, r));
    // affine vectors first (L2-resident), then the row: loads are
    // unconditional (clamped address; a missing w or b reads the GELU table
    // instead), so all are in flight at once; lanes past the row end zero
    // their values afterwards
    Affine<NV> af;
    af.load_sel(a.w, a.b, reinterpret_cast<const float*>(a.tab), lane, ne0);
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
    const float scale = wave_row_scale<NV, KIND>(v, lane, ne0, a.eps);
    wave_row_store<T, NV, ACT>(v, lane, ne0, scale, af, a.w != nullptr, a.b != nullptr, a.act, a.tab, yr);
}

// ---------------------------------------------------------------------------
// T3 embedding chain: h = f32(table[ids]) + f32(pos_table[pos_ids]) (one f32
// add, t3.cpp:446-455), optionally stored, then y = LN(h)*w + b
// (t3.cpp:465-466) -- one wave per token.
// ---------------------------------------------------------------------------

struct EmbedArgs {
    View src, ids, src2, ids2, h, y;
    const float* w;
    const float* b;
    float eps;
    int64_t n_tok;
    uint32_t* err;
};

template <int TYPE, int TYPE2, int NV>
__global__ __launch_bounds__(kMaxThreads) void k_embed_norm(EmbedArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) +
                      __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (t >= a.n_tok) return;   // uniform per wave
    const int64_t ne0 = a.y.ne[0];
    int64_t i10 = t, i11 = 0, i12 = 0;
    if (a.ids.ne[1] * a.ids.ne[2] > 1) {
        const int64_t n10 = a.ids.ne[0], n11 = a.ids.ne[1];
        i12 = t / (n11 * n10);
        i11 = (t - i12 * n11 * n10) / n10;
        i10 = t - i12 * n11 * n10 - i11 * n10;
    }
    const int32_t id = __builtin_amdgcn_readfirstlane(
        *reinterpret_cast<const int32_t*>(a.ids.data + i10 * a.ids.nb[0] + i11 * a.ids.nb[1] + i12 * a.ids.nb[2]));
    const int32_t id2 = __builtin_amdgcn_readfirstlane(
        *reinterpret_cast<const int32_t*>(a.ids2.data + i10 * a.ids2.nb[0] + i11 * a.ids2.nb[1] + i12 * a.ids2.nb[2]));
    char* yr = a.y.data + i10 * a.y.nb[1] + i11 * a.y.nb[2] + i12 * a.y.nb[3];
    char* hr = a.h.data ? a.h.data + i10 * a.h.nb[1] + i11 * a.h.nb[2] + i12 * a.h.nb[3] : nullptr;
    Affine<NV> af;
    af.load_sel(a.w, a.b, reinterpret_cast<const float*>(yr), lane, ne0);
    const bool bad = id < 0 || id >= a.src.ne[1] || id2 < 0 || id2 >= a.src2.ne[1];
    const int64_t r1 = bad ? 0 : id, r2 = bad ? 0 : id2;
    const char* s1 = a.src.data + r1 * a.src.nb[1] + i11 * a.src.nb[2] + i12 * a.src.nb[3];
    const char* s2 = a.src2.data + r2 * a.src2.nb[1] + i11 * a.src2.nb[2] + i12 * a.src2.nb[3];
    embed_ln_row<TYPE, TYPE2, NV>(s1, s2, af, a.w != nullptr, a.b != nullptr, hr, yr, ne0, a.eps, lane, bad, a.err);
}

// The common layout -- 1-D contiguous ids, 2-D tables, uniformly strided
// output rows, ne0 <= 1024 -- with a compact argument block: every field is
// read by one batch of scalar loads at entry, so the id loads issue
// immediately (the general kernel's View-based arguments took a second
// dependent round of argument loads).
struct EmbedFlat {
    const char* src;
    const char* src2;
    const int32_t* ids;
    const int32_t* ids2;
    const float* w;
    const float* b;
    char* h;
    char* y;
    int64_t src_nb1, src2_nb1, h_nb1, y_nb1;
    int32_t src_rows, src2_rows, n_tok, ne0;
    float eps;
    uint32_t* err;
};

// One workgroup per token, exactly n_tok workgroups: no bounds check and no
// read of the launch's block size, so nothing waits before the argument
// loads and the id loads are issued.  W waves share the token's row (wave w
// holds float4s [w*64*NV, (w+1)*64*NV)): with few tokens (a 512-token
// prefill on 256 CUs) one wave a row leaves most SIMDs idle while each
// wave walks its chain of dependent loads and reductions.
template <int TYPE, int TYPE2, int NV, int W>
__global__ __launch_bounds__(64 * W) void k_embed_norm_flat(EmbedFlat a) {
    __shared__ double lds[2 * W];
    const int lane = (threadIdx.x >> 6) * 64 * NV + (threadIdx.x & 63);   // the lane's first float4
    const int t = static_cast<int>(blockIdx.x);
    const int32_t id = __builtin_amdgcn_readfirstlane(a.ids[t]);
    const int32_t id2 = __builtin_amdgcn_readfirstlane(a.ids2[t]);
    // the other fields by the time the ids arrive (left alone, the compiler
    // loads the row strides only after the ids: one more scalar round trip
    // before the row loads); after the id loads, which stay scalar loads
    arg_now(a.src); arg_now(a.src2); arg_now(a.w); arg_now(a.b); arg_now(a.h); arg_now(a.y);
    arg_now(reinterpret_cast<const void*>(a.src_nb1)); arg_now(reinterpret_cast<const void*>(a.src2_nb1));
    arg_now(reinterpret_cast<const void*>(a.h_nb1)); arg_now(reinterpret_cast<const void*>(a.y_nb1));
    arg_now(static_cast<uint32_t>(a.src_rows)); arg_now(static_cast<uint32_t>(a.src2_rows));
    const int64_t ne0 = a.ne0;
    char* yr = a.y + t * a.y_nb1;
    char* hr = a.h ? a.h + t * a.h_nb1 : nullptr;
    Affine<NV> af;
    af.load_sel(a.w, a.b, reinterpret_cast<const float*>(yr), lane, ne0);
    // an out-of-range id reads row 0 and zeroes the outputs after the loads
    const bool bad = id < 0 || id >= a.src_rows || id2 < 0 || id2 >= a.src2_rows;
    const int64_t r1 = bad ? 0 : id, r2 = bad ? 0 : id2;
    embed_ln_row<TYPE, TYPE2, NV, W>(a.src + r1 * a.src_nb1, a.src2 + r2 * a.src2_nb1, af, a.w != nullptr,
                                     a.b != nullptr, hr, yr, ne0, a.eps, lane, bad, a.err, lds);
}

// ---------------------------------------------------------------------------
// The T3 input with the conditioning prefix (t3.cpp:432-466):
//   seq = concat(prefix, cast(get_rows(src_a, ids_a)), cast(get_rows(src_b,
//         ids_b))) along ne1; h = seq + cast(get_rows(src2, ids2)); LN(h).
// Token t's first row comes from the segment that holds it: a prefix row
// (F32, as the conditioning encoder wrote it), or a gathered table row;
// then the embedding kernel's row body.  One workgroup per token, W waves.
// ---------------------------------------------------------------------------

struct ConcatSeg {
    const char* base;      // table (gathered) or prefix rows
    const int32_t* ids;    // nullptr: the prefix (row t - start of the segment)
    int64_t nb1;
    int32_t rows;          // table rows (id bound)
    int32_t type;
};

struct EmbedConcat {
    ConcatSeg seg[3];
    int32_t end0, end1;    // the segments hold tokens [0, end0), [end0, end1), [end1, n_tok)
    const char* src2;
    const int32_t* ids2;
    int64_t src2_nb1;
    int32_t src2_rows;
    const float* w;
    const float* b;
    char* h;
    char* y;
    int64_t h_nb1, y_nb1;
    int32_t ne0;
    float eps;
    const uint16_t* tab;
    uint32_t* err;
};

template <int TYPE, int TYPE2, int NV, int W>
__device__ __forceinline__ void concat_row(const EmbedConcat& a, const char* s1, bool bad, const Affine<NV>& af,
                                           char* hr, char* yr, int lane, double* lds) {
    const int t = static_cast<int>(blockIdx.x);
    const int32_t id2 = __builtin_amdgcn_readfirstlane(a.ids2[t]);
    const bool bad2 = bad || id2 < 0 || id2 >= a.src2_rows;
    const char* s2 = a.src2 + static_cast<int64_t>(bad2 ? 0 : id2) * a.src2_nb1;
    embed_ln_row<TYPE, TYPE2, NV, W>(s1, s2, af, a.w != nullptr, a.b != nullptr, hr, yr, a.ne0, a.eps, lane, bad2,
                                     a.err, lds);
}

template <int TYPE2, int NV, int W>
__global__ __launch_bounds__(64 * W) void k_embed_concat_norm(EmbedConcat a) {
    __shared__ double lds[2 * W];
    const int lane = (threadIdx.x >> 6) * 64 * NV + (threadIdx.x & 63);
    const int t = static_cast<int>(blockIdx.x);
    const int k = t < a.end0 ? 0 : t < a.end1 ? 1 : 2;            // uniform
    const ConcatSeg& sg = a.seg[k];
    const int local = t - (k == 0 ? 0 : k == 1 ? a.end0 : a.end1);
    int32_t row = local;
    bool bad = false;
    if (sg.ids) {
        row = __builtin_amdgcn_readfirstlane(sg.ids[local]);
        bad = row < 0 || row >= sg.rows;
    }
    const char* s1 = sg.base + static_cast<int64_t>(bad ? 0 : row) * sg.nb1;
    char* yr = a.y + t * a.y_nb1;
    char* hr = a.h ? a.h + t * a.h_nb1 : nullptr;
    Affine<NV> af;
    af.load_sel(a.w, a.b, reinterpret_cast<const float*>(a.tab), lane, a.ne0);
    switch (sg.type) {   // uniform
        case CBX_TYPE_F32: concat_row<CBX_TYPE_F32, TYPE2, NV, W>(a, s1, bad, af, hr, yr, lane, lds); break;
        case CBX_TYPE_F16: concat_row<CBX_TYPE_F16, TYPE2, NV, W>(a, s1, bad, af, hr, yr, lane, lds); break;
        default: concat_row<CBX_TYPE_Q8_0, TYPE2, NV, W>(a, s1, bad, af, hr, yr, lane, lds); break;
    }
}

// ---------------------------------------------------------------------------
// workgroup-per-row fallback (ragged or unaligned rows, up to 8192 elements)
// ---------------------------------------------------------------------------

template <typename T, int NV, int KIND, bool ACT, bool VEC>
__global__ __launch_bounds__(kMaxThreads) void k_row_norm(View x, View y, const float* __restrict__ w,
                                                           const float* __restrict__ b, float eps, int act,
                                                           const uint16_t* __restrict__ tab, int64_t nr, bool fx,
                                                           bool fy) {
    __shared__ double red[kMaxThreads / WAVE];
    const int64_t ne0 = x.ne[0];
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const char* xr = x.data + row_offset(x, r, fx);
        char* yr = y.data + row_offset(y, r, fy);

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
                v[k] = Elt<T>::load4(xr + (j < ne0 ? j : 0) * Elt<T>::size);
                if (j >= ne0) v[k] = make_float4(0.f, 0.f, 0.f, 0.f);
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
                                                                const uint16_t* __restrict__ tab, int64_t nr,
                                                                bool fx, bool fy) {
    __shared__ double red[kMaxThreads / WAVE];
    const int64_t ne0 = x.ne[0];
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const char* xr = x.data + row_offset(x, r, fx);
        char* yr = y.data + row_offset(y, r, fy);
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

// ---------------------------------------------------------------------------
// launch selection
// ---------------------------------------------------------------------------

struct NormLaunch {
    View x, y;
    RowMap mx, my;
    const float* w;
    const float* b;
    float eps;
    int act;
    const uint16_t* tab;
    int64_t nr;
    bool fx, fy;
    dim3 grid, block;
    hipStream_t s;
};

template <typename T, int KIND, bool ACT, int WPB, bool FLAT>
void go_wave_w(const NormLaunch& L, int nv) {
    WaveNormArgs a;
    a.x = L.x.data;
    a.y = L.y.data;
    a.w = L.w;
    a.b = L.b;
    a.tab = L.tab;
    a.mx = L.mx;
    a.my = L.my;
    a.ne0 = static_cast<int32_t>(L.x.ne[0]);
    a.nr = static_cast<int32_t>(L.nr);
    a.eps = L.eps;
    a.act = L.act;
#define CBX_WAVE_CASE(N)                                                                       \
    case N:                                                                                   \
        hipLaunchKernelGGL((k_row_norm_wave<T, N, KIND, ACT, WPB, FLAT>), L.grid, L.block, 0, L.s, a); \
        break;
    switch (nv) {
        CBX_WAVE_CASE(1)
        CBX_WAVE_CASE(2)
        CBX_WAVE_CASE(4)
        CBX_WAVE_CASE(8)
        CBX_WAVE_CASE(16)
    }
#undef CBX_WAVE_CASE
}

// Strided-plane layouts (not FLAT) take one row per workgroup.
template <typename T, int KIND, bool ACT>
void go_wave(const NormLaunch& L, int nv) {
    if (!(L.mx.flat && L.my.flat)) go_wave_w<T, KIND, ACT, 1, false>(L, nv);
    else if (L.block.x == 64) go_wave_w<T, KIND, ACT, 1, true>(L, nv);
    else go_wave_w<T, KIND, ACT, 4, true>(L, nv);
}

template <typename T, int KIND, bool ACT, bool VEC>
void go_block(const NormLaunch& L, int nv) {
#define CBX_NORM_CASE(N)                                                                                         \
    case N:                                                                                                     \
        hipLaunchKernelGGL((k_row_norm<T, N, KIND, ACT, VEC>), L.grid, L.block, 0, L.s, L.x, L.y, L.w, L.b,     \
                           L.eps, L.act, L.tab, L.nr, L.fx, L.fy);                                              \
        break;
    switch (nv) {
        CBX_NORM_CASE(1)
        CBX_NORM_CASE(2)
        CBX_NORM_CASE(4)
        CBX_NORM_CASE(8)
        default:
            hipLaunchKernelGGL((k_row_norm_loop<T, KIND, ACT>), L.grid, L.block, 0, L.s, L.x, L.y, L.w, L.b, L.eps,
                               L.act, L.tab, L.nr, L.fx, L.fy);
    }
#undef CBX_NORM_CASE
}

template <typename T, int KIND>
void go(const NormLaunch& L, int nv, bool vec, bool wave) {
    const bool act = L.act != CBX_UNARY_NONE;
    if (wave) {
        if (act) go_wave<T, KIND, true>(L, nv);
        else go_wave<T, KIND, false>(L, nv);
    } else if (act) {
        if (vec) go_block<T, KIND, true, true>(L, nv);
        else go_block<T, KIND, true, false>(L, nv);
    } else {
        if (vec) go_block<T, KIND, false, true>(L, nv);
        else go_block<T, KIND, false, false>(L, nv);
    }
}

bool rows_aligned(const cbx_tensor* t, size_t a) {
    if (reinterpret_cast<uintptr_t>(t->data) % a) return false;
    for (int i = 1; i < 4; i++) if (t->nb[i] % a) return false;
    return true;
}

int pow2_nv(int64_t need) { return need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : need <= 16 ? 16 : 0; }

// Waves per workgroup for wave-per-row kernels: small row counts get one
// wave per workgroup so they spread over more CUs.
int waves_per_block(int64_t rows, const DeviceState* st) { return rows >= int64_t{8} * st->n_cu ? 4 : 1; }

constexpr int64_t kWaveMaxRow = 64 * 4 * 16;   // 4096 elements

}  // namespace

int launch_row_norm(int kind, const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int act,
                    cbx_tensor* y, DeviceState* st, hipStream_t s) {
    if (x->type != y->type) return set_error(CBX_ERR_UNSUPPORTED, "norm: x and y must have the same type");
    const int64_t ne0 = x->ne[0];
    const int64_t nr = nrows(x);
    const size_t a = x->type == CBX_TYPE_F32 ? 16 : 8;
    const bool vec = ne0 % 4 == 0 && rows_aligned(x, a) && rows_aligned(y, a);
    const bool wave = vec && ne0 <= kWaveMaxRow && (!w || reinterpret_cast<uintptr_t>(w->data) % 16 == 0) &&
                      (!b || reinterpret_cast<uintptr_t>(b->data) % 16 == 0);
    NormLaunch L;
    L.x = view_of(x);
    L.y = view_of(y);
    L.w = w ? static_cast<const float*>(w->data) : nullptr;
    L.b = b ? static_cast<const float*>(b->data) : nullptr;
    L.eps = eps;
    L.act = act;
    L.tab = st->gelu_table;
    L.nr = nr;
    L.fx = flat_rows(x);
    L.fy = flat_rows(y);
    L.mx = row_map(x);
    L.my = row_map(y);
    L.s = s;
    int nv;
    if (wave) {
        nv = pow2_nv(cdiv(ne0, 256));
        const int wpb = L.mx.flat && L.my.flat ? waves_per_block(nr, st) : 1;
        L.block = dim3(64 * wpb);
        L.grid = dim3(static_cast<unsigned>(cdiv(nr, wpb)));
        if (nr >= (int64_t{1} << 31)) return set_error(CBX_ERR_UNSUPPORTED, "norm: too many rows");
    } else {
        const int64_t quads = cdiv(ne0, 4);
        const int threads = static_cast<int>(std::min<int64_t>(kMaxThreads, std::max<int64_t>(WAVE, cdiv(quads, WAVE) * WAVE)));
        nv = pow2_nv(cdiv(quads, threads));
        if (nv == 16) nv = 0;   // past the block kernel's register budget
        L.block = dim3(threads);
        L.grid = dim3(static_cast<unsigned>(std::min<int64_t>(nr, int64_t{1} << 20)));
    }
    if (x->type == CBX_TYPE_F32) {
        if (kind == NORM_LN) go<float, NORM_LN>(L, nv, vec, wave);
        else go<float, NORM_RMS>(L, nv, vec, wave);
    } else {
        if (kind == NORM_LN) go<uint16_t, NORM_LN>(L, nv, vec, wave);
        else go<uint16_t, NORM_RMS>(L, nv, vec, wave);
    }
    return check_launch(kind == NORM_LN ? "layer_norm" : "rms_norm");
}

namespace {

template <int TYPE, int TYPE2>
void embed_nv(const EmbedArgs& a, int nv, dim3 grid, dim3 block, hipStream_t s) {
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_embed_norm<TYPE, TYPE2, 1>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_embed_norm<TYPE, TYPE2, 2>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_embed_norm<TYPE, TYPE2, 4>), grid, block, 0, s, a); break;
        case 8: hipLaunchKernelGGL((k_embed_norm<TYPE, TYPE2, 8>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((k_embed_norm<TYPE, TYPE2, 16>), grid, block, 0, s, a); break;
    }
}

// nv: vectors a lane for one wave a row; w: waves a row (nv % w == 0)
template <int TYPE, int TYPE2>
void embed_flat_nv(const EmbedFlat& a, int nv, int w, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(a.n_tok)), block(64 * w);
    switch (nv * 8 + w) {
        case 1 * 8 + 1: hipLaunchKernelGGL((k_embed_norm_flat<TYPE, TYPE2, 1, 1>), grid, block, 0, s, a); break;
        case 2 * 8 + 1: hipLaunchKernelGGL((k_embed_norm_flat<TYPE, TYPE2, 2, 1>), grid, block, 0, s, a); break;
        case 2 * 8 + 2: hipLaunchKernelGGL((k_embed_norm_flat<TYPE, TYPE2, 1, 2>), grid, block, 0, s, a); break;
        case 4 * 8 + 1: hipLaunchKernelGGL((k_embed_norm_flat<TYPE, TYPE2, 4, 1>), grid, block, 0, s, a); break;
        case 4 * 8 + 2: hipLaunchKernelGGL((k_embed_norm_flat<TYPE, TYPE2, 2, 2>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((k_embed_norm_flat<TYPE, TYPE2, 1, 4>), grid, block, 0, s, a); break;
    }
}

template <int TYPE>
void embed_flat_t2(int t2, const EmbedFlat& a, int nv, int w, hipStream_t s) {
    if (t2 == CBX_TYPE_F32) embed_flat_nv<TYPE, CBX_TYPE_F32>(a, nv, w, s);
    else if (t2 == CBX_TYPE_F16) embed_flat_nv<TYPE, CBX_TYPE_F16>(a, nv, w, s);
    else embed_flat_nv<TYPE, CBX_TYPE_Q8_0>(a, nv, w, s);
}

template <int TYPE>
void embed_t2(int t2, const EmbedArgs& a, int nv, dim3 grid, dim3 block, hipStream_t s) {
    if (t2 == CBX_TYPE_F32) embed_nv<TYPE, CBX_TYPE_F32>(a, nv, grid, block, s);
    else if (t2 == CBX_TYPE_F16) embed_nv<TYPE, CBX_TYPE_F16>(a, nv, grid, block, s);
    else embed_nv<TYPE, CBX_TYPE_Q8_0>(a, nv, grid, block, s);
}

bool table_vec_ok(const cbx_tensor* t) {
    if (t->type == CBX_TYPE_Q8_0) return (reinterpret_cast<uintptr_t>(t->data) & 1u) == 0;   // 16-bit quant loads
    const size_t al = t->type == CBX_TYPE_F32 ? 16 : 8;
    return rows_aligned(t, al);
}

}  // namespace

namespace {

template <int TYPE2>
void concat_go(const EmbedConcat& a, int n_tok, int nv, int w, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(n_tok)), block(64 * w);
    switch (nv * 8 + w) {
        case 1 * 8 + 1: hipLaunchKernelGGL((k_embed_concat_norm<TYPE2, 1, 1>), grid, block, 0, s, a); break;
        case 2 * 8 + 1: hipLaunchKernelGGL((k_embed_concat_norm<TYPE2, 2, 1>), grid, block, 0, s, a); break;
        case 2 * 8 + 2: hipLaunchKernelGGL((k_embed_concat_norm<TYPE2, 1, 2>), grid, block, 0, s, a); break;
        case 4 * 8 + 1: hipLaunchKernelGGL((k_embed_concat_norm<TYPE2, 4, 1>), grid, block, 0, s, a); break;
        case 4 * 8 + 2: hipLaunchKernelGGL((k_embed_concat_norm<TYPE2, 2, 2>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((k_embed_concat_norm<TYPE2, 1, 4>), grid, block, 0, s, a); break;
    }
}

ConcatSeg concat_seg(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* fallback) {
    ConcatSeg g;
    const cbx_tensor* t = src ? src : fallback;
    g.base = static_cast<const char*>(t->data);
    g.ids = ids ? static_cast<const int32_t*>(ids->data) : nullptr;
    g.nb1 = static_cast<int64_t>(t->nb[1]);
    g.rows = static_cast<int32_t>(t->ne[1]);
    g.type = src ? src->type : CBX_TYPE_F32;
    return g;
}

}  // namespace

int launch_embed_concat_norm(const cbx_tensor* prefix, const cbx_tensor* src_a, const cbx_tensor* ids_a,
                             const cbx_tensor* src_b, const cbx_tensor* ids_b, const cbx_tensor* src2,
                             const cbx_tensor* ids2, const cbx_tensor* w, const cbx_tensor* b, float eps,
                             cbx_tensor* h, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    const int64_t ne0 = y->ne[0];
    if (ne0 % 4 != 0 || ne0 > 1024 || !table_vec_ok(src_b) || (src_a && !table_vec_ok(src_a)) ||
        !table_vec_ok(src2) || (prefix && !rows_aligned(prefix, 16)) || !rows_aligned(y, 16) ||
        (h && !rows_aligned(h, 16)) || (w && reinterpret_cast<uintptr_t>(w->data) % 16) ||
        (b && reinterpret_cast<uintptr_t>(b->data) % 16)) {
        return set_error(CBX_ERR_UNSUPPORTED,
                         "get_rows_concat_add_layer_norm: needs ne0 % 4 == 0, ne0 <= 1024, 16-byte aligned rows, w, "
                         "b (Q8_0 tables: an even address)");
    }
    EmbedConcat a;
    const int64_t n_pre = prefix ? prefix->ne[1] : 0, n_a = ids_a ? ids_a->ne[0] : 0, n_b = ids_b->ne[0];
    const int64_t n_tok = n_pre + n_a + n_b;
    a.seg[0] = concat_seg(prefix, nullptr, src_b);
    a.seg[0].rows = static_cast<int32_t>(n_pre);
    a.seg[1] = concat_seg(src_a, ids_a, src_b);
    a.seg[2] = concat_seg(src_b, ids_b, src_b);
    a.end0 = static_cast<int32_t>(n_pre);
    a.end1 = static_cast<int32_t>(n_pre + n_a);
    a.src2 = static_cast<const char*>(src2->data);
    a.ids2 = static_cast<const int32_t*>(ids2->data);
    a.src2_nb1 = static_cast<int64_t>(src2->nb[1]);
    a.src2_rows = static_cast<int32_t>(src2->ne[1]);
    a.w = w ? static_cast<const float*>(w->data) : nullptr;
    a.b = b ? static_cast<const float*>(b->data) : nullptr;
    a.h = h ? static_cast<char*>(h->data) : nullptr;
    a.y = static_cast<char*>(y->data);
    a.h_nb1 = h ? static_cast<int64_t>(h->nb[1]) : 0;
    a.y_nb1 = static_cast<int64_t>(y->nb[1]);
    a.ne0 = static_cast<int32_t>(ne0);
    a.eps = eps;
    a.tab = st->gelu_table;
    a.err = st->err_word;
    const int nv = pow2_nv(cdiv(ne0, 256));
    int wr = 1;
    while (wr < 4 && wr < nv && n_tok * wr < int64_t{8} * st->n_cu) wr *= 2;
    switch (src2->type) {
        case CBX_TYPE_F32: concat_go<CBX_TYPE_F32>(a, static_cast<int>(n_tok), nv, wr, s); break;
        case CBX_TYPE_F16: concat_go<CBX_TYPE_F16>(a, static_cast<int>(n_tok), nv, wr, s); break;
        default: concat_go<CBX_TYPE_Q8_0>(a, static_cast<int>(n_tok), nv, wr, s); break;
    }
    return check_launch("get_rows_concat_add_layer_norm");
}

int launch_embed_norm(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* src2, const cbx_tensor* ids2,
                      const cbx_tensor* w, const cbx_tensor* b, float eps, cbx_tensor* h, cbx_tensor* y,
                      DeviceState* st, hipStream_t s) {
    const int64_t ne0 = y->ne[0];
    if (ne0 % 4 != 0 || ne0 > kWaveMaxRow || !table_vec_ok(src) || !table_vec_ok(src2) || !rows_aligned(y, 16) ||
        (h && !rows_aligned(h, 16)) || (w && reinterpret_cast<uintptr_t>(w->data) % 16) ||
        (b && reinterpret_cast<uintptr_t>(b->data) % 16)) {
        return set_error(CBX_ERR_UNSUPPORTED,
                         "get_rows_add_layer_norm: needs ne0 % 4 == 0, ne0 <= 4096, 16-byte aligned rows, w, b "
                         "(Q8_0 tables: an even address)");
    }
    const int64_t n_tok = ids->ne[0] * ids->ne[1] * ids->ne[2];
    const int nv = pow2_nv(cdiv(ne0, 256));
    const int wpb = waves_per_block(n_tok, st);
    const dim3 block(64 * wpb), grid(static_cast<unsigned>(cdiv(n_tok, wpb)));
    auto one_d = [](const cbx_tensor* i) {
        return i->ne[1] == 1 && i->ne[2] == 1 && (i->ne[0] <= 1 || i->nb[0] == sizeof(int32_t));
    };
    auto table_2d = [](const cbx_tensor* t) { return t->ne[2] == 1 && t->ne[3] == 1 && t->ne[1] < (int64_t{1} << 31); };
    if (nv <= 4 && one_d(ids) && one_d(ids2) && table_2d(src) && table_2d(src2) && flat_rows(y) &&
        (!h || flat_rows(h)) && n_tok < (int64_t{1} << 31)) {
        EmbedFlat f;
        f.src = static_cast<const char*>(src->data);
        f.src2 = static_cast<const char*>(src2->data);
        f.ids = static_cast<const int32_t*>(ids->data);
        f.ids2 = static_cast<const int32_t*>(ids2->data);
        f.w = w ? static_cast<const float*>(w->data) : nullptr;
        f.b = b ? static_cast<const float*>(b->data) : nullptr;
        f.h = h ? static_cast<char*>(h->data) : nullptr;
        f.y = static_cast<char*>(y->data);
        f.src_nb1 = static_cast<int64_t>(src->nb[1]);
        f.src2_nb1 = static_cast<int64_t>(src2->nb[1]);
        f.h_nb1 = h ? static_cast<int64_t>(h->nb[1]) : 0;
        f.y_nb1 = static_cast<int64_t>(y->nb[1]);
        f.src_rows = static_cast<int32_t>(src->ne[1]);
        f.src2_rows = static_cast<int32_t>(src2->ne[1]);
        f.n_tok = static_cast<int32_t>(n_tok);
        f.ne0 = static_cast<int32_t>(ne0);
        f.eps = eps;
        f.err = st->err_word;
        // waves a row: enough waves for about eight a CU, at most 4 and at
        // most one per vector a lane (the row split into whole float4 runs)
        int wr = 1;
        while (wr < 4 && wr < nv && n_tok * wr < int64_t{8} * st->n_cu) wr *= 2;
        switch (src->type) {
            case CBX_TYPE_F32: embed_flat_t2<CBX_TYPE_F32>(src2->type, f, nv, wr, s); break;
            case CBX_TYPE_F16: embed_flat_t2<CBX_TYPE_F16>(src2->type, f, nv, wr, s); break;
            default: embed_flat_t2<CBX_TYPE_Q8_0>(src2->type, f, nv, wr, s); break;
        }
        return check_launch("get_rows_add_layer_norm");
    }
    EmbedArgs a;
    a.src = view_of(src);
    a.ids = view_of(ids);
    a.src2 = view_of(src2);
    a.ids2 = view_of(ids2);
    a.h = h ? view_of(h) : null_view();
    a.y = view_of(y);
    a.w = w ? static_cast<const float*>(w->data) : nullptr;
    a.b = b ? static_cast<const float*>(b->data) : nullptr;
    a.eps = eps;
    a.n_tok = n_tok;
    a.err = st->err_word;
    switch (src->type) {
        case CBX_TYPE_F32: embed_t2<CBX_TYPE_F32>(src2->type, a, nv, grid, block, s); break;
        case CBX_TYPE_F16: embed_t2<CBX_TYPE_F16>(src2->type, a, nv, grid, block, s); break;
        default: embed_t2<CBX_TYPE_Q8_0>(src2->type, a, nv, grid, block, s); break;
    }
    return check_launch("get_rows_add_layer_norm");
}

}  // namespace cbx
