// k_softmax.hip -- the attention-score epilogue in one pass:
//
//   y = ggml_soft_max(ggml_diag_mask_inf(ggml_scale(x, s), n_past))
//
// (t3.cpp:513-518; without the mask, n_past < 0: cfm_decoder.cpp:218-220,
// flow_encoder.cpp:371-372, s3enc.cpp:260-262), and with the two score
// terms' sum in front, x = ggml_add(a, b) (flow_encoder.cpp:369-372: the
// content and the shifted position scores).  Per row of ne0 scores:
// [x = a + b (one f32 add),] t = x*s (one f32 multiply), t = -inf where
// column i > n_past + j (j = the row's ne1 index), m = max t,
// e = expf(t - m), sum of e in f64, y = e * (float)(1.0 / sum) --
// ggml-cpu's scalar order of operations.
//
// Rows up to 4096 with ne0 % 4 == 0: one wave per row, the row in
// registers (one read, one write), the max by a butterfly of lane shuffles
// (exact in any order), the sum by the f64 DPP butterfly; rows up to 2048
// with ne0 % 2 == 0 at 8-byte steps the same in float2s (the 25 Hz
// conformer blocks' 250 keys).  Few rows up to 4096 (a decode step's): a
// workgroup per row (a wave up to 1024), the row in registers, one kernel
// for every length.  Other rows up to 1024: a wave per row, the same
// kernel.  Longer ones: a workgroup per row, three passes.
#include "cbx_rowops.h"

namespace cbx {
namespace {

constexpr int kThreads = 256;
constexpr int kWaveMaxRow = 4096;

// Max over the 64 lanes of a wave, in every lane (a max is exact in any
// order).  wave_max: a butterfly of lane shuffles (LDS permutes).
// wave_max_dpp: the f64 sum's butterfly inside each 16-lane row (DPP moves,
// no LDS round trip), then the four row maxima read from lanes 0/16/32/48;
// all 64 lanes must be active.  The few-row decode kernel takes the DPP
// form (0.25 us a launch less: the T3 decode token, 24 softmax launches,
// 247-249 against 253-255 us); the wave-per-row kernel keeps the shuffles
// (DPP there: T3 prefill scores 8.0 against 8.15 us, CFM scores 8.4
// against 8.2 us).
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_f32<0x4E>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_f32<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_f32<0x140>(v));   // row_mirror
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// score after scale and mask; columns past the row end read as -inf
__device__ __forceinline__ float masked(float x, float s, int64_t col, int64_t limit) {
    return col > limit ? -INFINITY : x * s;
}

struct SoftMaxArgs {
    const char* x;
    const char* b;         // the second score term (ADD), x's shape
    char* y;
    RowMap mx, mb, my;
    int64_t n_past;
    int32_t ne0, nr;
    uint32_t n_q;          // x.ne1: the query index of a row is r % n_q
    float s;
};

// VW consecutive scores a lane per load: 4 (float4) for rows at 16-byte
// steps, 2 (float2) for rows at 8-byte steps (the 25 Hz conformer blocks'
// 250 keys, rows 1000 bytes apart)
template <int VW>
__device__ __forceinline__ float4 load_v(const char* p) {
    if constexpr (VW == 4) {
        return Elt<float>::load4(p);
    } else {
        const float2 t = *reinterpret_cast<const float2*>(p);
        return make_float4(t.x, t.y, 0.0f, 0.0f);
    }
}

template <int VW>
__device__ __forceinline__ void store_v(char* p, float4 v) {
    if constexpr (VW == 4) Elt<float>::store4(p, v);
    else *reinterpret_cast<float2*>(p) = make_float2(v.x, v.y);
}

// WPB rows per workgroup; with one, the grid is exactly one workgroup per
// row and nothing waits (bounds check, block size) before the loads issue.
// FLAT: rows at one stride each, so the row map's flag is not tested either.
template <int NV, int WPB, bool FLAT, bool ADD, int VW>
__global__ __launch_bounds__(64 * WPB) void k_soft_max_wave(SoftMaxArgs a) {
    // every field in the first batch of argument loads (left alone, the
    // compiler loads the row count first and the rest after its test: a
    // second scalar round trip before the row loads)
    arg_now(a.x); arg_now(a.y); arg_now(reinterpret_cast<const void*>(a.mx.nb1));
    arg_now(reinterpret_cast<const void*>(a.my.nb1)); arg_now(reinterpret_cast<const void*>(a.n_past));
    arg_now(static_cast<uint32_t>(a.ne0)); arg_now(static_cast<uint32_t>(a.nr)); arg_now(a.n_q);
    if constexpr (ADD) {
        arg_now(a.b); arg_now(reinterpret_cast<const void*>(a.mb.nb1));
    }
    const int lane = threadIdx.x & 63;
    uint32_t r = blockIdx.x;
    if constexpr (WPB > 1) {
        r = r * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (r >= static_cast<uint32_t>(a.nr)) return;   // uniform per wave
    }
    const int64_t ne0 = a.ne0;
    const float s = a.s;
    const int64_t n_past = a.n_past;
    const char* xr = a.x + (FLAT ? static_cast<int64_t>(r) * a.mx.nb1 : row_at(a.mx, r));
    char* yr = a.y + (FLAT ? static_cast<int64_t>(r) * a.my.nb1 : row_at(a.my, r));
    const char* br = ADD ? a.b + (FLAT ? static_cast<int64_t>(r) * a.mb.nb1 : row_at(a.mb, r)) : nullptr;
    // last unmasked column of this row
    const int64_t j = r % a.n_q;
    const int64_t lim = n_past >= 0 ? (n_past + j < ne0 - 1 ? n_past + j : ne0 - 1) : ne0 - 1;
    float4 v[NV], w[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t c = (lane + 64 * k) * VW;
        v[k] = load_v<VW>(xr + (c < ne0 ? c : 0) * 4);
        if constexpr (ADD) w[k] = load_v<VW>(br + (c < ne0 ? c : 0) * 4);
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t c = (lane + 64 * k) * VW;
#pragma unroll
        for (int e = 0; e < VW; e++) {
            const float x = ADD ? get(v[k], e) + get(w[k], e) : get(v[k], e);
            const float t = masked(x, s, c + e, lim);
            set(v[k], e, t);
            m = fmaxf(m, t);
        }
    }
    m = wave_max(m);
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
#pragma unroll
        for (int e = 0; e < VW; e++) {
            const float ev = expf(get(v[k], e) - m);
            set(v[k], e, ev);
            sum += static_cast<double>(ev);
        }
    }
    sum = wave_sum(sum);
    const float inv = static_cast<float>(1.0 / sum);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t c = (lane + 64 * k) * VW;
        if (c < ne0) {   // ne0 % VW == 0: whole vectors
            store_v<VW>(yr + c * 4, make_float4(v[k].x * inv, v[k].y * inv, v[k].z * inv, v[k].w * inv));
        }
    }
}

// Few rows of up to 4096 scores at any alignment (the decode step's H
// rows of n_past + 1 columns): one 256-lane workgroup a row, the row in
// registers (16 columns a lane, loads issued together), the max and the
// f64 sum over the workgroup.  One kernel for every length up to 4096, so a
// decode loop whose rows grow by one column a token launches the same
// kernel each token and a captured graph takes the new length in place.
// The row's address and query index come from the compact arguments with
// 32-bit index arithmetic, every field in the first batch of argument
// loads: a View's 64-bit divisions and the dependent argument loads they
// waited on put about 900 instructions before the first score load.
template <bool FLAT, bool ADD>
__global__ __launch_bounds__(kThreads) void k_soft_max_row(SoftMaxArgs a) {
    constexpr int K = kWaveMaxRow / kThreads;
    constexpr int NW = kThreads / WAVE;
    __shared__ float redf[NW];
    __shared__ double red[NW];
    arg_now(a.x); arg_now(a.y); arg_now(reinterpret_cast<const void*>(a.mx.nb1));
    arg_now(reinterpret_cast<const void*>(a.my.nb1)); arg_now(reinterpret_cast<const void*>(a.n_past));
    arg_now(static_cast<uint32_t>(a.ne0)); arg_now(a.n_q);
    if constexpr (ADD) {
        arg_now(a.b); arg_now(reinterpret_cast<const void*>(a.mb.nb1));
    }
    if constexpr (!FLAT) {
        for (const RowMap* m : {&a.mx, &a.my}) {
            arg_now(reinterpret_cast<const void*>(m->nb2)); arg_now(reinterpret_cast<const void*>(m->nb3));
            arg_now(m->ne1); arg_now(m->ne2);
        }
    }
    const uint32_t r = blockIdx.x;
    const int ne0 = a.ne0;
    const float* xr = reinterpret_cast<const float*>(a.x + (FLAT ? r * a.mx.nb1 : row_at(a.mx, r)));
    float* yr = reinterpret_cast<float*>(a.y + (FLAT ? r * a.my.nb1 : row_at(a.my, r)));
    const float* bq = ADD ? reinterpret_cast<const float*>(a.b + (FLAT ? r * a.mb.nb1 : row_at(a.mb, r))) : nullptr;
    const int64_t j = r % a.n_q;
    const int64_t lim = a.n_past >= 0 ? (a.n_past + j < ne0 - 1 ? a.n_past + j : ne0 - 1) : ne0 - 1;
    // the columns a lane holds: k < nk (uniform); the loads of those issue
    // together, the others are skipped (a decode row of 256 scores reads
    // one column a lane, not 16)
    const int nk = (ne0 + kThreads - 1) / kThreads;
    float v[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int c = threadIdx.x + k * kThreads;
        v[k] = -INFINITY;
        if (k < nk) v[k] = ADD ? xr[c < ne0 ? c : 0] + bq[c < ne0 ? c : 0] : xr[c < ne0 ? c : 0];
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int c = threadIdx.x + k * kThreads;
        v[k] = c < ne0 ? masked(v[k], a.s, c, lim) : -INFINITY;
        m = fmaxf(m, v[k]);
    }
    m = wave_max_dpp(m);
    if ((threadIdx.x & 63) == 0) redf[threadIdx.x >> 6] = m;
    __syncthreads();
    m = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) m = fmaxf(m, redf[w]);
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < K; k++) {
        if (k < nk) {
            const int c = threadIdx.x + k * kThreads;
            v[k] = c < ne0 ? expf(v[k] - m) : 0.0f;
            sum += static_cast<double>(v[k]);
        }
    }
    // the wave totals in index order (one barrier; the area is not the max's)
    sum = wave_sum(sum);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    sum = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) sum += red[w];
    const float inv = static_cast<float>(1.0 / sum);
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int c = threadIdx.x + k * kThreads;
        if (k < nk && c < ne0) yr[c] = v[k] * inv;
    }
}

// Rows of up to 1024 scores at any alignment (the T3 decode step's 16 rows
// of n_past + 1 columns, n_past < 1024; many rows of odd length): one wave
// a row, up to 16
// columns a lane (column lane + 64 k), the max and the f64 sum by DPP
// butterflies -- no LDS and no barrier.  One kernel for every length up to
// 1024, like k_soft_max_row.
template <bool FLAT, bool ADD>
__global__ __launch_bounds__(WAVE) void k_soft_max_row_w(SoftMaxArgs a) {
    constexpr int K = 1024 / WAVE;
    arg_now(a.x); arg_now(a.y); arg_now(reinterpret_cast<const void*>(a.mx.nb1));
    arg_now(reinterpret_cast<const void*>(a.my.nb1)); arg_now(reinterpret_cast<const void*>(a.n_past));
    arg_now(static_cast<uint32_t>(a.ne0)); arg_now(a.n_q);
    if constexpr (ADD) {
        arg_now(a.b); arg_now(reinterpret_cast<const void*>(a.mb.nb1));
    }
    if constexpr (!FLAT) {
        for (const RowMap* m : {&a.mx, &a.my}) {
            arg_now(reinterpret_cast<const void*>(m->nb2)); arg_now(reinterpret_cast<const void*>(m->nb3));
            arg_now(m->ne1); arg_now(m->ne2);
        }
    }
    const uint32_t r = blockIdx.x;
    const int ne0 = a.ne0, lane = threadIdx.x;
    const float* xr = reinterpret_cast<const float*>(a.x + (FLAT ? r * a.mx.nb1 : row_at(a.mx, r)));
    float* yr = reinterpret_cast<float*>(a.y + (FLAT ? r * a.my.nb1 : row_at(a.my, r)));
    const float* bq = ADD ? reinterpret_cast<const float*>(a.b + (FLAT ? r * a.mb.nb1 : row_at(a.mb, r))) : nullptr;
    const int64_t j = r % a.n_q;
    const int64_t lim = a.n_past >= 0 ? (a.n_past + j < ne0 - 1 ? a.n_past + j : ne0 - 1) : ne0 - 1;
    const int nk = (ne0 + WAVE - 1) / WAVE;   // uniform: the loads of k < nk issue together
    float v[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int c = lane + k * WAVE;
        v[k] = -INFINITY;
        if (k < nk) v[k] = ADD ? xr[c < ne0 ? c : 0] + bq[c < ne0 ? c : 0] : xr[c < ne0 ? c : 0];
    }
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int c = lane + k * WAVE;
        v[k] = c < ne0 ? masked(v[k], a.s, c, lim) : -INFINITY;
        m = fmaxf(m, v[k]);
    }
    m = wave_max_dpp(m);
    double sum = 0.0;
#pragma unroll
    for (int k = 0; k < K; k++) {
        if (k < nk) {
            const int c = lane + k * WAVE;
            v[k] = c < ne0 ? expf(v[k] - m) : 0.0f;
            sum += static_cast<double>(v[k]);
        }
    }
    sum = wave_sum(sum);
    const float inv = static_cast<float>(1.0 / sum);
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int c = lane + k * WAVE;
        if (k < nk && c < ne0) yr[c] = v[k] * inv;
    }
}

// Any row length: max, then the f64 sum of exponentials, then the output,
// each pass over the row (the exponentials are recomputed identically).
__global__ __launch_bounds__(kThreads) void k_soft_max_loop(View x, View b, View y, float s, int64_t n_past,
                                                            bool fx, bool fb, bool fy) {
    __shared__ double red[kThreads / WAVE];
    __shared__ float redf[kThreads / WAVE];
    const int64_t r = blockIdx.x;
    const int64_t ne0 = x.ne[0];
    const float* xr = reinterpret_cast<const float*>(x.data + row_offset(x, r, fx));
    float* yr = reinterpret_cast<float*>(y.data + row_offset(y, r, fy));
    // b.data null: no second term
    const float* br = b.data ? reinterpret_cast<const float*>(b.data + row_offset(b, r, fb)) : nullptr;
    const auto at = [&](int64_t c) { return br ? xr[c] + br[c] : xr[c]; };
    const int64_t j = r % x.ne[1];
    const int64_t lim = n_past >= 0 ? (n_past + j < ne0 - 1 ? n_past + j : ne0 - 1) : ne0 - 1;
    float m = -INFINITY;
    for (int64_t c = threadIdx.x; c < ne0; c += kThreads) m = fmaxf(m, masked(at(c), s, c, lim));
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) redf[threadIdx.x >> 6] = m;
    __syncthreads();
    m = -INFINITY;
    for (int w = 0; w < kThreads / WAVE; w++) m = fmaxf(m, redf[w]);
    double sum = 0.0;
    for (int64_t c = threadIdx.x; c < ne0; c += kThreads) sum += static_cast<double>(expf(masked(at(c), s, c, lim) - m));
    sum = block_sum(sum, red);
    const float inv = static_cast<float>(1.0 / sum);
    for (int64_t c = threadIdx.x; c < ne0; c += kThreads) yr[c] = expf(masked(at(c), s, c, lim) - m) * inv;
}

SoftMaxArgs sm_args(const cbx_tensor* x, const cbx_tensor* b, cbx_tensor* y, float s, int64_t n_past, int64_t nr) {
    SoftMaxArgs a;
    a.x = static_cast<const char*>(x->data);
    a.b = b ? static_cast<const char*>(b->data) : nullptr;
    a.y = static_cast<char*>(y->data);
    a.mx = row_map(x);
    a.mb = row_map(b ? b : x);
    a.my = row_map(y);
    a.n_past = n_past;
    a.ne0 = static_cast<int32_t>(x->ne[0]);
    a.nr = static_cast<int32_t>(nr);
    a.n_q = static_cast<uint32_t>(x->ne[1] > 0 ? x->ne[1] : 1);
    a.s = s;
    return a;
}

int waves_for(int64_t rows, const DeviceState* st) { return rows >= int64_t{8} * st->n_cu ? 4 : 1; }

template <int WPB, bool FLAT, bool ADD, int VW>
void sm_wave(int nv, const SoftMaxArgs& a, hipStream_t strm) {
    const dim3 grid(static_cast<unsigned>(cdiv(a.nr, WPB))), block(64 * WPB);
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_soft_max_wave<1, WPB, FLAT, ADD, VW>), grid, block, 0, strm, a); break;
        case 2: hipLaunchKernelGGL((k_soft_max_wave<2, WPB, FLAT, ADD, VW>), grid, block, 0, strm, a); break;
        case 4: hipLaunchKernelGGL((k_soft_max_wave<4, WPB, FLAT, ADD, VW>), grid, block, 0, strm, a); break;
        case 8: hipLaunchKernelGGL((k_soft_max_wave<8, WPB, FLAT, ADD, VW>), grid, block, 0, strm, a); break;
        default: hipLaunchKernelGGL((k_soft_max_wave<16, WPB, FLAT, ADD, VW>), grid, block, 0, strm, a); break;
    }
}

// the wave-per-row kernel for rows of VW-float vectors (NV of them a lane)
template <bool ADD, int VW>
void sm_waves(const SoftMaxArgs& a, int64_t ne0, const DeviceState* st, hipStream_t strm) {
    const int64_t need = cdiv(ne0, 64 * VW);
    const int nv = need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : need <= 8 ? 8 : 16;
    // strided-plane layouts take one row per workgroup through the row map
    if (!(a.mx.flat && a.my.flat && (!ADD || a.mb.flat))) sm_wave<1, false, ADD, VW>(nv, a, strm);
    else if (waves_for(a.nr, st) == 1) sm_wave<1, true, ADD, VW>(nv, a, strm);
    else sm_wave<4, true, ADD, VW>(nv, a, strm);
}

template <bool ADD>
void sm_launch(const SoftMaxArgs& a, int64_t ne0, bool vec, bool vec2, const View& vx, const View& vb,
               const View& vy, bool fx, bool fb, bool fy, const DeviceState* st, hipStream_t strm) {
    const int64_t nr = a.nr;
    if (ne0 <= kWaveMaxRow && nr < int64_t{4} * st->n_cu) {
        // few rows (a decode step's heads): one kernel whatever the length
        const dim3 grid(static_cast<unsigned>(nr));
        const bool flat = a.mx.flat && a.my.flat && (!ADD || a.mb.flat);
        if (ne0 <= 1024) {
            if (flat) hipLaunchKernelGGL((k_soft_max_row_w<true, ADD>), grid, dim3(WAVE), 0, strm, a);
            else hipLaunchKernelGGL((k_soft_max_row_w<false, ADD>), grid, dim3(WAVE), 0, strm, a);
        } else if (flat) {
            hipLaunchKernelGGL((k_soft_max_row<true, ADD>), grid, dim3(kThreads), 0, strm, a);
        } else {
            hipLaunchKernelGGL((k_soft_max_row<false, ADD>), grid, dim3(kThreads), 0, strm, a);
        }
    } else if (vec) {
        sm_waves<ADD, 4>(a, ne0, st, strm);
    } else if (vec2) {
        sm_waves<ADD, 2>(a, ne0, st, strm);
    } else if (ne0 <= 1024) {
        // many rows of odd length up to 1024: one wave a row, as for few
        // rows, not three passes
        const dim3 grid(static_cast<unsigned>(nr));
        if (a.mx.flat && a.my.flat && (!ADD || a.mb.flat)) {
            hipLaunchKernelGGL((k_soft_max_row_w<true, ADD>), grid, dim3(WAVE), 0, strm, a);
        } else {
            hipLaunchKernelGGL((k_soft_max_row_w<false, ADD>), grid, dim3(WAVE), 0, strm, a);
        }
    } else {
        hipLaunchKernelGGL(k_soft_max_loop, dim3(static_cast<unsigned>(nr)), dim3(kThreads), 0, strm, vx, vb, vy, a.s,
                           a.n_past, fx, fb, fy);
    }
}

// every row of t starts at a multiple of `al` bytes
bool vec_rows(const cbx_tensor* t, size_t al) {
    return reinterpret_cast<uintptr_t>(t->data) % al == 0 && t->nb[1] % al == 0 && (t->ne[2] <= 1 || t->nb[2] % al == 0) &&
           (t->ne[3] <= 1 || t->nb[3] % al == 0);
}

}  // namespace

int launch_soft_max(const cbx_tensor* x, const cbx_tensor* b, float s, int64_t n_past, cbx_tensor* y,
                    DeviceState* st, hipStream_t strm) {
    const int64_t nr = nrows(x), ne0 = x->ne[0];
    if (nr >= (int64_t{1} << 31)) return set_error(CBX_ERR_UNSUPPORTED, "soft_max: too many rows");
    const bool vec = ne0 <= kWaveMaxRow && ne0 % 4 == 0 && vec_rows(x, 16) && vec_rows(y, 16) && (!b || vec_rows(b, 16));
    const bool vec2 = ne0 <= kWaveMaxRow / 2 && ne0 % 2 == 0 && vec_rows(x, 8) && vec_rows(y, 8) && (!b || vec_rows(b, 8));
    View vb{};
    if (b) vb = view_of(b);
    const SoftMaxArgs a = sm_args(x, b, y, s, n_past, nr);
    if (b) {
        sm_launch<true>(a, ne0, vec, vec2, view_of(x), vb, view_of(y), flat_rows(x), flat_rows(b), flat_rows(y), st,
                        strm);
    } else {
        sm_launch<false>(a, ne0, vec, vec2, view_of(x), vb, view_of(y), flat_rows(x), false, flat_rows(y), st, strm);
    }
    return check_launch("soft_max");
}

}  // namespace cbx
