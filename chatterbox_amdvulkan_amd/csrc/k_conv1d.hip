// k_conv1d.hip -- the HiFT vocoder's conv1d on the reference's (C, T) layout
// (channel innermost) as an implicit GEMM on the matrix cores, with the
// activation that precedes the conv applied while the input is staged:
// Snake in the ResBlocks (hift_vocoder.cpp:119-138), LeakyReLU before
// conv_post (:748-749).  Bias and the ResBlock's residual add are fused into
// the store.
//
// Arithmetic class of the reference (conv_1d_f32, hift_vocoder.cpp:46-59):
// im2col rounds the conv input to f16, mul_mat rounds the weights to f16 and
// sums the products in f32.  Here: pro(x) in f32 (the five snake() ops, or
// leaky_relu) rounded to f16 (RNE) into LDS, weights pre-rounded to f16,
// v_mfma_f32_32x32x16_f16 products summed in f32, then + bias, then + res.
//
// GEMM view: output time t (M) x output channel co (N), reduced over input
// channel ci and tap k (K dimension).  A workgroup owns BT times x BC
// channels.  Per chunk of 32 input channels it stages one window of
// (BT-1)*stride + (K-1)*dilation + 1 input rows -- every tap's rows are
// shifted views of it, so each input element is loaded and activated once
// per chunk -- then runs, for every tap, the MFMAs of both 16-channel
// halves.  A fragments (8 f16 of one row) come from LDS, B fragments (8 f16
// of one output channel's weights) straight from the [co][k][ci] f16 weight
// copy (L2-resident), the next tap's loaded while this tap's MFMAs run.
//
// Fragment layout of v_mfma_f32_32x32x16_f16 (checked on the device):
// lane l holds A[l % 32][8*(l/32) + j] and B[8*(l/32) + j][l % 32], j < 8;
// accumulator register r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l % 32].
#include "cbx_device.h"

namespace cbx {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int KC = 32;          // input channels per staged chunk
constexpr int RS = KC + 8;      // LDS row stride in halves: 80 bytes, conflict-free 16-byte reads
constexpr int kThreads = 256;   // 4 waves

struct ConvArgs {
    const char* x;              // input row (time) t of batch b at x + b*x_nb2 + t*x_nb1
    const _Float16* w;          // [c_out_pad][k][c_in_pad]
    const float* alpha;         // snake alpha (c_in)
    const float* alpha_inv;     // snake alpha_inv (c_in)
    const float* bias;          // (c_out) or null
    const char* res;            // (c_out, t_out, B) or null
    char* y;
    int64_t x_nb1, x_nb2, y_nb1, y_nb2, r_nb1, r_nb2;
    int32_t c_in, c_in_pad, c_out, k, t_in, t_out, stride, pad, dil, win;
    float slope;
};

enum { PRO_NONE = 0, PRO_SNAKE = 1, PRO_LEAKY = 2 };

template <int PRO>
__device__ __forceinline__ float prologue(float v, float a, float ai, float slope) {
    if constexpr (PRO == PRO_SNAKE) {
        const float xa = v * a;
        const float sn = sinf(xa);
        const float s2 = sn * sn;
        const float m = s2 * ai;
        return v + m;
    } else if constexpr (PRO == PRO_LEAKY) {
        return act_leaky(v, slope);
    } else {
        return v;
    }
}

// WM x WN waves, each computing (MT*32 times) x (NT*32 channels).  VEC: c_in
// % 4 == 0 and 16-byte aligned rows (one float4 per 4 channels).
template <int PRO, int MT, int NT, int WM, int WN, bool VEC>
__global__ __launch_bounds__(kThreads) void k_conv1d(ConvArgs a) {
    extern __shared__ _Float16 win[];   // [a.win][RS]
    constexpr int BT = WM * MT * 32, BC = WN * NT * 32;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int t0 = blockIdx.x * BT;
    const int co0 = blockIdx.y * BC;
    const char* xb = a.x + static_cast<int64_t>(blockIdx.z) * a.x_nb2;
    const int base_t = t0 * a.stride - a.pad;   // input time of window row 0
    const int lrow = lane & 31, lk = 8 * (lane >> 5);

    floatx16 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mt][nt][r] = 0.0f;
        }
    }
    // this lane's weight row of each of its NT output-channel fragments
    const _Float16* wrow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int co = co0 + (wn * NT + nt) * 32 + lrow;
        wrow[nt] = a.w + static_cast<int64_t>(co) * a.k * a.c_in_pad + lk;
    }

    for (int ci0 = 0; ci0 < a.c_in; ci0 += KC) {
        __syncthreads();   // the previous chunk's fragments have been read
        // stage pro(x) for rows [base_t, base_t + win) x channels [ci0, ci0 + 32) as f16
        for (int e = tid; e < a.win * 8; e += kThreads) {
            const int r = e >> 3, cg = (e & 7) * 4;
            const int ti = base_t + r;
            const int ci = ci0 + cg;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (ti >= 0 && ti < a.t_in) {
                const float* src = reinterpret_cast<const float*>(xb + static_cast<int64_t>(ti) * a.x_nb1) + ci;
                if constexpr (VEC) {
                    if (ci < a.c_in) v = *reinterpret_cast<const float4*>(src);
                } else {
                    v.x = ci + 0 < a.c_in ? src[0] : 0.0f;
                    v.y = ci + 1 < a.c_in ? src[1] : 0.0f;
                    v.z = ci + 2 < a.c_in ? src[2] : 0.0f;
                    v.w = ci + 3 < a.c_in ? src[3] : 0.0f;
                }
                if constexpr (PRO != PRO_NONE) {
                    // padding channels (ci >= c_in) stay 0: snake(0) = leaky(0) = 0
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int c = ci + q < a.c_in ? ci + q : 0;
                        const float al = PRO == PRO_SNAKE ? a.alpha[c] : 0.0f;
                        const float ai = PRO == PRO_SNAKE ? a.alpha_inv[c] : 0.0f;
                        set(v, q, prologue<PRO>(get(v, q), al, ai, a.slope));
                    }
                }
            }
            half4 hv;
            hv[0] = static_cast<_Float16>(v.x);
            hv[1] = static_cast<_Float16>(v.y);
            hv[2] = static_cast<_Float16>(v.z);
            hv[3] = static_cast<_Float16>(v.w);
            *reinterpret_cast<half4*>(win + r * RS + cg) = hv;
        }
        __syncthreads();

        half8 bcur[2][NT], bnext[2][NT];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                bcur[hh][nt] = *reinterpret_cast<const half8*>(wrow[nt] + ci0 + hh * 16);
            }
        }
        for (int k = 0; k < a.k; k++) {
            // next tap's weights (the last tap re-reads its own: in bounds, unused)
            const int kn = k + 1 < a.k ? k + 1 : k;
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    bnext[hh][nt] = *reinterpret_cast<const half8*>(wrow[nt] + static_cast<int64_t>(kn) * a.c_in_pad +
                                                                    ci0 + hh * 16);
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                half8 av[MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    const int row = ((wm * MT + mt) * 32 + lrow) * a.stride + k * a.dil;
                    av[mt] = *reinterpret_cast<const half8*>(win + row * RS + hh * 16 + lk);
                }
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bcur[hh][nt], acc[mt][nt], 0, 0,
                                                                             0);
                    }
                }
            }
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) bcur[hh][nt] = bnext[hh][nt];
            }
        }
    }

    // y = (sum + bias) [+ res]: ggml_add of the bias, then the residual add
    const int64_t yb = static_cast<int64_t>(blockIdx.z) * a.y_nb2;
    const int64_t rb = static_cast<int64_t>(blockIdx.z) * a.r_nb2;
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int co = co0 + (wn * NT + nt) * 32 + lrow;
        if (co >= a.c_out) continue;
        const float bv = a.bias ? a.bias[co] : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int t = t0 + (wm * MT + mt) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (t >= a.t_out) continue;
                float v = acc[mt][nt][r];
                if (a.bias) v = v + bv;
                if (a.res) v = reinterpret_cast<const float*>(a.res + rb + static_cast<int64_t>(t) * a.r_nb1)[co] + v;
                reinterpret_cast<float*>(a.y + yb + static_cast<int64_t>(t) * a.y_nb1)[co] = v;
            }
        }
    }
}

// [c_out_pad][k][c_in_pad] f16 copy of a ggml (K, C_in, C_out) weight, zero
// padded; the f16 rounding is mul_mat's conversion of its F32 operand.
template <bool F16>
__global__ __launch_bounds__(256) void k_conv_weights(const char* w, int64_t nb0, int64_t nb1, int64_t nb2, int32_t K,
                                                      int32_t c_in, int32_t c_out, int32_t c_in_pad, int64_t total,
                                                      _Float16* out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= total) return;
    const int32_t ci = static_cast<int32_t>(i % c_in_pad);
    const int64_t q = i / c_in_pad;
    const int32_t k = static_cast<int32_t>(q % K);
    const int32_t co = static_cast<int32_t>(q / K);
    _Float16 v = static_cast<_Float16>(0.0f);
    if (ci < c_in && co < c_out) {
        const char* p = w + k * nb0 + ci * nb1 + co * nb2;
        if constexpr (F16) v = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(p));
        else v = static_cast<_Float16>(*reinterpret_cast<const float*>(p));
    }
    out[i] = v;
}

struct Tile {
    int mt, nt, wm, wn;
    int bt() const { return wm * mt * 32; }
    int bc() const { return wn * nt * 32; }
};

template <int PRO, int MT, int NT, int WM, int WN>
void conv_go(bool vec, dim3 grid, size_t lds, hipStream_t s, const ConvArgs& a) {
    if (vec) hipLaunchKernelGGL((k_conv1d<PRO, MT, NT, WM, WN, true>), grid, dim3(kThreads), lds, s, a);
    else hipLaunchKernelGGL((k_conv1d<PRO, MT, NT, WM, WN, false>), grid, dim3(kThreads), lds, s, a);
}

template <int PRO>
void conv_tile(const Tile& t, bool vec, dim3 grid, size_t lds, hipStream_t s, const ConvArgs& a) {
    if (t.wn == 2) conv_go<PRO, 2, 2, 2, 2>(vec, grid, lds, s, a);        // 128 x 128
    else if (t.mt == 2) conv_go<PRO, 2, 2, 4, 1>(vec, grid, lds, s, a);   // 256 x 64
    else if (t.wm == 1) conv_go<PRO, 1, 1, 1, 4>(vec, grid, lds, s, a);   // 32 x 128
    else conv_go<PRO, 1, 1, 4, 1>(vec, grid, lds, s, a);                  // 128 x 32
}

}  // namespace

// Output-channel padding of the prepared weights: a multiple of every tile width.
constexpr int kConvCoPad = 128;

int conv1d_weights_layout(int64_t c_in, int64_t c_out, int64_t* c_in_pad, int64_t* c_out_pad) {
    *c_in_pad = cdiv(c_in, KC) * KC;
    *c_out_pad = cdiv(c_out, kConvCoPad) * kConvCoPad;
    return CBX_OK;
}

int launch_conv1d_weights(const cbx_tensor* w, _Float16* out, int64_t c_in_pad, int64_t c_out_pad, hipStream_t s) {
    const int64_t total = c_out_pad * w->ne[0] * c_in_pad;
    const dim3 grid(static_cast<unsigned>(cdiv(total, 256)));
    const char* p = static_cast<const char*>(w->data);
    const int64_t nb0 = static_cast<int64_t>(w->nb[0]), nb1 = static_cast<int64_t>(w->nb[1]),
                  nb2 = static_cast<int64_t>(w->nb[2]);
    const int32_t K = static_cast<int32_t>(w->ne[0]), ci = static_cast<int32_t>(w->ne[1]),
                  co = static_cast<int32_t>(w->ne[2]);
    if (w->type == CBX_TYPE_F16) {
        hipLaunchKernelGGL((k_conv_weights<true>), grid, dim3(256), 0, s, p, nb0, nb1, nb2, K, ci, co,
                           static_cast<int32_t>(c_in_pad), total, out);
    } else {
        hipLaunchKernelGGL((k_conv_weights<false>), grid, dim3(256), 0, s, p, nb0, nb1, nb2, K, ci, co,
                           static_cast<int32_t>(c_in_pad), total, out);
    }
    return check_launch("conv1d_weights");
}

int launch_conv1d(const cbx_tensor* x, const _Float16* w16, int64_t k, int64_t c_in_pad, int64_t c_out, int stride,
                  int pad, int dil, int pro, const cbx_tensor* alpha, const cbx_tensor* alpha_inv, float slope,
                  const cbx_tensor* bias, const cbx_tensor* res, cbx_tensor* y, DeviceState* st, hipStream_t s) {
    ConvArgs a;
    a.x = static_cast<const char*>(x->data);
    a.w = w16;
    a.alpha = alpha ? static_cast<const float*>(alpha->data) : nullptr;
    a.alpha_inv = alpha_inv ? static_cast<const float*>(alpha_inv->data) : nullptr;
    a.bias = bias ? static_cast<const float*>(bias->data) : nullptr;
    a.res = res ? static_cast<const char*>(res->data) : nullptr;
    a.y = static_cast<char*>(y->data);
    a.x_nb1 = static_cast<int64_t>(x->nb[1]);
    a.x_nb2 = static_cast<int64_t>(x->nb[2]);
    a.y_nb1 = static_cast<int64_t>(y->nb[1]);
    a.y_nb2 = static_cast<int64_t>(y->nb[2]);
    a.r_nb1 = res ? static_cast<int64_t>(res->nb[1]) : 0;
    a.r_nb2 = res ? static_cast<int64_t>(res->nb[2]) : 0;
    a.c_in = static_cast<int32_t>(x->ne[0]);
    a.c_in_pad = static_cast<int32_t>(c_in_pad);
    a.c_out = static_cast<int32_t>(c_out);
    a.k = static_cast<int32_t>(k);
    a.t_in = static_cast<int32_t>(x->ne[1]);
    a.t_out = static_cast<int32_t>(y->ne[1]);
    a.stride = stride;
    a.pad = pad;
    a.dil = dil;
    a.slope = slope;
    const int64_t batch = x->ne[2];
    // tile: 128x128 when it gives >= 2 workgroups per CU, else 32x128 for
    // wide outputs; 256x64 / 128x32 for narrow ones
    const Tile big{2, 2, 2, 2}, tall{2, 2, 4, 1}, small{1, 1, 1, 4}, narrow{1, 1, 4, 1};
    auto n_wg = [&](const Tile& t) { return cdiv(a.t_out, t.bt()) * cdiv(c_out, t.bc()) * batch; };
    Tile t = c_out <= 32 ? narrow : c_out <= 64 ? tall : (n_wg(big) >= 2 * st->n_cu ? big : small);
    auto lds_of = [&](const Tile& tt) {
        return static_cast<size_t>((tt.bt() - 1) * stride + (k - 1) * dil + 1) * RS * sizeof(_Float16);
    };
    constexpr size_t kLdsMax = 64 * 1024;
    if (lds_of(t) > kLdsMax) t = c_out <= 32 ? narrow : small;   // strided convs: shorter windows
    if (lds_of(t) > kLdsMax) {
        return set_error(CBX_ERR_UNSUPPORTED, "conv1d: the input window of one tile exceeds 64 KiB of LDS");
    }
    a.win = (t.bt() - 1) * stride + static_cast<int32_t>(k - 1) * dil + 1;
    const bool vec = a.c_in % 4 == 0 && reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && a.x_nb1 % 16 == 0 &&
                     (batch <= 1 || a.x_nb2 % 16 == 0);
    const dim3 grid(static_cast<unsigned>(cdiv(a.t_out, t.bt())), static_cast<unsigned>(cdiv(c_out, t.bc())),
                    static_cast<unsigned>(batch));
    switch (pro) {
        case PRO_SNAKE: conv_tile<PRO_SNAKE>(t, vec, grid, lds_of(t), s, a); break;
        case PRO_LEAKY: conv_tile<PRO_LEAKY>(t, vec, grid, lds_of(t), s, a); break;
        default: conv_tile<PRO_NONE>(t, vec, grid, lds_of(t), s, a); break;
    }
    return check_launch("conv1d");
}

}  // namespace cbx
