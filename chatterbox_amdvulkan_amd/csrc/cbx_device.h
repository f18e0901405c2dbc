// cbx_device.h -- device-side helpers for gfx950 (wave64).
//
// Built with -ffp-contract=off: each float operation written below rounds
// once, in the order written, which is what lets the kernels reproduce
// ggml-cpu's results bit for bit where no transcendental function is
// involved.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "cbx_internal.h"

namespace cbx {

constexpr int WAVE = 64;

// ---- fp16 <-> fp32 (hardware v_cvt, round to nearest even, denormals kept)
__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// ---- 4-element vector loads/stores for f32 and f16 storage ---------------
template <typename T> struct Elt;
template <> struct Elt<float> {
    static __device__ __forceinline__ float4 load4(const char* p) {
        return *reinterpret_cast<const float4*>(p);
    }
    static __device__ __forceinline__ void store4(char* p, float4 v) {
        *reinterpret_cast<float4*>(p) = v;
    }
    static __device__ __forceinline__ float load1(const char* p) {
        return *reinterpret_cast<const float*>(p);
    }
    static __device__ __forceinline__ void store1(char* p, float v) {
        *reinterpret_cast<float*>(p) = v;
    }
    static constexpr int size = 4;
};
template <> struct Elt<uint16_t> {   // fp16 storage
    static __device__ __forceinline__ float4 load4(const char* p) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        return make_float4(h2f(u.x & 0xffffu), h2f(u.x >> 16), h2f(u.y & 0xffffu), h2f(u.y >> 16));
    }
    static __device__ __forceinline__ void store4(char* p, float4 v) {
        uint2 u;
        u.x = static_cast<uint32_t>(f2h(v.x)) | (static_cast<uint32_t>(f2h(v.y)) << 16);
        u.y = static_cast<uint32_t>(f2h(v.z)) | (static_cast<uint32_t>(f2h(v.w)) << 16);
        *reinterpret_cast<uint2*>(p) = u;
    }
    static __device__ __forceinline__ float load1(const char* p) {
        return h2f(*reinterpret_cast<const uint16_t*>(p));
    }
    static __device__ __forceinline__ void store1(char* p, float v) {
        *reinterpret_cast<uint16_t*>(p) = f2h(v);
    }
    static constexpr int size = 2;
};

// Streaming (nontemporal) 4-element loads/stores: data touched once is not
// kept in the caches.
typedef float cbx_f4v __attribute__((ext_vector_type(4)));
typedef unsigned int cbx_u2v __attribute__((ext_vector_type(2)));

template <typename T> struct Stream;
template <> struct Stream<float> {
    static __device__ __forceinline__ float4 load4(const char* p) {
        const cbx_f4v t = __builtin_nontemporal_load(reinterpret_cast<const cbx_f4v*>(p));
        return make_float4(t.x, t.y, t.z, t.w);
    }
    static __device__ __forceinline__ void store4(char* p, float4 v) {
        const cbx_f4v t = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(t, reinterpret_cast<cbx_f4v*>(p));
    }
};
template <> struct Stream<uint16_t> {
    static __device__ __forceinline__ float4 load4(const char* p) {
        const cbx_u2v u = __builtin_nontemporal_load(reinterpret_cast<const cbx_u2v*>(p));
        return make_float4(h2f(u.x & 0xffffu), h2f(u.x >> 16), h2f(u.y & 0xffffu), h2f(u.y >> 16));
    }
    static __device__ __forceinline__ void store4(char* p, float4 v) {
        cbx_u2v u;
        u.x = static_cast<uint32_t>(f2h(v.x)) | (static_cast<uint32_t>(f2h(v.y)) << 16);
        u.y = static_cast<uint32_t>(f2h(v.z)) | (static_cast<uint32_t>(f2h(v.w)) << 16);
        __builtin_nontemporal_store(u, reinterpret_cast<cbx_u2v*>(p));
    }
};

__device__ __forceinline__ float get(const float4& v, int k) {
    return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}
__device__ __forceinline__ void set(float4& v, int k, float x) {
    if (k == 0) v.x = x; else if (k == 1) v.y = x; else if (k == 2) v.z = x; else v.w = x;
}

// ---- kernel arguments --------------------------------------------------------
// The compiler loads a kernel argument where it is first used, and sinks
// that load into a conditional block when only the block uses it (a store
// guarded by a bounds test, say): the block then waits for a second round
// of argument loads.  Naming the values here, at the top of the kernel,
// makes them part of the first round.
__device__ __forceinline__ void arg_now(const void* p) { asm volatile("" ::"s"(p)); }
__device__ __forceinline__ void arg_now(uint32_t v) { asm volatile("" ::"s"(v)); }

// ---- early stores ------------------------------------------------------------
// A row kernel that stores one output (the embedding sum, the residual sum)
// before its reductions: if some loads may still be pending when that store
// issues (loads the compiler sank into a conditional block, the affine
// vectors), the compiler waits for them at their first use after the store
// with vmcnt(0) -- and on this GPU family vmcnt counts stores as well, so
// the arithmetic after the reductions waits for the early store's write
// acknowledgement.  Waiting for every vector memory operation just before
// the early store (an s_waitcnt the compiler's wait placement accounts for)
// leaves only the store pending.  Call it where every lane passes (not
// inside the store's own condition).
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)

// ---- reductions ----------------------------------------------------------
// DPP move of a double (two 32-bit halves) inside each 16-lane row.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_mov_dpp(static_cast<int>(u & 0xffffffffu), CTRL, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_mov_dpp(static_cast<int>(u >> 32), CTRL, 0xf, 0xf, true);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                          static_cast<uint32_t>(lo));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<int>(u & 0xffffffffu), lane);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<int>(u >> 32), lane);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Sum over the 64 lanes of a wave, identical in every lane: a butterfly
// inside each 16-lane row with DPP (quad_perm [1,0,3,2], quad_perm
// [2,3,0,1], row_half_mirror, row_mirror -- each pairs lanes so both
// partners add the same two values), then the four row sums read from
// lanes 0/16/32/48 and added in a fixed order.  All 64 lanes must be active.
__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_f64<0xB1>(v);
    v += dpp_f64<0x4E>(v);
    v += dpp_f64<0x141>(v);
    v += dpp_f64<0x140>(v);
    const double r0 = readlane_f64(v, 0), r1 = readlane_f64(v, 16);
    const double r2 = readlane_f64(v, 32), r3 = readlane_f64(v, 48);
    return (r0 + r1) + (r2 + r3);
}

// Sum over the block in a fixed order (lanes in a butterfly, waves in index
// order), so results do not vary from run to run.  `scratch` holds one
// double per wave; the function may be called repeatedly with the same
// scratch (it synchronises before returning).
__device__ __forceinline__ double block_sum(double v, double* scratch) {
    v = wave_sum(v);
    const int lane = threadIdx.x % WAVE, wid = threadIdx.x / WAVE;
    const int nw = (blockDim.x + WAVE - 1) / WAVE;
    if (lane == 0) scratch[wid] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; i++) t += scratch[i];
    __syncthreads();
    return t;
}

// ---- activations (ggml-cpu scalar semantics) -----------------------------
#define CBX_SQRT_2_INV 0.70710678118654752440084436210484f

__device__ __forceinline__ float act_silu(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float act_softplus(float x) {
    return (x > 20.0f) ? x : logf(1.0f + expf(x));
}
// mish() = x * tanh(softplus(x)) (cfm_decoder.cpp:36-38).  ggml's softplus
// is log(t) with t = 1 + e^x rounded to f32 (x <= 20), and
// tanh(log t) = (t^2 - 1) / (t^2 + 1) = n / (n + 2) with n = u (u + 2),
// u = t - 1 (exact: t is in [1, 2^29]).  Evaluating that instead of logf and
// tanhf keeps the one rounding that dominates the composition (of t, which
// decides the result for x < -9) and costs one expf and a reciprocal; the
// other roundings of logf and tanhf are an ulp or two each.  Past 20
// softplus is x and tanhf(x) is 1: the result is x.
__device__ __forceinline__ float act_mish(float x) {
    if (x > 20.0f) return x;
    const float t = 1.0f + expf(x);
    const float u = t - 1.0f;
    const float n = u * (u + 2.0f);
    return x * (n * __builtin_amdgcn_rcpf(n + 2.0f));
}
__device__ __forceinline__ float act_gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * CBX_SQRT_2_INV));
}
// ggml_gelu (f32): x <= -10 -> 0, x >= 10 -> x, else the fp16 table entry
// of h = f16(x) (the table cbx_init uploads), read from global memory.
__device__ __forceinline__ float act_gelu_tab(const uint16_t* __restrict__ tab, float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return h2f(tab[f2h(x)]);
}

// The same function with the table read only where it is needed.  For
// |x| < 10 the result is a function of h = f16(x) alone.  The table's
// 0.5 xf (1 + tanh a), a = sqrt(2/pi) xf (1 + 0.044715 xf^2), equals
// g = xf q with q = 1 / (1 + e), e = 2^-w, w = xf (K1 + K2 xf^2) (the inner
// polynomial with one fused multiply-add), evaluated with the hardware exp2
// and reciprocal: q carries the reciprocal's and the addition's roundings
// and what the rounding of w does to e (ln 2 |dw| relative; it grows with
// |w| only where e is large).  The table's own f32 evaluation loses up to
// ~1/(2q) ulps in 1 + tanh a (a cancellation for a < 0).  The f16 rounding
// of g is kept when g lies more than 8 + 16/q = 24 + 16 e f32 ulps from an
// f16 rounding midpoint (its low 13 bits); otherwise (f16-subnormal g, or
// too close to a midpoint) the exact table entry is used.  x <= -10 reads
// entry 0 (GELU(+0) = +0, ggml's result there); lanes that need no entry
// all read entry 0 too, so the load touches a single cache line in the
// common case.  Because the result depends on h only, running every f16
// code through this function checks it for every input.
#define CBX_GELU_K1 2.3022081983f          // 2 sqrt(2/pi) log2(e)
#define CBX_GELU_K2 0.10294324967f         // K1 * 0.044715

struct GeluPart {
    uint32_t idx;   // table entry to read: h, or 0 when g's rounding is sure or x <= -10
    float    g;
    bool     sure;
};

__device__ __forceinline__ GeluPart gelu_part(float x) {
    const uint32_t h = f2h(x);
    const float xf = h2f(static_cast<uint16_t>(h));
    const float w = xf * __builtin_fmaf(CBX_GELU_K2, xf * xf, CBX_GELU_K1);
    const float e = __builtin_amdgcn_exp2f(-w);   // 1/q - 1
    const float q = __builtin_amdgcn_rcpf(e + 1.0f);
    const float g = xf * q;
    const int32_t d = static_cast<int32_t>(__builtin_bit_cast(uint32_t, g) & 0x1fffu) - 0x1000;
    // x <= -10 gives xf <= -10, w < -125.9 and an infinite margin: never sure
    const float margin = __builtin_fmaf(e, 16.0f, 24.0f);
    const bool neg10 = x <= -10.0f;
    // bitwise & keeps this branch-free, so the table loads of several
    // elements issue together
    const bool sure = (__builtin_fabsf(static_cast<float>(d)) > margin) & (__builtin_fabsf(g) >= 0x1p-14f);
    return GeluPart{(sure | neg10) ? 0u : h, g, sure};
}

__device__ __forceinline__ float gelu_finish(float x, const GeluPart& p, uint16_t tv) {
    const float r = h2f(p.sure ? static_cast<uint16_t>(f2h(p.g)) : tv);
    return x >= 10.0f ? x : r;
}

__device__ __forceinline__ float act_gelu_fast(const uint16_t* __restrict__ tab, float x) {
    const GeluPart p = gelu_part(x);
    return gelu_finish(x, p, tab[p.idx]);
}

// Four elements: the arithmetic first, then the four table reads together.
__device__ __forceinline__ float4 act_gelu_fast4(const uint16_t* __restrict__ tab, float4 x) {
    const GeluPart p0 = gelu_part(x.x), p1 = gelu_part(x.y), p2 = gelu_part(x.z), p3 = gelu_part(x.w);
    const uint16_t t0 = tab[p0.idx], t1 = tab[p1.idx], t2 = tab[p2.idx], t3 = tab[p3.idx];
    return make_float4(gelu_finish(x.x, p0, t0), gelu_finish(x.y, p1, t1), gelu_finish(x.z, p2, t2),
                       gelu_finish(x.w, p3, t3));
}

// ---- row addressing --------------------------------------------------------
// Byte offset of row r (rows enumerate ne[1], ne[2], ne[3] in that order).
// `flat` means the row strides are uniform (nb2 = nb1*ne1, nb3 = nb2*ne2, or
// the dimension is 1), so no division is needed; otherwise r is split.
__device__ __forceinline__ int64_t row_offset(const View& t, int64_t r, bool flat) {
    if (flat) return r * t.nb[1];
    const int64_t i3 = r / (t.ne[2] * t.ne[1]);
    const int64_t rem = r - i3 * t.ne[2] * t.ne[1];
    const int64_t i2 = rem / t.ne[1];
    const int64_t i1 = rem - i2 * t.ne[1];
    return i1 * t.nb[1] + i2 * t.nb[2] + i3 * t.nb[3];
}
__device__ __forceinline__ float act_leaky(float x, float ns) {
    return ((x > 0.f) ? x : 0.f) + ns * ((x < 0.0f) ? x : 0.f);
}

// Arguments of sin below this magnitude take sin_sq_small; larger ones (and
// NaN) take the library sinf.
constexpr float kSinSmall = 65536.0f;

// sin(x)^2 for |x| < 2^16.  Cody-Waite reduction x = q*pi/2 + r with pi/2
// split into three f32 parts P1 + P2 + P3: x - q*P1 is exact (x and q*P1
// are multiples of the last place of P1 or finer, and the difference is
// under 1), the q*P2 and q*P3 corrections round once each in their FMAs,
// and the remaining q * (pi/2 - P1 - P2 - P3) is below 2^-57; then the
// Taylor polynomial of sin r on |r| <= pi/4 (+ rounding slack): the first
// omitted term is r^11/11! < 2.2e-9, under half an f32 ulp of the result.
// sin(x)^2 = sin(r)^2 for even q, cos(r)^2 = 1 - sin(r)^2 for odd q (in one
// rounding; it is >= 1/2 on |r| <= pi/4, so nothing cancels).
__device__ __forceinline__ float sin_sq_small(float x) {
    const float q = rintf(x * 0x1.45f306p-1f);   // x * 2/pi
    float r = fmaf(q, -0x1.921fb6p+0f, x);
    r = fmaf(q, 0x1.777a5cp-25f, r);
    r = fmaf(q, 0x1.ee59dap-50f, r);
    const float r2 = r * r;
    float ps = fmaf(r2, 1.0f / 362880.0f, -1.0f / 5040.0f);
    ps = fmaf(ps, r2, 1.0f / 120.0f);
    ps = fmaf(ps, r2, -1.0f / 6.0f);
    ps = fmaf(ps * r2, r, r);
    return (static_cast<int>(q) & 1) ? fmaf(-ps, ps, 1.0f) : ps * ps;
}

// snake(x) = x + sin(x*a)^2 * a_inv in the order of the five ggml ops of
// snake() (mul, sin, sqr, mul, add), sin^2 from sin_sq_small below 2^16
// and from the library sinf (a rarely taken branch) above.
__device__ __forceinline__ float snake_elem(float xv, float a, float ai) {
    const float xa = xv * a;
    float s2;
    if (fabsf(xa) < kSinSmall) {
        s2 = sin_sq_small(xa);
    } else {
        const float sn = sinf(xa);
        s2 = sn * sn;
    }
    const float m = s2 * ai;
    return xv + m;
}

// Runtime-selected activation for epilogues (op is uniform per launch).
__device__ __forceinline__ float apply_act(int op, float x, const uint16_t* tab, float param) {
    switch (op) {
        case CBX_UNARY_GELU:     return act_gelu_tab(tab, x);
        case CBX_UNARY_GELU_ERF: return act_gelu_erf(x);
        case CBX_UNARY_SILU:     return act_silu(x);
        case CBX_UNARY_TANH:     return tanhf(x);
        case CBX_UNARY_SOFTPLUS: return act_softplus(x);
        case CBX_UNARY_SIN:      return sinf(x);
        case CBX_UNARY_SQR:      return x * x;
        case CBX_UNARY_MISH:     return act_mish(x);
        case UNARY_LEAKY:        return act_leaky(x, param);
        default:                 return x;
    }
}

// The activation over every element a thread holds, the switch taken once:
// per element (apply_act in a loop) the branches around each case keep the
// compiler from interleaving independent elements, and a transcendental's
// latency is then paid element after element.
template <int NV>
__device__ __forceinline__ void apply_act_vec(int op, float4 (&v)[NV], const uint16_t* tab, float param) {
#define CBX_ACT_ALL(expr)                                         \
    _Pragma("unroll") for (int k = 0; k < NV; k++) {              \
        _Pragma("unroll") for (int e = 0; e < 4; e++) {           \
            const float x = get(v[k], e);                         \
            set(v[k], e, (expr));                                 \
        }                                                         \
    }
    switch (op) {
        case CBX_UNARY_GELU:
#pragma unroll
            for (int k = 0; k < NV; k++) v[k] = act_gelu_fast4(tab, v[k]);
            break;
        case CBX_UNARY_GELU_ERF: CBX_ACT_ALL(act_gelu_erf(x)); break;
        case CBX_UNARY_SILU:     CBX_ACT_ALL(act_silu(x)); break;
        case CBX_UNARY_TANH:     CBX_ACT_ALL(tanhf(x)); break;
        case CBX_UNARY_SOFTPLUS: CBX_ACT_ALL(act_softplus(x)); break;
        case CBX_UNARY_SIN:      CBX_ACT_ALL(sinf(x)); break;
        case CBX_UNARY_SQR:      CBX_ACT_ALL(x * x); break;
        case CBX_UNARY_MISH:     CBX_ACT_ALL(act_mish(x)); break;
        case UNARY_LEAKY:        CBX_ACT_ALL(act_leaky(x, param)); break;
        default: break;
    }
#undef CBX_ACT_ALL
}

}  // namespace cbx
