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

__device__ __forceinline__ float get(const float4& v, int k) {
    return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}
__device__ __forceinline__ void set(float4& v, int k, float x) {
    if (k == 0) v.x = x; else if (k == 1) v.y = x; else if (k == 2) v.z = x; else v.w = x;
}

// ---- reductions ----------------------------------------------------------
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int off = WAVE / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, WAVE);
    return v;
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
__device__ __forceinline__ float act_mish(float x) {
    const float sp = act_softplus(x);
    const float t = tanhf(sp);
    return x * t;
}
__device__ __forceinline__ float act_gelu_erf(float x) {
    return 0.5f * x * (1.0f + erff(x * CBX_SQRT_2_INV));
}
__device__ __forceinline__ float act_gelu_tab(const uint16_t* __restrict__ tab, float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return h2f(tab[f2h(x)]);
}
__device__ __forceinline__ float act_leaky(float x, float ns) {
    return ((x > 0.f) ? x : 0.f) + ns * ((x < 0.0f) ? x : 0.f);
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

}  // namespace cbx
