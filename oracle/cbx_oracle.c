/*
 * cbx_oracle.c -- CPU restatement of ggml-cpu op semantics for the fused
 * layer-op path.  TEST INFRASTRUCTURE ONLY (see cbx_oracle.h).
 *
 * Built with -ffp-contract=off: every float expression below is evaluated
 * with one IEEE rounding per operation, in the order written.  The ggml
 * functions being restated are named ("ggml: <function>") and the reference
 * call site that depends on each is cited.  ggml is an absent submodule of
 * the reference (chatterbox-cpp/third_party/ggml, .gitmodules:1-3, v0.12.0);
 * its behaviour is restated here from the published sources' algorithms.
 *
 * Threading mirrors ggml-cpu: rows are dealt to threads round-robin
 * (ir = ith; ir < nr; ir += nth); results do not depend on the thread count.
 */
#include "cbx_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define GELU_COEF_A    0.044715f
#define SQRT_2_OVER_PI 0.79788456080286535587989211986876f
#define SQRT_2_INV     0.70710678118654752440084436210484f

/* ------------------------------------------------------------------------ */
/* f16 <-> f32                                                              */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ggml: GGML_CPU_FP16_TO_FP32 -- exact widening (F16C vcvtph2ps on x86).
 * Used by get_rows on f16 tables (t3.cpp:440-455, flow_encoder.cpp:588). */
float cbxo_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp  = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0x1f) {                       /* inf / nan: keep payload */
        return u2f(sign | 0x7f800000u | (mant << 13));
    }
    if (exp == 0) {
        if (mant == 0) return u2f(sign);     /* +-0 */
        /* subnormal: value = mant * 2^-24, exactly representable in f32 */
        int e = -1;
        do { mant <<= 1; e++; } while ((mant & 0x400u) == 0);
        mant &= 0x3ffu;
        return u2f(sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13));
    }
    return u2f(sign | ((exp + 112u) << 23) | (mant << 13));
}

/* ggml: GGML_CPU_FP32_TO_FP16 -- round to nearest, ties to even
 * (F16C vcvtps2ph imm 0 on x86).  NaN is quieted, top payload bits kept. */
uint16_t cbxo_fp32_to_fp16(float f) {
    const uint32_t x    = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax   = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 */
    if (ax < 0x38800000u) {                                      /* < 2^-14 */
        if (ax <= 0x33000000u) return sign;                      /* <= 2^-25 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int)(ax >> 23);                 /* 14..24 */
        uint32_t h = m >> shift;
        const uint32_t rem  = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu));
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;     /* may carry into exp */
    return (uint16_t)(sign | h);
}

/* ------------------------------------------------------------------------ */
/* Q8_0                                                                     */
/* ------------------------------------------------------------------------ */

/* ggml: quantize_row_q8_0_ref -- d = amax/127, q = roundf(x * (1/d)).
 * Only builds test tables; the path under test is the dequantization. */
void cbxo_quantize_row_q8_0(const float* x, void* y, int64_t k) {
    const int64_t nb = k / CBXO_QK8_0;
    uint8_t* out = (uint8_t*)y;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < CBXO_QK8_0; j++) {
            const float v = fabsf(x[i * CBXO_QK8_0 + j]);
            amax = amax > v ? amax : v;
        }
        const float d  = amax / ((1 << 7) - 1);
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t dh = cbxo_fp32_to_fp16(d);
        uint8_t* blk = out + i * CBXO_Q8_0_BLOCK_BYTES;
        memcpy(blk, &dh, 2);
        for (int j = 0; j < CBXO_QK8_0; j++) {
            const float x0 = x[i * CBXO_QK8_0 + j] * id;
            const int8_t q = (int8_t)roundf(x0);
            memcpy(blk + 2 + j, &q, 1);
        }
    }
}

/* ggml: dequantize_row_q8_0 -- y = (float)qs[j] * fp16_to_fp32(d), one f32
 * multiply per element.  Bit-exact target for the Q8_0 gather. */
void cbxo_dequantize_row_q8_0(const void* x, float* y, int64_t k) {
    const int64_t nb = k / CBXO_QK8_0;
    const uint8_t* in = (const uint8_t*)x;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t* blk = in + i * CBXO_Q8_0_BLOCK_BYTES;
        uint16_t dh;
        memcpy(&dh, blk, 2);
        const float d = cbxo_fp16_to_fp32(dh);
        for (int j = 0; j < CBXO_QK8_0; j++) {
            int8_t q;
            memcpy(&q, blk + 2 + j, 1);
            y[i * CBXO_QK8_0 + j] = (float)q * d;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* element helpers                                                          */
/* ------------------------------------------------------------------------ */

static inline int64_t nrows(const cbxo_tensor* t) { return t->ne[1] * t->ne[2] * t->ne[3]; }
static inline int64_t nelem(const cbxo_tensor* t) { return t->ne[0] * nrows(t); }

static inline char* row_ptr(const cbxo_tensor* t, int64_t i1, int64_t i2, int64_t i3) {
    return (char*)t->data + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
}

static inline void split_row(const cbxo_tensor* t, int64_t ir, int64_t* i1, int64_t* i2, int64_t* i3) {
    *i3 = ir / (t->ne[2] * t->ne[1]);
    *i2 = (ir - *i3 * t->ne[2] * t->ne[1]) / t->ne[1];
    *i1 = ir - *i3 * t->ne[2] * t->ne[1] - *i2 * t->ne[1];
}

static inline float load_elem(const cbxo_tensor* t, const char* row, int64_t i0) {
    if (t->type == CBXO_TYPE_F16) {
        uint16_t h;
        memcpy(&h, row + i0 * t->nb[0], 2);
        return cbxo_fp16_to_fp32(h);
    }
    float f;
    memcpy(&f, row + i0 * t->nb[0], 4);
    return f;
}

static inline void store_elem(const cbxo_tensor* t, char* row, int64_t i0, float v) {
    if (t->type == CBXO_TYPE_F16) {
        const uint16_t h = cbxo_fp32_to_fp16(v);
        memcpy(row + i0 * t->nb[0], &h, 2);
    } else {
        memcpy(row + i0 * t->nb[0], &v, 4);
    }
}

static int same_shape(const cbxo_tensor* a, const cbxo_tensor* b) {
    for (int i = 0; i < 4; i++) if (a->ne[i] != b->ne[i]) return 0;
    return 1;
}

static int is_float_type(int t) { return t == CBXO_TYPE_F32 || t == CBXO_TYPE_F16; }

static int can_repeat(const cbxo_tensor* small, const cbxo_tensor* big) {
    for (int i = 0; i < 4; i++) {
        if (small->ne[i] <= 0 || big->ne[i] % small->ne[i] != 0) return 0;
    }
    return 1;
}

/* contiguous f32 temporary with the shape of t */
static cbxo_tensor make_tmp_f32(const cbxo_tensor* t) {
    cbxo_tensor r;
    memset(&r, 0, sizeof(r));
    r.type = CBXO_TYPE_F32;
    for (int i = 0; i < 4; i++) r.ne[i] = t->ne[i];
    r.nb[0] = 4;
    r.nb[1] = r.nb[0] * (size_t)r.ne[0];
    r.nb[2] = r.nb[1] * (size_t)r.ne[1];
    r.nb[3] = r.nb[2] * (size_t)r.ne[2];
    r.data = malloc((size_t)nelem(t) * 4 + 16);
    return r;
}

/* ------------------------------------------------------------------------ */
/* GELU fp16 table                                                          */
/* ------------------------------------------------------------------------ */

/* ggml: ggml_gelu_f32 = 0.5x(1 + tanhf(SQRT_2_OVER_PI x (1 + GELU_COEF_A x^2)));
 * the NumPy oracle text is reference_t3_forward.py:73-77 (gelu_new). */
float cbxo_gelu_f32(float x, int fma_variant) {
    float inner;
    if (fma_variant) inner = fmaf(GELU_COEF_A * x, x, 1.0f);
    else             inner = 1.0f + GELU_COEF_A * x * x;
    return 0.5f * x * (1.0f + tanhf(SQRT_2_OVER_PI * x * inner));
}

/* ggml: ggml_cpu_init fills ggml_table_gelu_f16[i] = f16(gelu(f32(i))). */
void cbxo_gelu_table(uint16_t* out, int fma_variant) {
    for (int i = 0; i < 65536; i++) {
        const float f = cbxo_fp16_to_fp32((uint16_t)i);
        out[i] = cbxo_fp32_to_fp16(cbxo_gelu_f32(f, fma_variant));
    }
}

static uint16_t g_gelu_table[65536];
static int g_gelu_ready = 0;

static const uint16_t* gelu_table(void) {
    if (!g_gelu_ready) {
#pragma omp critical(cbxo_gelu_init)
        {
            if (!g_gelu_ready) {
                cbxo_gelu_table(g_gelu_table, 0);
                g_gelu_ready = 1;
            }
        }
    }
    return g_gelu_table;
}

/* ggml: ggml_vec_gelu_f32 (GGML_GELU_FP16 defined): x <= -10 -> 0,
 * x >= 10 -> x, otherwise the table entry of f16(x).  t3.cpp:537. */
static inline float gelu_tab_f32(const uint16_t* tab, float x) {
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return cbxo_fp16_to_fp32(tab[cbxo_fp32_to_fp16(x)]);
}

/* ------------------------------------------------------------------------ */
/* scalar op bodies                                                         */
/* ------------------------------------------------------------------------ */

/* ggml: ggml_silu_f32 (cfm_decoder.cpp:466, flow_encoder.cpp:402) */
static inline float op_silu(float x) { return x / (1.0f + expf(-x)); }
/* ggml: op_softplus, threshold 20 (cfm_decoder.cpp:37) */
static inline float op_softplus(float x) { return (x > 20.0f) ? x : logf(1.0f + expf(x)); }
/* ggml: ggml_vec_gelu_erf_f32 (cfm_decoder.cpp:239, s3enc.cpp:177) */
static inline float op_gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * SQRT_2_INV)); }
/* mish() helper: mul(x, tanh(softplus(x))), each step rounded to f32 */
static inline float op_mish(float x) {
    const float sp = op_softplus(x);
    const float t  = tanhf(sp);
    return x * t;
}
/* ggml: ggml_vec_leaky_relu_f32 (hift_vocoder.cpp:686,748; flow_encoder.cpp:454) */
static inline float op_leaky(float x, float ns) {
    return ((x > 0.f) ? x : 0.f) + ns * ((x < 0.0f) ? x : 0.f);
}

static float unary_f32(int op, const uint16_t* tab, float x) {
    switch (op) {
        case CBXO_UNARY_GELU:     return gelu_tab_f32(tab, x);
        case CBXO_UNARY_GELU_ERF: return op_gelu_erf(x);
        case CBXO_UNARY_SILU:     return op_silu(x);
        case CBXO_UNARY_TANH:     return tanhf(x);
        case CBXO_UNARY_SOFTPLUS: return op_softplus(x);
        case CBXO_UNARY_SIN:      return sinf(x);
        case CBXO_UNARY_SQR:      return x * x;
        case CBXO_UNARY_MISH:     return op_mish(x);
        default:                  return NAN;
    }
}

/* ------------------------------------------------------------------------ */
/* get_rows                                                                 */
/* ------------------------------------------------------------------------ */

/* ggml: ggml_compute_forward_get_rows -- dst[:, i10, i11, i12] =
 * to_f32(src[:, ids[i10, i11, i12], i11, i12]); out-of-range ids abort in
 * ggml (GGML_ASSERT), here they return -2.  t3.cpp:440-455. */
int cbxo_get_rows(const cbxo_tensor* src, const cbxo_tensor* ids,
                  cbxo_tensor* dst, int nth) {
    if (ids->type != CBXO_TYPE_I32 || dst->type != CBXO_TYPE_F32) return -1;
    if (src->type == CBXO_TYPE_Q8_0 && src->ne[0] % CBXO_QK8_0) return -1;
    const int64_t nc = src->ne[0];
    const int64_t nr = ids->ne[0] * ids->ne[1] * ids->ne[2];
    int bad = 0;
#pragma omp parallel num_threads(nth) reduction(| : bad)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t i = ith; i < nr; i += nt) {
            const int64_t i12 = i / (ids->ne[1] * ids->ne[0]);
            const int64_t i11 = (i - i12 * ids->ne[1] * ids->ne[0]) / ids->ne[0];
            const int64_t i10 = i - i12 * ids->ne[1] * ids->ne[0] - i11 * ids->ne[0];
            int32_t i01;
            memcpy(&i01, (const char*)ids->data + i10 * ids->nb[0] + i11 * ids->nb[1] + i12 * ids->nb[2], 4);
            if (i01 < 0 || i01 >= src->ne[1]) { bad = 1; continue; }
            const char* s = (const char*)src->data + i01 * src->nb[1] + i11 * src->nb[2] + i12 * src->nb[3];
            float* d = (float*)row_ptr(dst, i10, i11, i12);
            if (src->type == CBXO_TYPE_Q8_0) {
                cbxo_dequantize_row_q8_0(s, d, nc);
            } else if (src->type == CBXO_TYPE_F16) {
                for (int64_t j = 0; j < nc; j++) {
                    uint16_t h;
                    memcpy(&h, s + j * src->nb[0], 2);
                    d[j] = cbxo_fp16_to_fp32(h);
                }
            } else {
                for (int64_t j = 0; j < nc; j++) memcpy(&d[j], s + j * src->nb[0], 4);
            }
        }
    }
    return bad ? -2 : 0;
}

/* ------------------------------------------------------------------------ */
/* binary broadcast ops                                                     */
/* ------------------------------------------------------------------------ */

/* ggml: ggml_compute_forward_add/mul (f32) -- b is repeated over a by index
 * modulo ne1x in every dimension.  layer_norm's mul/add (cfm_decoder.cpp:32),
 * snake's mul(alpha) (hift_vocoder.cpp:68). */
static int binary_op(int is_mul, const cbxo_tensor* a, const cbxo_tensor* b,
                     cbxo_tensor* dst, int nth) {
    if (!same_shape(a, dst) || !can_repeat(b, a)) return -1;
    if (!is_float_type(a->type) || !is_float_type(b->type) || !is_float_type(dst->type)) return -1;
    const int64_t nr = nrows(a);
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(a, ir, &i1, &i2, &i3);
            const char* ra = row_ptr(a, i1, i2, i3);
            const char* rb = row_ptr(b, i1 % b->ne[1], i2 % b->ne[2], i3 % b->ne[3]);
            char* rd = row_ptr(dst, i1, i2, i3);
            for (int64_t i0 = 0; i0 < a->ne[0]; i0++) {
                const float x = load_elem(a, ra, i0);
                const float y = load_elem(b, rb, i0 % b->ne[0]);
                store_elem(dst, rd, i0, is_mul ? x * y : x + y);
            }
        }
    }
    return 0;
}

int cbxo_add(const cbxo_tensor* a, const cbxo_tensor* b, cbxo_tensor* dst, int nth) {
    return binary_op(0, a, b, dst, nth);
}
int cbxo_mul(const cbxo_tensor* a, const cbxo_tensor* b, cbxo_tensor* dst, int nth) {
    return binary_op(1, a, b, dst, nth);
}

/* ------------------------------------------------------------------------ */
/* norms                                                                    */
/* ------------------------------------------------------------------------ */

/* ggml: ggml_compute_forward_norm_f32 -- mean = (float)(sum_f64 x) / n;
 * v = x - mean; var = (float)(sum_f64 (v*v) / n); y = v * (1/sqrtf(var+eps)).
 * Called through layer_norm() at t3.cpp:465,531,545, cfm_decoder.cpp:31,
 * flow_encoder.cpp:60, s3enc.cpp:102. */
static void norm_row(const float* x, float* y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)x[i];
    const float sumf = (float)sum;
    const float mean = sumf / (float)n;
    double sum2 = 0.0;
    for (int64_t i = 0; i < n; i++) {
        const float v = x[i] - mean;
        y[i] = v;
        sum2 += (double)(v * v);
    }
    const float variance = (float)(sum2 / (double)n);
    const float scale = 1.0f / sqrtf(variance + eps);
    for (int64_t i = 0; i < n; i++) y[i] *= scale;
}

/* ggml: ggml_compute_forward_rms_norm_f32 -- ms = (float)(sum_f64 (x*x) / n);
 * y = x * (1/sqrtf(ms+eps)).  No call site in the reference (Turbo T3 uses
 * LayerNorm); the decode-step workloads use it. */
static void rms_norm_row(const float* x, float* y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * scale;
}

typedef void (*row_fn)(const float*, float*, int64_t, float);

/* f32 or f16 rows; f16 rows are widened, normalised in f32, rounded once. */
static int row_norm_op(row_fn fn, const cbxo_tensor* x, float eps, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || !is_float_type(x->type) || !is_float_type(dst->type)) return -1;
    if (eps < 0.0f) return -1;
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        float* xi = (float*)malloc((size_t)n * 4 + 16);
        float* yo = (float*)malloc((size_t)n * 4 + 16);
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(x, ir, &i1, &i2, &i3);
            const char* rx = row_ptr(x, i1, i2, i3);
            char* rd = row_ptr(dst, i1, i2, i3);
            for (int64_t i = 0; i < n; i++) xi[i] = load_elem(x, rx, i);
            fn(xi, yo, n, eps);
            for (int64_t i = 0; i < n; i++) store_elem(dst, rd, i, yo[i]);
        }
        free(xi);
        free(yo);
    }
    return 0;
}

int cbxo_norm(const cbxo_tensor* x, float eps, cbxo_tensor* dst, int nth) {
    return row_norm_op(norm_row, x, eps, dst, nth);
}
int cbxo_rms_norm(const cbxo_tensor* x, float eps, cbxo_tensor* dst, int nth) {
    return row_norm_op(rms_norm_row, x, eps, dst, nth);
}

/* ggml: ggml_compute_forward_group_norm_f32 -- channels are ne[2]; group g
 * covers channels [g*cpg, min((g+1)*cpg, C)) with cpg = ceil(C/G), and all
 * of ne[0] x ne[1]; sums are f64, row partials added per row.  No call site
 * in the reference (its CFM uses LayerNorm+Mish, cfm_decoder.cpp:133-149);
 * the CFM group-norm workload uses it. */
int cbxo_group_norm(const cbxo_tensor* x, int n_groups, float eps, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    if (n_groups <= 0 || eps < 0.0f) return -1;
    const int64_t ne00 = x->ne[0], ne01 = x->ne[1], C = x->ne[2], ne03 = x->ne[3];
    const int64_t cpg = (C + n_groups - 1) / n_groups;
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t i = ith; i < n_groups; i += nt) {
            const int64_t start = i * cpg;
            int64_t end = start + cpg;
            if (end > C) end = C;
            if (start >= end) continue;
            const int64_t step = end - start;
            for (int64_t i03 = 0; i03 < ne03; i03++) {
                double sum = 0.0;
                for (int64_t i02 = start; i02 < end; i02++) {
                    for (int64_t i01 = 0; i01 < ne01; i01++) {
                        const float* xr = (const float*)row_ptr(x, i01, i02, i03);
                        double sumr = 0.0;
                        for (int64_t i00 = 0; i00 < ne00; i00++) sumr += (double)xr[i00];
                        sum += sumr;
                    }
                }
                const float mean = (float)(sum / (double)(ne00 * ne01 * step));
                double sum2 = 0.0;
                for (int64_t i02 = start; i02 < end; i02++) {
                    for (int64_t i01 = 0; i01 < ne01; i01++) {
                        const float* xr = (const float*)row_ptr(x, i01, i02, i03);
                        float* yr = (float*)row_ptr(dst, i01, i02, i03);
                        double sumr = 0.0;
                        for (int64_t i00 = 0; i00 < ne00; i00++) {
                            const float v = xr[i00] - mean;
                            yr[i00] = v;
                            sumr += (double)(v * v);
                        }
                        sum2 += sumr;
                    }
                }
                const float variance = (float)(sum2 / (double)(ne00 * ne01 * step));
                const float scale = 1.0f / sqrtf(variance + eps);
                for (int64_t i02 = start; i02 < end; i02++) {
                    for (int64_t i01 = 0; i01 < ne01; i01++) {
                        float* yr = (float*)row_ptr(dst, i01, i02, i03);
                        for (int64_t i00 = 0; i00 < ne00; i00++) yr[i00] *= scale;
                    }
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* unary / glu                                                              */
/* ------------------------------------------------------------------------ */

/* ggml unary ops on f32 and f16 tensors (f16: widen, op in f32, round; the
 * f16 GELU is the bare table lookup ggml_vec_gelu_f16). */
int cbxo_unary(int op, const cbxo_tensor* x, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || !is_float_type(x->type) || x->type != dst->type) return -1;
    if (op < 0 || op > CBXO_UNARY_MISH) return -1;
    const uint16_t* tab = gelu_table();
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(x, ir, &i1, &i2, &i3);
            const char* rx = row_ptr(x, i1, i2, i3);
            char* rd = row_ptr(dst, i1, i2, i3);
            for (int64_t i = 0; i < n; i++) {
                if (op == CBXO_UNARY_GELU && x->type == CBXO_TYPE_F16) {
                    uint16_t h;
                    memcpy(&h, rx + i * x->nb[0], 2);
                    memcpy(rd + i * dst->nb[0], &tab[h], 2);
                } else {
                    store_elem(dst, rd, i, unary_f32(op, tab, load_elem(x, rx, i)));
                }
            }
        }
    }
    return 0;
}

int cbxo_leaky_relu(const cbxo_tensor* x, float slope, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || !is_float_type(x->type) || x->type != dst->type) return -1;
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(x, ir, &i1, &i2, &i3);
            const char* rx = row_ptr(x, i1, i2, i3);
            char* rd = row_ptr(dst, i1, i2, i3);
            for (int64_t i = 0; i < n; i++) store_elem(dst, rd, i, op_leaky(load_elem(x, rx, i), slope));
        }
    }
    return 0;
}

/* ggml: ggml_vec_swiglu_f32/f16 -- y = silu(g) * u (ggml_swiglu_split).  No
 * call site in the reference; the decode-step workloads use it. */
int cbxo_swiglu(const cbxo_tensor* g, const cbxo_tensor* u, cbxo_tensor* dst, int nth) {
    if (!same_shape(g, dst) || !same_shape(u, dst)) return -1;
    if (!is_float_type(g->type) || g->type != u->type || g->type != dst->type) return -1;
    const int64_t nr = nrows(g), n = g->ne[0];
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(g, ir, &i1, &i2, &i3);
            const char* rg = row_ptr(g, i1, i2, i3);
            const char* ru = row_ptr(u, i1, i2, i3);
            char* rd = row_ptr(dst, i1, i2, i3);
            for (int64_t i = 0; i < n; i++) {
                const float gi = load_elem(g, rg, i);
                const float ui = load_elem(u, ru, i);
                store_elem(dst, rd, i, op_silu(gi) * ui);
            }
        }
    }
    return 0;
}

/* ggml: ggml_compute_forward_dup / ggml_cast between f32 and f16
 * (t3.cpp:441,447,454).  Element-wise convert with RNE on narrowing. */
int cbxo_cpy(const cbxo_tensor* src, cbxo_tensor* dst, int nth) {
    if (nelem(src) != nelem(dst) || !is_float_type(src->type) || !is_float_type(dst->type)) return -1;
    if (!same_shape(src, dst)) return -1;
    const int64_t nr = nrows(src), n = src->ne[0];
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(src, ir, &i1, &i2, &i3);
            const char* rs = row_ptr(src, i1, i2, i3);
            char* rd = row_ptr(dst, i1, i2, i3);
            for (int64_t i = 0; i < n; i++) {
                if (src->type == dst->type) {
                    memcpy(rd + i * dst->nb[0], rs + i * src->nb[0], src->type == CBXO_TYPE_F16 ? 2 : 4);
                } else {
                    store_elem(dst, rd, i, load_elem(src, rs, i));
                }
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* RoPE                                                                     */
/* ------------------------------------------------------------------------ */

/* ggml: ggml_rope_yarn_corr_dim / ggml_rope_yarn_corr_dims */
static float corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * (float)M_PI)) / (2 * logf(base));
}
void cbxo_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base,
                              float beta_fast, float beta_slow, float dims[2]) {
    const float start = floorf(corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base));
    const float end   = ceilf(corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base));
    dims[0] = start > 0.0f ? start : 0.0f;
    dims[1] = end < (float)(n_dims - 1) ? end : (float)(n_dims - 1);
}

/* ggml: rope_yarn_ramp / rope_yarn */
static float yarn_ramp(float low, float high, int64_t i0) {
    const float d = high - low;
    const float y = ((float)(i0 / 2) - low) / (d > 0.001f ? d : 0.001f);
    const float c = y < 0.0f ? 0.0f : y;
    return 1.0f - (c < 1.0f ? c : 1.0f);
}
static void rope_yarn(float theta_extrap, float freq_scale, const float corr_dims[2], int64_t i0,
                      float ext_factor, float mscale, float* cos_theta, float* sin_theta) {
    const float theta_interp = freq_scale * theta_extrap;
    float theta = theta_interp;
    if (ext_factor != 0.0f) {
        const float ramp_mix = yarn_ramp(corr_dims[0], corr_dims[1], i0) * ext_factor;
        theta = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
    }
    *cos_theta = cosf(theta) * mscale;
    *sin_theta = sinf(theta) * mscale;
}

/* ggml: ggml_rope_cache_init -- theta starts at the position and is
 * multiplied by theta_scale once per pair (an iterated f32 product, not
 * pow per index).  s3enc.cpp:215-229 is the reference's call. */
void cbxo_rope_cache_init(float theta_base, float freq_scale, const float* freq_factors,
                          const float corr_dims[2], int64_t ne0, float ext_factor, float mscale,
                          float* cache, float sin_sign, float theta_scale) {
    float theta = theta_base;
    for (int64_t i0 = 0; i0 < ne0; i0 += 2) {
        const float ff = freq_factors ? freq_factors[i0 / 2] : 1.0f;
        rope_yarn(theta / ff, freq_scale, corr_dims, i0, ext_factor, mscale, &cache[i0 + 0], &cache[i0 + 1]);
        cache[i0 + 1] *= sin_sign;
        theta *= theta_scale;
    }
}

/* ggml: ggml_compute_forward_rope (forward, modes NORMAL and NEOX) --
 * x ne = (head_dim, n_head, n_tok, batch), pos[i2] is the token position;
 * dims >= n_dims are copied.  NEOX pairs (i, i + n_dims/2). */
int cbxo_rope_ext(const cbxo_tensor* x, const cbxo_tensor* pos, const float* freq_factors,
                  int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
                  float ext_factor, float attn_factor, float beta_fast, float beta_slow,
                  cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || !is_float_type(x->type) || x->type != dst->type) return -1;
    if (pos->type != CBXO_TYPE_I32 || pos->ne[0] != x->ne[2]) return -1;
    if (n_dims <= 0 || n_dims % 2 || n_dims > x->ne[0]) return -1;
    if (mode != 0 && mode != 2) return -1;
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    float corr_dims[2];
    cbxo_rope_yarn_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, corr_dims);
    const int64_t ne0 = x->ne[0], ne1 = x->ne[1], ne2 = x->ne[2], ne3 = x->ne[3];
    const int64_t nrow2 = ne2 * ne3;
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        float* cache = (float*)malloc((size_t)ne0 * 4 + 16);
        for (int64_t r = ith; r < nrow2; r += nt) {
            const int64_t i3 = r / ne2, i2 = r % ne2;
            int32_t p;
            memcpy(&p, (const char*)pos->data + i2 * pos->nb[0], 4);
            cbxo_rope_cache_init((float)p, freq_scale, freq_factors, corr_dims, ne0, ext_factor,
                                 attn_factor, cache, 1.0f, theta_scale);
            for (int64_t i1 = 0; i1 < ne1; i1++) {
                const char* rs = row_ptr(x, i1, i2, i3);
                char* rd = row_ptr(dst, i1, i2, i3);
                for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
                    const float c = cache[i0 + 0], s = cache[i0 + 1];
                    const int64_t ia = (mode == 2) ? i0 / 2 : i0;
                    const int64_t ib = (mode == 2) ? i0 / 2 + n_dims / 2 : i0 + 1;
                    const float x0 = load_elem(x, rs, ia);
                    const float x1 = load_elem(x, rs, ib);
                    store_elem(dst, rd, ia, x0 * c - x1 * s);
                    store_elem(dst, rd, ib, x0 * s + x1 * c);
                }
                for (int64_t i0 = n_dims; i0 < ne0; i0++) {
                    if (x->type == CBXO_TYPE_F16) memcpy(rd + i0 * dst->nb[0], rs + i0 * x->nb[0], 2);
                    else memcpy(rd + i0 * dst->nb[0], rs + i0 * x->nb[0], 4);
                }
            }
        }
        free(cache);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* compositions                                                             */
/* ------------------------------------------------------------------------ */

static void free_tmp(cbxo_tensor* t) { free(t->data); t->data = NULL; }

/* widen x to a contiguous f32 tensor (exact) */
static cbxo_tensor widen(const cbxo_tensor* x, int nth) {
    cbxo_tensor t = make_tmp_f32(x);
    cbxo_cpy(x, &t, nth);
    return t;
}

/* layer_norm() = ggml_norm -> ggml_mul(w) -> ggml_add(b), each an f32 tensor
 * (cfm_decoder.cpp:29-33, t3.cpp:465-466).  f16 x/dst: f32 inside, one
 * rounding at the end. */
int cbxo_layer_norm(const cbxo_tensor* x, const cbxo_tensor* w, const cbxo_tensor* b,
                    float eps, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || !is_float_type(x->type) || !is_float_type(dst->type)) return -1;
    if ((w && !can_repeat(w, x)) || (b && !can_repeat(b, x))) return -1;
    cbxo_tensor xf = widen(x, nth);
    cbxo_tensor t = make_tmp_f32(x);
    int rc = cbxo_norm(&xf, eps, &t, nth);
    if (!rc && w) rc = cbxo_mul(&t, w, &t, nth);
    if (!rc && b) rc = cbxo_add(&t, b, &t, nth);
    if (!rc) rc = cbxo_cpy(&t, dst, nth);
    free_tmp(&xf);
    free_tmp(&t);
    return rc;
}

int cbxo_rms_norm_mul(const cbxo_tensor* x, const cbxo_tensor* g, float eps,
                      cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || !is_float_type(x->type) || !is_float_type(dst->type)) return -1;
    if (g && !can_repeat(g, x)) return -1;
    cbxo_tensor xf = widen(x, nth);
    cbxo_tensor t = make_tmp_f32(x);
    int rc = cbxo_rms_norm(&xf, eps, &t, nth);
    if (!rc && g) rc = cbxo_mul(&t, g, &t, nth);
    if (!rc) rc = cbxo_cpy(&t, dst, nth);
    free_tmp(&xf);
    free_tmp(&t);
    return rc;
}

int cbxo_group_norm_affine(const cbxo_tensor* x, int n_groups, float eps,
                           const cbxo_tensor* w, const cbxo_tensor* b, int fuse_mish,
                           cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    if ((w && !can_repeat(w, x)) || (b && !can_repeat(b, x))) return -1;
    cbxo_tensor t = make_tmp_f32(x);
    int rc = cbxo_group_norm(x, n_groups, eps, &t, nth);
    if (!rc && w) rc = cbxo_mul(&t, w, &t, nth);
    if (!rc && b) rc = cbxo_add(&t, b, &t, nth);
    if (!rc && fuse_mish) rc = cbxo_unary(CBXO_UNARY_MISH, &t, &t, nth);
    if (!rc) rc = cbxo_cpy(&t, dst, nth);
    free_tmp(&t);
    return rc;
}

/* snake(): xa = mul(x, alpha); s = sin(xa); s2 = sqr(s); m = mul(s2, alpha_inv);
 * y = add(x, m).  hift_vocoder.cpp:64-73; alpha_inv = 1/(alpha + 1e-9) is
 * precomputed by the caller as at hift_vocoder.cpp:413-427. */
int cbxo_snake(const cbxo_tensor* x, const cbxo_tensor* alpha, const cbxo_tensor* alpha_inv,
               cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    if (!can_repeat(alpha, x) || !can_repeat(alpha_inv, x)) return -1;
    if (alpha->type != CBXO_TYPE_F32 || alpha_inv->type != CBXO_TYPE_F32) return -1;
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel num_threads(nth)
    {
        const int ith = omp_get_thread_num(), nt = omp_get_num_threads();
        for (int64_t ir = ith; ir < nr; ir += nt) {
            int64_t i1, i2, i3;
            split_row(x, ir, &i1, &i2, &i3);
            const float* rx = (const float*)row_ptr(x, i1, i2, i3);
            const float* ra = (const float*)row_ptr(alpha, i1 % alpha->ne[1], i2 % alpha->ne[2], i3 % alpha->ne[3]);
            const float* ri = (const float*)row_ptr(alpha_inv, i1 % alpha_inv->ne[1], i2 % alpha_inv->ne[2], i3 % alpha_inv->ne[3]);
            float* rd = (float*)row_ptr(dst, i1, i2, i3);
            for (int64_t i = 0; i < n; i++) {
                const float xv = rx[i];
                const float xa = xv * ra[i % alpha->ne[0]];
                const float s  = sinf(xa);
                const float s2 = s * s;
                const float m  = s2 * ri[i % alpha_inv->ne[0]];
                rd[i] = xv + m;
            }
        }
    }
    return 0;
}

/* T3 input embedding: get_rows(table, ids) + get_rows(pos_table, pos_ids),
 * both cast to f32, then one f32 add (t3.cpp:446-455). */
int cbxo_get_rows_add(const cbxo_tensor* src, const cbxo_tensor* ids,
                      const cbxo_tensor* src2, const cbxo_tensor* ids2,
                      cbxo_tensor* dst, int nth) {
    if (dst->type != CBXO_TYPE_F32) return -1;
    cbxo_tensor a = make_tmp_f32(dst), b = make_tmp_f32(dst);
    int rc = cbxo_get_rows(src, ids, &a, nth);
    if (!rc) rc = cbxo_get_rows(src2, ids2, &b, nth);
    if (!rc) rc = cbxo_add(&a, &b, dst, nth);
    free_tmp(&a);
    free_tmp(&b);
    return rc;
}

/* ggml: ggml_compute_forward_scale_f32 (bias 0) -- copy, then y[i] *= s. */
int cbxo_scale(const cbxo_tensor* x, float sc, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel for num_threads(nth) schedule(static, 1)
    for (int64_t ir = 0; ir < nr; ir++) {
        int64_t i1, i2, i3;
        split_row(x, ir, &i1, &i2, &i3);
        const float* rx = (const float*)row_ptr(x, i1, i2, i3);
        float* rd = (float*)row_ptr(dst, i1, i2, i3);
        for (int64_t i = 0; i < n; i++) rd[i] = rx[i] * sc;
    }
    return 0;
}

/* ggml: ggml_compute_forward_diag_mask_f32 with value -INFINITY -- column i
 * of row j is masked when i > n_past + j (t3.cpp:514-517 relies on this
 * shift for incremental attention). */
int cbxo_diag_mask_inf(const cbxo_tensor* x, int n_past, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    if (n_past < 0) return -1;
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel for num_threads(nth) schedule(static, 1)
    for (int64_t ir = 0; ir < nr; ir++) {
        int64_t i1, i2, i3;
        split_row(x, ir, &i1, &i2, &i3);
        const float* rx = (const float*)row_ptr(x, i1, i2, i3);
        float* rd = (float*)row_ptr(dst, i1, i2, i3);
        for (int64_t i = 0; i < n; i++) rd[i] = i > (int64_t)n_past + i1 ? -INFINITY : rx[i];
    }
    return 0;
}

/* ggml: ggml_compute_forward_soft_max_f32 (scale 1, no mask, no ALiBi) with
 * the scalar ggml_vec_soft_max_f32: max over the row, e_i = expf(x_i - max)
 * summed in f64, then every e_i times (float)(1.0 / sum). */
int cbxo_soft_max(const cbxo_tensor* x, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    const int64_t nr = nrows(x), n = x->ne[0];
#pragma omp parallel for num_threads(nth) schedule(static, 1)
    for (int64_t ir = 0; ir < nr; ir++) {
        int64_t i1, i2, i3;
        split_row(x, ir, &i1, &i2, &i3);
        const float* rx = (const float*)row_ptr(x, i1, i2, i3);
        float* rd = (float*)row_ptr(dst, i1, i2, i3);
        float mx = -INFINITY;
        for (int64_t i = 0; i < n; i++) mx = mx > rx[i] ? mx : rx[i];   /* ggml's MAX(max, x) */
        double sum = 0.0;
        for (int64_t i = 0; i < n; i++) {
            const float e = expf(rx[i] - mx);
            sum += (double)e;
            rd[i] = e;
        }
        const float inv = (float)(1.0 / sum);
        for (int64_t i = 0; i < n; i++) rd[i] *= inv;
    }
    return 0;
}

int cbxo_scale_diag_mask_soft_max(const cbxo_tensor* x, float sc, int n_past, cbxo_tensor* dst, int nth) {
    if (!same_shape(x, dst) || x->type != CBXO_TYPE_F32 || dst->type != CBXO_TYPE_F32) return -1;
    cbxo_tensor t = make_tmp_f32(x);
    int rc = cbxo_scale(x, sc, &t, nth);
    if (!rc && n_past >= 0) rc = cbxo_diag_mask_inf(&t, n_past, &t, nth);
    if (!rc) rc = cbxo_soft_max(&t, dst, nth);
    free_tmp(&t);
    return rc;
}

/* ------------------------------------------------------------------------ */
/* conv1d_CT with a fused prologue (hift_vocoder.cpp:46-59,77-93,119-138)   */
/* ------------------------------------------------------------------------ */

/* ggml: conv_1d_f32 = im2col(w, x, s, 0, p, 0, d, 0, false, F16) then
 * mul_mat(im2col, w_2d) with F32 precision: element (ic*K + k, ol) of the
 * im2col matrix is f16(x[ic][ol*s + k*d - p]), 0 outside [0, T_in); mul_mat
 * converts w to F16 (its F16 operand's dot type) and sums the products.
 * Then ggml_add of the (1, C_out) bias, the transposes, and the ResBlock's
 * residual ggml_add(x, h).  Prologues: snake() (hift_vocoder.cpp:64-73) as
 * five f32 ops; leaky_relu as ggml_vec_leaky_relu_f32. */
int cbxo_conv1d(const cbxo_tensor* x, const cbxo_tensor* w, int stride, int pad, int dilation, int prologue,
                const cbxo_tensor* alpha, const cbxo_tensor* alpha_inv, float slope, const cbxo_tensor* bias,
                const cbxo_tensor* res, cbxo_tensor* y, int nth) {
    if (x->type != CBXO_TYPE_F32 || y->type != CBXO_TYPE_F32) return -1;
    if (w->type != CBXO_TYPE_F32 && w->type != CBXO_TYPE_F16) return -1;
    if (stride < 1 || pad < 0 || dilation < 1 || x->ne[3] != 1) return -1;
    const int64_t C_in = x->ne[0], T_in = x->ne[1], B = x->ne[2];
    const int64_t K = w->ne[0], C_out = w->ne[2];
    if (w->ne[1] != C_in || w->ne[3] != 1) return -1;
    const int64_t T_out = (T_in + 2 * pad - dilation * (K - 1) - 1) / stride + 1;
    if (T_out < 1 || y->ne[0] != C_out || y->ne[1] != T_out || y->ne[2] != B || y->ne[3] != 1) return -1;
    if (bias && (bias->type != CBXO_TYPE_F32 || bias->ne[0] != C_out)) return -1;
    if (res && (res->type != CBXO_TYPE_F32 || !same_shape(res, y))) return -1;
    if (prologue == 1 && (!alpha || !alpha_inv || alpha->ne[0] != C_in || alpha_inv->ne[0] != C_in)) return -1;
    if (prologue < 0 || prologue > 2) return -1;
    /* the f16 im2col source: pro(x) rounded to f16, per (b, t, ic) */
    float* h = (float*)malloc(sizeof(float) * (size_t)(C_in * T_in * B));
    float* wf = (float*)malloc(sizeof(float) * (size_t)(C_out * K * C_in));   /* [oc][k][ic] */
    if (!h || !wf) { free(h); free(wf); return -1; }
    for (int64_t b = 0; b < B; b++) {
        for (int64_t t = 0; t < T_in; t++) {
            const float* rx = (const float*)row_ptr(x, t, b, 0);
            for (int64_t ic = 0; ic < C_in; ic++) {
                float v = rx[ic];
                if (prologue == 1) {
                    const float a = ((const float*)alpha->data)[ic];
                    const float ai = ((const float*)alpha_inv->data)[ic];
                    const float xa = v * a;
                    const float sn = sinf(xa);
                    const float s2 = sn * sn;
                    const float m = s2 * ai;
                    v = v + m;
                } else if (prologue == 2) {
                    v = op_leaky(v, slope);
                }
                h[(b * T_in + t) * C_in + ic] = cbxo_fp16_to_fp32(cbxo_fp32_to_fp16(v));
            }
        }
    }
    for (int64_t oc = 0; oc < C_out; oc++) {
        for (int64_t ic = 0; ic < C_in; ic++) {
            const char* rw = row_ptr(w, ic, oc, 0);
            for (int64_t k = 0; k < K; k++) {
                const float v = load_elem(w, rw, k);
                wf[(oc * K + k) * C_in + ic] = cbxo_fp16_to_fp32(cbxo_fp32_to_fp16(v));
            }
        }
    }
#pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t bt = 0; bt < B * T_out; bt++) {
        const int64_t b = bt / T_out, t = bt % T_out;
        float* ry = (float*)row_ptr(y, t, b, 0);
        const float* rr = res ? (const float*)row_ptr(res, t, b, 0) : NULL;
        for (int64_t oc = 0; oc < C_out; oc++) {
            double acc = 0.0;
            for (int64_t k = 0; k < K; k++) {
                const int64_t ti = t * stride + k * dilation - pad;
                if (ti < 0 || ti >= T_in) continue;
                const float* hr = h + (b * T_in + ti) * C_in;
                const float* wr = wf + (oc * K + k) * C_in;
                for (int64_t ic = 0; ic < C_in; ic++) acc += (double)hr[ic] * (double)wr[ic];
            }
            float v = (float)acc;
            if (bias) v = v + ((const float*)bias->data)[oc];
            if (rr) v = rr[oc] + v;
            ry[oc] = v;
        }
    }
    free(h);
    free(wf);
    return 0;
}

/* conv_transpose1d_CT (hift_vocoder.cpp:96-115): ggml_conv_transpose_1d with
 * p0 = 0, d0 = 1 converts the input and the kernel to f16 and adds, for each
 * input time i and tap k, the f16 dot product over C_in into full[i*s + k]
 * (f32); the reference then views [pad, pad + T_out) and adds the bias.
 * Here the same f16 operands and every product of an output summed in f64,
 * then the bias.  x (C_in, T_in, B); w (K, C_out, C_in) F32/F16; y (C_out,
 * T_out, B), T_out = (T_in - 1) s + K - 2 pad.  The prologue (leaky_relu at
 * hift_vocoder.cpp:686) is applied in f32 before the f16 rounding.        */
int cbxo_conv_transpose1d(const cbxo_tensor* x, const cbxo_tensor* w, int stride, int pad, int prologue,
                          const cbxo_tensor* alpha, const cbxo_tensor* alpha_inv, float slope,
                          const cbxo_tensor* bias, cbxo_tensor* y, int nth) {
    if (x->type != CBXO_TYPE_F32 || y->type != CBXO_TYPE_F32) return -1;
    if (w->type != CBXO_TYPE_F32 && w->type != CBXO_TYPE_F16) return -1;
    if (stride < 1 || pad < 0 || x->ne[3] != 1) return -1;
    const int64_t C_in = x->ne[0], T_in = x->ne[1], B = x->ne[2];
    const int64_t K = w->ne[0], C_out = w->ne[1];
    if (w->ne[2] != C_in || w->ne[3] != 1 || T_in < 1) return -1;
    const int64_t T_out = (T_in - 1) * stride + K - 2 * (int64_t)pad;
    if (T_out < 1 || y->ne[0] != C_out || y->ne[1] != T_out || y->ne[2] != B || y->ne[3] != 1) return -1;
    if (bias && (bias->type != CBXO_TYPE_F32 || bias->ne[0] != C_out)) return -1;
    if (prologue == 1 && (!alpha || !alpha_inv || alpha->ne[0] != C_in || alpha_inv->ne[0] != C_in)) return -1;
    if (prologue < 0 || prologue > 2) return -1;
    float* h = (float*)malloc(sizeof(float) * (size_t)(C_in * T_in * B));
    float* wf = (float*)malloc(sizeof(float) * (size_t)(C_out * K * C_in));   /* [oc][k][ic] */
    if (!h || !wf) { free(h); free(wf); return -1; }
    for (int64_t b = 0; b < B; b++) {
        for (int64_t t = 0; t < T_in; t++) {
            const float* rx = (const float*)row_ptr(x, t, b, 0);
            for (int64_t ic = 0; ic < C_in; ic++) {
                float v = rx[ic];
                if (prologue == 1) {
                    const float a = ((const float*)alpha->data)[ic];
                    const float ai = ((const float*)alpha_inv->data)[ic];
                    const float xa = v * a;
                    const float sn = sinf(xa);
                    const float s2 = sn * sn;
                    const float m = s2 * ai;
                    v = v + m;
                } else if (prologue == 2) {
                    v = op_leaky(v, slope);
                }
                h[(b * T_in + t) * C_in + ic] = cbxo_fp16_to_fp32(cbxo_fp32_to_fp16(v));
            }
        }
    }
    /* w element (k, oc, ic) sits in row (oc, ic) of the ggml layout */
    for (int64_t ic = 0; ic < C_in; ic++) {
        for (int64_t oc = 0; oc < C_out; oc++) {
            const char* rw = row_ptr(w, oc, ic, 0);
            for (int64_t k = 0; k < K; k++) {
                const float v = load_elem(w, rw, k);
                wf[(oc * K + k) * C_in + ic] = cbxo_fp16_to_fp32(cbxo_fp32_to_fp16(v));
            }
        }
    }
#pragma omp parallel for num_threads(nth) schedule(static)
    for (int64_t bt = 0; bt < B * T_out; bt++) {
        const int64_t b = bt / T_out, t = bt % T_out;
        const int64_t tf = t + pad;   /* time in the uncropped output */
        float* ry = (float*)row_ptr(y, t, b, 0);
        for (int64_t oc = 0; oc < C_out; oc++) {
            double acc = 0.0;
            for (int64_t k = tf % stride; k < K; k += stride) {
                const int64_t i = (tf - k) / stride;
                if (tf < k || i >= T_in) continue;
                const float* hr = h + (b * T_in + i) * C_in;
                const float* wr = wf + (oc * K + k) * C_in;
                for (int64_t ic = 0; ic < C_in; ic++) acc += (double)hr[ic] * (double)wr[ic];
            }
            float v = (float)acc;
            if (bias) v = v + ((const float*)bias->data)[oc];
            ry[oc] = v;
        }
    }
    free(h);
    free(wf);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* the T3 decode step's element-wise nodes (t3.cpp:446-546, N_new = 1)       */
/* ------------------------------------------------------------------------ */

static cbxo_tensor f32_2d(const float* p, int64_t ne0, int64_t ne1) {
    cbxo_tensor t;
    memset(&t, 0, sizeof(t));
    t.data = (void*)p;
    t.type = CBXO_TYPE_F32;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = 1;
    t.ne[3] = 1;
    t.nb[0] = 4;
    t.nb[1] = 4 * (size_t)ne0;
    t.nb[2] = t.nb[1] * (size_t)ne1;
    t.nb[3] = t.nb[2];
    return t;
}

int cbxo_t3_token_step(const cbxo_tensor* tok_table, int32_t token, const cbxo_tensor* pos_table,
                       int32_t position, int64_t d_ff, int64_t n_head, int32_t n_past, float eps,
                       const cbxo_t3_block* blocks, int32_t n_blocks, const float* out_w, const float* out_b,
                       float* h0, float* y) {
    const int64_t D = tok_table->ne[0];
    if (pos_table->ne[0] != D || n_head <= 0 || D % n_head || n_past < 0 || n_blocks < 0) return -1;
    const int64_t n_kv = (int64_t)n_past + 1;
    /* the reference's score scale, 1/sqrt(head size) in f32 (t3.cpp:513) */
    const float kq_scale = 1.0f / sqrtf((float)(D / n_head));
    float* tmp = (float*)malloc(sizeof(float) * (size_t)(2 * D + d_ff));
    if (!tmp) return -1;
    float* t0 = tmp;          /* (D) a row before its next add / norm */
    float* t1 = tmp + D;      /* (D) */
    int rc = 0;
    /* the input embedding: get_rows -> cast(F32), twice, then add */
    const int32_t ids[2] = {token, position};
    cbxo_tensor tid = f32_2d(NULL, 1, 1), pid = f32_2d(NULL, 1, 1);
    tid.data = (void*)&ids[0];
    tid.type = CBXO_TYPE_I32;
    pid.data = (void*)&ids[1];
    pid.type = CBXO_TYPE_I32;
    cbxo_tensor r0 = f32_2d(t0, D, 1), r1 = f32_2d(t1, D, 1), th = f32_2d(h0, D, 1);
    rc = cbxo_get_rows(tok_table, &tid, &r0, 1);
    if (!rc) rc = cbxo_get_rows(pos_table, &pid, &r1, 1);
    if (!rc) rc = cbxo_add(&r0, &r1, &th, 1);
    const float* h = h0;
    for (int32_t il = 0; il < n_blocks && !rc; il++) {
        const cbxo_t3_block* B = &blocks[il];
        cbxo_tensor hin = f32_2d(h, D, 1);
        cbxo_tensor w1 = f32_2d(B->ln1_w, D, 1), b1 = f32_2d(B->ln1_b, D, 1), l1 = f32_2d(B->ln1, D, 1);
        rc = cbxo_layer_norm(&hin, &w1, &b1, eps, &l1, 1);
        cbxo_tensor qm = f32_2d(B->qkv_mm, 3 * D, 1), qb = f32_2d(B->qkv_b, 3 * D, 1), qo = f32_2d(B->qkv, 3 * D, 1);
        if (!rc) rc = cbxo_add(&qm, &qb, &qo, 1);
        cbxo_tensor kq = f32_2d(B->kq, n_kv, n_head), pr = f32_2d(B->probs, n_kv, n_head);
        if (!rc) rc = cbxo_scale_diag_mask_soft_max(&kq, kq_scale, n_past, &pr, 1);
        /* attn_residual = add(add(out_mm, out_b), h) */
        cbxo_tensor om = f32_2d(B->out_mm, D, 1), ob = f32_2d(B->out_b, D, 1), ar = f32_2d(B->attn_res, D, 1);
        if (!rc) rc = cbxo_add(&om, &ob, &r0, 1);
        if (!rc) rc = cbxo_add(&r0, &hin, &ar, 1);
        cbxo_tensor w2 = f32_2d(B->ln2_w, D, 1), b2 = f32_2d(B->ln2_b, D, 1), l2 = f32_2d(B->ln2, D, 1);
        if (!rc) rc = cbxo_layer_norm(&ar, &w2, &b2, eps, &l2, 1);
        /* gelu(add(fc_mm, fc_b)) */
        cbxo_tensor fm = f32_2d(B->fc_mm, d_ff, 1), fb = f32_2d(B->fc_b, d_ff, 1), fs = f32_2d(tmp + 2 * D, d_ff, 1);
        cbxo_tensor go = f32_2d(B->gelu, d_ff, 1);
        if (!rc) rc = cbxo_add(&fm, &fb, &fs, 1);
        if (!rc) rc = cbxo_unary(CBXO_UNARY_GELU, &fs, &go, 1);
        /* h = add(add(proj_mm, proj_b), attn_residual) */
        cbxo_tensor pm = f32_2d(B->proj_mm, D, 1), pb = f32_2d(B->proj_b, D, 1), ho = f32_2d(B->h, D, 1);
        if (!rc) rc = cbxo_add(&pm, &pb, &r0, 1);
        if (!rc) rc = cbxo_add(&r0, &ar, &ho, 1);
        h = B->h;
    }
    if (!rc) {
        cbxo_tensor hin = f32_2d(h, D, 1), w = f32_2d(out_w, D, 1), b = f32_2d(out_b, D, 1), yo = f32_2d(y, D, 1);
        rc = cbxo_layer_norm(&hin, &w, &b, eps, &yo, 1);
    }
    free(tmp);
    return rc;
}
