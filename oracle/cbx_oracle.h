/*
 * cbx_oracle.h -- CPU restatement of the ggml-cpu arithmetic used by
 * chatterbox-cpp's fused layer-op path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * op library and the timed CPU baseline of bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product (libcbxops) never links, loads or calls it.
 *
 * What it restates and why: every op on the path is a ggml_* call made by the
 * reference's graph builders (chatterbox-cpp/src/t3.cpp, cfm_decoder.cpp,
 * hift_vocoder.cpp, flow_encoder.cpp, s3enc.cpp).  The arithmetic itself lives
 * in the ggml submodule (chatterbox-cpp/third_party/ggml, .gitmodules:1-3,
 * pinned v0.12.0 per chatterbox-cpp/README.md:36), which is not vendored in
 * the reference checkout.  Each function below restates the published
 * ggml-cpu behaviour of one op (scalar code path, ISO C evaluation: no FMA
 * contraction), in this library's own code, and names the reference call site
 * whose semantics it fixes.
 *
 * Parity pins (tests/test_oracle_*.py): closed forms evaluated in float64,
 * numpy's independent float16 conversion, exhaustive enumeration of all 65536
 * f16 codes, invariants (LN of a constant row, rotation norm preservation,
 * group-norm moments), brute force on tiny inputs, and committed golden
 * vectors under tests/golden/.  Functions with no such pin are marked
 * "parity unpinned" in their comment; none is at present.
 *
 * Tensors use ggml's layout: ne[0] is the innermost (contiguous) dimension,
 * nb[] are byte strides.  Types use ggml_type numbering.
 */
#ifndef CBX_ORACLE_H
#define CBX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    CBXO_TYPE_F32  = 0,
    CBXO_TYPE_F16  = 1,
    CBXO_TYPE_Q8_0 = 8,
    CBXO_TYPE_I32  = 26,
};

/* ggml_unary_op / ggml_glu_op subset used by the path. */
enum {
    CBXO_UNARY_GELU      = 0,  /* ggml_gelu      (t3.cpp:537)            */
    CBXO_UNARY_GELU_ERF  = 1,  /* ggml_gelu_erf  (cfm_decoder.cpp:239)   */
    CBXO_UNARY_SILU      = 2,  /* ggml_silu      (cfm_decoder.cpp:466)   */
    CBXO_UNARY_TANH      = 3,  /* ggml_tanh      (cfm_decoder.cpp:37)    */
    CBXO_UNARY_SOFTPLUS  = 4,  /* ggml_softplus  (cfm_decoder.cpp:37)    */
    CBXO_UNARY_SIN       = 5,  /* ggml_sin       (hift_vocoder.cpp:69)   */
    CBXO_UNARY_SQR       = 6,  /* ggml_sqr       (hift_vocoder.cpp:70)   */
    CBXO_UNARY_MISH      = 7,  /* mish() helper  (cfm_decoder.cpp:36-38) */
};

typedef struct cbxo_tensor {
    void*    data;
    int32_t  type;
    int32_t  reserved;
    int64_t  ne[4];
    size_t   nb[4];
} cbxo_tensor;

#define CBXO_QK8_0 32
#define CBXO_Q8_0_BLOCK_BYTES 34   /* ggml block_q8_0: f16 d + int8 qs[32] */

/* ---- scalar conversions ------------------------------------------------ */
float    cbxo_fp16_to_fp32(uint16_t h);
uint16_t cbxo_fp32_to_fp16(float f);   /* round to nearest even */

/* ---- Q8_0 (ggml-quants reference rule) --------------------------------- */
void cbxo_quantize_row_q8_0(const float* x, void* y, int64_t k);
void cbxo_dequantize_row_q8_0(const void* x, float* y, int64_t k);

/* ---- GELU fp16 table (ggml_cpu_init) ----------------------------------- */
/* fma_variant = 0: ISO C evaluation of 0.5x(1+tanh(s x (1 + a x^2)));
 * fma_variant = 1: the same with (a*x)*x + 1 contracted to one fmaf, which
 * is what gcc/clang emit for ggml-cpu on FMA hardware at default flags.   */
void  cbxo_gelu_table(uint16_t* out65536, int fma_variant);
float cbxo_gelu_f32(float x, int fma_variant);

/* ---- ops (return 0, or a negative value on invalid input) -------------- */
int cbxo_get_rows(const cbxo_tensor* src, const cbxo_tensor* ids,
                  cbxo_tensor* dst, int n_threads);
int cbxo_add(const cbxo_tensor* a, const cbxo_tensor* b, cbxo_tensor* dst,
             int n_threads);
int cbxo_mul(const cbxo_tensor* a, const cbxo_tensor* b, cbxo_tensor* dst,
             int n_threads);
int cbxo_norm(const cbxo_tensor* x, float eps, cbxo_tensor* dst,
              int n_threads);
int cbxo_rms_norm(const cbxo_tensor* x, float eps, cbxo_tensor* dst,
                  int n_threads);
int cbxo_group_norm(const cbxo_tensor* x, int n_groups, float eps,
                    cbxo_tensor* dst, int n_threads);
int cbxo_unary(int op, const cbxo_tensor* x, cbxo_tensor* dst, int n_threads);
int cbxo_leaky_relu(const cbxo_tensor* x, float slope, cbxo_tensor* dst,
                    int n_threads);
int cbxo_swiglu(const cbxo_tensor* g, const cbxo_tensor* u, cbxo_tensor* dst,
                int n_threads);
int cbxo_cpy(const cbxo_tensor* src, cbxo_tensor* dst, int n_threads);

/* RoPE: the ggml_rope_ext argument list.  mode 0 = NORMAL, 2 = NEOX. */
void cbxo_rope_yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base,
                              float beta_fast, float beta_slow, float dims[2]);
void cbxo_rope_cache_init(float theta_base, float freq_scale,
                          const float* freq_factors, const float corr_dims[2],
                          int64_t ne0, float ext_factor, float mscale,
                          float* cache, float sin_sign, float theta_scale);
int cbxo_rope_ext(const cbxo_tensor* x, const cbxo_tensor* pos,
                  const float* freq_factors, int n_dims, int mode,
                  int n_ctx_orig, float freq_base, float freq_scale,
                  float ext_factor, float attn_factor, float beta_fast,
                  float beta_slow, cbxo_tensor* dst, int n_threads);

/* ggml_scale(x, s): y = x * s, one f32 multiply per element.             */
int cbxo_scale(const cbxo_tensor* x, float s, cbxo_tensor* dst, int n_threads);
/* ggml_diag_mask_inf(x, n_past): element i of row j (j = ne1 index) is set
 * to -INFINITY when i > n_past + j, in every ne2 x ne3 slice.            */
int cbxo_diag_mask_inf(const cbxo_tensor* x, int n_past, cbxo_tensor* dst, int n_threads);
/* ggml_soft_max(x) over ne0: m = max, e = expf(x - m), sum in f64,
 * y = e * (float)(1.0 / sum).                                            */
int cbxo_soft_max(const cbxo_tensor* x, cbxo_tensor* dst, int n_threads);

/* ---- compositions made by the reference's graph builders --------------- */
/* layer_norm(): norm -> mul(w) -> add(b)  (cfm_decoder.cpp:29-33,
 * t3.cpp:465-466); w and b may be NULL (plain ggml_norm then).           */
int cbxo_layer_norm(const cbxo_tensor* x, const cbxo_tensor* w,
                    const cbxo_tensor* b, float eps, cbxo_tensor* dst,
                    int n_threads);
/* rms_norm -> mul(g); f16 x/dst are computed in f32 and rounded once.    */
int cbxo_rms_norm_mul(const cbxo_tensor* x, const cbxo_tensor* g, float eps,
                      cbxo_tensor* dst, int n_threads);
/* group_norm -> mul(w) -> add(b) -> optional mish.                       */
int cbxo_group_norm_affine(const cbxo_tensor* x, int n_groups, float eps,
                           const cbxo_tensor* w, const cbxo_tensor* b,
                           int fuse_mish, cbxo_tensor* dst, int n_threads);
/* snake(): x + sin^2(x*alpha) * alpha_inv (hift_vocoder.cpp:64-73).      */
int cbxo_snake(const cbxo_tensor* x, const cbxo_tensor* alpha,
               const cbxo_tensor* alpha_inv, cbxo_tensor* dst, int n_threads);
/* attention scores: soft_max(diag_mask_inf(scale(x, s), n_past))
 * (t3.cpp:513-518); n_past < 0 leaves out the mask, as the encoders do
 * (cfm_decoder.cpp:218-220, flow_encoder.cpp:371-372, s3enc.cpp:260-262). */
int cbxo_scale_diag_mask_soft_max(const cbxo_tensor* x, float s, int n_past,
                                  cbxo_tensor* dst, int n_threads);
/* get_rows(tok) + get_rows(pos) (t3.cpp:440-455).                        */
int cbxo_get_rows_add(const cbxo_tensor* src, const cbxo_tensor* ids,
                      const cbxo_tensor* src2, const cbxo_tensor* ids2,
                      cbxo_tensor* dst, int n_threads);
/* conv1d_CT(pro(x)) [+ bias] [+ res] on the reference's (C, T) layout
 * (hift_vocoder.cpp:46-59,77-93,119-138): im2col to F16, the weights
 * converted to F16 by mul_mat, products summed, the f32 result plus the
 * bias, then plus res.  x (C_in, T_in, B) F32; w (K, C_in, C_out) F32/F16;
 * bias (C_out) or NULL; res (C_out, T_out, B) or NULL; y (C_out, T_out, B).
 * prologue 0: none, 1: snake (alpha, alpha_inv (C_in)), 2: leaky_relu.
 * The sum is accumulated in f64 (the reference's f32 SIMD accumulation
 * order depends on the host ISA).                                         */
int cbxo_conv1d(const cbxo_tensor* x, const cbxo_tensor* w, int stride,
                int pad, int dilation, int prologue,
                const cbxo_tensor* alpha, const cbxo_tensor* alpha_inv,
                float slope, const cbxo_tensor* bias, const cbxo_tensor* res,
                cbxo_tensor* y, int n_threads);
/* conv_transpose1d_CT(pro(x)) [+ bias] (hift_vocoder.cpp:96-115):
 * ggml_conv_transpose_1d (f16 input and kernel, p0 = 0, d0 = 1), the view
 * that strips pad from both ends of the time axis, then the bias.  x (C_in,
 * T_in, B) F32; w (K, C_out, C_in) F32/F16; y (C_out, T_out, B), T_out =
 * (T_in - 1) stride + K - 2 pad.  f64 accumulation as cbxo_conv1d.        */
int cbxo_conv_transpose1d(const cbxo_tensor* x, const cbxo_tensor* w,
                          int stride, int pad, int prologue,
                          const cbxo_tensor* alpha,
                          const cbxo_tensor* alpha_inv, float slope,
                          const cbxo_tensor* bias, cbxo_tensor* y,
                          int n_threads);

/* ---- the T3 decode step's element-wise nodes --------------------------- */
/* One T3 block at N_new = 1 (t3.cpp:460-542) with its matmul outputs given:
 * the parameters it adds or scales by, those outputs, and where each of its
 * element-wise results goes.  F32, contiguous.  D = model width, F = FFN
 * width, H = heads, n_kv = n_past + 1 attention columns a head.            */
typedef struct cbxo_t3_block {
    const float *ln1_w, *ln1_b;  /* (D) LN-1 (t3.cpp:465-466)               */
    const float *qkv_b;          /* (3D) (t3.cpp:470)                       */
    const float *out_b;          /* (D) (t3.cpp:526)                        */
    const float *ln2_w, *ln2_b;  /* (D) LN-2 (t3.cpp:531-532)               */
    const float *fc_b;           /* (F) (t3.cpp:536)                        */
    const float *proj_b;         /* (D) (t3.cpp:540)                        */
    const float *qkv_mm;         /* (3D) mul_mat(qkv_w, ln1)                */
    const float *kq;             /* (H, n_kv) mul_mat(K, Q)                 */
    const float *out_mm;         /* (D) mul_mat(out_w, attention)           */
    const float *fc_mm;          /* (F) mul_mat(fc_w, ln2)                  */
    const float *proj_mm;        /* (D) mul_mat(proj_w, gelu)               */
    float *ln1;                  /* (D) LN-1 of the block's input h         */
    float *qkv;                  /* (3D) qkv_mm + qkv_b                     */
    float *probs;                /* (H, n_kv) soft_max(mask(scale(kq)))     */
    float *attn_res;             /* (D) (out_mm + out_b) + h                */
    float *ln2;                  /* (D) LN-2 of attn_res                    */
    float *gelu;                 /* (F) gelu(fc_mm + fc_b)                  */
    float *h;                    /* (D) (proj_mm + proj_b) + attn_res       */
} cbxo_t3_block;

/* The element-wise nodes of one T3 decode step at N_new = 1 in the order
 * the reference builds them (t3.cpp:446-455 the input embedding of
 * `token` at `position`: get_rows -> cast, twice, then add; then per
 * block LN-1, the qkv bias, scale(1/sqrt(D/H)) -> diag_mask_inf(n_past)
 * -> soft_max, the output bias and residual, LN-2, the fc bias and GELU,
 * the projection bias and residual; t3.cpp:545-546 the final LN into y).
 * tok_table, pos_table: F32 or F16 (D wide).  h0 (D) gets the embedding
 * sum.  One thread: at N_new = 1 every op is one row.  Returns 0, or a
 * negative value on invalid input.                                        */
int cbxo_t3_token_step(const cbxo_tensor* tok_table, int32_t token,
                       const cbxo_tensor* pos_table, int32_t position,
                       int64_t d_ff, int64_t n_head, int32_t n_past,
                       float eps, const cbxo_t3_block* blocks,
                       int32_t n_blocks, const float* out_w,
                       const float* out_b, float* h0, float* y);

#ifdef __cplusplus
}
#endif
#endif
