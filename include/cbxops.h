/*
 * cbxops.h -- C ABI of the MI355X (gfx950) fused layer-op library.
 *
 * Each entry point replaces one ggml op, or one composition of ggml ops,
 * that chatterbox-cpp's graph builders call on the fused layer-op path, with
 * the same tensor layout (ggml ne[]/nb[]: ne[0] innermost, byte strides) and
 * the same arithmetic as ggml's CPU backend.  Every entry point:
 *   - takes device pointers owned by the caller and a HIP stream;
 *   - allocates nothing and launches asynchronously on that stream;
 *   - returns CBX_OK (0) or a negative cbx_status, with a message available
 *     from cbx_last_error() on the calling thread (the convention of the
 *     reference's own C ABI, chatterbox-cpp/src/chatterbox_capi.cpp:14-18).
 * Unlike ggml (GGML_ASSERT), no call aborts the process.
 *
 * Threading: calls are stream-ordered; calls on different streams may run
 * concurrently.  cbx_init / cbx_shutdown / cbx_rope_cache_* are not
 * thread-safe against each other.
 */
#ifndef CBXOPS_H
#define CBXOPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same handle type as HIP's hipStream_t (NULL = the null stream). */
struct ihipStream_t;
typedef struct ihipStream_t* cbx_stream;

/* Element types, numbered as ggml_type. */
typedef enum cbx_type {
    CBX_TYPE_F32  = 0,
    CBX_TYPE_F16  = 1,
    CBX_TYPE_Q8_0 = 8,   /* blocks of 32: f16 scale d + int8 qs[32], 34 bytes */
    CBX_TYPE_I32  = 26,
} cbx_type;

typedef enum cbx_status {
    CBX_OK                  = 0,
    CBX_ERR_INVALID_ARG     = -1,  /* bad pointer, shape, stride or type   */
    CBX_ERR_UNSUPPORTED     = -2,  /* valid ggml op, layout not supported  */
    CBX_ERR_NOT_INITIALIZED = -3,  /* cbx_init() not called for the device */
    CBX_ERR_HIP             = -4,  /* a HIP runtime call failed            */
} cbx_status;

/* A ggml-layout tensor view.  For Q8_0, ne[0] counts elements (a multiple
 * of 32) and nb[0] is the block size, 34, as in ggml. */
typedef struct cbx_tensor {
    void*    data;
    int32_t  type;      /* cbx_type */
    int32_t  reserved;  /* must be 0 */
    int64_t  ne[4];
    size_t   nb[4];
} cbx_tensor;

/* Activations for cbx_unary and the fused epilogues. */
typedef enum cbx_unary_op {
    CBX_UNARY_NONE     = -1, /* epilogue only: no activation                           */
    CBX_UNARY_GELU     = 0,  /* ggml_gelu, fp16-table semantics (t3.cpp:537)           */
    CBX_UNARY_GELU_ERF = 1,  /* ggml_gelu_erf (cfm_decoder.cpp:239, s3enc.cpp:177)      */
    CBX_UNARY_SILU     = 2,  /* ggml_silu (cfm_decoder.cpp:466, flow_encoder.cpp:402)   */
    CBX_UNARY_TANH     = 3,  /* ggml_tanh (cfm_decoder.cpp:37)                          */
    CBX_UNARY_SOFTPLUS = 4,  /* ggml_softplus (cfm_decoder.cpp:37)                      */
    CBX_UNARY_SIN      = 5,  /* ggml_sin (hift_vocoder.cpp:69)                          */
    CBX_UNARY_SQR      = 6,  /* ggml_sqr (hift_vocoder.cpp:70)                          */
    CBX_UNARY_MISH     = 7,  /* mish() = mul(x, tanh(softplus(x))) (cfm_decoder.cpp:36-38) */
} cbx_unary_op;

/* ---- library lifecycle -------------------------------------------------- */

/* Prepares `device` for use: uploads the 65536-entry fp16 GELU table (the
 * table ggml_cpu_init builds for ggml_gelu), and a sticky device error word.
 * The analogue of ggml_cpu_init(); call once per device before any op.     */
int  cbx_init(int device);
/* Releases every device's state.  No op may be in flight. */
void cbx_shutdown(void);
/* Message of the last failed call on this thread ("" if none). */
const char* cbx_last_error(void);
const char* cbx_version(void);
/* Reads (and with clear != 0 resets) the device error word of `device`,
 * synchronising the device first.  Bit 0: a get_rows index was out of
 * range (ggml aborts there; this library writes zeros to that row).
 * Bit 1: reserved, never raised (in-place GroupNorm calls do not take the
 * split reduction, the only path that raised it).                          */
int  cbx_device_errors(int device, uint32_t* flags_out, int clear);

/* ---- gather and conversion ---------------------------------------------- */

/* ggml_get_rows(src, ids) then ggml_cast(F32): dst[:, i10, i11, i12] =
 * to_f32(src[:, ids[i10, i11, i12], i11, i12]).  src F32, F16 or Q8_0; ids
 * I32; dst F32 with ne = (src.ne0, ids.ne0, ids.ne1, ids.ne2).
 * Replaces t3.cpp:440-447 and flow_encoder.cpp:588-590.                    */
int cbx_get_rows(const cbx_tensor* src, const cbx_tensor* ids,
                 cbx_tensor* dst, cbx_stream stream);

/* ggml_add(get_rows(src, ids), get_rows(src2, ids2)) in one pass: the T3
 * token + learned-position embedding (t3.cpp:446-455).                     */
int cbx_get_rows_add(const cbx_tensor* src, const cbx_tensor* ids,
                     const cbx_tensor* src2, const cbx_tensor* ids2,
                     cbx_tensor* dst, cbx_stream stream);

/* The T3 input embedding and the first LayerNorm it feeds, in one pass:
 * h = ggml_add(get_rows(src, ids), get_rows(src2, ids2)) (t3.cpp:446-455),
 * y = layer_norm(h, w, b, eps) (t3.cpp:465-466).  h (F32, y's shape) is
 * stored when non-NULL -- it is the residual stream.  Needs ne0 % 4 == 0,
 * ne0 <= 4096 and 16-byte aligned rows.                                    */
int cbx_get_rows_add_layer_norm(const cbx_tensor* src, const cbx_tensor* ids,
                                const cbx_tensor* src2, const cbx_tensor* ids2,
                                const cbx_tensor* w, const cbx_tensor* b,
                                float eps, cbx_tensor* h, cbx_tensor* y,
                                cbx_stream stream);

/* The T3 input when the sequence starts with the conditioning prefix
 * (t3.cpp:432-466), in one pass:
 *   seq = ggml_concat(ggml_concat(prefix, cast(get_rows(src_a, ids_a)), 1),
 *                     cast(get_rows(src_b, ids_b)), 1)
 *   h   = ggml_add(seq, cast(get_rows(src2, ids2)))
 *   y   = layer_norm(h, w, b, eps)
 * prefix: F32 (D, n_prefix, 1, 1) rows already computed (the conditioning
 * encoder's output, t3.cpp:434-436), or NULL; src_a/ids_a (the prompt's
 * speech tokens, t3.cpp:439-442) may be NULL; src_b/ids_b (the text tokens,
 * t3.cpp:445-448) and src2/ids2 (positions, :452-454) are required.
 * Tables: 2-D F32/F16/Q8_0 with ne0 = D; ids: contiguous 1-D I32; y (and h,
 * stored when non-NULL): F32 (D, N, 1, 1) with N = n_prefix + len(ids_a) +
 * len(ids_b) = len(ids2).  D % 4 == 0, D <= 1024, 16-byte aligned rows.
 * Out-of-range ids: as cbx_get_rows_add_layer_norm.                        */
int cbx_get_rows_concat_add_layer_norm(const cbx_tensor* prefix,
                                       const cbx_tensor* src_a, const cbx_tensor* ids_a,
                                       const cbx_tensor* src_b, const cbx_tensor* ids_b,
                                       const cbx_tensor* src2, const cbx_tensor* ids2,
                                       const cbx_tensor* w, const cbx_tensor* b,
                                       float eps, cbx_tensor* h, cbx_tensor* y,
                                       cbx_stream stream);

/* ggml_cpy / ggml_cast between F32 and F16 (round to nearest even), same
 * shape (t3.cpp:441,447,454).                                              */
int cbx_cpy(const cbx_tensor* src, cbx_tensor* dst, cbx_stream stream);

/* ---- norms -------------------------------------------------------------- */

/* ggml_norm(x, eps) over ne[0] (F32 or F16 storage, f32/f64 arithmetic). */
int cbx_norm(const cbx_tensor* x, float eps, cbx_tensor* y, cbx_stream stream);

/* layer_norm() = ggml_add(ggml_mul(ggml_norm(x, eps), w), b) in one pass
 * (cfm_decoder.cpp:29-33; t3.cpp:465-466,531-532,545-546;
 * flow_encoder.cpp:58-62; s3enc.cpp:100-104).  w, b: F32 with ne =
 * (x.ne0,1,1,1), or NULL.  act: CBX_UNARY_NONE, or an activation applied
 * to the result (CBX_UNARY_MISH fuses causal_block1d's LN -> Mish,
 * cfm_decoder.cpp:143-146).                                                */
int cbx_layer_norm(const cbx_tensor* x, const cbx_tensor* w,
                   const cbx_tensor* b, float eps, int act, cbx_tensor* y,
                   cbx_stream stream);

/* ggml_rms_norm(x, eps). */
int cbx_rms_norm(const cbx_tensor* x, float eps, cbx_tensor* y,
                 cbx_stream stream);

/* ggml_mul(ggml_rms_norm(x, eps), g) in one pass; g F32 (x.ne0,1,1,1) or
 * NULL.  F16 x/y: f32 arithmetic, one rounding at the store.              */
int cbx_rms_norm_mul(const cbx_tensor* x, const cbx_tensor* g, float eps,
                     cbx_tensor* y, cbx_stream stream);

/* ggml_group_norm(x, n_groups, eps) [-> mul(w) -> add(b)] [-> act] in one
 * pass.  Channels are ne[2] (ggml's convention), F32.  w, b: F32 with ne =
 * (1,1,ne2,1), or NULL.  act: CBX_UNARY_NONE or an activation.  y may be x.
 * A few large groups out of place (the CFM decoder's) run as the split
 * reduction of cbx_group_norm_ws over the library's own scratch (the set
 * the stream hashes to; see cbx_group_norm_noalloc), when cbx_init found
 * the device's dispatch compatible with it (cbx_group_norm_split_enabled);
 * everything else, in place included, one workgroup reduces each group.
 * The results are the same bits either way.                               */
int cbx_group_norm(const cbx_tensor* x, int n_groups, float eps,
                   const cbx_tensor* w, const cbx_tensor* b, int act,
                   cbx_tensor* y, cbx_stream stream);

/* cbx_group_norm with the statistics split over many workgroups.  A few
 * large groups (the CFM decoder's two CFG items x 8 groups) run as chunks:
 * each workgroup reads and reduces only its chunk, and the chunks' f64
 * partial sums meet in the workspace -- one HBM read of x, no workgroup
 * reducing a whole group.  Same results as cbx_group_norm, bit for bit.
 * In-place calls (y overlapping x) and layouts the split does not cover
 * (strided groups, many small groups) run as one workgroup per group.
 * A workspace serves one call at a time at full speed: calls that overlap
 * in time on one workspace still give exact results (every partial carries
 * its launch's 64-bit tag), but their chunks stop waiting for each other's
 * partials and each recomputes the group, so give concurrent streams a
 * workspace each.
 *
 * The workspace (128 KiB of device memory on the current device, zeroed once;
 * nothing in it needs clearing between calls) has no counterpart in ggml, whose CPU group
 * norm reduces each group on one thread; cbx_group_norm_workspace_create /
 * _destroy are the explicit init/destroy pair of the op.                  */
typedef struct cbx_group_norm_workspace cbx_group_norm_workspace;
int  cbx_group_norm_workspace_create(cbx_group_norm_workspace** out);
void cbx_group_norm_workspace_destroy(cbx_group_norm_workspace* ws);
/* A chunk workgroup waits at most max_wait_us for the group's other
 * chunks, then computes every chunk's partial itself from x (which the
 * split never overwrites: it runs out of place only); 0: never wait (each
 * wave reduces the whole group itself); CBX_GN_WAIT_AUTO (the default):
 * ten times the launch's expected length, at least 20 us.  n_chunks: chunks
 * per group, 0 (default) = automatic, else 2..32.  The results do not
 * depend on either.  For tests and tuning.                                */
#define CBX_GN_WAIT_AUTO 0xFFFFFFFFu
int  cbx_group_norm_workspace_tune(cbx_group_norm_workspace* ws,
                                   uint32_t max_wait_us, int32_t n_chunks);
/* 1 when cbx_init found that the device deals workgroups to its XCDs by
 * index mod 8 (checked with a probe kernel), so the split runs; 0 when it
 * did not (every GroupNorm then reduces a group in one workgroup); or a
 * negative cbx_status.                                                    */
int  cbx_group_norm_split_enabled(int device);
int  cbx_group_norm_ws(const cbx_tensor* x, int n_groups, float eps,
                       const cbx_tensor* w, const cbx_tensor* b, int act,
                       cbx_tensor* y, cbx_group_norm_workspace* ws,
                       cbx_stream stream);

/* cbx_group_norm_ws without a workspace: the same kernels and results, the
 * exchange words in the library's own static device memory (8 sets of
 * 128 KiB, 1 MiB per GPU, set up by cbx_init, held until the process ends;
 * a call uses the set its stream's handle hashes to).  No counterpart in
 * the reference: for callers that cannot allocate device memory at all --
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  The call allocates nothing.  n_groups x x.ne[3] is limited to
 * 1024 group instances (larger: CBX_ERR_UNSUPPORTED).  Calls that overlap
 * in time on one GPU race for a set when their streams hash to the same
 * one: their results stay exact (tagged partials, and a chunk that stops
 * waiting recomputes the group from x), but they lose the split's speed;
 * keep such calls on one stream, or ordered by events.                     */
int  cbx_group_norm_noalloc(const cbx_tensor* x, int n_groups, float eps,
                            const cbx_tensor* w, const cbx_tensor* b, int act,
                            cbx_tensor* y, cbx_stream stream);

/* The residual join and the LayerNorm that reads it, in one pass:
 *   s = ggml_add(ggml_add(a, a_bias), r)     (a_bias NULL: ggml_add(a, r);
 *                                             r NULL: ggml_add(a, a_bias))
 *   y = act(layer_norm(s, w, b, eps))
 * (t3.cpp:528-532: attn_residual = add(add(mul_mat, out_b), h), then the
 * pre-FFN LayerNorm; t3.cpp:539-541 with the next block's :465-466 or the
 * final LayerNorm :545-546; s3enc.cpp:273-276; flow_encoder.cpp:395-399;
 * with no residual, a linear's bias and the LayerNorm after it,
 * flow_encoder.cpp:414-415).  r may be NULL only when a_bias is not.
 * a, r, s, y: F32, one shape, ne0 % 4 == 0, ne0 <= 4096, 16-byte aligned
 * rows; a_bias, w, b: F32 (x.ne0,1,1,1), 16-byte aligned, or NULL.  s (the
 * residual stream) is stored when non-NULL; it may be a or r but must not
 * overlap y.  act: CBX_UNARY_NONE or an activation.                        */
int cbx_add_layer_norm(const cbx_tensor* a, const cbx_tensor* a_bias,
                       const cbx_tensor* r, const cbx_tensor* w,
                       const cbx_tensor* b, float eps, int act, cbx_tensor* s,
                       cbx_tensor* y, cbx_stream stream);

/* causal_block1d's tail in one pass (cfm_decoder.cpp:143-148): LayerNorm,
 * the activation (Mish there), then the frame mask:
 *   y = ggml_mul(act(layer_norm(x, w, b, eps)), mask)
 * mask: contiguous F32 with ne = (1, x.ne1, 1, 1), the reference's (1, T).
 * Layouts as cbx_add_layer_norm; y may be x.                               */
int cbx_layer_norm_mask(const cbx_tensor* x, const cbx_tensor* w,
                        const cbx_tensor* b, float eps, int act,
                        const cbx_tensor* mask, cbx_tensor* y,
                        cbx_stream stream);

/* ---- rotary embedding --------------------------------------------------- */

/* A device-resident cos/sin table for ggml_rope_ext's parameters, for
 * positions [0, n_pos).  Built on the host with ggml's semantics (theta
 * iterated as an f32 product, YaRN ramp, attn_factor) and uploaded once;
 * the per-position rows are staged in LDS by cbx_rope_ext.  Allocates
 * device memory on the current device.  freq_factors: host array of
 * n_dims/2 floats, or NULL.                                                */
typedef struct cbx_rope_cache cbx_rope_cache;
int  cbx_rope_cache_create(int n_dims, int mode, int n_ctx_orig,
                           float freq_base, float freq_scale,
                           float ext_factor, float attn_factor,
                           float beta_fast, float beta_slow,
                           const float* freq_factors, int32_t n_pos,
                           cbx_rope_cache** out);
void cbx_rope_cache_destroy(cbx_rope_cache* cache);

/* ggml_rope_ext(x, pos, NULL, n_dims, mode, ...) with the cache's
 * parameters (s3enc.cpp:215-229).  x, y: F32 or F16, ne = (head_dim,
 * n_head, n_tok, batch); pos: I32 [n_tok].  Positions outside [0, n_pos)
 * are computed on the device (same theta recurrence, device cosf/sinf).   */
int cbx_rope_ext(const cbx_tensor* x, const cbx_tensor* pos,
                 const cbx_rope_cache* cache, cbx_tensor* y,
                 cbx_stream stream);

/* LayerNorm + affine of each token row, then RoPE of the row viewed as
 * heads, in one pass:
 *   ggml_rope_ext(ggml_reshape_4d(layer_norm(x, w, b, eps), head_dim,
 *                 x.ne0/head_dim, x.ne1, x.ne2), pos, NULL, ...cache...)
 * (layer_norm as cfm_decoder.cpp:29-33, rope as s3enc.cpp:215-229).
 * x, y: F32, ne = (C, n_tok, batch, 1) with C <= 1024, C % head_dim == 0,
 * head_dim % 4 == 0, n_dims <= head_dim; pos: I32 [n_tok]; w, b as for
 * cbx_layer_norm.  Same results as cbx_layer_norm then cbx_rope_ext.       */
int cbx_layer_norm_rope(const cbx_tensor* x, const cbx_tensor* w,
                        const cbx_tensor* b, float eps, int64_t head_dim,
                        const cbx_tensor* pos, const cbx_rope_cache* cache,
                        cbx_tensor* y, cbx_stream stream);

/* ---- attention-score epilogue ------------------------------------------ */

/* ggml_soft_max(ggml_diag_mask_inf(ggml_scale(x, scale), n_past)) over ne0
 * in one pass (t3.cpp:513-518: scale 1/sqrt(Hd), causal mask shifted by the
 * cached positions).  n_past < 0 leaves out the mask:
 * ggml_soft_max(ggml_scale(x, scale)) (cfm_decoder.cpp:218-220,
 * flow_encoder.cpp:371-372, s3enc.cpp:260-262).  x, y: F32 with the same
 * shape, ne = (n_keys, n_queries, n_head, batch); the mask hides key i from
 * query j (ne1 index) when i > n_past + j.  y may be x.                     */
int cbx_scale_diag_mask_soft_max(const cbx_tensor* x, float scale,
                                 int32_t n_past, cbx_tensor* y,
                                 cbx_stream stream);

/* The same with the two score terms' sum in front:
 * ggml_soft_max(ggml_scale(ggml_add(a, b), scale)) (flow_encoder.cpp:
 * 369-372: the content scores AC and the shifted position scores BD of the
 * relative-position attention), a + b rounded to f32 before the scale, the
 * mask as above when n_past >= 0.  a, b, y: F32 with the same shape; y may
 * be a or b itself and must not overlap them otherwise.                     */
int cbx_add_scale_diag_mask_soft_max(const cbx_tensor* a, const cbx_tensor* b,
                                     float scale, int32_t n_past,
                                     cbx_tensor* y, cbx_stream stream);

/* ---- activations -------------------------------------------------------- */

/* One ggml unary op (cbx_unary_op), F32 or F16, x and y same shape. */
int cbx_unary(int op, const cbx_tensor* x, cbx_tensor* y, cbx_stream stream);
int cbx_gelu(const cbx_tensor* x, cbx_tensor* y, cbx_stream stream);
int cbx_gelu_erf(const cbx_tensor* x, cbx_tensor* y, cbx_stream stream);
int cbx_silu(const cbx_tensor* x, cbx_tensor* y, cbx_stream stream);
int cbx_mish(const cbx_tensor* x, cbx_tensor* y, cbx_stream stream);

/* ggml_leaky_relu(x, slope, false) (hift_vocoder.cpp:686,748;
 * flow_encoder.cpp:454). */
int cbx_leaky_relu(const cbx_tensor* x, float slope, cbx_tensor* y,
                   cbx_stream stream);

/* A bias add and the activation reading it: y = act(ggml_add(x, bias))
 * (t3.cpp:535-537 fc bias -> ggml_gelu; cfm_decoder.cpp:237-239 and
 * s3enc.cpp:176-177,279-280 -> ggml_gelu_erf; flow_encoder.cpp:401-402 and
 * cfm_decoder.cpp:464-466 -> ggml_silu).  x, y: F32 same shape; bias:
 * contiguous F32 with ne = (x.ne0,1,1,1), or (1,x.ne1,1,1) for the (1, C)
 * bias of a time-major tensor (s3enc.cpp:117-120).  act CBX_UNARY_NONE
 * leaves the bias add alone.                                               */
int cbx_bias_act(int act, const cbx_tensor* x, const cbx_tensor* bias,
                 cbx_tensor* y, cbx_stream stream);

/* ggml_add(a, b) / ggml_mul(a, b) with b repeated to a's shape
 * (ggml_can_repeat(b, a): every a.ne[i] a multiple of b.ne[i]): y = a + b or
 * a * b, one f32 rounding.  The CFM decoder's mul(x, mask (1, T)) before its
 * 1x1 convs and around final_proj (cfm_decoder.cpp:176,553,555) and the
 * residual join that ends a transformer stack (:244).  F32; a, y the same shape,
 * any strides (nb[0] the element size); y may be a itself, and must not
 * overlap b.                                                              */
typedef enum {
    CBX_BINARY_ADD = 0,
    CBX_BINARY_MUL = 1,
} cbx_binary_op;
int cbx_binary(int op, const cbx_tensor* a, const cbx_tensor* b, cbx_tensor* y,
               cbx_stream stream);

/* ggml_add(r, ggml_add(x, bias)) in one pass: y = r + (x + bias), each add
 * one f32 rounding, the inner one first.  bias repeats to x's shape and x
 * to r's (ggml_can_repeat).  The projections whose biased output joins a
 * residual with no norm between: a transformer stack's last ff.2
 * (cfm_decoder.cpp:242-244) and a resnet's time MLP, its (C_out) output
 * broadcast over the frames (:162-165).  F32, any strides (nb[0] the
 * element size); y the shape of r and may be r itself (or x, when x has
 * r's shape); y must not overlap bias.                                    */
int cbx_bias_residual(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* r,
                      cbx_tensor* y, cbx_stream stream);

/* ggml_add(s, u) and ggml_add(s, v) of one s = ggml_add(x, bias), s not
 * stored: yu = (x + bias) + u, yv = (x + bias) + v, each add one f32
 * rounding.  The relative-position attention's query terms: q's bias, then
 * pos_bias_u and pos_bias_v over the (64, 8, T) query heads
 * (flow_encoder.cpp:320, 341-345).  bias, u and v repeat to x's shape
 * (ggml_can_repeat); yu and yv have x's shape.  F32, any strides (nb[0]
 * the element size); yu and yv overlap neither each other nor an input.   */
int cbx_bias_add_pair(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* u,
                      const cbx_tensor* v, cbx_tensor* yu, cbx_tensor* yv,
                      cbx_stream stream);

/* Two independent ggml_add(x, bias) in one launch: y0 = x0 + b0 and
 * y1 = x1 + b1, each one f32 rounding, as cbx_bias_act with no activation.
 * Two adjacent bias adds that do not read each other: the projections of v
 * and k (flow_encoder.cpp:320-322), of q and v (s3enc.cpp:205-207).  Each
 * bias contiguous with ne = (x.ne0,1,1,1) or (1,x.ne1,1,1); each y has its
 * x's shape and may be that x itself; neither y may overlap its bias or
 * the other add's tensors.                                                  */
int cbx_bias_add_two(const cbx_tensor* x0, const cbx_tensor* b0, cbx_tensor* y0,
                     const cbx_tensor* x1, const cbx_tensor* b1, cbx_tensor* y1,
                     cbx_stream stream);

/* ggml_scale(x, s): y = x * s, one f32 rounding.  The mean of a HiFT
 * stage's three resblocks, scale(sum, 1/3) (hift_vocoder.cpp:736).  F32,
 * any strides (nb[0] the element size); y x's shape, and may be x itself
 * (no other overlap).                                                     */
int cbx_scale(const cbx_tensor* x, float s, cbx_tensor* y, cbx_stream stream);

/* ggml_concat(a, b, dim): y.ne[dim] = a.ne[dim] + b.ne[dim], the other
 * dims equal to a's and b's; a's elements first (cfm_decoder.cpp:489-491
 * packing x, mu, spks, cond along the channels; :530 the skip join; :476
 * the time embeddings).  F32
 * or F16 (all three the same type), any strides; y must not overlap a or b.
 * dim 0..3.                                                               */
int cbx_concat(const cbx_tensor* a, const cbx_tensor* b, int dim, cbx_tensor* y,
               cbx_stream stream);

/* ggml_swiglu_split(g, u) = silu(g) * u, F32 or F16. */
int cbx_swiglu(const cbx_tensor* g, const cbx_tensor* u, cbx_tensor* y,
               cbx_stream stream);

/* snake() = x + sin^2(x * alpha) * alpha_inv in one pass
 * (hift_vocoder.cpp:64-73; alpha_inv = 1/(alpha + 1e-9) precomputed by the
 * caller as at hift_vocoder.cpp:413-427).  x, y F32; alpha, alpha_inv F32
 * with ne = (x.ne0,1,1,1) (channel innermost, the reference's (C, T)
 * layout) or (1,x.ne1,1,1) (channel outer).                                */
int cbx_snake(const cbx_tensor* x, const cbx_tensor* alpha,
              const cbx_tensor* alpha_inv, cbx_tensor* y, cbx_stream stream);

/* ---- HiFT convolutions -------------------------------------------------- */

/* Weights of one conv1d, prepared once for the matrix cores: an f16 copy of
 * a ggml (K, C_in, C_out) F32/F16 weight (the reference's ConvW.w,
 * hift_vocoder.cpp:77-93; PyTorch (C_out, C_in, K) order), rounded as the
 * reference's mul_mat rounds its F32 operand to F16.  Allocates device
 * memory on the current device; returns when the copy is complete (the
 * source may then be freed).  K <= 64, C_in and C_out <= 8192.            */
typedef struct cbx_conv1d_weights cbx_conv1d_weights;
int  cbx_conv1d_weights_create(const cbx_tensor* w, cbx_stream stream,
                               cbx_conv1d_weights** out);
void cbx_conv1d_weights_destroy(cbx_conv1d_weights* w);

typedef enum cbx_conv_prologue {
    CBX_CONV_PRO_NONE       = 0,
    CBX_CONV_PRO_SNAKE      = 1,  /* snake(x) = x + sin^2(x*alpha)*alpha_inv  */
    CBX_CONV_PRO_LEAKY_RELU = 2,  /* leaky_relu(x, slope)                     */
} cbx_conv_prologue;

/* conv1d_CT(pro(x)) (+ bias) (+ res) in one kernel, on the reference's
 * (C, T) layout, channel innermost (hift_vocoder.cpp:46-59,77-93):
 *   y[t][co] = res[t][co] + (bias[co] + sum_{ci,k} f16(w[co][ci][k]) *
 *              f16(pro(x)[t*stride + k*dilation - pad][ci]))
 * with zero padding outside [0, T_in): the ResBlock sublayer's snake ->
 * conv and snake -> conv -> + x (hift_vocoder.cpp:119-138) are two calls;
 * leaky_relu -> conv_post (:748-749) one.  Products are summed in f32 on
 * the matrix cores, as the reference's im2col (F16) + mul_mat (PREC_F32)
 * sums them (order differs).  x: F32 (C_in, T_in, B, 1), rows of C_in
 * contiguous floats; y, res: F32 (C_out, T_out, B, 1), T_out = (T_in +
 * 2 pad - dilation (K - 1) - 1) / stride + 1; bias: F32 C_out or NULL;
 * alpha, alpha_inv: F32 C_in (snake only).  y may be res, not x.           */
int cbx_conv1d(const cbx_tensor* x, const cbx_conv1d_weights* w, int stride,
               int pad, int dilation, int prologue, const cbx_tensor* alpha,
               const cbx_tensor* alpha_inv, float slope,
               const cbx_tensor* bias, const cbx_tensor* res, cbx_tensor* y,
               cbx_stream stream);

/* cbx_conv1d with a HiFT stage's ResBlock sum folded into it
 * (hift_vocoder.cpp:731-736: sum = ggml_add(sum, r), then x =
 * ggml_scale(sum, 1/3) after the last resblock):
 *   y = (acc + r) * scale,  r = cbx_conv1d's output (res required for the
 * ResBlock's last conv; may be NULL)
 * each step one f32 rounding in that order; scale 1.0f multiplies by
 * nothing.  acc: F32 with y's shape, not overlapping y.                    */
int cbx_conv1d_sum(const cbx_tensor* x, const cbx_conv1d_weights* w, int stride,
                   int pad, int dilation, int prologue, const cbx_tensor* alpha,
                   const cbx_tensor* alpha_inv, float slope,
                   const cbx_tensor* bias, const cbx_tensor* res,
                   const cbx_tensor* acc, float scale, cbx_tensor* y,
                   cbx_stream stream);

/* Weights of one transposed conv1d with stride `stride` (the HiFT
 * upsamplers' ups.i, hift_vocoder.cpp:96-115, 255-259): a ggml (K, C_out,
 * C_in) F32/F16 weight (PyTorch ConvTranspose1d's (C_in, C_out, K) order)
 * split into `stride` phases for the matrix cores, rounded to f16 as the
 * reference's conv_transpose_1d rounds an F32 kernel.  Same handle type,
 * lifetime and limits as cbx_conv1d_weights_create; stride 1..64.  A
 * handle made here is only accepted by cbx_conv_transpose1d, and one made
 * by cbx_conv1d_weights_create only by cbx_conv1d.                        */
int cbx_conv_transpose1d_weights_create(const cbx_tensor* w, int stride,
                                        cbx_stream stream,
                                        cbx_conv1d_weights** out);

/* conv_transpose1d_CT(pro(x)) (+ bias) in one kernel, on the reference's
 * (C, T) layout (hift_vocoder.cpp:96-115, called at :686-687 right after
 * leaky_relu, which is the prologue here):
 *   full[i*stride + k][co] += f16(w[ci][co][k]) * f16(pro(x)[i][ci]),
 *   y[t][co] = bias[co] + full[t + pad][co],  0 <= t < T_out,
 * T_out = (T_in - 1) * stride + K - 2 pad -- ggml_conv_transpose_1d (p0 = 0,
 * d0 = 1), the view that strips `pad` from both ends, then the bias add.
 * Computed as `stride` phase convs on the matrix cores, products summed in
 * f32 (the reference sums per-tap f16 dot products; order differs).
 * x: F32 (C_in, T_in, B, 1); y: F32 (C_out, T_out, B, 1), not
 * overlapping x; bias: F32 C_out or NULL; alpha, alpha_inv: snake only.   */
int cbx_conv_transpose1d(const cbx_tensor* x, const cbx_conv1d_weights* w,
                         int pad, int prologue, const cbx_tensor* alpha,
                         const cbx_tensor* alpha_inv, float slope,
                         const cbx_tensor* bias, cbx_tensor* y,
                         cbx_stream stream);

/* The CFM decoder's CausalConv1d with causal_block1d's pre-mask in one
 * kernel (cfm_decoder.cpp:89-120, called at :139-142 after
 * h = ggml_mul(x, mask)): transpose -> cont -> left pad of K - 1 zero
 * frames (left_pad_TC, :66-77) -> im2col (F16) -> mul_mat (PREC_F32) ->
 * + bias -> transpose -> cont.
 *   y[t][co] = bias[co] + sum_{ci,k} f16(w[co][ci][k]) *
 *              f16(x[t + k - (K - 1)][ci] * mask[t + k - (K - 1)])
 * with zero frames before t = 0.  Weights from cbx_conv1d_weights_create.
 * x: F32 (C_in, T, B, 1); y: F32 (C_out, T, B, 1), not overlapping x;
 * mask: F32 with T contiguous elements (ggml (1, T)) or NULL; bias: F32
 * C_out or NULL.                                                           */
int cbx_causal_conv1d(const cbx_tensor* x, const cbx_conv1d_weights* w,
                      const cbx_tensor* mask, const cbx_tensor* bias,
                      cbx_tensor* y, cbx_stream stream);

/* ---- model tables from a GGUF file ---------------------------------------- */

/* The reference reads its weights with ggml's gguf reader: the header,
 * key/values and tensor directory first, then each tensor's bytes from
 * data_offset + offset, uploaded to the backend (chatterbox-cpp/src/
 * model.cpp:41-121).  These entry points do the same for device memory the
 * caller owns, so the token/position tables of a GGUF (F32, F16 or Q8_0,
 * e.g. token_embd.text.weight, position_embd.weight) feed cbx_get_rows*
 * directly.  Host code; only cbx_gguf_upload touches the device.          */
typedef struct cbx_gguf cbx_gguf;

typedef struct cbx_gguf_tensor_info {
    const char* name;         /* valid until cbx_gguf_close               */
    int32_t     type;         /* ggml_type numbering                       */
    int32_t     n_dims;
    int64_t     ne[4];        /* unused dimensions are 1                   */
    size_t      nbytes;       /* bytes of the tensor's data                */
    size_t      file_offset;  /* absolute offset of the data in the file  */
} cbx_gguf_tensor_info;

/* Parses a GGUF v2/v3 file (gguf_init_from_file with no_alloc,
 * model.cpp:46-57): checks the magic, version, every key's encoding, the
 * alignment, each tensor's type, shape and that its data lies inside the
 * file.  Keeps string-valued keys (general.architecture, ...).            */
int         cbx_gguf_open(const char* path, cbx_gguf** out);
void        cbx_gguf_close(cbx_gguf* gguf);
int64_t     cbx_gguf_n_tensors(const cbx_gguf* gguf);
/* Index of the tensor named `name`, or -1.                                 */
int64_t     cbx_gguf_find_tensor(const cbx_gguf* gguf, const char* name);
/* Value of a string key, or NULL (model.cpp:32-36).                        */
const char* cbx_gguf_get_str(const cbx_gguf* gguf, const char* key);
int         cbx_gguf_tensor(const cbx_gguf* gguf, int64_t index,
                            cbx_gguf_tensor_info* out);
/* A contiguous descriptor of tensor `index` whose data sits at `data`
 * (F32, F16, Q8_0 or I32; ggml strides, nb[0] = block size).              */
int         cbx_gguf_describe(const cbx_gguf* gguf, int64_t index, void* data,
                              cbx_tensor* out);
/* Copies tensor `index`'s bytes from the file to device memory `dst`
 * (at least nbytes) on `stream`, staged through host memory; returns when
 * the copy has completed (model.cpp:97-121).                               */
int         cbx_gguf_upload(const cbx_gguf* gguf, int64_t index, void* dst,
                            size_t dst_bytes, cbx_stream stream);

/* ---- one launch for several independent ops ------------------------------ */

/* A ggml graph step often holds several small ops that do not depend on
 * each other (RoPE on q and on k, s3enc.cpp:217-226; a decode step's norm,
 * rotary and gate ops); each as its own kernel pays a fixed launch cost
 * larger than its work.  cbx_run_ops runs up to CBX_MAX_OPS of them in one
 * kernel launch, workgroup ranges mapped to ops, with the same results as
 * the single-op entry points.  No counterpart in ggml's API: it is the
 * launch-level analogue of the scheduler running several graph nodes.     */
typedef enum cbx_op_kind {
    CBX_OP_LAYER_NORM              = 1, /* src0 x, src1 w|NULL, src2 b|NULL -> dst0 y; eps, act           */
    CBX_OP_RMS_NORM                = 2, /* src0 x, src1 g|NULL -> dst0 y; eps                            */
    CBX_OP_UNARY                   = 3, /* src0 x -> dst0 y; act = the cbx_unary_op                      */
    CBX_OP_LEAKY_RELU              = 4, /* src0 x -> dst0 y; param = negative slope                      */
    CBX_OP_SWIGLU                  = 5, /* src0 g, src1 u -> dst0 y                                       */
    CBX_OP_ROPE                    = 6, /* src0 x, src1 pos -> dst0 y; rope = table                       */
    CBX_OP_GET_ROWS                = 7, /* src0 table, src1 ids [, src2 table2, src3 ids2: added] -> dst0 */
    CBX_OP_GET_ROWS_ADD_LAYER_NORM = 8, /* src0..3 as GET_ROWS, src4 w, src5 b -> dst0 h|NULL, dst1 y; eps */
    CBX_OP_SNAKE                   = 9, /* src0 x, src1 alpha, src2 alpha_inv -> dst0 y                   */
    CBX_OP_GROUP_NORM              = 10, /* src0 x, src1 w|NULL, src2 b|NULL -> dst0 y; iparam n_groups,
                                            eps, act (NONE or MISH): the split reduction, out of place   */
    CBX_OP_LAYER_NORM_ROPE         = 11, /* src0 x, src1 w|NULL, src2 b|NULL, src3 pos -> dst0 y;
                                            iparam head_dim, eps, rope = table                           */
} cbx_op_kind;

typedef struct cbx_op {
    int32_t               kind;    /* cbx_op_kind */
    int32_t               act;     /* cbx_unary_op (CBX_OP_UNARY, CBX_OP_LAYER_NORM epilogue,
                                      CBX_OP_GROUP_NORM) */
    float                 eps;
    float                 param;
    const cbx_tensor*     src[6];
    cbx_tensor*           dst[2];
    const cbx_rope_cache* rope;
    int32_t               iparam;  /* CBX_OP_GROUP_NORM: n_groups; CBX_OP_LAYER_NORM_ROPE: head_dim */
    int32_t               reserved; /* must be 0 */
} cbx_op;

#define CBX_MAX_OPS 12

/* Runs ops[0..n_ops) in one kernel launch on `stream`.  The ops must be
 * independent: no op may write memory that another op of the call reads
 * or writes (checked on the host; an op's dst may be its own src for the
 * norms, RoPE and the element-wise ops).  Operands follow the single-op
 * rules, restricted to the layouts the one-launch kernel handles (anything
 * else returns CBX_ERR_UNSUPPORTED and launches nothing):
 *   - rows at one uniform byte stride, nb[0] = element size;
 *   - norms: ne0 % 4 == 0 and ne0 <= 1024, rows and w/b 16-byte (F32) or
 *     8-byte (F16) aligned;
 *   - UNARY / LEAKY_RELU / SWIGLU: contiguous, same alignment, any length;
 *   - ROPE: n_dims <= 512 (columns n_dims..ne0 are copied, as ggml does);
 *   - gathers: 1-D ids, 2-D tables, ne0 % 4 == 0 (<= 1024 with LayerNorm),
 *     F32 destination rows 16-byte aligned;
 *   - SNAKE: F32, contiguous, 16-byte aligned, ne0 % 4 == 0;
 *   - GROUP_NORM: the layouts and sizes cbx_group_norm runs as the split
 *     reduction (contiguous groups, out of place, a few large groups; no
 *     activation or Mish; at most 4 vectors a lane), its chunk workgroups
 *     resident at once with every other GROUP_NORM of the call (at most 2
 *     a CU in all, 1024 chunk slots in all); the exchange words in the
 *     library's scratch set for `stream`, as cbx_group_norm_noalloc's;
 *   - LAYER_NORM_ROPE: cbx_layer_norm_rope's operands with F32 rows at one
 *     stride, the rotation partners of a head in one wave (head_dim / 4
 *     divides 64; NEOX: n_dims % 8 == 0 and n_dims / 8 a power of two;
 *     NORMAL: n_dims % 4 == 0) and a 16-byte aligned table.
 * GROUP_NORM ops run first in the launch (their workgroups get the CUs
 * first, so all of a group's chunks are resident); the results do not
 * depend on the order.                                                    */
int cbx_run_ops(const cbx_op* ops, int n_ops, cbx_stream stream);

/* ---- ggml-style node lists ------------------------------------------------ */

/* The reference's graph builders emit the ops of this library as short node
 * chains that its backend scheduler then runs one node at a time
 * (ggml_backend_sched_graph_compute, chatterbox-cpp/src/backend.cpp:108-122;
 * the chains: layer_norm cfm_decoder.cpp:29-33, mish cfm_decoder.cpp:36-38,
 * snake hift_vocoder.cpp:64-73, T3 input t3.cpp:446-466, attention scores
 * t3.cpp:513-518).  A backend's graph_compute can pass its nodes here in
 * graph order: the planner takes, at each node, the longest known chain
 * whose intermediate results no other node reads and the caller does not
 * keep, and runs it as one fused call; everything else runs as the
 * single-node entry points, or is reported as not supported.
 *
 * Tensors are given once, in an array; nodes refer to them by index.  A
 * node reads src[] (-1 = none) and writes dst, ggml's broadcast rules
 * apply to ADD/MUL operands, and a VIEW node only re-describes its
 * source's memory (ggml's VIEW, RESHAPE, PERMUTE, TRANSPOSE: no launch).
 *
 * The HiFT convolutions arrive as the node runs conv1d_CT and
 * conv_transpose1d_CT emit (hift_vocoder.cpp:77-116), optionally after
 * snake() or leaky_relu and, for conv1d, before the ResBlock's residual
 * add (:131-135):
 *   conv1d:  VIEW (transpose) -> CPY (cont) -> IM2COL -> VIEW (2-D) ->
 *            VIEW (weight 2-D) -> MUL_MAT -> VIEW (3-D) [-> VIEW (bias as
 *            (1, C_out)) -> ADD] -> VIEW (transpose) -> CPY (cont)
 *   transposed: VIEW (transpose) -> CPY (cont) -> CONV_TRANSPOSE_1D ->
 *            VIEW (crop) -> CPY (cont) [-> VIEW (bias) -> ADD] -> VIEW
 *            (transpose) -> CPY (cont)
 * and run as one cbx_conv1d / cbx_conv_transpose1d call with the weights
 * the backend prepared at load time, given on the MUL_MAT /
 * CONV_TRANSPOSE_1D node (conv_w).  The CFM decoder's causal_conv1d
 * (cfm_decoder.cpp:89-120), optionally after causal_block1d's
 * MUL(x, mask), runs as one cbx_causal_conv1d call:
 *   VIEW (transpose) -> CPY (cont) -> VIEW (its first K-1 frames) -> CPY
 *   -> SCALE (0) -> CONCAT (zeros, cont; dim 0) -> IM2COL (1, 0, 1) ->
 *   VIEW (2-D) -> VIEW (weight 2-D) -> MUL_MAT [-> VIEW (bias) -> ADD] ->
 *   VIEW (transpose) -> CPY (cont)
 * The T3 input with the conditioning prefix (t3.cpp:432-466) runs as one
 * cbx_get_rows_concat_add_layer_norm call:
 *   [GET_ROWS (prompt) [-> CPY] -> CONCAT (prefix, ., dim 1) ->] GET_ROWS
 *   (text) [-> CPY] -> CONCAT (., ., dim 1) -> GET_ROWS (positions)
 *   [-> CPY] -> ADD -> NORM -> MUL -> ADD
 * (without the prompt segment the text gather's CONCAT takes the prefix).  */
typedef enum cbx_gop {
    CBX_GOP_VIEW          = 0,  /* dst describes src0's memory                       */
    CBX_GOP_GET_ROWS      = 1,  /* src0 table, src1 ids I32                           */
    CBX_GOP_ADD           = 2,  /* src0 + src1 (a bias add, or inside a chain)        */
    CBX_GOP_MUL           = 3,  /* src0 * src1 (only inside a chain)                  */
    CBX_GOP_SCALE         = 4,  /* src0 * fparam                                      */
    CBX_GOP_NORM          = 5,  /* fparam = eps                                       */
    CBX_GOP_RMS_NORM      = 6,  /* fparam = eps                                       */
    CBX_GOP_GROUP_NORM    = 7,  /* iparam = n_groups, fparam = eps                    */
    CBX_GOP_ROPE          = 8,  /* src0 x, src1 pos I32; rope = the parameters' cache */
    CBX_GOP_SOFT_MAX      = 9,  /* fparam = scale (ggml_soft_max: 1.0); no mask src  */
    CBX_GOP_DIAG_MASK_INF = 10, /* iparam = n_past (only before SOFT_MAX)             */
    CBX_GOP_UNARY         = 11, /* iparam = cbx_unary_op (GELU .. SQR)                */
    CBX_GOP_LEAKY_RELU    = 12, /* fparam = negative slope                            */
    CBX_GOP_CPY           = 13, /* ggml_cpy / ggml_cast to dst's type (F32, F16)      */
    CBX_GOP_IM2COL        = 14, /* src0 kernel (shape), src1 data; conv = s0, p0, d0 */
    CBX_GOP_MUL_MAT       = 15, /* src0 x src1 (only inside a conv1d chain); conv_w */
    CBX_GOP_CONV_TRANSPOSE_1D = 16, /* src0 kernel, src1 data; conv[0] = s0; conv_w */
    CBX_GOP_CONCAT        = 17, /* src0 then src1 along dim iparam              */
} cbx_gop;

typedef struct cbx_gnode {
    int32_t               op;      /* cbx_gop                                  */
    int32_t               dst;     /* tensor index                             */
    int32_t               src[2];  /* tensor indices, -1 = none                */
    int32_t               iparam;
    float                 fparam;
    const cbx_rope_cache* rope;    /* CBX_GOP_ROPE                             */
    int32_t               conv[3]; /* CBX_GOP_IM2COL: stride, padding, dilation;
                                      CONV_TRANSPOSE_1D: stride (p0 0, d0 1)  */
    const cbx_conv1d_weights* conv_w; /* MUL_MAT of a conv1d chain, CONV_TRANSPOSE_1D:
                                      the weights prepared from its kernel   */
} cbx_gnode;

/* What one planned launch runs: nodes [first_node, first_node + n_nodes). */
typedef enum cbx_glaunch_kind {
    CBX_GL_UNSUPPORTED = 0,   /* one node the library does not run              */
    CBX_GL_VIEW,              /* one VIEW node: nothing to launch               */
    CBX_GL_GET_ROWS,          /* get_rows [-> cast]                             */
    CBX_GL_GET_ROWS_ADD,      /* get_rows [-> cast] -> get_rows [-> cast] -> add */
    CBX_GL_GET_ROWS_ADD_LAYER_NORM, /* ... -> add -> norm -> mul -> add         */
    CBX_GL_NORM,              /* norm                                           */
    CBX_GL_LAYER_NORM,        /* norm -> mul -> add [-> softplus -> tanh -> mul] */
    CBX_GL_LAYER_NORM_ROPE,   /* norm -> mul -> add -> view -> rope             */
    CBX_GL_RMS_NORM,          /* rms_norm [-> mul]                              */
    CBX_GL_GROUP_NORM,        /* group_norm [-> mul -> add] [-> mish chain]     */
    CBX_GL_SOFT_MAX,          /* [scale ->] [diag_mask_inf ->] soft_max         */
    CBX_GL_SNAKE,             /* mul -> sin -> sqr -> mul -> add                */
    CBX_GL_UNARY,             /* one unary op, or softplus -> tanh -> mul (mish) */
    CBX_GL_SWIGLU,            /* silu -> mul                                    */
    CBX_GL_LEAKY_RELU,
    CBX_GL_ROPE,
    CBX_GL_CPY,
    CBX_GL_ADD_LAYER_NORM,    /* [add(x, bias) ->] add(., r) -> norm -> mul -> add [-> mish chain] */
    CBX_GL_LAYER_NORM_MASK,   /* norm -> mul -> add [-> mish chain] -> mul(., mask (1, ne1)) */
    CBX_GL_BIAS_ACT,          /* add(x, bias) [-> unary op | -> mish chain]     */
    CBX_GL_CONV1D,            /* [snake | leaky_relu ->] conv1d chain [-> add(x, .)] */
    CBX_GL_CONV_TRANSPOSE1D,  /* [snake | leaky_relu ->] transposed conv chain  */
    CBX_GL_CAUSAL_CONV1D,     /* [mul(x, mask (1, T)) ->] causal conv chain     */
    CBX_GL_GET_ROWS_CONCAT_ADD_LAYER_NORM, /* [get_rows [-> cast] -> concat(prefix, .) ->]
                                 get_rows [-> cast] -> concat -> get_rows [-> cast]
                                 -> add -> norm -> mul -> add (t3.cpp:432-466)   */
    CBX_GL_BINARY,            /* one add or mul whose second operand repeats to the
                                 first's shape (cbx_binary): a per-frame mask, a
                                 residual join no norm follows. flags: the op   */
    CBX_GL_CONCAT,            /* one concat (cbx_concat)                        */
    CBX_GL_BIAS_RESIDUAL,     /* add(x, bias) [-> view (same dims)] -> add(r, .)
                                 with no norm after it (cbx_bias_residual)      */
    CBX_GL_SCALE,             /* one scale no soft_max follows (cbx_scale)      */
    CBX_GL_BIAS_ADD_PAIR,     /* add(x, bias) -> view (a contiguous reshape) ->
                                 [views of other tensors] add(., u), add(., v)
                                 (cbx_bias_add_pair)                            */
    CBX_GL_BIAS_ADD_TWO,      /* two lone bias adds in a row, independent of
                                 each other (cbx_bias_add_two)                  */
    CBX_GL_ROPE_TWO,          /* two rope nodes in a row on separate tensors
                                 (cbx_run_ops; the two cbx_rope_ext calls for
                                 layouts it does not take)                      */
} cbx_glaunch_kind;

typedef struct cbx_glaunch {
    int32_t kind;         /* cbx_glaunch_kind                                   */
    int32_t first_node;
    int32_t n_nodes;
    int32_t flags;        /* bit 0: an intermediate the fused kernel may skip
                             storing (the embedding sum h nobody reads).
                             Conv kinds: bits 0-1 the prologue (0 none, 1
                             snake, 2 leaky_relu, 3 the frame mask), bit 2 a
                             bias add, bit 3 the residual add; CONV1D also
                             bit 4 an add of another tensor after the
                             residual add and bit 5 a scale after that (the
                             ResBlock sum and mean, cbx_conv1d_sum).          */
} cbx_glaunch;

/* Splits nodes[0..n_nodes) into launches, in order, covering every node
 * (CBX_GL_UNSUPPORTED for a node that starts no chain the library runs).
 * keep[0..n_keep): tensor indices read after the node list (graph outputs,
 * inputs of another backend's nodes): never left unstored.  Chains are
 * matched on op structure, operand roles and broadcast shapes; the entry
 * point a launch maps to checks the rest of the layout when it runs.
 * Host only.  *n_launches gets the count even when max_launches is short. */
int cbx_graph_plan(const cbx_tensor* tensors, int32_t n_tensors,
                   const cbx_gnode* nodes, int32_t n_nodes,
                   const int32_t* keep, int32_t n_keep,
                   cbx_glaunch* launches, int32_t max_launches,
                   int32_t* n_launches);

/* Runs one planned launch on `stream` (CBX_GL_UNSUPPORTED: returns
 * CBX_ERR_UNSUPPORTED and launches nothing).                               */
int cbx_graph_launch(const cbx_tensor* tensors, int32_t n_tensors,
                     const cbx_gnode* nodes, int32_t n_nodes,
                     const cbx_glaunch* launch, cbx_stream stream);

/* Plans and runs the whole node list on `stream`.  If any node is
 * unsupported, returns CBX_ERR_UNSUPPORTED naming it and launches nothing.
 * *n_launches (may be NULL) gets the number of kernel launches issued.    */
int cbx_graph_compute(const cbx_tensor* tensors, int32_t n_tensors,
                      const cbx_gnode* nodes, int32_t n_nodes,
                      const int32_t* keep, int32_t n_keep,
                      cbx_stream stream, int32_t* n_launches);

/* The same node list planned once and recorded into a HIP graph, for a
 * caller that runs one list again and again over the same buffers (a
 * decode or sampling loop: each step's graph_compute in
 * t3.cpp:604, cfm_decoder.cpp:596, hift_vocoder.cpp:765 rebuilds and
 * re-runs an identical node list).  The graph holds the tensors' addresses
 * and shapes and the nodes' parameters as they are at creation; each
 * cbx_graph_exec_launch replays every launch on `stream` (one host call,
 * whatever the launch count) over whatever the buffers hold then.  A
 * change of address, shape or parameter needs cbx_graph_exec_update.  Launch on the
 * device current at creation.  Unsupported nodes: CBX_ERR_UNSUPPORTED as in
 * cbx_graph_compute.  *n_launches (may be NULL) gets the kernel launch
 * count of one replay.  Each exec holds a HIP stream of its own, which its
 * captures are recorded on (nothing runs on it), and two instantiations of
 * the graph, which take turns (cbx_graph_exec_update), until it is
 * destroyed.  Destroy waits for the exec's own replays (not for other work
 * on the device); every stream it was launched on must still exist then. */
typedef struct cbx_graph_exec cbx_graph_exec;
int  cbx_graph_exec_create(const cbx_tensor* tensors, int32_t n_tensors,
                           const cbx_gnode* nodes, int32_t n_nodes,
                           const int32_t* keep, int32_t n_keep,
                           cbx_graph_exec** out, int32_t* n_launches);
int  cbx_graph_exec_launch(cbx_graph_exec* exec, cbx_stream stream);
void cbx_graph_exec_destroy(cbx_graph_exec* exec);

/* The exec re-pointed at the list as it is now (the next step of the same
 * loop: t3.cpp:604's decode graph with the position and the KV views of the
 * next token).  The list is planned and recorded again; when it gives the
 * same launches with other arguments (addresses, shapes, positions), the
 * instantiated graph takes them in place (*in_place = 1), otherwise it is
 * re-instantiated (*in_place = 0).  Stream-ordered: the exec's two
 * instantiations take turns, and an update re-points the one not replayed
 * since the previous update, after waiting (on events recorded by that
 * update) for its replays -- all issued before the previous update -- and
 * for nothing else.  So replays queued so far keep the arguments they were
 * queued with, the replay launched just before this update may still run
 * while the host updates (a per-step loop keeps the device busy), and other
 * streams' work is never waited for.  Every stream the exec was launched on
 * since the previous update must still exist.  On an error of planning or
 * recording (an unsupported node, a bad layout) `exec` is left as it was;
 * after CBX_ERR_HIP (the new graph could not be instantiated) destroy it.
 * Same device as at creation.  *n_launches and *in_place may be NULL.      */
int  cbx_graph_exec_update(cbx_graph_exec* exec,
                           const cbx_tensor* tensors, int32_t n_tensors,
                           const cbx_gnode* nodes, int32_t n_nodes,
                           const int32_t* keep, int32_t n_keep,
                           int32_t* n_launches, int32_t* in_place);

#ifdef __cplusplus
}
#endif
#endif /* CBXOPS_H */
