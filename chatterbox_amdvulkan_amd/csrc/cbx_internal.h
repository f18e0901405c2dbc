// cbx_internal.h -- definitions shared by the host ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/cbxops.h"

namespace cbx {

// A tensor view passed to kernels by value.
struct View {
    char*   data;
    int64_t ne[4];
    int64_t nb[4];
};

inline View view_of(const cbx_tensor* t) {
    View v;
    v.data = static_cast<char*>(t->data);
    for (int i = 0; i < 4; i++) {
        v.ne[i] = t->ne[i];
        v.nb[i] = static_cast<int64_t>(t->nb[i]);
    }
    return v;
}

// Rows of t (ne[1..3]) sit at uniform byte steps of nb[1].
// (Each dimension k >= 2 with ne[k] > 1 has nb[k] = nb[1] * ne[1] * ... * ne[k-1].)
inline bool flat_rows(const cbx_tensor* t) {
    size_t step = t->nb[1] * static_cast<size_t>(t->ne[1]);
    for (int k = 2; k < 4; k++) {
        if (t->ne[k] > 1 && t->nb[k] != step) return false;
        step *= static_cast<size_t>(t->ne[k]);
    }
    return true;
}

inline View null_view() {
    View v;
    v.data = nullptr;
    for (int i = 0; i < 4; i++) { v.ne[i] = 1; v.nb[i] = 0; }
    return v;
}

// Per-device state created by cbx_init.
struct DeviceState {
    bool      ready = false;
    int       n_cu = 0;
    uint16_t* gelu_table = nullptr;   // 65536 fp16 codes
    uint32_t* err_word = nullptr;     // sticky device error bits
    void*     gn_scratch = nullptr;   // this device's address of the static group norm scratch
    bool      gn_split_ok = false;    // dispatch deals workgroups to XCDs by index mod 8 (probed)
};

// Device error bits.
enum : uint32_t {
    DEV_ERR_ROW_INDEX = 1u,   // a get_rows index was out of range (row zeroed)
    DEV_ERR_RESERVED1 = 2u,   // no longer raised (in-place GroupNorm never takes the split)
};

// ---- host helpers implemented in cbx_api.cpp ----------------------------
int  set_error(int code, const std::string& msg);
void clear_error();
// Current device's state, or nullptr (and an error recorded) when cbx_init
// has not been called for it.
DeviceState* current_state(int* code);
int  check_launch(const char* what);

int64_t nelements(const cbx_tensor* t);
int64_t nrows(const cbx_tensor* t);
size_t  type_size(int type);
bool    is_contiguous(const cbx_tensor* t);
bool    rows_contiguous(const cbx_tensor* t);   // nb[0] == element size
bool    same_shape(const cbx_tensor* a, const cbx_tensor* b);
bool    bytes_overlap(const cbx_tensor* a, const cbx_tensor* b);   // the byte ranges of the two tensors meet
// Validates pointer, type, non-negative sizes and nb[0] for a float/int
// tensor.  Returns 0 or a negative status with the error recorded.
int validate(const cbx_tensor* t, const char* what, const char* name);

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Kernel launchers, one per translation unit.
int launch_get_rows(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* src2,
                    const cbx_tensor* ids2, cbx_tensor* dst, DeviceState* st, hipStream_t s);
int launch_cpy(const cbx_tensor* src, cbx_tensor* dst, DeviceState* st, hipStream_t s);
int launch_row_norm(int kind, const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b,
                    float eps, int act, cbx_tensor* y, DeviceState* st, hipStream_t s);
int launch_embed_norm(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* src2, const cbx_tensor* ids2,
                      const cbx_tensor* w, const cbx_tensor* b, float eps, cbx_tensor* h, cbx_tensor* y,
                      DeviceState* st, hipStream_t s);
// The T3 input with the conditioning prefix: rows of concat(prefix,
// get_rows(src_a, ids_a), get_rows(src_b, ids_b)) + get_rows(src2, ids2),
// then LayerNorm (prefix and src_a/ids_a may be null).
int launch_embed_concat_norm(const cbx_tensor* prefix, const cbx_tensor* src_a, const cbx_tensor* ids_a,
                             const cbx_tensor* src_b, const cbx_tensor* ids_b, const cbx_tensor* src2,
                             const cbx_tensor* ids2, const cbx_tensor* w, const cbx_tensor* b, float eps,
                             cbx_tensor* h, cbx_tensor* y, DeviceState* st, hipStream_t s);
int launch_group_norm(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w,
                      const cbx_tensor* b, int act, cbx_tensor* y, DeviceState* st,
                      hipStream_t s);
// The split-reduction GroupNorm over a workspace of
// group_norm_workspace_bytes() (zeroed once; never needs clearing again);
// in-place calls and layouts it does not cover go to launch_group_norm.
// wait_ticks: the longest wait of a workgroup for the others, in 100 MHz
// ticks (0: never wait; kGnWaitAuto: from the launch's size);
// n_chunks_req: chunks per group, 0 = automatic.
constexpr uint64_t kGnWaitAuto = ~uint64_t{0};
size_t group_norm_workspace_bytes();
// The current device's address of the library's static split-GroupNorm
// scratch (sets of group_norm_workspace_bytes()), for cbx_group_norm and
// cbx_group_norm_noalloc; called once per device by cbx_init.  The split
// handles up to group_norm_scratch_slots() group instances x chunks.
int group_norm_scratch_setup(void** out);
size_t group_norm_scratch_slots();
// The scratch set a call on stream s uses.
void* group_norm_scratch_for(const DeviceState* st, hipStream_t s);
// Launches a probe on the current device and sets *ok when workgroups with
// equal index mod 8 ran on one XCD (the split's assumption).
int group_norm_probe_xcd(bool* ok);
int launch_group_norm_split(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                            int act, cbx_tensor* y, void* workspace, uint64_t wait_ticks, int n_chunks_req,
                            DeviceState* st, hipStream_t s);
int launch_unary(int op, float param, const cbx_tensor* x, cbx_tensor* y, DeviceState* st,
                 hipStream_t s);
int launch_swiglu(const cbx_tensor* g, const cbx_tensor* u, cbx_tensor* y, DeviceState* st,
                  hipStream_t s);
int launch_bias_act(int op, const cbx_tensor* x, const cbx_tensor* bias, cbx_tensor* y, DeviceState* st,
                    hipStream_t s);
// cbx_binary and cbx_concat (k_binary.hip), arguments checked by the caller.
int launch_binary(int op, const cbx_tensor* a, const cbx_tensor* b, cbx_tensor* y, hipStream_t s);
int launch_scale(const cbx_tensor* x, float s, cbx_tensor* y, hipStream_t strm);
int launch_bias_add_two(const cbx_tensor* x0, const cbx_tensor* b0, cbx_tensor* y0, const cbx_tensor* x1,
                        const cbx_tensor* b1, cbx_tensor* y1, DeviceState* st, hipStream_t s);
int launch_bias_add_pair(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* u, const cbx_tensor* v,
                         cbx_tensor* yu, cbx_tensor* yv, hipStream_t s);
int launch_bias_residual(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* r, cbx_tensor* y,
                         hipStream_t s);
int launch_concat(const cbx_tensor* a, const cbx_tensor* b, int dim, cbx_tensor* y, hipStream_t s);
// LayerNorm with a residual-join prologue (r, optional a_bias; s stored
// when non-null) or a per-row mask epilogue (mask non-null, r null).
int launch_layer_norm_ext(const cbx_tensor* a, const cbx_tensor* a_bias, const cbx_tensor* r, const cbx_tensor* w,
                          const cbx_tensor* b, const cbx_tensor* mask, float eps, int act, cbx_tensor* s,
                          cbx_tensor* y, DeviceState* st, hipStream_t strm, const char* what);
// launch_conv1d's prologue past the public ones: x times a per-frame mask
// (passed as alpha, t_in floats)
constexpr int kConvProMask = 3;
// conv1d and transposed conv1d (k_conv1d.hip): padded extents of the
// prepared f16 weights, the weight conversion (up == 0: conv1d weight
// (K, C_in, C_out); up >= 1: transposed weight (K, C_out, C_in) split into
// max(up, 1) phases of `taps` taps), and the conv itself (up > 1: the
// transposed conv's phases, crop outputs cut from each end, w_ph halves of
// weights per phase).
int conv1d_weights_layout(int64_t c_in, int64_t c_out, int64_t* c_in_pad, int64_t* c_out_pad);
int launch_conv1d_weights(const cbx_tensor* w, int up, int64_t taps, _Float16* out, int64_t c_in_pad,
                          int64_t c_out_pad, hipStream_t s);
int launch_conv1d(const cbx_tensor* x, const _Float16* w16, int64_t k, int64_t c_in_pad, int64_t c_out, int stride,
                  int pad, int dil, int up, int crop, int64_t w_ph, int pro, const cbx_tensor* alpha,
                  const cbx_tensor* alpha_inv, float slope, const cbx_tensor* bias, const cbx_tensor* res, cbx_tensor* y,
                  DeviceState* st, hipStream_t s, const cbx_tensor* acc = nullptr, float oscale = 1.0f);
// Whether prepared weights were made from a weight of these extents: a
// conv1d weight (K, C_in, C_out) when up == 0, else a transposed weight
// (K, C_out, C_in) split for stride up.
bool conv1d_weights_match(const cbx_conv1d_weights* w, int up, int64_t k, int64_t c_in, int64_t c_out);
// Serial numbers distinct for every handle the process creates (0 for NULL).
uint64_t rope_cache_serial(const cbx_rope_cache* c);
uint64_t conv1d_weights_serial(const cbx_conv1d_weights* w);
int launch_snake(const cbx_tensor* x, const cbx_tensor* a, const cbx_tensor* ai, cbx_tensor* y,
                 DeviceState* st, hipStream_t s);

struct RopeParams {
    int   n_dims;
    int   mode;
    int   n_ctx_orig;
    float freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow;
    float theta_scale;
    float corr_dims[2];
};
int launch_rope(const cbx_tensor* x, const cbx_tensor* pos, const RopeParams& p,
                const float2* table, int32_t n_pos, const float* freq_factors_dev,
                cbx_tensor* y, DeviceState* st, hipStream_t s);
// b: the second score term added in front (x's shape), or null
int launch_soft_max(const cbx_tensor* x, const cbx_tensor* b, float s, int64_t n_past, cbx_tensor* y,
                    DeviceState* st, hipStream_t strm);
int launch_layer_norm_rope(const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int64_t head_dim,
                           const cbx_tensor* pos, const RopeParams& p, const float2* table, int32_t n_pos,
                           const float* ff, cbx_tensor* y, DeviceState* st, hipStream_t s);

// ---- one-launch op batch --------------------------------------------------
// A tensor of a batched op: base pointer and the byte step between rows
// (for id vectors: between elements).
struct BTen {
    char*   p;
    int64_t nb1;
};

// The split-reduction GroupNorm's arguments (its standalone kernel and the
// op batch's GroupNorm): the group instances' chunk workgroups, the
// workspace of tagged exchange words ([2 stages][slots x 4 waves][2 words],
// a stage kSplitStageWords long), the wait bound in 100 MHz ticks.
struct GnSplit {
    const char* x;
    char* y;
    const float* w;
    const float* b;
    uint64_t* word;
    const uint16_t* tab;
    int64_t x_nb3, y_nb3;    // batch strides (bytes)
    uint64_t wait_ticks;
    uint32_t n_chunks, n_gi, n_groups, per_ch, cpg, C;   // per_ch = ne0 * ne1
    float eps;
    int32_t act;
};

// The split GroupNorm of x (chunks per group automatic, or n_chunks_req)
// over workspace words from chunk slot first_slot on: fills *sp, the grid
// (*n_slots workgroups, a multiple of 8), the vectors a lane holds (*nv) and
// the chunk slots it uses (*slots_used), or returns false with *why when
// the split does not apply (in place, strided groups, too many or too few
// chunks, a grid not resident at once, a device whose dispatch was not seen
// to deal workgroups to XCDs by index mod 8).
bool group_norm_split_args(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                           int act, const cbx_tensor* y, void* workspace, uint32_t first_slot, uint64_t wait_ticks,
                           int n_chunks_req, const DeviceState* st, GnSplit* sp, uint32_t* n_slots, int* nv,
                           uint32_t* slots_used, const char** why);

// One op of a batch, in kernel-argument memory.  Field use by kind:
//   norms:     t0 x, t1 w, t2 b, t6 y; ne0, rows; nv vectors per lane; t_x type;
//              aux3 waves a row (1: four rows a workgroup; 4: one row)
//   unary/leaky/swiglu: t0 (t1) -> t6; n elements in `rows`; t_x type
//   rope:      t0 x, t1 pos, t6 y; ne0 head_dim, aux heads, aux2 ne2, rows tokens;
//              nv 1: four pairs a lane with vector loads, 0: one pair a lane
//   get_rows(+add)(+LN): t0 table, t1 ids, t2 table2, t3 ids2, t4 w, t5 b,
//              t6 dst (h), t7 y; t_x/t_x2 table types; aux/aux2 table rows
//   snake:     t0 x, t1 a, t2 ai, t6 y; act 1 = alpha along ne0; aux C,
//              aux2 cmask, aux3 ne0/4
//   group norm (split): gn; nv vectors per lane; aux 0 no activation, 2 Mish
//   layer norm + rope: t0 x, t1 pos, t2 w, t3 b, t6 y; ne0 row length,
//              aux head size, aux2 tokens (x.ne1), rows; nv vectors per lane;
//              table/ff/n_pos/rp the cache's
struct BOp {
    int32_t     kind;
    int32_t     act;
    int32_t     nv;
    int32_t     t_x, t_x2;
    float       eps, param;
    int64_t     ne0, rows, aux, aux2, aux3;
    union {
        BTen    t[8];
        GnSplit gn;
    };
    const void* table;       // rope cos/sin table or the GELU table
    const float* ff;         // rope freq factors (device) or nullptr
    int32_t     n_pos;
    RopeParams  rp;
};

static_assert(sizeof(GnSplit) <= sizeof(BTen) * 8, "the split GroupNorm's arguments share the tensor slots");
constexpr int kBatchMaxOps = CBX_MAX_OPS;

struct BatchArgs {
    int32_t   n;
    uint32_t  blk0[kBatchMaxOps];   // first workgroup of each op, contiguous for one scalar load batch
    uint32_t* err;
    BOp       op[kBatchMaxOps];
};
static_assert(sizeof(BatchArgs) <= 4096, "batch arguments must fit the kernel argument segment");

int launch_batch(const BatchArgs& a, uint32_t total_blocks, hipStream_t s);

// Row-norm kinds.
enum { NORM_LN = 0, NORM_RMS = 1 };
// Pseudo unary op used internally for leaky_relu.
enum { UNARY_LEAKY = 100 };

}  // namespace cbx
