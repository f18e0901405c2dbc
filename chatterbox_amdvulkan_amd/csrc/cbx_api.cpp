// cbx_api.cpp -- the C ABI: argument validation, error reporting, per-device
// state, and the host-built constant tables (fp16 GELU, RoPE cos/sin).
//
// Built with -ffp-contract=off like the kernels: the tables below are
// evaluated with one rounding per operation, as ggml-cpu's scalar code is.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "cbx_internal.h"

namespace cbx {

namespace {

thread_local std::string g_last_error;
constexpr int kMaxDevices = 64;
DeviceState g_dev[kMaxDevices];

}  // namespace

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return set_error(CBX_ERR_HIP, std::string(what) + ": kernel launch failed: " + hipGetErrorString(e));
    }
    return CBX_OK;
}

DeviceState* current_state(int* code) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *code = set_error(CBX_ERR_HIP, "hipGetDevice failed");
        return nullptr;
    }
    if (!g_dev[dev].ready) {
        *code = set_error(CBX_ERR_NOT_INITIALIZED, "cbx_init() has not been called for device " + std::to_string(dev));
        return nullptr;
    }
    *code = CBX_OK;
    return &g_dev[dev];
}

size_t type_size(int type) {
    switch (type) {
        case CBX_TYPE_F32: return 4;
        case CBX_TYPE_F16: return 2;
        case CBX_TYPE_Q8_0: return 34;
        case CBX_TYPE_I32: return 4;
        default: return 0;
    }
}

static int64_t row_elems_per_block(int type) { return type == CBX_TYPE_Q8_0 ? 32 : 1; }

int64_t nrows(const cbx_tensor* t) { return t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t nelements(const cbx_tensor* t) { return t->ne[0] * nrows(t); }

bool rows_contiguous(const cbx_tensor* t) { return t->nb[0] == type_size(t->type); }

bool is_contiguous(const cbx_tensor* t) {
    if (!rows_contiguous(t)) return false;
    size_t expect = type_size(t->type) * static_cast<size_t>(t->ne[0] / row_elems_per_block(t->type));
    for (int i = 1; i < 4; i++) {
        if (t->ne[i] > 1 && t->nb[i] != expect) return false;
        expect *= static_cast<size_t>(t->ne[i]);
    }
    return true;
}

bool same_shape(const cbx_tensor* a, const cbx_tensor* b) {
    for (int i = 0; i < 4; i++) if (a->ne[i] != b->ne[i]) return false;
    return true;
}

int validate(const cbx_tensor* t, const char* what, const char* name) {
    const std::string where = std::string(what) + ": " + name;
    if (!t) return set_error(CBX_ERR_INVALID_ARG, where + " is NULL");
    if (type_size(t->type) == 0) return set_error(CBX_ERR_INVALID_ARG, where + " has an unknown type " + std::to_string(t->type));
    if (t->reserved != 0) return set_error(CBX_ERR_INVALID_ARG, where + ".reserved must be 0");
    for (int i = 0; i < 4; i++) {
        if (t->ne[i] < 0) return set_error(CBX_ERR_INVALID_ARG, where + " has a negative ne[" + std::to_string(i) + "]");
    }
    if (t->type == CBX_TYPE_Q8_0 && t->ne[0] % 32 != 0) {
        return set_error(CBX_ERR_INVALID_ARG, where + ": Q8_0 ne[0] must be a multiple of 32");
    }
    if (nelements(t) == 0) return CBX_OK;   // nothing is read or written
    if (!rows_contiguous(t)) {
        return set_error(CBX_ERR_UNSUPPORTED, where + ": nb[0] must equal the element (block) size");
    }
    if (nelements(t) > 0 && t->data == nullptr) return set_error(CBX_ERR_INVALID_ARG, where + ".data is NULL");
    return CBX_OK;
}

// ---------------------------------------------------------------------------
// Host-built GELU table: entry h = f16(gelu(f32(h))) with
// gelu(x) = 0.5x(1 + tanhf(sqrt(2/pi) x (1 + 0.044715 x^2))), the table that
// ggml_cpu_init builds for ggml_gelu's f32 path (t3.cpp:537).
// ---------------------------------------------------------------------------
static void build_gelu_table(std::vector<uint16_t>& tab) {
    const float coef_a = 0.044715f;
    const float sqrt_2_over_pi = 0.79788456080286535587989211986876f;
    tab.resize(65536);
    for (uint32_t h = 0; h < 65536; h++) {
        const float x = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h)));
        const float inner = 1.0f + coef_a * x * x;
        const float g = 0.5f * x * (1.0f + tanhf(sqrt_2_over_pi * x * inner));
        tab[h] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(g));
    }
}

// ---------------------------------------------------------------------------
// RoPE: ggml's YaRN helpers, restated for the host-side table.
// ---------------------------------------------------------------------------
static float yarn_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * static_cast<float>(M_PI))) / (2 * logf(base));
}

static void yarn_corr_dims(int n_dims, int n_ctx_orig, float freq_base, float beta_fast,
                           float beta_slow, float dims[2]) {
    const float start = floorf(yarn_corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base));
    const float end = ceilf(yarn_corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base));
    dims[0] = start > 0.0f ? start : 0.0f;
    dims[1] = end < static_cast<float>(n_dims - 1) ? end : static_cast<float>(n_dims - 1);
}

static void yarn_cos_sin(float theta_extrap, int64_t i0, const RopeParams& p, float* c, float* s) {
    const float theta_interp = p.freq_scale * theta_extrap;
    float theta = theta_interp;
    float mscale = p.attn_factor;
    if (p.ext_factor != 0.0f) {
        const float d = p.corr_dims[1] - p.corr_dims[0];
        const float y = (static_cast<float>(i0 / 2) - p.corr_dims[0]) / (d > 0.001f ? d : 0.001f);
        const float cl = y < 0.0f ? 0.0f : y;
        const float ramp_mix = (1.0f - (cl < 1.0f ? cl : 1.0f)) * p.ext_factor;
        theta = theta_interp * (1 - ramp_mix) + theta_extrap * ramp_mix;
        mscale *= 1.0f + 0.1f * logf(1.0f / p.freq_scale);
    }
    *c = cosf(theta) * mscale;
    *s = sinf(theta) * mscale;
}

bool bytes_overlap(const cbx_tensor* a, const cbx_tensor* b) {
    auto span = [](const cbx_tensor* t) {
        size_t hi = type_size(t->type);
        for (int i = 0; i < 4; i++) hi += static_cast<size_t>(t->ne[i] > 0 ? t->ne[i] - 1 : 0) * t->nb[i];
        return hi;
    };
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(a->data), b0 = reinterpret_cast<uintptr_t>(b->data);
    return a0 < b0 + span(b) && b0 < a0 + span(a);
}

}  // namespace cbx

struct cbx_conv1d_weights {
    uint64_t  serial;   // distinct for every handle this process creates
    int       device;
    int       up;       // 0: conv1d weights; >= 1: transposed conv with this stride
    int64_t   k;        // the weight's taps
    int64_t   taps;     // taps per phase as stored (k for conv1d)
    int64_t   c_in, c_out, c_in_pad, c_out_pad;
    int64_t   w_ph;     // halves per phase
    _Float16* data;     // [phase][c_out_pad / 32][taps][c_in_pad / 16][64][8]
};

bool cbx::conv1d_weights_match(const cbx_conv1d_weights* w, int up, int64_t k, int64_t c_in, int64_t c_out) {
    return w && w->up == up && w->k == k && w->c_in == c_in && w->c_out == c_out;
}

struct cbx_rope_cache {
    uint64_t         serial;       // distinct for every handle this process creates
    int              device;
    cbx::RopeParams  p;
    int32_t          n_pos;
    float2*          table;        // [n_pos][n_dims/2] (cos, sin)
    float*           freq_factors; // device copy or nullptr
};

// Serial numbers of the handles: a graph exec compares them to tell a
// handle from a new one at the same address.
static std::atomic<uint64_t> g_handle_serial{1};

uint64_t cbx::rope_cache_serial(const cbx_rope_cache* c) { return c ? c->serial : 0; }
uint64_t cbx::conv1d_weights_serial(const cbx_conv1d_weights* w) { return w ? w->serial : 0; }

using namespace cbx;

extern "C" {

const char* cbx_last_error(void) { return g_last_error.c_str(); }

const char* cbx_version(void) { return "cbxops 0.1.0 (gfx950)"; }

int cbx_init(int device) {
    clear_error();
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        return set_error(CBX_ERR_HIP, "cbx_init: no HIP device");
    }
    if (device < 0 || device >= count || device >= kMaxDevices) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_init: device " + std::to_string(device) + " out of range");
    }
    DeviceState& st = g_dev[device];
    if (st.ready) return CBX_OK;
    int prev = 0;
    hipGetDevice(&prev);
    if (hipSetDevice(device) != hipSuccess) return set_error(CBX_ERR_HIP, "cbx_init: hipSetDevice failed");
    int rc = CBX_OK;
    std::vector<uint16_t> tab;
    build_gelu_table(tab);
    if (hipDeviceGetAttribute(&st.n_cu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
        st.n_cu <= 0) {
        st.n_cu = 256;
    }
    if (hipMalloc(reinterpret_cast<void**>(&st.gelu_table), 65536 * sizeof(uint16_t)) != hipSuccess ||
        hipMalloc(reinterpret_cast<void**>(&st.err_word), sizeof(uint32_t)) != hipSuccess) {
        rc = set_error(CBX_ERR_HIP, "cbx_init: hipMalloc failed");
    } else if (hipMemcpy(st.gelu_table, tab.data(), 65536 * sizeof(uint16_t), hipMemcpyHostToDevice) != hipSuccess ||
               hipMemset(st.err_word, 0, sizeof(uint32_t)) != hipSuccess ||
               hipDeviceSynchronize() != hipSuccess) {
        rc = set_error(CBX_ERR_HIP, "cbx_init: upload failed");
    }
    if (rc == CBX_OK) rc = group_norm_scratch_setup(&st.gn_scratch);
    if (rc == CBX_OK) rc = group_norm_probe_xcd(&st.gn_split_ok);
    if (rc != CBX_OK) {
        if (st.gelu_table) hipFree(st.gelu_table);
        if (st.err_word) hipFree(st.err_word);
        st = DeviceState();
    } else {
        st.ready = true;
    }
    hipSetDevice(prev);
    return rc;
}

void cbx_shutdown(void) {
    int prev = 0;
    hipGetDevice(&prev);
    for (int d = 0; d < kMaxDevices; d++) {
        DeviceState& st = g_dev[d];
        if (!st.ready) continue;
        hipSetDevice(d);
        hipDeviceSynchronize();
        hipFree(st.gelu_table);
        hipFree(st.err_word);
        st = DeviceState();
    }
    hipSetDevice(prev);
}

int cbx_device_errors(int device, uint32_t* flags_out, int clear) {
    clear_error();
    if (device < 0 || device >= kMaxDevices || !g_dev[device].ready) {
        return set_error(CBX_ERR_NOT_INITIALIZED, "cbx_device_errors: device not initialised");
    }
    if (!flags_out) return set_error(CBX_ERR_INVALID_ARG, "cbx_device_errors: flags_out is NULL");
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(device);
    int rc = CBX_OK;
    uint32_t v = 0;
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(&v, g_dev[device].err_word, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) {
        rc = set_error(CBX_ERR_HIP, "cbx_device_errors: read failed");
    } else if (clear && (hipMemset(g_dev[device].err_word, 0, sizeof(uint32_t)) != hipSuccess ||
                         hipDeviceSynchronize() != hipSuccess)) {
        rc = set_error(CBX_ERR_HIP, "cbx_device_errors: clear failed");
    }
    *flags_out = v;
    hipSetDevice(prev);
    return rc;
}

// ---- gather / conversion ---------------------------------------------------

static int check_gather(const char* what, const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* dst) {
    int rc;
    if ((rc = validate(src, what, "src")) || (rc = validate(ids, what, "ids")) || (rc = validate(dst, what, "dst"))) return rc;
    if (src->type != CBX_TYPE_F32 && src->type != CBX_TYPE_F16 && src->type != CBX_TYPE_Q8_0) {
        return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": src must be F32, F16 or Q8_0");
    }
    if (ids->type != CBX_TYPE_I32) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": ids must be I32");
    if (dst->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": dst must be F32");
    if (ids->ne[3] != 1) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": ids must have ne[3] == 1");
    if (dst->ne[0] != src->ne[0] || dst->ne[1] != ids->ne[0] || dst->ne[2] != ids->ne[1] || dst->ne[3] != ids->ne[2]) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": dst shape must be (src.ne0, ids.ne0, ids.ne1, ids.ne2)");
    }
    if (src->ne[2] != ids->ne[1] || src->ne[3] != ids->ne[2]) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": src.ne2/ne3 must equal ids.ne1/ne2");
    }
    // every id would be out of range (ggml aborts); the kernels read row 0
    // in place of a bad id, so a table without rows is refused here
    if (src->ne[1] == 0 && nelements(dst) > 0) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": src has no rows to gather from");
    }
    return CBX_OK;
}

int cbx_get_rows(const cbx_tensor* src, const cbx_tensor* ids, cbx_tensor* dst, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_gather("cbx_get_rows", src, ids, dst))) return rc;
    if (nelements(dst) == 0) return CBX_OK;
    return launch_get_rows(src, ids, nullptr, nullptr, dst, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_get_rows_add(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* src2,
                     const cbx_tensor* ids2, cbx_tensor* dst, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_gather("cbx_get_rows_add", src, ids, dst)) || (rc = check_gather("cbx_get_rows_add", src2, ids2, dst))) return rc;
    if (nelements(dst) == 0) return CBX_OK;
    return launch_get_rows(src, ids, src2, ids2, dst, st, reinterpret_cast<hipStream_t>(stream));
}

static int check_row_param(const cbx_tensor* p, const cbx_tensor* x, const char* what, const char* name);
static bool overlaps(const cbx_tensor* a, const cbx_tensor* b);

int cbx_get_rows_add_layer_norm(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* src2,
                                const cbx_tensor* ids2, const cbx_tensor* w, const cbx_tensor* b, float eps,
                                cbx_tensor* h, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_get_rows_add_layer_norm";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_gather(what, src, ids, y)) || (rc = check_gather(what, src2, ids2, y))) return rc;
    if (h) {
        if ((rc = validate(h, what, "h"))) return rc;
        if (h->type != CBX_TYPE_F32 || !same_shape(h, y)) {
            return set_error(CBX_ERR_INVALID_ARG, "cbx_get_rows_add_layer_norm: h must be F32 with y's shape");
        }
    }
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, "cbx_get_rows_add_layer_norm: eps must be >= 0");
    if ((rc = check_row_param(w, y, what, "w")) || (rc = check_row_param(b, y, what, "b"))) return rc;
    if (nelements(y) == 0) return CBX_OK;
    return launch_embed_norm(src, ids, src2, ids2, w, b, eps, h, y, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_get_rows_concat_add_layer_norm(const cbx_tensor* prefix, const cbx_tensor* src_a, const cbx_tensor* ids_a,
                                       const cbx_tensor* src_b, const cbx_tensor* ids_b, const cbx_tensor* src2,
                                       const cbx_tensor* ids2, const cbx_tensor* w, const cbx_tensor* b, float eps,
                                       cbx_tensor* h, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_get_rows_concat_add_layer_norm";
    const std::string f(what);
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(y, what, "y"))) return rc;
    if (y->type != CBX_TYPE_F32 || y->ne[2] != 1 || y->ne[3] != 1) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": y must be F32 (D, N, 1, 1)");
    }
    const int64_t D = y->ne[0];
    // a gathered segment: a 2-D table of D-wide rows and 1-D contiguous I32 ids
    auto seg = [&](const cbx_tensor* src, const cbx_tensor* ids, const char* ns, const char* ni) -> int {
        int r;
        if ((r = validate(src, what, ns)) || (r = validate(ids, what, ni))) return r;
        if (src->type != CBX_TYPE_F32 && src->type != CBX_TYPE_F16 && src->type != CBX_TYPE_Q8_0) {
            return set_error(CBX_ERR_UNSUPPORTED, f + ": tables must be F32, F16 or Q8_0");
        }
        if (src->ne[0] != D || src->ne[2] != 1 || src->ne[3] != 1 || src->ne[1] == 0 || src->ne[1] >= (int64_t{1} << 31)) {
            return set_error(CBX_ERR_INVALID_ARG, f + ": tables must be 2-D with ne0 = y.ne0 and 1..2^31-1 rows");
        }
        if (ids->type != CBX_TYPE_I32 || ids->ne[1] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1 ||
            (ids->ne[0] > 1 && ids->nb[0] != sizeof(int32_t))) {
            return set_error(CBX_ERR_INVALID_ARG, f + ": ids must be contiguous 1-D I32");
        }
        return CBX_OK;
    };
    if (!src_b || !ids_b || !src2 || !ids2) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": src_b, ids_b, src2 and ids2 are required");
    }
    if ((src_a == nullptr) != (ids_a == nullptr)) return set_error(CBX_ERR_INVALID_ARG, f + ": src_a and ids_a go together");
    if ((rc = seg(src_b, ids_b, "src_b", "ids_b")) || (rc = seg(src2, ids2, "src2", "ids2"))) return rc;
    if (src_a && (rc = seg(src_a, ids_a, "src_a", "ids_a"))) return rc;
    int64_t n_pre = 0;
    if (prefix) {
        if ((rc = validate(prefix, what, "prefix"))) return rc;
        if (prefix->type != CBX_TYPE_F32 || prefix->ne[0] != D || prefix->ne[2] != 1 || prefix->ne[3] != 1) {
            return set_error(CBX_ERR_INVALID_ARG, f + ": prefix must be F32 (y.ne0, n_prefix, 1, 1)");
        }
        n_pre = prefix->ne[1];
    }
    const int64_t n_tok = n_pre + (ids_a ? ids_a->ne[0] : 0) + ids_b->ne[0];
    if (y->ne[1] != n_tok || ids2->ne[0] != n_tok) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": y.ne1 and ids2 must count the prefix rows plus both ids");
    }
    if (n_tok >= (int64_t{1} << 31)) return set_error(CBX_ERR_UNSUPPORTED, f + ": too many rows");
    if (h) {
        if ((rc = validate(h, what, "h"))) return rc;
        if (h->type != CBX_TYPE_F32 || !same_shape(h, y)) return set_error(CBX_ERR_INVALID_ARG, f + ": h must be F32 with y's shape");
    }
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, f + ": eps must be >= 0");
    if ((rc = check_row_param(w, y, what, "w")) || (rc = check_row_param(b, y, what, "b"))) return rc;
    if (n_tok == 0 || D == 0) return CBX_OK;
    // outputs written by other workgroups must not alias what rows are read from
    for (const cbx_tensor* in : {prefix, src_a, ids_a, src_b, ids_b, src2, ids2, w, b}) {
        if (in && (overlaps(in, y) || (h && overlaps(in, h)))) {
            return set_error(CBX_ERR_INVALID_ARG, f + ": h and y must not overlap the inputs");
        }
    }
    if (h && overlaps(h, y)) return set_error(CBX_ERR_INVALID_ARG, f + ": h and y overlap");
    return launch_embed_concat_norm(prefix, src_a, ids_a, src_b, ids_b, src2, ids2, w, b, eps, h, y, st,
                                    reinterpret_cast<hipStream_t>(stream));
}

int cbx_cpy(const cbx_tensor* src, cbx_tensor* dst, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(src, "cbx_cpy", "src")) || (rc = validate(dst, "cbx_cpy", "dst"))) return rc;
    if ((src->type != CBX_TYPE_F32 && src->type != CBX_TYPE_F16) || (dst->type != CBX_TYPE_F32 && dst->type != CBX_TYPE_F16)) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_cpy: F32/F16 only");
    }
    if (!same_shape(src, dst)) return set_error(CBX_ERR_INVALID_ARG, "cbx_cpy: shapes differ");
    if (nelements(dst) == 0) return CBX_OK;
    return launch_cpy(src, dst, st, reinterpret_cast<hipStream_t>(stream));
}

// ---- norms -------------------------------------------------------------------

static int check_float(const cbx_tensor* t, const char* what, const char* name) {
    int rc = validate(t, what, name);
    if (rc) return rc;
    if (t->type != CBX_TYPE_F32 && t->type != CBX_TYPE_F16) {
        return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": " + name + " must be F32 or F16");
    }
    return CBX_OK;
}

static int check_act(int act, const char* what) {
    if (act < CBX_UNARY_NONE || act > CBX_UNARY_MISH) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": unknown activation " + std::to_string(act));
    }
    return CBX_OK;
}

// affine vector: F32, ne == (ne0, 1, 1, 1), contiguous
static int check_row_param(const cbx_tensor* p, const cbx_tensor* x, const char* what, const char* name) {
    if (!p) return CBX_OK;
    int rc = validate(p, what, name);
    if (rc) return rc;
    if (p->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": " + name + " must be F32");
    if (p->ne[0] != x->ne[0] || p->ne[1] != 1 || p->ne[2] != 1 || p->ne[3] != 1) {
        return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": " + name + " must have ne = (x.ne0, 1, 1, 1)");
    }
    return CBX_OK;
}

static int row_norm_entry(const char* what, int kind, const cbx_tensor* x, const cbx_tensor* w,
                          const cbx_tensor* b, float eps, int act, cbx_tensor* y, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_float(x, what, "x")) || (rc = check_float(y, what, "y"))) return rc;
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": x and y shapes differ");
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": eps must be >= 0");
    if ((rc = check_row_param(w, x, what, "w")) || (rc = check_row_param(b, x, what, "b")) || (rc = check_act(act, what))) return rc;
    if (nelements(x) == 0) return CBX_OK;
    return launch_row_norm(kind, x, w, b, eps, act, y, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_norm(const cbx_tensor* x, float eps, cbx_tensor* y, cbx_stream stream) {
    return row_norm_entry("cbx_norm", NORM_LN, x, nullptr, nullptr, eps, CBX_UNARY_NONE, y, stream);
}

int cbx_layer_norm(const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int act,
                   cbx_tensor* y, cbx_stream stream) {
    return row_norm_entry("cbx_layer_norm", NORM_LN, x, w, b, eps, act, y, stream);
}

int cbx_rms_norm(const cbx_tensor* x, float eps, cbx_tensor* y, cbx_stream stream) {
    return row_norm_entry("cbx_rms_norm", NORM_RMS, x, nullptr, nullptr, eps, CBX_UNARY_NONE, y, stream);
}

int cbx_rms_norm_mul(const cbx_tensor* x, const cbx_tensor* g, float eps, cbx_tensor* y, cbx_stream stream) {
    return row_norm_entry("cbx_rms_norm_mul", NORM_RMS, x, g, nullptr, eps, CBX_UNARY_NONE, y, stream);
}

// F32 operand of a fused LayerNorm with x's shape.
static int check_f32_like(const cbx_tensor* t, const cbx_tensor* x, const char* what, const char* name) {
    int rc = validate(t, what, name);
    if (rc) return rc;
    if (t->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": " + name + " must be F32");
    if (!same_shape(t, x)) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": " + name + " must have x's shape");
    return CBX_OK;
}

// Byte ranges of two tensors' rows overlap.
static bool overlaps(const cbx_tensor* a, const cbx_tensor* b) { return bytes_overlap(a, b); }

int cbx_add_layer_norm(const cbx_tensor* a, const cbx_tensor* a_bias, const cbx_tensor* r, const cbx_tensor* w,
                       const cbx_tensor* b, float eps, int act, cbx_tensor* s, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_add_layer_norm";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(a, what, "a"))) return rc;
    if (a->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, "cbx_add_layer_norm: a must be F32");
    if (!r && !a_bias) return set_error(CBX_ERR_INVALID_ARG, "cbx_add_layer_norm: r may be NULL only with a_bias");
    if ((r && (rc = check_f32_like(r, a, what, "r"))) || (rc = check_f32_like(y, a, what, "y")) ||
        (s && (rc = check_f32_like(s, a, what, "s")))) return rc;
    if ((rc = check_row_param(a_bias, a, what, "a_bias")) || (rc = check_row_param(w, a, what, "w")) ||
        (rc = check_row_param(b, a, what, "b")) || (rc = check_act(act, what))) return rc;
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, "cbx_add_layer_norm: eps must be >= 0");
    if (nelements(a) == 0) return CBX_OK;
    if (s && overlaps(s, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_add_layer_norm: s and y overlap");
    return launch_layer_norm_ext(a, a_bias, r, w, b, nullptr, eps, act, s, y, st, reinterpret_cast<hipStream_t>(stream),
                                 what);
}

int cbx_layer_norm_mask(const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int act,
                        const cbx_tensor* mask, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_layer_norm_mask";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x"))) return rc;
    if (x->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, "cbx_layer_norm_mask: x must be F32");
    if ((rc = check_f32_like(y, x, what, "y"))) return rc;
    if ((rc = check_row_param(w, x, what, "w")) || (rc = check_row_param(b, x, what, "b")) ||
        (rc = check_act(act, what)) || (rc = validate(mask, what, "mask"))) return rc;
    if (mask->type != CBX_TYPE_F32 || mask->ne[0] != 1 || mask->ne[1] != x->ne[1] || mask->ne[2] != 1 ||
        mask->ne[3] != 1 || (mask->ne[1] > 1 && mask->nb[1] != sizeof(float))) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_layer_norm_mask: mask must be contiguous F32 with ne = (1, x.ne1, 1, 1)");
    }
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_mask: eps must be >= 0");
    if (nelements(x) == 0) return CBX_OK;
    return launch_layer_norm_ext(x, nullptr, nullptr, w, b, mask, eps, act, nullptr, y, st,
                                 reinterpret_cast<hipStream_t>(stream), what);
}

static int check_group_norm(const char* what, const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w,
                            const cbx_tensor* b, int act, const cbx_tensor* y) {
    const std::string f(what);
    int rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y"))) return rc;
    if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, f + ": F32 only");
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, f + ": x and y shapes differ");
    if (n_groups <= 0) return set_error(CBX_ERR_INVALID_ARG, f + ": n_groups must be > 0");
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, f + ": eps must be >= 0");
    if ((rc = check_act(act, what))) return rc;
    for (const cbx_tensor* p : {w, b}) {
        if (!p) continue;
        if ((rc = validate(p, what, p == w ? "w" : "b"))) return rc;
        if (p->type != CBX_TYPE_F32 || p->ne[0] != 1 || p->ne[1] != 1 || p->ne[2] != x->ne[2] || p->ne[3] != 1 ||
            (p->ne[2] > 1 && p->nb[2] != sizeof(float))) {
            return set_error(CBX_ERR_UNSUPPORTED, f + ": w/b must be contiguous F32 with ne = (1, 1, x.ne2, 1)");
        }
    }
    // in place means y is x (same memory and strides); any other overlap of
    // y with x, w or b would have other workgroups' stores race with reads
    if (nelements(x) > 0 && overlaps(x, y)) {
        bool same = x->data == y->data;
        for (int i = 0; i < 4; i++) same = same && x->nb[i] == y->nb[i];
        if (!same) return set_error(CBX_ERR_INVALID_ARG, f + ": y must be x itself or not overlap it");
    }
    if ((w && overlaps(w, y)) || (b && overlaps(b, y))) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": w and b must not overlap y");
    }
    return CBX_OK;
}

int cbx_group_norm(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                   int act, cbx_tensor* y, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_group_norm("cbx_group_norm", x, n_groups, eps, w, b, act, y))) return rc;
    if (nelements(x) == 0) return CBX_OK;
    // a few large groups out of place: the split reduction over the
    // library's scratch set for this stream (the split itself sends in-place
    // calls and the layouts it does not cover to launch_group_norm)
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (int64_t{n_groups} * x->ne[3] <= static_cast<int64_t>(group_norm_scratch_slots())) {
        return launch_group_norm_split(x, n_groups, eps, w, b, act, y, group_norm_scratch_for(st, s), kGnWaitAuto, 0,
                                       st, s);
    }
    return launch_group_norm(x, n_groups, eps, w, b, act, y, st, s);
}

struct cbx_group_norm_workspace {
    int      device;
    void*    mem;          // the partials' tagged exchange words, zeroed once
    uint64_t wait_ticks;   // 100 MHz real-time counter ticks; kGnWaitAuto: from the launch's size
    int32_t  n_chunks;     // 0: automatic
};

int cbx_group_norm_workspace_create(cbx_group_norm_workspace** out) {
    clear_error();
    if (!out) return set_error(CBX_ERR_INVALID_ARG, "cbx_group_norm_workspace_create: out is NULL");
    *out = nullptr;
    int rc;
    if (!current_state(&rc)) return rc;
    auto* ws = new (std::nothrow) cbx_group_norm_workspace();
    if (!ws) return set_error(CBX_ERR_HIP, "cbx_group_norm_workspace_create: out of host memory");
    hipGetDevice(&ws->device);
    ws->wait_ticks = kGnWaitAuto;
    ws->n_chunks = 0;
    const size_t bytes = group_norm_workspace_bytes();
    if (hipMalloc(&ws->mem, bytes) != hipSuccess) {
        delete ws;
        return set_error(CBX_ERR_HIP, "cbx_group_norm_workspace_create: hipMalloc failed");
    }
    if (hipMemset(ws->mem, 0, bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        hipFree(ws->mem);
        delete ws;
        return set_error(CBX_ERR_HIP, "cbx_group_norm_workspace_create: clearing failed");
    }
    *out = ws;
    return CBX_OK;
}

void cbx_group_norm_workspace_destroy(cbx_group_norm_workspace* ws) {
    if (!ws) return;
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(ws->device);
    hipDeviceSynchronize();
    hipFree(ws->mem);
    hipSetDevice(prev);
    delete ws;
}

int cbx_group_norm_workspace_tune(cbx_group_norm_workspace* ws, uint32_t max_wait_us, int32_t n_chunks) {
    clear_error();
    if (!ws) return set_error(CBX_ERR_INVALID_ARG, "cbx_group_norm_workspace_tune: ws is NULL");
    if (n_chunks < 0 || n_chunks > 32) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_group_norm_workspace_tune: n_chunks must be 0 (automatic) .. 32");
    }
    ws->wait_ticks = max_wait_us == CBX_GN_WAIT_AUTO ? kGnWaitAuto : static_cast<uint64_t>(max_wait_us) * 100;
    ws->n_chunks = n_chunks;
    return CBX_OK;
}

int cbx_group_norm_split_enabled(int device) {
    clear_error();
    if (device < 0 || device >= kMaxDevices) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_group_norm_split_enabled: device out of range");
    }
    const DeviceState& st = g_dev[device];
    if (!st.ready) {
        return set_error(CBX_ERR_NOT_INITIALIZED,
                         "cbx_init() has not been called for device " + std::to_string(device));
    }
    return st.gn_split_ok ? 1 : 0;
}

int cbx_group_norm_ws(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                      int act, cbx_tensor* y, cbx_group_norm_workspace* ws, cbx_stream stream) {
    const char* what = "cbx_group_norm_ws";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!ws) return set_error(CBX_ERR_INVALID_ARG, "cbx_group_norm_ws: ws is NULL");
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != ws->device) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_group_norm_ws: the workspace belongs to another device");
    }
    if ((rc = check_group_norm(what, x, n_groups, eps, w, b, act, y))) return rc;
    if (nelements(x) == 0) return CBX_OK;
    return launch_group_norm_split(x, n_groups, eps, w, b, act, y, ws->mem, ws->wait_ticks, ws->n_chunks, st,
                                   reinterpret_cast<hipStream_t>(stream));
}

int cbx_group_norm_noalloc(const cbx_tensor* x, int n_groups, float eps, const cbx_tensor* w, const cbx_tensor* b,
                           int act, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_group_norm_noalloc";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_group_norm(what, x, n_groups, eps, w, b, act, y))) return rc;
    const int64_t n_gi = int64_t{n_groups} * x->ne[3];
    if (n_gi > static_cast<int64_t>(group_norm_scratch_slots())) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_group_norm_noalloc: n_groups x ne[3] = " + std::to_string(n_gi) +
                                                  " exceeds the " + std::to_string(group_norm_scratch_slots()) +
                                                  " group instances of the library's static scratch");
    }
    if (nelements(x) == 0) return CBX_OK;
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    return launch_group_norm_split(x, n_groups, eps, w, b, act, y, group_norm_scratch_for(st, s), kGnWaitAuto, 0, st,
                                   s);
}

// ---- rope --------------------------------------------------------------------

int cbx_rope_cache_create(int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
                          float ext_factor, float attn_factor, float beta_fast, float beta_slow,
                          const float* freq_factors, int32_t n_pos, cbx_rope_cache** out) {
    clear_error();
    if (!out) return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_cache_create: out is NULL");
    *out = nullptr;
    if (n_dims <= 0 || n_dims % 2 != 0) return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_cache_create: n_dims must be even and > 0");
    if (mode != 0 && mode != 2) return set_error(CBX_ERR_UNSUPPORTED, "cbx_rope_cache_create: mode must be 0 (NORMAL) or 2 (NEOX)");
    if (n_pos < 0 || static_cast<int64_t>(n_pos) * (n_dims / 2) > (int64_t{1} << 28)) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_cache_create: n_pos out of range");
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(CBX_ERR_HIP, "cbx_rope_cache_create: hipGetDevice failed");
    RopeParams p{};
    p.n_dims = n_dims;
    p.mode = mode;
    p.n_ctx_orig = n_ctx_orig;
    p.freq_base = freq_base;
    p.freq_scale = freq_scale;
    p.ext_factor = ext_factor;
    p.attn_factor = attn_factor;
    p.beta_fast = beta_fast;
    p.beta_slow = beta_slow;
    p.theta_scale = powf(freq_base, -2.0f / n_dims);
    yarn_corr_dims(n_dims, n_ctx_orig, freq_base, beta_fast, beta_slow, p.corr_dims);

    const int half = n_dims / 2;
    std::vector<float2> tab(static_cast<size_t>(n_pos) * half);
    for (int32_t pos = 0; pos < n_pos; pos++) {
        // theta_i = pos * theta_scale^i as ggml_rope_cache_init forms it
        float theta = static_cast<float>(pos);
        for (int i = 0; i < half; i++) {
            const float ff = freq_factors ? freq_factors[i] : 1.0f;
            float c, s;
            yarn_cos_sin(theta / ff, 2 * i, p, &c, &s);
            tab[static_cast<size_t>(pos) * half + i] = make_float2(c, s);
            theta *= p.theta_scale;
        }
    }
    auto* cache = new cbx_rope_cache();
    cache->serial = g_handle_serial.fetch_add(1);
    cache->device = dev;
    cache->p = p;
    cache->n_pos = n_pos;
    cache->table = nullptr;
    cache->freq_factors = nullptr;
    bool ok = true;
    if (n_pos > 0) {
        ok = hipMalloc(reinterpret_cast<void**>(&cache->table), tab.size() * sizeof(float2)) == hipSuccess &&
             hipMemcpy(cache->table, tab.data(), tab.size() * sizeof(float2), hipMemcpyHostToDevice) == hipSuccess;
    }
    if (ok && freq_factors) {
        ok = hipMalloc(reinterpret_cast<void**>(&cache->freq_factors), half * sizeof(float)) == hipSuccess &&
             hipMemcpy(cache->freq_factors, freq_factors, half * sizeof(float), hipMemcpyHostToDevice) == hipSuccess;
    }
    if (!ok) {
        cbx_rope_cache_destroy(cache);
        return set_error(CBX_ERR_HIP, "cbx_rope_cache_create: device allocation/upload failed");
    }
    *out = cache;
    return CBX_OK;
}

void cbx_rope_cache_destroy(cbx_rope_cache* cache) {
    if (!cache) return;
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(cache->device);
    hipDeviceSynchronize();
    if (cache->table) hipFree(cache->table);
    if (cache->freq_factors) hipFree(cache->freq_factors);
    hipSetDevice(prev);
    delete cache;
}

int cbx_rope_ext(const cbx_tensor* x, const cbx_tensor* pos, const cbx_rope_cache* cache, cbx_tensor* y,
                 cbx_stream stream) {
    const char* what = "cbx_rope_ext";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!cache) return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_ext: cache is NULL");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev != cache->device) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_ext: cache belongs to another device");
    }
    if ((rc = check_float(x, what, "x")) || (rc = check_float(y, what, "y")) || (rc = validate(pos, what, "pos"))) return rc;
    if (x->type != y->type) return set_error(CBX_ERR_UNSUPPORTED, "cbx_rope_ext: x and y types differ");
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_ext: x and y shapes differ");
    if (pos->type != CBX_TYPE_I32 || pos->ne[0] != x->ne[2] || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_ext: pos must be I32 with ne = (x.ne2, 1, 1, 1)");
    }
    if (cache->p.n_dims > x->ne[0]) return set_error(CBX_ERR_INVALID_ARG, "cbx_rope_ext: n_dims > x.ne0");
    if (nelements(x) == 0) return CBX_OK;
    return launch_rope(x, pos, cache->p, cache->table, cache->n_pos, cache->freq_factors, y, st,
                       reinterpret_cast<hipStream_t>(stream));
}

int cbx_layer_norm_rope(const cbx_tensor* x, const cbx_tensor* w, const cbx_tensor* b, float eps, int64_t head_dim,
                        const cbx_tensor* pos, const cbx_rope_cache* cache, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_layer_norm_rope";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!cache) return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: cache is NULL");
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev != cache->device) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: cache belongs to another device");
    }
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y")) || (rc = validate(pos, what, "pos"))) return rc;
    if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, "cbx_layer_norm_rope: F32 only");
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: x and y shapes differ");
    if (!(eps >= 0.0f)) return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: eps must be >= 0");
    if ((rc = check_row_param(w, x, what, "w")) || (rc = check_row_param(b, x, what, "b"))) return rc;
    if (head_dim <= 0 || head_dim % 4 || x->ne[0] % head_dim) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: head_dim must divide x.ne0 and be a multiple of 4");
    }
    if (cache->p.n_dims > head_dim) return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: n_dims > head_dim");
    if (x->ne[3] != 1) return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: x must be at most 3-D (C, n_tok, batch)");
    if (pos->type != CBX_TYPE_I32 || pos->ne[0] != x->ne[1] || pos->ne[1] != 1 || pos->ne[2] != 1 || pos->ne[3] != 1) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_layer_norm_rope: pos must be I32 with ne = (x.ne1, 1, 1, 1)");
    }
    if (x->ne[0] > 1024 || cache->p.n_dims / 2 > 256 || reinterpret_cast<uintptr_t>(x->data) % 16 ||
        reinterpret_cast<uintptr_t>(y->data) % 16 || (w && reinterpret_cast<uintptr_t>(w->data) % 16) ||
        (b && reinterpret_cast<uintptr_t>(b->data) % 16)) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_layer_norm_rope: rows of at most 1024 elements, 16-byte aligned");
    }
    for (const cbx_tensor* t : {x, static_cast<const cbx_tensor*>(y)}) {
        for (int k = 1; k < 4; k++) {
            if (t->ne[k] > 1 && t->nb[k] % 16) {
                return set_error(CBX_ERR_UNSUPPORTED, "cbx_layer_norm_rope: row strides must be multiples of 16 bytes");
            }
        }
    }
    if (nelements(x) == 0) return CBX_OK;
    return launch_layer_norm_rope(x, w, b, eps, head_dim, pos, cache->p, cache->table, cache->n_pos,
                                  cache->freq_factors, y, st, reinterpret_cast<hipStream_t>(stream));
}

// ---- attention-score epilogue ---------------------------------------------------

int cbx_scale_diag_mask_soft_max(const cbx_tensor* x, float scale, int32_t n_past, cbx_tensor* y,
                                 cbx_stream stream) {
    const char* what = "cbx_scale_diag_mask_soft_max";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y"))) return rc;
    if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_scale_diag_mask_soft_max: F32 only");
    }
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_scale_diag_mask_soft_max: x and y shapes differ");
    if (nelements(x) == 0) return CBX_OK;
    return launch_soft_max(x, nullptr, scale, n_past, y, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_add_scale_diag_mask_soft_max(const cbx_tensor* a, const cbx_tensor* b, float scale, int32_t n_past,
                                     cbx_tensor* y, cbx_stream stream) {
    const std::string f = "cbx_add_scale_diag_mask_soft_max";
    const char* what = f.c_str();
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(a, what, "a")) || (rc = validate(b, what, "b")) || (rc = validate(y, what, "y"))) return rc;
    if (a->type != CBX_TYPE_F32 || b->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) {
        return set_error(CBX_ERR_UNSUPPORTED, f + ": F32 only");
    }
    if (!same_shape(a, b) || !same_shape(a, y)) return set_error(CBX_ERR_INVALID_ARG, f + ": a, b and y shapes differ");
    if (nelements(a) == 0) return CBX_OK;
    // each row is read whole before it is stored: y may be a or b itself,
    // any other overlap would race with other rows' reads
    for (const cbx_tensor* p : {a, b}) {
        if (!overlaps(p, y)) continue;
        bool same = p->data == y->data;
        for (int i = 0; i < 4; i++) same = same && p->nb[i] == y->nb[i];
        if (!same) return set_error(CBX_ERR_INVALID_ARG, f + ": y must be a or b itself or overlap neither");
    }
    return launch_soft_max(a, b, scale, n_past, y, st, reinterpret_cast<hipStream_t>(stream));
}

// ---- activations -------------------------------------------------------------

static int unary_entry(const char* what, int op, float param, const cbx_tensor* x, cbx_tensor* y,
                       cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_float(x, what, "x")) || (rc = check_float(y, what, "y"))) return rc;
    if (x->type != y->type) return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": x and y types differ");
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": x and y shapes differ");
    if (nelements(x) == 0) return CBX_OK;
    return launch_unary(op, param, x, y, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_unary(int op, const cbx_tensor* x, cbx_tensor* y, cbx_stream stream) {
    if (op < CBX_UNARY_GELU || op > CBX_UNARY_MISH) {
        clear_error();
        return set_error(CBX_ERR_INVALID_ARG, "cbx_unary: unknown op " + std::to_string(op));
    }
    return unary_entry("cbx_unary", op, 0.0f, x, y, stream);
}
int cbx_gelu(const cbx_tensor* x, cbx_tensor* y, cbx_stream s) { return unary_entry("cbx_gelu", CBX_UNARY_GELU, 0.0f, x, y, s); }
int cbx_gelu_erf(const cbx_tensor* x, cbx_tensor* y, cbx_stream s) { return unary_entry("cbx_gelu_erf", CBX_UNARY_GELU_ERF, 0.0f, x, y, s); }
int cbx_silu(const cbx_tensor* x, cbx_tensor* y, cbx_stream s) { return unary_entry("cbx_silu", CBX_UNARY_SILU, 0.0f, x, y, s); }
int cbx_mish(const cbx_tensor* x, cbx_tensor* y, cbx_stream s) { return unary_entry("cbx_mish", CBX_UNARY_MISH, 0.0f, x, y, s); }

int cbx_leaky_relu(const cbx_tensor* x, float slope, cbx_tensor* y, cbx_stream stream) {
    return unary_entry("cbx_leaky_relu", UNARY_LEAKY, slope, x, y, stream);
}

int cbx_swiglu(const cbx_tensor* g, const cbx_tensor* u, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_swiglu";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = check_float(g, what, "g")) || (rc = check_float(u, what, "u")) || (rc = check_float(y, what, "y"))) return rc;
    if (g->type != u->type || g->type != y->type) return set_error(CBX_ERR_UNSUPPORTED, "cbx_swiglu: g, u, y types differ");
    if (!same_shape(g, y) || !same_shape(u, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_swiglu: shapes differ");
    if (nelements(y) == 0) return CBX_OK;
    return launch_swiglu(g, u, y, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_bias_act(int act, const cbx_tensor* x, const cbx_tensor* bias, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_bias_act";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y")) || (rc = validate(bias, what, "bias")) ||
        (rc = check_act(act, what))) return rc;
    if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32 || bias->type != CBX_TYPE_F32) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_bias_act: F32 only");
    }
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_act: x and y shapes differ");
    const bool inner = bias->ne[0] == x->ne[0] && bias->ne[1] == 1 && bias->ne[2] == 1 && bias->ne[3] == 1;
    const bool outer = bias->ne[0] == 1 && bias->ne[1] == x->ne[1] && bias->ne[2] == 1 && bias->ne[3] == 1;
    if (!inner && !outer) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_bias_act: bias must have ne = (x.ne0,1,1,1) or (1,x.ne1,1,1)");
    }
    if (!is_contiguous(bias)) return set_error(CBX_ERR_UNSUPPORTED, "cbx_bias_act: bias must be contiguous");
    if (nelements(x) == 0) return CBX_OK;
    return launch_bias_act(act, x, bias, y, st, reinterpret_cast<hipStream_t>(stream));
}

int cbx_bias_add_two(const cbx_tensor* x0, const cbx_tensor* b0, cbx_tensor* y0, const cbx_tensor* x1,
                     const cbx_tensor* b1, cbx_tensor* y1, cbx_stream stream) {
    const char* what = "cbx_bias_add_two";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    const cbx_tensor* xs[2] = {x0, x1};
    const cbx_tensor* bs[2] = {b0, b1};
    const cbx_tensor* ys[2] = {y0, y1};
    for (int k = 0; k < 2; k++) {
        if ((rc = validate(xs[k], what, k ? "x1" : "x0")) || (rc = validate(bs[k], what, k ? "b1" : "b0")) ||
            (rc = validate(ys[k], what, k ? "y1" : "y0"))) {
            return rc;
        }
        const cbx_tensor *x = xs[k], *b = bs[k], *y = ys[k];
        if (x->type != CBX_TYPE_F32 || b->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) {
            return set_error(CBX_ERR_UNSUPPORTED, "cbx_bias_add_two: F32 only");
        }
        if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_add_two: an x and its y differ in shape");
        const bool inner = b->ne[0] == x->ne[0] && b->ne[1] == 1 && b->ne[2] == 1 && b->ne[3] == 1;
        const bool outer = b->ne[0] == 1 && b->ne[1] == x->ne[1] && b->ne[2] == 1 && b->ne[3] == 1;
        if ((!inner && !outer) || !is_contiguous(b)) {
            return set_error(CBX_ERR_UNSUPPORTED,
                             "cbx_bias_add_two: each bias contiguous with ne = (x.ne0,1,1,1) or (1,x.ne1,1,1)");
        }
    }
    // the two adds run side by side: neither output may meet the other
    // add's operands or output, nor its own bias (read by every row)
    if (overlaps(y0, x1) || overlaps(y0, b1) || overlaps(y0, y1) || overlaps(y1, x0) || overlaps(y1, b0)) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_add_two: an output overlaps the other add's tensors");
    }
    if (overlaps(y0, b0) || overlaps(y1, b1)) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_add_two: an output overlaps its bias");
    }
    return launch_bias_add_two(x0, b0, y0, x1, b1, y1, st, reinterpret_cast<hipStream_t>(stream));
}

// ---- conv1d -------------------------------------------------------------------

static int conv_weights_create(const cbx_tensor* w, int up, cbx_stream stream, cbx_conv1d_weights** out,
                               const char* what) {
    clear_error();
    if (!out) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": out is NULL");
    *out = nullptr;
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(w, what, "w"))) return rc;
    if (w->type != CBX_TYPE_F32 && w->type != CBX_TYPE_F16) {
        return set_error(CBX_ERR_UNSUPPORTED, std::string(what) + ": w must be F32 or F16");
    }
    if (w->ne[0] < 1 || w->ne[0] > 64 || w->ne[1] < 1 || w->ne[1] > 8192 || w->ne[2] < 1 || w->ne[2] > 8192 ||
        w->ne[3] != 1) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + (up == 0 ? ": w must be (K <= 64, C_in <= 8192, C_out <= 8192, 1)"
                                                                           : ": w must be (K <= 64, C_out <= 8192, C_in <= 8192, 1)"));
    }
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return set_error(CBX_ERR_HIP, std::string(what) + ": hipGetDevice failed");
    auto* cw = new cbx_conv1d_weights();
    cw->serial = g_handle_serial.fetch_add(1);
    cw->device = dev;
    cw->up = up;
    cw->k = w->ne[0];
    cw->taps = up == 0 ? cw->k : cdiv(cw->k, static_cast<int64_t>(up));
    cw->c_in = up == 0 ? w->ne[1] : w->ne[2];
    cw->c_out = up == 0 ? w->ne[2] : w->ne[1];
    conv1d_weights_layout(cw->c_in, cw->c_out, &cw->c_in_pad, &cw->c_out_pad);
    cw->w_ph = cw->c_out_pad * cw->taps * cw->c_in_pad;
    const int64_t n_ph = up == 0 ? 1 : up;
    const size_t bytes = static_cast<size_t>(n_ph * cw->w_ph) * sizeof(_Float16);
    if (hipMalloc(reinterpret_cast<void**>(&cw->data), bytes) != hipSuccess) {
        delete cw;
        return set_error(CBX_ERR_HIP, std::string(what) + ": hipMalloc failed");
    }
    const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    rc = launch_conv1d_weights(w, up, cw->taps, cw->data, cw->c_in_pad, cw->c_out_pad, s);
    if (!rc && hipStreamSynchronize(s) != hipSuccess) {
        rc = set_error(CBX_ERR_HIP, std::string(what) + ": stream synchronisation failed");
    }
    if (rc) {
        hipFree(cw->data);
        delete cw;
        return rc;
    }
    *out = cw;
    return CBX_OK;
}

int cbx_conv1d_weights_create(const cbx_tensor* w, cbx_stream stream, cbx_conv1d_weights** out) {
    return conv_weights_create(w, 0, stream, out, "cbx_conv1d_weights_create");
}

int cbx_conv_transpose1d_weights_create(const cbx_tensor* w, int stride, cbx_stream stream,
                                        cbx_conv1d_weights** out) {
    if (stride < 1 || stride > 64) {
        clear_error();
        if (out) *out = nullptr;
        return set_error(CBX_ERR_INVALID_ARG, "cbx_conv_transpose1d_weights_create: stride must be 1..64");
    }
    return conv_weights_create(w, stride, stream, out, "cbx_conv_transpose1d_weights_create");
}

void cbx_conv1d_weights_destroy(cbx_conv1d_weights* w) {
    if (!w) return;
    int prev = 0;
    hipGetDevice(&prev);
    hipSetDevice(w->device);
    hipDeviceSynchronize();
    hipFree(w->data);
    hipSetDevice(prev);
    delete w;
}

// Checks shared by cbx_conv1d and cbx_conv_transpose1d: the handle's device
// and kind, x against the weights, y's shape (t_out), bias, res, the snake
// vectors, and that y does not overlap x.  Sets *empty for an empty y.
static int check_conv_io(const char* what, const cbx_conv1d_weights* w, bool transposed, int prologue,
                         const cbx_tensor* x, const cbx_tensor* alpha, const cbx_tensor* alpha_inv,
                         const cbx_tensor* bias, const cbx_tensor* res, const cbx_tensor* y, int64_t t_out,
                         const char* t_out_rule, bool* empty) {
    const std::string f(what);
    int rc;
    if (!w) return set_error(CBX_ERR_INVALID_ARG, f + ": weights are NULL");
    if ((w->up != 0) != transposed) {
        return set_error(CBX_ERR_INVALID_ARG, f + (transposed ? ": the weights were made for cbx_conv1d"
                                                              : ": the weights were made for cbx_conv_transpose1d"));
    }
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev != w->device) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": the weights belong to another device");
    }
    if (y->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, f + ": F32 only");
    if (y->ne[0] != w->c_out || y->ne[1] != t_out || y->ne[2] != x->ne[2] || y->ne[3] != 1) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": y must be (C_out, T_out, B, 1), " + t_out_rule);
    }
    if (x->ne[1] >= (int64_t{1} << 30) || t_out >= (int64_t{1} << 30) ||
        x->ne[2] * (transposed ? w->up : 1) >= 65536) {
        return set_error(CBX_ERR_UNSUPPORTED, f + (transposed ? ": T must be below 2^30 and B * stride below 65536"
                                                              : ": T must be below 2^30 and B below 65536"));
    }
    if (bias) {
        if ((rc = validate(bias, what, "bias"))) return rc;
        if (bias->type != CBX_TYPE_F32 || nelements(bias) != w->c_out || !is_contiguous(bias)) {
            return set_error(CBX_ERR_INVALID_ARG, f + ": bias must be contiguous F32 with C_out elements");
        }
    }
    if (res) {
        if ((rc = validate(res, what, "res"))) return rc;
        if (res->type != CBX_TYPE_F32 || !same_shape(res, y)) {
            return set_error(CBX_ERR_INVALID_ARG, f + ": res must be F32 with y's shape");
        }
    }
    if (prologue == CBX_CONV_PRO_SNAKE) {
        for (const cbx_tensor* p : {alpha, alpha_inv}) {
            if ((rc = validate(p, what, p == alpha ? "alpha" : "alpha_inv"))) return rc;
            if (p->type != CBX_TYPE_F32 || nelements(p) != w->c_in || !is_contiguous(p)) {
                return set_error(CBX_ERR_INVALID_ARG, f + ": alpha and alpha_inv must be contiguous F32 with C_in elements");
            }
        }
    }
    *empty = nelements(y) == 0;
    if (*empty) return CBX_OK;
    if (overlaps(x, y)) return set_error(CBX_ERR_INVALID_ARG, f + ": y must not overlap x");
    // Other workgroups' tile stores would race with this workgroup's reads
    // of bias / alpha (staging) and res (epilogue): none may share y's bytes,
    // except res being exactly y (same data and strides: each output is read
    // and then written by the one thread that owns it).
    if (bias && overlaps(bias, y)) return set_error(CBX_ERR_INVALID_ARG, f + ": bias must not overlap y");
    if (prologue == CBX_CONV_PRO_SNAKE && (overlaps(alpha, y) || overlaps(alpha_inv, y))) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": alpha and alpha_inv must not overlap y");
    }
    if (res && overlaps(res, y)) {
        bool same = res->data == y->data;
        for (int i = 0; i < 4; i++) same = same && res->nb[i] == y->nb[i];
        if (!same) return set_error(CBX_ERR_INVALID_ARG, f + ": res must be y itself or not overlap it");
    }
    return CBX_OK;
}

// x must be F32 (C_in, T_in, B, 1) with the weights' C_in; the prologue known.
static int check_conv_x(const char* what, const cbx_conv1d_weights* w, const cbx_tensor* x, int prologue) {
    const std::string f(what);
    if (x->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, f + ": F32 only");
    if (prologue < CBX_CONV_PRO_NONE || prologue > CBX_CONV_PRO_LEAKY_RELU) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": unknown prologue");
    }
    if (w && (x->ne[0] != w->c_in || x->ne[3] != 1)) {
        return set_error(CBX_ERR_INVALID_ARG, f + ": x must be (C_in, T_in, B, 1) with the weights' C_in");
    }
    return CBX_OK;
}

// cbx_conv1d and cbx_conv1d_sum: acc (with its scale) only from the latter
static int conv1d_common(const char* what, const cbx_tensor* x, const cbx_conv1d_weights* w, int stride, int pad,
                         int dilation, int prologue, const cbx_tensor* alpha, const cbx_tensor* alpha_inv, float slope,
                         const cbx_tensor* bias, const cbx_tensor* res, const cbx_tensor* acc, float scale,
                         cbx_tensor* y, cbx_stream stream);

int cbx_conv1d(const cbx_tensor* x, const cbx_conv1d_weights* w, int stride, int pad, int dilation, int prologue,
               const cbx_tensor* alpha, const cbx_tensor* alpha_inv, float slope, const cbx_tensor* bias,
               const cbx_tensor* res, cbx_tensor* y, cbx_stream stream) {
    return conv1d_common("cbx_conv1d", x, w, stride, pad, dilation, prologue, alpha, alpha_inv, slope, bias, res,
                         nullptr, 1.0f, y, stream);
}

int cbx_conv1d_sum(const cbx_tensor* x, const cbx_conv1d_weights* w, int stride, int pad, int dilation, int prologue,
                   const cbx_tensor* alpha, const cbx_tensor* alpha_inv, float slope, const cbx_tensor* bias,
                   const cbx_tensor* res, const cbx_tensor* acc, float scale, cbx_tensor* y, cbx_stream stream) {
    if (!acc) {
        clear_error();
        return set_error(CBX_ERR_INVALID_ARG, "cbx_conv1d_sum: acc is NULL (cbx_conv1d has no sum)");
    }
    return conv1d_common("cbx_conv1d_sum", x, w, stride, pad, dilation, prologue, alpha, alpha_inv, slope, bias, res,
                         acc, scale, y, stream);
}

static int conv1d_common(const char* what, const cbx_tensor* x, const cbx_conv1d_weights* w, int stride, int pad,
                         int dilation, int prologue, const cbx_tensor* alpha, const cbx_tensor* alpha_inv, float slope,
                         const cbx_tensor* bias, const cbx_tensor* res, const cbx_tensor* acc, float scale,
                         cbx_tensor* y, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!w) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": weights are NULL");
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y"))) return rc;
    if ((rc = check_conv_x(what, w, x, prologue))) return rc;
    if (stride < 1 || pad < 0 || dilation < 1 || stride > 64 || pad > (1 << 20) || dilation > 1024) {
        return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": stride must be 1..64, pad >= 0, dilation 1..1024");
    }
    const int64_t t_in = x->ne[1];
    const int64_t span = dilation * (w->k - 1) + 1;
    const int64_t t_out = t_in + 2 * pad >= span ? (t_in + 2 * pad - span) / stride + 1 : 0;
    bool empty = false;
    if ((rc = check_conv_io(what, w, false, prologue, x, alpha, alpha_inv, bias, res, y, t_out,
                            "T_out = (T_in + 2 pad - dilation (K - 1) - 1) / stride + 1", &empty))) {
        return rc;
    }
    if (empty) return CBX_OK;
    if (acc) {
        if ((rc = validate(acc, what, "acc"))) return rc;
        if (acc->type != CBX_TYPE_F32 || !same_shape(acc, y)) {
            return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": acc must be F32 with y's shape");
        }
        // read in the epilogue while other workgroups store their tiles
        if (overlaps(acc, y)) return set_error(CBX_ERR_INVALID_ARG, std::string(what) + ": acc must not overlap y");
    }
    return launch_conv1d(x, w->data, w->k, w->c_in_pad, w->c_out, stride, pad, dilation, 1, 0, w->w_ph, prologue,
                         prologue == CBX_CONV_PRO_SNAKE ? alpha : nullptr,
                         prologue == CBX_CONV_PRO_SNAKE ? alpha_inv : nullptr, slope, bias, res, y, st,
                         reinterpret_cast<hipStream_t>(stream), acc, scale);
}

int cbx_conv_transpose1d(const cbx_tensor* x, const cbx_conv1d_weights* w, int pad, int prologue,
                         const cbx_tensor* alpha, const cbx_tensor* alpha_inv, float slope, const cbx_tensor* bias,
                         cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_conv_transpose1d";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!w) return set_error(CBX_ERR_INVALID_ARG, "cbx_conv_transpose1d: weights are NULL");
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y"))) return rc;
    if ((rc = check_conv_x(what, w, x, prologue))) return rc;
    const int64_t t_in = x->ne[1];
    const int64_t full = t_in > 0 ? (t_in - 1) * w->up + w->k : 0;
    if (pad < 0 || (t_in > 0 && 2 * static_cast<int64_t>(pad) >= full)) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_conv_transpose1d: pad must be >= 0 and leave T_out >= 1");
    }
    const int64_t t_out = t_in > 0 ? full - 2 * static_cast<int64_t>(pad) : 0;
    bool empty = false;
    if ((rc = check_conv_io(what, w, true, prologue, x, alpha, alpha_inv, bias, nullptr, y, t_out,
                            "T_out = (T_in - 1) * stride + K - 2 pad", &empty))) {
        return rc;
    }
    if (empty) return CBX_OK;
    // stride 1: a single phase, i.e. a conv with the taps reversed and
    // padding K - 1 - pad; larger strides run their phases side by side
    const int up = w->up;
    return launch_conv1d(x, w->data, w->taps, w->c_in_pad, w->c_out, 1, up == 1 ? static_cast<int>(w->k) - 1 - pad : 0,
                         1, up, pad, w->w_ph, prologue, prologue == CBX_CONV_PRO_SNAKE ? alpha : nullptr,
                         prologue == CBX_CONV_PRO_SNAKE ? alpha_inv : nullptr, slope, bias, nullptr, y, st,
                         reinterpret_cast<hipStream_t>(stream));
}

int cbx_causal_conv1d(const cbx_tensor* x, const cbx_conv1d_weights* w, const cbx_tensor* mask,
                      const cbx_tensor* bias, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_causal_conv1d";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!w) return set_error(CBX_ERR_INVALID_ARG, "cbx_causal_conv1d: weights are NULL");
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y"))) return rc;
    if ((rc = check_conv_x(what, w, x, CBX_CONV_PRO_NONE))) return rc;
    if (mask) {
        if ((rc = validate(mask, what, "mask"))) return rc;
        if (mask->type != CBX_TYPE_F32 || nelements(mask) != x->ne[1] || !is_contiguous(mask)) {
            return set_error(CBX_ERR_INVALID_ARG, "cbx_causal_conv1d: mask must be contiguous F32 with T elements");
        }
    }
    bool empty = false;
    if ((rc = check_conv_io(what, w, false, CBX_CONV_PRO_NONE, x, nullptr, nullptr, bias, nullptr, y, x->ne[1],
                            "T_out = T_in (left padding K - 1)", &empty))) {
        return rc;
    }
    if (empty) return CBX_OK;
    if (mask && overlaps(mask, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_causal_conv1d: y must not overlap mask");
    // a stride-1 conv with K - 1 zero frames on the left; y's length (T_in)
    // ends the window, so no frame past T_in - 1 is read
    return launch_conv1d(x, w->data, w->k, w->c_in_pad, w->c_out, 1, static_cast<int>(w->k) - 1, 1, 1, 0, w->w_ph,
                         mask ? kConvProMask : CBX_CONV_PRO_NONE, mask, nullptr, 0.0f, bias, nullptr, y, st,
                         reinterpret_cast<hipStream_t>(stream));
}

int cbx_snake(const cbx_tensor* x, const cbx_tensor* alpha, const cbx_tensor* alpha_inv, cbx_tensor* y,
              cbx_stream stream) {
    const char* what = "cbx_snake";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y")) || (rc = validate(alpha, what, "alpha")) ||
        (rc = validate(alpha_inv, what, "alpha_inv"))) return rc;
    if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32 || alpha->type != CBX_TYPE_F32 || alpha_inv->type != CBX_TYPE_F32) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_snake: F32 only");
    }
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_snake: x and y shapes differ");
    if (!same_shape(alpha, alpha_inv)) return set_error(CBX_ERR_INVALID_ARG, "cbx_snake: alpha and alpha_inv shapes differ");
    const bool inner = alpha->ne[0] == x->ne[0] && alpha->ne[1] == 1 && alpha->ne[2] == 1 && alpha->ne[3] == 1;
    const bool outer = alpha->ne[0] == 1 && alpha->ne[1] == x->ne[1] && alpha->ne[2] == 1 && alpha->ne[3] == 1;
    if (!inner && !outer) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_snake: alpha must have ne = (x.ne0,1,1,1) or (1,x.ne1,1,1)");
    }
    if (!is_contiguous(alpha) || !is_contiguous(alpha_inv)) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_snake: alpha and alpha_inv must be contiguous");
    }
    if (nelements(x) == 0) return CBX_OK;
    return launch_snake(x, alpha, alpha_inv, y, st, reinterpret_cast<hipStream_t>(stream));
}

}  // extern "C"

// ---- one launch for several independent ops --------------------------------

namespace {

// [lo, hi) bytes a tensor spans (empty tensors span nothing)
bool byte_range(const cbx_tensor* t, uintptr_t* lo, uintptr_t* hi) {
    if (!t || nelements(t) == 0) return false;
    const size_t row = t->type == CBX_TYPE_Q8_0 ? static_cast<size_t>(t->ne[0] / 32) * 34
                                                 : static_cast<size_t>(t->ne[0]) * type_size(t->type);
    size_t span = row;
    for (int k = 1; k < 4; k++) span += static_cast<size_t>(t->ne[k] - 1) * t->nb[k];
    *lo = reinterpret_cast<uintptr_t>(t->data);
    *hi = *lo + span;
    return true;
}

bool rows_aligned_to(const cbx_tensor* t, size_t a) {
    if (reinterpret_cast<uintptr_t>(t->data) % a) return false;
    for (int k = 1; k < 4; k++) if (t->ne[k] > 1 && t->nb[k] % a) return false;
    return true;
}

BTen bten(const cbx_tensor* t, int64_t step) {
    BTen b;
    b.p = t ? static_cast<char*>(t->data) : nullptr;
    b.nb1 = step;
    return b;
}

int batch_fail(int i, int code, const std::string& msg) {
    return set_error(code, "cbx_run_ops: op " + std::to_string(i) + ": " + msg);
}

// Fills b from o (validated) and returns the op's workgroup count in *nblk.
// GroupNorm ops take chunk slots of the stream's scratch set from *gn_slot on.
int build_op(int i, const cbx_op& o, BOp& b, DeviceState* st, hipStream_t strm, uint32_t* gn_slot, int64_t* nblk) {
    const char* what = "cbx_run_ops";
    int rc;
    b.kind = o.kind;
    b.act = o.act;
    b.eps = o.eps;
    b.param = o.param;
    b.table = st->gelu_table;
    b.ff = nullptr;
    b.n_pos = 0;
    b.nv = 1;
    for (auto& t : b.t) t = bten(nullptr, 0);
    *nblk = 0;
    switch (o.kind) {
        case CBX_OP_LAYER_NORM:
        case CBX_OP_RMS_NORM: {
            const cbx_tensor *x = o.src[0], *w = o.src[1], *bb = o.kind == CBX_OP_LAYER_NORM ? o.src[2] : nullptr;
            const cbx_tensor* y = o.dst[0];
            if ((rc = check_float(x, what, "x")) || (rc = check_float(y, what, "y"))) return rc;
            if (x->type != y->type || !same_shape(x, y)) return batch_fail(i, CBX_ERR_INVALID_ARG, "x and y differ in type or shape");
            if (!(o.eps >= 0.0f)) return batch_fail(i, CBX_ERR_INVALID_ARG, "eps must be >= 0");
            if ((rc = check_row_param(w, x, what, "w")) || (rc = check_row_param(bb, x, what, "b")) || (rc = check_act(o.act, what))) return rc;
            if (o.kind == CBX_OP_RMS_NORM && o.act != CBX_UNARY_NONE) return batch_fail(i, CBX_ERR_UNSUPPORTED, "RMS norm takes no activation");
            const size_t al = x->type == CBX_TYPE_F32 ? 16 : 8;
            if (x->ne[0] % 4 || x->ne[0] > 1024 || !flat_rows(x) || !flat_rows(y) || !rows_aligned_to(x, al) ||
                !rows_aligned_to(y, al) || (w && reinterpret_cast<uintptr_t>(w->data) % 16) ||
                (bb && reinterpret_cast<uintptr_t>(bb->data) % 16)) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED, "norm rows must be <= 1024 elements, ne0 % 4 == 0, uniformly strided and aligned");
            }
            b.t_x = x->type;
            b.ne0 = x->ne[0];
            b.rows = nrows(x);
            b.nv = x->ne[0] <= 256 ? 1 : x->ne[0] <= 512 ? 2 : 4;
            b.t[0] = bten(x, static_cast<int64_t>(x->nb[1]));
            b.t[1] = bten(w, 0);
            b.t[2] = bten(bb, 0);
            b.t[6] = bten(y, static_cast<int64_t>(y->nb[1]));
            // rows of 513..1024 and few of them (a decode step's 1..64
            // streams): one row a workgroup, shared by its 4 waves (aux3 = 4)
            // instead of 4 rows a workgroup, one wave each (aux3 = 1)
            b.aux3 = b.nv == 4 && b.rows <= int64_t{4} * st->n_cu ? 4 : 1;
            *nblk = b.aux3 == 4 ? b.rows : cdiv(b.rows, 4);
            return CBX_OK;
        }
        case CBX_OP_UNARY:
        case CBX_OP_LEAKY_RELU:
        case CBX_OP_SWIGLU: {
            const bool glu = o.kind == CBX_OP_SWIGLU;
            const cbx_tensor *x = o.src[0], *u = glu ? o.src[1] : nullptr, *y = o.dst[0];
            if ((rc = check_float(x, what, "x")) || (rc = check_float(y, what, "y")) || (glu && (rc = check_float(u, what, "u")))) return rc;
            if (x->type != y->type || !same_shape(x, y) || (glu && (u->type != x->type || !same_shape(u, x)))) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "operands differ in type or shape");
            }
            if (o.kind == CBX_OP_UNARY && (o.act < CBX_UNARY_GELU || o.act > CBX_UNARY_MISH)) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "unknown unary op " + std::to_string(o.act));
            }
            const size_t al = x->type == CBX_TYPE_F32 ? 16 : 8;
            for (const cbx_tensor* t : {x, u, static_cast<const cbx_tensor*>(y)}) {
                if (t && (!is_contiguous(t) || reinterpret_cast<uintptr_t>(t->data) % al)) {
                    return batch_fail(i, CBX_ERR_UNSUPPORTED, "element-wise operands must be contiguous and aligned");
                }
            }
            b.t_x = x->type;
            b.rows = nelements(x);
            b.t[0] = bten(x, 0);
            b.t[1] = bten(u, 0);
            b.t[6] = bten(y, 0);
            *nblk = b.rows ? cdiv(b.rows / 4 + 1, 256) : 0;
            return CBX_OK;
        }
        case CBX_OP_ROPE: {
            const cbx_tensor *x = o.src[0], *pos = o.src[1], *y = o.dst[0];
            const cbx_rope_cache* c = o.rope;
            if (!c) return batch_fail(i, CBX_ERR_INVALID_ARG, "rope is NULL");
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || dev != c->device) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "rope table belongs to another device");
            }
            if ((rc = check_float(x, what, "x")) || (rc = check_float(y, what, "y")) || (rc = validate(pos, what, "pos"))) return rc;
            if (x->type != y->type || !same_shape(x, y)) return batch_fail(i, CBX_ERR_INVALID_ARG, "x and y differ in type or shape");
            if (pos->type != CBX_TYPE_I32 || pos->ne[0] != x->ne[2] || nelements(pos) != pos->ne[0]) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "pos must be I32 with ne = (x.ne2, 1, 1, 1)");
            }
            if (c->p.n_dims > x->ne[0]) return batch_fail(i, CBX_ERR_INVALID_ARG, "n_dims > x.ne0");
            if (c->p.n_dims / 2 > 256 || !flat_rows(x) || !flat_rows(y) || x->ne[1] * x->ne[0] >= (int64_t{1} << 31)) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED, "rope needs n_dims <= 512 and uniformly strided rows");
            }
            b.t_x = x->type;
            b.ne0 = x->ne[0];
            b.rows = x->ne[2] * x->ne[3];
            b.aux = x->ne[1];
            b.aux2 = x->ne[2];
            b.t[0] = bten(x, static_cast<int64_t>(x->nb[1]));
            b.t[1] = bten(pos, static_cast<int64_t>(pos->nb[0]));
            b.t[6] = bten(y, static_cast<int64_t>(y->nb[1]));
            b.table = c->table;
            b.ff = c->freq_factors;
            b.n_pos = c->n_pos;
            b.rp = c->p;
            // nv = 1: four pairs a lane with 4-element vector loads of x and
            // y and 16-byte cos/sin loads (n_dims % 8 == 0, rows aligned to
            // the vector size, the table to 16 bytes); 0: a pair a lane
            {
                const size_t vb = 4 * type_size(x->type);
                const bool al = reinterpret_cast<uintptr_t>(x->data) % vb == 0 &&
                                reinterpret_cast<uintptr_t>(y->data) % vb == 0 && x->nb[1] % vb == 0 &&
                                y->nb[1] % vb == 0 && reinterpret_cast<uintptr_t>(c->table) % 16 == 0;
                b.nv = al && c->p.n_dims % 8 == 0 ? 1 : 0;
            }
            *nblk = nelements(x) ? b.rows : 0;
            return CBX_OK;
        }
        case CBX_OP_GET_ROWS:
        case CBX_OP_GET_ROWS_ADD_LAYER_NORM: {
            const bool ln = o.kind == CBX_OP_GET_ROWS_ADD_LAYER_NORM;
            const cbx_tensor *src = o.src[0], *ids = o.src[1], *src2 = o.src[2], *ids2 = o.src[3];
            cbx_tensor* y = ln ? o.dst[1] : o.dst[0];
            cbx_tensor* h = ln ? o.dst[0] : nullptr;
            if ((rc = check_gather(what, src, ids, y))) return rc;
            if ((src2 || ids2 || ln) && (rc = check_gather(what, src2, ids2, y))) return rc;
            if (h && ((rc = validate(h, what, "h")) || h->type != CBX_TYPE_F32 || !same_shape(h, y))) {
                return rc ? rc : batch_fail(i, CBX_ERR_INVALID_ARG, "h must be F32 with y's shape");
            }
            if (ln) {
                if (!(o.eps >= 0.0f)) return batch_fail(i, CBX_ERR_INVALID_ARG, "eps must be >= 0");
                if ((rc = check_row_param(o.src[4], y, what, "w")) || (rc = check_row_param(o.src[5], y, what, "b"))) return rc;
            }
            auto table_ok = [](const cbx_tensor* t) {
                if (!t) return true;
                if (t->ne[2] != 1 || t->ne[3] != 1) return false;
                if (t->type == CBX_TYPE_Q8_0) return (reinterpret_cast<uintptr_t>(t->data) & 1u) == 0;
                return rows_aligned_to(t, t->type == CBX_TYPE_F32 ? 16 : 8);
            };
            if (ids->ne[1] != 1 || ids->ne[2] != 1 || y->ne[0] % 4 || !table_ok(src) || !table_ok(src2) ||
                !flat_rows(y) || !rows_aligned_to(y, 16) || (h && (!flat_rows(h) || !rows_aligned_to(h, 16))) ||
                (ln && (y->ne[0] > 1024 || (o.src[4] && reinterpret_cast<uintptr_t>(o.src[4]->data) % 16) ||
                        (o.src[5] && reinterpret_cast<uintptr_t>(o.src[5]->data) % 16)))) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED,
                                  "gathers need 1-D ids, 2-D tables, ne0 % 4 == 0 (<= 1024 with LayerNorm) and aligned rows");
            }
            b.t_x = src->type;
            b.t_x2 = src2 ? src2->type : -1;
            b.ne0 = y->ne[0];
            b.rows = ids->ne[0];
            b.aux = src->ne[1];
            b.aux2 = src2 ? src2->ne[1] : 0;
            b.t[0] = bten(src, static_cast<int64_t>(src->nb[1]));
            b.t[1] = bten(ids, static_cast<int64_t>(ids->nb[0]));
            b.t[2] = bten(src2, src2 ? static_cast<int64_t>(src2->nb[1]) : 0);
            b.t[3] = bten(ids2, ids2 ? static_cast<int64_t>(ids2->nb[0]) : 0);
            if (ln) {
                b.t[4] = bten(o.src[4], 0);
                b.t[5] = bten(o.src[5], 0);
                b.t[6] = bten(h, h ? static_cast<int64_t>(h->nb[1]) : 0);
                b.t[7] = bten(y, static_cast<int64_t>(y->nb[1]));
                b.nv = y->ne[0] <= 256 ? 1 : y->ne[0] <= 512 ? 2 : 4;
                // rows of 513..1024 and few tokens against the CUs: one
                // token a workgroup over its 4 waves (aux3 = 4) instead of
                // four tokens a workgroup, one wave each
                b.aux3 = b.nv == 4 && b.rows <= int64_t{4} * st->n_cu ? 4 : 1;
                *nblk = b.aux3 == 4 ? b.rows : cdiv(b.rows, 4);
            } else {
                b.t[6] = bten(y, static_cast<int64_t>(y->nb[1]));
                *nblk = b.rows;
            }
            if (nelements(y) == 0) *nblk = 0;
            return CBX_OK;
        }
        case CBX_OP_SNAKE: {
            const cbx_tensor *x = o.src[0], *a = o.src[1], *ai = o.src[2], *y = o.dst[0];
            if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y")) || (rc = validate(a, what, "alpha")) ||
                (rc = validate(ai, what, "alpha_inv"))) return rc;
            if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32 || a->type != CBX_TYPE_F32 || ai->type != CBX_TYPE_F32) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED, "snake is F32 only");
            }
            if (!same_shape(x, y) || !same_shape(a, ai)) return batch_fail(i, CBX_ERR_INVALID_ARG, "shapes differ");
            const bool inner = a->ne[0] == x->ne[0] && a->ne[1] == 1 && a->ne[2] == 1 && a->ne[3] == 1 && x->ne[0] > 1;
            const bool outer = a->ne[0] == 1 && a->ne[1] == x->ne[1] && a->ne[2] == 1 && a->ne[3] == 1;
            if (!inner && !outer) return batch_fail(i, CBX_ERR_UNSUPPORTED, "alpha must be (x.ne0,1,1,1) or (1,x.ne1,1,1)");
            const int64_t n = nelements(x);
            if (!is_contiguous(x) || !is_contiguous(y) || !is_contiguous(a) || !is_contiguous(ai) || x->ne[0] % 4 ||
                n >= (int64_t{1} << 32) || reinterpret_cast<uintptr_t>(x->data) % 16 ||
                reinterpret_cast<uintptr_t>(y->data) % 16 || reinterpret_cast<uintptr_t>(a->data) % 16 ||
                reinterpret_cast<uintptr_t>(ai->data) % 16) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED, "snake needs contiguous aligned tensors, ne0 % 4 == 0");
            }
            const int64_t C = inner ? x->ne[0] : x->ne[1];
            b.act = inner ? 1 : 0;
            b.rows = n;
            b.aux = C;
            b.aux2 = (C & (C - 1)) == 0 ? C - 1 : 0;
            b.aux3 = x->ne[0] / 4;
            b.t[0] = bten(x, 0);
            b.t[1] = bten(a, 0);
            b.t[2] = bten(ai, 0);
            b.t[6] = bten(y, 0);
            *nblk = cdiv(n / 4, 256);
            return CBX_OK;
        }
        case CBX_OP_GROUP_NORM: {
            const cbx_tensor *x = o.src[0], *w = o.src[1], *bb = o.src[2], *y = o.dst[0];
            if ((rc = check_group_norm(what, x, o.iparam, o.eps, w, bb, o.act, y))) return rc;
            if (o.act != CBX_UNARY_NONE && o.act != CBX_UNARY_MISH) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED, "group norm takes no activation or Mish");
            }
            if (nelements(x) == 0) return CBX_OK;
            GnSplit sp;
            uint32_t n_slots = 0, used = 0;
            int nv = 1;
            const char* why = nullptr;
            if (!group_norm_split_args(x, o.iparam, o.eps, w, bb, o.act, y, group_norm_scratch_for(st, strm), *gn_slot,
                                       kGnWaitAuto, 0, st, &sp, &n_slots, &nv, &used, &why)) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED, std::string("group norm does not take the split reduction: ") +
                                                              why);
            }
            if (nv > 4) return batch_fail(i, CBX_ERR_UNSUPPORTED, "group norm chunks of more than 4 vectors a lane");
            b.gn = sp;
            b.nv = nv;
            b.aux = o.act == CBX_UNARY_MISH ? 2 : 0;
            *gn_slot += used;
            *nblk = n_slots;
            return CBX_OK;
        }
        case CBX_OP_LAYER_NORM_ROPE: {
            const cbx_tensor *x = o.src[0], *w = o.src[1], *bb = o.src[2], *pos = o.src[3], *y = o.dst[0];
            const cbx_rope_cache* c = o.rope;
            if (!c) return batch_fail(i, CBX_ERR_INVALID_ARG, "rope is NULL");
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || dev != c->device) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "rope table belongs to another device");
            }
            if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y")) || (rc = validate(pos, what, "pos"))) return rc;
            if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) return batch_fail(i, CBX_ERR_UNSUPPORTED, "F32 only");
            if (!same_shape(x, y)) return batch_fail(i, CBX_ERR_INVALID_ARG, "x and y shapes differ");
            if (!(o.eps >= 0.0f)) return batch_fail(i, CBX_ERR_INVALID_ARG, "eps must be >= 0");
            if ((rc = check_row_param(w, x, what, "w")) || (rc = check_row_param(bb, x, what, "b"))) return rc;
            const int64_t hd = o.iparam;
            if (hd <= 0 || hd % 4 || x->ne[0] % hd) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "head_dim must divide x.ne0 and be a multiple of 4");
            }
            if (c->p.n_dims > hd) return batch_fail(i, CBX_ERR_INVALID_ARG, "n_dims > head_dim");
            if (x->ne[3] != 1) return batch_fail(i, CBX_ERR_INVALID_ARG, "x must be at most 3-D (C, n_tok, batch)");
            if (pos->type != CBX_TYPE_I32 || pos->ne[0] != x->ne[1] || pos->ne[1] != 1 || pos->ne[2] != 1 ||
                pos->ne[3] != 1) {
                return batch_fail(i, CBX_ERR_INVALID_ARG, "pos must be I32 with ne = (x.ne1, 1, 1, 1)");
            }
            const int64_t hq = hd / 4, dq = c->p.n_dims / 8;
            const bool neox = c->p.mode == 2;
            const bool xs = flat_rows(x) && flat_rows(y) && rows_aligned_to(x, 16) && rows_aligned_to(y, 16) &&
                            reinterpret_cast<uintptr_t>(c->table) % 16 == 0 && 64 % hq == 0 &&
                            (neox ? c->p.n_dims % 8 == 0 && dq > 0 && (dq & (dq - 1)) == 0 : c->p.n_dims % 4 == 0);
            if (x->ne[0] > 1024 || !xs || (w && reinterpret_cast<uintptr_t>(w->data) % 16) ||
                (bb && reinterpret_cast<uintptr_t>(bb->data) % 16) || x->ne[1] * x->ne[2] >= (int64_t{1} << 31)) {
                return batch_fail(i, CBX_ERR_UNSUPPORTED,
                                  "layer norm + rope needs rows <= 1024 at one 16-byte aligned stride and a head's "
                                  "rotation partners in one wave");
            }
            b.t_x = CBX_TYPE_F32;
            b.ne0 = x->ne[0];
            b.aux = hd;
            b.aux2 = x->ne[1];
            b.rows = x->ne[1] * x->ne[2];
            b.t[0] = bten(x, static_cast<int64_t>(x->nb[1]));
            b.t[1] = bten(pos, static_cast<int64_t>(pos->nb[0]));
            b.t[2] = bten(w, 0);
            b.t[3] = bten(bb, 0);
            b.t[6] = bten(y, static_cast<int64_t>(y->nb[1]));
            b.table = c->table;
            b.ff = c->freq_factors;
            b.n_pos = c->n_pos;
            b.rp = c->p;
            b.nv = x->ne[0] <= 256 ? 1 : x->ne[0] <= 512 ? 2 : 4;
            *nblk = nelements(x) ? cdiv(b.rows, 4) : 0;
            return CBX_OK;
        }
        default:
            return batch_fail(i, CBX_ERR_INVALID_ARG, "unknown op kind " + std::to_string(o.kind));
    }
}

}  // namespace

extern "C" int cbx_run_ops(const cbx_op* ops, int n_ops, cbx_stream stream) {
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if (!ops || n_ops <= 0 || n_ops > CBX_MAX_OPS) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_run_ops: n_ops must be in 1.." + std::to_string(CBX_MAX_OPS));
    }
    BatchArgs a{};
    a.n = n_ops;
    a.err = st->err_word;
    const hipStream_t strm = reinterpret_cast<hipStream_t>(stream);
    // GroupNorm ops first: their block ranges then start at multiples of 8
    // (each takes a multiple of 8 workgroups) and their chunk workgroups are
    // dispatched before any other op's, so a group's chunks are resident
    // together
    int order[CBX_MAX_OPS];
    int n_order = 0;
    for (int pass = 0; pass < 2; pass++) {
        for (int i = 0; i < n_ops; i++) {
            if ((ops[i].kind == CBX_OP_GROUP_NORM) == (pass == 0)) order[n_order++] = i;
        }
    }
    int64_t total = 0, gn_blocks = 0, nbk[CBX_MAX_OPS];
    uint32_t gn_slot = 0;
    for (int k = 0; k < n_ops; k++) {
        const int i = order[k];
        if (ops[i].reserved != 0) return batch_fail(i, CBX_ERR_INVALID_ARG, "reserved must be 0");
        if ((rc = build_op(i, ops[i], a.op[k], st, strm, &gn_slot, &nbk[k]))) return rc;
        if (ops[i].kind == CBX_OP_GROUP_NORM) gn_blocks += nbk[k];
        total += nbk[k];
        if (total >= (int64_t{1} << 31)) return set_error(CBX_ERR_UNSUPPORTED, "cbx_run_ops: too many workgroups");
    }
    // an embedding + LayerNorm beside more than 2 other workgroups a CU
    // takes one wave a token (four tokens a workgroup): its four-wave form's
    // longer-lived workgroups would hold the CUs the other ops need (the
    // prefill chain with GELU: 6.93 against 6.54 us a launch)
    for (int k = 0; k < n_ops; k++) {
        BOp& b = a.op[k];
        if (b.kind == CBX_OP_GET_ROWS_ADD_LAYER_NORM && b.aux3 == 4 && total - nbk[k] > int64_t{2} * st->n_cu) {
            total -= nbk[k];
            b.aux3 = 1;
            nbk[k] = cdiv(b.rows, 4);
            total += nbk[k];
        }
    }
    // a launch of more workgroups than about 6 a CU takes two rounds: its
    // f32 element-wise ops then take two vectors a lane (half the
    // workgroups), the rest stay as they are
    if (total > int64_t{6} * st->n_cu) {
        for (int k = 0; k < n_ops; k++) {
            BOp& b = a.op[k];
            if ((b.kind == CBX_OP_UNARY || b.kind == CBX_OP_LEAKY_RELU) && b.t_x == CBX_TYPE_F32 && nbk[k] > 0) {
                total -= nbk[k];
                b.aux3 = 2;
                nbk[k] = cdiv(b.rows / 4 + 1, 512);
                total += nbk[k];
            }
        }
    }
    total = 0;
    for (int k = 0; k < kBatchMaxOps; k++) {
        // past the last op: an offset no workgroup reaches
        a.blk0[k] = k < n_ops ? static_cast<uint32_t>(total) : UINT32_MAX;
        if (k < n_ops) total += nbk[k];
    }
    if (gn_blocks > int64_t{2} * st->n_cu) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_run_ops: the group norms' chunk workgroups are more than 2 a CU");
    }
    // independence: no op writes what another op reads or writes
    for (int i = 0; i < n_ops; i++) {
        for (const cbx_tensor* d : ops[i].dst) {
            uintptr_t dl, dh;
            if (!byte_range(d, &dl, &dh)) continue;
            for (int j = 0; j < n_ops; j++) {
                if (j == i) continue;
                const cbx_tensor* other[8] = {ops[j].src[0], ops[j].src[1], ops[j].src[2], ops[j].src[3],
                                              ops[j].src[4], ops[j].src[5], ops[j].dst[0], ops[j].dst[1]};
                for (const cbx_tensor* t : other) {
                    uintptr_t tl, th;
                    if (byte_range(t, &tl, &th) && dl < th && tl < dh) {
                        return set_error(CBX_ERR_INVALID_ARG, "cbx_run_ops: op " + std::to_string(i) +
                                                                  " writes memory that op " + std::to_string(j) + " uses");
                    }
                }
            }
        }
    }
    if (total == 0) return CBX_OK;
    return launch_batch(a, static_cast<uint32_t>(total), reinterpret_cast<hipStream_t>(stream));
}

// ---- ggml_add / ggml_mul with repeat, ggml_concat ------------------------------

namespace {

bool same_view(const cbx_tensor* a, const cbx_tensor* b) {
    if (a->data != b->data || !same_shape(a, b)) return false;
    for (int k = 0; k < 4; k++) if (a->ne[k] > 1 && a->nb[k] != b->nb[k]) return false;
    return true;
}

}  // namespace

extern "C" int cbx_binary(int op, const cbx_tensor* a, const cbx_tensor* b, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_binary";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(a, what, "a")) || (rc = validate(b, what, "b")) || (rc = validate(y, what, "y"))) return rc;
    if (op != CBX_BINARY_ADD && op != CBX_BINARY_MUL) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_binary: unknown op " + std::to_string(op));
    }
    if (a->type != CBX_TYPE_F32 || b->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_binary: F32 only");
    }
    if (!same_shape(a, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_binary: a and y shapes differ");
    if (nelements(a) == 0) return CBX_OK;
    for (int k = 0; k < 4; k++) {
        if (b->ne[k] < 1 || a->ne[k] % b->ne[k] != 0) {
            return set_error(CBX_ERR_INVALID_ARG, "cbx_binary: b must repeat to a's shape (every a.ne[i] a multiple of b.ne[i])");
        }
    }
    if (overlaps(y, b) || (overlaps(y, a) && !same_view(y, a))) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_binary: y overlaps b, or a other than as a itself");
    }
    return launch_binary(op, a, b, y, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cbx_bias_residual(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* r, cbx_tensor* y,
                                 cbx_stream stream) {
    const char* what = "cbx_bias_residual";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(bias, what, "bias")) || (rc = validate(r, what, "r")) ||
        (rc = validate(y, what, "y"))) {
        return rc;
    }
    if (x->type != CBX_TYPE_F32 || bias->type != CBX_TYPE_F32 || r->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_bias_residual: F32 only");
    }
    if (!same_shape(r, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_residual: r and y shapes differ");
    if (nelements(r) == 0) return CBX_OK;
    for (int k = 0; k < 4; k++) {
        if (x->ne[k] < 1 || r->ne[k] % x->ne[k] != 0 || bias->ne[k] < 1 || x->ne[k] % bias->ne[k] != 0) {
            return set_error(CBX_ERR_INVALID_ARG,
                             "cbx_bias_residual: bias must repeat to x's shape and x to r's (every ne[i] a multiple)");
        }
    }
    if (overlaps(y, bias) || (overlaps(y, r) && !same_view(y, r)) ||
        (overlaps(y, x) && !(same_shape(x, r) && same_view(y, x)))) {
        return set_error(CBX_ERR_INVALID_ARG,
                         "cbx_bias_residual: y overlaps bias, r other than as r itself, or x other than as x itself");
    }
    return launch_bias_residual(x, bias, r, y, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cbx_bias_add_pair(const cbx_tensor* x, const cbx_tensor* bias, const cbx_tensor* u,
                                 const cbx_tensor* v, cbx_tensor* yu, cbx_tensor* yv, cbx_stream stream) {
    const char* what = "cbx_bias_add_pair";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(bias, what, "bias")) || (rc = validate(u, what, "u")) ||
        (rc = validate(v, what, "v")) || (rc = validate(yu, what, "yu")) || (rc = validate(yv, what, "yv"))) {
        return rc;
    }
    for (const cbx_tensor* p : {x, bias, u, v, static_cast<const cbx_tensor*>(yu), static_cast<const cbx_tensor*>(yv)}) {
        if (p->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, "cbx_bias_add_pair: F32 only");
    }
    if (!same_shape(x, yu) || !same_shape(x, yv)) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_add_pair: yu and yv must have x's shape");
    }
    if (nelements(x) == 0) return CBX_OK;
    for (const cbx_tensor* p : {bias, u, v}) {
        for (int k = 0; k < 4; k++) {
            if (p->ne[k] < 1 || x->ne[k] % p->ne[k] != 0) {
                return set_error(CBX_ERR_INVALID_ARG,
                                 "cbx_bias_add_pair: bias, u and v must repeat to x's shape (every ne[i] a multiple)");
            }
        }
    }
    for (const cbx_tensor* p : {x, bias, u, v}) {
        if (overlaps(yu, p) || overlaps(yv, p)) {
            return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_add_pair: yu or yv overlaps an input");
        }
    }
    if (overlaps(yu, yv)) return set_error(CBX_ERR_INVALID_ARG, "cbx_bias_add_pair: yu and yv overlap");
    return launch_bias_add_pair(x, bias, u, v, yu, yv, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cbx_scale(const cbx_tensor* x, float sc, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_scale";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(x, what, "x")) || (rc = validate(y, what, "y"))) return rc;
    if (x->type != CBX_TYPE_F32 || y->type != CBX_TYPE_F32) return set_error(CBX_ERR_UNSUPPORTED, "cbx_scale: F32 only");
    if (!same_shape(x, y)) return set_error(CBX_ERR_INVALID_ARG, "cbx_scale: x and y shapes differ");
    if (overlaps(y, x) && !same_view(y, x)) return set_error(CBX_ERR_INVALID_ARG, "cbx_scale: y overlaps x other than as x itself");
    if (nelements(x) == 0) return CBX_OK;
    return launch_scale(x, sc, y, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int cbx_concat(const cbx_tensor* a, const cbx_tensor* b, int dim, cbx_tensor* y, cbx_stream stream) {
    const char* what = "cbx_concat";
    clear_error();
    int rc;
    DeviceState* st = current_state(&rc);
    if (!st) return rc;
    if ((rc = validate(a, what, "a")) || (rc = validate(b, what, "b")) || (rc = validate(y, what, "y"))) return rc;
    if (dim < 0 || dim > 3) return set_error(CBX_ERR_INVALID_ARG, "cbx_concat: dim must be 0..3");
    if ((a->type != CBX_TYPE_F32 && a->type != CBX_TYPE_F16) || b->type != a->type || y->type != a->type) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_concat: a, b and y must all be F32 or all F16");
    }
    for (int k = 0; k < 4; k++) {
        const bool ok = k == dim ? y->ne[k] == a->ne[k] + b->ne[k] : (a->ne[k] == y->ne[k] && b->ne[k] == y->ne[k]);
        if (!ok) {
            return set_error(CBX_ERR_INVALID_ARG, "cbx_concat: y.ne[dim] must be a.ne[dim] + b.ne[dim] and the other dims equal");
        }
    }
    if (overlaps(y, a) || overlaps(y, b)) return set_error(CBX_ERR_INVALID_ARG, "cbx_concat: y overlaps a or b");
    if (nelements(y) == 0) return CBX_OK;
    return launch_concat(a, b, dim, y, reinterpret_cast<hipStream_t>(stream));
}
