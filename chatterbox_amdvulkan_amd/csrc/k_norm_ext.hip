// k_norm_ext.hip -- LayerNorm with the element-wise nodes that the
// reference's graph builders put right before or after it, in one pass:
//
//   residual join + LayerNorm (t3.cpp:528-532, 539-546; s3enc.cpp:273-276;
//   flow_encoder.cpp:395-399):
//       s = (a + a_bias) + r      (two ggml_add nodes; a_bias optional)
//       y = act(LN(s) * w + b)    (s stored: it is the residual stream)
//   causal_block1d's tail (cfm_decoder.cpp:143-148):
//       y = act(LN(x) * w + b) * mask[row]      (mask (1, T): one per frame)
//
// One wave per row, as the plain LayerNorm kernel: each lane holds NV
// 4-element vectors of the row in registers, the two reductions are
// wave-local f64 butterflies, every f32 operation rounds once in the order
// of the ggml nodes it replaces.  HBM traffic per row: the residual join
// reads two rows and writes two (s, y) where the ggml nodes read and write
// nine; the masked form reads one and writes one.
#include "cbx_rowops.h"

namespace cbx {
namespace {

// the prologue: none, s = a + r, s = (a + bias) + r, s = a + bias
enum { PRO_NONE = 0, PRO_RESID = 1, PRO_BIAS_RESID = 2, PRO_BIAS = 3 };

struct LnExtArgs {
    const char* a;
    const char* r;
    const float* ab;     // a_bias (PRO_BIAS_RESID)
    const float* w;
    const float* b;
    const float* mask;   // one scale per ne1 index (MASK)
    const uint16_t* tab;
    char* s;             // the sum, or nullptr
    char* y;
    RowMap ma, mr, ms, my;
    int32_t ne0, nr;
    float eps;
    int32_t act;
};

// Byte offset of row r: FLAT rows sit at one stride (no index split and no
// test of the map's flag, so nothing waits on an argument before the loads).
template <bool FLAT>
__device__ __forceinline__ int64_t row_off(const RowMap& m, uint32_t r) {
    if constexpr (FLAT) return static_cast<int64_t>(r) * m.nb1;
    else return row_at(m, r);
}

// WPB rows a workgroup (one wave each), or, with WPR > 1, one row shared by
// WPR waves (wave w holds float4s [w*64*NV, (w+1)*64*NV) of it): few rows
// (a 512-token prefill on 256 CUs) leave most SIMDs idle at one wave a row.
template <int NV, bool ACT, int PRO, bool MASK, int WPB, bool FLAT, int WPR = 1>
__global__ __launch_bounds__(64 * WPB * WPR) void k_ln_ext(LnExtArgs p) {
    static_assert(WPB == 1 || WPR == 1, "rows a workgroup or waves a row, not both");
    __shared__ double lds[2 * WPR];
    // the rows' addresses in the first batch of argument loads (left alone,
    // the compiler loads the affine pointers first and the row pointers and
    // strides in a second scalar round trip before the row loads)
    arg_now(p.a); arg_now(p.r); arg_now(p.ab); arg_now(p.w); arg_now(p.b); arg_now(p.s); arg_now(p.y);
    arg_now(reinterpret_cast<const void*>(p.ma.nb1)); arg_now(reinterpret_cast<const void*>(p.mr.nb1));
    arg_now(reinterpret_cast<const void*>(p.ms.nb1)); arg_now(reinterpret_cast<const void*>(p.my.nb1));
    arg_now(static_cast<uint32_t>(p.ne0)); arg_now(static_cast<uint32_t>(p.nr));
    if constexpr (MASK) {
        arg_now(p.mask);
        arg_now(p.ma.ne1);
    }
    if constexpr (!FLAT) {
        for (const RowMap* m : {&p.ma, &p.mr, &p.ms, &p.my}) {
            arg_now(reinterpret_cast<const void*>(m->nb2)); arg_now(reinterpret_cast<const void*>(m->nb3));
            arg_now(m->ne1); arg_now(m->ne2); arg_now(m->flat);
        }
    }
    const int lane = WPR > 1 ? (threadIdx.x >> 6) * 64 * NV + (threadIdx.x & 63) : (threadIdx.x & 63);
    uint32_t row = blockIdx.x;
    if constexpr (WPB > 1) {
        row = row * WPB + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
        if (row >= static_cast<uint32_t>(p.nr)) return;   // uniform per wave
    }
    const int64_t ne0 = p.ne0;
    const char* ar = p.a + row_off<FLAT>(p.ma, row);
    char* yr = p.y + row_off<FLAT>(p.my, row);
    char* sr = p.s + row_off<FLAT>(p.ms, row);   // only stored through when p.s is set
    Affine<NV> af;
    af.load_sel(p.w, p.b, reinterpret_cast<const float*>(p.tab), lane, ne0);
    // several waves a row: w and b issue ahead of the row loads, as in the
    // embedding's LayerNorm
    if constexpr (WPR > 1) __builtin_amdgcn_sched_barrier(0);
    float m = 1.0f;
    if constexpr (MASK) m = p.mask[row % p.ma.ne1];
    // every load is unconditional (clamped address) so all are in flight
    // together; lanes past the row end zero their values afterwards
    float4 v[NV], q[NV], c[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        const int64_t jc = j < ne0 ? j : 0;
        v[k] = *reinterpret_cast<const float4*>(ar + jc * 4);
        if constexpr (PRO == PRO_BIAS_RESID || PRO == PRO_BIAS) c[k] = *reinterpret_cast<const float4*>(p.ab + jc);
    }
    if constexpr (PRO == PRO_RESID || PRO == PRO_BIAS_RESID) {
        const char* rr = p.r + row_off<FLAT>(p.mr, row);
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int64_t j = (lane + 64 * k) * 4;
            q[k] = *reinterpret_cast<const float4*>(rr + (j < ne0 ? j : 0) * 4);
        }
    }
    // the sums by selects, not a branch (a branch would take the loads into
    // its block); the sum, when stored, with nothing else pending
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const bool in = (lane + 64 * k) * 4 < ne0;
        float4 t = v[k];
        if constexpr (PRO == PRO_BIAS_RESID || PRO == PRO_BIAS) {
            t = make_float4(t.x + c[k].x, t.y + c[k].y, t.z + c[k].z, t.w + c[k].w);
        }
        if constexpr (PRO == PRO_RESID || PRO == PRO_BIAS_RESID) {
            t = make_float4(t.x + q[k].x, t.y + q[k].y, t.z + q[k].z, t.w + q[k].w);
        }
        v[k] = make_float4(in ? t.x : 0.f, in ? t.y : 0.f, in ? t.z : 0.f, in ? t.w : 0.f);
    }
    if constexpr (PRO != PRO_NONE) {
        wait_vector_memory();
        if (p.s) {
#pragma unroll
            for (int k = 0; k < NV; k++) {
                const int64_t j = (lane + 64 * k) * 4;
                if (j < ne0) Stream<float>::store4(sr + j * 4, v[k]);
            }
        }
    }
    const float scale = row_scale_w<NV, NORM_LN, WPR>(v, lane, ne0, p.eps, lds);
    const bool hw = p.w != nullptr, hb = p.b != nullptr;
#pragma unroll
    for (int k = 0; k < NV; k++) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float t = get(v[k], e) * scale;
            if (hw) t = t * get(af.w[k], e);
            if (hb) t = t + get(af.b[k], e);
            set(v[k], e, t);
        }
    }
    if constexpr (ACT) apply_act_vec<NV>(p.act, v, p.tab, 0.0f);
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int64_t j = (lane + 64 * k) * 4;
        if (j < ne0) {
            float4 o = v[k];
            if constexpr (MASK) o = make_float4(o.x * m, o.y * m, o.z * m, o.w * m);
            Stream<float>::store4(yr + j * 4, o);
        }
    }
}

template <bool ACT, int PRO, bool MASK, int WPB, bool FLAT>
void go_nv(const LnExtArgs& a, int nv, dim3 grid, hipStream_t s) {
    const dim3 block(64 * WPB);
    switch (nv) {
        case 1: hipLaunchKernelGGL((k_ln_ext<1, ACT, PRO, MASK, WPB, FLAT>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_ln_ext<2, ACT, PRO, MASK, WPB, FLAT>), grid, block, 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_ln_ext<4, ACT, PRO, MASK, WPB, FLAT>), grid, block, 0, s, a); break;
        case 8: hipLaunchKernelGGL((k_ln_ext<8, ACT, PRO, MASK, WPB, FLAT>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((k_ln_ext<16, ACT, PRO, MASK, WPB, FLAT>), grid, block, 0, s, a); break;
    }
}

// One row a workgroup shared by wpr waves (nv: vectors a lane for one wave
// a row; each wave then holds nv / wpr).
template <bool ACT, int PRO, bool MASK>
void go_wpr(const LnExtArgs& a, int nv, int wpr, dim3 grid, hipStream_t s) {
    const dim3 block(64 * wpr);
    switch (nv * 8 + wpr) {
        case 2 * 8 + 2: hipLaunchKernelGGL((k_ln_ext<1, ACT, PRO, MASK, 1, true, 2>), grid, block, 0, s, a); break;
        case 4 * 8 + 2: hipLaunchKernelGGL((k_ln_ext<2, ACT, PRO, MASK, 1, true, 2>), grid, block, 0, s, a); break;
        case 4 * 8 + 4: hipLaunchKernelGGL((k_ln_ext<1, ACT, PRO, MASK, 1, true, 4>), grid, block, 0, s, a); break;
        case 8 * 8 + 2: hipLaunchKernelGGL((k_ln_ext<4, ACT, PRO, MASK, 1, true, 2>), grid, block, 0, s, a); break;
        case 8 * 8 + 4: hipLaunchKernelGGL((k_ln_ext<2, ACT, PRO, MASK, 1, true, 4>), grid, block, 0, s, a); break;
        case 16 * 8 + 2: hipLaunchKernelGGL((k_ln_ext<8, ACT, PRO, MASK, 1, true, 2>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((k_ln_ext<4, ACT, PRO, MASK, 1, true, 4>), grid, block, 0, s, a); break;   // 16, 4
    }
}

// Uniformly strided tensors take the FLAT kernels (four rows per workgroup
// past 2048 rows, one row shared by wpr waves when the rows are few); any
// other layout the general row map, one row each.
template <int PRO, bool MASK>
void go_pro(const LnExtArgs& a, bool act, int nv, int wpb, int wpr, bool flat, int64_t nr, hipStream_t s) {
    if (flat && wpr > 1) {
        const dim3 grid(static_cast<unsigned>(nr));
        if (act) go_wpr<true, PRO, MASK>(a, nv, wpr, grid, s);
        else go_wpr<false, PRO, MASK>(a, nv, wpr, grid, s);
        return;
    }
    if (!flat) {
        const dim3 grid(static_cast<unsigned>(nr));
        if (act) go_nv<true, PRO, MASK, 1, false>(a, nv, grid, s);
        else go_nv<false, PRO, MASK, 1, false>(a, nv, grid, s);
        return;
    }
    const dim3 grid(static_cast<unsigned>(cdiv(nr, wpb)));
    if (wpb == 1) {
        if (act) go_nv<true, PRO, MASK, 1, true>(a, nv, grid, s);
        else go_nv<false, PRO, MASK, 1, true>(a, nv, grid, s);
    } else {
        if (act) go_nv<true, PRO, MASK, 4, true>(a, nv, grid, s);
        else go_nv<false, PRO, MASK, 4, true>(a, nv, grid, s);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

bool rows16(const cbx_tensor* t) {
    if (!aligned16(t->data)) return false;
    for (int i = 1; i < 4; i++) if (t->nb[i] % 16) return false;
    return true;
}

}  // namespace

int launch_layer_norm_ext(const cbx_tensor* a, const cbx_tensor* a_bias, const cbx_tensor* r, const cbx_tensor* w,
                          const cbx_tensor* b, const cbx_tensor* mask, float eps, int act, cbx_tensor* s,
                          cbx_tensor* y, DeviceState* st, hipStream_t strm, const char* what) {
    const int64_t ne0 = a->ne[0];
    const int64_t nr = nrows(a);
    bool ok = ne0 % 4 == 0 && ne0 <= 4096 && nr < (int64_t{1} << 31) && rows16(a) && rows16(y) &&
              (!r || rows16(r)) && (!s || rows16(s));
    for (const cbx_tensor* v : {a_bias, w, b}) ok = ok && (!v || aligned16(v->data));
    if (!ok) {
        return set_error(CBX_ERR_UNSUPPORTED, std::string(what) +
                                                  ": needs ne0 % 4 == 0, ne0 <= 4096, fewer than 2^31 rows, and "
                                                  "16-byte aligned rows and vectors");
    }
    LnExtArgs p;
    p.a = static_cast<const char*>(a->data);
    p.r = r ? static_cast<const char*>(r->data) : nullptr;
    p.ab = a_bias ? static_cast<const float*>(a_bias->data) : nullptr;
    p.w = w ? static_cast<const float*>(w->data) : nullptr;
    p.b = b ? static_cast<const float*>(b->data) : nullptr;
    p.mask = mask ? static_cast<const float*>(mask->data) : nullptr;
    p.tab = st->gelu_table;
    p.s = s ? static_cast<char*>(s->data) : nullptr;
    p.y = static_cast<char*>(y->data);
    p.ma = row_map(a);
    p.mr = r ? row_map(r) : p.ma;
    p.ms = s ? row_map(s) : p.ma;
    p.my = row_map(y);
    p.ne0 = static_cast<int32_t>(ne0);
    p.nr = static_cast<int32_t>(nr);
    p.eps = eps;
    p.act = act;
    const int nv = ne0 <= 256 ? 1 : ne0 <= 512 ? 2 : ne0 <= 1024 ? 4 : ne0 <= 2048 ? 8 : 16;
    const int wpb = nr >= int64_t{8} * st->n_cu ? 4 : 1;
    // waves a row: enough for about eight waves a CU, at most 4 and at most
    // one per vector a lane
    int wpr = 1;
    while (wpr < 4 && wpr < nv && nr * wpr < int64_t{8} * st->n_cu) wpr *= 2;
    const bool has_act = act != CBX_UNARY_NONE;
    const bool flat = p.ma.flat && p.my.flat && (!r || p.mr.flat) && (!s || p.ms.flat);
    if (mask) go_pro<PRO_NONE, true>(p, has_act, nv, wpb, wpr, flat, nr, strm);
    else if (a_bias && !r) go_pro<PRO_BIAS, false>(p, has_act, nv, wpb, wpr, flat, nr, strm);
    else if (a_bias) go_pro<PRO_BIAS_RESID, false>(p, has_act, nv, wpb, wpr, flat, nr, strm);
    else go_pro<PRO_RESID, false>(p, has_act, nv, wpb, wpr, flat, nr, strm);
    return check_launch(what);
}

}  // namespace cbx
