// k_rows.hip -- embedding gather (F32 / F16 / Q8_0 tables, optional fused
// second gather + add) and F32<->F16 conversion.
//
// Gather: one workgroup per output row; lanes move 4 consecutive elements
// each (16-byte stores), so a wave writes 1 KiB contiguous.  Q8_0 rows are
// dequantised in registers: each 4-element group reads its block's f16
// scale and four int8 quants and forms q * d with one f32 multiply, exactly
// dequantize_row_q8_0.  The second gather's row is added with one f32 add,
// exactly ggml_add of the two gathered tensors (t3.cpp:446-455).
#include "cbx_rowops.h"

namespace cbx {
namespace {

enum { T_F32 = CBX_TYPE_F32, T_F16 = CBX_TYPE_F16, T_Q8 = CBX_TYPE_Q8_0 };

// 4 elements starting at element j (j % 4 == 0) of a table row.
template <int TYPE>
__device__ __forceinline__ float4 load_row4(const char* row, int64_t j) {
    return load_table4<TYPE>(row, j);
}

template <int TYPE>
__device__ __forceinline__ float load_row1(const char* row, int64_t j) {
    if constexpr (TYPE == T_F32) {
        return *reinterpret_cast<const float*>(row + j * 4);
    } else if constexpr (TYPE == T_F16) {
        return h2f(*reinterpret_cast<const uint16_t*>(row + j * 2));
    } else {
        const char* blk = row + (j >> 5) * 34;
        const float d = h2f(*reinterpret_cast<const uint16_t*>(blk));
        return static_cast<float>(*reinterpret_cast<const int8_t*>(blk + 2 + (j & 31))) * d;
    }
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
    return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

constexpr int kGatherThreads = 256;

// TYPE2 < 0: plain gather.  VEC: rows are 16-byte aligned and ne0 % 4 == 0.
// Exactly one workgroup per output row, of a fixed size: no loop bound or
// block size to wait for before the id load.
// A table operand: base, strides of its rows and of dims 2 and 3, row count.
struct GTable {
    const char* p;
    int64_t nb1, nb2, nb3;
    int64_t rows;
};

// An id operand (int32): base and the byte strides of its three dims.
struct GIds {
    const char* p;
    int64_t nb0, nb1, nb2;
};

struct GatherArgs {
    GTable src, src2;
    GIds ids, ids2;
    char* dst;
    int64_t dnb1, dnb2, dnb3;
    uint32_t n10, n11;     // ids ne0, ne1: output row r is (r % n10, (r / n10) % n11, r / (n10 * n11))
    int32_t ne0;
    uint32_t* err;
};

template <int TYPE, int TYPE2, bool VEC>
__global__ __launch_bounds__(kGatherThreads) void k_get_rows(GatherArgs a) {
    const int64_t ne0 = a.ne0;
    const uint32_t r = blockIdx.x;
    const uint32_t i10 = r % a.n10, q = r / a.n10;
    const uint32_t i11 = q % a.n11, i12 = q / a.n11;
    const int32_t id = *reinterpret_cast<const int32_t*>(a.ids.p + i10 * a.ids.nb0 + i11 * a.ids.nb1 + i12 * a.ids.nb2);
    bool ok = id >= 0 && id < a.src.rows;
    int32_t id2 = 0;
    if constexpr (TYPE2 >= 0) {
        id2 = *reinterpret_cast<const int32_t*>(a.ids2.p + i10 * a.ids2.nb0 + i11 * a.ids2.nb1 + i12 * a.ids2.nb2);
        ok = ok && id2 >= 0 && id2 < a.src2.rows;
    }
    // the table and output fields in the argument loads that go out with
    // the ids' (left alone, the compiler loads some only after the ids have
    // arrived: one more scalar round trip before the row loads)
    arg_now(a.src.p); arg_now(reinterpret_cast<const void*>(a.src.nb1));
    arg_now(reinterpret_cast<const void*>(a.src.nb2)); arg_now(reinterpret_cast<const void*>(a.src.nb3));
    arg_now(reinterpret_cast<const void*>(a.src.rows)); arg_now(a.dst);
    arg_now(reinterpret_cast<const void*>(a.dnb1)); arg_now(reinterpret_cast<const void*>(a.dnb2));
    arg_now(reinterpret_cast<const void*>(a.dnb3)); arg_now(static_cast<uint32_t>(a.ne0));
    if constexpr (TYPE2 >= 0) {
        arg_now(a.src2.p); arg_now(reinterpret_cast<const void*>(a.src2.nb1));
        arg_now(reinterpret_cast<const void*>(a.src2.nb2)); arg_now(reinterpret_cast<const void*>(a.src2.nb3));
        arg_now(reinterpret_cast<const void*>(a.src2.rows));
    }
    char* d = a.dst + i10 * a.dnb1 + i11 * a.dnb2 + i12 * a.dnb3;
    // ggml aborts on an out-of-range index; here the row is zeroed and the
    // sticky device error bit is raised for the host to read.  A bad id
    // reads row 0 (the table has rows) and the values are replaced by zeros,
    // so no branch stands between the id and the row loads.
    const int64_t r1 = ok ? id : 0, r2 = ok ? id2 : 0;
    const char* s = a.src.p + r1 * a.src.nb1 + i11 * a.src.nb2 + i12 * a.src.nb3;
    const char* s2 = nullptr;
    if constexpr (TYPE2 >= 0) s2 = a.src2.p + r2 * a.src2.nb1 + i11 * a.src2.nb2 + i12 * a.src2.nb3;
    if constexpr (VEC) {
        for (int64_t j = threadIdx.x * 4; j < ne0; j += kGatherThreads * 4) {
            float4 v = load_row4<TYPE>(s, j);
            if constexpr (TYPE2 >= 0) v = add4(v, load_row4<TYPE2>(s2, j));
            *reinterpret_cast<float4*>(d + j * 4) = ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    } else {
        for (int64_t j = threadIdx.x; j < ne0; j += kGatherThreads) {
            float v = load_row1<TYPE>(s, j);
            if constexpr (TYPE2 >= 0) v = v + load_row1<TYPE2>(s2, j);
            reinterpret_cast<float*>(d)[j] = ok ? v : 0.0f;
        }
    }
    if (!ok && threadIdx.x == 0) atomicOr(a.err, static_cast<uint32_t>(DEV_ERR_ROW_INDEX));
}

GTable gtable(const cbx_tensor* t) {
    GTable g;
    g.p = t ? static_cast<const char*>(t->data) : nullptr;
    g.nb1 = t ? static_cast<int64_t>(t->nb[1]) : 0;
    g.nb2 = t ? static_cast<int64_t>(t->nb[2]) : 0;
    g.nb3 = t ? static_cast<int64_t>(t->nb[3]) : 0;
    g.rows = t ? t->ne[1] : 0;
    return g;
}

GIds gids(const cbx_tensor* t) {
    GIds g;
    g.p = t ? static_cast<const char*>(t->data) : nullptr;
    g.nb0 = t ? static_cast<int64_t>(t->nb[0]) : 0;
    g.nb1 = t ? static_cast<int64_t>(t->nb[1]) : 0;
    g.nb2 = t ? static_cast<int64_t>(t->nb[2]) : 0;
    return g;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

// Can the table be read 4 elements at a time with aligned vector loads?
bool vec_ok_table(const cbx_tensor* t) {
    if (!t) return true;
    if (t->type == CBX_TYPE_Q8_0) return (reinterpret_cast<uintptr_t>(t->data) & 1u) == 0;   // 16-bit quant loads
    const size_t a = t->type == CBX_TYPE_F32 ? 16 : 8;
    if (reinterpret_cast<uintptr_t>(t->data) % a) return false;
    for (int i = 1; i < 4; i++) if (t->nb[i] % a) return false;
    return t->ne[0] % 4 == 0;
}

template <int TYPE, int TYPE2>
int launch_gather_t(bool vec, dim3 grid, dim3 block, hipStream_t s, const GatherArgs& a) {
    if (vec) {
        hipLaunchKernelGGL((k_get_rows<TYPE, TYPE2, true>), grid, block, 0, s, a);
    } else {
        hipLaunchKernelGGL((k_get_rows<TYPE, TYPE2, false>), grid, block, 0, s, a);
    }
    return check_launch("get_rows");
}

template <int TYPE>
int launch_gather_t1(int type2, bool vec, dim3 grid, dim3 block, hipStream_t s, const GatherArgs& a) {
    switch (type2) {
        case -1: return launch_gather_t<TYPE, -1>(vec, grid, block, s, a);
        case T_F32: return launch_gather_t<TYPE, T_F32>(vec, grid, block, s, a);
        case T_F16: return launch_gather_t<TYPE, T_F16>(vec, grid, block, s, a);
        default: return launch_gather_t<TYPE, T_Q8>(vec, grid, block, s, a);
    }
}

// ---- F32 <-> F16 conversion -------------------------------------------------

template <typename TS, typename TD>
__global__ __launch_bounds__(256) void k_cpy_flat(const char* __restrict__ x, char* __restrict__ y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t n4 = n >> 2;
    if (i < n4) {
        Stream<TD>::store4(y + i * 4 * Elt<TD>::size, Stream<TS>::load4(x + i * 4 * Elt<TS>::size));
    } else if (i == n4) {
        for (int64_t j = n4 * 4; j < n; j++) Elt<TD>::store1(y + j * Elt<TD>::size, Elt<TS>::load1(x + j * Elt<TS>::size));
    }
}

template <typename TS, typename TD>
__global__ __launch_bounds__(256) void k_cpy_rows(View x, View y, int64_t nr, bool fx, bool fy) {
    for (int64_t r = blockIdx.x; r < nr; r += gridDim.x) {
        const char* xr = x.data + row_offset(x, r, fx);
        char* yr = y.data + row_offset(y, r, fy);
        for (int64_t j = threadIdx.x; j < x.ne[0]; j += blockDim.x) {
            Elt<TD>::store1(yr + j * Elt<TD>::size, Elt<TS>::load1(xr + j * Elt<TS>::size));
        }
    }
}

template <typename TS, typename TD>
int launch_cpy_t(const cbx_tensor* src, cbx_tensor* dst, DeviceState* st, hipStream_t s) {
    const int64_t n = nelements(src);
    const bool flat = is_contiguous(src) && is_contiguous(dst) && aligned16(src->data) && aligned16(dst->data) &&
                      (n >> 2) + 1 < (int64_t{1} << 39);
    if (flat) {
        const int64_t blocks = cdiv((n >> 2) + 1, 256);
        hipLaunchKernelGGL((k_cpy_flat<TS, TD>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                           static_cast<const char*>(src->data), static_cast<char*>(dst->data), n);
    } else {
        const int64_t nr = nrows(src);
        const int64_t blocks = std::min<int64_t>(nr, int64_t{1} << 20);
        hipLaunchKernelGGL((k_cpy_rows<TS, TD>), dim3(blocks), dim3(256), 0, s, view_of(src), view_of(dst), nr,
                           flat_rows(src), flat_rows(dst));
    }
    return check_launch("cpy");
}

}  // namespace

int launch_get_rows(const cbx_tensor* src, const cbx_tensor* ids, const cbx_tensor* src2, const cbx_tensor* ids2,
                    cbx_tensor* dst, DeviceState* st, hipStream_t s) {
    const int64_t n = ids->ne[0] * ids->ne[1] * ids->ne[2];
    const bool vec = dst->ne[0] % 4 == 0 && vec_ok_table(src) && vec_ok_table(src2) && aligned16(dst->data) &&
                     dst->nb[1] % 16 == 0 && dst->nb[2] % 16 == 0 && dst->nb[3] % 16 == 0;
    if (n >= (int64_t{1} << 31) || dst->ne[0] >= (int64_t{1} << 31)) {
        return set_error(CBX_ERR_UNSUPPORTED, "get_rows: too many rows or columns");
    }
    const dim3 grid(static_cast<unsigned>(n)), block(kGatherThreads);
    GatherArgs a;
    a.src = gtable(src);
    a.src2 = gtable(src2);
    a.ids = gids(ids);
    a.ids2 = gids(ids2);
    a.dst = static_cast<char*>(dst->data);
    a.dnb1 = static_cast<int64_t>(dst->nb[1]);
    a.dnb2 = static_cast<int64_t>(dst->nb[2]);
    a.dnb3 = static_cast<int64_t>(dst->nb[3]);
    a.n10 = static_cast<uint32_t>(ids->ne[0]);
    a.n11 = static_cast<uint32_t>(ids->ne[1]);
    a.ne0 = static_cast<int32_t>(dst->ne[0]);
    a.err = st->err_word;
    const int t2 = src2 ? src2->type : -1;
    switch (src->type) {
        case T_F32: return launch_gather_t1<T_F32>(t2, vec, grid, block, s, a);
        case T_F16: return launch_gather_t1<T_F16>(t2, vec, grid, block, s, a);
        default: return launch_gather_t1<T_Q8>(t2, vec, grid, block, s, a);
    }
}

int launch_cpy(const cbx_tensor* src, cbx_tensor* dst, DeviceState* st, hipStream_t s) {
    const bool s16 = src->type == CBX_TYPE_F16, d16 = dst->type == CBX_TYPE_F16;
    if (!s16 && !d16) return launch_cpy_t<float, float>(src, dst, st, s);
    if (!s16 && d16) return launch_cpy_t<float, uint16_t>(src, dst, st, s);
    if (s16 && !d16) return launch_cpy_t<uint16_t, float>(src, dst, st, s);
    return launch_cpy_t<uint16_t, uint16_t>(src, dst, st, s);
}

}  // namespace cbx
