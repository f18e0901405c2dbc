// k_conv1d.hip -- the HiFT vocoder's conv1d on the reference's (C, T) layout
// (channel innermost) as an implicit GEMM on the matrix cores, with the
// activation that precedes the conv applied while the input is staged:
// Snake in the ResBlocks (hift_vocoder.cpp:119-138), LeakyReLU before
// conv_post (:748-749), and for the CFM decoder's causal conv the frame mask
// of causal_block1d (cfm_decoder.cpp:89-120,139; K-1 frames of left
// padding).  Bias and the ResBlock's residual add are fused into the store.
//
// Arithmetic class of the reference (conv_1d_f32, hift_vocoder.cpp:46-59):
// im2col rounds the conv input to f16, mul_mat rounds the weights to f16 and
// sums the products in f32.  Here: pro(x) in f32 (the five snake() ops, or
// leaky_relu) rounded to f16 (RNE) into LDS, weights pre-rounded to f16,
// v_mfma_f32_32x32x16_f16 products summed in f32, then + bias, then + res.
//
// GEMM view: output time t (M) x output channel co (N), reduced over input
// channel ci and tap k.  A workgroup owns BT times x BC channels.  It stages
// the activated f16 input window -- (BT-1)*stride + (K-1)*dilation + 1 rows
// of all input channels (of a chunk of them when they do not fit the
// 160 KiB of LDS) -- once; every tap's A rows are shifted views of it, so
// each input element is loaded and activated once per workgroup.  Then each
// wave runs K * C_in/16 steps, each MT x NT MFMAs: A fragments (8 f16 of one
// window row) from LDS, read one step ahead; B fragments from the prepared
// weights, whose fragment-major layout makes each one a contiguous KiB,
// read PF steps ahead into a register ring so the L2 latency hides under
// the MFMAs.  Each workgroup starts its sweep of the steps at its own
// offset, so the workgroups sharing an L2 spread their fragment reads over
// it instead of all reading the same KiB.  The finished tile goes through
// LDS to row-contiguous float4 stores (with the bias and residual reads).
//
// The transposed conv of the upsamplers (hift_vocoder.cpp:96-115) runs on
// the same kernel: output phase ph of stride s is a stride-1 conv of the
// input with that phase's taps reversed, so the s phases are s such convs
// side by side in grid z, each writing every s-th output row.
//
// Fragment layout of v_mfma_f32_32x32x16_f16 (checked on the device):
// lane l holds A[l % 32][8*(l/32) + j] and B[8*(l/32) + j][l % 32], j < 8;
// accumulator register r of lane l is D[8*(r/4) + 4*(l/32) + r%4][l % 32].
#include <mutex>
#include <set>
#include <utility>

#include "cbx_device.h"

namespace cbx {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kBlk = 16;              // input channels per MFMA step (the K of one MFMA)
constexpr int kChanAlign = 32;        // input channels are padded to this
constexpr size_t kLdsMax = 160 * 1024;

struct ConvArgs {
    const char* x;              // input row (time) t of batch b at x + b*x_nb2 + t*x_nb1
    const _Float16* w;          // fragment-major: [c_out_pad/32][k][c_in_pad/16][64 lanes][8]
    const float* alpha;         // snake alpha (c_in); the frame mask (t_in values) for PRO_MASK
    const float* alpha_inv;     // snake alpha_inv (c_in)
    const float* bias;          // (c_out) or null
    const char* res;            // (c_out, t_out, B) or null
    char* y;
    int64_t x_nb1, x_nb2, y_nb1, y_nb2, r_nb1, r_nb2;
    int32_t c_in, c_in_pad, c_out, k, t_in, t_out, stride, pad, dil;
    int32_t win;                // window rows
    int32_t kch;                // input channels staged per chunk (a multiple of 32)
    int32_t up;                 // transposed conv with stride up > 1: blockIdx.z = b * up + phase
    int32_t crop;               // transposed: outputs cropped from each end
    int64_t w_ph;               // transposed: halves of prepared weights per phase
    int32_t vout;               // c_out % 4 == 0 and 16-byte aligned y, res and bias: float4 stores
    int32_t n_tt, n_ct;         // time tiles and channel tiles of the grid (work item w = (z*n_tt + t)*n_ct + c)
    float slope;
    const char* acc;            // (c_out, t_out, B) added after the residual, or null (stride-1 convs only)
    int64_t a_nb1, a_nb2;
    float oscale;               // the sum times oscale when scaled
    int32_t scaled;
};

// The ResBlock sum after the residual add (hift_vocoder.cpp:731-736):
// s4 (acc's float4, read with the residual's) + v, then times oscale when
// scaled -- ggml_add(sum, r) and ggml_scale, each one f32 rounding, in
// that order.  acc has y's (t, co) layout.
__device__ __forceinline__ float4 sum_scale(float4 v, float4 s4, float oscale, int32_t scaled) {
    v = make_float4(s4.x + v.x, s4.y + v.y, s4.z + v.z, s4.w + v.w);
    if (scaled) v = make_float4(v.x * oscale, v.y * oscale, v.z * oscale, v.w * oscale);
    return v;
}

// PRO_MASK: x times a per-frame mask (the CFM causal block's pre-mask)
enum { PRO_NONE = 0, PRO_SNAKE = 1, PRO_LEAKY = 2, PRO_MASK = 3 };

// Snake's sin^2 is sin_sq_small (cbx_device.h) for arguments below
// kSinSmall; windows holding a larger argument are fixed up element by
// element with the library sinf in a separate, rarely entered pass, so the
// unrolled staging loop carries one short straight-line sin.

// WM x WN x KS waves: the output tile is WM x WN wave tiles of (MT*32
// times) x (NT*32 output channels), and KS waves share each wave tile,
// splitting the reduction's steps between them (their partial sums are
// added in LDS at the end, in a fixed order).
// VEC: c_in % 4 == 0 and 16-byte aligned rows (one float4 per 4 channels).
// PF: depth of the B fragment ring; it divides every wave's step count, so
// the step loop has no guard and its loads no condition, and the compiler
// waits for exactly the fragment each step uses.
template <int PRO, int MT, int NT, int WM, int WN, int KS, bool VEC, int PF>
__global__ __launch_bounds__(64 * WM * WN * KS) __attribute__((amdgpu_waves_per_eu(KS > 1 ? 2 : 1))) void k_conv1d(
    ConvArgs a) {
    extern __shared__ _Float16 lds[];   // [a.win][a.kch + 8], then alpha and alpha_inv of a chunk (snake)
    constexpr int BT = WM * MT * 32, BC = WN * NT * 32, NTH = 64 * WM * WN * KS;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave / (WM * WN), wt = wave - ks * (WM * WN);
    const int wm = wt / WN, wn = wt % WN;
    // workgroup L of a 1-D grid runs on XCD L % 8 (round-robin dispatch);
    // work items are numbered so that consecutive ones -- the channel tiles
    // of one time tile, then neighbouring time tiles, which read the same or
    // overlapping windows -- run on one XCD and meet in its L2
    const unsigned L = blockIdx.x, n_wg = gridDim.x;
    const unsigned q8 = n_wg >> 3, r8 = n_wg & 7, xcd = L & 7, j8 = L >> 3;
    const unsigned w = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int ct = static_cast<int>(w % static_cast<unsigned>(a.n_ct));
    const unsigned wr = w / static_cast<unsigned>(a.n_ct);
    const int tt = static_cast<int>(wr % static_cast<unsigned>(a.n_tt));
    const int t0 = tt * BT;
    const int co0 = ct * BC;
    int bz = static_cast<int>(wr / static_cast<unsigned>(a.n_tt)), pad = a.pad, t_out = a.t_out;
    int64_t y_off = 0, y_step = a.y_nb1, r_off = 0, r_step = a.r_nb1;
    const _Float16* wbase = a.w;
    if (a.up > 1) {
        // transposed conv, one phase ph of the full output t' = t + crop:
        // t' = up*m + ph takes tap ph + j*up from input m - j.  Its outputs
        // t = c1 + up*u (u = 0, 1, ..) are a stride-1 conv of the input with
        // the phase's taps in reverse order and padding k - 1 - m(c1).
        const int ph = bz % a.up;
        bz /= a.up;
        const int c1 = ((ph - a.crop) % a.up + a.up) % a.up;
        pad = a.k - 1 - (c1 + a.crop - ph) / a.up;
        t_out = c1 < a.t_out ? (a.t_out - c1 + a.up - 1) / a.up : 0;
        y_off = c1 * a.y_nb1;
        y_step = a.up * a.y_nb1;
        r_off = c1 * a.r_nb1;
        r_step = a.up * a.r_nb1;
        wbase += ph * a.w_ph;
    }
    if (t0 >= t_out) return;   // a phase with fewer outputs than the grid covers (uniform)
    const char* xb = a.x + static_cast<int64_t>(bz) * a.x_nb2;
    const int base_t = t0 * a.stride - pad;     // input time of window row 0
    const int lrow = lane & 31, lk = 8 * (lane >> 5);
    const int cs = a.kch + 8;                   // LDS row stride (halves): conflict-free 16-byte reads
    const int nblk = a.c_in_pad / kBlk;         // 16-channel blocks of the weights

    floatx16 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
#pragma unroll
            for (int r = 0; r < 16; r++) acc[mt][nt][r] = 0.0f;
        }
    }
    // fragment (co tile, k = 0, block 0) of each of the lane's NT output tiles
    const _Float16* wf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; nt++) {
        const int co_t = (co0 >> 5) + wn * NT + nt;
        wf[nt] = wbase + static_cast<int64_t>(co_t) * a.k * nblk * 512 + lane * 8;
    }
    // LDS offset (halves) of the lane's A row of each tile mt at tap 0, block 0
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = ((wm * MT + mt) * 32 + lrow) * a.stride * cs + lk;

    for (int ci0 = 0; ci0 < a.c_in; ci0 += a.kch) {
        const int kch = a.c_in - ci0 < a.kch ? ((a.c_in - ci0 + kChanAlign - 1) / kChanAlign) * kChanAlign : a.kch;
        if (ci0 > 0) __syncthreads();   // the previous chunk's fragments have been read
        // snake: this chunk's alpha and alpha_inv into LDS, so the activation
        // below reads them without a global round trip per element; a flag
        // word after them marks a window with an argument of sin past
        // kSinSmall
        float* sal = reinterpret_cast<float*>(lds + a.win * cs);
        int* big_flag = reinterpret_cast<int*>(sal + 2 * a.kch);
        if constexpr (PRO == PRO_SNAKE) {
            for (int c = tid; c < kch; c += NTH) {
                const int cc = ci0 + c < a.c_in ? ci0 + c : 0;
                sal[c] = a.alpha[cc];
                sal[a.kch + c] = a.alpha_inv[cc];
            }
            if (tid == 0) *big_flag = 0;
            __syncthreads();
        }
        // stage pro(x) rows [base_t, base_t + win) x channels [ci0, ci0 + kch)
        // as f16.  Thread tid owns the 4-channel group g = tid % gpr in rows
        // tid / gpr + dr * j: dr = NTH / gpr rows per pass (the host keeps
        // kch <= 4 * NTH); threads past dr * gpr repeat another thread's
        // group and rows and write the same values.  Batches of kStage
        // passes that end inside the window run without a row guard.  Every
        // load is issued unconditionally -- from the prepared weights
        // (always valid) where the element lies outside x -- and zeroed
        // afterwards, so all kStage loads of a lane are in flight together.
        constexpr int kStage = 8;
        const int gpr = kch >> 2;                 // groups per row
        const int dr = NTH / gpr;
        const int tq = tid < dr * gpr ? tid : tid - dr * gpr;
        const int r0 = tq / gpr, cg = 4 * (tq - r0 * gpr), ci = ci0 + cg;
        const float* safe = reinterpret_cast<const float*>(a.w);
        float4 al4 = make_float4(0.f, 0.f, 0.f, 0.f), ai4 = al4;   // snake: the group's alpha, alpha_inv
        if constexpr (PRO == PRO_SNAKE) {
            al4 = *reinterpret_cast<const float4*>(sal + cg);
            ai4 = *reinterpret_cast<const float4*>(sal + a.kch + cg);
        }
        float mx = 0.0f;   // snake: the largest |x * alpha| staged (NaN needs no fix-up: both sins give NaN)
        auto stage_batch = [&](int p0, auto guarded) {
            constexpr bool G = decltype(guarded)::value;
            float4 v[kStage];
            float mv[kStage];   // PRO_MASK: the row's mask value
#pragma unroll
            for (int i = 0; i < kStage; i++) {
                const int rr = r0 + (p0 + i) * dr, ti = base_t + rr;
                const bool row_ok = (!G || rr < a.win) && ti >= 0 && ti < a.t_in;
                const float* row = reinterpret_cast<const float*>(xb + static_cast<int64_t>(row_ok ? ti : 0) * a.x_nb1);
                if constexpr (PRO == PRO_MASK) {
                    const float m = *(row_ok ? a.alpha + ti : safe);
                    mv[i] = row_ok ? m : 0.0f;
                }
                if constexpr (VEC) {
                    const bool ok = row_ok && ci < a.c_in;
                    const float4 t = *reinterpret_cast<const float4*>(ok ? row + ci : safe);
                    v[i] = ok ? t : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const bool ok = row_ok && ci + q < a.c_in;
                        const float t = *(ok ? row + ci + q : safe);
                        set(v[i], q, ok ? t : 0.0f);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kStage; i++) {
                const int rr = r0 + (p0 + i) * dr;
                if (!G || rr < a.win) {
                    float4 t = v[i];
                    // pro(0) = 0: padding rows and channels stay 0
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if constexpr (PRO == PRO_SNAKE) {
                            // snake(x) = x + sin(x*a)^2 * a_inv in the reference's op order
                            const float xv = get(t, q), xa = xv * get(al4, q);
                            mx = fmaxf(mx, fabsf(xa));
                            set(t, q, xv + sin_sq_small(xa) * get(ai4, q));
                        } else if constexpr (PRO == PRO_LEAKY) {
                            set(t, q, act_leaky(get(t, q), a.slope));
                        } else if constexpr (PRO == PRO_MASK) {
                            set(t, q, get(t, q) * mv[i]);
                        }
                    }
                    half4 hv;
                    hv[0] = static_cast<_Float16>(t.x);
                    hv[1] = static_cast<_Float16>(t.y);
                    hv[2] = static_cast<_Float16>(t.z);
                    hv[3] = static_cast<_Float16>(t.w);
                    *reinterpret_cast<half4*>(lds + rr * cs + cg) = hv;
                }
            }
        };
        int p0 = 0;
        for (; (p0 + kStage) * dr <= a.win; p0 += kStage) stage_batch(p0, std::false_type{});
        if (p0 * dr < a.win) stage_batch(p0, std::true_type{});
        if constexpr (PRO == PRO_SNAKE) {
            if (!(mx < kSinSmall)) *big_flag = 1;
        }
        __syncthreads();
        if constexpr (PRO == PRO_SNAKE) {
            // rare: arguments of sin at or past kSinSmall get the library
            // sinf, element by element, over the staged window
            if (*big_flag) {
                for (int e = tid; e < a.win * kch; e += NTH) {
                    const int r = e / kch, c = e - r * kch;
                    const int ti = base_t + r, ci = ci0 + c;
                    if (ti < 0 || ti >= a.t_in || ci >= a.c_in) continue;
                    const float v = reinterpret_cast<const float*>(xb + static_cast<int64_t>(ti) * a.x_nb1)[ci];
                    const float xa = v * sal[c];
                    if (fabsf(xa) < kSinSmall) continue;
                    const float sn = sinf(xa);
                    const float s2 = sn * sn;
                    const float m = s2 * sal[a.kch + c];
                    lds[r * cs + c] = static_cast<_Float16>(v + m);
                }
                __syncthreads();
            }
        }

        // steps s = k * nb + cb over this chunk's 16-channel blocks.  A of
        // tile mt at lds + arow[mt] + aoff, aoff = k*dil*cs + cb*16; B of tile
        // nt at wf[nt] + boff, boff = (k*nblk + cb0 + cb)*512.  Both offsets
        // are wave-uniform and stepped by counters (no division in the loop).
        // Each workgroup starts its sweep at its own step and wraps around
        // (the order of the f32 sum is free): workgroups that share an L2 do
        // not all fetch the same weight fragment at the same time.
        const int nb = kch / kBlk, cb0 = ci0 / kBlk;
        const int n_steps = a.k * nb;
        const int a_wrap = a.dil * cs - nb * kBlk;            // (k, nb) -> (k + 1, 0)
        const int64_t b_wrap = static_cast<int64_t>(nblk - nb) * 512;
        const int64_t b_first = static_cast<int64_t>(cb0) * 512;
        // this wave's share: n_w consecutive steps (mod n_steps) from its
        // start -- steps [s_lo, s_lo + n_w) of the chunk's, the KS shares as
        // even as the count allows (they differ by at most one; an odd share
        // runs its last step after the paired ones, PF 2 only)
        const int s_lo = ks * n_steps / KS;
        const int n_w = (ks + 1) * n_steps / KS - s_lo;
        const int s_start = static_cast<int>((j8 * 3u + static_cast<unsigned>(s_lo)) % static_cast<unsigned>(n_steps));
        const int k_start = s_start / nb, cb_start = s_start - k_start * nb;
        const int a_start = k_start * a.dil * cs + cb_start * kBlk;
        const int64_t b_start = (static_cast<int64_t>(k_start) * nblk + cb0 + cb_start) * 512;
        int k_a = k_start, cb_a = cb_start, aoff = a_start;      // A of the next step to read
        int k_b = k_start, cb_b = cb_start;
        int64_t boff = b_start;                                  // B of the next step to fetch
        auto next_a = [&]() {
            aoff += kBlk;
            if (++cb_a == nb) {
                cb_a = 0;
                aoff += a_wrap;
                if (++k_a == a.k) {
                    k_a = 0;
                    aoff = 0;
                }
            }
        };
        auto next_b = [&]() {
            boff += 512;
            if (++cb_b == nb) {
                cb_b = 0;
                boff += b_wrap;
                if (++k_b == a.k) {
                    k_b = 0;
                    boff = b_first;
                }
            }
        };
        half8 ring[PF][NT];
#pragma unroll
        for (int p = 0; p < PF; p++) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) ring[p][nt] = *reinterpret_cast<const half8*>(wf[nt] + boff);
            next_b();
        }
        half8 av[2][MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) av[0][mt] = *reinterpret_cast<const half8*>(lds + arow[mt] + aoff);
        next_a();
        const int n_pair = n_w - n_w % PF;   // the steps the ring runs in whole groups
        for (int s0 = 0; s0 < n_pair; s0 += PF) {
#pragma unroll
            for (int p = 0; p < PF; p++) {
                const int s = s0 + p;
                const int cur = p & 1;   // PF is even: the parity of s
                // A of step s + 1 (past the end: the first step's again, unused)
                const int an = s + 1 < n_w ? aoff : a_start;
#pragma unroll
                for (int mt = 0; mt < MT; mt++) av[cur ^ 1][mt] = *reinterpret_cast<const half8*>(lds + arow[mt] + an);
                next_a();
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cur][mt], ring[p][nt], acc[mt][nt], 0,
                                                                             0, 0);
                    }
                }
                // B of step s + PF (past the end: the first step's again, unused)
                const int64_t bn = s + PF < n_w ? boff : b_start;
#pragma unroll
                for (int nt = 0; nt < NT; nt++) ring[p][nt] = *reinterpret_cast<const half8*>(wf[nt] + bn);
                next_b();
            }
        }
        if constexpr (PF == 2) {
            // an odd share's last step: its A came in av[0] and its B in
            // ring[0] with the last pair (n_w is wave-uniform)
            if (n_w & 1) {
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[0][mt], ring[0][nt], acc[mt][nt], 0,
                                                                             0, 0);
                    }
                }
            }
        }
    }

    // y = (sum + bias) [+ res]: ggml_add of the bias, then the residual add.
    // Each wave parks its tile in LDS (row-major, the window is no longer
    // read), then writes whole rows: with vout, one float4 per lane, a row
    // segment of NT*32 channels per NT*8 lanes.
    __syncthreads();
    constexpr int EPS = NT * 32 + 4;   // tile row stride in floats
    float* ep = reinterpret_cast<float*>(lds) + wt * (MT * 32 * EPS);
    const int64_t yb = static_cast<int64_t>(bz) * a.y_nb2 + y_off;
    const int64_t rb = static_cast<int64_t>(bz) * a.r_nb2 + r_off;
    const int tw = t0 + wm * MT * 32, cw = co0 + wn * NT * 32;
    // vout: wave ks of the KS that share the wave tile stores NIT row groups
    // of RPI rows, one float4 per lane; its residual float4s are read before
    // the last turn's barrier, all at once (the accumulators are in LDS by
    // then), so their latency overlaps the tile exchange
    constexpr int CPR = NT * 8;                    // float4 per tile row
    constexpr int RPI = 64 / CPR;                  // tile rows per store instruction
    constexpr int NIT = MT * 32 / (RPI * KS);
    const int c4 = (lane % CPR) * 4, co4 = cw + c4, rl0 = lane / CPR + ks * RPI;
    const bool cok = co4 < a.c_out;                // c_out % 4 == 0: the whole float4
    float4 q[NIT];
    // the KS partial sums of a wave tile meet in its LDS tile: wave ks = 1
    // writes its sum, ks = 2 .. KS-1 add theirs in turn, ks = 0 adds last
    // (one barrier per turn; with KS = 1 wave 0 just writes)
#pragma unroll
    for (int turn = 1; turn <= KS; turn++) {
        if (ks == turn % KS) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        float* e = ep + (mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)) * EPS + nt * 32 + lrow;
                        *e = turn == 1 ? acc[mt][nt][r] : *e + acc[mt][nt][r];
                    }
                }
            }
        }
        if (turn == KS && a.vout && a.res) {
#pragma unroll
            for (int i = 0; i < NIT; i++) {
                const int t = tw + rl0 + i * RPI * KS;
                const int tc = t < t_out ? t : t_out - 1;
                q[i] = *reinterpret_cast<const float4*>(a.res + rb + static_cast<int64_t>(tc) * r_step +
                                                        static_cast<int64_t>(cok ? co4 : 0) * 4);
            }
        }

        __syncthreads();
    }
    if (a.vout) {
        float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.bias && cok) bv = *reinterpret_cast<const float4*>(a.bias + co4);
#pragma unroll
        for (int i = 0; i < NIT; i++) {
            const int rl = rl0 + i * RPI * KS, t = tw + rl;
            if (t < t_out && cok) {
                float4 v = *reinterpret_cast<const float4*>(ep + rl * EPS + c4);
                if (a.bias) v = make_float4(v.x + bv.x, v.y + bv.y, v.z + bv.z, v.w + bv.w);
                if (a.res) v = make_float4(q[i].x + v.x, q[i].y + v.y, q[i].z + v.z, q[i].w + v.w);
                // the ResBlock sum so far (stride-1 convs: y's rows), read here:
                // held from before the barrier like q it would cost the large
                // tiles an occupancy step, sum or not
                if (a.acc) {
                    v = sum_scale(v,
                                  *reinterpret_cast<const float4*>(a.acc + static_cast<int64_t>(bz) * a.a_nb2 +
                                                                   static_cast<int64_t>(t) * a.a_nb1 +
                                                                   static_cast<int64_t>(co4) * 4),
                                  a.oscale, a.scaled);
                }
                *reinterpret_cast<float4*>(a.y + yb + static_cast<int64_t>(t) * y_step + static_cast<int64_t>(co4) * 4) =
                    v;
            }
        }
    } else {
        for (int i = lane + ks * 64; i < MT * 32 * NT * 32; i += 64 * KS) {
            const int rl = i / (NT * 32), c = i % (NT * 32);
            const int t = tw + rl, co = cw + c;
            if (t < t_out && co < a.c_out) {
                float v = ep[rl * EPS + c];
                if (a.bias) v = v + a.bias[co];
                if (a.res) v = reinterpret_cast<const float*>(a.res + rb + static_cast<int64_t>(t) * r_step)[co] + v;
                if (a.acc) {
                    v = reinterpret_cast<const float*>(a.acc + static_cast<int64_t>(bz) * a.a_nb2 +
                                                       static_cast<int64_t>(t) * a.a_nb1)[co] + v;
                    if (a.scaled) v = v * a.oscale;
                }
                reinterpret_cast<float*>(a.y + yb + static_cast<int64_t>(t) * y_step)[co] = v;
            }
        }
    }
}

// ---- pipelined form ---------------------------------------------------------
// Long stride-1 convs (the vocoder's ResBlock convs on 48000-frame stages):
// in k_conv1d every workgroup of the launch is resident at once, so all of
// them stage their windows together (HBM busy, matrix cores idle), then run
// the MFMA loop together (HBM idle), then store together.  Here one
// workgroup per CU owns one output tile of BT = WM*MT*32 frames x BC =
// WN*NT*32 channels with 8 waves: waves 0-3 run the MFMA loop (one wave
// tile each), waves 4-7 stage the activated input window of the next
// 64-channel chunk into the other of two LDS buffers meanwhile, one
// barrier per chunk; so staging overlaps the matrix cores for all chunks
// but the first (which all 8 waves stage).  The B fragments stream from
// global memory through a register ring PF steps deep that runs on across
// chunk boundaries (the weights do not wait for the staging).  The staging
// waves read the residual while the last chunk runs, then store the tile
// (parked in LDS by the MFMA waves) as row-contiguous float4 with the bias
// and residual added.  The arithmetic per output is k_conv1d's (f16
// operands, f32 sums), in another order of the reduction's steps.
constexpr int kPipeKch = 64;          // input channels per chunk
constexpr int kPipeThreads = 512;     // 4 MFMA waves + 4 staging waves
constexpr int kPipeCs = kPipeKch + 8; // LDS row stride of a window buffer (halves)

// OCC: waves per SIMD the register budget is sized for (2: one workgroup a
// CU; 4: two, whose phases then also overlap each other's)
template <int PRO, int MT, int NT, int WM, int WN, int PF, int OCC>
__global__ __launch_bounds__(kPipeThreads) __attribute__((amdgpu_waves_per_eu(OCC))) void k_conv1d_pipe(ConvArgs a) {
    static_assert(WM * WN == 4, "four MFMA waves");
    constexpr int NB = kPipeKch / kBlk;   // 16-channel blocks per chunk
    constexpr int BT = WM * MT * 32, BC = WN * NT * 32;
    constexpr int NPT = kPipeThreads / 2;  // staging threads
    constexpr int cs = kPipeCs;
    extern __shared__ _Float16 lds[];      // two window buffers of a.win rows; then the output tile
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool stager = wave >= 4;
    // work item w of the launch, numbered as in k_conv1d (consecutive items
    // on one XCD)
    const unsigned L = blockIdx.x, n_wg = gridDim.x;
    const unsigned q8 = n_wg >> 3, r8 = n_wg & 7, xcd = L & 7, j8 = L >> 3;
    const unsigned w = xcd < r8 ? xcd * (q8 + 1) + j8 : r8 * (q8 + 1) + (xcd - r8) * q8 + j8;
    const int ct = static_cast<int>(w % static_cast<unsigned>(a.n_ct));
    const unsigned wr = w / static_cast<unsigned>(a.n_ct);
    const int tt = static_cast<int>(wr % static_cast<unsigned>(a.n_tt));
    const int bz = static_cast<int>(wr / static_cast<unsigned>(a.n_tt));
    const int t0 = tt * BT, co0 = ct * BC;
    const char* xb = a.x + static_cast<int64_t>(bz) * a.x_nb2;
    const int base_t = t0 - a.pad;           // input time of window row 0 (stride 1)
    const int buf_h = a.win * cs;            // halves per window buffer
    const int nchunks = a.c_in / kPipeKch;   // the host keeps c_in % 64 == 0
    const int nblk = a.c_in_pad / kBlk;

    // stage chunk c -- rows [base_t, base_t + win) x channels [64c, 64c + 64)
    // of pro(x) as f16 -- into buffer c & 1, with NTH threads from thread
    // tb: thread pt owns the 4-channel group cg of rows pt / 16 + (NTH/16) j.
    // The loads of a batch of KST rows are all issued before any is used
    // (rows outside x read the prepared weights, a valid address, and are
    // zeroed); a batch covers a 192-frame tile's window of a K 11 d 5 conv.
    // (the lambda captures copies of the fields it reads: a reference to the
    // by-value kernel argument would put the argument block in scratch)
    _Float16* const lds0 = lds;
    const float* const alpha = a.alpha;
    const float* const alpha_inv = a.alpha_inv;
    const float* const safe = reinterpret_cast<const float*>(a.w);
    const int win = a.win, t_in = a.t_in;
    const int64_t x_nb1 = a.x_nb1;
    const float slope = a.slope;
    auto stage = [=](int c, int tb, auto nth_c, auto kst_c) {
        constexpr int NTH = decltype(nth_c)::value, KST = decltype(kst_c)::value;
        _Float16* buf = lds0 + (c & 1) * buf_h;
        constexpr int gpr = kPipeKch / 4;    // 4-channel groups per row
        constexpr int dr = NTH / gpr;        // rows per pass
        const int pt = tid - tb;
        const int r0 = pt / gpr, cg = 4 * (pt % gpr), ci = c * kPipeKch + cg;
        float al[4] = {0.f, 0.f, 0.f, 0.f}, ai[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (PRO == PRO_SNAKE) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                al[q] = alpha[ci + q];
                ai[q] = alpha_inv[ci + q];
            }
        }
        float mx = 0.0f;   // snake: the largest |x * alpha| staged (NaN needs no fix-up: both sins give NaN)
        for (int p0 = 0; p0 * dr < win; p0 += KST) {
            float4 v[KST];
#pragma unroll
            for (int i = 0; i < KST; i++) {
                const int rr = r0 + (p0 + i) * dr, ti = base_t + rr;
                const bool ok = rr < win && ti >= 0 && ti < t_in;
                const float* row = reinterpret_cast<const float*>(xb + static_cast<int64_t>(ok ? ti : 0) * x_nb1);
                const float4 t = *reinterpret_cast<const float4*>(ok ? row + ci : safe);
                v[i] = ok ? t : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < KST; i++) {
                const int rr = r0 + (p0 + i) * dr;
                if (rr < win) {
                    float4 t = v[i];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if constexpr (PRO == PRO_SNAKE) {
                            // snake(x) = x + sin(x*a)^2 * a_inv in the reference's op order
                            const float xv = get(t, q), xa = xv * al[q];
                            mx = fmaxf(mx, fabsf(xa));
                            set(t, q, xv + sin_sq_small(xa) * ai[q]);
                        } else if constexpr (PRO == PRO_LEAKY) {
                            set(t, q, act_leaky(get(t, q), slope));
                        }
                    }
                    half4 hv;
                    hv[0] = static_cast<_Float16>(t.x);
                    hv[1] = static_cast<_Float16>(t.y);
                    hv[2] = static_cast<_Float16>(t.z);
                    hv[3] = static_cast<_Float16>(t.w);
                    *reinterpret_cast<half4*>(buf + rr * cs + cg) = hv;
                }
            }
        }
        if constexpr (PRO == PRO_SNAKE) {
            // rare: this thread's elements with an argument of sin at or past
            // kSinSmall get the library sinf (only this thread wrote them)
            if (!(mx < kSinSmall)) {
                for (int rr = r0; rr < win; rr += dr) {
                    const int ti = base_t + rr;
                    if (ti < 0 || ti >= t_in) continue;
                    const float* row = reinterpret_cast<const float*>(xb + static_cast<int64_t>(ti) * x_nb1);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const float xv = row[ci + q], xa = xv * al[q];
                        if (fabsf(xa) < kSinSmall) continue;
                        const float sn = sinf(xa);
                        const float s2 = sn * sn;
                        const float m = s2 * ai[q];
                        buf[rr * cs + cg + q] = static_cast<_Float16>(xv + m);
                    }
                }
            }
        }
    };

    // The two kinds of wave run separate loops with the same barriers (one
    // after chunk 0 is staged -- by all eight waves --, one per chunk, one
    // after the tile is parked), so the accumulators and the B ring are
    // live only in the MFMA waves' code and the staging and epilogue
    // registers only in the staging waves'.  The staging waves read the
    // residual while the last chunk runs on the matrix cores, and store the
    // tile.
    constexpr int EPS = BC + 4;                     // parked tile row stride (floats)
    constexpr int C4 = BC / 4;                      // float4 per tile row
    constexpr int NIT = BT * C4 / NPT;              // float4 of the tile per staging thread
    static_assert(NPT % C4 == 0 && (BT * C4) % NPT == 0, "staging threads cover whole rows");
    float* ep = reinterpret_cast<float*>(lds);      // over the window buffers, no longer read
    if (stager) {
        stage(0, 0, std::integral_constant<int, kPipeThreads>{}, std::integral_constant<int, 8>{});
        __syncthreads();
        const int pt = tid - NPT;
        const int c4 = 4 * (pt % C4), co = co0 + c4, rl0 = pt / C4;
        const int64_t yb = static_cast<int64_t>(bz) * a.y_nb2, rb = static_cast<int64_t>(bz) * a.r_nb2;
        for (int c = 0; c + 1 < nchunks; c++) {
            stage(c + 1, NPT, std::integral_constant<int, NPT>{}, std::integral_constant<int, 16>{});
            __syncthreads();
        }
        // the last chunk's turn: nothing to stage, the residual is read
        float4 q[NIT], q2[NIT];
        if (a.res) {
#pragma unroll
            for (int i = 0; i < NIT; i++) {
                const int t = t0 + rl0 + i * (NPT / C4);
                const int tc = t < a.t_out ? t : a.t_out - 1;
                q[i] = *reinterpret_cast<const float4*>(a.res + rb + static_cast<int64_t>(tc) * a.r_nb1 +
                                                        static_cast<int64_t>(co) * 4);
            }
        }
        if (a.acc) {   // the ResBlock sum so far, read with the residual
#pragma unroll
            for (int i = 0; i < NIT; i++) {
                const int t = t0 + rl0 + i * (NPT / C4);
                const int tc = t < a.t_out ? t : a.t_out - 1;
                q2[i] = *reinterpret_cast<const float4*>(a.acc + static_cast<int64_t>(bz) * a.a_nb2 +
                                                         static_cast<int64_t>(tc) * a.a_nb1 + static_cast<int64_t>(co) * 4);
            }
        }
        __syncthreads();
        __syncthreads();
        // y = (sum + bias) [+ res]: ggml_add of the bias, then the residual add
        const float4 bv = a.bias ? *reinterpret_cast<const float4*>(a.bias + co) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < NIT; i++) {
            const int rl = rl0 + i * (NPT / C4), t = t0 + rl;
            if (t < a.t_out) {
                float4 v = *reinterpret_cast<const float4*>(ep + rl * EPS + c4);
                if (a.bias) v = make_float4(v.x + bv.x, v.y + bv.y, v.z + bv.z, v.w + bv.w);
                if (a.res) v = make_float4(q[i].x + v.x, q[i].y + v.y, q[i].z + v.z, q[i].w + v.w);
                if (a.acc) v = sum_scale(v, q2[i], a.oscale, a.scaled);
                *reinterpret_cast<float4*>(a.y + yb + static_cast<int64_t>(t) * a.y_nb1 +
                                           static_cast<int64_t>(co) * 4) = v;
            }
        }
    } else {
        floatx16 acc[MT][NT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                for (int r = 0; r < 16; r++) acc[mt][nt][r] = 0.0f;
            }
        }
        const int wm = wave / WN, wn = wave % WN;
        const int lrow = lane & 31, lk = 8 * (lane >> 5);
        const _Float16* wf[NT];
#pragma unroll
        for (int nt = 0; nt < NT; nt++) {
            const int co_t = (co0 >> 5) + wn * NT + nt;
            wf[nt] = a.w + static_cast<int64_t>(co_t) * a.k * nblk * 512 + lane * 8;
        }
        int arow[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) arow[mt] = ((wm * MT + mt) * 32 + lrow) * cs + lk;
        // The steps in order: g = (c * K + k) * NB + blk over the chunks c,
        // taps k (from the workgroup's first tap k0, cyclically: the
        // workgroups that share an L2 start on different taps) and 16-channel
        // blocks blk; B of a step at (k * nblk + c * NB + blk) * 512.  B of
        // step g sits in ring slot g % PF, read PF steps ahead across chunk
        // boundaries (the weights do not wait for the staging); A is read
        // from LDS one step ahead within a chunk, the first step of a chunk
        // after the chunk's barrier.
        half8 ring[PF][NT];
        const int k0 = static_cast<int>(j8 % static_cast<unsigned>(a.k));
        int cB = 0, iB = 0, kB = k0, bB = 0;   // the step whose B is read next (tap kB, its iB-th)
        auto b_next = [&](int slot) {
            const int64_t off = (static_cast<int64_t>(kB) * nblk + cB * NB + bB) * 512;
#pragma unroll
            for (int nt = 0; nt < NT; nt++) ring[slot][nt] = *reinterpret_cast<const half8*>(wf[nt] + off);
            if (++bB == NB) {
                bB = 0;
                kB = kB + 1 == a.k ? 0 : kB + 1;
                if (++iB == a.k) {
                    iB = 0;
                    if (++cB == nchunks) cB = 0;   // past the last step: the first steps' again (unused)
                }
            }
        };
#pragma unroll
        for (int q = 0; q < PF; q++) b_next(q);
        stage(0, 0, std::integral_constant<int, kPipeThreads>{}, std::integral_constant<int, 8>{});
        __syncthreads();
        const _Float16* buf = lds;
        half8 av[2][MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            av[0][mt] = *reinterpret_cast<const half8*>(buf + arow[mt] + k0 * a.dil * cs);
        }
        int cA = 0, iA = 0, kA = k0, bA = 0;   // the step whose A is in av[p & 1]
        const int total = nchunks * a.k * NB;  // a multiple of PF (the host's choice)
        for (int g0 = 0; g0 < total; g0 += PF) {
#pragma unroll
            for (int p = 0; p < PF; p++) {
                const int cur = p & 1;
                int bN = bA + 1, kN = kA, iN = iA, cN = cA;
                if (bN == NB) {
                    bN = 0;
                    kN = kN + 1 == a.k ? 0 : kN + 1;
                    if (++iN == a.k) {
                        iN = 0;
                        ++cN;
                    }
                }
                const bool same = cN == cA;
                if (same) {
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        av[cur ^ 1][mt] = *reinterpret_cast<const half8*>(buf + arow[mt] + kN * a.dil * cs + bN * kBlk);
                    }
                }
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                    for (int nt = 0; nt < NT; nt++) {
                        acc[mt][nt] =
                            __builtin_amdgcn_mfma_f32_32x32x16_f16(av[cur][mt], ring[p][nt], acc[mt][nt], 0, 0, 0);
                    }
                }
                b_next(p);
                if (!same && cN < nchunks) {
                    // chunk cN begins: its window has been staged once every
                    // wave is here
                    __syncthreads();
                    buf = lds + (cN & 1) * buf_h;
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        av[cur ^ 1][mt] = *reinterpret_cast<const half8*>(buf + arow[mt] + k0 * a.dil * cs);
                    }
                }
                cA = cN;
                iA = iN;
                kA = kN;
                bA = bN;
            }
        }
        __syncthreads();
        // the tile to LDS: rows of BC + 4 floats
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = (wm * MT + mt) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    ep[row * EPS + (wn * NT + nt) * 32 + lrow] = acc[mt][nt][r];
                }
            }
        }
        __syncthreads();
    }
}

// Fragment-major f16 copy of a conv weight, zero padded: fragment (phase,
// co tile, tap, 16-channel block) is 64 lanes x 8 halves, lane l holding
// w[co_tile*32 + l%32][block*16 + 8*(l/32) + j] at that tap -- one MFMA B
// operand, one contiguous KiB.  conv1d (up == 0): ggml (K, C_in, C_out), one
// phase, tap k.  Transposed conv with stride up: ggml (K, C_out, C_in), up
// phases of `taps` taps, stored tap kp of phase ph being the weight's tap
// ph + (taps - 1 - kp)*up (zero past K).  The f16 rounding is the
// reference's conversion of an F32 weight.
struct WPrep {
    const char* w;
    int64_t nb_k, nb_ci, nb_co;   // byte strides of tap, input and output channel
    int32_t K, taps, up, c_in, c_out, nblk, co_tiles;
    int64_t total;
};

template <bool F16>
__global__ __launch_bounds__(256) void k_conv_weights(WPrep p, _Float16* out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= p.total) return;
    const int64_t frag = i >> 9;
    const int32_t lane = static_cast<int32_t>((i >> 3) & 63), j = static_cast<int32_t>(i & 7);
    const int32_t cb = static_cast<int32_t>(frag % p.nblk);
    const int64_t q = frag / p.nblk;
    const int32_t kp = static_cast<int32_t>(q % p.taps);
    const int64_t q2 = q / p.taps;
    const int32_t co_t = static_cast<int32_t>(q2 % p.co_tiles), ph = static_cast<int32_t>(q2 / p.co_tiles);
    const int32_t k = p.up == 0 ? kp : ph + (p.taps - 1 - kp) * p.up;
    const int32_t co = co_t * 32 + (lane & 31);
    const int32_t ci = cb * 16 + 8 * (lane >> 5) + j;
    _Float16 v = static_cast<_Float16>(0.0f);
    if (ci < p.c_in && co < p.c_out && k < p.K) {
        const char* e = p.w + k * p.nb_k + ci * p.nb_ci + co * p.nb_co;
        if constexpr (F16) v = __builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(e));
        else v = static_cast<_Float16>(*reinterpret_cast<const float*>(e));
    }
    out[i] = v;
}

struct Tile {
    int mt, nt, wm, wn, ks;   // ks: the most waves that share a wave tile (split of the reduction)
    int bt() const { return wm * mt * 32; }
    int bc() const { return wn * nt * 32; }
};

template <typename K>
void conv_launch(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t s, const ConvArgs& a) {
    // windows past 64 KiB use the larger LDS of gfx950 (160 KiB per
    // workgroup): raise the limit of each kernel once per device (every
    // instantiation has the same function type, so the record is keyed on
    // the kernel's address)
    if (lds > 64 * 1024) {
        static std::mutex mu;
        static std::set<std::pair<int, const void*>> raised;
        const void* fn = reinterpret_cast<const void*>(kernel);
        int dev = -1;
        (void)hipGetDevice(&dev);
        std::lock_guard<std::mutex> lock(mu);
        if (raised.count({dev, fn}) == 0 &&
            hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsMax)) ==
                hipSuccess) {
            raised.insert({dev, fn});
        }
    }
    hipLaunchKernelGGL(kernel, grid, block, lds, s, a);
}

// (VEC, PF) in {(1, 4), (1, 2), (0, 2)}: unaligned rows take the shorter ring
template <int PRO, int MT, int NT, int WM, int WN, int KS>
void conv_go(bool vec, bool pf4, dim3 grid, size_t lds, hipStream_t s, const ConvArgs& a) {
    const dim3 block(64 * WM * WN * KS);
    if (!vec) conv_launch(k_conv1d<PRO, MT, NT, WM, WN, KS, false, 2>, grid, block, lds, s, a);
    else if (pf4) conv_launch(k_conv1d<PRO, MT, NT, WM, WN, KS, true, 4>, grid, block, lds, s, a);
    else conv_launch(k_conv1d<PRO, MT, NT, WM, WN, KS, true, 2>, grid, block, lds, s, a);
}

template <int PRO, int MT, int NT, int WM, int WN, int KSMAX>
void conv_ks(int ks, bool vec, bool pf4, dim3 grid, size_t lds, hipStream_t s, const ConvArgs& a) {
    if (ks == KSMAX) conv_go<PRO, MT, NT, WM, WN, KSMAX>(vec, pf4, grid, lds, s, a);
    else if (KSMAX == 4 && ks == 2) conv_go<PRO, MT, NT, WM, WN, (KSMAX == 4 ? 2 : 1)>(vec, pf4, grid, lds, s, a);
    else conv_go<PRO, MT, NT, WM, WN, 1>(vec, pf4, grid, lds, s, a);
}

// the tile shapes below, by index
template <int PRO>
void conv_tile(int t, int ks, bool vec, bool pf4, dim3 grid, size_t lds, hipStream_t s, const ConvArgs& a) {
    switch (t) {
        case 0: conv_ks<PRO, 4, 2, 2, 1, 2>(ks, vec, pf4, grid, lds, s, a); break;   // 256 x 64
        case 1: conv_ks<PRO, 4, 2, 1, 2, 2>(ks, vec, pf4, grid, lds, s, a); break;   // 128 x 128
        case 2: conv_ks<PRO, 2, 2, 1, 2, 2>(ks, vec, pf4, grid, lds, s, a); break;   // 64 x 128
        case 3: conv_ks<PRO, 2, 2, 1, 1, 4>(ks, vec, pf4, grid, lds, s, a); break;   // 64 x 64
        case 4: conv_ks<PRO, 4, 1, 2, 1, 2>(ks, vec, pf4, grid, lds, s, a); break;   // 256 x 32
        case 5: conv_ks<PRO, 3, 2, 1, 2, 2>(ks, vec, pf4, grid, lds, s, a); break;   // 96 x 128
        case 6: conv_ks<PRO, 3, 2, 2, 1, 2>(ks, vec, pf4, grid, lds, s, a); break;   // 192 x 64
        case 7: conv_ks<PRO, 3, 2, 1, 1, 4>(ks, vec, pf4, grid, lds, s, a); break;   // 96 x 64
        case 8: conv_ks<PRO, 1, 2, 1, 1, 4>(ks, vec, pf4, grid, lds, s, a); break;   // 32 x 64
        default: conv_ks<PRO, 1, 1, 1, 1, 4>(ks, vec, pf4, grid, lds, s, a); break;  // 32 x 32
    }
}

constexpr Tile kTiles[10] = {{4, 2, 2, 1, 2}, {4, 2, 1, 2, 2}, {2, 2, 1, 2, 2}, {2, 2, 1, 1, 4}, {4, 1, 2, 1, 2},
                             {3, 2, 1, 2, 2}, {3, 2, 2, 1, 2}, {3, 2, 1, 1, 4}, {1, 2, 1, 1, 4}, {1, 1, 1, 1, 4}};

}  // namespace

// Output-channel padding of the prepared weights: a multiple of every tile width.
constexpr int kConvCoPad = 128;

int conv1d_weights_layout(int64_t c_in, int64_t c_out, int64_t* c_in_pad, int64_t* c_out_pad) {
    *c_in_pad = cdiv(c_in, kChanAlign) * kChanAlign;
    *c_out_pad = cdiv(c_out, kConvCoPad) * kConvCoPad;
    return CBX_OK;
}

int launch_conv1d_weights(const cbx_tensor* w, int up, int64_t taps, _Float16* out, int64_t c_in_pad,
                          int64_t c_out_pad, hipStream_t s) {
    WPrep p;
    p.w = static_cast<const char*>(w->data);
    p.nb_k = static_cast<int64_t>(w->nb[0]);
    // conv1d: (K, C_in, C_out); transposed: (K, C_out, C_in)
    p.nb_ci = static_cast<int64_t>(up == 0 ? w->nb[1] : w->nb[2]);
    p.nb_co = static_cast<int64_t>(up == 0 ? w->nb[2] : w->nb[1]);
    p.K = static_cast<int32_t>(w->ne[0]);
    p.taps = static_cast<int32_t>(taps);
    p.up = up;
    p.c_in = static_cast<int32_t>(up == 0 ? w->ne[1] : w->ne[2]);
    p.c_out = static_cast<int32_t>(up == 0 ? w->ne[2] : w->ne[1]);
    p.nblk = static_cast<int32_t>(c_in_pad / kBlk);
    p.co_tiles = static_cast<int32_t>(c_out_pad / 32);
    const int64_t n_ph = up == 0 ? 1 : up;
    p.total = n_ph * c_out_pad * taps * c_in_pad;   // = phases * co tiles * taps * blocks * 512
    const dim3 grid(static_cast<unsigned>(cdiv(p.total, 256)));
    if (w->type == CBX_TYPE_F16) hipLaunchKernelGGL((k_conv_weights<true>), grid, dim3(256), 0, s, p, out);
    else hipLaunchKernelGGL((k_conv_weights<false>), grid, dim3(256), 0, s, p, out);
    return check_launch("conv1d_weights");
}

int launch_conv1d(const cbx_tensor* x, const _Float16* w16, int64_t k, int64_t c_in_pad, int64_t c_out, int stride,
                  int pad, int dil, int up, int crop, int64_t w_ph, int pro, const cbx_tensor* alpha,
                  const cbx_tensor* alpha_inv, float slope, const cbx_tensor* bias, const cbx_tensor* res, cbx_tensor* y,
                  DeviceState* st, hipStream_t s, const cbx_tensor* acc, float oscale) {
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
    a.acc = acc ? static_cast<const char*>(acc->data) : nullptr;
    a.a_nb1 = acc ? static_cast<int64_t>(acc->nb[1]) : 0;
    a.a_nb2 = acc ? static_cast<int64_t>(acc->nb[2]) : 0;
    a.oscale = oscale;
    a.scaled = acc && oscale != 1.0f;
    a.c_in = static_cast<int32_t>(x->ne[0]);
    a.c_in_pad = static_cast<int32_t>(c_in_pad);
    a.c_out = static_cast<int32_t>(c_out);
    a.k = static_cast<int32_t>(k);
    a.t_in = static_cast<int32_t>(x->ne[1]);
    a.t_out = static_cast<int32_t>(y->ne[1]);
    a.stride = stride;
    a.pad = pad;
    a.dil = dil;
    a.up = up;
    a.crop = crop;
    a.w_ph = w_ph;
    a.slope = slope;
    // long stride-1 convs with K >= 3, C_in % 64 == 0 and C_out % 64 == 0
    // take the pipelined kernel: 96 x 128 tiles (128 x 64 when C_out is not a
    // multiple of 128), two workgroups a CU, when they fill the CUs' two
    // slots evenly (at least 3/4 of the slots of every round busy, and a
    // workgroup on every CU); else, with K >= 5 and C_out % 128 == 0,
    // 192 x 128 tiles one a CU on the same terms for one slot (and at least
    // half the CUs).  One workgroup a CU has too short a matrix-core phase
    // at K 3 to hide staging behind; two a CU overlap each other's
    if (up == 1 && stride == 1 && k >= 3 && (pro == PRO_NONE || pro == PRO_SNAKE || pro == PRO_LEAKY) &&
        a.c_in % kPipeKch == 0 && c_out % 64 == 0) {
        auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
        const bool one = x->ne[2] <= 1;
        const bool vec_in = al16(a.x) && a.x_nb1 % 16 == 0 && (one || a.x_nb2 % 16 == 0);
        const bool vec_out = al16(a.y) && a.y_nb1 % 16 == 0 && (one || a.y_nb2 % 16 == 0) && (!a.bias || al16(a.bias)) &&
                             (!a.res || (al16(a.res) && a.r_nb1 % 16 == 0 && (one || a.r_nb2 % 16 == 0))) &&
                             (!a.acc || (al16(a.acc) && a.a_nb1 % 16 == 0 && (one || a.a_nb2 % 16 == 0)));
        bool narrow = c_out % 128 != 0;   // 64-channel output tiles: 128 x 64, two a CU
        const int64_t n_cu = st->n_cu > 0 ? st->n_cu : 1;
        auto items_of = [&](int64_t bt, int64_t bc) {
            return cdiv(static_cast<int64_t>(a.t_out), bt) * (c_out / bc) * x->ne[2];
        };
        auto lds_of = [&](int64_t bt, int64_t bc) {
            const int64_t pwin = bt + (k - 1) * static_cast<int64_t>(dil);
            return std::max<size_t>(2 * static_cast<size_t>(pwin) * kPipeCs * sizeof(_Float16),
                                    static_cast<size_t>(bt) * (bc + 4) * sizeof(float));
        };
        // at least `need` workgroups, and every round fills 3/4 of the slots
        auto fills = [&](int64_t items, int64_t slots, int64_t need) {
            return items >= need && 4 * items >= 3 * cdiv(items, slots) * slots && items < (int64_t{1} << 31);
        };
        const int64_t t2 = narrow ? 128 : 96;   // rows of the two-a-CU tile
        const int64_t i2 = items_of(t2, narrow ? 64 : 128), i192 = items_of(192, 128);
        bool two = 2 * lds_of(t2, narrow ? 64 : 128) <= kLdsMax && fills(i2, 2 * n_cu, n_cu);
        const bool one192 = !two && !narrow && k >= 5 && fills(i192, n_cu, (n_cu + 1) / 2);
        // neither, with 128-channel multiples: 128 x 64 tiles two a CU when
        // they give every CU a workgroup, however unevenly they fill the
        // second slots (the 128 x 20000 stage of a 500-frame decode, 314
        // workgroups: K 11 24.1 -> 20.3 us, K 7 18.3 -> 17.2, K 3 14.4 ->
        // 13.7 against k_conv1d's 32 x 64 tiles)
        if (!two && !one192 && !narrow) {
            const int64_t in = items_of(128, 64);
            if (in >= n_cu && in < (int64_t{1} << 31) && 2 * lds_of(128, 64) <= kLdsMax) narrow = two = true;
        }
        const int64_t PBC = narrow ? 64 : 128;
        const int64_t PBT = two ? (narrow ? 128 : 96) : 192, items = items_of(PBT, PBC);
        const size_t plds = lds_of(PBT, PBC);
        if (vec_in && vec_out && plds <= kLdsMax && (two || one192)) {
            a.win = static_cast<int32_t>(PBT + (k - 1) * static_cast<int64_t>(dil));
            a.kch = kPipeKch;
            a.vout = 1;
            a.n_tt = static_cast<int32_t>(cdiv(static_cast<int64_t>(a.t_out), PBT));
            a.n_ct = static_cast<int32_t>(c_out / PBC);
            const dim3 grid(static_cast<unsigned>(items)), block(kPipeThreads);
            // the B ring 8 steps (two taps) deep when the step count allows
            const bool pf8 = (a.c_in / kPipeKch) * k % 2 == 0;
#define CBX_PIPE(P)                                                                                       \
    do {                                                                                                  \
        if (narrow && pf8) conv_launch(k_conv1d_pipe<P, 2, 1, 2, 2, 8, 4>, grid, block, plds, s, a);     \
        else if (narrow) conv_launch(k_conv1d_pipe<P, 2, 1, 2, 2, 4, 4>, grid, block, plds, s, a);       \
        else if (two && pf8) conv_launch(k_conv1d_pipe<P, 3, 1, 1, 4, 8, 4>, grid, block, plds, s, a);   \
        else if (two) conv_launch(k_conv1d_pipe<P, 3, 1, 1, 4, 4, 4>, grid, block, plds, s, a);          \
        else if (pf8) conv_launch(k_conv1d_pipe<P, 3, 2, 2, 2, 8, 2>, grid, block, plds, s, a);          \
        else conv_launch(k_conv1d_pipe<P, 3, 2, 2, 2, 4, 2>, grid, block, plds, s, a);                   \
    } while (0)
            switch (pro) {
                case PRO_SNAKE: CBX_PIPE(PRO_SNAKE); break;
                case PRO_LEAKY: CBX_PIPE(PRO_LEAKY); break;
                default: CBX_PIPE(PRO_NONE); break;
            }
#undef CBX_PIPE
            return check_launch("conv1d");
        }
    }
    // a transposed conv with stride up > 1 runs its up output phases as
    // stride-1 convs of ceil(T_out / up) rows each, side by side in grid z
    const int64_t batch = x->ne[2] * (up > 1 ? up : 1);
    const int64_t rows = up > 1 ? cdiv(a.t_out, up) : a.t_out;
    auto n_wg = [&](const Tile& t) { return cdiv(rows, t.bt()) * cdiv(c_out, t.bc()) * batch; };
    auto win_of = [&](const Tile& t) { return (t.bt() - 1) * static_cast<int64_t>(stride) + (k - 1) * dil + 1; };
    // the window of at least 32 channels must fit the LDS; strided convs fall back to 64-row tiles
    auto fits = [&](int64_t w) { return w * (kChanAlign + 8) * 2 + 8 * kChanAlign + 16 <= static_cast<int64_t>(kLdsMax); };
    // tile: all workgroups are resident at once (two per CU), so the launch
    // lasts as long as its busiest CU.  Score = (average output per CU /
    // the busiest CU's) x (share of the two workgroup slots per CU filled),
    // with the 4-way split tiles (small, twice the weight reads per MFMA)
    // discounted; ties go to the larger tile.  Measured on the vocoder's
    // and the CFM decoder's shapes this picks the fastest tile or one within
    // 3% of it.
    int ti = 4;
    {
        // outputs of up to 32 channels: 256 x 32 or 32 x 32 tiles (conv_post,
        // 64 -> 18 channels: 12.1 against 16.0 us on 60001 frames, 7.8
        // against 15.3 us on 2000, on 32 x 32).  (256 x 32 tiles for the 64-
        // channel upsampler: 18.1 against 21.0 us on 20000 frames in, 27.8
        // against 21.8 us on 30000 -- two uneven rounds -- not taken.)
        static constexpr int kWide[5] = {1, 5, 2, 3, 8}, kNarrow[5] = {0, 6, 7, 3, 8}, kOne[2] = {4, 9};
        const int* cand = c_out <= 32 ? kOne : c_out <= 64 ? kNarrow : kWide;
        const int n_cand = c_out <= 32 ? 2 : 5;
        const double n_cu = st->n_cu > 0 ? st->n_cu : 1;
        const double avg = static_cast<double>(rows) * static_cast<double>(c_out) * static_cast<double>(batch) / n_cu;
        double best = -1.0;
        ti = c_out <= 32 ? 4 : 3;
        for (int c = 0; c < n_cand; c++) {
            const Tile& t = kTiles[cand[c]];
            if (!fits(win_of(t))) continue;
            const double n = static_cast<double>(n_wg(t));
            const double busiest = std::ceil(n / n_cu) * t.bt() * t.bc();
            const double score = avg / busiest * std::min(1.0, n / (2.0 * n_cu)) * (t.ks == 4 ? 0.7 : 1.0);
            if (score > best + 1e-9) {
                best = score;
                ti = cand[c];
            }
        }
    }
    // 32 x 64 tiles that leave CUs without a workgroup (the CFM decoder's
    // causal convs on 500 frames: 64 or 128 of them) split each tile's
    // channels in two: [2,256,500] -> 256 6.86 against 7.6 us, [2,512,500]
    // 9.35 against 10.3 us; where 32 x 64 tiles fill the CUs the narrower
    // ones are slower (256 x 6000 K11 45 against 27.5 us)
    if (ti == 8 && n_wg(kTiles[8]) < st->n_cu) ti = 9;
    if (!fits(win_of(kTiles[ti]))) ti = 3;
    const int64_t win = win_of(kTiles[ti]);
    if (!fits(win)) {
        return set_error(CBX_ERR_UNSUPPORTED, "conv1d: one tile's input window exceeds the LDS");
    }
    // channels per chunk: all of them when they fit the LDS, else the most
    // that do, and at most 4 per thread of the workgroup (a thread stages
    // one 4-channel group of a window row per pass)
    const int64_t kch_lds = std::min<int64_t>(
        (static_cast<int64_t>(kLdsMax) / (win * 2 + 8) - 8) / kChanAlign * kChanAlign, c_in_pad);
    const Tile& t = kTiles[ti];
    // waves per wave tile (ks) and the chunks' steps (K * channels / 16)
    int64_t kch = 0, n_full = 0, n_last = 0;
    auto plan_chunks = [&](int ks_) {
        kch = std::min<int64_t>(kch_lds, 4 * 64 * t.wm * t.wn * ks_);
        const int64_t last = c_in_pad - (cdiv(c_in_pad, kch) - 1) * kch;
        n_full = k * (kch / kBlk);
        n_last = k * (last / kBlk);
    };
    auto steps_ok = [&](int ks_, int pf) { return n_full % (ks_ * pf) == 0 && n_last % (ks_ * pf) == 0; };
    // fewer waves while a chunk's steps split unevenly into shares under 8:
    // the shares may be uneven (differ by one) on the 2-deep ring, and are
    // equal multiples of 4 on the 4-deep one.  Long uneven shares keep the
    // waves (conv_pre, 80 input channels, 42 steps: 11.5 -> 6.7 us on four
    // waves against one; the CFM decoder's 320-channel causal conv, 60: 10.6
    // -> 7.6 us against two); short ones do not pay for the partial-sum
    // exchange (conv_post, 28 steps: 12.4 us on two waves, 14.2 on four)
    int ks = t.ks;
    plan_chunks(ks);
    while (ks > 1 && (std::min(n_full, n_last) < 2 * ks ||
                      (!steps_ok(ks, 2) && std::min(n_full, n_last) < 8 * ks))) {
        plan_chunks(ks /= 2);
    }
    const bool pf4 = steps_ok(ks, 4);
    a.win = static_cast<int32_t>(win);
    a.kch = static_cast<int32_t>(kch);
    // the window (+ snake's alpha, alpha_inv and flag), then the output
    // tile of every wave tile (rows of NT*32 + 4 floats) in the same memory
    const size_t win_bytes = static_cast<size_t>(win) * static_cast<size_t>(kch + 8) * sizeof(_Float16) +
                             (pro == PRO_SNAKE ? (2 * static_cast<size_t>(kch) + 4) * sizeof(float) : 0);
    const size_t out_bytes = static_cast<size_t>(t.wm * t.wn) * t.mt * 32 * (t.nt * 32 + 4) * sizeof(float);
    const size_t lds = std::max(win_bytes, out_bytes);
    const bool vec = a.c_in % 4 == 0 && reinterpret_cast<uintptr_t>(a.x) % 16 == 0 && a.x_nb1 % 16 == 0 &&
                     (x->ne[2] <= 1 || a.x_nb2 % 16 == 0);
    auto al16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool one = x->ne[2] <= 1;
    a.vout = c_out % 4 == 0 && al16(a.y) && a.y_nb1 % 16 == 0 && (one || a.y_nb2 % 16 == 0) &&
             (!a.bias || al16(a.bias)) && (!a.res || (al16(a.res) && a.r_nb1 % 16 == 0 && (one || a.r_nb2 % 16 == 0))) &&
             (!a.acc || (al16(a.acc) && a.a_nb1 % 16 == 0 && (one || a.a_nb2 % 16 == 0)));
    a.n_tt = static_cast<int32_t>(cdiv(rows, t.bt()));
    a.n_ct = static_cast<int32_t>(cdiv(c_out, t.bc()));
    const int64_t n_items = static_cast<int64_t>(a.n_tt) * a.n_ct * batch;
    if (n_items >= (int64_t{1} << 31)) return set_error(CBX_ERR_UNSUPPORTED, "conv1d: too many output tiles");
    const dim3 grid(static_cast<unsigned>(n_items));
    switch (pro) {
        case PRO_SNAKE: conv_tile<PRO_SNAKE>(ti, ks, vec, pf4, grid, lds, s, a); break;
        case PRO_LEAKY: conv_tile<PRO_LEAKY>(ti, ks, vec, pf4, grid, lds, s, a); break;
        case PRO_MASK: conv_tile<PRO_MASK>(ti, ks, vec, pf4, grid, lds, s, a); break;
        default: conv_tile<PRO_NONE>(ti, ks, vec, pf4, grid, lds, s, a); break;
    }
    return check_launch("conv1d");
}

}  // namespace cbx
