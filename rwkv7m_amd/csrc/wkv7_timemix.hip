// Fused producers and consumer of the WKV-7 call inside the RWKV-7 time mix
// (src/rwkv7m/model/nnx_model.py:592-730).
//
// Producers (nnx_model.py:630 and :683-694), per token row and head:
//   w      = -softplus(-w_raw) - 0.5
//   kk     = (k * k_k) / sqrt(sum_head (k * k_k)^2 + 1e-24)
//   k'     = k * (1 + (a - 1) * k_a)
//   neg_kk = -kk,   kka = kk * a
// Consumer (nnx_model.py:709-727): GroupNorm ln_x over each head (fp32
// statistics, E[y^2] - E[y]^2 variance clamped at 0, epsilon eps), plus the
// bonus (sum_head r * k' * r_k) * v, times the gate g:
//   out = (GN(y) + (sum_head r k' r_k) v) * g
// and the backward of both.  All four kernels are HBM-bound elementwise
// passes with one or two reductions over the N channels of a head.
//
// Data: every activation is [rows][C] (C = H * N, head h owns channels
// h*N .. h*N+N-1; rows = tokens in any order, batch-major [B, T] in the
// model), bf16 or fp32, contiguous, 16-byte aligned.  Parameters are fp32
// [C].  Arithmetic is fp32; each output is rounded to the activation dtype
// once, at its store.
//
// Work split: one thread owns 8 consecutive channels of a row (one 16-byte
// load per bf16 tensor), N/8 neighbouring lanes own a head and reduce with
// DPP lane permutations (quad_perm, row_half_mirror, row_mirror) inside
// their 16-lane row.  A block is 256 threads over a column tile of up to
// 2048 channels; narrower rows stack several rows per block.  The grid holds
// as many blocks as the device keeps resident, and each block strides over
// the rows with the next row's loads in flight while it computes the current
// one.  Transcendentals use the hardware exp2/log2/rcp/rsq instructions
// (about 1 ulp) and bf16 stores the packed round-to-nearest-even convert.
// Parameter gradients: each thread sums its channels over its rows, the
// block adds its row slots in LDS and writes one partial row of C floats per
// row group; a second kernel adds the row groups in a fixed order, so the
// result does not depend on scheduling.

#include "wkv7_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

constexpr int kVPT = 8;                       // channels per thread
constexpr int kBlock = 256;                   // threads per block
constexpr int kTileCh = kBlock * kVPT;        // channels per column tile
constexpr int kMaxGroups = 1024;              // row groups (partial rows)

struct Geom {
    int64_t rows;
    int C;      // channels per row
    int tpt;    // threads per row of one column tile
    int rpi;    // rows a block handles at once
    int ncol;   // column tiles
    int groups; // row groups (blocks per column tile)
};

// Geometry with at most kMaxGroups row groups in all; the launch may use
// fewer (what the device keeps resident), never more, so the backward's
// workspace is sized from this alone.
Geom make_geom(int64_t rows, int64_t C) {
    Geom g;
    g.rows = rows;
    g.C = int(C);
    const int ct = C < kTileCh ? int(C) : kTileCh;
    g.tpt = ct / kVPT;
    g.rpi = kBlock / g.tpt;
    if (g.rpi < 1) g.rpi = 1;
    g.ncol = int((C + kTileCh - 1) / kTileCh);
    const int64_t r = rows > 0 ? rows : 1;  // no rows: one (zero) group
    int64_t want = (r + g.rpi - 1) / g.rpi;
    int64_t cap = kMaxGroups / g.ncol;
    if (cap < 1) cap = 1;
    g.groups = int(want < cap ? want : cap);
    return g;
}

// ---------------------------------------------------------------------------
// Loads, stores, reductions, fast math
// ---------------------------------------------------------------------------

template <typename E>
struct Raw;
template <>
struct Raw<bf16_t> {
    uint4 u;
};
template <>
struct Raw<float> {
    float4 a, b;
};

__device__ __forceinline__ Raw<bf16_t> ldraw(const bf16_t* p) {
    return {*reinterpret_cast<const uint4*>(p)};
}
__device__ __forceinline__ Raw<float> ldraw(const float* p) {
    return {reinterpret_cast<const float4*>(p)[0],
            reinterpret_cast<const float4*>(p)[1]};
}

__device__ __forceinline__ void unpack(const Raw<bf16_t>& r,
                                       float (&o)[kVPT]) {
    const uint32_t w[4] = {r.u.x, r.u.y, r.u.z, r.u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ void unpack(const Raw<float>& r,
                                       float (&o)[kVPT]) {
    o[0] = r.a.x; o[1] = r.a.y; o[2] = r.a.z; o[3] = r.a.w;
    o[4] = r.b.x; o[5] = r.b.y; o[6] = r.b.z; o[7] = r.b.w;
}

__device__ __forceinline__ void ld8(const float* p, float (&o)[kVPT]) {
    unpack(ldraw(p), o);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    const f32x2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t,
                              __builtin_convertvector(f, bf16x2_t));
}

__device__ __forceinline__ void st8(bf16_t* p, const float (&x)[kVPT]) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]),
                   pack_bf16(x[4], x[5]), pack_bf16(x[6], x[7]));
}
__device__ __forceinline__ void st8(float* p, const float (&x)[kVPT]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over the TPH lanes of a head (aligned groups inside a 16-lane DPP
// row).  Each step adds a lane's partial sum to its partner's, so every lane
// of the group ends with the same bits.
template <int TPH>
__device__ __forceinline__ float head_sum(float x) {
    if (TPH >= 2) x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
    if (TPH >= 4) x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
    if (TPH >= 8) x += dpp<0x141>(x);  // row_half_mirror
    if (TPH >= 16) x += dpp<0x140>(x); // row_mirror
    return x;
}

template <int TPH>
__device__ __forceinline__ float head_sum8(const float (&x)[kVPT]) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kVPT; ++i) s += x[i];
    return head_sum<TPH>(s);
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * kLog2e);
}

// -softplus(-x) - 0.5 = min(x, 0) - log(1 + exp(-|x|)) - 0.5
__device__ __forceinline__ float decay_clamp(float x) {
    const float t = fast_exp(-fabsf(x));
    return fminf(x, 0.f) - __builtin_amdgcn_logf(1.f + t) * kLn2 - 0.5f;
}

// Thread coordinates inside the launch geometry.
struct Lane {
    int sub;      // row slot inside the block
    int c0;       // first channel
    bool active;  // owns channels (the last column tile can be partial)
    int grp;      // row group
};

__device__ __forceinline__ Lane lane_of(const Geom& g) {
    Lane l;
    const int t = threadIdx.x;
    l.sub = t / g.tpt;
    const int tile = blockIdx.x % g.ncol;
    l.grp = blockIdx.x / g.ncol;
    l.c0 = tile * kTileCh + (t % g.tpt) * kVPT;
    l.active = l.sub < g.rpi && l.c0 < g.C;
    return l;
}

// Runs body(offset, raw) over the thread's rows; the next row's NT loads
// are issued before the current row is processed.
template <typename E, int NT, typename Body>
__device__ __forceinline__ void row_loop(const Geom& g, const Lane& l,
                                         const E* const (&src)[NT],
                                         Body&& body) {
    const int64_t step = int64_t(g.groups) * g.rpi;
    int64_t row = int64_t(l.grp) * g.rpi + l.sub;
    if (row >= g.rows) return;
    Raw<E> cur[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) cur[t] = ldraw(src[t] + row * g.C + l.c0);
    while (true) {
        const int64_t nrow = row + step;
        const bool more = nrow < g.rows;
        Raw<E> nxt[NT];
        if (more) {
#pragma unroll
            for (int t = 0; t < NT; ++t)
                nxt[t] = ldraw(src[t] + nrow * g.C + l.c0);
        }
        body(row * g.C + l.c0, cur);
        if (!more) break;
#pragma unroll
        for (int t = 0; t < NT; ++t) cur[t] = nxt[t];
        row = nrow;
    }
}

// Adds the block's row slots of acc (one value per owned channel) in LDS and
// writes them as partial row `grp` of `part` ([groups][C]).
__device__ __forceinline__ void block_partial(const Geom& g, const Lane& l,
                                              const float (&acc)[kVPT],
                                              float* __restrict__ part,
                                              float* lds) {
    if (g.rpi == 1) {
        if (l.active) st8(part + int64_t(l.grp) * g.C + l.c0, acc);
        return;
    }
    __syncthreads();
    if (l.sub < g.rpi) {
#pragma unroll
        for (int i = 0; i < kVPT; ++i)
            lds[threadIdx.x * kVPT + i] = l.active ? acc[i] : 0.f;
    }
    __syncthreads();
    if (l.sub == 0 && l.active) {
        float s[kVPT];
#pragma unroll
        for (int i = 0; i < kVPT; ++i) s[i] = 0.f;
        for (int r = 0; r < g.rpi; ++r) {
            const float* q = lds + (r * g.tpt + threadIdx.x) * kVPT;
#pragma unroll
            for (int i = 0; i < kVPT; ++i) s[i] += q[i];
        }
        st8(part + int64_t(l.grp) * g.C + l.c0, s);
    }
}

// Stages the block's column tile of NP parameters in LDS (parameter p at
// prm[p * kTileCh + channel within the tile]).  The backward kernels read
// them back per row instead of holding them in registers: the registers go
// to loads in flight.
template <int NP>
__device__ __forceinline__ void stage_params(const Geom& g, const Lane& l,
                                             const float* const (&src)[NP],
                                             float* prm) {
    if (l.sub == 0 && l.active) {
        const int lt = threadIdx.x % g.tpt;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            float v[kVPT];
            ld8(src[p] + l.c0, v);
            st8(prm + p * kTileCh + lt * kVPT, v);
        }
    }
    __syncthreads();
}

// This thread's first channel in the staged tile, opaque to the optimiser
// so that per-row LDS reads of the parameters stay inside the row loop.
__device__ __forceinline__ int param_slot(const Geom& g) {
    int off = (threadIdx.x % g.tpt) * kVPT;
    asm volatile("" : "+v"(off));
    return off;
}

__device__ __forceinline__ void lds8(const float* p, float (&o)[kVPT]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// ---------------------------------------------------------------------------
// Producers
// ---------------------------------------------------------------------------

template <typename E, int TPH>
__global__ __launch_bounds__(kBlock) void tm_inputs_fwd_kernel(
    Geom g, TmInputsArgs A) {
    const Lane l = lane_of(g);
    if (!l.active) return;
    E* __restrict__ w_out = static_cast<E*>(A.w);
    E* __restrict__ k_out = static_cast<E*>(A.k_out);
    E* __restrict__ nkk_out = static_cast<E*>(A.neg_kk);
    E* __restrict__ kka_out = static_cast<E*>(A.kka);
    float kk_p[kVPT], ka_p[kVPT];
    ld8(A.k_k + l.c0, kk_p);
    ld8(A.k_a + l.c0, ka_p);
    const E* const src[3] = {static_cast<const E*>(A.w_raw),
                             static_cast<const E*>(A.k),
                             static_cast<const E*>(A.a)};
    row_loop<E, 3>(g, l, src, [&](int64_t o, const Raw<E> (&raw)[3]) {
        float x[kVPT], k[kVPT], a[kVPT];
        unpack(raw[0], x);
        unpack(raw[1], k);
        unpack(raw[2], a);
        float kk[kVPT], sq[kVPT];
#pragma unroll
        for (int i = 0; i < kVPT; ++i) {
            kk[i] = k[i] * kk_p[i];
            sq[i] = kk[i] * kk[i];
        }
        const float inv = __builtin_amdgcn_rsqf(head_sum8<TPH>(sq) + 1e-24f);
        float w[kVPT], kp[kVPT], nkk[kVPT], kka[kVPT];
#pragma unroll
        for (int i = 0; i < kVPT; ++i) {
            w[i] = decay_clamp(x[i]);
            kp[i] = k[i] * (1.f + (a[i] - 1.f) * ka_p[i]);
            const float n = kk[i] * inv;
            nkk[i] = -n;
            kka[i] = n * a[i];
        }
        st8(w_out + o, w);
        st8(k_out + o, kp);
        st8(nkk_out + o, nkk);
        st8(kka_out + o, kka);
    });
}

template <typename E, int TPH, bool DK2>
__global__ __launch_bounds__(kBlock) void tm_inputs_bwd_kernel(
    Geom g, TmInputsBwdArgs A) {
    __shared__ float prm[2 * kTileCh];  // k_k, k_a; then the partials
    const Lane l = lane_of(g);
    E* __restrict__ dx_out = static_cast<E*>(A.dw_raw);
    E* __restrict__ dk_out = static_cast<E*>(A.dk);
    E* __restrict__ da_out = static_cast<E*>(A.da);
    float acc_kk[kVPT], acc_ka[kVPT];
#pragma unroll
    for (int i = 0; i < kVPT; ++i) acc_kk[i] = acc_ka[i] = 0.f;
    const float* const psrc[2] = {A.k_k, A.k_a};
    stage_params<2>(g, l, psrc, prm);
    if (l.active) {
        constexpr int NT = DK2 ? 8 : 7;
        const E* src[NT];
        src[0] = static_cast<const E*>(A.w_raw);
        src[1] = static_cast<const E*>(A.k);
        src[2] = static_cast<const E*>(A.a);
        src[3] = static_cast<const E*>(A.dw);
        src[4] = static_cast<const E*>(A.dk_out);
        src[5] = static_cast<const E*>(A.dneg_kk);
        src[6] = static_cast<const E*>(A.dkka);
        if (DK2) src[NT - 1] = static_cast<const E*>(A.dk_out2);
        const E* const(&csrc)[NT] = src;
        row_loop<E, NT>(g, l, csrc, [&](int64_t o, const Raw<E> (&raw)[NT]) {
            float x[kVPT], k[kVPT], a[kVPT], dw[kVPT], dkp[kVPT],
                dnkk[kVPT], dkka[kVPT], kk_p[kVPT], ka_p[kVPT];
            const int ps = param_slot(g);
            lds8(prm + ps, kk_p);
            lds8(prm + kTileCh + ps, ka_p);
            unpack(raw[0], x);
            unpack(raw[1], k);
            unpack(raw[2], a);
            unpack(raw[3], dw);
            unpack(raw[4], dkp);
            unpack(raw[5], dnkk);
            unpack(raw[6], dkka);
            if (DK2) {
                float d2[kVPT];
                unpack(raw[NT - 1], d2);
#pragma unroll
                for (int i = 0; i < kVPT; ++i) dkp[i] += d2[i];
            }
            float kk0[kVPT], sq[kVPT];
#pragma unroll
            for (int i = 0; i < kVPT; ++i) {
                kk0[i] = k[i] * kk_p[i];
                sq[i] = kk0[i] * kk0[i];
            }
            const float inv =
                __builtin_amdgcn_rsqf(head_sum8<TPH>(sq) + 1e-24f);
            float n[kVPT], gk[kVPT], dot[kVPT];
#pragma unroll
            for (int i = 0; i < kVPT; ++i) {
                n[i] = kk0[i] * inv;
                gk[i] = dkka[i] * a[i] - dnkk[i];  // d loss / d kk
                dot[i] = gk[i] * n[i];
            }
            const float proj = head_sum8<TPH>(dot);
            float dx[kVPT], dk[kVPT], da[kVPT];
#pragma unroll
            for (int i = 0; i < kVPT; ++i) {
                // dw * sigmoid(-x)
                dx[i] = dw[i] * __builtin_amdgcn_rcpf(1.f + fast_exp(x[i]));
                const float dkk0 = (gk[i] - n[i] * proj) * inv;
                dk[i] = dkk0 * kk_p[i] +
                        dkp[i] * (1.f + (a[i] - 1.f) * ka_p[i]);
                da[i] = dkka[i] * n[i] + dkp[i] * k[i] * ka_p[i];
                acc_kk[i] += dkk0 * k[i];
                acc_ka[i] += dkp[i] * k[i] * (a[i] - 1.f);
            }
            st8(dx_out + o, dx);
            st8(dk_out + o, dk);
            st8(da_out + o, da);
        });
    }
    const int64_t pc = int64_t(g.groups) * g.C;
    block_partial(g, l, acc_kk, A.workspace, prm);
    block_partial(g, l, acc_ka, A.workspace + pc, prm);
}

// ---------------------------------------------------------------------------
// Consumer
// ---------------------------------------------------------------------------

template <typename E, int TPH>
__global__ __launch_bounds__(kBlock) void tm_output_fwd_kernel(
    Geom g, TmOutputArgs A) {
    const Lane l = lane_of(g);
    if (!l.active) return;
    E* __restrict__ out = static_cast<E*>(A.out);
    float rk_p[kVPT], sc_p[kVPT], bi_p[kVPT];
    ld8(A.r_k + l.c0, rk_p);
    ld8(A.scale + l.c0, sc_p);
    ld8(A.bias + l.c0, bi_p);
    const float inv_n = 1.f / float(TPH * kVPT);
    const float eps = A.eps;
    const E* const src[5] = {
        static_cast<const E*>(A.y), static_cast<const E*>(A.r),
        static_cast<const E*>(A.k), static_cast<const E*>(A.v),
        static_cast<const E*>(A.g)};
    row_loop<E, 5>(g, l, src, [&](int64_t o, const Raw<E> (&raw)[5]) {
        float y[kVPT], r[kVPT], k[kVPT], v[kVPT], gt[kVPT];
        unpack(raw[0], y);
        unpack(raw[1], r);
        unpack(raw[2], k);
        unpack(raw[3], v);
        unpack(raw[4], gt);
        float s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int i = 0; i < kVPT; ++i) {
            s1 += y[i];
            s2 += y[i] * y[i];
            s3 += r[i] * k[i] * rk_p[i];
        }
        s1 = head_sum<TPH>(s1);
        s2 = head_sum<TPH>(s2);
        s3 = head_sum<TPH>(s3);
        const float mean = s1 * inv_n;
        const float var = fmaxf(s2 * inv_n - mean * mean, 0.f);
        const float rstd = __builtin_amdgcn_rsqf(var + eps);
        float z[kVPT];
#pragma unroll
        for (int i = 0; i < kVPT; ++i)
            z[i] = ((y[i] - mean) * rstd * sc_p[i] + bi_p[i] + s3 * v[i]) *
                   gt[i];
        st8(out + o, z);
    });
}

template <typename E, int TPH>
__global__ __launch_bounds__(kBlock) void tm_output_bwd_kernel(
    Geom g, TmOutputBwdArgs A) {
    __shared__ float prm[3 * kTileCh];  // r_k, scale, bias; then partials
    const Lane l = lane_of(g);
    E* __restrict__ dy_out = static_cast<E*>(A.dy);
    E* __restrict__ dr_out = static_cast<E*>(A.dr);
    E* __restrict__ dk_out = static_cast<E*>(A.dk);
    E* __restrict__ dv_out = static_cast<E*>(A.dv);
    E* __restrict__ dg_out = static_cast<E*>(A.dg);
    float acc_rk[kVPT], acc_sc[kVPT], acc_bi[kVPT];
#pragma unroll
    for (int i = 0; i < kVPT; ++i) acc_rk[i] = acc_sc[i] = acc_bi[i] = 0.f;
    const float* const psrc[3] = {A.r_k, A.scale, A.bias};
    stage_params<3>(g, l, psrc, prm);
    if (l.active) {
        const float inv_n = 1.f / float(TPH * kVPT);
        const float eps = A.eps;
        const E* const src[6] = {
            static_cast<const E*>(A.y), static_cast<const E*>(A.r),
            static_cast<const E*>(A.k), static_cast<const E*>(A.v),
            static_cast<const E*>(A.g), static_cast<const E*>(A.dout)};
        row_loop<E, 6>(g, l, src, [&](int64_t o, const Raw<E> (&raw)[6]) {
            float y[kVPT], r[kVPT], k[kVPT], v[kVPT], gt[kVPT], d[kVPT];
            float rk_p[kVPT], sc_p[kVPT], bi_p[kVPT];
            const int ps = param_slot(g);
            lds8(prm + ps, rk_p);
            lds8(prm + kTileCh + ps, sc_p);
            lds8(prm + 2 * kTileCh + ps, bi_p);
            unpack(raw[0], y);
            unpack(raw[1], r);
            unpack(raw[2], k);
            unpack(raw[3], v);
            unpack(raw[4], gt);
            unpack(raw[5], d);
            float s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
            for (int i = 0; i < kVPT; ++i) {
                s1 += y[i];
                s2 += y[i] * y[i];
                s3 += r[i] * k[i] * rk_p[i];
            }
            s1 = head_sum<TPH>(s1);
            s2 = head_sum<TPH>(s2);
            s3 = head_sum<TPH>(s3);
            const float mean = s1 * inv_n;
            const float var = fmaxf(s2 * inv_n - mean * mean, 0.f);
            const float rstd = __builtin_amdgcn_rsqf(var + eps);
            float xh[kVPT], dz[kVPT], dg[kVPT], dv[kVPT], dxh[kVPT];
            float t1 = 0.f, t2 = 0.f, t3 = 0.f;
#pragma unroll
            for (int i = 0; i < kVPT; ++i) {
                xh[i] = (y[i] - mean) * rstd;
                const float z = xh[i] * sc_p[i] + bi_p[i] + s3 * v[i];
                dg[i] = d[i] * z;
                dz[i] = d[i] * gt[i];
                dv[i] = dz[i] * s3;
                dxh[i] = dz[i] * sc_p[i];
                t1 += dz[i] * v[i];
                t2 += dxh[i];
                t3 += dxh[i] * xh[i];
                acc_sc[i] += dz[i] * xh[i];
                acc_bi[i] += dz[i];
            }
            const float ds = head_sum<TPH>(t1);
            const float m1 = head_sum<TPH>(t2) * inv_n;
            const float m2 = head_sum<TPH>(t3) * inv_n;
            float dy[kVPT], dr[kVPT], dk[kVPT];
#pragma unroll
            for (int i = 0; i < kVPT; ++i) {
                dy[i] = rstd * (dxh[i] - m1 - xh[i] * m2);
                dr[i] = ds * k[i] * rk_p[i];
                dk[i] = ds * r[i] * rk_p[i];
                acc_rk[i] += ds * r[i] * k[i];
            }
            st8(dy_out + o, dy);
            st8(dr_out + o, dr);
            st8(dk_out + o, dk);
            st8(dv_out + o, dv);
            st8(dg_out + o, dg);
        });
    }
    const int64_t pc = int64_t(g.groups) * g.C;
    block_partial(g, l, acc_rk, A.workspace, prm);
    block_partial(g, l, acc_sc, A.workspace + pc, prm);
    block_partial(g, l, acc_bi, A.workspace + 2 * pc, prm);
}

// out[p][c] = sum over row groups of part[p][grp][c].  A block of 1024
// threads takes 64 columns; its 16 slices of 64 threads take every 16th row
// group, each thread with 8 independent running sums (so 8 loads are in
// flight), and the slices are added in LDS in slice order.  The order of
// every addition is fixed by the shape alone.
constexpr int kSumCols = 64;
constexpr int kSumSlices = 16;
constexpr int kSumThreads = kSumCols * kSumSlices;

__global__ __launch_bounds__(kSumThreads) void tm_partial_sum_kernel(
    const float* __restrict__ part, int groups, int C, int nparam,
    float* out0, float* out1, float* out2) {
    __shared__ float red[kSumSlices][kSumCols];
    const int col = threadIdx.x % kSumCols;
    const int slice = threadIdx.x / kSumCols;
    const int c = blockIdx.x * kSumCols + col;
    const int p = blockIdx.y;
    float s[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) s[u] = 0.f;
    if (c < C && p < nparam) {
        const float* q = part + int64_t(p) * groups * C + c;
        int gi = slice;
        for (; gi + 7 * kSumSlices < groups; gi += 8 * kSumSlices) {
#pragma unroll
            for (int u = 0; u < 8; ++u)
                s[u] += q[int64_t(gi + u * kSumSlices) * C];
        }
        for (; gi < groups; gi += kSumSlices) s[0] += q[int64_t(gi) * C];
    }
    red[slice][col] = ((s[0] + s[1]) + (s[2] + s[3])) +
                      ((s[4] + s[5]) + (s[6] + s[7]));
    __syncthreads();
    if (slice == 0 && c < C && p < nparam) {
        float r = 0.f;
#pragma unroll
        for (int k = 0; k < kSumSlices; ++k) r += red[k][col];
        float* out = p == 0 ? out0 : (p == 1 ? out1 : out2);
        out[c] = r;
    }
}

hipError_t finish_partials(const Geom& g, const float* part, int nparam,
                           float* o0, float* o1, float* o2,
                           hipStream_t stream) {
    dim3 grid((g.C + kSumCols - 1) / kSumCols, nparam);
    hipLaunchKernelGGL(tm_partial_sum_kernel, grid, dim3(kSumThreads), 0,
                       stream, part, g.groups, g.C, nparam, o0, o1, o2);
    return hipGetLastError();
}

// Launches kern over g, with the row groups cut to what the current device
// keeps resident (so no block waits for a second round); g.groups is
// updated to the launched count.
template <typename Args>
hipError_t launch_resident(void (*kern)(Geom, Args), Geom& g, const Args& A,
                           hipStream_t stream) {
    int dev = 0, cus = 0, per_cu = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                                  dev);
    if (e == hipSuccess)
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(kern), kBlock, 0);
    if (e != hipSuccess) return e;
    const int64_t resident = int64_t(cus) * (per_cu > 0 ? per_cu : 1);
    int64_t cap = resident / g.ncol;
    if (cap < 1) cap = 1;
    if (g.groups > cap) g.groups = int(cap);
    hipLaunchKernelGGL(kern, dim3(unsigned(g.groups) * unsigned(g.ncol)),
                       dim3(kBlock), 0, stream, g, A);
    return hipGetLastError();
}

// The kernel instance for the activation type and head size (N / 8 lanes
// per head); nullptr for an unsupported head size.
#define RWKV7M_TM_PICK(NAME, ARGS)                                        \
    template <typename E>                                                 \
    auto pick_##NAME(int tph) -> void (*)(Geom, ARGS) {                   \
        switch (tph) {                                                    \
        case 1: return NAME<E, 1>;                                        \
        case 2: return NAME<E, 2>;                                        \
        case 4: return NAME<E, 4>;                                        \
        case 8: return NAME<E, 8>;                                        \
        case 16: return NAME<E, 16>;                                      \
        default: return nullptr;                                          \
        }                                                                 \
    }
RWKV7M_TM_PICK(tm_inputs_fwd_kernel, TmInputsArgs)
RWKV7M_TM_PICK(tm_output_fwd_kernel, TmOutputArgs)
RWKV7M_TM_PICK(tm_output_bwd_kernel, TmOutputBwdArgs)
#undef RWKV7M_TM_PICK

template <typename E, bool DK2>
auto pick_inputs_bwd(int tph) -> void (*)(Geom, TmInputsBwdArgs) {
    switch (tph) {
    case 1: return tm_inputs_bwd_kernel<E, 1, DK2>;
    case 2: return tm_inputs_bwd_kernel<E, 2, DK2>;
    case 4: return tm_inputs_bwd_kernel<E, 4, DK2>;
    case 8: return tm_inputs_bwd_kernel<E, 8, DK2>;
    case 16: return tm_inputs_bwd_kernel<E, 16, DK2>;
    default: return nullptr;
    }
}

}  // namespace

int64_t timemix_workspace_floats(int64_t rows, int64_t C) {
    if (rows < 0 || C <= 0) return 0;
    return 3 * int64_t(make_geom(rows, C).groups) * C;
}

hipError_t launch_timemix_inputs(bool bf16, int N, const TmInputsArgs& A,
                                 hipStream_t stream) {
    if (A.rows == 0) return hipSuccess;
    Geom g = make_geom(A.rows, A.C);
    const int tph = N / kVPT;
    auto kern = bf16 ? pick_tm_inputs_fwd_kernel<bf16_t>(tph)
                     : pick_tm_inputs_fwd_kernel<float>(tph);
    if (!kern) return hipErrorInvalidValue;
    return launch_resident(kern, g, A, stream);
}

hipError_t launch_timemix_inputs_backward(bool bf16, int N,
                                          const TmInputsBwdArgs& A,
                                          hipStream_t stream) {
    Geom g = make_geom(A.rows, A.C);
    const int tph = N / kVPT;
    const bool dk2 = A.dk_out2 != nullptr;
    auto kern = bf16 ? (dk2 ? pick_inputs_bwd<bf16_t, true>(tph)
                            : pick_inputs_bwd<bf16_t, false>(tph))
                     : (dk2 ? pick_inputs_bwd<float, true>(tph)
                            : pick_inputs_bwd<float, false>(tph));
    if (!kern) return hipErrorInvalidValue;
    hipError_t e = launch_resident(kern, g, A, stream);
    if (e != hipSuccess) return e;
    return finish_partials(g, A.workspace, 2, A.dk_k, A.dk_a, nullptr,
                           stream);
}

hipError_t launch_timemix_output(bool bf16, int N, const TmOutputArgs& A,
                                 hipStream_t stream) {
    if (A.rows == 0) return hipSuccess;
    Geom g = make_geom(A.rows, A.C);
    const int tph = N / kVPT;
    auto kern = bf16 ? pick_tm_output_fwd_kernel<bf16_t>(tph)
                     : pick_tm_output_fwd_kernel<float>(tph);
    if (!kern) return hipErrorInvalidValue;
    return launch_resident(kern, g, A, stream);
}

hipError_t launch_timemix_output_backward(bool bf16, int N,
                                          const TmOutputBwdArgs& A,
                                          hipStream_t stream) {
    Geom g = make_geom(A.rows, A.C);
    const int tph = N / kVPT;
    auto kern = bf16 ? pick_tm_output_bwd_kernel<bf16_t>(tph)
                     : pick_tm_output_bwd_kernel<float>(tph);
    if (!kern) return hipErrorInvalidValue;
    hipError_t e = launch_resident(kern, g, A, stream);
    if (e != hipSuccess) return e;
    return finish_partials(g, A.workspace, 3, A.dr_k, A.dscale, A.dbias,
                           stream);
}

}  // namespace rwkv7m
