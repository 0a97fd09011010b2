// State-level screening read path (phase read_screening_only) for gfx950:
// the slot recurrence and the per-token read of NNXStateLevelScreening
// (src/rwkv7m/model/nnx_model.py:999-1160, helpers in
// src/rwkv7m/model/screening.py).
//
// With writes disabled the slot update does not read the slots' keys:
//   delta_t[m] = tanh(base_t + slot_term[m])      (compute_slot_delta)
//   S_{t+1}[m] = S_t[m] + mu[m] (delta_t[m] - S_t[m])
// so the whole sequence of slots is one linear recurrence per (b, m, d),
// independent across those, and the reads at every token can run in
// parallel once the slots are known.  The host projects the slots (one
// library GEMM for keys and values of every (b, t, m)) between the two
// kernels below.
//
// slot scan, forward: S_t for every step (the slots step t reads, rounded
//   to the compute dtype as the reference casts them for its projections),
//   the per-step squared update norm |mu (delta - S)|^2 summed over each
//   64-channel group, and S_T.  delta is rounded to the compute dtype, as
//   the reference materialises it.
// slot scan, backward: G_t = (1 - mu) G_{t+1} + dS_t, d pre_t = mu G_{t+1}
//   (1 - tanh^2), d mu += G_{t+1} (delta_t - S_t).
// screen_read_fwd:  one wave per token: keys and values unit-normalised,
//   sim = q . k, relevance = trim_square (or the leaky blend) times the age
//   weight, z = sum_m rel_m v_m, u = tanh_norm(z).
// screen_read_bwd:  the adjoint of the read, recomputing the forward.
//
// Lanes hold channels (d = lane + 64 j), so every load of a key, value or
// slot row is one coalesced access, and per-slot dot products are 64-lane
// sums.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

constexpr int kScreenChunk = 32;  // steps per chunk of the slot scan
constexpr int kKJ = 2;            // key channels per lane (d_k <= 128)
constexpr int kVJ = 8;  // value channels per lane (d_v <= 512)

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float lane_value(float x, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Sum over the 64 lanes of a wave (every lane active), the same bits in every
// lane: DPP butterflies inside each 16-lane row (quad_perm [1,0,3,2],
// [2,3,0,1], row_half_mirror, row_mirror), then the four row sums read from
// lanes 0, 16, 32 and 48 and added pairwise.
__device__ __forceinline__ float wave_sum(float x) {
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
    return (lane_value(x, 0) + lane_value(x, 16)) +
           (lane_value(x, 32) + lane_value(x, 48));
}

__device__ __forceinline__ float ld1(const float* p) { return *p; }
__device__ __forceinline__ float ld1(const bf16_t* p) {
    return bf16_to_f32(*p);
}
__device__ __forceinline__ void st1(float* p, float x) { *p = x; }
__device__ __forceinline__ void st1(bf16_t* p, float x) {
    *p = f32_to_bf16(x);
}
// Value after a round trip through the element type.
__device__ __forceinline__ float rnd(float x, const float*) { return x; }
__device__ __forceinline__ float rnd(float x, const bf16_t*) {
    return bf16_to_f32(f32_to_bf16(x));
}

__device__ __forceinline__ float sigm(float x) {
    return 1.f / (1.f + expf(-x));
}

// ---------------------------------------------------------------------------
// Slot recurrence
// ---------------------------------------------------------------------------

// The recurrence is affine with a constant rate per slot, so it runs in
// chunks of kScreenChunk steps, three launches per direction:
//   local:  each chunk from a zero start (forward: the chunk's end value;
//           backward: the cotangent it adds at the chunk's start);
//   carry:  one lane per (b, m, d) walks the chunks, S_end = a^n S_start +
//           local (a = 1 - mu, n = the chunk's steps), storing every chunk's
//           true start (and S_T / d S_0);
//   emit:   each chunk again from its true start, writing the per-step
//           outputs.
// Workspace (fp32): two (forward) or three (backward) arrays of
// [chunks][B][M][ds].  Every chunk of every (b, m, 64 channels) is one
// wave, so the grid has T / kScreenChunk times more waves than one walk.

// Wave -> (chunk, b, m, 64-channel group); lane -> channel.
struct ScanLane {
    int64_t b, c, bmd;  // bmd: the lane's (b, m, d) index in [B][M][ds]
    int m, dw, d, ndw;
    int64_t t0, t1;  // the chunk's steps
    bool valid, act;
};

__device__ __forceinline__ ScanLane scan_lane(const ScreenScanArgs& A) {
    ScanLane s;
    int64_t w = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    s.ndw = int((A.ds + 63) / 64);
    s.dw = int(w % s.ndw);
    w /= s.ndw;
    s.m = int(w % A.M);
    w /= A.M;
    s.b = w % A.B;
    s.c = w / A.B;
    const int64_t nc = (A.T + kScreenChunk - 1) / kScreenChunk;
    s.valid = s.c < nc;
    s.d = s.dw * 64 + lane;
    s.act = s.valid && s.d < A.ds;
    s.bmd = (s.b * A.M + s.m) * A.ds + s.d;
    s.t0 = s.c * kScreenChunk;
    s.t1 = s.t0 + kScreenChunk < A.T ? s.t0 + kScreenChunk : A.T;
    return s;
}

__device__ __forceinline__ int64_t n_bmd(const ScreenScanArgs& A) {
    return A.B * A.M * A.ds;
}

__device__ __forceinline__ int64_t n_chunks(const ScreenScanArgs& A) {
    return (A.T + kScreenChunk - 1) / kScreenChunk;
}

// forward, local: the chunk's end value from a zero start
template <typename E>
__global__ __launch_bounds__(256) void scan_fwd_local_kernel(
    ScreenScanArgs A) {
    const ScanLane s = scan_lane(A);
    if (!s.act) return;
    const E* bp = static_cast<const E*>(A.base) + s.b * A.T * A.ds + s.d;
    const float st = A.slot_term[int64_t(s.m) * A.ds + s.d];
    const float mu = A.mu[s.m];
    float bv[kScreenChunk];
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u)
        bv[u] = s.t0 + u < s.t1 ? ld1(bp + (s.t0 + u) * A.ds) : 0.f;
    float S = 0.f;
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u)
        if (s.t0 + u < s.t1) S += mu * (rnd(tanhf(bv[u] + st), bp) - S);
    A.workspace[s.c * n_bmd(A) + s.bmd] = S;
}

// forward, carry: every chunk's start; S_T
__global__ __launch_bounds__(256) void scan_fwd_carry_kernel(
    ScreenScanArgs A) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t n = n_bmd(A);
    if (i >= n) return;
    const float a = 1.f - A.mu[int((i / A.ds) % A.M)];
    const int64_t nc = n_chunks(A);
    const float* loc = A.workspace;
    float* start = A.workspace + nc * n;
    float S = A.slots0[i];
    for (int64_t c = 0; c < nc; ++c) {
        start[c * n + i] = S;
        const int64_t len = (c + 1) * kScreenChunk < A.T
                                ? kScreenChunk
                                : A.T - c * kScreenChunk;
        S = powf(a, float(len)) * S + loc[c * n + i];
    }
    A.slots_T[i] = S;
}

// forward, emit: S_t for every step of the chunk and the update norms
template <typename E>
__global__ __launch_bounds__(256) void scan_fwd_emit_kernel(
    ScreenScanArgs A) {
    const ScanLane s = scan_lane(A);
    if (!s.valid) return;
    const int64_t M = A.M, ds = A.ds, T = A.T, n = n_bmd(A);
    const E* bp = static_cast<const E*>(A.base) + s.b * T * ds + s.d;
    E* op = static_cast<E*>(A.slots_seq) + (s.b * T * M + s.m) * ds + s.d;
    float* up = A.upd2 + (s.b * T * M + s.m) * s.ndw + s.dw;
    const float st = s.act ? A.slot_term[int64_t(s.m) * ds + s.d] : 0.f;
    const float mu = A.mu[s.m];
    float bv[kScreenChunk], u2[kScreenChunk];
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u)
        bv[u] = s.act && s.t0 + u < s.t1 ? ld1(bp + (s.t0 + u) * ds) : 0.f;
    float S = s.act ? A.workspace[(n_chunks(A) + s.c) * n + s.bmd] : 0.f;
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u) {
        const int64_t t = s.t0 + u;
        const float delta = rnd(tanhf(bv[u] + st), bp);
        if (s.act && t < s.t1) st1(op + t * M * ds, S);
        const float du = mu * (delta - S);
        u2[u] = s.act ? du * du : 0.f;
        S += du;
    }
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u) u2[u] = wave_sum(u2[u]);
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int u = 0; u < kScreenChunk; ++u)
            if (s.t0 + u < s.t1) up[(s.t0 + u) * M * s.ndw] = u2[u];
    }
}

// backward, local: the cotangent a chunk adds at its start, from zero at
// its end: sum over its steps of a^(t - t0) dS_t
template <typename E>
__global__ __launch_bounds__(256) void scan_bwd_local_kernel(
    ScreenScanArgs A) {
    const ScanLane s = scan_lane(A);
    if (!s.act) return;
    const int64_t M = A.M, ds = A.ds, T = A.T;
    const E* dp =
        static_cast<const E*>(A.d_slots_seq) + (s.b * T * M + s.m) * ds + s.d;
    const float a = 1.f - A.mu[s.m];
    float dv[kScreenChunk];
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u)
        dv[u] = s.t0 + u < s.t1 ? ld1(dp + (s.t0 + u) * M * ds) : 0.f;
    float G = 0.f;
#pragma unroll
    for (int u = kScreenChunk - 1; u >= 0; --u) G = a * G + dv[u];
    A.workspace[s.c * n_bmd(A) + s.bmd] = G;
}

// backward, carry: the cotangent of S at every chunk's end; d S_0
__global__ __launch_bounds__(256) void scan_bwd_carry_kernel(
    ScreenScanArgs A) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t n = n_bmd(A);
    if (i >= n) return;
    const float a = 1.f - A.mu[int((i / A.ds) % A.M)];
    const int64_t nc = n_chunks(A);
    const float* loc = A.workspace;
    float* end = A.workspace + nc * n;
    float G = A.d_slots_T ? A.d_slots_T[i] : 0.f;
    for (int64_t c = nc - 1; c >= 0; --c) {
        end[c * n + i] = G;
        const int64_t len = (c + 1) * kScreenChunk < A.T
                                ? kScreenChunk
                                : A.T - c * kScreenChunk;
        G = powf(a, float(len)) * G + loc[c * n + i];
    }
    A.d_slots0[i] = G;
}

// backward, emit: d pre_t and the chunk's part of d mu
template <typename E>
__global__ __launch_bounds__(256) void scan_bwd_emit_kernel(
    ScreenScanArgs A) {
    const ScanLane s = scan_lane(A);
    if (!s.act) return;
    const int64_t M = A.M, ds = A.ds, T = A.T, n = n_bmd(A);
    const E* bp = static_cast<const E*>(A.base) + s.b * T * ds + s.d;
    const int64_t o0 = (s.b * T * M + s.m) * ds + s.d;
    const E* sp = static_cast<const E*>(A.slots_seq) + o0;
    const E* dp = static_cast<const E*>(A.d_slots_seq) + o0;
    float* pp = A.d_pre + o0;
    const float st = A.slot_term[int64_t(s.m) * ds + s.d];
    const float mu = A.mu[s.m];
    float bv[kScreenChunk], sv[kScreenChunk], dv[kScreenChunk];
#pragma unroll
    for (int u = 0; u < kScreenChunk; ++u) {
        const bool in = s.t0 + u < s.t1;
        const int64_t o = (s.t0 + u) * M * ds;
        bv[u] = in ? ld1(bp + (s.t0 + u) * ds) : 0.f;
        sv[u] = in ? ld1(sp + o) : 0.f;
        dv[u] = in ? ld1(dp + o) : 0.f;
    }
    float G = A.workspace[(n_chunks(A) + s.c) * n + s.bmd];
    float dmu = 0.f;
#pragma unroll
    for (int u = kScreenChunk - 1; u >= 0; --u) {
        if (s.t0 + u >= s.t1) continue;
        const float th = tanhf(bv[u] + st);
        const float delta = rnd(th, bp);
        dmu += G * (delta - sv[u]);
        pp[(s.t0 + u) * M * ds] = mu * G * (1.f - th * th);
        G = (1.f - mu) * G + dv[u];
    }
    A.workspace[(2 * n_chunks(A) + s.c) * n + s.bmd] = dmu;
}

// backward: d mu per (b, m, d), the chunks added in chunk order
__global__ __launch_bounds__(256) void scan_bwd_dmu_kernel(
    ScreenScanArgs A) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t n = n_bmd(A);
    if (i >= n) return;
    const int64_t nc = n_chunks(A);
    const float* part = A.workspace + 2 * nc * n;
    float s = 0.f;
    for (int64_t c = 0; c < nc; ++c) s += part[c * n + i];
    A.d_mu_part[i] = s;
}

// ---------------------------------------------------------------------------
// Per-token read
// ---------------------------------------------------------------------------

struct ReadMath {
    float tau, den, alpha, gamma, cap, eps;
    bool leaky;
    // relevance before the age weight, and its derivative in sim
    __device__ __forceinline__ float rel0(float sim, float* dsim) const {
        const float x = (sim - tau) / den;
        const float r = fmaxf(x, 0.f);
        float v = r * r, d = 2.f * r / den;
        if (leaky) {
            const float sg = sigm(gamma * (sim - tau));
            v = (1.f - alpha) * v + alpha * sg;
            d = (1.f - alpha) * d + alpha * gamma * sg * (1.f - sg);
        }
        *dsim = d;
        return v;
    }
    // d rel0 / d tau, given d rel0 / d sim
    __device__ __forceinline__ float dtau(float sim, float dsim) const {
        const float x = (sim - tau) / den;
        const float r = fmaxf(x, 0.f);
        float d = 2.f * r * (x - 1.f) / den;
        if (leaky) {
            const float sg = sigm(gamma * (sim - tau));
            d = (1.f - alpha) * d - alpha * gamma * sg * (1.f - sg);
        }
        (void)dsim;
        return d;
    }
};

__device__ __forceinline__ ReadMath read_math(const ScreenReadArgs& A) {
    ReadMath r;
    r.tau = *A.tau;
    r.den = 1.f - r.tau + A.trim_eps;
    r.alpha = A.leaky_alpha;
    r.gamma = A.leaky_gamma;
    r.cap = A.cap;
    r.eps = A.eps;
    r.leaky = A.leaky != 0;
    return r;
}

// One wave per token; returns false for waves past the last token.
__device__ __forceinline__ bool read_token(const ScreenReadArgs& A,
                                           int64_t* tok) {
    *tok = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    return *tok < A.B * A.T;
}

template <typename E>
__global__ __launch_bounds__(256) void screen_read_fwd_kernel(
    ScreenReadArgs A) {
    int64_t tok;
    if (!read_token(A, &tok)) return;
    const int lane = threadIdx.x & 63;
    const int dk = A.dk, dv = A.dv, M = A.M;
    const int64_t b = tok / A.T, t_tok = tok % A.T;
    const E* proj = static_cast<const E*>(A.proj) + tok * M * (dk + dv);
    const ReadMath rm = read_math(A);
    float q[kKJ];
#pragma unroll
    for (int j = 0; j < kKJ; ++j) {
        const int d = lane + 64 * j;
        q[j] = d < dk ? A.q[tok * dk + d] : 0.f;
    }
    float z[kVJ];
#pragma unroll
    for (int j = 0; j < kVJ; ++j) z[j] = 0.f;
    float rel_lane = 0.f;  // lane m keeps rel_m
    for (int m = 0; m < M; ++m) {
        const E* kp = proj + int64_t(m) * (dk + dv);
        float nk = 0.f, dot = 0.f;
#pragma unroll
        for (int j = 0; j < kKJ; ++j) {
            const int d = lane + 64 * j;
            const float k = d < dk ? ld1(kp + d) : 0.f;
            nk += k * k;
            dot += k * q[j];
        }
        nk = wave_sum(nk);
        dot = wave_sum(dot);
        const float sim = dot / sqrtf(nk + rm.eps * rm.eps);
        float dsim;
        float rel = rm.rel0(sim, &dsim);
        if (A.age_w)
            rel *= A.age_w[b * A.age_bstride + t_tok * A.age_tstride + m];
        const E* vp = kp + dk;
        float v[kVJ], nv = 0.f;
#pragma unroll
        for (int j = 0; j < kVJ; ++j) {
            const int d = lane + 64 * j;
            v[j] = d < dv ? ld1(vp + d) : 0.f;
            nv += v[j] * v[j];
        }
        float scale = rel;
        if (A.value_unit_norm)
            scale = rel / sqrtf(wave_sum(nv) + rm.eps * rm.eps);
#pragma unroll
        for (int j = 0; j < kVJ; ++j) z[j] += scale * v[j];
        if (lane == m) rel_lane = rel;
    }
    float zz = 0.f;
#pragma unroll
    for (int j = 0; j < kVJ; ++j) zz += z[j] * z[j];
    zz = wave_sum(zz);
    const float n = sqrtf(zz + rm.eps * rm.eps);
    const float s = rm.cap * tanhf(n / rm.cap) / n;
    E* u = static_cast<E*>(A.u) + tok * dv;
#pragma unroll
    for (int j = 0; j < kVJ; ++j) {
        const int d = lane + 64 * j;
        if (d < dv) st1(u + d, s * z[j]);
    }
    if (lane < M) A.rel[tok * M + lane] = rel_lane;
    if (lane == 0) {
        A.z_norm[tok] = sqrtf(zz);
        A.u_norm[tok] = s * sqrtf(zz);
    }
}

template <typename E>
__global__ __launch_bounds__(256) void screen_read_bwd_kernel(
    ScreenReadArgs A) {
    int64_t tok;
    if (!read_token(A, &tok)) return;
    const int lane = threadIdx.x & 63;
    const int dk = A.dk, dv = A.dv, M = A.M;
    const int64_t b = tok / A.T, t_tok = tok % A.T;
    const E* proj = static_cast<const E*>(A.proj) + tok * M * (dk + dv);
    E* dproj = static_cast<E*>(A.d_proj) + tok * M * (dk + dv);
    const ReadMath rm = read_math(A);
    const float eps2 = rm.eps * rm.eps;
    float q[kKJ];
#pragma unroll
    for (int j = 0; j < kKJ; ++j) {
        const int d = lane + 64 * j;
        q[j] = d < dk ? A.q[tok * dk + d] : 0.f;
    }
    // forward recompute: per-slot sim, rel0, weights (lane m keeps slot m)
    float z[kVJ];
#pragma unroll
    for (int j = 0; j < kVJ; ++j) z[j] = 0.f;
    float l_sim = 0.f, l_nk = 0.f, l_nv = 1.f, l_rel = 0.f, l_rel0 = 0.f,
          l_dsim = 0.f, l_aw = 1.f;
    for (int m = 0; m < M; ++m) {
        const E* kp = proj + int64_t(m) * (dk + dv);
        float nk = 0.f, dot = 0.f;
#pragma unroll
        for (int j = 0; j < kKJ; ++j) {
            const int d = lane + 64 * j;
            const float k = d < dk ? ld1(kp + d) : 0.f;
            nk += k * k;
            dot += k * q[j];
        }
        nk = sqrtf(wave_sum(nk) + eps2);
        const float sim = wave_sum(dot) / nk;
        float dsim;
        const float r0 = rm.rel0(sim, &dsim);
        const float aw =
            A.age_w ? A.age_w[b * A.age_bstride + t_tok * A.age_tstride + m]
                    : 1.f;
        const float rel = r0 * aw;
        const E* vp = kp + dk;
        float v[kVJ], nv = 0.f;
#pragma unroll
        for (int j = 0; j < kVJ; ++j) {
            const int d = lane + 64 * j;
            v[j] = d < dv ? ld1(vp + d) : 0.f;
            nv += v[j] * v[j];
        }
        nv = A.value_unit_norm ? sqrtf(wave_sum(nv) + eps2) : 1.f;
#pragma unroll
        for (int j = 0; j < kVJ; ++j) z[j] += (rel / nv) * v[j];
        if (lane == m) {
            l_sim = sim;
            l_nk = nk;
            l_nv = nv;
            l_rel = rel;
            l_rel0 = r0;
            l_dsim = dsim;
            l_aw = aw;
        }
    }
    // u = s(n) z:  dz = s du + (s'(n) / n) (z . du) z
    float zz = 0.f, zdu = 0.f, du[kVJ];
    const E* dup = static_cast<const E*>(A.du) + tok * dv;
#pragma unroll
    for (int j = 0; j < kVJ; ++j) {
        const int d = lane + 64 * j;
        du[j] = d < dv ? ld1(dup + d) : 0.f;
        zz += z[j] * z[j];
        zdu += z[j] * du[j];
    }
    zz = wave_sum(zz);
    zdu = wave_sum(zdu);
    const float n = sqrtf(zz + eps2);
    const float th = tanhf(n / rm.cap);
    const float s = rm.cap * th / n;
    const float sp = ((1.f - th * th) - s) / n;
    float dz[kVJ];
#pragma unroll
    for (int j = 0; j < kVJ; ++j) dz[j] = s * du[j] + (sp / n) * zdu * z[j];
    // per slot: value gradients, then relevance -> similarity -> keys, q
    float dq[kKJ];
#pragma unroll
    for (int j = 0; j < kKJ; ++j) dq[j] = 0.f;
    float dtau = 0.f;
    for (int m = 0; m < M; ++m) {
        const float sim = __shfl(l_sim, m), nk = __shfl(l_nk, m);
        const float nv = __shfl(l_nv, m), rel = __shfl(l_rel, m);
        const float r0 = __shfl(l_rel0, m), dsim0 = __shfl(l_dsim, m);
        const float aw = __shfl(l_aw, m);
        const E* kp = proj + int64_t(m) * (dk + dv);
        const E* vp = kp + dk;
        float v[kVJ], vdz = 0.f;
#pragma unroll
        for (int j = 0; j < kVJ; ++j) {
            const int d = lane + 64 * j;
            v[j] = d < dv ? ld1(vp + d) / nv : 0.f;
            vdz += v[j] * dz[j];
        }
        vdz = wave_sum(vdz);
        E* dvp = dproj + int64_t(m) * (dk + dv) + dk;
#pragma unroll
        for (int j = 0; j < kVJ; ++j) {
            const int d = lane + 64 * j;
            if (d < dv) {
                const float g = A.value_unit_norm
                                    ? rel * (dz[j] - v[j] * vdz) / nv
                                    : rel * dz[j];
                st1(dvp + d, g);
            }
        }
        const float drel = vdz + (A.d_rel ? A.d_rel[tok * M + m] : 0.f);
        const float drel0 = drel * aw;
        const float dsim = drel0 * dsim0;
        dtau += drel0 * rm.dtau(sim, dsim0);
        E* dkp = dproj + int64_t(m) * (dk + dv);
#pragma unroll
        for (int j = 0; j < kKJ; ++j) {
            const int d = lane + 64 * j;
            if (d < dk) {
                const float k = ld1(kp + d) / nk;
                st1(dkp + d, dsim * (q[j] - k * sim) / nk);
                dq[j] += dsim * k;
            }
        }
        if (lane == 0) A.g_age[tok * M + m] = drel * r0;
    }
#pragma unroll
    for (int j = 0; j < kKJ; ++j) {
        const int d = lane + 64 * j;
        if (d < dk) A.dq[tok * dk + d] = dq[j];
    }
    if (lane == 0) A.d_tau[tok] = dtau;
}

// ---------------------------------------------------------------------------
// Write phase (read_write): the slot recurrence with write screening
// ---------------------------------------------------------------------------
//
// With writes enabled the update's strength depends on the current slots
// (nnx_model.py:1103-1115):
//   k_w = unit_norm(round(S_t + slot_embed) W_kw)   (write keys)
//   rel_w = trim_square(q_w . k_w, tau_w)
//   S_{t+1} = S_t + mu max(rel_w, floor) (delta_t - S_t)
//   ages_{t+1} = rel_w > 1e-3 ? 0 : ages_t + 1
// so each (b, slot) walks the steps in order.  Two waves per (b, slot):
// wave 0 runs the steps, with the slot's channels c = lane + 64 i in
// registers and the write key's GEMV through LDS; wave 1 stages the next
// chunk of per-step inputs into the other half of a double buffer, and the
// two meet at one barrier per chunk.  Inside a step only wave 0 touches the
// step's LDS, and one wave's LDS operations complete in order, so a step
// needs no barrier.  The backward replays each step from the stored fp32
// S_t in reverse.
constexpr int kWThreads = 128;
constexpr int kWMaxCh = 16;  // channels per lane (d_slot <= 1024)
constexpr int kWLdsWeights = 16384;  // fp32 weights staged in LDS up to 64 KB
constexpr int kWStage = 2048;        // floats per staged array and buffer
constexpr int kWBatch = 16;          // loads in flight per lane when staging
constexpr int kWMaxSteps = 32;

struct alignas(16) WriteSmem {
    float sk[1024];              // the step's write-key input
    float dk[128];               // d k_raw (backward)
    float q[2][kWStage];         // write queries [u][dk]
    float x0[2][kWStage];        // forward: delta; backward: tanh
    float x1[2][kWStage];        // backward: S_t (fp32)
    float x2[2][kWStage];        // backward: d slots_seq
    float drel[2][kWMaxSteps], dage[2][kWMaxSteps];
};

// Steps per staged chunk.
__device__ __forceinline__ int write_chunk(int ds, int dk) {
    int n = kWStage / (ds > dk ? ds : dk);
    return n < kWMaxSteps ? n : kWMaxSteps;
}

// Orders the chain wave's LDS accesses across lanes: a code-motion barrier
// (the hardware keeps one wave's LDS operations in order).
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The write-key weights [ds][dk], staged in dynamic LDS (kLds) or read from
// global memory.  The choice is a template parameter so that the GEMV reads
// through LDS (or global) loads, not flat loads, which wait for the stores
// and loads still in flight as well.
template <bool kLds>
__device__ __forceinline__ const float* write_weights(const ScreenWriteArgs& A,
                                                      float* lds) {
    if constexpr (!kLds) {
        return A.kw;
    } else {
        const int n = int(A.ds) * A.dk;
        for (int i = threadIdx.x; i < n; i += kWThreads) lds[i] = A.kw[i];
        __syncthreads();
        return lds;
    }
}

// One wave stages rows [n][width] that are `stride` elements apart in global
// memory (src points at the chunk's first row) into dst[n * width] as fp32:
// batches of kWBatch loads per lane from clamped in-bounds addresses with no
// branch, so that a batch's loads are in flight together.  add (a
// per-column fp32 row, or nullptr) is added to each value, and f maps the
// sum to what is stored.
template <typename E, typename F>
__device__ __forceinline__ void stage_rows(float* dst, const E* src,
                                           int64_t stride, int n, int width,
                                           const float* add, F f, int lane) {
    const int tot = n * width;
    for (int b0 = 0; b0 < tot; b0 += 64 * kWBatch) {
        float v[kWBatch], a[kWBatch];
#pragma unroll
        for (int r = 0; r < kWBatch; ++r) {
            const int idx = b0 + lane + 64 * r;
            const int ic = idx < tot ? idx : tot - 1;
            const int u = ic / width;
            const int col = ic - u * width;
            v[r] = ld1(src + u * stride + col);
            a[r] = add ? add[col] : 0.f;
        }
#pragma unroll
        for (int r = 0; r < kWBatch; ++r) {
            const int idx = b0 + lane + 64 * r;
            if (idx < tot) dst[idx] = f(v[r] + a[r]);
        }
    }
}

// k_raw[j] = sum_c sk[c] W[c][j] for j = lane, lane + 64 (eight running
// sums over c mod 8, added pairwise), rounded to the element type; 0 for
// j >= dk.  The forward and the backward call this same code, so both see
// the same key bits.
template <typename E>
__device__ __forceinline__ void write_gemv(const float* W, const float* sk,
                                           int ds, int dk, int lane,
                                           float (&k)[2]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        k[h] = 0.f;
        if (64 * h >= dk) continue;
        const int j = lane + 64 * h;
        const int jc = j < dk ? j : dk - 1;
        float a[8] = {};
        int c = 0;
        for (; c + 8 <= ds; c += 8) {
            float w[8], x[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) w[r] = W[(c + r) * dk + jc];
#pragma unroll
            for (int r = 0; r < 8; ++r) x[r] = sk[c + r];
#pragma unroll
            for (int r = 0; r < 8; ++r) a[r] += x[r] * w[r];
        }
        for (; c < ds; ++c) a[0] += sk[c] * W[c * dk + jc];
        const float v = ((a[0] + a[1]) + (a[2] + a[3])) +
                        ((a[4] + a[5]) + (a[6] + a[7]));
        k[h] = j < dk ? rnd(v, static_cast<const E*>(nullptr)) : 0.f;
    }
}

// The same GEMV with the lane's weight column W[0..127][lane] in registers
// (d_slot <= 128, dk <= 64; rows past d_slot hold zeros, and so does sk).
constexpr int kWRegC = 128;

template <typename E>
__device__ __forceinline__ void write_gemv_reg(const float (&wr)[kWRegC],
                                               const float* sk, int dk,
                                               int lane, float (&k)[2]) {
    float a[8] = {};
#pragma unroll
    for (int c = 0; c < kWRegC; c += 8) {
        float x[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) x[r] = sk[c + r];
#pragma unroll
        for (int r = 0; r < 8; ++r) a[r] += x[r] * wr[c + r];
    }
    const float v = ((a[0] + a[1]) + (a[2] + a[3])) +
                    ((a[4] + a[5]) + (a[6] + a[7]));
    k[0] = lane < dk ? rnd(v, static_cast<const E*>(nullptr)) : 0.f;
    k[1] = 0.f;
}

// Loads the lane's weight column for write_gemv_reg and clears sk (its
// channels past d_slot are read as zeros).
template <bool kReg>
__device__ __forceinline__ void write_reg_init(const float* W, int ds, int dk,
                                               int lane, float* wr,
                                               float* sk) {
    if constexpr (kReg) {
        const int jc = lane < dk ? lane : dk - 1;
#pragma unroll
        for (int c = 0; c < kWRegC; ++c)
            wr[c] = c < ds ? W[c * dk + jc] : 0.f;
    }
    for (int i = threadIdx.x; i < 1024; i += kWThreads) sk[i] = 0.f;
}

// d s_key[c] = sum_j W[c][j] dk[j] for this lane's channel c.  Lanes hold
// different channels, so each lane starts its sum at its own column block
// (lane mod 16 blocks of four) and the LDS reads of W rows spread over the
// banks; with dk a multiple of 4 the rows are read 16 bytes at a time.
__device__ __forceinline__ float write_gemv_t(const float* W,
                                              const float* dkv, int c, int dk,
                                              int lane) {
    float a[4] = {};
    if ((dk & 3) == 0) {
        const int n4 = dk >> 2;
        const int r4 = (lane & 15) % n4;
        const float4* w4 = reinterpret_cast<const float4*>(W + c * dk);
        const float4* d4 = reinterpret_cast<const float4*>(dkv);
        int j = 0;
        for (; j + 4 <= n4; j += 4) {
            float4 w[4], d[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                int x = r4 + j + r;
                x = x >= n4 ? x - n4 : x;
                w[r] = w4[x];
                d[r] = d4[x];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                a[0] += w[r].x * d[r].x;
                a[1] += w[r].y * d[r].y;
                a[2] += w[r].z * d[r].z;
                a[3] += w[r].w * d[r].w;
            }
        }
        for (; j < n4; ++j) {
            int x = r4 + j;
            x = x >= n4 ? x - n4 : x;
            const float4 w = w4[x], d = d4[x];
            a[0] += w.x * d.x;
            a[1] += w.y * d.y;
            a[2] += w.z * d.z;
            a[3] += w.w * d.w;
        }
    } else {
        const int r0 = lane % dk;
        for (int j = 0; j < dk; ++j) {
            int x = r0 + j;
            x = x >= dk ? x - dk : x;
            a[j & 3] += W[c * dk + x] * dkv[x];
        }
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

template <typename E, bool kLds, bool kReg>
__global__ __launch_bounds__(kWThreads)
__attribute__((amdgpu_waves_per_eu(1, 1))) void screen_write_fwd_kernel(
    ScreenWriteArgs A) {
    __shared__ WriteSmem sm;
    extern __shared__ __align__(16) float wlds[];
    const float* W = write_weights<kLds>(A, wlds);
    const int tid = threadIdx.x, lane = tid & 63;
    const bool chain = tid < 64;  // wave 0: the steps; wave 1: staging
    // channels per lane: at most 2 with the weights in registers
    // (d_slot <= 128)
    constexpr int NCH = kReg ? 2 : kWMaxCh;
    float wr[kReg ? kWRegC : 1];
    write_reg_init<kReg>(W, int(A.ds), A.dk, lane, wr, sm.sk);
    const int64_t b = blockIdx.x / A.M;
    const int m = int(blockIdx.x % A.M);
    const int64_t T = A.T, M = A.M;
    const int ds = int(A.ds), dk = A.dk;
    const E* base = static_cast<const E*>(A.base) + b * T * ds;
    const float* qw = A.q_w + b * T * dk;
    const float* st_m = A.slot_term + m * ds;
    E* seq = static_cast<E*>(A.slots_seq);
    const float mu = A.mu[m], tau = *A.tau_w;
    const float den = 1.f - tau + A.eps;
    const int chunk = write_chunk(ds, dk);
    const int64_t nchunks = (T + chunk - 1) / chunk;
    auto stage = [&](int64_t ci) {
        const int64_t t0 = ci * chunk;
        const int n = int(T - t0 < chunk ? T - t0 : chunk);
        const int buf = int(ci & 1);
        // delta_t = round(tanh(base_t + slot_term))
        stage_rows(sm.x0[buf], base + t0 * ds, ds, n, ds, st_m,
                   [&](float x) { return rnd(tanhf(x), base); }, lane);
        stage_rows(sm.q[buf], qw + t0 * dk, dk, n, dk, nullptr,
                   [](float x) { return x; }, lane);
    };
    float S[NCH], e[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        const bool in = chain && c < ds;
        S[i] = in ? A.slots0[(b * M + m) * ds + c] : 0.f;
        e[i] = in ? A.slot_embed[m * ds + c] : 0.f;
    }
    float age = A.ages0[b * M + m];
    if (!chain && nchunks > 0) stage(0);
    __syncthreads();
    for (int64_t ci = 0; ci < nchunks; ++ci) {
        if (!chain) {
            if (ci + 1 < nchunks) stage(ci + 1);
        } else {
            const int buf = int(ci & 1);
            const int64_t t0 = ci * chunk;
            const int n = int(T - t0 < chunk ? T - t0 : chunk);
            const float* dl = sm.x0[buf];
            const float* qs = sm.q[buf];
            for (int u = 0; u < n; ++u) {
                const int64_t t = t0 + u;
                // the step's staged inputs, read before the fence so that
                // their latency overlaps the GEMV
                float qv[2], dlt[NCH];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = lane + 64 * h;
                    qv[h] = j < dk ? qs[u * dk + j] : 0.f;
                }
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    dlt[i] = 0.f;
                    if (64 * i >= ds) break;
                    const int c = lane + 64 * i;
                    if (c < ds) {
                        dlt[i] = dl[u * ds + c];
                        sm.sk[c] = rnd(S[i] + e[i], base);
                    }
                }
                wave_sync();
                float k[2];
                if constexpr (kReg)
                    write_gemv_reg<E>(wr, sm.sk, dk, lane, k);
                else
                    write_gemv<E>(W, sm.sk, ds, dk, lane, k);
                float kk = 0.f, dot = 0.f;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = lane + 64 * h;
                    kk += k[h] * k[h];
                    dot += j < dk ? k[h] * qv[h] : 0.f;
                }
                kk = wave_sum(kk);
                dot = wave_sum(dot);
                const float sim = dot / sqrtf(kk + A.eps * A.eps);
                const float x = fmaxf((sim - tau) / den, 0.f);
                const float rw = x * x;
                const int64_t row = (b * T + t) * M + m;
                if (lane == 0) {
                    A.rel_w[row] = rw;
                    A.ages_seq[row] = age;
                }
                age = rw > 1e-3f ? 0.f : age + 1.f;
                const float strength = mu * fmaxf(rw, A.floor);
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    if (64 * i >= ds) break;
                    const int c = lane + 64 * i;
                    const bool in = c < ds;
                    if (in) {
                        st1(seq + row * ds + c, S[i]);
                        A.slots32[row * ds + c] = S[i];
                    }
                    const float u_ = in ? strength * (dlt[i] - S[i]) : 0.f;
                    const float u2 = wave_sum(u_ * u_);
                    if (lane == 0) A.upd2[row * ((ds + 63) / 64) + i] = u2;
                    S[i] += u_;
                }
                wave_sync();  // this step's GEMV reads come before the next
                              // step's writes of sk
            }
        }
        __syncthreads();  // chunk ci is read, chunk ci + 1 is staged
    }
    if (chain) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = lane + 64 * i;
            if (c < ds) A.slots_T[(b * M + m) * ds + c] = S[i];
        }
        if (lane == 0) A.ages_T[b * M + m] = age;
    }
}

template <typename E, bool kLds, bool kReg>
__global__ __launch_bounds__(kWThreads)
__attribute__((amdgpu_waves_per_eu(1, 1))) void screen_write_bwd_kernel(
    ScreenWriteArgs A) {
    __shared__ WriteSmem sm;
    extern __shared__ __align__(16) float wlds[];
    const float* W = write_weights<kLds>(A, wlds);
    const int tid = threadIdx.x, lane = tid & 63;
    const bool chain = tid < 64;  // wave 0: the steps; wave 1: staging
    // channels per lane: at most 2 with the weights in registers
    // (d_slot <= 128)
    constexpr int NCH = kReg ? 2 : kWMaxCh;
    float wr[kReg ? kWRegC : 1];
    write_reg_init<kReg>(W, int(A.ds), A.dk, lane, wr, sm.sk);
    // with kReg also the rows W[lane + 64 i][0..63] of the lane's channels,
    // for the transposed GEMV (sm.dk past dk reads as zero)
    float wt[kReg ? 2 : 1][kReg ? 64 : 1];
    if constexpr (kReg) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = lane + 64 * i;
#pragma unroll
            for (int j = 0; j < 64; ++j)
                wt[i][j] = c < int(A.ds) && j < A.dk ? W[c * A.dk + j] : 0.f;
        }
    }
    for (int j = threadIdx.x; j < 128; j += kWThreads) sm.dk[j] = 0.f;
    const int64_t b = blockIdx.x / A.M;
    const int m = int(blockIdx.x % A.M);
    const int64_t T = A.T, M = A.M;
    const int ds = int(A.ds), dk = A.dk;
    const E* base = static_cast<const E*>(A.base) + b * T * ds;
    const float* st_m = A.slot_term + m * ds;
    // per-(b, slot) bases: row (b, t, m) of a [B][T][M][x] array is
    // t * M * x past them
    const int64_t bm0 = b * T * M + m;
    const float* s32_bm = A.slots32 + bm0 * ds;
    const E* dseq_bm = static_cast<const E*>(A.d_slots_seq) + bm0 * ds;
    const float* qw_b = A.q_w + b * T * dk;
    float* dpre_bm = A.d_pre + bm0 * ds;
    float* dqw_bm = A.dq_w + bm0 * dk;
    float* dkraw_bm = A.d_kraw + bm0 * dk;
    float* dtau_bm = A.d_tau_w + bm0;
    const int64_t Mds = M * ds, Mdk = M * dk;
    const float mu = A.mu[m], tau = *A.tau_w;
    const float den = 1.f - tau + A.eps;
    const int chunk = write_chunk(ds, dk);
    const int64_t nchunks = (T + chunk - 1) / chunk;
    auto stage = [&](int64_t ci) {
        const int64_t t0 = ci * chunk;
        const int n = int(T - t0 < chunk ? T - t0 : chunk);
        const int buf = int(ci & 1);
        const int64_t row0 = bm0 + t0 * M;  // (b, t0, m)
        const auto id = [](float x) { return x; };
        stage_rows(sm.x0[buf], base + t0 * ds, ds, n, ds, st_m,
                   [](float x) { return tanhf(x); }, lane);
        stage_rows(sm.x1[buf], s32_bm + t0 * Mds, Mds, n, ds, nullptr, id,
                   lane);
        stage_rows(sm.x2[buf], dseq_bm + t0 * Mds, Mds, n, ds, nullptr, id,
                   lane);
        stage_rows(sm.q[buf], qw_b + t0 * dk, dk, n, dk, nullptr, id, lane);
        if (lane < n) {
            sm.drel[buf][lane] = A.d_rel_w ? A.d_rel_w[row0 + lane * M] : 0.f;
            sm.dage[buf][lane] =
                A.d_ages_seq ? A.d_ages_seq[row0 + lane * M] : 0.f;
        }
    };
    float G[NCH], e[NCH], de[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + 64 * i;
        const bool in = chain && c < ds;
        G[i] = in && A.d_slots_T ? A.d_slots_T[(b * M + m) * ds + c] : 0.f;
        e[i] = in ? A.slot_embed[m * ds + c] : 0.f;
        de[i] = 0.f;
    }
    float dage = A.d_ages_T ? A.d_ages_T[b * M + m] : 0.f;
    float dmu = 0.f;
    if (!chain && nchunks > 0) stage(nchunks - 1);
    __syncthreads();
    for (int64_t ci = nchunks - 1; ci >= 0; --ci) {
        if (!chain) {
            if (ci > 0) stage(ci - 1);
        } else {
            const int buf = int(ci & 1);
            const int64_t t0 = ci * chunk;
            const int n = int(T - t0 < chunk ? T - t0 : chunk);
            for (int u = n - 1; u >= 0; --u) {
                const int64_t tt = t0 + u;
                float th[NCH] = {}, dsv[NCH] = {};
                float qv[2];
                // the step's staged inputs, read before the fence so that
                // their latency overlaps the GEMV
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = lane + 64 * h;
                    qv[h] = j < dk ? sm.q[buf][u * dk + j] : 0.f;
                }
                const float drel_u = sm.drel[buf][u];
                const float dage_u = sm.dage[buf][u];
                float part = 0.f;  // sum_c G (delta - S), this lane's part
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    if (64 * i >= ds) break;
                    const int c = lane + 64 * i;
                    if (c < ds) {
                        const float S = sm.x1[buf][u * ds + c];
                        th[i] = sm.x0[buf][u * ds + c];
                        dsv[i] = sm.x2[buf][u * ds + c];
                        part += G[i] * (rnd(th[i], base) - S);
                        sm.sk[c] = rnd(S + e[i], base);
                    }
                }
                const float dstr = wave_sum(part);
                wave_sync();
                float k[2];
                if constexpr (kReg)
                    write_gemv_reg<E>(wr, sm.sk, dk, lane, k);
                else
                    write_gemv<E>(W, sm.sk, ds, dk, lane, k);
                float kk = 0.f, dot = 0.f;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    kk += k[h] * k[h];
                    dot += k[h] * qv[h];
                }
                const float kn = sqrtf(wave_sum(kk) + A.eps * A.eps);
                const float sim = wave_sum(dot) / kn;
                const float x = (sim - tau) / den;
                const float r = fmaxf(x, 0.f);
                const float rw = r * r;
                const bool above = rw > A.floor;
                dmu += dstr * fmaxf(rw, A.floor);
                const float drw = drel_u + (above ? dstr * mu : 0.f);
                const float dsim = drw * 2.f * r / den;
                // d k_hat = dsim q;
                // d k_raw = (d k_hat - k_hat (k_hat . d k_hat)) / kn
                float kh[2], kd = 0.f;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    kh[h] = k[h] / kn;
                    kd += kh[h] * qv[h];
                }
                kd = wave_sum(kd) * dsim;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int j = lane + 64 * h;
                    const float dkr = (dsim * qv[h] - kh[h] * kd) / kn;
                    if (j < dk) {
                        dqw_bm[tt * Mdk + j] = dsim * kh[h];
                        dkraw_bm[tt * Mdk + j] = dkr;
                        sm.dk[j] = dkr;
                    }
                }
                if (lane == 0)
                    dtau_bm[tt * M] = drw * 2.f * r * (x - 1.f) / den;
                const float strength = mu * fmaxf(rw, A.floor);
                // ages: step t read ages_t; ages_{t+1} = rw > 1e-3 ? 0 :
                // ages_t + 1
                dage = dage_u + (rw > 1e-3f ? 0.f : dage);
                wave_sync();
                float dskr[2] = {};
                if constexpr (kReg) {
                    // d s_key for both channels of the lane, dk read as
                    // broadcasts 16 bytes at a time
                    float a0[4] = {}, a1[4] = {};
#pragma unroll
                    for (int j = 0; j < 64; j += 4) {
                        const float4 d =
                            *reinterpret_cast<const float4*>(sm.dk + j);
                        a0[0] += wt[0][j] * d.x;
                        a0[1] += wt[0][j + 1] * d.y;
                        a0[2] += wt[0][j + 2] * d.z;
                        a0[3] += wt[0][j + 3] * d.w;
                        a1[0] += wt[1][j] * d.x;
                        a1[1] += wt[1][j + 1] * d.y;
                        a1[2] += wt[1][j + 2] * d.z;
                        a1[3] += wt[1][j + 3] * d.w;
                    }
                    dskr[0] = (a0[0] + a0[1]) + (a0[2] + a0[3]);
                    dskr[1] = (a1[0] + a1[1]) + (a1[2] + a1[3]);
                }
#pragma unroll
                for (int i = 0; i < NCH; ++i) {
                    if (64 * i >= ds) break;
                    const int c = lane + 64 * i;
                    if (c >= ds) continue;
                    float dsk;
                    if constexpr (kReg)
                        dsk = dskr[i < 2 ? i : 0];
                    else
                        dsk = write_gemv_t(W, sm.dk, c, dk, lane);
                    de[i] += dsk;
                    dpre_bm[tt * Mds + c] =
                        strength * G[i] * (1.f - th[i] * th[i]);
                    G[i] = G[i] * (1.f - strength) + dsk + dsv[i];
                }
                wave_sync();  // this step's reads of sk and dk come before
                              // the next step's writes
            }
        }
        __syncthreads();  // chunk ci is read, chunk ci - 1 is staged
    }
    if (chain) {
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = lane + 64 * i;
            if (c < ds) {
                A.d_slots0[(b * M + m) * ds + c] = G[i];
                A.d_embed_part[(b * M + m) * ds + c] = de[i];
            }
        }
        if (lane == 0) {
            A.d_ages0[b * M + m] = dage;
            A.d_mu_bm[b * M + m] = dmu;
        }
    }
}

template <typename E, bool kLds, bool kReg>
void launch_write(bool backward, const ScreenWriteArgs& A, size_t lds,
                  hipStream_t stream) {
    const dim3 grid{unsigned(A.B * A.M)}, block{unsigned(kWThreads)};
    if (backward)
        hipLaunchKernelGGL((screen_write_bwd_kernel<E, kLds, kReg>), grid,
                           block, lds, stream, A);
    else
        hipLaunchKernelGGL((screen_write_fwd_kernel<E, kLds, kReg>), grid,
                           block, lds, stream, A);
}

// Weights in registers for d_slot <= 128 and dk <= 64 (the forward then
// reads them once from global memory; the backward's transposed GEMV still
// reads rows from LDS), else through LDS when they fit, else from global.
template <typename E>
void launch_write_e(bool backward, const ScreenWriteArgs& A,
                    hipStream_t stream) {
    const int64_t nw = A.ds * A.dk;
    const bool reg = A.ds <= kWRegC && A.dk <= 64;
    const bool in_lds = nw <= kWLdsWeights && (backward || !reg);
    const size_t lds = in_lds ? size_t(nw) * sizeof(float) : 0;
    if (reg) {
        if (in_lds) launch_write<E, true, true>(backward, A, lds, stream);
        else launch_write<E, false, true>(backward, A, lds, stream);
    } else {
        if (in_lds) launch_write<E, true, false>(backward, A, lds, stream);
        else launch_write<E, false, false>(backward, A, lds, stream);
    }
}

unsigned blocks_for_waves(int64_t waves) {
    return unsigned((waves + 3) / 4);  // 4 waves of 64 per 256-thread block
}

}  // namespace

int64_t screen_scan_workspace_floats(int64_t B, int64_t T, int64_t M,
                                     int64_t ds) {
    const int64_t nc = (T + kScreenChunk - 1) / kScreenChunk;
    return 3 * (nc > 0 ? nc : 1) * B * M * ds;
}

hipError_t launch_screen_scan(bool bf16, bool backward,
                              const ScreenScanArgs& A, hipStream_t stream) {
    const int64_t n = A.B * A.M * A.ds;
    if (n == 0) return hipSuccess;
    const int64_t nc = (A.T + kScreenChunk - 1) / kScreenChunk;
    const dim3 block(256), grid_n(unsigned((n + 255) / 256));
    const dim3 grid_c(blocks_for_waves(nc * A.B * A.M * ((A.ds + 63) / 64)));
#define RWKV7M_SC(K)                                                      \
    do {                                                                  \
        if (bf16)                                                         \
            hipLaunchKernelGGL(K<bf16_t>, grid_c, block, 0, stream, A);   \
        else                                                              \
            hipLaunchKernelGGL(K<float>, grid_c, block, 0, stream, A);    \
    } while (0)
    if (!backward) {
        if (nc > 0) RWKV7M_SC(scan_fwd_local_kernel);
        hipLaunchKernelGGL(scan_fwd_carry_kernel, grid_n, block, 0, stream, A);
        if (nc > 0) RWKV7M_SC(scan_fwd_emit_kernel);
    } else {
        if (nc > 0) RWKV7M_SC(scan_bwd_local_kernel);
        hipLaunchKernelGGL(scan_bwd_carry_kernel, grid_n, block, 0, stream, A);
        if (nc > 0) RWKV7M_SC(scan_bwd_emit_kernel);
        hipLaunchKernelGGL(scan_bwd_dmu_kernel, grid_n, block, 0, stream, A);
    }
#undef RWKV7M_SC
    return hipGetLastError();
}

hipError_t launch_screen_write(bool bf16, bool backward,
                               const ScreenWriteArgs& A, hipStream_t stream) {
    if (A.B * A.M == 0) return hipSuccess;
    if (bf16)
        launch_write_e<bf16_t>(backward, A, stream);
    else
        launch_write_e<float>(backward, A, stream);
    return hipGetLastError();
}

hipError_t launch_screen_read(bool bf16, bool backward,
                              const ScreenReadArgs& A, hipStream_t stream) {
    const int64_t waves = A.B * A.T;
    if (waves == 0) return hipSuccess;
    const dim3 grid(blocks_for_waves(waves)), block(256);
    if (!backward) {
        if (bf16)
            hipLaunchKernelGGL(screen_read_fwd_kernel<bf16_t>, grid, block, 0,
                               stream, A);
        else
            hipLaunchKernelGGL(screen_read_fwd_kernel<float>, grid, block, 0,
                               stream, A);
    } else {
        if (bf16)
            hipLaunchKernelGGL(screen_read_bwd_kernel<bf16_t>, grid, block, 0,
                               stream, A);
        else
            hipLaunchKernelGGL(screen_read_bwd_kernel<float>, grid, block, 0,
                               stream, A);
    }
    return hipGetLastError();
}

}  // namespace rwkv7m
