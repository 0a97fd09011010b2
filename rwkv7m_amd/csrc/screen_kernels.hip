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
// screen_scan_fwd:  one lane per (b, m, d) walks t = 0 .. T-1 and writes
//   S_t (the slots step t reads, rounded to the compute dtype as the
//   reference casts them for its projections), the per-step squared update
//   norm |mu (delta - S)|^2 summed over each 64-channel wave, and S_T.
//   delta is rounded to the compute dtype, as the reference materialises it.
// screen_scan_bwd:  the reverse walk: G_t = (1 - mu) G_{t+1} + dS_t,
//   d pre_t = mu G_{t+1} (1 - tanh^2), d mu += G_{t+1} (delta_t - S_t).
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

constexpr int kKJ = 2;  // key channels per lane (d_k <= 128)
constexpr int kVJ = 8;  // value channels per lane (d_v <= 512)

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
    return x;
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

// Wave -> (b, m, 64-channel group); lane -> channel.
struct ScanLane {
    int64_t b;
    int m, dw, d, ndw;
    bool valid, act;
};

__device__ __forceinline__ ScanLane scan_lane(const ScreenScanArgs& A) {
    ScanLane s;
    const int64_t w = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    s.ndw = int((A.ds + 63) / 64);
    s.dw = int(w % s.ndw);
    const int64_t bm = w / s.ndw;
    s.m = int(bm % A.M);
    s.b = bm / A.M;
    s.valid = s.b < A.B;
    s.d = s.dw * 64 + lane;
    s.act = s.valid && s.d < A.ds;
    return s;
}

template <typename E>
__global__ __launch_bounds__(256) void screen_scan_fwd_kernel(
    ScreenScanArgs A) {
    const ScanLane s = scan_lane(A);
    if (!s.valid) return;
    const E* base = static_cast<const E*>(A.base);
    E* seq = static_cast<E*>(A.slots_seq);
    const int64_t M = A.M, ds = A.ds, T = A.T;
    const int64_t sbm = (s.b * M + s.m) * ds + s.d;
    float S = s.act ? A.slots0[sbm] : 0.f;
    const float st = s.act ? A.slot_term[int64_t(s.m) * ds + s.d] : 0.f;
    const float mu = A.mu[s.m];
    const E* bp = base + s.b * T * ds + s.d;
    E* op = seq + (s.b * T * M + s.m) * ds + s.d;
    float* up = A.upd2 + (s.b * T * M + s.m) * s.ndw + s.dw;
    for (int64_t t = 0; t < T; ++t) {
        const float pre = (s.act ? ld1(bp + t * ds) : 0.f) + st;
        const float delta = rnd(tanhf(pre), bp);
        if (s.act) st1(op + t * M * ds, S);
        const float u = mu * (delta - S);
        const float u2 = wave_sum(s.act ? u * u : 0.f);
        if ((threadIdx.x & 63) == 0) up[t * M * s.ndw] = u2;
        S += u;
    }
    if (s.act) A.slots_T[sbm] = S;
}

template <typename E>
__global__ __launch_bounds__(256) void screen_scan_bwd_kernel(
    ScreenScanArgs A) {
    const ScanLane s = scan_lane(A);
    if (!s.valid || !s.act) return;
    const E* base = static_cast<const E*>(A.base);
    const E* seq = static_cast<const E*>(A.slots_seq);
    const E* dseq = static_cast<const E*>(A.d_slots_seq);
    const int64_t M = A.M, ds = A.ds, T = A.T;
    const int64_t sbm = (s.b * M + s.m) * ds + s.d;
    float G = A.d_slots_T ? A.d_slots_T[sbm] : 0.f;
    const float st = A.slot_term[int64_t(s.m) * ds + s.d];
    const float mu = A.mu[s.m];
    const E* bp = base + s.b * T * ds + s.d;
    const int64_t o0 = (s.b * T * M + s.m) * ds + s.d;
    float dmu = 0.f;
    for (int64_t t = T - 1; t >= 0; --t) {
        const int64_t o = o0 + t * M * ds;
        const float th = tanhf(ld1(bp + t * ds) + st);
        const float delta = rnd(th, bp);
        dmu += G * (delta - ld1(seq + o));
        A.d_pre[o] = mu * G * (1.f - th * th);
        G = G * (1.f - mu) + ld1(dseq + o);
    }
    A.d_slots0[sbm] = G;
    A.d_mu_part[sbm] = dmu;
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
    r.tau = A.tau;
    r.den = 1.f - A.tau + A.trim_eps;
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
    const int64_t b = tok / A.T;
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
        if (A.age_w) rel *= A.age_w[b * M + m];
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
    const int64_t b = tok / A.T;
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
        const float aw = A.age_w ? A.age_w[b * M + m] : 1.f;
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

unsigned blocks_for_waves(int64_t waves) {
    return unsigned((waves + 3) / 4);  // 4 waves of 64 per 256-thread block
}

}  // namespace

hipError_t launch_screen_scan(bool bf16, bool backward,
                              const ScreenScanArgs& A, hipStream_t stream) {
    const int64_t waves = A.B * A.M * ((A.ds + 63) / 64);
    if (waves == 0) return hipSuccess;
    const dim3 grid(blocks_for_waves(waves)), block(256);
    if (!backward) {
        if (bf16)
            hipLaunchKernelGGL(screen_scan_fwd_kernel<bf16_t>, grid, block, 0,
                               stream, A);
        else
            hipLaunchKernelGGL(screen_scan_fwd_kernel<float>, grid, block, 0,
                               stream, A);
    } else {
        if (bf16)
            hipLaunchKernelGGL(screen_scan_bwd_kernel<bf16_t>, grid, block, 0,
                               stream, A);
        else
            hipLaunchKernelGGL(screen_scan_bwd_kernel<float>, grid, block, 0,
                               stream, A);
    }
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
