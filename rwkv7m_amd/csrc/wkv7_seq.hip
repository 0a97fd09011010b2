// Sequential WKV-7 kernels for gfx950: one workgroup per (batch, head), or
// at N = 128 two, each owning half the state rows.
//
// Each state row i is owned by G consecutive lanes, each holding C = N / G
// contiguous columns in VGPRs, so the row-local parts of the recurrence
// (sa = S a, y = S r, the rank-2 update) need only a G-lane butterfly.
// Token vectors are staged through LDS in blocks.  These kernels carry the
// fp32 path, every head size, and the exact fallback of the chunked path.
//
// Math (reference src/rwkv7m/model/rwkv_core.py:54-86):
//   d = exp(-exp(w));  sa = S a;  S = S diag(d) + sa b^T + v k^T;  y = S r
// Reverse equations (reference src/rwkv7m/kernels/wkv_pallas_gpu.py:221-257),
// with S_{t-1} recomputed forward from checkpoints instead of divided out.

#include <mutex>
#include <type_traits>

#include "wkv7_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

template <int N>
struct SeqShape {
    // A head's N state rows over RS workgroups, each owning NR consecutive
    // rows: rows are independent in the recurrence, and only the backward's
    // five column sums cross them (each workgroup's partial sums are added
    // by a second kernel).  Split where one workgroup would hold more than
    // 64 x 64 state values: the register file then holds C = 8 per lane.
    static constexpr int RS = (N >= 128) ? 2 : 1;
    static constexpr int NR = N / RS;
    static constexpr int G = N >= 16 ? 16 : N;
    static constexpr int C = N / G;
    static constexpr int THREADS = NR * G;
    static constexpr int WAVE_LANES = THREADS < 64 ? THREADS : 64;
    static constexpr int NWAVES = (THREADS + 63) / 64;
    static constexpr int SUB = (N >= 128) ? 4 : (N >= 64 ? 8 : 16);
    static constexpr int TB = 16;
    // The backward's LDS besides the saved states (bytes) with RB
    // reduction buffers: the staged vectors, the reduction buffers and dv.
    static constexpr int bwd_lds(int rb) {
        return 4 * (8 * SUB * N + rb * NWAVES * 5 * N + SUB * N);
    }
    static constexpr int ks_fit(int rb) {
        return (163840 - 512 - bwd_lds(rb)) / (4 * NR * N);
    }
    // Reduction buffers: two (a token's sums are written while the
    // previous token's are read), or one and a second barrier per token
    // where that makes room for two saved states.
    static constexpr int RB = (ks_fit(2) < 2 && ks_fit(1) >= 2) ? 1 : 2;
    // Sub-interval start states the backward keeps in LDS (fp32, the
    // workgroup's NR x N each) so that it recomputes each from the nearest
    // saved one instead of from the interval's checkpoint; 0 where fewer
    // than two fit (one saves no advance).
    static constexpr int KS_FIT = ks_fit(RB);
    static constexpr int KSAVE = KS_FIT < 2 ? 0 : (KS_FIT > 16 ? 16 : KS_FIT);
};

// A prefetched vector element as loaded (its bits), converted to fp32 only
// when written to LDS, so that no instruction waits for the load before
// then.  Loads go through the global address space.
template <typename VT>
struct RawOf {
    using type = VT;
};
__device__ __forceinline__ float raw_load(const float* p) {
    return *(const __attribute__((address_space(1))) float*)p;
}
__device__ __forceinline__ bf16_t raw_load(const bf16_t* p) {
    return *(const __attribute__((address_space(1))) bf16_t*)p;
}
__device__ __forceinline__ float raw_to_f(float x) { return x; }
__device__ __forceinline__ float raw_to_f(bf16_t x) {
    return __uint_as_float(uint32_t(x) << 16);
}

// Forward.  ckpt == nullptr: no aux.  s_t may alias s0.  CT is the
// checkpoint element type (float or bf16_t).
template <int N, typename VT, typename CT>
__global__ void __launch_bounds__(SeqShape<N>::THREADS)
wkv7_seq_fwd_kernel(int64_t T, int64_t BH, VecLayout lay,
                    const VT* __restrict__ r,
                    const VT* __restrict__ w, const VT* __restrict__ k,
                    const VT* __restrict__ v, const VT* __restrict__ a,
                    const VT* __restrict__ b, const float* s0, VT* y,
                    float* s_t, CT* ckpt, int64_t ci) {
    using Sh = SeqShape<N>;
    constexpr int G = Sh::G, C = Sh::C, TB = Sh::TB, TH = Sh::THREADS;
    constexpr int64_t NN = int64_t(N) * N;
    __shared__ float sh[6][TB][N];  // r, decay, k, v, a, b
    __shared__ float sh_y[TB][N];

    constexpr int NR = Sh::NR;
    const int64_t bh = blockIdx.x / Sh::RS;
    const int split = int(blockIdx.x % Sh::RS);
    const int tid = threadIdx.x;
    const int row = split * NR + tid / G, col0 = (tid % G) * C;
    const int64_t my = bh * NN + int64_t(row) * N + col0;
    const int64_t hoff = lay.head(bh, N);

    float S[C];
#pragma unroll
    for (int c = 0; c < C; ++c) S[c] = s0[my + c];
    if (ckpt) {
#pragma unroll
        for (int c = 0; c < C; ++c) store_f(ckpt + my + c, S[c]);
    }
    const VT* srcs[6] = {r, w, k, v, a, b};

    // Each block's vectors are loaded into registers (this thread's
    // elements e = tid + i * TH) during the previous block's steps, where
    // that takes a few registers (PF); small heads load them in place.
    // Elements past the block load token 0 of r instead (every load is
    // unconditional, so none is waited for before its use) and are not
    // written.
    constexpr int PF = (6 * TB * N + TH - 1) / TH;
    constexpr bool AHEAD = PF <= 12;
    typename RawOf<VT>::type pf[AHEAD ? PF : 1];
    auto load_block = [&](int64_t t0) __attribute__((always_inline)) {
        const int nt = int(T - t0 < TB ? T - t0 : TB);
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            const int e = tid + i * TH;
            const int vec = e / (TB * N), rem = e - vec * TB * N;
            const int u = rem / N, j = rem - u * N;
            const bool ok = e < 6 * TB * N && u < nt;
            pf[i] = raw_load(ok ? srcs[ok ? vec : 0] + (t0 + u) * lay.ts +
                                      hoff + j
                                : r + hoff);
        }
    };
    if constexpr (AHEAD) {
        if (T > 0) load_block(0);
    }
    for (int64_t t0 = 0; t0 < T; t0 += TB) {
        const int nt = int(T - t0 < TB ? T - t0 : TB);
        if constexpr (AHEAD) {
#pragma unroll
            for (int i = 0; i < PF; ++i) {
                const int e = tid + i * TH;
                const int vec = e / (TB * N), rem = e - vec * TB * N;
                const int u = rem / N, j = rem - u * N;
                if (e < 6 * TB * N && u < nt) {
                    const float x = raw_to_f(pf[i]);
                    sh[vec][u][j] = vec == 1 ? expf(-expf(x)) : x;
                }
            }
        } else {
            for (int e = tid; e < 6 * TB * N; e += TH) {
                const int vec = e / (TB * N), rem = e - vec * TB * N;
                const int u = rem / N, j = rem - u * N;
                if (u < nt) {
                    float x = load_f(srcs[vec] + (t0 + u) * lay.ts + hoff + j);
                    if (vec == 1) x = expf(-expf(x));
                    sh[vec][u][j] = x;
                }
            }
        }
        __syncthreads();
        if constexpr (AHEAD) {
            if (t0 + TB < T) load_block(t0 + TB);
        }
        // The block's steps.  Where checkpoints fall only on a block's last
        // token (intervals that are multiples of TB, and the end of the
        // sequence), they are stored after the loop, so that the loop holds
        // no global store (one makes the compiler wait for the next block's
        // loads before it).
        auto steps = [&](auto ck_in_loop) __attribute__((always_inline)) {
            for (int u = 0; u < nt; ++u) {
                float sa = 0.f;
#pragma unroll
                for (int c = 0; c < C; ++c) sa += S[c] * sh[4][u][col0 + c];
                sa = group_sum<G>(sa);
                const float vi = sh[3][u][row];
                float acc = 0.f;
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    S[c] = S[c] * sh[1][u][col0 + c] +
                           sa * sh[5][u][col0 + c] + vi * sh[2][u][col0 + c];
                    acc += S[c] * sh[0][u][col0 + c];
                }
                acc = group_sum<G>(acc);
                if (col0 == 0) sh_y[u][row] = acc;
                if constexpr (decltype(ck_in_loop)::value) {
                    const int64_t t = t0 + u;
                    if ((t + 1) % ci == 0 || t + 1 == T) {
                        CT* dst = ckpt + ((t + ci) / ci) * BH * NN + my;
#pragma unroll
                        for (int c = 0; c < C; ++c) store_f(dst + c, S[c]);
                    }
                }
            }
        };
        if (ckpt && ci % TB != 0) {
            steps(std::true_type{});
        } else {
            steps(std::false_type{});
            const int64_t t = t0 + nt - 1;
            if (ckpt && ((t + 1) % ci == 0 || t + 1 == T)) {
                CT* dst = ckpt + ((t + ci) / ci) * BH * NN + my;
#pragma unroll
                for (int c = 0; c < C; ++c) store_f(dst + c, S[c]);
            }
        }
        __syncthreads();
        for (int e = tid; e < nt * NR; e += TH) {
            const int u = e / NR, i = split * NR + (e - u * NR);
            store_f(y + (t0 + u) * lay.ts + hoff + i, sh_y[u][i]);
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) s_t[my + c] = S[c];
}

// The backward's staged vectors, sh[8][SUB][N]: 0 r, 1 decay, 2 k, 3 v,
// 4 a, 5 b, 6 dy, 7 exp(w), for `count` tokens from t0.  Loaded into each
// thread's registers first (its elements e = tid + i * THREADS of the
// seven vectors), so that the loads of the next block can be issued before
// the current one is used, then written to LDS.
// Small heads (more than 8 elements per thread) load in place instead:
// stage_load only records the block and stage_write loads it.
template <int N, typename VT>
struct StageRegs {
    static constexpr int PF =
        (7 * SeqShape<N>::SUB * N + SeqShape<N>::THREADS - 1) /
        SeqShape<N>::THREADS;
    static constexpr bool AHEAD = PF <= 8;
    typename RawOf<VT>::type x[AHEAD ? PF : 1];  // raw bits (see RawOf)
    int64_t t0 = -1;
    int count = 0;
    const void* dy = nullptr;
};

template <int N, typename VT>
__device__ __forceinline__ void stage_load(
    StageRegs<N, VT>& R, int64_t t0, int count, int64_t tstr, int64_t hoff,
    const VT* r, const VT* w, const VT* k, const VT* v, const VT* a,
    const VT* b, const VT* dy) {
    using Sh = SeqShape<N>;
    constexpr int SUB = Sh::SUB, TH = Sh::THREADS;
    if constexpr (StageRegs<N, VT>::AHEAD) {
        const VT* srcs[7] = {r, w, k, v, a, b, dy};
        // (unconditional loads: elements outside the block, and dy when
        // there is none, load token 0 of r and are not written as loaded)
#pragma unroll
        for (int i = 0; i < StageRegs<N, VT>::PF; ++i) {
            const int e = threadIdx.x + i * TH;
            const int vec = e / (SUB * N), rem = e - vec * SUB * N;
            const int u = rem / N, j = rem - u * N;
            const bool ok = e < 7 * SUB * N && u < count && (vec != 6 || dy);
            R.x[i] = raw_load(ok ? srcs[ok ? vec : 0] + (t0 + u) * tstr +
                                       hoff + j
                                 : r + hoff);
        }
    }
    R.t0 = t0;
    R.count = count;
    R.dy = dy;
}

template <int N, typename VT>
__device__ __forceinline__ void stage_write(
    const StageRegs<N, VT>& R, float (*sh)[SeqShape<N>::SUB][N], int64_t tstr,
    int64_t hoff, const VT* r, const VT* w, const VT* k, const VT* v,
    const VT* a, const VT* b) {
    using Sh = SeqShape<N>;
    constexpr int SUB = Sh::SUB, TH = Sh::THREADS;
    if constexpr (!StageRegs<N, VT>::AHEAD) {
        const VT* dy = static_cast<const VT*>(R.dy);
        const VT* srcs[7] = {r, w, k, v, a, b, dy};
        for (int e = threadIdx.x; e < 7 * SUB * N; e += TH) {
            const int vec = e / (SUB * N), rem = e - vec * SUB * N;
            const int u = rem / N, j = rem - u * N;
            if (u < R.count) {
                const int64_t off = (R.t0 + u) * tstr + hoff + j;
                if (vec == 1) {
                    const float ew = expf(load_f(w + off));
                    sh[1][u][j] = expf(-ew);
                    sh[7][u][j] = ew;
                } else {
                    sh[vec][u][j] =
                        vec == 6 && !dy ? 0.f : load_f(srcs[vec] + off);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < StageRegs<N, VT>::PF; ++i) {
        const int e = threadIdx.x + i * TH;
        const int vec = e / (SUB * N), rem = e - vec * SUB * N;
        const int u = rem / N, j = rem - u * N;
        if (e < 7 * SUB * N && u < R.count) {
            const float x = raw_to_f(R.x[i]);
            if (vec == 1) {
                const float ew = expf(x);
                sh[1][u][j] = expf(-ew);
                sh[7][u][j] = ew;
            } else {
                sh[vec][u][j] = vec == 6 && !R.dy ? 0.f : x;
            }
        }
    }
}

template <int N, typename VT, typename CT>
__global__ void __launch_bounds__(SeqShape<N>::THREADS)
wkv7_seq_bwd_kernel(int64_t T, int64_t BH, VecLayout lay,
                    const VT* __restrict__ r,
                    const VT* __restrict__ w, const VT* __restrict__ k,
                    const VT* __restrict__ v, const VT* __restrict__ a,
                    const VT* __restrict__ b, const VT* __restrict__ dy,
                    const float* ds_t,
                    const CT* __restrict__ ckpt, int64_t ci, VT* dr,
                    VT* dw, VT* dk, VT* dv, VT* da, VT* db, float* ds0,
                    int marked_only, const VT* __restrict__ add_dr,
                    const VT* __restrict__ add_dk,
                    const VT* __restrict__ add_dv, int64_t c_lo,
                    int64_t c_hi, float* __restrict__ part, int64_t pt0,
                    int64_t pT) {
    using Sh = SeqShape<N>;
    constexpr int G = Sh::G, C = Sh::C, SUB = Sh::SUB, TH = Sh::THREADS;
    constexpr int WL = Sh::WAVE_LANES, NW = Sh::NWAVES;
    constexpr int64_t NN = int64_t(N) * N;
    constexpr int KS = Sh::KSAVE;
    __shared__ float sh[8][SUB][N];
    __shared__ float red[Sh::RB][NW][5][N];
    __shared__ float sh_dv[SUB][N];
    // saved sub-interval start states, each thread's own C values
    __shared__ float saved[KS > 0 ? KS : 1][KS > 0 ? TH * C : 1];

    constexpr int NR = Sh::NR;
    const int64_t bh = blockIdx.x / Sh::RS;
    const int split = int(blockIdx.x % Sh::RS);
    // marked_only (one workgroup per head): serve only the heads another
    // kernel left to this exact pass (their dS0 holds kExactPassMark);
    // every other head is complete
    if (marked_only &&
        __float_as_uint(ds0[bh * NN]) != kExactPassMark)
        return;
    const int tid = threadIdx.x;
    const int row = split * NR + tid / G, col0 = (tid % G) * C;
    const int wave = tid / 64, lane = tid % 64;
    const int64_t my = bh * NN + int64_t(row) * N + col0;
    const int64_t hoff = lay.head(bh, N);
    VT* gout[5] = {dr, dw, db, dk, da};

    float dS[C];
#pragma unroll
    for (int c = 0; c < C; ++c) dS[c] = ds_t ? ds_t[my + c] : 0.f;

    int buf = 0;
    // one full sub-interval of steps on Sx with the staged vectors (the
    // staging buffers are free again on exit)
    auto advance = [&](float (&Sx)[C]) __attribute__((always_inline)) {
        for (int u = 0; u < SUB; ++u) {
            float sa = 0.f;
#pragma unroll
            for (int cc = 0; cc < C; ++cc) sa += Sx[cc] * sh[4][u][col0 + cc];
            sa = group_sum<G>(sa);
            const float vi = sh[3][u][row];
#pragma unroll
            for (int cc = 0; cc < C; ++cc)
                Sx[cc] = Sx[cc] * sh[1][u][col0 + cc] +
                         sa * sh[5][u][col0 + cc] + vi * sh[2][u][col0 + cc];
        }
        __syncthreads();
    };
    // intervals c_lo .. c_hi - 1 (a time segment of the whole backward when
    // the column sums go through `part`), the last first
    for (int64_t c = c_hi - 1; c >= c_lo; --c) {
        const int64_t ta = c * ci;
        const int64_t tb = (ta + ci < T) ? ta + ci : T;
        const int64_t nsub = (tb - ta + SUB - 1) / SUB;
        // Sub-intervals in reverse, in blocks of KS counted from the
        // interval's end (a partial block holds the first sub-intervals,
        // the cheapest to reach): each block's start states are formed
        // once, from the checkpoint, and saved; each sub-interval then
        // starts from its saved state (KS = 0: every sub-interval from the
        // checkpoint).  The same steps in the same order either way.
        const int64_t per = KS > 0 ? KS : 1;
        const int64_t skew = (per - nsub % per) % per;
        for (int64_t s_lo = ((nsub - 1 + skew) / per) * per - skew;
             s_lo > -per; s_lo -= per) {
        const int64_t s_hi = s_lo + per;
        if (s_lo < 0) s_lo = 0;  // the partial first block (then the last)
        float Sx[C];
#pragma unroll
        for (int cc = 0; cc < C; ++cc)
            Sx[cc] = load_f(ckpt + c * BH * NN + my + cc);
        {
            // The advances of this block, sub-intervals 0 .. s_lo - 1 to
            // reach its start, then (saving each start state) s_lo ..
            // s_hi - 2: each sub-interval's vectors are loaded into
            // registers while the previous one's steps run.
            const int64_t n_adv = KS > 0 ? s_hi - 1 : s_lo;
            StageRegs<N, VT> pf;
            if (n_adv > 0)
                stage_load<N, VT>(pf, ta, SUB, lay.ts, hoff, r, w, k, v, a, b,
                                  nullptr);
            for (int64_t q = 0; q < n_adv; ++q) {
                if (KS > 0 && q >= s_lo) {
#pragma unroll
                    for (int cc = 0; cc < C; ++cc)
                        saved[q - s_lo][tid * C + cc] = Sx[cc];
                }
                stage_write<N, VT>(pf, sh, lay.ts, hoff, r, w, k, v, a, b);
                __syncthreads();
                if (q + 1 < n_adv)
                    stage_load<N, VT>(pf, ta + (q + 1) * SUB, SUB, lay.ts,
                                      hoff, r, w, k, v, a, b, nullptr);
                advance(Sx);
            }
            // the start state of the block's last sub-interval
            if constexpr (KS > 0) {
#pragma unroll
                for (int cc = 0; cc < C; ++cc)
                    saved[s_hi - 1 - s_lo][tid * C + cc] = Sx[cc];
            }
        }
        StageRegs<N, VT> rp;  // the reverse's next sub-interval, loaded ahead
        for (int64_t s = s_hi - 1; s >= s_lo; --s) {
            float St[SUB + 1][C];
            float sa_r[SUB];
#pragma unroll
            for (int cc = 0; cc < C; ++cc)
                St[0][cc] = KS > 0 ? saved[s - s_lo][tid * C + cc] : Sx[cc];
            const int64_t ts = ta + s * SUB;
            const int nt = int(tb - ts < SUB ? tb - ts : SUB);
            if (s == s_hi - 1)
                stage_load<N, VT>(rp, ts, nt, lay.ts, hoff, r, w, k, v, a, b,
                                  dy);
            stage_write<N, VT>(rp, sh, lay.ts, hoff, r, w, k, v, a, b);
            __syncthreads();
            if (s > s_lo)
                stage_load<N, VT>(rp, ts - SUB, SUB, lay.ts, hoff, r, w, k, v,
                                  a, b, dy);
            // recompute the sub-interval's states: St[u] = S before token u
#pragma unroll
            for (int u = 0; u < SUB; ++u) {
                if (u < nt) {
                    float sa = 0.f;
#pragma unroll
                    for (int cc = 0; cc < C; ++cc)
                        sa += St[u][cc] * sh[4][u][col0 + cc];
                    sa = group_sum<G>(sa);
                    sa_r[u] = sa;
                    const float vi = sh[3][u][row];
#pragma unroll
                    for (int cc = 0; cc < C; ++cc)
                        St[u + 1][cc] = St[u][cc] * sh[1][u][col0 + cc] +
                                        sa * sh[5][u][col0 + cc] +
                                        vi * sh[2][u][col0 + cc];
                }
            }
            // reverse over the sub-interval
#pragma unroll
            for (int u = SUB - 1; u >= 0; --u) {
                if (u < nt) {
                    const float dyi = sh[6][u][row], vi = sh[3][u][row];
                    const float sa = sa_r[u];
                    float Gc[C];
                    float dsa = 0.f, dvv = 0.f;
#pragma unroll
                    for (int cc = 0; cc < C; ++cc) {
                        Gc[cc] = dS[cc] + dyi * sh[0][u][col0 + cc];
                        dsa += Gc[cc] * sh[5][u][col0 + cc];
                        dvv += Gc[cc] * sh[2][u][col0 + cc];
                    }
                    dsa = group_sum<G>(dsa);
                    dvv = group_sum<G>(dvv);
                    if (col0 == 0) sh_dv[u][row] = dvv;
                    // this lane's terms of the five column sums (over the
                    // state rows i): q 0 dr, 1 d decay, 2 dkka, 3 dk,
                    // 4 dneg_kk, each summed over the wave's rows into
                    // red[buf][wave][q] one sum at a time (so that only one
                    // sum's C terms are live)
                    auto term = [&](int q, int cc) __attribute__((always_inline)) {
                        return q == 0   ? St[u + 1][cc] * dyi
                               : q == 1 ? Gc[cc] * St[u][cc]
                               : q == 2 ? Gc[cc] * sa
                               : q == 3 ? Gc[cc] * vi
                                        : St[u][cc] * dsa;
                    };
                    if constexpr (G == 16 && WL == 64 && C % 4 == 0) {
                        // Sums over the wave's four rows as a reduce-scatter:
                        // a permlane16 swap of terms j and j + C/2 leaves
                        // term j summed over rows {0, 1} in row 0 and over
                        // {2, 3} in row 2, term j + C/2 likewise in rows 1
                        // and 3; a permlane32 swap of those results j and
                        // j + C/4 completes j and j + C/2 in rows 0 and 1,
                        // j + C/4 and j + 3C/4 in rows 2 and 3.  3C/4 swaps
                        // per sum instead of 2C, and every lane stores.
                        constexpr int H1 = C / 2, H2 = C / 4;
                        const int rw = lane >> 4;
                        const int vo = ((rw & 1) ? H1 : 0) + ((rw & 2) ? H2 : 0);
#pragma unroll
                        for (int q = 0; q < 5; ++q) {
                            float w1[H1];
#pragma unroll
                            for (int jj = 0; jj < H1; ++jj) {
                                const auto x = __builtin_amdgcn_permlane16_swap(
                                    __float_as_uint(term(q, jj)),
                                    __float_as_uint(term(q, jj + H1)), false,
                                    false);
                                w1[jj] = __uint_as_float(x[0]) +
                                         __uint_as_float(x[1]);
                            }
#pragma unroll
                            for (int jj = 0; jj < H2; ++jj) {
                                const auto x = __builtin_amdgcn_permlane32_swap(
                                    __float_as_uint(w1[jj]),
                                    __float_as_uint(w1[jj + H2]), false, false);
                                red[buf][wave][q][col0 + jj + vo] =
                                    __uint_as_float(x[0]) + __uint_as_float(x[1]);
                            }
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < 5; ++q)
#pragma unroll
                            for (int cc = 0; cc < C; ++cc) {
                                const float x =
                                    cross_group_sum<G, WL>(term(q, cc));
                                if (lane < G) red[buf][wave][q][col0 + cc] = x;
                            }
                    }
#pragma unroll
                    for (int cc = 0; cc < C; ++cc)
                        dS[cc] = Gc[cc] * sh[1][u][col0 + cc] +
                                 dsa * sh[4][u][col0 + cc];
                    __syncthreads();
                    const int64_t t = ts + u;
                    for (int e = tid; e < 5 * N; e += TH) {
                        const int q = e / N, j = e - q * N;
                        float acc = 0.f;
#pragma unroll
                        for (int ww = 0; ww < NW; ++ww) acc += red[buf][ww][q][j];
                        if constexpr (Sh::RS > 1) {
                            // this workgroup's rows' share, for the sum
                            // kernel: part[split][t - pt0][bh][q][j]
                            part[((split * pT + (t - pt0)) * BH + bh) * 5 * N +
                                 e] = acc;
                            continue;
                        }
                        if (q == 1) acc *= -sh[7][u][j] * sh[1][u][j];
                        const int64_t off = t * lay.ts + hoff + j;
                        // cotangents of r and k from other uses, added in
                        // fp32 before rounding
                        if (q == 0 && add_dr) acc += load_f(add_dr + off);
                        if (q == 3 && add_dk) acc += load_f(add_dk + off);
                        store_f(gout[q] + off, acc);
                    }
                    if constexpr (Sh::RB == 2)
                        buf ^= 1;
                    else
                        __syncthreads();
                }
            }
            __syncthreads();
            for (int e = tid; e < nt * NR; e += TH) {
                const int u = e / NR, i = split * NR + (e - u * NR);
                const int64_t off = (ts + u) * lay.ts + hoff + i;
                store_f(dv + off,
                        sh_dv[u][i] + (add_dv ? load_f(add_dv + off) : 0.f));
            }
            __syncthreads();
        }
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) ds0[my + c] = dS[c];
}

// The column sums of a row-split backward: for each of nt tokens from t0,
// head and column, the RS workgroups' shares from part[RS][nt][BH][5][N]
// added, then, as in the one-workgroup backward, the decay gradient's
// factor -e^w d applied, the added cotangents summed in and the result
// rounded and stored (q: 0 dr, 1 dw, 2 db, 3 dk, 4 da).
template <int N, typename VT>
__global__ void __launch_bounds__(256)
wkv7_seq_colsum_kernel(int64_t nt, int64_t t0, int64_t BH, VecLayout lay,
                       const float* __restrict__ part,
                       const VT* __restrict__ w,
                       const VT* __restrict__ add_dr,
                       const VT* __restrict__ add_dk, VT* dr, VT* dw, VT* db,
                       VT* dk, VT* da) {
    constexpr int RS = SeqShape<N>::RS;
    const int64_t per = BH * 5 * N;  // values per token
    const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (e >= nt * per) return;
    const int64_t tl = e / per;
    const int64_t rem = e - tl * per;
    const int64_t bh = rem / (5 * N);
    const int qj = int(rem - bh * (5 * N));
    const int q = qj / N, j = qj - q * N;
    float acc = 0.f;
#pragma unroll
    for (int sp = 0; sp < RS; ++sp) acc += part[sp * nt * per + e];
    const int64_t off = (t0 + tl) * lay.ts + lay.head(bh, N) + j;
    if (q == 1) {
        const float ew = expf(load_f(w + off));
        acc *= -ew * expf(-ew);
    }
    if (q == 0 && add_dr) acc += load_f(add_dr + off);
    if (q == 3 && add_dk) acc += load_f(add_dk + off);
    VT* gout[5] = {dr, dw, db, dk, da};
    store_f(gout[q] + off, acc);
}

// Device memory for the row-split backward's partial column sums: a
// stream-ordered pool per device that keeps what it has reserved (so
// repeated calls reuse it instead of mapping new memory each time).
constexpr int kPoolDevices = 64;
std::mutex g_pool_mu;
hipMemPool_t g_pool[kPoolDevices];

hipError_t part_alloc(float** out, size_t bytes, hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kPoolDevices) return hipErrorInvalidDevice;
    {
        std::lock_guard<std::mutex> lock(g_pool_mu);
        if (g_pool[dev] == nullptr) {
            hipMemPoolProps props{};
            props.allocType = hipMemAllocationTypePinned;
            props.location.type = hipMemLocationTypeDevice;
            props.location.id = dev;
            hipMemPool_t pool = nullptr;
            e = hipMemPoolCreate(&pool, &props);
            if (e != hipSuccess) return e;
            uint64_t keep = UINT64_MAX;
            e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold,
                                       &keep);
            if (e != hipSuccess) {
                hipMemPoolDestroy(pool);
                return e;
            }
            g_pool[dev] = pool;
        }
    }
    return hipMallocFromPoolAsync(reinterpret_cast<void**>(out), bytes,
                                  g_pool[dev], stream);
}

// Partial column sums held at once by a row-split backward (bytes): the
// backward runs in time segments of whole intervals that fit it.
constexpr int64_t kPartBytes = int64_t(128) << 20;

template <int N, typename VT, typename CT>
hipError_t launch_fwd_nc(const SeqFwdArgs& p, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_seq_fwd_kernel<N, VT, CT>),
                       dim3(unsigned(BH * SeqShape<N>::RS)),
                       dim3(SeqShape<N>::THREADS), 0, stream, p.T, BH, p.lay,
                       static_cast<const VT*>(p.r),
                       static_cast<const VT*>(p.w),
                       static_cast<const VT*>(p.k),
                       static_cast<const VT*>(p.v),
                       static_cast<const VT*>(p.a),
                       static_cast<const VT*>(p.b), p.s0,
                       static_cast<VT*>(p.y), p.s_t,
                       static_cast<CT*>(p.ckpt), p.ci);
    return hipGetLastError();
}

template <int N, typename VT>
hipError_t launch_fwd_n(const SeqFwdArgs& p, hipStream_t stream) {
    return p.ckpt_bf16 ? launch_fwd_nc<N, VT, bf16_t>(p, stream)
                       : launch_fwd_nc<N, VT, float>(p, stream);
}

template <int N, typename VT, typename CT>
hipError_t launch_bwd_seg(const SeqBwdArgs& p, const float* ds_in,
                          int64_t c_lo, int64_t c_hi, float* part, int64_t pt0,
                          int64_t pT, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_seq_bwd_kernel<N, VT, CT>),
                       dim3(unsigned(BH * SeqShape<N>::RS)),
                       dim3(SeqShape<N>::THREADS), 0, stream, p.T, BH, p.lay,
                       static_cast<const VT*>(p.r),
                       static_cast<const VT*>(p.w),
                       static_cast<const VT*>(p.k),
                       static_cast<const VT*>(p.v),
                       static_cast<const VT*>(p.a),
                       static_cast<const VT*>(p.b),
                       static_cast<const VT*>(p.dy), ds_in,
                       static_cast<const CT*>(p.ckpt), p.ci,
                       static_cast<VT*>(p.dr), static_cast<VT*>(p.dw),
                       static_cast<VT*>(p.dk), static_cast<VT*>(p.dv),
                       static_cast<VT*>(p.da), static_cast<VT*>(p.db),
                       p.ds0, p.marked_only ? 1 : 0,
                       static_cast<const VT*>(p.add_dr),
                       static_cast<const VT*>(p.add_dk),
                       static_cast<const VT*>(p.add_dv), c_lo, c_hi, part,
                       pt0, pT);
    return hipGetLastError();
}

template <int N, typename VT, typename CT>
hipError_t launch_bwd_nc(const SeqBwdArgs& p, hipStream_t stream) {
    const int64_t nint = (p.T + p.ci - 1) / p.ci;
    constexpr int RS = SeqShape<N>::RS;
    if constexpr (RS == 1) {
        return launch_bwd_seg<N, VT, CT>(p, p.ds_t, 0, nint, nullptr, 0, 0,
                                         stream);
    } else {
        // (the exact pass's marks live in one head's dS0, which every split
        // of the head would read while another writes its rows)
        if (p.marked_only) return hipErrorInvalidValue;
        const int64_t BH = p.B * p.H;
        const int64_t tok_bytes = int64_t(RS) * BH * 5 * N * 4;
        int64_t seg = kPartBytes / (tok_bytes * p.ci);
        if (seg < 1) seg = 1;
        if (seg > nint) seg = nint;
        const int64_t seg_tok = seg * p.ci < p.T ? seg * p.ci : p.T;
        float* part = nullptr;
        hipError_t e = part_alloc(&part, size_t(seg_tok * tok_bytes), stream);
        if (e != hipSuccess) return e;
        // segments of `seg` intervals, the last first; dS passes from one to
        // the next through dS0 (each lane reads its own values before it
        // writes them)
        for (int64_t c_hi = nint; c_hi > 0 && e == hipSuccess;) {
            const int64_t c_lo = c_hi - seg > 0 ? c_hi - seg : 0;
            const int64_t t0 = c_lo * p.ci;
            const int64_t t1 = c_hi * p.ci < p.T ? c_hi * p.ci : p.T;
            e = launch_bwd_seg<N, VT, CT>(p, c_hi == nint ? p.ds_t : p.ds0,
                                          c_lo, c_hi, part, t0, t1 - t0,
                                          stream);
            if (e != hipSuccess) break;
            const int64_t n = (t1 - t0) * BH * 5 * N;
            hipLaunchKernelGGL((wkv7_seq_colsum_kernel<N, VT>),
                               dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                               stream, t1 - t0, t0, BH, p.lay, part,
                               static_cast<const VT*>(p.w),
                               static_cast<const VT*>(p.add_dr),
                               static_cast<const VT*>(p.add_dk),
                               static_cast<VT*>(p.dr), static_cast<VT*>(p.dw),
                               static_cast<VT*>(p.db), static_cast<VT*>(p.dk),
                               static_cast<VT*>(p.da));
            e = hipGetLastError();
            c_hi = c_lo;
        }
        const hipError_t f = hipFreeAsync(part, stream);
        return e != hipSuccess ? e : f;
    }
}

template <int N, typename VT>
hipError_t launch_bwd_n(const SeqBwdArgs& p, hipStream_t stream) {
    return p.ckpt_bf16 ? launch_bwd_nc<N, VT, bf16_t>(p, stream)
                       : launch_bwd_nc<N, VT, float>(p, stream);
}

template <typename VT>
hipError_t dispatch_fwd(const SeqFwdArgs& p, hipStream_t s) {
    switch (p.N) {
        case 1: return launch_fwd_n<1, VT>(p, s);
        case 2: return launch_fwd_n<2, VT>(p, s);
        case 4: return launch_fwd_n<4, VT>(p, s);
        case 8: return launch_fwd_n<8, VT>(p, s);
        case 16: return launch_fwd_n<16, VT>(p, s);
        case 32: return launch_fwd_n<32, VT>(p, s);
        case 64: return launch_fwd_n<64, VT>(p, s);
        case 128: return launch_fwd_n<128, VT>(p, s);
        default: return hipErrorInvalidValue;
    }
}

template <typename VT>
hipError_t dispatch_bwd(const SeqBwdArgs& p, hipStream_t s) {
    switch (p.N) {
        case 1: return launch_bwd_n<1, VT>(p, s);
        case 2: return launch_bwd_n<2, VT>(p, s);
        case 4: return launch_bwd_n<4, VT>(p, s);
        case 8: return launch_bwd_n<8, VT>(p, s);
        case 16: return launch_bwd_n<16, VT>(p, s);
        case 32: return launch_bwd_n<32, VT>(p, s);
        case 64: return launch_bwd_n<64, VT>(p, s);
        case 128: return launch_bwd_n<128, VT>(p, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_seq_forward(const SeqFwdArgs& p, hipStream_t stream) {
    return p.bf16 ? dispatch_fwd<bf16_t>(p, stream)
                  : dispatch_fwd<float>(p, stream);
}

hipError_t launch_seq_backward(const SeqBwdArgs& p, hipStream_t stream) {
    return p.bf16 ? dispatch_bwd<bf16_t>(p, stream)
                  : dispatch_bwd<float>(p, stream);
}

}  // namespace rwkv7m
