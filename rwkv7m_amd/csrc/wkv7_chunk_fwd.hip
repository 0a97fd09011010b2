// Chunked WKV-7 forward for gfx950: bf16 vectors, fp32 state, N = 64.
//
// One workgroup (4 waves) per (batch, head) walks the sequence in chunks of
// L tokens (L = 16, 32 or 64).  Within a chunk the recurrence
// (reference src/rwkv7m/model/rwkv_core.py:54-86)
//
//   S_t = S_{t-1} diag(d_t) + (S_{t-1} a_t) b_t^T + v_t k_t^T,  y_t = S_t r_t
//
// is solved in closed form.  With g_t the running sum of log d over the
// chunk and a reference point g_ref at the chunk middle, the decayed
// factors are (token-major, L x N)
//
//   A~_t = a_t e^{g_{t-1}-g_ref}   R~_t = r_t e^{g_t-g_ref}
//   B~_s = b_s e^{g_ref-g_s}       K~_s = k_s e^{g_ref-g_s}
//   B^_s = b_s e^{g_L-g_s}         K^_s = k_s e^{g_L-g_s}
//
// and the L x L matrices Aab = A~ B~^T, Aak = A~ K~^T (strictly lower),
// Arb = R~ B~^T, Ark = R~ K~^T (lower, with diagonal).  Writing S' for the
// chunk-start state with columns scaled by e^{g_ref}:
//
//   X   = (I - Aab)^{-1} (A~ S'^T + Aak V)      (X_t = S_{t-1} a_t = "sa")
//   Y   = R~ S'^T + Arb X + Ark V
//   S_L = S_0 diag(e^{g_L}) + X^T B^ + V^T K^
//
// Every product is a bf16 MFMA (v_mfma_f32_16x16x32_bf16) with fp32
// accumulation; the state stays fp32 in MFMA accumulator registers for the
// whole sequence.  The unit lower-triangular inverse is built from 16x16
// diagonal blocks (fp32 forward substitution) merged with MFMA.  A chunk
// whose decay range exceeds what the factored form represents (more than
// kHalfRange of log-decay on either side of g_ref: far outside the model's
// clamped range) is run by an exact fp32 sequential loop instead.

#include "wkv7_chunk_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

using chunk::CN;
using chunk::kHalfRange;
using chunk::NTHREADS;
using chunk::PN;

template <int L>
struct FwdSmem {
    static constexpr int PL = L + 8;
    static constexpr int NB = L / 16;
    // factors, token-major [t][j]; Ybuf aliases A once A and R are dead
    bf16_t A[L][PN], R[L][PN], Bt[L][PN], Kt[L][PN];
    // factors and values, feature-major [j][t]
    bf16_t Bh[CN][PL], Kh[CN][PL], Vt[CN][PL];
    // chunk-start state (columns scaled by e^{g_ref}), [i][j]
    bf16_t S[CN][PN];
    union {
        bf16_t raw[6][L][CN];  // r, w, k, v, neg_kk, kka of the chunk
        struct {
            bf16_t Aak[L][PL], Arb[L][PL], Ark[L][PL];
            bf16_t Minv[L][PL], Aab[L][PL];
            float AabD[NB][16][17];
            union {
                bf16_t MinvT[L][PL];
                struct {
                    bf16_t U[CN][PL];
                    bf16_t X[CN][PL];
                } ux;
            };
            bf16_t Z[4][16][24];
        } m;
    };
    float tot[4][CN];
    float eL[CN], eRef[CN];
    int flag;
};

template <int L>
__global__ void __launch_bounds__(NTHREADS)
wkv7_chunk_fwd_kernel(int64_t T, int64_t BH, const bf16_t* __restrict__ r,
                      const bf16_t* __restrict__ w,
                      const bf16_t* __restrict__ k,
                      const bf16_t* __restrict__ v,
                      const bf16_t* __restrict__ a,
                      const bf16_t* __restrict__ b, const float* s0,
                      bf16_t* __restrict__ y, float* s_t, float* ckpt,
                      int64_t ckpt_every) {
    using Sm = FwdSmem<L>;
    constexpr int PL = Sm::PL, NB = Sm::NB, TPG = L / 4;
    __shared__ Sm sm;

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = blockIdx.x;
    const int64_t sbase = bh * CN * CN;
    const bf16_t* src[6] = {r, w, k, v, a, b};

    // State S^T in accumulator layout: S[nt][e] = S[i][j] with
    // i = 16*nt + lr, j = 16*wv + 4*lq + e.
    f32x4_t S[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
        const float4 x = *reinterpret_cast<const float4*>(
            s0 + sbase + (16 * nt + lr) * CN + 16 * wv + 4 * lq);
        S[nt][0] = x.x; S[nt][1] = x.y; S[nt][2] = x.z; S[nt][3] = x.w;
        if (ckpt)
            *reinterpret_cast<float4*>(ckpt + sbase + (16 * nt + lr) * CN +
                                       16 * wv + 4 * lq) = x;
    }

    const int64_t nchunks = (T + L - 1) / L;
    for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t t0 = c * L;
        const int n = int(T - t0 < L ? T - t0 : L);
        __syncthreads();  // previous chunk is done with every buffer
        chunk::load_rows<L, 6>(sm.raw, src, t0, T, BH, bh, tid);
        if (tid == 0) sm.flag = 0;
        __syncthreads();

        // ---- A1: running log-decay and the decayed factors -------------
        const int j = lane, grp = wv;
        float cs[TPG];
        {
            float run = 0.f;
#pragma unroll
            for (int u = 0; u < TPG; ++u) {
                const int t = grp * TPG + u;
                const float lam =
                    (t < n) ? -__expf(bf16_to_f32(sm.raw[1][t][j])) : 0.f;
                run += lam;
                cs[u] = run;
            }
            sm.tot[grp][j] = run;
        }
        __syncthreads();
        {
            const float t0v = sm.tot[0][j], t1v = sm.tot[1][j];
            const float t2v = sm.tot[2][j], t3v = sm.tot[3][j];
            const float G = t0v + t1v + t2v + t3v;
            const float gref = t0v + t1v;  // g at token L/2 - 1
            const float off = grp == 0 ? 0.f
                              : grp == 1 ? t0v
                              : grp == 2 ? t0v + t1v
                                         : t0v + t1v + t2v;
            if (-gref > kHalfRange || gref - G > kHalfRange) sm.flag = 1;
            if (grp == 0) {
                sm.eL[j] = __expf(G);
                sm.eRef[j] = __expf(gref);
            }
            const float eLR = __expf(G - gref);
            float eprev = __expf(off - gref);
            uint32_t ph[TPG / 2], pk[TPG / 2], pv[TPG / 2];
#pragma unroll
            for (int u = 0; u < TPG; ++u) {
                const int t = grp * TPG + u;
                const float g = off + cs[u];
                const float eg = __expf(g - gref);
                const float eng = __expf(gref - g);
                const float egl = eLR * eng;
                const float av = bf16_to_f32(sm.raw[4][t][j]);
                const float rv = bf16_to_f32(sm.raw[0][t][j]);
                const float kv = bf16_to_f32(sm.raw[2][t][j]);
                const float bv = bf16_to_f32(sm.raw[5][t][j]);
                const bf16_t vv = sm.raw[3][t][j];
                sm.A[t][j] = to_bf16(av * eprev);
                sm.R[t][j] = to_bf16(rv * eg);
                sm.Bt[t][j] = to_bf16(bv * eng);
                sm.Kt[t][j] = to_bf16(kv * eng);
                const uint32_t hb = to_bf16(bv * egl), hk = to_bf16(kv * egl);
                if (u & 1) {
                    ph[u / 2] |= hb << 16;
                    pk[u / 2] |= hk << 16;
                    pv[u / 2] |= uint32_t(vv) << 16;
                } else {
                    ph[u / 2] = hb;
                    pk[u / 2] = hk;
                    pv[u / 2] = vv;
                }
                eprev = eg;
            }
#pragma unroll
            for (int q = 0; q < TPG / 8; ++q) {
                const int col = grp * TPG + 8 * q;
                *reinterpret_cast<uint4*>(&sm.Bh[j][col]) = make_uint4(
                    ph[4 * q], ph[4 * q + 1], ph[4 * q + 2], ph[4 * q + 3]);
                *reinterpret_cast<uint4*>(&sm.Kh[j][col]) = make_uint4(
                    pk[4 * q], pk[4 * q + 1], pk[4 * q + 2], pk[4 * q + 3]);
                *reinterpret_cast<uint4*>(&sm.Vt[j][col]) = make_uint4(
                    pv[4 * q], pv[4 * q + 1], pv[4 * q + 2], pv[4 * q + 3]);
            }
            if constexpr (TPG % 8 == 4) {
                const int col = grp * TPG + TPG - 4;
                constexpr int q = TPG / 8;
                *reinterpret_cast<uint2*>(&sm.Bh[j][col]) =
                    make_uint2(ph[4 * q], ph[4 * q + 1]);
                *reinterpret_cast<uint2*>(&sm.Kh[j][col]) =
                    make_uint2(pk[4 * q], pk[4 * q + 1]);
                *reinterpret_cast<uint2*>(&sm.Vt[j][col]) =
                    make_uint2(pv[4 * q], pv[4 * q + 1]);
            }
        }
        __syncthreads();

        if (sm.flag) {
            // ---- exact sequential fallback for this chunk -------------
            float* Sf = reinterpret_cast<float*>(&sm.A[0][0]);  // [64][65]
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    Sf[(16 * nt + lr) * 65 + 16 * wv + 4 * lq + e] = S[nt][e];
            __syncthreads();
            const int i = tid >> 2, qq = tid & 3;
            float Sl[16];
#pragma unroll
            for (int c2 = 0; c2 < 16; ++c2) Sl[c2] = Sf[i * 65 + 16 * qq + c2];
            for (int t = 0; t < n; ++t) {
                float sa = 0.f;
#pragma unroll
                for (int c2 = 0; c2 < 16; ++c2)
                    sa += Sl[c2] * bf16_to_f32(sm.raw[4][t][16 * qq + c2]);
                sa += __shfl_xor(sa, 1);
                sa += __shfl_xor(sa, 2);
                const float vi = bf16_to_f32(sm.raw[3][t][i]);
                float acc = 0.f;
#pragma unroll
                for (int c2 = 0; c2 < 16; ++c2) {
                    const int jj = 16 * qq + c2;
                    const float d =
                        expf(-expf(bf16_to_f32(sm.raw[1][t][jj])));
                    Sl[c2] = Sl[c2] * d +
                             sa * bf16_to_f32(sm.raw[5][t][jj]) +
                             vi * bf16_to_f32(sm.raw[2][t][jj]);
                    acc += Sl[c2] * bf16_to_f32(sm.raw[0][t][jj]);
                }
                acc += __shfl_xor(acc, 1);
                acc += __shfl_xor(acc, 2);
                if (qq == 0) y[((t0 + t) * BH + bh) * CN + i] = to_bf16(acc);
            }
#pragma unroll
            for (int c2 = 0; c2 < 16; ++c2) Sf[i * 65 + 16 * qq + c2] = Sl[c2];
            __syncthreads();
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    S[nt][e] = Sf[(16 * nt + lr) * 65 + 16 * wv + 4 * lq + e];
        } else {
            // ---- B0: scaled chunk-start state to LDS (bf16, [i][j]) ---
            {
                float er[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) er[e] = sm.eRef[16 * wv + 4 * lq + e];
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    uint2 p;
                    p.x = pack_bf16x2(S[nt][0] * er[0], S[nt][1] * er[1]);
                    p.y = pack_bf16x2(S[nt][2] * er[2], S[nt][3] * er[3]);
                    *reinterpret_cast<uint2*>(
                        &sm.S[16 * nt + lr][16 * wv + 4 * lq]) = p;
                }
            }
            // ---- A2: the four L x L matrices (lower tiles) -------------
#pragma unroll
            for (int it = 0; it < NB * NB; ++it) {
                const int ti = wv + 4 * it;
                const int mat = ti / (NB * NB), rem = ti % (NB * NB);
                const int mt = rem / NB, nt = rem % NB;
                bf16_t* dst = mat == 0 ? &sm.m.Aab[0][0]
                              : mat == 1 ? &sm.m.Aak[0][0]
                              : mat == 2 ? &sm.m.Arb[0][0]
                                         : &sm.m.Ark[0][0];
                dst += 16 * mt * PL + 16 * nt;
                f32x4_t acc = zero4();
                if (nt <= mt) {
                    const bf16_t* Aop = mat < 2 ? &sm.A[16 * mt][0]
                                                : &sm.R[16 * mt][0];
                    const bf16_t* Bop = (mat & 1) ? &sm.Kt[16 * nt][0]
                                                  : &sm.Bt[16 * nt][0];
                    mma_nt<CN>(acc, Aop, PN, Bop, PN, lane);
                    const bool strict = mat < 2;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int tt = 16 * mt + 4 * lq + e, ss = 16 * nt + lr;
                        const bool keep = strict ? (ss < tt) : (ss <= tt);
                        acc[e] = keep ? acc[e] : 0.f;
                    }
                    if (mat == 0 && mt == nt) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            sm.m.AabD[mt][4 * lq + e][lr] = acc[e];
                    }
                }
                store_tile_bf16(acc, dst, PL, lane);
            }
            __syncthreads();
            // ---- A3: Minv = (I - Aab)^{-1} -----------------------------
            chunk::build_minv<L>(sm.m.AabD, &sm.m.Aab[0][0], &sm.m.Minv[0][0],
                                 &sm.m.MinvT[0][0], sm.m.Z, tid);
            // ---- B1: U = A~ S'^T + Aak V (stored transposed) and the
            //          state/value part of Y^T -----------------------------
            f32x4_t Yacc[NB];
#pragma unroll
            for (int mt = 0; mt < NB; ++mt) {
                f32x4_t u = zero4();
                mma_nt<CN>(u, &sm.A[16 * mt][0], PN, &sm.S[16 * wv][0], PN,
                           lane);
                mma_nt<L>(u, &sm.m.Aak[16 * mt][0], PL, &sm.Vt[16 * wv][0],
                          PL, lane);
                Yacc[mt] = zero4();
                mma_nt<CN>(Yacc[mt], &sm.S[16 * wv][0], PN, &sm.R[16 * mt][0],
                           PN, lane);
                mma_nt<L>(Yacc[mt], &sm.Vt[16 * wv][0], PL,
                          &sm.m.Ark[16 * mt][0], PL, lane);
                // U tile (t in mt, i in wv) -> U[i][t]; U aliases MinvT,
                // whose last reads (the merges) precede the barrier above
                store_tile_bf16_t(u, &sm.m.ux.U[16 * wv][16 * mt], PL, lane);
            }
            __syncthreads();
            // ---- B2: X = Minv U (stored transposed) ---------------------
#pragma unroll
            for (int mt = 0; mt < NB; ++mt) {
                f32x4_t x = zero4();
                mma_nt<L>(x, &sm.m.Minv[16 * mt][0], PL, &sm.m.ux.U[16 * wv][0],
                          PL, lane);
                store_tile_bf16_t(x, &sm.m.ux.X[16 * wv][16 * mt], PL, lane);
            }
            __syncthreads();
            // ---- B3: Y^T += X^T Arb^T; S^T = e^{g_L} S^T + B^^T X + K^^T V
            bf16_t(*Ybuf)[PN] = sm.A;
#pragma unroll
            for (int mt = 0; mt < NB; ++mt) {
                mma_nt<L>(Yacc[mt], &sm.m.ux.X[16 * wv][0], PL,
                          &sm.m.Arb[16 * mt][0], PL, lane);
                store_tile_bf16_t(Yacc[mt], &Ybuf[16 * mt][16 * wv], PN, lane);
            }
            {
                float el[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) el[e] = sm.eL[16 * wv + 4 * lq + e];
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) S[nt][e] *= el[e];
                    mma_nt<L>(S[nt], &sm.Bh[16 * wv][0], PL,
                              &sm.m.ux.X[16 * nt][0], PL, lane);
                    mma_nt<L>(S[nt], &sm.Kh[16 * wv][0], PL,
                              &sm.Vt[16 * nt][0], PL, lane);
                }
            }
            __syncthreads();
            // ---- B4: y rows of the chunk to HBM ------------------------
#pragma unroll
            for (int p = 0; p < (L + 31) / 32; ++p) {
                const int t = p * 32 + (tid >> 3), seg = tid & 7;
                if (t < n)
                    *reinterpret_cast<uint4*>(
                        y + ((t0 + t) * BH + bh) * CN + seg * 8) =
                        *reinterpret_cast<const uint4*>(&Ybuf[t][seg * 8]);
            }
        }
        if (ckpt && (((c + 1) % ckpt_every) == 0 || c + 1 == nchunks)) {
            float* dst = ckpt + ((c + ckpt_every) / ckpt_every) * BH * CN * CN +
                         sbase;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                *reinterpret_cast<float4*>(dst + (16 * nt + lr) * CN + 16 * wv +
                                           4 * lq) =
                    make_float4(S[nt][0], S[nt][1], S[nt][2], S[nt][3]);
        }
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
        *reinterpret_cast<float4*>(s_t + sbase + (16 * nt + lr) * CN +
                                   16 * wv + 4 * lq) =
            make_float4(S[nt][0], S[nt][1], S[nt][2], S[nt][3]);
}

template <int L>
hipError_t launch_l(const ChunkFwdArgs& p, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_chunk_fwd_kernel<L>), dim3(unsigned(BH)),
                       dim3(NTHREADS), 0, stream, p.T, BH,
                       static_cast<const bf16_t*>(p.r),
                       static_cast<const bf16_t*>(p.w),
                       static_cast<const bf16_t*>(p.k),
                       static_cast<const bf16_t*>(p.v),
                       static_cast<const bf16_t*>(p.a),
                       static_cast<const bf16_t*>(p.b), p.s0,
                       static_cast<bf16_t*>(p.y), p.s_t, p.ckpt,
                       p.ckpt_every);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_chunk_forward(const ChunkFwdArgs& p, hipStream_t stream) {
    switch (p.L) {
        case 16: return launch_l<16>(p, stream);
        case 32: return launch_l<32>(p, stream);
        case 64: return launch_l<64>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rwkv7m
