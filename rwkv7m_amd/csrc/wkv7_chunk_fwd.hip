// Chunked WKV-7 forward for gfx950: bf16 vectors, fp32 state, N = 64.
//
// One workgroup (8 waves) per (batch, head) walks the sequence in chunks of
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
// whole sequence (the checkpoints the backward reads are its bf16 roundings,
// one per chunk).  The unit lower-triangular inverse is built from 16x16
// diagonal blocks, each the product (I+A)(I+A^2)(I+A^4)(I+A^8) of the
// nilpotent strictly lower block A, merged with MFMA.  A chunk
// whose decay range exceeds what the factored form represents (more than
// kHalfRange of log-decay on either side of g_ref: far outside the model's
// clamped range) is run by an exact fp32 sequential loop instead.

#include "wkv7_chunk_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

using chunk::CN;
using chunk::kHalfRange;
using chunk::PN;

// Waves per workgroup: 8 waves keep every value in registers (up to 256
// VGPRs per wave); a register spill would cost far more than the fewer waves,
// because a scratch reload waits for every HBM load and store the wave has in
// flight (one shared counter).
constexpr int FWD_WAVES = 8;

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
            bf16_t AabTD[NB][16][24];
            bf16_t MinvT[L][PL];
            struct {
                bf16_t U[CN][PL];
                bf16_t X[CN][PL];
            } ux;
            bf16_t Z[4][16][24];
        } m;
    };
    float tot[FWD_WAVES][CN];
    float eL[CN], eRef[CN];
    int flag;
};

template <int L>
__global__ void __launch_bounds__(FWD_WAVES * 64)
wkv7_chunk_fwd_kernel(int64_t T, int64_t BH, const bf16_t* __restrict__ r,
                      const bf16_t* __restrict__ w,
                      const bf16_t* __restrict__ k,
                      const bf16_t* __restrict__ v,
                      const bf16_t* __restrict__ a,
                      const bf16_t* __restrict__ b, const float* s0,
                      bf16_t* __restrict__ y, float* s_t, bf16_t* ckpt) {
    using Sm = FwdSmem<L>;
    constexpr int NW = FWD_WAVES, NTH = NW * 64;
    constexpr int PL = Sm::PL, NB = Sm::NB, TPG = L / NW;
    constexpr int ST = 16 / NW;  // state tiles per wave
    static_assert(L % NW == 0 && 16 % NW == 0, "wave layout");
    __shared__ Sm sm;

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = blockIdx.x;
    const int64_t sbase = bh * CN * CN;
    const chunk::VecPtrs src{r, w, k, v, a, b, nullptr};

    // State tiles of this wave: tile si = ST*wv + q covers S[i][j] with
    // i = 16*(si & 3) + lr, j = 16*(si >> 2) + 4*lq + e (tiles of S^T).
    f32x4_t S[ST];
    int64_t soff[ST];
#pragma unroll
    for (int q = 0; q < ST; ++q) {
        const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
        soff[q] = sbase + (16 * ib + lr) * CN + 16 * jb + 4 * lq;
        const float4 x = *reinterpret_cast<const float4*>(s0 + soff[q]);
        S[q][0] = x.x; S[q][1] = x.y; S[q][2] = x.z; S[q][3] = x.w;
        if (ckpt) *reinterpret_cast<uint2*>(ckpt + soff[q]) = pack4(S[q]);
    }

    // The next chunk's six vectors are fetched into registers while the
    // current chunk computes (16-byte segments, 8 per 64-wide row).  Only
    // the loader waves (upper half) load and only the store waves (lower
    // half) store: vmcnt counts loads and stores of a wave together, so a
    // loader wave's wait before a stash never covers stores in flight.
    constexpr int LOADERS = NTH / 2;
    const bool loader = tid >= LOADERS;
    const int ltid = tid - LOADERS;
    constexpr int SEG = 6 * L * 8;
    constexpr int NPRE = (SEG + LOADERS - 1) / LOADERS;
    uint4 pre[NPRE];
    // Each loader thread's segments sit at the same place of every chunk:
    // their addresses are formed once, and a fetch only adds t0 * BH * 64.
    const bf16_t* pbase[NPRE];
    int ptok[NPRE];
#pragma unroll
    for (int p = 0; p < NPRE; ++p) {
        const int seg = p * LOADERS + (loader ? ltid : 0);
        const int row = seg >> 3, s8 = seg & 7;
        const int vec = row / L, t = row % L;
        ptok[p] = (seg < SEG) ? t : int(1 << 30);
        pbase[p] = src.get(vec < 6 ? vec : 0) + (int64_t(t) * BH + bh) * CN + s8 * 8;
    }
    const int64_t chunk_stride = int64_t(L) * BH * CN;
    auto fetch = [&](int64_t t0f) {
        const int64_t off = (t0f / L) * chunk_stride;
#pragma unroll
        for (int p = 0; p < NPRE; ++p) {
            pre[p] = make_uint4(0, 0, 0, 0);
            if (t0f + ptok[p] < T)
                pre[p] = *reinterpret_cast<const uint4*>(pbase[p] + off);
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int p = 0; p < NPRE; ++p) {
            const int seg = p * LOADERS + ltid;
            if (seg < SEG) {
                const int row = seg >> 3, s8 = seg & 7;
                *reinterpret_cast<uint4*>(
                    &sm.raw[row / L][row % L][s8 * 8]) = pre[p];
            }
        }
    };
    // Checkpoint tiles of the loader waves go to HBM through the store
    // waves, staged in LDS (Bh/Kh/Vt, free after B3) as [tile - 8][lane].
    uint2* ck_stage = reinterpret_cast<uint2*>(&sm.Bh[0][0]);
    static_assert(sizeof(sm.Bh) * 3 >= 8 * 64 * 8, "checkpoint staging");

    // Pipeline: chunk c+1's vectors sit in LDS (raw) while chunk c+2's are
    // in flight to the loader waves' registers.
    const int64_t nchunks = (T + L - 1) / L;
    if (loader) {
        fetch(0);
        stash();
    }
    // Everything loaded before the loop (state, first chunk) has arrived:
    // without this wait the compiler guards first uses inside the loop with
    // vmcnt waits that, in later iterations, drain the prefetch and the
    // stores in flight.
    __builtin_amdgcn_s_waitcnt(0);
    if (loader && nchunks > 1) fetch(L);
    if (tid == 0) sm.flag = 0;
    __syncthreads();
    for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t t0 = c * L;
        const int n = int(T - t0 < L ? T - t0 : L);

        // ---- A1: running log-decay and the decayed factors -------------
        // thread: column j = lane, tokens [grp*TPG, grp*TPG + TPG)
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
            float off = 0.f, G = 0.f, gref = 0.f;
#pragma unroll
            for (int g2 = 0; g2 < NW; ++g2) {
                const float tv = sm.tot[g2][j];
                G += tv;
                if (g2 < grp) off += tv;
                if (g2 == NW / 2 - 1) gref = G;  // g at token L/2 - 1
            }
            if (-gref > kHalfRange || gref - G > kHalfRange) sm.flag = 1;
            if (grp == 0) {
                sm.eL[j] = __expf(G);
                sm.eRef[j] = __expf(gref);
            }
            const float eLR = __expf(G - gref);
            float eprev = __expf(off - gref);
            bf16_t hb[TPG], hk[TPG], hv[TPG];
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
                sm.A[t][j] = to_bf16(av * eprev);
                sm.R[t][j] = to_bf16(rv * eg);
                sm.Bt[t][j] = to_bf16(bv * eng);
                sm.Kt[t][j] = to_bf16(kv * eng);
                hb[u] = to_bf16(bv * egl);
                hk[u] = to_bf16(kv * egl);
                hv[u] = sm.raw[3][t][j];
                eprev = eg;
            }
            chunk::put_row<TPG>(&sm.Bh[j][grp * TPG], hb);
            chunk::put_row<TPG>(&sm.Kh[j][grp * TPG], hk);
            chunk::put_row<TPG>(&sm.Vt[j][grp * TPG], hv);
        }
        __syncthreads();
        // read once: thread 0 clears the flag again at the end of the chunk
        const bool fallback = sm.flag != 0;

        if (fallback) {
            // ---- exact sequential fallback for this chunk -------------
            // thread: row i = tid / NW, columns CPT*(tid % NW) .. + CPT-1
            constexpr int CPT = CN / NW;
            float* Sf = reinterpret_cast<float*>(&sm.A[0][0]);  // [64][65]
            static_assert(sizeof(sm.A) * 4 + sizeof(sm.Bh) * 3 >=
                              64 * 65 * 4, "Sf fits");
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    Sf[(16 * ib + lr) * 65 + 16 * jb + 4 * lq + e] = S[q][e];
            }
            __syncthreads();
            const int i = tid / NW, c0 = CPT * (tid % NW);
            float Sl[CPT];
#pragma unroll
            for (int c2 = 0; c2 < CPT; ++c2) Sl[c2] = Sf[i * 65 + c0 + c2];
            for (int t = 0; t < n; ++t) {
                float sa = 0.f;
#pragma unroll
                for (int c2 = 0; c2 < CPT; ++c2)
                    sa += Sl[c2] * bf16_to_f32(sm.raw[4][t][c0 + c2]);
                sa = group_sum<NW>(sa);
                const float vi = bf16_to_f32(sm.raw[3][t][i]);
                float acc = 0.f;
#pragma unroll
                for (int c2 = 0; c2 < CPT; ++c2) {
                    const int jj = c0 + c2;
                    const float d =
                        expf(-expf(bf16_to_f32(sm.raw[1][t][jj])));
                    Sl[c2] = Sl[c2] * d +
                             sa * bf16_to_f32(sm.raw[5][t][jj]) +
                             vi * bf16_to_f32(sm.raw[2][t][jj]);
                    acc += Sl[c2] * bf16_to_f32(sm.raw[0][t][jj]);
                }
                acc = group_sum<NW>(acc);
                if (tid % NW == 0)
                    y[((t0 + t) * BH + bh) * CN + i] = to_bf16(acc);
            }
#pragma unroll
            for (int c2 = 0; c2 < CPT; ++c2) Sf[i * 65 + c0 + c2] = Sl[c2];
            __syncthreads();
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    S[q][e] = Sf[(16 * ib + lr) * 65 + 16 * jb + 4 * lq + e];
            }
            __syncthreads();  // Sf (aliasing the staging area) is read
        } else {
            // ---- B0: scaled chunk-start state to LDS (bf16, [i][j]) ---
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
                float er[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) er[e] = sm.eRef[16 * jb + 4 * lq + e];
                uint2 p;
                p.x = pack_bf16x2(S[q][0] * er[0], S[q][1] * er[1]);
                p.y = pack_bf16x2(S[q][2] * er[2], S[q][3] * er[3]);
                *reinterpret_cast<uint2*>(
                    &sm.S[16 * ib + lr][16 * jb + 4 * lq]) = p;
            }
            // ---- A2: the four L x L matrices (lower tiles) -------------
            constexpr int NT2 = 4 * NB * NB;
#pragma unroll
            for (int it = 0; it < (NT2 + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < NT2) {
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
                            const int tt = 16 * mt + 4 * lq + e;
                            const int ss = 16 * nt + lr;
                            const bool keep = strict ? (ss < tt) : (ss <= tt);
                            acc[e] = keep ? acc[e] : 0.f;
                        }
                        if (mat == 0 && mt == nt)
                            store_tile_bf16_t(acc, &sm.m.AabTD[mt][0][0], 24,
                                              lane);
                    }
                    store_tile_bf16(acc, dst, PL, lane);
                }
            }
            __syncthreads();
            // ---- A3 + B1: Minv = (I - Aab)^{-1} on waves 0 .. NB-1 while
            // the other waves form U = A~ S'^T + Aak V (stored transposed)
            // and the state/value part of Y^T.  B1 tiles 0 .. 4NB-1 are U
            // (t block mt, i block ui), 4NB .. 8NB-1 are Y^T (i block yi,
            // t block yt), dealt round-robin over waves NB .. NW-1.
            constexpr int NT1 = 8 * NB, NWB = NW - NB;
            constexpr int IT1 = (NT1 + NWB - 1) / NWB;
            f32x4_t Yacc[IT1];
#pragma unroll
            for (int it = 0; it < IT1; ++it) Yacc[it] = zero4();
            auto b1 = [&] {
#pragma unroll
                for (int it = 0; it < IT1; ++it) {
                    const int ti = (wv - NB) + NWB * it;
                    if (ti < 4 * NB) {
                        const int mt = ti >> 2, ui = ti & 3;
                        f32x4_t u = zero4();
                        mma_nt<CN>(u, &sm.A[16 * mt][0], PN, &sm.S[16 * ui][0],
                                   PN, lane);
                        mma_nt<L>(u, &sm.m.Aak[16 * mt][0], PL,
                                  &sm.Vt[16 * ui][0], PL, lane);
                        store_tile_bf16_t(u, &sm.m.ux.U[16 * ui][16 * mt], PL,
                                          lane);
                    } else if (ti < NT1) {
                        const int yt = (ti - 4 * NB) % NB;
                        const int yi = (ti - 4 * NB) / NB;
                        mma_nt<CN>(Yacc[it], &sm.S[16 * yi][0], PN,
                                   &sm.R[16 * yt][0], PN, lane);
                        mma_nt<L>(Yacc[it], &sm.Vt[16 * yi][0], PL,
                                  &sm.m.Ark[16 * yt][0], PL, lane);
                    }
                }
            };
            // product scratch in Bt/Kt (dead after A2)
            static_assert(sizeof(sm.Bt) * 2 >= NB * 5 * 16 * 24 * 2, "W fits");
            chunk::build_minv<L, NTH>(
                &sm.m.Aab[0][0], sm.m.AabTD, &sm.m.Minv[0][0],
                &sm.m.MinvT[0][0], sm.m.Z,
                reinterpret_cast<bf16_t(*)[5][16][24]>(&sm.Bt[0][0]), tid, b1);
            // ---- B2: X = Minv U (stored transposed) ---------------------
#pragma unroll
            for (int it = 0; it < (4 * NB + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < 4 * NB) {
                    const int mt = ti >> 2, xi = ti & 3;
                    f32x4_t x = zero4();
                    mma_nt<L>(x, &sm.m.Minv[16 * mt][0], PL,
                              &sm.m.ux.U[16 * xi][0], PL, lane);
                    store_tile_bf16_t(x, &sm.m.ux.X[16 * xi][16 * mt], PL,
                                      lane);
                }
            }
            __syncthreads();
            // ---- B3: Y^T += X^T Arb^T; S^T = e^{g_L} S^T + B^^T X + K^^T V
            bf16_t(*Ybuf)[PN] = sm.A;
            if (wv >= NB) {
#pragma unroll
                for (int it = 0; it < IT1; ++it) {
                    const int ti = (wv - NB) + NWB * it;
                    if (ti >= 4 * NB && ti < NT1) {
                        const int yt = (ti - 4 * NB) % NB;
                        const int yi = (ti - 4 * NB) / NB;
                        mma_nt<L>(Yacc[it], &sm.m.ux.X[16 * yi][0], PL,
                                  &sm.m.Arb[16 * yt][0], PL, lane);
                        store_tile_bf16_t(Yacc[it], &Ybuf[16 * yt][16 * yi],
                                          PN, lane);
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    S[q][e] *= sm.eL[16 * jb + 4 * lq + e];
                mma_nt<L>(S[q], &sm.Bh[16 * jb][0], PL, &sm.m.ux.X[16 * ib][0],
                          PL, lane);
                mma_nt<L>(S[q], &sm.Kh[16 * jb][0], PL, &sm.Vt[16 * ib][0],
                          PL, lane);
            }
            __syncthreads();
            // ---- B4: y rows of the chunk to HBM (store waves) ---------
            for (int sg = tid; sg < 8 * L; sg += LOADERS) {
                if (loader) break;
                const int t = sg >> 3, s8 = sg & 7;
                if (t < n)
                    *reinterpret_cast<uint4*>(
                        y + ((t0 + t) * BH + bh) * CN + s8 * 8) =
                        *reinterpret_cast<const uint4*>(&Ybuf[t][s8 * 8]);
            }
        }
        // ---- next chunk's vectors to LDS; checkpoint tiles ---------------
        const bool want_ckpt = ckpt != nullptr;
        bf16_t* cdst = ckpt + (c + 1) * BH * CN * CN;
        if (loader) {
            stash();
            if (want_ckpt) {
#pragma unroll
                for (int q = 0; q < ST; ++q)
                    ck_stage[(ST * wv + q - 8) * 64 + lane] = pack4(S[q]);
            }
            if (c + 2 < nchunks) fetch(t0 + 2 * L);
        } else if (want_ckpt) {
#pragma unroll
            for (int q = 0; q < ST; ++q)
                *reinterpret_cast<uint2*>(cdst + soff[q]) = pack4(S[q]);
        }
        if (tid == 0) sm.flag = 0;
        __syncthreads();
        if (want_ckpt && !loader) {
            // the store waves write the loader waves' tiles 8 .. 15
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = 8 + ST * wv + q, jb = si >> 2, ib = si & 3;
                *reinterpret_cast<uint2*>(
                    cdst + sbase + (16 * ib + lr) * CN + 16 * jb + 4 * lq) =
                    ck_stage[(ST * wv + q) * 64 + lane];
            }
        }
    }
#pragma unroll
    for (int q = 0; q < ST; ++q)
        *reinterpret_cast<float4*>(s_t + soff[q]) =
            make_float4(S[q][0], S[q][1], S[q][2], S[q][3]);
}

template <int L>
hipError_t launch_l(const ChunkFwdArgs& p, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_chunk_fwd_kernel<L>), dim3(unsigned(BH)),
                       dim3(FWD_WAVES * 64), 0, stream, p.T, BH,
                       static_cast<const bf16_t*>(p.r),
                       static_cast<const bf16_t*>(p.w),
                       static_cast<const bf16_t*>(p.k),
                       static_cast<const bf16_t*>(p.v),
                       static_cast<const bf16_t*>(p.a),
                       static_cast<const bf16_t*>(p.b), p.s0,
                       static_cast<bf16_t*>(p.y), p.s_t,
                       static_cast<bf16_t*>(p.ckpt));
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
