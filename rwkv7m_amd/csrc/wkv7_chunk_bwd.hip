// Chunked WKV-7 backward for gfx950: bf16 vectors, fp32 state, N = 64,
// chunk length L in {16, 32} (= the forward's checkpoint interval).
//
// One workgroup (8 waves) per (batch, head) walks the chunks in reverse.
// For each chunk it reads the chunk-start state S_0 from the forward's bf16
// checkpoints, rebuilds the forward's factors (wkv7_chunk_common.h: A~, R~,
// B~, K~, Aab, Aak, Arb, Ark, Minv) and
//
//   U = A~ S'^T + Aak V,  X = Minv U     (X_t = S_{t-1} a_t)
//
// and applies the adjoint of every product.  With D the cotangent of the
// chunk-end state S_L, D' = D diag(e^{g_L-g_ref}) and dY the cotangent of
// the chunk's outputs:
//
//   dX  = B~ D'^T + Arb^T dY          dU  = Minv^T dX
//   dV  = K~ D'^T + Ark^T dY + Aak^T dU
//   dArb = lower(dY X^T)  dArk = lower(dY V^T)          (with diagonal)
//   dAab = slower(dU X^T) dAak = slower(dU V^T)         (strict)
//   dR~ = dY S' + dArb B~ + dArk K~     dA~ = dU S' + dAab B~ + dAak K~
//   dB~ = dAab^T A~ + dArb^T R~ + X D'  dK~ = dAak^T A~ + dArk^T R~ + V D'
//   D_0 = D diag(e^{g_L}) + (dY^T R~ + dU^T A~) diag(e^{g_ref})
//
// (dB~ and dK~ include the B^, K^ terms of S_L) and the input gradients
// follow by the factors' scalings.  The decay gradient uses the identity
// (exact for the chunk with S_0 and D fixed)
//
//   dlog d_t = sum_{t' >= t} (r dr - b db - k dk)_{t'} + (a da)_{t'+1}
//              + sum_i D[i, :] S_L[i, :]
//
// and dw = dlog d * (-e^w).  These are the reference's reverse equations
// (src/rwkv7m/kernels/wkv_pallas_gpu.py:221-257) summed over a chunk; the
// states come from checkpoints (recompute), never from dividing by the
// decay.  Seven barrier-separated phases per chunk:
//
//   1  factors; S_0 tiles
//   2  S', D' to LDS; sum_i D S_L; the inverse (wave 0, in registers);
//      Aak, Arb, Ark, dArk
//   3  U, dX
//   4  X, dU
//   5  dArb, dAab, dAak; dV (to HBM); D_0
//   6  dR~, dA~, dB~, dK~ (fp32 to LDS)
//   7  input gradients and the decay gradient (to HBM); next chunk's data
//
// Every product is a bf16 MFMA with fp32 accumulation, operands read in
// whichever order they are stored (transposing LDS loads).  A chunk outside
// the factored form's range runs an exact fp32 sequential reverse pass.

#include "wkv7_chunk_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

using chunk::CN;
using chunk::fkr;
using chunk::frk;
using chunk::PN;

constexpr int BWD_WAVES = chunk::NWAVES;
constexpr int BWD_THREADS = chunk::NTHREADS;

template <int L>
struct BwdSmem {
    static constexpr int PL = L + 8;
    static constexpr int NB = L / 16;
    // the chunk's vectors: r, w, k, v, neg_kk, kka, dy ([t][j])
    bf16_t raw[7][L][PN];
    bf16_t S0s[CN][PN];  // the next chunk's S_0 checkpoint (staging), [i][j]
    bf16_t At[L][PN], Rt[L][PN], Bt[L][PN], Kt[L][PN];  // factors, [t][j]
    union {
        struct {
            bf16_t Sp[CN][PN];  // S' = S_0 diag(e^{g_ref}), [i][j]
            bf16_t Dl[CN][PN];  // D' = D diag(e^{g_L - g_ref}), [i][j]
            bf16_t X[L][PN], dU[L][PN];  // [t][i]
        };
        // phase 7 to the next chunk's phase 1: the chunk's gradients
        // dr, dw, dk, dneg_kk, dkka, dv (bf16, [t][j]) on their way to HBM
        bf16_t stg[6][L][PN];
    };
    // cotangents of the L x L matrices, stored transposed
    bf16_t dArb[L][PL], dArk[L][PL], dAab[L][PL], dAak[L][PL];
    union {
        struct {  // phases 2 .. 5
            bf16_t Aak[L][PL], Arb[L][PL], Ark[L][PL];
            bf16_t MinvT[L][PL];
            bf16_t Ut[CN][PL], dXt[CN][PL];  // [i][t]
        } m;
        struct {  // phases 6, 7: dR~, dA~, dB~, dK~ ([t][j])
            float gR[L][CN + 4], gA[L][CN + 4], gB[L][CN + 4], gK[L][CN + 4];
        } g;
        struct {  // exact fallback
            float Sf[CN * 65], Df[CN * 65], red[BWD_WAVES * 5 * CN];
        } fb;
    };
    alignas(16) float eL[CN];
    alignas(16) float eRef[CN];
    alignas(16) float eLR[CN];
    alignas(16) float part[2][CN];  // sum_i D S_L over the two halves of i
    int flag;
};

// Exact fp32 sequential reverse pass over one chunk (the fallback for decays
// outside the factored form's range).  S_0 and D come in and D goes out
// through fp32 LDS copies Sf, Df ([64][65]); red is [NW][5][64] scratch.
// Thread: row i = tid / NW, columns CPT * (tid % NW) .. + CPT - 1.
template <int L, int NW>
__device__ void seq_chunk_backward(const bf16_t (*raw)[L][PN], int n,
                                   const float* Sf, float* Df, float* red,
                                   int64_t t0, int64_t tstr, int64_t hoff,
                                   bf16_t* dr, bf16_t* dw, bf16_t* dk,
                                   bf16_t* dv, bf16_t* da, bf16_t* db,
                                   int tid) {
    constexpr int SUB = 4, CPT = CN / NW, NTH = NW * 64;
    const int i = tid / NW, qq = tid % NW, wv = tid >> 6, lane = tid & 63;
    float dS[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) dS[c] = Df[i * 65 + CPT * qq + c];
    auto ld = [&](int vec, int t, int jj) {
        return bf16_to_f32(raw[vec][t][jj]);
    };
    const int nsb = (n + SUB - 1) / SUB;
    for (int sb = nsb - 1; sb >= 0; --sb) {
        const int ts = sb * SUB;
        const int cnt = n - ts < SUB ? n - ts : SUB;
        float St[SUB + 1][CPT];
        float sa_r[SUB];
#pragma unroll
        for (int c = 0; c < CPT; ++c) St[0][c] = Sf[i * 65 + CPT * qq + c];
        for (int t = 0; t < ts; ++t) {
            float sa = 0.f;
#pragma unroll
            for (int c = 0; c < CPT; ++c)
                sa += St[0][c] * ld(4, t, CPT * qq + c);
            sa = group_sum<NW>(sa);
            const float vi = ld(3, t, i);
#pragma unroll
            for (int c = 0; c < CPT; ++c) {
                const int jj = CPT * qq + c;
                St[0][c] = St[0][c] * expf(-expf(ld(1, t, jj))) +
                           sa * ld(5, t, jj) + vi * ld(2, t, jj);
            }
        }
#pragma unroll
        for (int u = 0; u < SUB; ++u) {
            if (u < cnt) {
                const int t = ts + u;
                float sa = 0.f;
#pragma unroll
                for (int c = 0; c < CPT; ++c)
                    sa += St[u][c] * ld(4, t, CPT * qq + c);
                sa = group_sum<NW>(sa);
                sa_r[u] = sa;
                const float vi = ld(3, t, i);
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    const int jj = CPT * qq + c;
                    St[u + 1][c] = St[u][c] * expf(-expf(ld(1, t, jj))) +
                                   sa * ld(5, t, jj) + vi * ld(2, t, jj);
                }
            }
        }
#pragma unroll
        for (int u = SUB - 1; u >= 0; --u) {
            if (u < cnt) {
                const int t = ts + u;
                const float dyi = ld(6, t, i), vi = ld(3, t, i);
                const float sa = sa_r[u];
                float G[CPT];
                float dsa = 0.f, dvv = 0.f;
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    const int jj = CPT * qq + c;
                    G[c] = dS[c] + dyi * ld(0, t, jj);
                    dsa += G[c] * ld(5, t, jj);
                    dvv += G[c] * ld(2, t, jj);
                }
                dsa = group_sum<NW>(dsa);
                dvv = group_sum<NW>(dvv);
                if (qq == 0) dv[(t0 + t) * tstr + hoff + i] = to_bf16(dvv);
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    float p[5];
                    p[0] = St[u + 1][c] * dyi;  // dr
                    p[1] = G[c] * St[u][c];     // d decay
                    p[2] = G[c] * sa;           // dkka
                    p[3] = G[c] * vi;           // dk
                    p[4] = St[u][c] * dsa;      // dneg_kk
#pragma unroll
                    for (int q = 0; q < 5; ++q) {
                        float x = cross_group_sum<NW, 64>(p[q]);
                        if (lane < NW) red[(wv * 5 + q) * CN + CPT * qq + c] = x;
                    }
                }
                __syncthreads();
                for (int e = tid; e < 5 * CN; e += NTH) {
                    const int q = e / CN, jj = e % CN;
                    float s = 0.f;
#pragma unroll
                    for (int w2 = 0; w2 < NTH / 64; ++w2)
                        s += red[(w2 * 5 + q) * CN + jj];
                    const int64_t off = (t0 + t) * tstr + hoff + jj;
                    if (q == 0) {
                        dr[off] = to_bf16(s);
                    } else if (q == 1) {
                        const float ew = expf(ld(1, t, jj));
                        dw[off] = to_bf16(s * (-ew * expf(-ew)));
                    } else if (q == 2) {
                        db[off] = to_bf16(s);
                    } else if (q == 3) {
                        dk[off] = to_bf16(s);
                    } else {
                        da[off] = to_bf16(s);
                    }
                }
                __syncthreads();
#pragma unroll
                for (int c = 0; c < CPT; ++c) {
                    const int jj = CPT * qq + c;
                    dS[c] = G[c] * expf(-expf(ld(1, t, jj))) +
                            dsa * ld(4, t, jj);
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) Df[i * 65 + CPT * qq + c] = dS[c];
}

template <int L>
__global__ void __launch_bounds__(BWD_THREADS)
wkv7_chunk_bwd_kernel(int64_t T, int64_t BH, VecLayout lay,
                      const bf16_t* __restrict__ r,
                      const bf16_t* __restrict__ w,
                      const bf16_t* __restrict__ k,
                      const bf16_t* __restrict__ v,
                      const bf16_t* __restrict__ a,
                      const bf16_t* __restrict__ b,
                      const bf16_t* __restrict__ dy,
                      const float* __restrict__ ds_t,
                      const bf16_t* __restrict__ ckpt, bf16_t* dr, bf16_t* dw,
                      bf16_t* dk, bf16_t* dv, bf16_t* da, bf16_t* db,
                      float* ds0) {
    using Sm = BwdSmem<L>;
    constexpr int NW = BWD_WAVES, NTH = BWD_THREADS;
    constexpr int PL = Sm::PL, NB = Sm::NB;
    constexpr int CPL = chunk::LaneFactors<L, NW>::CPL;
    constexpr int TPM = NB * (NB + 1) / 2;  // lower tiles of an L x L matrix
    static_assert(L == 16 || L == 32, "chunk length");
    __shared__ Sm sm;

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = blockIdx.x;
    const int64_t sbase = bh * CN * CN;
    const int64_t hoff = lay.head(bh, CN);  // the head's vector offset
    const int64_t NN = CN * CN;
    const chunk::VecPtrs src{r, w, k, v, a, b, dy};
    const int64_t nch = (T + L - 1) / L;

    // ---- state-layout tiles: wave wv holds tiles si = 2wv, 2wv+1 of the
    // transposed 64 x 64 matrices D, S_0, S_L: rows j = 16*(si >> 2) +
    // 4*lq + e, column i = 16*(si & 3) + lr
    int toff[2];
    f32x4_t D[2], SL[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
        toff[q] = (16 * ib + lr) * CN + 16 * jb + 4 * lq;
        D[q] = zero4();
        if (ds_t) {
            const float4 x =
                *reinterpret_cast<const float4*>(ds_t + sbase + toff[q]);
            D[q][0] = x.x; D[q][1] = x.y; D[q][2] = x.z; D[q][3] = x.w;
        }
        SL[q] = unpack4(*reinterpret_cast<const uint2*>(
            ckpt + nch * BH * NN + sbase + toff[q]));
    }

    if (tid == 0) sm.flag = 0;
    {
        bf16_t(*const mats[4])[PL] = {sm.dArb, sm.dArk, sm.dAab, sm.dAak};
        chunk::zero_upper<L>(mats, 4, tid, NTH);
    }

    // ---- the chunk's vectors and S_0, prefetched one chunk ahead --------
    // HBM addresses are a per-chunk scalar base plus a 32-bit per-lane
    // offset (t * ts + column, ts the token stride; the host keeps L * ts
    // below 2^31).
    constexpr int SEGV = 7 * L * 8;  // 16-byte segments of the 7 vectors
    constexpr int NPRE = (SEGV + NTH - 1) / NTH;
    static_assert(CN * CN * 2 / 16 == NTH, "one S_0 segment per thread");
    static_assert((8 * L) % 64 == 0 && SEGV % 64 == 0,
                  "each wave loads from one vector");
    const uint32_t TS = uint32_t(lay.ts);
    // part p of this wave: one vector (the same for all 64 lanes), or none
    const bf16_t* vp[NPRE];
#pragma unroll
    for (int p = 0; p < NPRE; ++p) {
        const int wseg = __builtin_amdgcn_readfirstlane((p * NTH + tid) & ~63);
        vp[p] = wseg < SEGV ? src.get(wseg / (8 * L)) : nullptr;
    }
    uint4 pre[NPRE], pres;
    // part p < NPRE: one 16-byte segment of the vectors; part NPRE: S_0
    // (lane offsets are formed at each fetch: kept across the loop they
    // would hold registers for the whole run)
    auto fetch_part = [&](int64_t cc, int part, int tidv) {
        const int64_t cbase = cc * L * lay.ts + hoff;
        const int ncc = int(T - cc * L < L ? T - cc * L : L);
#pragma unroll
        for (int p = 0; p < NPRE; ++p) {
            if (p == part) {
                const uint32_t seg = uint32_t(p * NTH + tidv);
                const uint32_t t = (seg >> 3) & (L - 1), s8 = seg & 7;
                pre[p] = make_uint4(0, 0, 0, 0);
                if (vp[p] != nullptr && int(t) < ncc)
                    pre[p] = *reinterpret_cast<const uint4*>(
                        (vp[p] + cbase) + (t * TS + s8 * 8));
            }
        }
        if (part == NPRE)
            pres = *reinterpret_cast<const uint4*>(
                (ckpt + cc * BH * NN + sbase) + uint32_t(8 * tidv));
    };
    auto fetch = [&](int64_t cc, int tidv) {
#pragma unroll
        for (int p = 0; p <= NPRE; ++p) fetch_part(cc, p, tidv);
    };
    auto stash = [&]() {
#pragma unroll
        for (int p = 0; p < NPRE; ++p) {
            const int seg = p * NTH + tid;
            if (seg < SEGV) {
                const int row = seg >> 3, s8 = seg & 7;
                *reinterpret_cast<uint4*>(&sm.raw[row / L][row % L][s8 * 8]) =
                    pre[p];
            }
        }
        *reinterpret_cast<uint4*>(&sm.S0s[tid >> 3][8 * (tid & 7)]) = pres;
    };
    fetch(nch - 1, tid);
    stash();
    // everything loaded before the loop has arrived: the loop's waits then
    // only count the prefetch and the stores
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // Each chunk's HBM traffic is spread over its phases instead of one
    // burst per chunk: the previous chunk's S_0 (phase 2) and vectors (a
    // part per phase, 3 .. 5) are fetched early enough to have arrived by
    // the stash in phase 7.  The gradients computed in phase 7 are staged in
    // LDS (stg) and written at the start of the next chunk as whole 128-byte
    // token rows, 16 bytes a lane: a lane's own elements would give every
    // store 32 rows of 8 or 16 bytes each.
    constexpr int SEGG = 6 * L * 8;  // 16-byte segments of the staged rows
    constexpr int NFL = (SEGG + NTH - 1) / NTH;
    static_assert((8 * L) % 64 == 0, "each wave stores one gradient");
    int64_t pend_cbase = -1;  // the staged chunk's scalar base (-1: none)
    int pend_n = 0;           // its valid tokens
    auto flush = [&](int tidv) {
#pragma unroll
        for (int p = 0; p < NFL; ++p) {
            const int seg = p * NTH + tidv;
            const int wseg = __builtin_amdgcn_readfirstlane(seg & ~63);
            const int g = wseg / (8 * L);
            const uint32_t t = (uint32_t(seg) >> 3) & (L - 1), s8 = seg & 7;
            if (wseg < SEGG && int(t) < pend_n) {
                bf16_t* dst = g == 0   ? dr
                              : g == 1 ? dw
                              : g == 2 ? dk
                              : g == 3 ? da
                              : g == 4 ? db
                                       : dv;
                *reinterpret_cast<uint4*>((dst + pend_cbase) +
                                          (t * TS + s8 * 8)) =
                    *reinterpret_cast<const uint4*>(&sm.stg[g][t][8 * s8]);
            }
        }
    };

    for (int64_t c = nch - 1; c >= 0; --c) {
        const int64_t t0 = c * L;
        const int n = int(T - t0 < L ? T - t0 : L);
        // Lane-derived LDS addresses are formed inside each iteration: hoisted
        // out of the loop they would each hold a register for the whole run.
        int tid_it = threadIdx.x;
        asm volatile("" : "+v"(tid_it));
        const int tid = tid_it, lane = tid & 63, lr = lane & 15, lq = lane >> 4;
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        // dV tile of this wave: rows i = 16*vib + 4*lq + e, column
        // s = 16*vsb + lr
        const int vib = wv & 3, vsb = wv >> 2;
        const bool has_v = vsb < NB;
        int toff[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
            toff[q] = (16 * ib + lr) * CN + 16 * jb + 4 * lq;
        }

        // ================= 1: factors; S_0 tiles =========================
        if (pend_cbase >= 0) flush(tid);  // the previous chunk's gradients
        chunk::LaneFactors<L, NW> fl;
        chunk::chunk_factors<L, NW>(sm.raw, n, wv, lane, sm.At, sm.Rt, sm.Bt,
                                    sm.Kt, sm.eL, sm.eRef, sm.eLR, &sm.flag,
                                    fl);
        // fl keeps r, k, neg_kk, kka of the lane's elements (fp32) for the
        // decay gradient after the chunk's vectors have been replaced
        f32x4_t S0[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
            S0[q] = unpack4(*reinterpret_cast<const uint2*>(
                &sm.S0s[16 * ib + lr][16 * jb + 4 * lq]));
        }
        __syncthreads();
        // read once: thread 0 clears the flag again at the end of the chunk
        const bool fallback = sm.flag != 0;

        if (fallback) {
            // ---- exact sequential reverse pass for this chunk -------------
            pend_cbase = -1;
            if (c >= 1) fetch(c - 1, tid);
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int at = (toff[q] / CN) * 65 + toff[q] % CN + e;
                    sm.fb.Sf[at] = S0[q][e];
                    sm.fb.Df[at] = D[q][e];
                }
            __syncthreads();
            seq_chunk_backward<L, NW>(sm.raw, n, sm.fb.Sf, sm.fb.Df, sm.fb.red,
                                      t0, lay.ts, hoff, dr, dw, dk, dv, da, db,
                                      tid);
            __syncthreads();
            if (c >= 1) stash();
            chunk::wait_vmem();
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    D[q][e] = sm.fb.Df[(toff[q] / CN) * 65 + toff[q] % CN + e];
        } else {
            // ================= 2 ==========================================
            if (c >= 1) fetch_part(c - 1, NPRE, tid);  // S_0 first
            // S' = S_0 e^{g_ref} and D' = D e^{g_L - g_ref} ([i][j]);
            // sum_i D[i][j] S_L[i][j] per column (the decay's tail)
            {
                float tl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
                    const int j = 16 * jb + 4 * lq;
                    const float4 er =
                        *reinterpret_cast<const float4*>(&sm.eRef[j]);
                    const float4 elr =
                        *reinterpret_cast<const float4*>(&sm.eLR[j]);
                    f32x4_t sp, dp;
                    sp[0] = S0[q][0] * er.x; sp[1] = S0[q][1] * er.y;
                    sp[2] = S0[q][2] * er.z; sp[3] = S0[q][3] * er.w;
                    dp[0] = D[q][0] * elr.x; dp[1] = D[q][1] * elr.y;
                    dp[2] = D[q][2] * elr.z; dp[3] = D[q][3] * elr.w;
                    store_tile_bf16_t(sp, &sm.Sp[16 * ib][16 * jb], PN, lane);
                    store_tile_bf16_t(dp, &sm.Dl[16 * ib][16 * jb], PN, lane);
#pragma unroll
                    for (int e = 0; e < 4; ++e) tl[e] += D[q][e] * SL[q][e];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) tl[e] = chunk::row_sum16(tl[e]);
                if (lr == 0) {
                    const int j = 16 * ((2 * wv) >> 2) + 4 * lq;
                    *reinterpret_cast<float4*>(&sm.part[wv & 1][j]) =
                        make_float4(tl[0], tl[1], tl[2], tl[3]);
                }
            }
            if (wv == 0) {
                chunk::minv_regs<L>(sm.At, sm.Bt, sm.m.MinvT, lane);
            } else {
                // Aak (strict), Arb, Ark (with diagonal), dArk = dY V^T
                // (with diagonal); the matrices' blocks above the diagonal
                // (overwritten by the union each chunk) are cleared
                constexpr int NJ = 4 * TPM + (NB == 2 ? 4 : 0);
                for (int ti = wv - 1; ti < NJ; ti += NW - 1) {
                    if (ti < 4 * TPM) {
                        const int mat = ti / TPM;
                        int tb, sb;
                        chunk::lower_tile_index(ti % TPM, tb, sb);
                        chunk::lower_tile<L>(
                            mat == 0 ? sm.At : mat == 3 ? sm.raw[6] : sm.Rt,
                            mat == 1 ? sm.Bt : mat == 3 ? sm.raw[3] : sm.Kt,
                            mat == 0   ? sm.m.Aak
                            : mat == 1 ? sm.m.Arb
                            : mat == 2 ? sm.m.Ark
                                       : sm.dArk,
                            tb, sb, mat == 0, lane);
                    } else {
                        const int m = ti - 4 * TPM;
                        bf16_t(*dst)[PL] = m == 0   ? sm.m.Aak
                                           : m == 1 ? sm.m.Arb
                                           : m == 2 ? sm.m.Ark
                                                    : sm.m.MinvT;
                        store_tile_bf16_t(zero4(), &dst[16][0], PL, lane);
                    }
                }
            }
            __syncthreads();

            // ================= 3 ==========================================
            if (c >= 1) fetch_part(c - 1, 0, tid);
            {
                // U = A~ S'^T + Aak V -> Ut[i][t];
                // dX = B~ D'^T + Arb^T dY -> dXt[i][t].  NB = 2: every wave
                // the U and the dX tile (t block wv / 4, i block wv % 4);
                // NB = 1: waves 0-3 U, waves 4-7 dX.
#pragma unroll
                for (int it = 0; it < NB; ++it) {
                    const bool isX = NB == 2 ? it == 1 : wv >= 4;
                    const int tb = NB == 2 ? wv >> 2 : 0, ib = wv & 3;
                    f32x4_t acc = zero4();
                    if (!isX) {
#pragma unroll
                        for (int k0 = 0; k0 < CN; k0 += 32)
                            mfma(acc, frag_rk(&sm.At[16 * tb][k0], PN, lane),
                                 frag_rk(&sm.Sp[16 * ib][k0], PN, lane));
                        mfma(acc, fkr<L>(&sm.m.Aak[0][16 * tb], PL, lane),
                             fkr<L>(&sm.raw[3][0][16 * ib], PN, lane));
                        store_tile_bf16_t(acc, &sm.m.Ut[16 * ib][16 * tb], PL,
                                          lane);
                    } else {
#pragma unroll
                        for (int k0 = 0; k0 < CN; k0 += 32)
                            mfma(acc, frag_rk(&sm.Bt[16 * tb][k0], PN, lane),
                                 frag_rk(&sm.Dl[16 * ib][k0], PN, lane));
                        mfma(acc, frk<L>(&sm.m.Arb[16 * tb][0], PL, lane),
                             fkr<L>(&sm.raw[6][0][16 * ib], PN, lane));
                        store_tile_bf16_t(acc, &sm.m.dXt[16 * ib][16 * tb],
                                          PL, lane);
                    }
                }
            }
            __syncthreads();

            // ================= 4 ==========================================
            if (c >= 1) fetch_part(c - 1, 1, tid);
            // X = Minv U -> X[t][i]; dU = Minv^T dX -> dU[t][i].  NB = 2:
            // every wave one X and one dU tile (t block wv / 4, i block
            // wv % 4); NB = 1: waves 0-3 X, waves 4-7 dU.
#pragma unroll
            for (int it = 0; it < NB; ++it) {
                const bool isdU = NB == 2 ? it == 1 : wv >= 4;
                const int tb = NB == 2 ? wv >> 2 : 0, ib = wv & 3;
                f32x4_t acc = zero4();
                if (!isdU) {
                    mfma(acc, frk<L>(&sm.m.Ut[16 * ib][0], PL, lane),
                         fkr<L>(&sm.m.MinvT[0][16 * tb], PL, lane));
                    store_tile_bf16_t(acc, &sm.X[16 * tb][16 * ib], PN, lane);
                } else {
                    mfma(acc, frk<L>(&sm.m.dXt[16 * ib][0], PL, lane),
                         frk<L>(&sm.m.MinvT[16 * tb][0], PL, lane));
                    store_tile_bf16_t(acc, &sm.dU[16 * tb][16 * ib], PN, lane);
                }
            }
            __syncthreads();

            // ================= 5 ==========================================
            if (c >= 1 && NPRE > 2) fetch_part(c - 1, 2, tid);
            if (c >= 1 && NPRE > 3) fetch_part(c - 1, 3, tid);
            // dArb = dY X^T (with diagonal), dAab = dU X^T, dAak = dU V^T
            // (strict)
            for (int ti = wv; ti < 3 * TPM; ti += NW) {
                const int mat = ti / TPM;
                int tb, sb;
                chunk::lower_tile_index(ti % TPM, tb, sb);
                chunk::lower_tile<L>(mat == 0 ? sm.raw[6] : sm.dU,
                                     mat == 2 ? sm.raw[3] : sm.X,
                                     mat == 0   ? sm.dArb
                                     : mat == 1 ? sm.dAab
                                                : sm.dAak,
                                     tb, sb, mat != 0, lane);
            }
            // dV = D' K~^T + dY^T Ark + dU^T Aak (transposed tile), stored
            // with the other gradients
            f32x4_t dvt = zero4();
            if (has_v) {
                f32x4_t& acc = dvt;
#pragma unroll
                for (int k0 = 0; k0 < CN; k0 += 32)
                    mfma(acc, frag_rk(&sm.Dl[16 * vib][k0], PN, lane),
                         frag_rk(&sm.Kt[16 * vsb][k0], PN, lane));
                mfma(acc, fkr<L>(&sm.raw[6][0][16 * vib], PN, lane),
                     frk<L>(&sm.m.Ark[16 * vsb][0], PL, lane));
                mfma(acc, fkr<L>(&sm.dU[0][16 * vib], PN, lane),
                     frk<L>(&sm.m.Aak[16 * vsb][0], PL, lane));
            }
            // D_0 = D e^{g_L} + (dY^T R~ + dU^T A~) e^{g_ref} (state layout)
            f32x4_t Dn[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
                f32x4_t acc = zero4();
                mfma(acc, fkr<L>(&sm.Rt[0][16 * jb], PN, lane),
                     fkr<L>(&sm.raw[6][0][16 * ib], PN, lane));
                mfma(acc, fkr<L>(&sm.At[0][16 * jb], PN, lane),
                     fkr<L>(&sm.dU[0][16 * ib], PN, lane));
                const int j = 16 * jb + 4 * lq;
                const float4 el = *reinterpret_cast<const float4*>(&sm.eL[j]);
                const float4 er =
                    *reinterpret_cast<const float4*>(&sm.eRef[j]);
                Dn[q][0] = D[q][0] * el.x + acc[0] * er.x;
                Dn[q][1] = D[q][1] * el.y + acc[1] * er.y;
                Dn[q][2] = D[q][2] * el.z + acc[2] * er.z;
                Dn[q][3] = D[q][3] * el.w + acc[3] * er.w;
            }
            __syncthreads();

            // ================= 6 ==========================================
            // one transposed tile (t block tb, j block jb) of dR~, dA~, dB~
            // or dK~ (gsel 0 .. 3)
            auto grad_tile = [&](int gsel, int tb, int jb) {
                f32x4_t acc = zero4();
                float(*gdst)[CN + 4];
                if (gsel == 0) {
                    // dR~ = dY S' + dArb B~ + dArk K~
#pragma unroll
                    for (int k0 = 0; k0 < CN; k0 += 32)
                        mfma(acc, frag_kr(&sm.Sp[k0][16 * jb], PN, lane),
                             frag_rk(&sm.raw[6][16 * tb][k0], PN, lane));
                    mfma(acc, fkr<L>(&sm.Bt[0][16 * jb], PN, lane),
                         fkr<L>(&sm.dArb[0][16 * tb], PL, lane));
                    mfma(acc, fkr<L>(&sm.Kt[0][16 * jb], PN, lane),
                         fkr<L>(&sm.dArk[0][16 * tb], PL, lane));
                    gdst = sm.g.gR;
                } else if (gsel == 1) {
                    // dA~ = dU S' + dAab B~ + dAak K~
#pragma unroll
                    for (int k0 = 0; k0 < CN; k0 += 32)
                        mfma(acc, frag_kr(&sm.Sp[k0][16 * jb], PN, lane),
                             frag_rk(&sm.dU[16 * tb][k0], PN, lane));
                    mfma(acc, fkr<L>(&sm.Bt[0][16 * jb], PN, lane),
                         fkr<L>(&sm.dAab[0][16 * tb], PL, lane));
                    mfma(acc, fkr<L>(&sm.Kt[0][16 * jb], PN, lane),
                         fkr<L>(&sm.dAak[0][16 * tb], PL, lane));
                    gdst = sm.g.gA;
                } else if (gsel == 2) {
                    // dB~ = dAab^T A~ + dArb^T R~ + X D'
                    mfma(acc, fkr<L>(&sm.At[0][16 * jb], PN, lane),
                         frk<L>(&sm.dAab[16 * tb][0], PL, lane));
                    mfma(acc, fkr<L>(&sm.Rt[0][16 * jb], PN, lane),
                         frk<L>(&sm.dArb[16 * tb][0], PL, lane));
#pragma unroll
                    for (int k0 = 0; k0 < CN; k0 += 32)
                        mfma(acc, frag_kr(&sm.Dl[k0][16 * jb], PN, lane),
                             frag_rk(&sm.X[16 * tb][k0], PN, lane));
                    gdst = sm.g.gB;
                } else {
                    // dK~ = dAak^T A~ + dArk^T R~ + V D'
                    mfma(acc, fkr<L>(&sm.At[0][16 * jb], PN, lane),
                         frk<L>(&sm.dAak[16 * tb][0], PL, lane));
                    mfma(acc, fkr<L>(&sm.Rt[0][16 * jb], PN, lane),
                         frk<L>(&sm.dArk[16 * tb][0], PL, lane));
#pragma unroll
                    for (int k0 = 0; k0 < CN; k0 += 32)
                        mfma(acc, frag_kr(&sm.Dl[k0][16 * jb], PN, lane),
                             frag_rk(&sm.raw[3][16 * tb][k0], PN, lane));
                    gdst = sm.g.gK;
                }
                *reinterpret_cast<float4*>(
                    &gdst[16 * tb + lr][16 * jb + 4 * lq]) =
                    make_float4(acc[0], acc[1], acc[2], acc[3]);
            };
            // transposed tiles of dR~, dA~, dB~, dK~ -> g[t][j] (fp32).
            // NB = 2: every wave the (t block wv / 4, j block wv % 4) tile of
            // all four, two at a time; NB = 1: two of the four (wv / 4 picks
            // which), j block wv % 4.
            if constexpr (NB == 2) {
                // the two tiles of a pair share their S' or D' fragments and
                // the factor fragments (loaded once)
                const int tb = wv >> 2, jb = wv & 3;
                auto store_g = [&](float(*gdst)[CN + 4], const f32x4_t& acc) {
                    *reinterpret_cast<float4*>(
                        &gdst[16 * tb + lr][16 * jb + 4 * lq]) =
                        make_float4(acc[0], acc[1], acc[2], acc[3]);
                };
                {
                    // dR~ = dY S' + dArb B~ + dArk K~,
                    // dA~ = dU S' + dAab B~ + dAak K~
                    f32x4_t aR = zero4(), aA = zero4();
#pragma unroll
                    for (int k0 = 0; k0 < CN; k0 += 32) {
                        const bf16x8_t sp = frag_kr(&sm.Sp[k0][16 * jb], PN, lane);
                        mfma(aR, sp, frag_rk(&sm.raw[6][16 * tb][k0], PN, lane));
                        mfma(aA, sp, frag_rk(&sm.dU[16 * tb][k0], PN, lane));
                    }
                    const bf16x8_t fb = fkr<L>(&sm.Bt[0][16 * jb], PN, lane);
                    const bf16x8_t fk = fkr<L>(&sm.Kt[0][16 * jb], PN, lane);
                    mfma(aR, fb, fkr<L>(&sm.dArb[0][16 * tb], PL, lane));
                    mfma(aA, fb, fkr<L>(&sm.dAab[0][16 * tb], PL, lane));
                    mfma(aR, fk, fkr<L>(&sm.dArk[0][16 * tb], PL, lane));
                    mfma(aA, fk, fkr<L>(&sm.dAak[0][16 * tb], PL, lane));
                    store_g(sm.g.gR, aR);
                    store_g(sm.g.gA, aA);
                }
                __builtin_amdgcn_sched_barrier(0);
                {
                    // dB~ = dAab^T A~ + dArb^T R~ + X D',
                    // dK~ = dAak^T A~ + dArk^T R~ + V D'
                    f32x4_t aB = zero4(), aK = zero4();
                    const bf16x8_t fa = fkr<L>(&sm.At[0][16 * jb], PN, lane);
                    const bf16x8_t fr = fkr<L>(&sm.Rt[0][16 * jb], PN, lane);
                    mfma(aB, fa, frk<L>(&sm.dAab[16 * tb][0], PL, lane));
                    mfma(aK, fa, frk<L>(&sm.dAak[16 * tb][0], PL, lane));
                    mfma(aB, fr, frk<L>(&sm.dArb[16 * tb][0], PL, lane));
                    mfma(aK, fr, frk<L>(&sm.dArk[16 * tb][0], PL, lane));
#pragma unroll
                    for (int k0 = 0; k0 < CN; k0 += 32) {
                        const bf16x8_t dl = frag_kr(&sm.Dl[k0][16 * jb], PN, lane);
                        mfma(aB, dl, frag_rk(&sm.X[16 * tb][k0], PN, lane));
                        mfma(aK, dl, frag_rk(&sm.raw[3][16 * tb][k0], PN, lane));
                    }
                    store_g(sm.g.gB, aB);
                    store_g(sm.g.gK, aK);
                }
            } else {
                grad_tile(wv >> 2, 0, wv & 3);
                grad_tile(2 + (wv >> 2), 0, wv & 3);
            }
            __syncthreads();

            // ================= 7: input gradients ===========================
            // The chunk's vectors are no longer read: the previous chunk's go
            // to LDS first, so that waiting for their loads does not also wait
            // for this chunk's stores (one counter covers loads and stores).
            if (c >= 1) stash();
            chunk::wait_vmem();
            {
                const int t = fl.t, j0 = fl.j0;
                float gRv[CPL], gAv[CPL], gBv[CPL], gKv[CPL];
                auto ldg = [&](const float(*g)[CN + 4], float* dst) {
#pragma unroll
                    for (int e = 0; e < CPL; ++e) dst[e] = g[t][j0 + e];
                };
                ldg(sm.g.gR, gRv); ldg(sm.g.gA, gAv);
                ldg(sm.g.gB, gBv); ldg(sm.g.gK, gKv);
                const float *rv = fl.r, *kv = fl.k, *av = fl.a, *bv = fl.b;
                float drv[CPL], dav[CPL], dbv[CPL], dkv[CPL], dwv[CPL];
                constexpr float kLn2 = 0.6931471805599453f;
#pragma unroll
                for (int e = 0; e < CPL; ++e) {
                    drv[e] = gRv[e] * fl.eg[e];
                    dav[e] = gAv[e] * fl.eprev[e];
                    dbv[e] = gBv[e] * fl.eng[e];
                    dkv[e] = gKv[e] * fl.eng[e];
                    const float f = rv[e] * drv[e] - bv[e] * dbv[e] -
                                    kv[e] * dkv[e] +
                                    chunk::next_token<L>(av[e] * dav[e],
                                                         lane);
                    const float tail =
                        sm.part[0][j0 + e] + sm.part[1][j0 + e];
                    dwv[e] = (chunk::suffix_scan_lanes<L>(f, lane) + tail) *
                             fl.lam[e] * kLn2;
                }
                // stage the gradients (the rows of padding tokens are
                // staged but never written out)
                chunk::store_cols<CPL>(&sm.stg[0][t][j0], drv);
                chunk::store_cols<CPL>(&sm.stg[1][t][j0], dwv);
                chunk::store_cols<CPL>(&sm.stg[2][t][j0], dkv);
                chunk::store_cols<CPL>(&sm.stg[3][t][j0], dav);
                chunk::store_cols<CPL>(&sm.stg[4][t][j0], dbv);
                if (has_v)
                    store_tile_bf16_t(dvt, &sm.stg[5][16 * vsb][16 * vib], PN,
                                      lane);
                pend_cbase = t0 * lay.ts + hoff;
                pend_n = n;
            }
            D[0] = Dn[0];
            D[1] = Dn[1];
        }
        SL[0] = S0[0];
        SL[1] = S0[1];
        if (tid == 0) sm.flag = 0;
        __syncthreads();
    }
    if (pend_cbase >= 0) flush(tid);
#pragma unroll
    for (int q = 0; q < 2; ++q)
        *reinterpret_cast<float4*>(ds0 + sbase + toff[q]) =
            make_float4(D[q][0], D[q][1], D[q][2], D[q][3]);
}

template <int L>
hipError_t launch_l(const ChunkBwdArgs& p, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_chunk_bwd_kernel<L>), dim3(unsigned(BH)),
                       dim3(BWD_THREADS), 0, stream, p.T, BH, p.lay,
                       static_cast<const bf16_t*>(p.r),
                       static_cast<const bf16_t*>(p.w),
                       static_cast<const bf16_t*>(p.k),
                       static_cast<const bf16_t*>(p.v),
                       static_cast<const bf16_t*>(p.a),
                       static_cast<const bf16_t*>(p.b),
                       static_cast<const bf16_t*>(p.dy), p.ds_t,
                       static_cast<const bf16_t*>(p.ckpt),
                       static_cast<bf16_t*>(p.dr), static_cast<bf16_t*>(p.dw),
                       static_cast<bf16_t*>(p.dk), static_cast<bf16_t*>(p.dv),
                       static_cast<bf16_t*>(p.da), static_cast<bf16_t*>(p.db),
                       p.ds0);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_chunk_backward(const ChunkBwdArgs& p, hipStream_t stream) {
    switch (p.L) {
        case 16: return launch_l<16>(p, stream);
        case 32: return launch_l<32>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rwkv7m
