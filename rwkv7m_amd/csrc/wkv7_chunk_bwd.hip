// Chunked WKV-7 backward for gfx950: bf16 vectors, fp32 state, N = 64,
// chunk length L in {16, 32} (= the forward's checkpoint interval).
//
// One workgroup (8 waves) per (batch, head) walks the chunks in reverse.
// For each chunk it reloads the chunk-start state S_0 from the forward's
// checkpoints, rebuilds the forward's factors (see wkv7_chunk_fwd.hip:
// A~, R~, B~, K~, B^, K^, Aab, Aak, Arb, Ark, Minv, U, X) and applies the
// adjoint of every product.  With D the cotangent of the chunk-end state
// S_L and dY the cotangent of the chunk's outputs:
//
//   dX  = B^ D^T + Arb^T dY          dU  = Minv^T dX
//   dV  = K^ D^T + Ark^T dY + Aak^T dU
//   dArb = lower(dY X^T)  dArk = lower(dY V^T)          (with diagonal)
//   dAab = slower(dU X^T) dAak = slower(dU V^T)         (strict)
//   dR~ = dY S' + dArb B~ + dArk K~     dA~ = dU S' + dAab B~ + dAak K~
//   dB~ + dB^ e^{gL-gref} = dAab^T A~ + dArb^T R~ + X D'
//   dK~ + dK^ e^{gL-gref} = dAak^T A~ + dArk^T R~ + V D'      (D' = D e^{gL-gref})
//   D_0 = D e^{gL} + (dY^T R~ + dU^T A~) e^{gref}            (cotangent of S_0)
//
// and the input gradients follow by the factors' scalings.  The decay
// gradient uses the identity (exact for the chunk with S_0 and D fixed)
//
//   dlog d_t = sum_{t' >= t} (r dr - b db - k dk)_{t'} + (a da)_{t'+1}
//              + sum_i D[i, :] S_L[i, :]
//
// and dw = dlog d * (-e^w).  These are the reference's reverse equations
// (src/rwkv7m/kernels/wkv_pallas_gpu.py:221-257) summed over a chunk; the
// states come from checkpoints (recompute), never from dividing by the
// decay.  A chunk outside the factored form's range runs an exact fp32
// sequential reverse pass instead.

#include "wkv7_chunk_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

using chunk::CN;
using chunk::kHalfRange;
using chunk::PN;

// 8 waves: every value stays in registers (a spill reload would wait for
// all HBM traffic the wave has in flight).  Every wave prefetches a share
// of the next chunk's vectors and checkpoint, one chunk ahead, and each
// chunk ends with stash (LDS <- registers), then this chunk's gradient
// stores, then the next fetch: vmcnt counts a wave's loads and stores
// together, so the wait before a stash covers only a chunk-old store.
constexpr int BWD_WAVES = 8;

template <int L>
struct BwdSmem {
    static constexpr int PL = L + 8, NB = L / 16, PG = CN + 4;
    // ---- persistent within a chunk (written by the factor pass) ----------
    bf16_t BtT[CN][PL], KtT[CN][PL], AtT[CN][PL], RtT[CN][PL];  // [j][t]
    bf16_t V[L][PN], dY[L][PN];                                  // [t][i]
    // ---- from the matrix pass on ------------------------------------------
    bf16_t AakT[L][PL], ArkT[L][PL], ArbT[L][PL];  // [s][t]
    bf16_t Minv[L][PL], MinvT[L][PL];
    // ---- state copies: S' / D ([i][j]) then S'^T / D'^T ([j][i]) --------
    bf16_t St0[CN][PN], St1[CN][PN];
    // ---- factor-pass outputs used up to the dV / D pass, then the rows of
    //      the six gradients on their way to HBM --------------------------
    union {
        struct {
            bf16_t At[L][PN], Bh[L][PN], Kh[L][PN];  // [t][j]
            bf16_t Vt[CN][PL], dYt[CN][PL];          // [i][t]
            bf16_t Aak[L][PL];                       // [t][s]
        } f;
        bf16_t gout[6][L][CN];  // dr, dw, dk, dv, dneg_kk, dkka
    };
    // ---- X, dU ([t][i]) ---------------------------------------------------
    bf16_t X[L][PN], dU[L][PN];
    union {
        struct {  // factor and matrix passes
            bf16_t raw[7][L][CN];  // r, w, k, v, neg_kk, kka, dy
            union {
                bf16_t S0f[CN][CN];  // the next chunk's S_0, staged
                struct {
                    bf16_t Rt[L][PN], Bt[L][PN], Kt[L][PN];  // [t][j]
                    bf16_t Aab[L][PL];
                    bf16_t AabTD[NB][16][24];
                    bf16_t Z[4][16][24];
                } m;
            };
        } e1;
        struct {  // U, X, dX, dU passes
            bf16_t Ut[CN][PL], dXt[CN][PL], dUt[CN][PL];  // [i][t]
        } e2;
        struct {  // Q matrices and the gradient accumulators
            bf16_t dArb[L][PL], dArk[L][PL], dAab[L][PL], dAak[L][PL];
            bf16_t dArbT[L][PL], dArkT[L][PL], dAabT[L][PL], dAakT[L][PL];
            float gR[L][PG], gA[L][PG], gB[L][PG], gK[L][PG];
        } e3;
    };
    float tot[BWD_WAVES][CN];
    float qx[BWD_WAVES][CN];
    float eL[CN], eRef[CN], eLR[CN], tail[CN];
    int flag;
};

// Exact fp32 sequential reverse pass over one chunk (the fallback for decays
// outside the factored form's range).  S_0 and D come in and D goes out
// through fp32 LDS copies Sf, Df ([64][65]); red is [NW][5][64] scratch.
// Thread: row i = tid / NW, columns CPT * (tid % NW) .. + CPT - 1.
template <int L, int NW>
__device__ void seq_chunk_backward(const bf16_t (*raw)[L][CN], int n,
                                   const float* Sf, float* Df, float* red,
                                   int64_t t0, int64_t BH, int64_t bh,
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
                if (qq == 0) dv[((t0 + t) * BH + bh) * CN + i] = to_bf16(dvv);
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
                    const int64_t off = ((t0 + t) * BH + bh) * CN + jj;
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
__global__ void __launch_bounds__(BWD_WAVES * 64)
wkv7_chunk_bwd_kernel(int64_t T, int64_t BH, const bf16_t* __restrict__ r,
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
    constexpr int NW = BWD_WAVES, NTH = NW * 64;
    constexpr int PL = Sm::PL, NB = Sm::NB, TPG = L / NW;
    constexpr int ST = 16 / NW;  // state tiles per wave
    static_assert(L % NW == 0 && 16 % NW == 0, "wave layout");
    __shared__ Sm sm;

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = blockIdx.x;
    const int64_t sbase = bh * CN * CN;
    const int64_t NN = CN * CN;
    const chunk::VecPtrs src{r, w, k, v, a, b, dy};

    // State tiles of this wave: tile si = ST*wv + q covers X[i][j] with
    // i = 16*(si & 3) + lr, j = 16*(si >> 2) + 4*lq + e.
    int toff[ST];
#pragma unroll
    for (int q = 0; q < ST; ++q) {
        const int si = ST * wv + q;
        toff[q] = (16 * (si & 3) + lr) * CN + 16 * (si >> 2) + 4 * lq;
    }
    auto load_tiles = [&](f32x4_t* dst, const float* p) {
#pragma unroll
        for (int q = 0; q < ST; ++q) {
            float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p) x = *reinterpret_cast<const float4*>(p + sbase + toff[q]);
            dst[q][0] = x.x; dst[q][1] = x.y; dst[q][2] = x.z; dst[q][3] = x.w;
        }
    };
    auto load_tiles_bf16 = [&](f32x4_t* dst, const bf16_t* p) {
#pragma unroll
        for (int q = 0; q < ST; ++q)
            dst[q] = unpack4(
                *reinterpret_cast<const uint2*>(p + sbase + toff[q]));
    };

    // ---- prefetch: the next chunk's 7 vectors and S_0 --------------------
    constexpr int LOADERS = NTH;
    const int ltid = tid;
    constexpr int SEGV = 7 * L * 8;  // 16-byte segments of the 7 vectors
    constexpr int NPV = (SEGV + LOADERS - 1) / LOADERS;
    constexpr int NPS = CN * CN * 2 / 16 / LOADERS;  // S_0 segments
    static_assert(NPS * 16 * LOADERS == CN * CN * 2, "S_0 segments");
    uint4 prev[NPV];
    uint4 pres[NPS];
    auto fetch = [&](int64_t cc, int ltid) {  // chunk cc's data into registers
        const int64_t t0f = cc * L;
#pragma unroll
        for (int p = 0; p < NPV; ++p) {
            const int seg = p * LOADERS + ltid;
            prev[p] = make_uint4(0, 0, 0, 0);
            if (seg < SEGV) {
                const int row = seg >> 3, s8 = seg & 7;
                const int vec = row / L, t = row % L;
                const bf16_t* base = src.get(vec);
                if (t0f + t < T && base != nullptr)
                    prev[p] = *reinterpret_cast<const uint4*>(
                        base + ((t0f + t) * BH + bh) * CN + s8 * 8);
            }
        }
        const bf16_t* cp = ckpt + cc * BH * NN + sbase;
#pragma unroll
        for (int p = 0; p < NPS; ++p)
            pres[p] = *reinterpret_cast<const uint4*>(cp +
                                                      8 * (p * LOADERS + ltid));
    };
    auto stash = [&](int ltid) {
#pragma unroll
        for (int p = 0; p < NPV; ++p) {
            const int seg = p * LOADERS + ltid;
            if (seg < SEGV) {
                const int row = seg >> 3, s8 = seg & 7;
                *reinterpret_cast<uint4*>(
                    &sm.e1.raw[row / L][row % L][s8 * 8]) = prev[p];
            }
        }
#pragma unroll
        for (int p = 0; p < NPS; ++p)
            *reinterpret_cast<uint4*>(&sm.e1.S0f[0][0] +
                                      8 * (p * LOADERS + ltid)) = pres[p];
    };

    f32x4_t D[ST], SL[ST], S0[ST];
    load_tiles(D, ds_t);
    const int64_t nchunks = (T + L - 1) / L;
    load_tiles_bf16(SL, ckpt + nchunks * BH * NN);
    fetch(nchunks - 1, ltid);
    stash(ltid);
    // everything loaded before the loop has arrived (see the forward kernel)
    __builtin_amdgcn_s_waitcnt(0);
    if (nchunks > 1) fetch(nchunks - 2, ltid);
    if (tid == 0) sm.flag = 0;
    __syncthreads();

    for (int64_t c = nchunks - 1; c >= 0; --c) {
        const int64_t t0 = c * L;
        const int n = int(T - t0 < L ? T - t0 : L);
        // Lane-derived LDS addresses are formed inside each iteration: hoisted
        // out of the loop they would each hold a register for the whole run.
        int tid_it = threadIdx.x;
        asm volatile("" : "+v"(tid_it));
        const int tid = tid_it, lane = tid & 63, lr = lane & 15, lq = lane >> 4;
        int toff[ST];
#pragma unroll
        for (int q = 0; q < ST; ++q) {
            const int si = ST * wv + q;
            toff[q] = (16 * (si & 3) + lr) * CN + 16 * (si >> 2) + 4 * lq;
        }
        // this chunk's S_0 from the staging area
#pragma unroll
        for (int q = 0; q < ST; ++q)
            S0[q] = unpack4(
                *reinterpret_cast<const uint2*>(&sm.e1.S0f[0][0] + toff[q]));

        // ---- factor pass (thread: column j = lane, tokens of group wv) ---
        const int j = lane, grp = wv;
        float lam[TPG], gg[TPG];
        uint32_t prk[TPG], pab[TPG];  // (r, k) and (a, b) as bf16 pairs
        {
            float run = 0.f;
#pragma unroll
            for (int u = 0; u < TPG; ++u) {
                const int t = grp * TPG + u;
                const float l =
                    (t < n) ? -__expf(bf16_to_f32(sm.e1.raw[1][t][j])) : 0.f;
                lam[u] = l;
                run += l;
                gg[u] = run;
            }
            sm.tot[grp][j] = run;
        }
        __syncthreads();
        float gref, off;
        {
            float G = 0.f;
            off = 0.f;
            gref = 0.f;
#pragma unroll
            for (int g2 = 0; g2 < NW; ++g2) {
                const float tv = sm.tot[g2][j];
                G += tv;
                if (g2 < grp) off += tv;
                if (g2 == NW / 2 - 1) gref = G;
            }
            if (-gref > kHalfRange || gref - G > kHalfRange) sm.flag = 1;
            if (grp == 0) {
                sm.eL[j] = __expf(G);
                sm.eRef[j] = __expf(gref);
                sm.eLR[j] = __expf(G - gref);
            }
            const float eLR = __expf(G - gref);
            float eprev = __expf(off - gref);
            bf16_t hA[TPG], hR[TPG], hB[TPG], hK[TPG], hV[TPG], hY[TPG];
#pragma unroll
            for (int u = 0; u < TPG; ++u) {
                const int t = grp * TPG + u;
                gg[u] += off;
                const float eg = __expf(gg[u] - gref);
                const float eng = __expf(gref - gg[u]);
                const float egl = eLR * eng;
                const bf16_t ra = sm.e1.raw[4][t][j], rr = sm.e1.raw[0][t][j];
                const bf16_t rk = sm.e1.raw[2][t][j], rb = sm.e1.raw[5][t][j];
                prk[u] = uint32_t(rr) | (uint32_t(rk) << 16);
                pab[u] = uint32_t(ra) | (uint32_t(rb) << 16);
                const float av = bf16_to_f32(ra), rv = bf16_to_f32(rr);
                const float kv = bf16_to_f32(rk), bv = bf16_to_f32(rb);
                hV[u] = sm.e1.raw[3][t][j];
                hY[u] = sm.e1.raw[6][t][j];
                hA[u] = to_bf16(av * eprev);
                hR[u] = to_bf16(rv * eg);
                hB[u] = to_bf16(bv * eng);
                hK[u] = to_bf16(kv * eng);
                sm.f.At[t][j] = hA[u];
                sm.e1.m.Rt[t][j] = hR[u];
                sm.e1.m.Bt[t][j] = hB[u];
                sm.e1.m.Kt[t][j] = hK[u];
                sm.f.Bh[t][j] = to_bf16(bv * egl);
                sm.f.Kh[t][j] = to_bf16(kv * egl);
                sm.V[t][j] = hV[u];
                sm.dY[t][j] = hY[u];
                eprev = eg;
            }
            chunk::put_row<TPG>(&sm.AtT[j][grp * TPG], hA);
            chunk::put_row<TPG>(&sm.RtT[j][grp * TPG], hR);
            chunk::put_row<TPG>(&sm.BtT[j][grp * TPG], hB);
            chunk::put_row<TPG>(&sm.KtT[j][grp * TPG], hK);
            chunk::put_row<TPG>(&sm.f.Vt[j][grp * TPG], hV);
            chunk::put_row<TPG>(&sm.f.dYt[j][grp * TPG], hY);
        }
        __syncthreads();
        // read once: thread 0 clears the flag again at the end of the chunk
        const bool fallback = sm.flag != 0;

        if (fallback) {
            // ---- exact sequential fallback for this chunk ---------------
            float* Sf = reinterpret_cast<float*>(&sm.BtT[0][0]);
            float* Df = reinterpret_cast<float*>(&sm.f.At[0][0]);
            float* red = reinterpret_cast<float*>(&sm.AakT[0][0]);
            static_assert(offsetof(Sm, AakT) - offsetof(Sm, BtT) >= 64 * 65 * 4,
                          "Sf fits (BtT .. dY)");
            static_assert(offsetof(Sm, dU) + sizeof(sm.dU) - offsetof(Sm, f) >=
                              64 * 65 * 4,
                          "Df fits (f, X, dU are contiguous)");
            static_assert(offsetof(Sm, f) - offsetof(Sm, AakT) >= NW * 5 * 64 * 4,
                          "red fits (AakT .. St1)");
#pragma unroll
            for (int q = 0; q < ST; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    Sf[toff[q] / CN * 65 + toff[q] % CN + e] = S0[q][e];
                    Df[toff[q] / CN * 65 + toff[q] % CN + e] = D[q][e];
                }
            __syncthreads();
            seq_chunk_backward<L, NW>(sm.e1.raw, n, Sf, Df, red, t0, BH, bh,
                                      dr, dw, dk, dv, da, db, tid);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < ST; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    D[q][e] = Df[toff[q] / CN * 65 + toff[q] % CN + e];
            __syncthreads();  // Df/Sf are read before the regions are reused
        } else {
            // ---- matrix pass: Aab (+ diagonal blocks transposed), Aak (+T),
            //      ArbT, ArkT; state copies S' = S0 e^{gref} and D ([i][j])
            constexpr int NT2 = 4 * NB * NB;
#pragma unroll 1
            for (int it = 0; it < (NT2 + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < NT2) {
                    const int mat = ti / (NB * NB), rem = ti % (NB * NB);
                    const int mt = rem / NB, nt = rem % NB;
                    f32x4_t acc = zero4();
                    if (nt <= mt) {
                        const bf16_t* Aop = mat < 2 ? &sm.f.At[16 * mt][0]
                                                    : &sm.e1.m.Rt[16 * mt][0];
                        const bf16_t* Bop = (mat & 1)
                                                ? &sm.e1.m.Kt[16 * nt][0]
                                                : &sm.e1.m.Bt[16 * nt][0];
                        mma_nt<CN>(acc, Aop, PN, Bop, PN, lane);
                        const bool strict = mat < 2;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int tt = 16 * mt + 4 * lq + e;
                            const int ss = 16 * nt + lr;
                            acc[e] = (strict ? (ss < tt) : (ss <= tt)) ? acc[e]
                                                                       : 0.f;
                        }
                        if (mat == 0 && mt == nt)
                            store_tile_bf16_t(acc, &sm.e1.m.AabTD[mt][0][0], 24,
                                              lane);
                    }
                    if (mat == 0) {
                        store_tile_bf16(acc, &sm.e1.m.Aab[16 * mt][16 * nt],
                                        PL, lane);
                    } else if (mat == 1) {
                        store_tile_bf16(acc, &sm.f.Aak[16 * mt][16 * nt], PL,
                                        lane);
                        store_tile_bf16_t(acc, &sm.AakT[16 * nt][16 * mt], PL,
                                          lane);
                    } else if (mat == 2) {
                        store_tile_bf16_t(acc, &sm.ArbT[16 * nt][16 * mt], PL,
                                          lane);
                    } else {
                        store_tile_bf16_t(acc, &sm.ArkT[16 * nt][16 * mt], PL,
                                          lane);
                    }
                }
            }
            {
                float dl[ST][4];
#pragma unroll
                for (int q = 0; q < ST; ++q) {
                    const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
                    float er[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        er[e] = sm.eRef[16 * jb + 4 * lq + e];
                    uint2 p;
                    p.x = pack_bf16x2(S0[q][0] * er[0], S0[q][1] * er[1]);
                    p.y = pack_bf16x2(S0[q][2] * er[2], S0[q][3] * er[3]);
                    *reinterpret_cast<uint2*>(
                        &sm.St0[16 * ib + lr][16 * jb + 4 * lq]) = p;
                    p.x = pack_bf16x2(D[q][0], D[q][1]);
                    p.y = pack_bf16x2(D[q][2], D[q][3]);
                    *reinterpret_cast<uint2*>(
                        &sm.St1[16 * ib + lr][16 * jb + 4 * lq]) = p;
                    // decay tail: sum_i D[i][j] S_L[i][j] over this tile
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        dl[q][e] = group_sum<16>(D[q][e] * SL[q][e]);
                }
                // tiles of one j block (4 of them) are summed through LDS:
                // tot[] is free here (the factor pass read it before)
#pragma unroll
                for (int q = 0; q < ST; ++q) {
                    const int si = ST * wv + q;
                    if (lr == 0) {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            sm.tot[si & 3][16 * (si >> 2) + 4 * lq + e] = dl[q][e];
                    }
                }
            }
            __syncthreads();
            if (tid < CN)
                sm.tail[tid] = sm.tot[0][tid] + sm.tot[1][tid] +
                               sm.tot[2][tid] + sm.tot[3][tid];
            // ---- Minv on waves 0 .. NB-1; U = A~ S'^T + Aak V on the rest
            constexpr int NWB = NW - NB;
            auto upass = [&] {
#pragma unroll
                for (int it = 0; it < (4 * NB + NWB - 1) / NWB; ++it) {
                    const int ti = (wv - NB) + NWB * it;
                    if (ti < 4 * NB) {
                        const int mt = ti >> 2, ui = ti & 3;
                        f32x4_t u = zero4();
                        mma_nt<CN>(u, &sm.f.At[16 * mt][0], PN,
                                   &sm.St0[16 * ui][0], PN, lane);
                        mma_nt<L>(u, &sm.f.Aak[16 * mt][0], PL,
                                  &sm.f.Vt[16 * ui][0], PL, lane);
                        store_tile_bf16_t(u, &sm.e2.Ut[16 * ui][16 * mt], PL,
                                          lane);
                    }
                }
            };
            static_assert(sizeof(sm.e1.m.Bt) * 2 >= NB * 5 * 16 * 24 * 2,
                          "W fits");
            static_assert(offsetof(Sm, e2) + sizeof(sm.e2.Ut) <=
                              offsetof(Sm, e1) + offsetof(decltype(sm.e1), m) +
                              offsetof(decltype(sm.e1.m), Bt),
                          "U does not overlap the inverse's inputs");
            chunk::build_minv<L, NTH>(
                &sm.e1.m.Aab[0][0], sm.e1.m.AabTD, &sm.Minv[0][0],
                &sm.MinvT[0][0], sm.e1.m.Z,
                reinterpret_cast<bf16_t(*)[5][16][24]>(&sm.e1.m.Bt[0][0]), tid,
                upass);
            // ---- X^T = U^T Minv^T -> X [t][i];  dX = B^ D^T + Arb^T dY ---
            constexpr int NTX = 8 * NB;
#pragma unroll
            for (int it = 0; it < (NTX + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < 4 * NB) {
                    const int mt = ti >> 2, xi = ti & 3;
                    f32x4_t x = zero4();
                    mma_nt<L>(x, &sm.e2.Ut[16 * xi][0], PL,
                              &sm.Minv[16 * mt][0], PL, lane);
                    store_tile_bf16_t(x, &sm.X[16 * mt][16 * xi], PN, lane);
                } else if (ti < NTX) {
                    const int mt = (ti - 4 * NB) >> 2, xi = (ti - 4 * NB) & 3;
                    f32x4_t dx = zero4();
                    mma_nt<CN>(dx, &sm.f.Bh[16 * mt][0], PN,
                               &sm.St1[16 * xi][0], PN, lane);
                    mma_nt<L>(dx, &sm.ArbT[16 * mt][0], PL,
                              &sm.f.dYt[16 * xi][0], PL, lane);
                    store_tile_bf16_t(dx, &sm.e2.dXt[16 * xi][16 * mt], PL,
                                      lane);
                }
            }
            __syncthreads();
            // ---- dU = Minv^T dX -> dU [t][i], dU^T [i][t] -----------------
#pragma unroll
            for (int it = 0; it < (4 * NB + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < 4 * NB) {
                    const int mt = ti >> 2, ui = ti & 3;
                    f32x4_t du = zero4();
                    mma_nt<L>(du, &sm.MinvT[16 * mt][0], PL,
                              &sm.e2.dXt[16 * ui][0], PL, lane);
                    store_tile_bf16(du, &sm.dU[16 * mt][16 * ui], PN, lane);
                    store_tile_bf16_t(du, &sm.e2.dUt[16 * ui][16 * mt], PL,
                                      lane);
                }
            }
            __syncthreads();
            // ---- dV = K^ D^T + Ark^T dY + Aak^T dU (kept for the output);
            //      new D = D e^{gL} + (dY^T R~ + dU^T A~) e^{gref} -----------
            constexpr int NTV = 4 * NB, ITV = (NTV + NW - 1) / NW;
            f32x4_t dvt[ITV];
#pragma unroll
            for (int it = 0; it < ITV; ++it) {
                const int ti = wv + NW * it;
                dvt[it] = zero4();
                if (ti < NTV) {
                    const int mt = ti >> 2, vi = ti & 3;
                    mma_nt<CN>(dvt[it], &sm.f.Kh[16 * mt][0], PN,
                               &sm.St1[16 * vi][0], PN, lane);
                    mma_nt<L>(dvt[it], &sm.ArkT[16 * mt][0], PL,
                              &sm.f.dYt[16 * vi][0], PL, lane);
                    mma_nt<L>(dvt[it], &sm.AakT[16 * mt][0], PL,
                              &sm.e2.dUt[16 * vi][0], PL, lane);
                }
            }
            f32x4_t Dn[ST];
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
                f32x4_t acc = zero4();
                mma_nt<L>(acc, &sm.RtT[16 * jb][0], PL, &sm.f.dYt[16 * ib][0],
                          PL, lane);
                mma_nt<L>(acc, &sm.AtT[16 * jb][0], PL, &sm.e2.dUt[16 * ib][0],
                          PL, lane);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int jj = 16 * jb + 4 * lq + e;
                    Dn[q][e] = D[q][e] * sm.eL[jj] + acc[e] * sm.eRef[jj];
                }
            }
            __syncthreads();
            // ---- Q matrices; S'^T, D'^T ([j][i]) --------------------------
#pragma unroll 1
            for (int it = 0; it < (NT2 + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < NT2) {
                    const int mat = ti / (NB * NB), rem = ti % (NB * NB);
                    const int mt = rem / NB, nt = rem % NB;
                    f32x4_t acc = zero4();
                    if (nt <= mt) {
                        const bf16_t* Aop = mat < 2 ? &sm.dY[16 * mt][0]
                                                    : &sm.dU[16 * mt][0];
                        const bf16_t* Bop = (mat & 1) ? &sm.V[16 * nt][0]
                                                      : &sm.X[16 * nt][0];
                        mma_nt<CN>(acc, Aop, PN, Bop, PN, lane);
                        const bool strict = mat >= 2;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int tt = 16 * mt + 4 * lq + e;
                            const int ss = 16 * nt + lr;
                            acc[e] = (strict ? (ss < tt) : (ss <= tt)) ? acc[e]
                                                                       : 0.f;
                        }
                    }
                    bf16_t(*qm)[PL] = mat == 0   ? sm.e3.dArb
                                      : mat == 1 ? sm.e3.dArk
                                      : mat == 2 ? sm.e3.dAab
                                                 : sm.e3.dAak;
                    bf16_t(*qt)[PL] = mat == 0   ? sm.e3.dArbT
                                      : mat == 1 ? sm.e3.dArkT
                                      : mat == 2 ? sm.e3.dAabT
                                                 : sm.e3.dAakT;
                    store_tile_bf16(acc, &qm[16 * mt][16 * nt], PL, lane);
                    store_tile_bf16_t(acc, &qt[16 * nt][16 * mt], PL, lane);
                }
            }
#pragma unroll
            for (int q = 0; q < ST; ++q) {
                const int si = ST * wv + q, jb = si >> 2, ib = si & 3;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int jj = 16 * jb + 4 * lq + e, ii = 16 * ib + lr;
                    sm.St0[jj][ii] = to_bf16(S0[q][e] * sm.eRef[jj]);
                    sm.St1[jj][ii] = to_bf16(D[q][e] * sm.eLR[jj]);
                }
                D[q] = Dn[q];
            }
            __syncthreads();
            // ---- gradients of the factors (fp32 to LDS) -------------------
            // tiles: 4 gradients x NB token blocks x 4 column blocks
            constexpr int NTG = 16 * NB;
#pragma unroll 1
            for (int it = 0; it < (NTG + NW - 1) / NW; ++it) {
                const int ti = wv + NW * it;
                if (ti < NTG) {
                    const int gsel = ti / (4 * NB), rem = ti % (4 * NB);
                    const int mt = rem >> 2, jb = rem & 3;
                    f32x4_t g = zero4();
                    float(*gdst)[Sm::PG];
                    if (gsel == 0) {  // dR~ = dY S' + dArb B~ + dArk K~
                        mma_nt<CN>(g, &sm.dY[16 * mt][0], PN,
                                   &sm.St0[16 * jb][0], PN, lane);
                        mma_nt<L>(g, &sm.e3.dArb[16 * mt][0], PL,
                                  &sm.BtT[16 * jb][0], PL, lane);
                        mma_nt<L>(g, &sm.e3.dArk[16 * mt][0], PL,
                                  &sm.KtT[16 * jb][0], PL, lane);
                        gdst = sm.e3.gR;
                    } else if (gsel == 1) {  // dA~ = dU S' + dAab B~ + dAak K~
                        mma_nt<CN>(g, &sm.dU[16 * mt][0], PN,
                                   &sm.St0[16 * jb][0], PN, lane);
                        mma_nt<L>(g, &sm.e3.dAab[16 * mt][0], PL,
                                  &sm.BtT[16 * jb][0], PL, lane);
                        mma_nt<L>(g, &sm.e3.dAak[16 * mt][0], PL,
                                  &sm.KtT[16 * jb][0], PL, lane);
                        gdst = sm.e3.gA;
                    } else if (gsel == 2) {  // dB' = dAab^T A~ + dArb^T R~ + X D'
                        mma_nt<L>(g, &sm.e3.dAabT[16 * mt][0], PL,
                                  &sm.AtT[16 * jb][0], PL, lane);
                        mma_nt<L>(g, &sm.e3.dArbT[16 * mt][0], PL,
                                  &sm.RtT[16 * jb][0], PL, lane);
                        mma_nt<CN>(g, &sm.X[16 * mt][0], PN,
                                   &sm.St1[16 * jb][0], PN, lane);
                        gdst = sm.e3.gB;
                    } else {  // dK' = dAak^T A~ + dArk^T R~ + V D'
                        mma_nt<L>(g, &sm.e3.dAakT[16 * mt][0], PL,
                                  &sm.AtT[16 * jb][0], PL, lane);
                        mma_nt<L>(g, &sm.e3.dArkT[16 * mt][0], PL,
                                  &sm.RtT[16 * jb][0], PL, lane);
                        mma_nt<CN>(g, &sm.V[16 * mt][0], PN,
                                   &sm.St1[16 * jb][0], PN, lane);
                        gdst = sm.e3.gK;
                    }
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        gdst[16 * mt + 4 * lq + e][16 * jb + lr] = g[e];
                }
            }
            // dv tiles (from the dV pass) into the output rows
#pragma unroll
            for (int it = 0; it < ITV; ++it) {
                const int ti = wv + NW * it;
                if (ti < NTV) {
                    const int mt = ti >> 2, vi = ti & 3;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        sm.gout[3][16 * mt + 4 * lq + e][16 * vi + lr] =
                            to_bf16(dvt[it][e]);
                }
            }
            __syncthreads();
            // ---- input gradients (thread: column j, tokens of group wv) --
            {
                float pp[TPG], qv[TPG], drv[TPG], dav[TPG], dbv[TPG], dkv[TPG];
#pragma unroll
                for (int u = 0; u < TPG; ++u) {
                    const int t = grp * TPG + u;
                    const float gprev = u == 0 ? off : gg[u - 1];
                    drv[u] = sm.e3.gR[t][j] * __expf(gg[u] - gref);
                    dav[u] = sm.e3.gA[t][j] * __expf(gprev - gref);
                    const float eng = __expf(gref - gg[u]);
                    dbv[u] = sm.e3.gB[t][j] * eng;
                    dkv[u] = sm.e3.gK[t][j] * eng;
                    const float rv = bf16_to_f32(bf16_t(prk[u] & 0xffffu));
                    const float kv = bf16_to_f32(bf16_t(prk[u] >> 16));
                    const float av = bf16_to_f32(bf16_t(pab[u] & 0xffffu));
                    const float bv = bf16_to_f32(bf16_t(pab[u] >> 16));
                    pp[u] = rv * drv[u] - bv * dbv[u] - kv * dkv[u];
                    qv[u] = av * dav[u];
                }
                sm.qx[grp][j] = qv[0];
                __syncthreads();
                const float qnext = grp < NW - 1 ? sm.qx[grp + 1][j] : 0.f;
                float f[TPG];
#pragma unroll
                for (int u = 0; u < TPG; ++u)
                    f[u] = pp[u] + (u + 1 < TPG ? qv[u + 1] : qnext);
                float suf = 0.f;
#pragma unroll
                for (int u = TPG - 1; u >= 0; --u) {
                    suf += f[u];
                    f[u] = suf;
                }
                sm.tot[grp][j] = suf;
                __syncthreads();
                float later = sm.tail[j];
                for (int g2 = grp + 1; g2 < NW; ++g2) later += sm.tot[g2][j];
#pragma unroll
                for (int u = 0; u < TPG; ++u) {
                    const int t = grp * TPG + u;
                    sm.gout[0][t][j] = to_bf16(drv[u]);
                    sm.gout[1][t][j] = to_bf16((f[u] + later) * lam[u]);
                    sm.gout[2][t][j] = to_bf16(dkv[u]);
                    sm.gout[4][t][j] = to_bf16(dav[u]);
                    sm.gout[5][t][j] = to_bf16(dbv[u]);
                }
            }
        }
        __syncthreads();
        // ---- next chunk's data to LDS; gradients to HBM; next fetch --------
        stash(tid);
        if (!fallback) {
            for (int sg = tid; sg < 6 * L * 8; sg += NTH) {
                const int row = sg >> 3, s8 = sg & 7;
                const int g = row / L, t = row % L;
                if (t < n) {
                    bf16_t* o = g == 0   ? dr
                                : g == 1 ? dw
                                : g == 2 ? dk
                                : g == 3 ? dv
                                : g == 4 ? da
                                         : db;
                    *reinterpret_cast<uint4*>(
                        o + ((t0 + t) * BH + bh) * CN + s8 * 8) =
                        *reinterpret_cast<const uint4*>(&sm.gout[g][t][s8 * 8]);
                }
            }
        }
        if (c >= 2) fetch(c - 2, tid);
#pragma unroll
        for (int q = 0; q < ST; ++q) SL[q] = S0[q];
        if (tid == 0) sm.flag = 0;
        __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < ST; ++q)
        *reinterpret_cast<float4*>(ds0 + sbase + toff[q]) =
            make_float4(D[q][0], D[q][1], D[q][2], D[q][3]);
}

template <int L>
hipError_t launch_l(const ChunkBwdArgs& p, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_chunk_bwd_kernel<L>), dim3(unsigned(BH)),
                       dim3(BWD_WAVES * 64), 0, stream, p.T, BH,
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
