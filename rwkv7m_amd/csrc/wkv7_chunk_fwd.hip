// Chunked WKV-7 forward for gfx950: bf16 vectors, fp32 state, N = 64.
//
// One workgroup (8 waves) per (batch, head) walks the sequence in chunks of
// L tokens (L = 16 or 32).  Within a chunk the recurrence
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
//   B^ = B~ diag(e^{g_L-g_ref})    K^ = K~ diag(e^{g_L-g_ref})
//
// and the L x L matrices Aab = A~ B~^T, Aak = A~ K~^T (strictly lower),
// Arb = R~ B~^T, Ark = R~ K~^T (lower, with diagonal).  With S' the chunk-
// start state with columns scaled by e^{g_ref}, Minv = (I - Aab)^{-1},
// W = Minv A~ and U = Minv Aak V, the rows X_t = S_{t-1} a_t are
// X = W S'^T + U, and
//
//   Y   = Q S'^T + P                      Q = R~ + Arb W,  P = Arb U + Ark V
//   S_L = S_0 diag(e^{g_L}) + S' M + C    M = W^T B^,      C = U^T B^ + V^T K^
//
// Everything but the two products with S' depends on the chunk's inputs
// alone, so the state chain from one chunk to the next is one 64x64x64
// product: the workgroup builds chunk c+1's Q, P, M and C while it advances
// the state through chunk c.  Five barrier-separated phases per chunk:
//
//   F  c+1: factors (in-wave scan of the log-decay)  c: S' -> LDS, S e^{g_L} + C
//   M  c+1: matrices; wave 0 the inverse             c: S += S' M, Y = Q S'^T + P
//   I  c+1: Aak V; C += V^T K^; P += Ark V; next vectors
//   W  c+1: W = Minv A~, U = Minv (Aak V)
//   Q  c+1: Q, M; C += U^T B^; P += Arb U
//
// Every product is a bf16 MFMA (v_mfma_f32_16x16x32_bf16) with fp32
// accumulation.  Operands stored with the contraction index strided are read
// with gfx950's transposing LDS load, so no transposed copies are made.  The
// state S, C and P stay fp32 in accumulator registers; B^ and K^ enter only
// as the column scaling e^{g_L-g_ref} of M and C.  Minv is formed in one
// wave's registers (the 16x16 diagonal blocks as the product
// (I+A)(I+A^2)(I+A^4)(I+A^8) of the nilpotent strictly lower block A).  A chunk whose decay range exceeds what the
// factored form represents (more than kHalfRange of log-decay on either side
// of g_ref: far outside the model's clamped range) runs an exact fp32
// sequential loop instead.

#include "wkv7_chunk_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

using chunk::CN;
using chunk::fkr;
using chunk::frk;
using chunk::PN;

constexpr int FWD_WAVES = chunk::NWAVES;
constexpr int FWD_THREADS = chunk::NTHREADS;

template <int L>
struct FwdSmem {
    static constexpr int PL = L + 8;
    static constexpr int NB = L / 16;
    // the next chunk's vectors: r, w, k, v, neg_kk, kka ([t][j])
    bf16_t raw[6][L][PN];
    union {
        struct {
            // factors of the chunk being prepared, token-major [t][j]
            bf16_t At[L][PN], Rt[L][PN], Bt[L][PN], Kt[L][PN], Vc[L][PN];
            // S' of the chunk being advanced, [i][j]
            bf16_t Sp[CN][PN];
        } f;
        float fb[CN][CN + 1];  // exact fallback: the state in fp32
    };
    // L x L matrices, stored transposed: X[s][t] holds entry (t, s)
    bf16_t Aak[L][PL], Arb[L][PL], Ark[L][PL], MinvT[L][PL];
    bf16_t AakV[CN][PL];       // [i][s]
    bf16_t Wt[CN][PL];         // [j][t] = W[t][j]
    bf16_t Ut[CN][PL];         // [i][t] = U[t][i]
    // the next chunk's inputs to the state step, double-buffered
    bf16_t Q[2][L][PN];    // [t][j]
    bf16_t Mt[2][CN][PN];  // [j][j'] = M[j'][j]
    // e^{g_L}, e^{g_ref}, e^{g_L - g_ref} per column
    alignas(16) float eL[2][CN];
    alignas(16) float eRef[2][CN];
    alignas(16) float eLR[2][CN];
    int flag[2];
};

// Exact fp32 sequential forward over one chunk, reading the vectors from
// HBM (the path for chunks outside the factored form's range).  S is the
// state in LDS ([64][65]); thread: row i = tid / NW, CPT columns.
template <int NW>
__device__ void seq_chunk_forward(float (*S)[CN + 1], int n, int64_t t0,
                                  int64_t tstr, int64_t hoff,
                                  const chunk::VecPtrs& src,
                                  bf16_t* __restrict__ y, int tid) {
    constexpr int CPT = CN / NW;
    const int i = tid / NW, c0 = CPT * (tid % NW);
    float Sl[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) Sl[c] = S[i][c0 + c];
    for (int t = 0; t < n; ++t) {
        const int64_t off = (t0 + t) * tstr + hoff;
        float sa = 0.f;
#pragma unroll
        for (int c = 0; c < CPT; ++c)
            sa += Sl[c] * bf16_to_f32(src.p4[off + c0 + c]);
        sa = group_sum<NW>(sa);
        const float vi = bf16_to_f32(src.p3[off + i]);
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int j = c0 + c;
            const float d = expf(-expf(bf16_to_f32(src.p1[off + j])));
            Sl[c] = Sl[c] * d + sa * bf16_to_f32(src.p5[off + j]) +
                    vi * bf16_to_f32(src.p2[off + j]);
            acc += Sl[c] * bf16_to_f32(src.p0[off + j]);
        }
        acc = group_sum<NW>(acc);
        if (tid % NW == 0) y[off + i] = to_bf16(acc);
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) S[i][c0 + c] = Sl[c];
}

template <int L>
__global__ void __launch_bounds__(FWD_THREADS)
wkv7_chunk_fwd_kernel(int64_t T, int64_t BH, VecLayout lay,
                      const bf16_t* __restrict__ r,
                      const bf16_t* __restrict__ w,
                      const bf16_t* __restrict__ k,
                      const bf16_t* __restrict__ v,
                      const bf16_t* __restrict__ a,
                      const bf16_t* __restrict__ b, const float* s0,
                      bf16_t* __restrict__ y, float* s_t, bf16_t* ckpt) {
    using Sm = FwdSmem<L>;
    constexpr int NW = FWD_WAVES, NTH = FWD_THREADS;
    constexpr int PL = Sm::PL, NB = Sm::NB;
    constexpr int CPL = L / 8;   // factor columns per lane
    static_assert(L == 16 || L == 32, "chunk length");
    __shared__ Sm sm;

    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = blockIdx.x;
    const int64_t sbase = bh * CN * CN;
    const int64_t hoff = lay.head(bh, CN);  // the head's vector offset
    const int64_t NN = CN * CN;
    const chunk::VecPtrs src{r, w, k, v, a, b, nullptr};
    const int64_t nch = (T + L - 1) / L;

    // ---- state: wave wv holds the S^T tiles si = 2wv, 2wv+1 --------------
    // tile si: rows j = 16*(si >> 2) + 4*lq + e, column i = 16*(si & 3) + lr
    f32x4_t S[2], Cacc[2], Pacc;
    int soff[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
        soff[q] = (16 * ib + lr) * CN + 16 * jb + 4 * lq;
        const float4 x =
            *reinterpret_cast<const float4*>(s0 + sbase + soff[q]);
        S[q][0] = x.x; S[q][1] = x.y; S[q][2] = x.z; S[q][3] = x.w;
        Cacc[q] = zero4();
    }
    Pacc = zero4();
    // Y^T tile of this wave (all 8 waves at L = 32, waves 0..3 at L = 16):
    // rows i = 16*yib + 4*lq + e, column t = 16*ytb + lr; yib is the i block
    // of one of the wave's state tiles, so the two share the S' operand
    const int yib = ((2 * wv) & 3) | ((wv >> 1) & 1), ytb = wv >> 2;
    const bool has_y = ytb < NB;

    // the matrices' and Minv's blocks above the diagonal stay zero
    {
        bf16_t(*const mats[4])[PL] = {sm.Aak, sm.Arb, sm.Ark, sm.MinvT};
        chunk::zero_upper<L>(mats, 4, tid, NTH);
    }
    if (tid < 2) sm.flag[tid] = 0;

    // ---- the vectors, prefetched one chunk ahead into registers ----------
    // HBM addresses are a per-chunk scalar base plus a 32-bit per-lane
    // offset (t * ts + column, ts the token stride; the host keeps L * ts
    // below 2^31).
    constexpr int SEG = 6 * L * 8;  // 16-byte segments of one chunk
    constexpr int NPRE = (SEG + NTH - 1) / NTH;
    static_assert((8 * L) % 64 == 0 && SEG % 64 == 0,
                  "each wave loads from one vector");
    const uint32_t TS = uint32_t(lay.ts);
    // part p of this wave: one vector (the same for all 64 lanes), or none
    const bf16_t* vp[NPRE];
#pragma unroll
    for (int p = 0; p < NPRE; ++p) {
        const int wseg = __builtin_amdgcn_readfirstlane((p * NTH + tid) & ~63);
        vp[p] = wseg < SEG ? src.get(wseg / (8 * L)) : nullptr;
    }
    uint4 pre[NPRE];
    auto fetch = [&](int64_t cc) {
        const int64_t cbase = cc * L * lay.ts + hoff;
        const int ncc = int(T - cc * L < L ? T - cc * L : L);
#pragma unroll
        for (int p = 0; p < NPRE; ++p) {
            const uint32_t seg = uint32_t(p * NTH + tid);
            const uint32_t t = (seg >> 3) & (L - 1), s8 = seg & 7;
            pre[p] = make_uint4(0, 0, 0, 0);
            if (vp[p] != nullptr && int(t) < ncc)
                pre[p] = *reinterpret_cast<const uint4*>(
                    (vp[p] + cbase) + (t * TS + s8 * 8));
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int p = 0; p < NPRE; ++p) {
            const int seg = p * NTH + tid;
            if (seg < SEG) {
                const int row = seg >> 3, s8 = seg & 7;
                *reinterpret_cast<uint4*>(&sm.raw[row / L][row % L][s8 * 8]) =
                    pre[p];
            }
        }
    };
    fetch(0);
    stash();
    // everything loaded before the loop has arrived: the loop's waits then
    // only count the prefetch and the stores
    __builtin_amdgcn_s_waitcnt(0);
    if (nch > 1) fetch(1);
    __syncthreads();

    // Iteration c advances the state through chunk c (c >= 0) and prepares
    // chunk c + 1 (c + 1 < nch).
    for (int64_t c = -1; c < nch; ++c) {
        const bool adv = c >= 0, prep = c + 1 < nch;
        const int cur = int(c & 1), nxt = int((c + 1) & 1);
        const int64_t t0 = c * L;
        const int n = adv ? int(T - t0 < L ? T - t0 : L) : 0;
        const int n1 = prep ? int(T - t0 - L < L ? T - t0 - L : L) : 0;
        const bool fallback = adv && sm.flag[cur] != 0;

        if (fallback) {
            // ---- chunk c by the exact sequential loop -----------------
            if (ckpt) {
#pragma unroll
                for (int q = 0; q < 2; ++q)
                    *reinterpret_cast<uint2*>(ckpt + c * BH * NN + sbase +
                                              soff[q]) = pack4(S[q]);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    sm.fb[soff[q] / CN][soff[q] % CN + e] = S[q][e];
            __syncthreads();
            seq_chunk_forward<NW>(sm.fb, n, t0, lay.ts, hoff, src, y, tid);
            __syncthreads();
#pragma unroll
            for (int q = 0; q < 2; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    S[q][e] = sm.fb[soff[q] / CN][soff[q] % CN + e];
            __syncthreads();  // fb aliases the factor arrays
        }

        // ================= phase F =======================================
        if (adv && !fallback) {
            // checkpoint c; S' = S e^{g_ref} to LDS; S <- S e^{g_L} + C
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
                if (ckpt)
                    *reinterpret_cast<uint2*>(ckpt + c * BH * NN + sbase +
                                              soff[q]) = pack4(S[q]);
                const int j = 16 * jb + 4 * lq;
                const float4 er = *reinterpret_cast<const float4*>(&sm.eRef[cur][j]);
                const float4 el = *reinterpret_cast<const float4*>(&sm.eL[cur][j]);
                const float4 elr = *reinterpret_cast<const float4*>(&sm.eLR[cur][j]);
                f32x4_t sp;
                sp[0] = S[q][0] * er.x; sp[1] = S[q][1] * er.y;
                sp[2] = S[q][2] * er.z; sp[3] = S[q][3] * er.w;
                S[q][0] = S[q][0] * el.x + Cacc[q][0] * elr.x;
                S[q][1] = S[q][1] * el.y + Cacc[q][1] * elr.y;
                S[q][2] = S[q][2] * el.z + Cacc[q][2] * elr.z;
                S[q][3] = S[q][3] * el.w + Cacc[q][3] * elr.w;
                store_tile_bf16_t(sp, &sm.f.Sp[16 * ib][16 * jb], PN, lane);
            }
        }
        if (prep) {
            // factors of chunk c+1; v is copied as it is
            chunk::LaneFactors<L, NW> fl;
            chunk::chunk_factors<L, NW>(sm.raw, n1, wv, lane, sm.f.At, sm.f.Rt,
                                    sm.f.Bt, sm.f.Kt, sm.eL[nxt],
                                    sm.eRef[nxt], sm.eLR[nxt], &sm.flag[nxt],
                                    fl);
            const int t = fl.t, j0 = fl.j0;
            if constexpr (CPL == 4)
                *reinterpret_cast<uint2*>(&sm.f.Vc[t][j0]) =
                    *reinterpret_cast<const uint2*>(&sm.raw[3][t][j0]);
            else
                *reinterpret_cast<uint32_t*>(&sm.f.Vc[t][j0]) =
                    *reinterpret_cast<const uint32_t*>(&sm.raw[3][t][j0]);
        }
        __syncthreads();

        // ================= phase M =======================================
        if (adv && !fallback) {
            // S^T += M^T S'^T and Y^T = P^T + S' Q^T (K = 64)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
#pragma unroll
                for (int k0 = 0; k0 < CN; k0 += 32)
                    mfma(S[q], frag_rk(&sm.Mt[cur][16 * jb][k0], PN, lane),
                         frag_rk(&sm.f.Sp[16 * ib][k0], PN, lane));
            }
            if (has_y) {
                f32x4_t yy = Pacc;
#pragma unroll
                for (int k0 = 0; k0 < CN; k0 += 32)
                    mfma(yy, frag_rk(&sm.f.Sp[16 * yib][k0], PN, lane),
                         frag_rk(&sm.Q[cur][16 * ytb][k0], PN, lane));
                const int tt = 16 * ytb + lr;
                if (tt < n)
                    *reinterpret_cast<uint2*>(
                        (y + (t0 * lay.ts + hoff)) +
                        (uint32_t(tt) * TS + 16 * yib + 4 * lq)) =
                        pack4(yy);
            }
        }
        if (adv && tid == 0) sm.flag[cur] = 0;
        Pacc = zero4();
        Cacc[0] = zero4();
        Cacc[1] = zero4();
        if (prep) {
            if (wv == 0) {
                chunk::minv_regs<L>(sm.f.At, sm.f.Bt, sm.MinvT, lane);
            } else {
                // Aak (strict), Arb, Ark (with diagonal): lower tiles
                constexpr int TPM = NB * (NB + 1) / 2;
                for (int ti = wv - 1; ti < 3 * TPM; ti += NW - 1) {
                    const int mat = ti / TPM;
                    int tb, sb;
                    chunk::lower_tile_index(ti % TPM, tb, sb);
                    chunk::lower_tile<L>(mat == 0 ? sm.f.At : sm.f.Rt,
                                         mat == 1 ? sm.f.Bt : sm.f.Kt,
                                         mat == 0   ? sm.Aak
                                         : mat == 1 ? sm.Arb
                                                    : sm.Ark,
                                         tb, sb, mat == 0, lane);
                }
            }
        }
        __syncthreads();

        // ================= phase I =======================================
        if (prep) {
            // Aak V -> AakV[i][s]: one tile (s block wv / 4, i block wv % 4)
            // per wave (NB = 2) or per wave 0..3 (NB = 1)
            if (NB == 2 || wv < 4) {
                const int sb = wv >> 2, ib = wv & 3;
                f32x4_t acc = zero4();
                mfma(acc, fkr<L>(&sm.Aak[0][16 * sb], PL, lane),
                     fkr<L>(&sm.f.Vc[0][16 * ib], PN, lane));
                store_tile_bf16_t(acc, &sm.AakV[16 * ib][16 * sb], PL, lane);
            }
            // C^T += K~^T V (scaled as above), P^T += V^T Ark^T
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
                mfma(Cacc[q], fkr<L>(&sm.f.Kt[0][16 * jb], PN, lane),
                     fkr<L>(&sm.f.Vc[0][16 * ib], PN, lane));
            }
            if (has_y)
                mfma(Pacc, fkr<L>(&sm.f.Vc[0][16 * yib], PN, lane),
                     fkr<L>(&sm.Ark[0][16 * ytb], PL, lane));
        }
        if (c + 2 < nch) {
            stash();
            if (c + 3 < nch) fetch(c + 3);
        }
        __syncthreads();

        // ================= phase W =======================================
        if (prep) {
            // W = Minv A~ -> Wt[j][t]; U = Minv (Aak V) -> Ut[i][t]
            for (int ti = wv; ti < 8 * NB; ti += NW) {
                const bool isU = ti >= 4 * NB;
                const int rem = ti % (4 * NB), tb = rem / 4, xb = rem % 4;
                f32x4_t acc = zero4();
                const bf16x8_t fa = fkr<L>(&sm.MinvT[0][16 * tb], PL, lane);
                if (isU) {
                    mfma(acc, fa, frk<L>(&sm.AakV[16 * xb][0], PL, lane));
                    store_tile_bf16_t(acc, &sm.Ut[16 * xb][16 * tb], PL, lane);
                } else {
                    mfma(acc, fa, fkr<L>(&sm.f.At[0][16 * xb], PN, lane));
                    store_tile_bf16_t(acc, &sm.Wt[16 * xb][16 * tb], PL, lane);
                }
            }
        }
        __syncthreads();

        // ================= phase Q =======================================
        if (prep) {
            // Q^T = R~^T + W^T Arb^T -> Q[t][j]  (tiles: j block x t block)
            for (int ti = wv; ti < 4 * NB; ti += NW) {
                const int jb = ti % 4, tb = ti / 4;
                f32x4_t acc = unpack4(*reinterpret_cast<const uint2*>(
                    &sm.f.Rt[16 * tb + lr][16 * jb + 4 * lq]));
                mfma(acc, frk<L>(&sm.Wt[16 * jb][0], PL, lane),
                     fkr<L>(&sm.Arb[0][16 * tb], PL, lane));
                store_tile_bf16_t(acc, &sm.Q[nxt][16 * tb][16 * jb], PN,
                                  lane);
            }
            // M = W^T B^ = (W^T B~) diag(e^{g_L-g_ref}) -> Mt[j][j']
            // (tiles: j' block x j block)
            for (int ti = wv; ti < 16; ti += NW) {
                const int jpb = ti % 4, jb = ti / 4;
                f32x4_t acc = zero4();
                mfma(acc, frk<L>(&sm.Wt[16 * jpb][0], PL, lane),
                     fkr<L>(&sm.f.Bt[0][16 * jb], PN, lane));
                const float sc = sm.eLR[nxt][16 * jb + lr];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] *= sc;
                store_tile_bf16_t(acc, &sm.Mt[nxt][16 * jb][16 * jpb], PN,
                                  lane);
            }
            // C^T += B~^T U (scaled by e^{g_L-g_ref} when applied) and
            // P^T += U^T Arb^T
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int si = 2 * wv + q, jb = si >> 2, ib = si & 3;
                mfma(Cacc[q], fkr<L>(&sm.f.Bt[0][16 * jb], PN, lane),
                     frk<L>(&sm.Ut[16 * ib][0], PL, lane));
            }
            if (has_y)
                mfma(Pacc, frk<L>(&sm.Ut[16 * yib][0], PL, lane),
                     fkr<L>(&sm.Arb[0][16 * ytb], PL, lane));
        }
        __syncthreads();
    }

    // ---- final state -----------------------------------------------------
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        *reinterpret_cast<float4*>(s_t + sbase + soff[q]) =
            make_float4(S[q][0], S[q][1], S[q][2], S[q][3]);
        if (ckpt)
            *reinterpret_cast<uint2*>(ckpt + nch * BH * NN + sbase +
                                      soff[q]) = pack4(S[q]);
    }
}

template <int L>
hipError_t launch_l(const ChunkFwdArgs& p, hipStream_t stream) {
    const int64_t BH = p.B * p.H;
    hipLaunchKernelGGL((wkv7_chunk_fwd_kernel<L>), dim3(unsigned(BH)),
                       dim3(FWD_THREADS), 0, stream, p.T, BH, p.lay,
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
        default: return hipErrorInvalidValue;
    }
}

}  // namespace rwkv7m
