// Chunked WKV-7 forward for gfx950 with the state rows split over waves:
// bf16 vectors, fp32 state, N = 64, chunks of 16 tokens.
//
// The recurrence (reference src/rwkv7m/model/rwkv_core.py:54-86)
//
//   S_t = S_{t-1} diag(d_t) + (S_{t-1} a_t) b_t^T + v_t k_t^T,  y_t = S_t r_t
//
// acts on each row i of the state separately: row i needs only v_t[i] of
// the value side and yields only y_t[i].  Over a chunk, in the closed form
// below (g = running log2-decay, g_ref its value at token 7; A~, R~, B~, K~
// the decayed factors of wkv7_wave_bwd.hip),
//
//   X = W^ bf16(S_0)^T + U,   S_L = S_0 diag(2^{g_L}) + X^T B^ + V^T K^,
//   Y^T = bf16(S_0) Q^^T + P^T
//
// with W^ = Minv A~ diag(2^{g_ref}) and Q^ = diag(2^{g_ref}) (R~ + Arb W)^T
// depending on the chunk's key-side vectors only, and U = Minv Aak V,
// P = Arb U + Ark V linear in the value rows.
//
// One workgroup of 12 waves per (batch, head):
//   * waves 4..11, the producers: producer p builds chunks p, p + 8, ...:
//     the decayed factors, the 16 x 16 matrices, the inverse, W^, U and Q^,
//     all in registers, and hands them to a ring of three LDS slots;
//   * waves 0..3, the chains: chain ib holds rows 16 ib .. 16 ib + 15 of the
//     fp32 state in registers for the whole sequence and, chunk after
//     chunk, forms its rows of X (2 MFMAs), advances its rows (8 MFMAs),
//     forms its rows of y (4 MFMAs) and stores them with its rows of the
//     checkpoint when one is due.  A chain reads a chunk's operands from
//     the slot while the previous chunk's products run, so that its step
//     waits on no LDS read.
// The four chains run independent recurrences; the kernel runs at the
// producers' rate.
//
// Register layouts (lane l, r = l % 16, q = l / 16).  A 16 x 16 accumulator
// tile D(X) holds X[4q + e][r] (e = 0..3).  As operands of
// v_mfma_f32_16x16x16_bf16, the lane's four values (kq) are X as the B
// operand and X^T as the A operand.  Token-major matrices X[t][j] (16 x 64)
// come two ways:
//   T layout: lane holds X[r][16 kb + 4q + e] (kb = 0..3): the tiles
//             D((X^T)_kb), for products contracting over j;
//   J layout: lane holds X[4q + e][16 jb + r]: the tiles D(X_jb), for
//             products contracting over t.
// Vectors arrive in the T layout; A~, B^, K^ and V are turned into the J
// layout through a per-producer LDS buffer and gfx950's transposing LDS
// load.  Products over K = 64 pair two T tiles into one
// v_mfma_f32_16x16x32_bf16 operand (the same slot order on both sides).  A
// chain's state rows sit in the accumulator layout D(S^T_{j'b, ib}), which
// is at the same time the bf16 operand layout of the state step.  A
// 16x16x16 product never accumulates onto a 16x16x32 result or the other way
// round: every such hand-over goes through a VALU operation.

#include <atomic>

#include "wkv7_wave_common.h"

namespace rwkv7m {
namespace {

using namespace wave;

constexpr int NCHAIN = 4;    // chain waves (16 state rows each)
constexpr int NPROD = 8;     // producer waves
constexpr int NSLOT = 3;     // hand-over ring
constexpr int NYBUF = 4;     // y staging buffers (y of chunk c: c % NYBUF)
constexpr int WTHREADS = 64 * (NCHAIN + NPROD);
// Every hand-over wait is bounded (WaitCfg::limit polls of ~64 cycles; a
// wave waits for at most a few other chunks, and the default bound is orders
// of magnitude above that), so every wave exits.  A wait that gives up marks
// the workgroup failed; every other wave reads that mark within eight polls
// of its current wait and leaves its loop, so a lost hand-over costs one
// wait's budget, not one per remaining chunk.  The workgroup's outputs are
// then overwritten with NaN and the device's failure counter is raised
// (wkv7_status.hip).

// Per producer: the next chunk's six vectors as loaded, and, once the
// factors are formed, the four J-layout matrices on their way through the
// transposing read.  raw[p][h][s][u] holds the 16-byte segment s (columns
// 8s .. 8s + 7) of token 8h + u: the T-layout reads of one vector are then
// one address plus constant offsets.
union ProdStage {
    uint4 raw[6][2][8][8];
    bf16_t xp[4][WL][XPITCH];  // A~, B^, K^, V ([t][j])
};

// One chunk's hand-over from a producer to the chains, as register images
// (element [..][lane] is that lane's operand).
struct Slot {
    bf16x8_t W[2][64];     // A operands of W^ (T layout pairs, K = 64)
    bf16x8_t Q[2][64];     // B operands of Q^^T: tiles 2jp, 2jp + 1
    i16x4_t B[4][64];      // B^ (J layout)
    i16x4_t K[4][64];      // K^ (J layout)
    i16x4_t U[4][64];      // D(U_ib)
    i16x4_t V[4][64];      // V (J layout)
    i16x4_t Arb[64];       // D(Arb^T)
    i16x4_t Ark[64];       // D(Ark^T)
    float eL[WN];          // 2^{g_L} per column
};

// A chain's 16 rows of a checkpoint on their way to global memory: written
// in the chain's register layout, read back as whole rows (16 bytes per
// lane) and stored one chunk later.  Each chain uses only its own rows.
typedef bf16_t CkRows[16][XPITCH];

struct WaveFwdSmem {
    Slot slot[NSLOT];
    CkRows ck[NCHAIN];
    ProdStage st[NPROD];
    float eref[NPROD][WN];  // per producer: 2^{g_ref} per column
    float eL[NPROD][WN];    // per producer: 2^{g_L} per column
    // y of chunk c on its way to global memory, buffer c % NYBUF: each chain
    // writes its 16 columns and the producer of chunk c + 4 stores the 16
    // rows whole (the slot wait it does anyway proves the four tiles are
    // there, and it publishes chunk c + 4 before any chain can stage
    // chunk c + NYBUF); the last NYBUF chunks are stored after the loops.
    // Four chains each storing their own quarter of every 128-byte row, at
    // their own times, cost about twice what y's bytes do.
    bf16_t ys[NYBUF][WL][XPITCH];
    int ychunk[NYBUF];      // the chunk whose y the buffer holds (-1: none)
    int ready[NSLOT];       // 2 c + exact for the chunk c the slot holds
                            // (exact: it needs the exact sequential pass;
                            // -1: none yet)
    int done[NSLOT];        // chains finished with the slot, over all uses
    int failed;             // a bounded wait of this workgroup gave up
};


// Most workgroups one head's forward is split over (see FwdArgs::nseg).
constexpr int kMaxFwdSegments = 2;

struct FwdArgs {
    int64_t T, BH;
    VecLayout lay;
    const bf16_t *r, *w, *k, *v, *a, *b;
    const float* s0;
    bf16_t* y;
    float* s_t;
    bf16_t* ckpt;  // nullptr, or bf16 checkpoints every cstride chunks
    int cstride;   // checkpoint interval / 16
    int cshift;    // log2(cstride)
    WaitCfg wait;
    // Workgroups per head and, per segment g, the chunks [seg_lo[g],
    // seg_hi[g]) whose y and checkpoints that workgroup writes; it carries
    // the state through the chunks before them without writing anything.
    // Workgroup blockIdx.x serves head blockIdx.x / nseg, segment
    // blockIdx.x % nseg; the segment with seg_hi == the chunk count also
    // writes S_T and the last checkpoint.
    int nseg;
    int seg_lo[kMaxFwdSegments], seg_hi[kMaxFwdSegments];
};

__device__ __forceinline__ int64_t head_of(const FwdArgs& A) {
    return int64_t(blockIdx.x) / A.nseg;
}
__device__ __forceinline__ int seg_of(const FwdArgs& A) {
    return int(blockIdx.x % unsigned(A.nseg));
}

// ---------------------------------------------------------------------------
// The staged y of chunk yc (buffer yb) as whole rows: lane l stores the
// 16-byte pieces l % 8 of tokens l / 8 and 8 + l / 8 (two stores per lane,
// every 128-byte row written whole); tokens past the end store at or past
// the range's bound and are dropped.
__device__ __forceinline__ void store_y_rows(const FwdArgs& A,
                                             WaveFwdSmem& sm, int yb, int yc,
                                             int64_t hoff, int lane) {
    const int64_t ty = int64_t(yc) * WL;
    const int ny = int(A.T - ty < WL ? A.T - ty : WL);
    const uint32_t TS = uint32_t(A.lay.ts);
    const __amdgpu_buffer_rsrc_t rs = out_rsrc(
        A.y + (ty * A.lay.ts + hoff), (uint32_t(ny - 1) * TS + WN) * 2);
    const int yt = lane >> 3, yo = 8 * (lane & 7);
    const uint4 y0 = *reinterpret_cast<const uint4*>(&sm.ys[yb][yt][yo]);
    const uint4 y1 = *reinterpret_cast<const uint4*>(&sm.ys[yb][8 + yt][yo]);
    lds_drain();  // the buffer may be staged again once the reads are done
    store16(rs, (uint32_t(yt) * TS + yo) * 2, y0);
    store16(rs, (uint32_t(8 + yt) * TS + yo) * 2, y1);
}

// ---------------------------------------------------------------------------
// Producer p: chunks p, p + NPROD, ...
__device__ __forceinline__ void produce(const FwdArgs& A, WaveFwdSmem& sm,
                                        int p, int lane) {
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = head_of(A);
    const int64_t hoff = A.lay.head(bh, WN);
    const int64_t T = A.T;
    const int nch = int((T + WL - 1) / WL);
    const uint32_t TS = uint32_t(A.lay.ts);
    const VecPtrs src{A.r, A.w, A.k, A.v, A.a, A.b, nullptr};
    ProdStage& stg = sm.st[p];
    bf16_t (*const xp)[WL][XPITCH] = stg.xp;
    int* const vdone = sm.done;
    int* const vready = sm.ready;

    // A chunk's vectors go straight to the stage in LDS (16 bytes per lane,
    // global_load_lds_dwordx4, which writes lane l's data at 16 l): lane l
    // of load (vector, h) fetches segment l / 8 of token 8h + l % 8.  Tokens
    // past the end re-read the last token (zeroed when read).
    const int ldu = lane & 7, ldseg = lane >> 3;
    auto fetch = [&](int c) {
        const int64_t cbase = int64_t(c) * WL * A.lay.ts + hoff;
        const int n = int(T - int64_t(c) * WL < WL ? T - int64_t(c) * WL : WL);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = 8 * h + ldu;
            const uint32_t off = (uint32_t(t < n ? t : n - 1) * TS +
                                  8 * ldseg) * sizeof(bf16_t);
#pragma unroll
            for (int vv = 0; vv < 6; ++vv)
                dma16(src.get(vv) + cbase, off, lds_addr(&stg.raw[vv][h][0][0]));
        }
    };
    // the T layout read of vector vv: token lr, columns 16 kb + 4 lq .. + 3
    // (segment 2 kb + lq / 2, half lq % 2)
    const bf16_t* const rbase = reinterpret_cast<const bf16_t*>(
        &stg.raw[0][lr >> 3][lq >> 1][lr & 7]) + 4 * (lq & 1);
    auto read_t = [&](int vv, int kb) -> uint2 {
        return *reinterpret_cast<const uint2*>(rbase + vv * (2 * 8 * 8 * 8) +
                                               kb * (2 * 8 * 8));
    };
    // this workgroup's chunks end at c_hi (the chunks before its own it
    // only carries the state through)
    const int c_hi = A.seg_hi[seg_of(A)];
    if (p < c_hi) fetch(p);

    // y stores issued after the next chunk's vector loads (their count: the
    // wait for those loads lets them run on)
    int ystores = 0;
    for (int c = p; c < c_hi; c += NPROD) {
        const int n = int(T - int64_t(c) * WL < WL ? T - int64_t(c) * WL : WL);
        const bool valid = lr < n;
        // this chunk's vectors (vector memory operations complete in issue
        // order)
        if (ystores)
            __builtin_amdgcn_s_waitcnt(0x0f72);  // vmcnt(2)
        else
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        ystores = 0;
        asm volatile("" ::: "memory");
        uint2 raw[6][4];
#pragma unroll
        for (int vv = 0; vv < 6; ++vv)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) raw[vv][kb] = read_t(vv, kb);
        if (n < WL) {
            // padding tokens: zero vectors and w = -inf (bf16), so that
            // they decay by nothing
#pragma unroll
            for (int vv = 0; vv < 6; ++vv) {
                const uint2 pad = vv == 1 ? make_uint2(0xff80ff80u, 0xff80ff80u)
                                          : make_uint2(0, 0);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    raw[vv][kb] = valid ? raw[vv][kb] : pad;
            }
        }

        // ---- factors (T layout, fp32) --------------------------------------
        // lam = log2 d_t, g its running sum over the chunk, g_ref = g at
        // token 7, g_L = g at token 15 (padding tokens decay by nothing)
        f32x4_t fA[4], fR[4], fB[4], fK[4];
        float lo = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const f32x4_t wr = unpack4(raw[1][kb]);
            const f32x4_t ar = unpack4(raw[4][kb]), br = unpack4(raw[5][kb]);
            const f32x4_t rr = unpack4(raw[0][kb]), kr = unpack4(raw[2][kb]);
            f32x4_t sLR, sp4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ew = __builtin_amdgcn_exp2f(wr[e] * kLog2e);
                const float g = scan16(-ew * kLog2e);
                const float gref = row_bcast<7>(g), gL = row_bcast<15>(g);
                lo = fminf(lo, fminf(gref, gL - gref));
                const float dg = g - gref;
                const float eg = __builtin_amdgcn_exp2f(dg);
                const float eng = __builtin_amdgcn_exp2f(-dg);
                // token 0: 2^{-g_ref} (its A~ factor); tokens 1, 2: the
                // column's 2^{g_ref}, 2^{g_L}
                const float sp = __builtin_amdgcn_exp2f(
                    lr == 0 ? -gref : lr == 1 ? gref : gL);
                const float eprev = row_prev(eg, sp);
                sp4[e] = sp;
                sLR[e] = pin_lanes(row_bcast<15>(eg));
                fA[kb][e] = ar[e] * eprev;
                fR[kb][e] = rr[e] * eg;
                fB[kb][e] = br[e] * eng;
                fK[kb][e] = kr[e] * eng;
            }
            // per-column 2^{g_ref} (token 1) and 2^{g_L} (token 2)
            if (lr == 1)
                *reinterpret_cast<f32x4_t*>(&sm.eref[p][16 * kb + 4 * lq]) = sp4;
            if (lr == 2)
                *reinterpret_cast<f32x4_t*>(&sm.eL[p][16 * kb + 4 * lq]) = sp4;
            f32x4_t bh4, kh4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                bh4[e] = fB[kb][e] * sLR[e];
                kh4[e] = fK[kb][e] * sLR[e];
            }
            *reinterpret_cast<uint2*>(&xp[0][lr][16 * kb + 4 * lq]) =
                pack4(fA[kb]);
            *reinterpret_cast<uint2*>(&xp[1][lr][16 * kb + 4 * lq]) =
                pack4(bh4);
            *reinterpret_cast<uint2*>(&xp[2][lr][16 * kb + 4 * lq]) =
                pack4(kh4);
            *reinterpret_cast<uint2*>(&xp[3][lr][16 * kb + 4 * lq]) =
                raw[3][kb];
        }
        // the factored form needs g_ref >= -H and g_L - g_ref >= -H
        const bool exact =
            __builtin_amdgcn_ballot_w64(lo < -kHalfRange * kLog2e) != 0;

        i16x4_t tA[4], tR[4], tB[4], tK[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            tA[kb] = kq(fA[kb]);
            tR[kb] = kq(fR[kb]);
            tB[kb] = kq(fB[kb]);
            tK[kb] = kq(fK[kb]);
        }

        // ---- the 16 x 16 matrices (K = 64) ---------------------------------
        // D(Aab), D(Aab^T) for the inverse; D(Aak^T), D(Arb^T), D(Ark^T)
        f32x4_t mA = zero4(), mAT = zero4(), mAakT = zero4(), mArbT = zero4(),
                mArkT = zero4();
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            const bf16x8_t a8 = pk8(tA[2 * kp], tA[2 * kp + 1]);
            const bf16x8_t b8 = pk8(tB[2 * kp], tB[2 * kp + 1]);
            const bf16x8_t k8 = pk8(tK[2 * kp], tK[2 * kp + 1]);
            const bf16x8_t r8 = pk8(tR[2 * kp], tR[2 * kp + 1]);
            mfma(mA, a8, b8);     // Aab[t][s] = A~_t . B~_s
            mfma(mAT, b8, a8);    // Aab^T
            mfma(mAakT, k8, a8);  // Aak^T[u][s] = K~_u . A~_s
            mfma(mArbT, b8, r8);  // Arb^T[s][t] = B~_s . R~_t
            mfma(mArkT, k8, r8);  // Ark^T[s][t] = K~_s . R~_t
        }
        mA = mask4(mA, lr, lq, true, true);          // s < t
        mAT = mask4(mAT, lr, lq, true, false);       // s < t
        mAakT = mask4(mAakT, lr, lq, true, false);   // u < s
        mArbT = mask4(mArbT, lr, lq, false, false);  // s <= t
        mArkT = mask4(mArkT, lr, lq, false, false);

        // ---- Minv = (I - Aab)^{-1} = (I + A)(I + A^2)(I + A^4)(I + A^8) ----
        f32x4_t dMT;
        {
            const i16x4_t pA = kq(mA), pT = kq(mAT);
            f32x4_t x2 = zero4(), t2 = zero4();
            mfma16(x2, pT, pA);  // A A
            mfma16(t2, pA, pT);  // A^T A^T
            const i16x4_t px2 = kq(x2), pt2 = kq(t2);
            f32x4_t q1t;  // Q1^T = I + A^T + (A^2)^T + (A^2)^T A^T
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float one = (4 * lq + e == lr) ? 1.f : 0.f;
                q1t[e] = one + mAT[e] + t2[e];
            }
            mfma16(q1t, px2, pT);
            f32x4_t x4 = zero4(), t4 = zero4();
            mfma16(x4, pt2, px2);  // A^4
            mfma16(t4, px2, pt2);  // (A^4)^T
            const i16x4_t pq1t = kq(q1t), px4 = kq(x4), pt4 = kq(t4);
            f32x4_t q2t = q1t, x8 = zero4();
            mfma16(q2t, px4, pq1t);  // (Q1 + Q1 A^4)^T
            mfma16(x8, pt4, px4);    // A^8
            dMT = q2t;
            mfma16(dMT, kq(x8), kq(q2t));  // Minv^T = (Q2 + Q2 A^8)^T
        }

        // ---- products over the chunk (K = 16) ------------------------------
        const i16x4_t kMinv = kq(dMT);  // A operand: Minv
        const i16x4_t kMinvB = kMinv;   // B operand: Minv^T
        const i16x4_t kAak = kq(mAakT), kArbT = kq(mArbT),
                      kArkT = kq(mArkT);
        wave_lds_fence();
        i16x4_t jA[4], jB[4], jK[4], jV[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            jA[jb] = read_j(xp[0], jb, lane);
            jB[jb] = read_j(xp[1], jb, lane);
            jK[jb] = read_j(xp[2], jb, lane);
            jV[jb] = read_j(xp[3], jb, lane);
        }
        // the stage is free once these reads are done: the next chunk's
        // vectors load during the rest of this one
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
        if (c + NPROD < c_hi) fetch(c + NPROD);

        // 2^{g_ref} of column 16 jb + lr (W's columns in the J layout) and
        // of rows 16 jb + 4 lq + e (the T layout): folded into W and R~, so
        // that the state enters the chains as bf16(S_0)
        float erj[4];
        f32x4_t ert[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            erj[jb] = sm.eref[p][16 * jb + lr];
            ert[jb] = *reinterpret_cast<const f32x4_t*>(
                &sm.eref[p][16 * jb + 4 * lq]);
        }
        i16x4_t kW[4], kU[4], kQ[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            f32x4_t x = zero4();
            mfma16(x, kMinv, jA[jb]);  // W = Minv A~ : D(W_jb)
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] *= erj[jb];
            kW[jb] = kq(x);            // W diag(2^{g_ref})
            f32x4_t av = zero4();
            mfma16(av, kAak, jV[jb]);  // Aak V : D((Aak V)_ib)
            f32x4_t u = zero4();
            mfma16(u, kMinv, kq(av));  // U = Minv Aak V : D(U_ib)
            kU[jb] = kq(u);
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            // Q^ = diag(2^{g_ref}) R~^T + (W diag(2^{g_ref}))^T Arb^T
            f32x4_t x = unpack4(__builtin_bit_cast(uint2, tR[jb]));
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] *= ert[jb][e];
            mfma16(x, kW[jb], kArbT);
            kQ[jb] = kq(x);
        }

        // W^ = W diag(2^{g_ref}) in the T layout, D(W^T_kb) = A~_kb^T
        // Minv^T scaled per column: the chains' A operands of W^ bf16(S_0)^T
        i16x4_t wt[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            f32x4_t x = zero4();
            mfma16(x, jA[kb], kMinvB);
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] *= ert[kb][e];
            wt[kb] = kq(x);
        }

        // ---- hand the chunk to the chains ---------------------------------
        const int s = c % NSLOT;
        const int uses = c / NSLOT;  // earlier uses of this slot
        // a wave that gives up marks the workgroup failed; every other wave
        // then stops at its next wait (within eight polls)
        const int got = poll_or_stop(vdone + s, A.wait.limit, &sm.failed,
                                     [&](int d) { return d >= NCHAIN * uses; });
        if (got <= 0) {
            if (got < 0) wait_failed(&sm.failed, A.wait.failures, lane);
            break;
        }
        // y of chunk c - 4: its four tiles were staged before chunk c - 3's
        // slot came back (done above)
        {
            const int yb = c & (NYBUF - 1);
            const int ych =
                __builtin_amdgcn_readfirstlane(lds_load(&sm.ychunk[yb]));
            if (ych >= 0) {
                store_y_rows(A, sm, yb, ych, hoff, lane);
                if (lane == 0) lds_store(&sm.ychunk[yb], -1);
                ystores = 2;
            }
        }
        Slot& sl = sm.slot[s];
        sl.W[0][lane] = pk8(wt[0], wt[1]);
        sl.W[1][lane] = pk8(wt[2], wt[3]);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            sl.B[jb][lane] = jB[jb];
            sl.K[jb][lane] = jK[jb];
            sl.U[jb][lane] = kU[jb];
            sl.V[jb][lane] = jV[jb];
        }
        sl.Q[0][lane] = pk8(kQ[0], kQ[1]);
        sl.Q[1][lane] = pk8(kQ[2], kQ[3]);
        sl.Arb[lane] = kArbT;
        sl.Ark[lane] = kArkT;
        if (lane < 16)
            *reinterpret_cast<f32x4_t*>(&sl.eL[4 * lane]) =
                *reinterpret_cast<const f32x4_t*>(&sm.eL[p][4 * lane]);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        asm volatile("" ::: "memory");
        if (lane == 0) lds_store(vready + s, 2 * c + (exact ? 1 : 0));
    }
}

// ---------------------------------------------------------------------------
// Chain ib: state rows 16 ib .. 16 ib + 15 through every chunk.
__device__ __forceinline__ void chain(const FwdArgs& A, WaveFwdSmem& sm,
                                      int ib, int lane) {
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = head_of(A);
    const int64_t sbase = bh * WN * WN;
    const int64_t hoff = A.lay.head(bh, WN);
    const int64_t T = A.T;
    const int nch = int((T + WL - 1) / WL);
    const int64_t NN = WN * WN;
    const uint32_t TS = uint32_t(A.lay.ts);
    int* const vready = sm.ready;
    const int row = 16 * ib + lr;  // the lane's state row

    // the chains are the serial path: they take issue priority over the
    // producers sharing their SIMDs
    __builtin_amdgcn_s_setprio(2);
    // S tiles D(S^T_{j'b, ib}): lane holds S[row][16 j'b + 4 lq + e]
    f32x4_t S[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
        S[jb] = *reinterpret_cast<const f32x4_t*>(A.s0 + sbase + row * WN +
                                                  16 * jb + 4 * lq);
    // the loop's only global memory operations are stores: with the state
    // loads complete here, no wait for those stores lands inside the loop
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)

    // A chunk's operands, read from its slot at the end of the previous
    // chunk's step, while that step's products run.  The slot's ready word
    // (2 c + exact) is loaded as that step is issued, so the check rarely
    // waits.
    struct SlotRegs {
        bf16x8_t W0, W1, Q0, Q1;
        i16x4_t U, V, Arb, Ark, B[4], K[4];
        f32x4_t eL[4];
        int exact;
    };
    // false when the workgroup failed (this wave's wait gave up, or another
    // wave's did)
    auto take = [&](int c, int s, int word, SlotRegs& r) -> bool {
        if ((word >> 1) != c) {
            const int got = poll_or_stop(vready + s, A.wait.limit, &sm.failed,
                                         [&](int x) {
                                             word = x;
                                             return (x >> 1) == c;
                                         });
            if (got <= 0) {
                if (got < 0) wait_failed(&sm.failed, A.wait.failures, lane);
                return false;
            }
        }
        const Slot& sl = sm.slot[s];
        r.exact = word & 1;
        r.W0 = sl.W[0][lane];
        r.W1 = sl.W[1][lane];
        r.U = sl.U[ib][lane];
        r.V = sl.V[ib][lane];
#pragma unroll
        for (int jpb = 0; jpb < 4; ++jpb) {
            r.B[jpb] = sl.B[jpb][lane];
            r.K[jpb] = sl.K[jpb][lane];
            r.eL[jpb] = *reinterpret_cast<const f32x4_t*>(
                &sl.eL[16 * jpb + 4 * lq]);
        }
        r.Q0 = sl.Q[0][lane];
        r.Q1 = sl.Q[1][lane];
        r.Arb = sl.Arb[lane];
        r.Ark = sl.Ark[lane];
        return true;
    };
    // y of the previous chunk as its two products, added and stored one
    // iteration late (complete by then): rows of chunk yc (yc < 0: none)
    // (into y buffer yc % NYBUF, whole rows stored by a producer)
    f32x4_t yq = zero4(), yp = zero4();
    int yc = -1;
    auto store_y = [&]() {
        f32x4_t yy;
#pragma unroll
        for (int e = 0; e < 4; ++e) yy[e] = yq[e] + yp[e];
        const int yb = yc & (NYBUF - 1);
        *reinterpret_cast<uint2*>(&sm.ys[yb][lr][16 * ib + 4 * lq]) =
            pack4(yy);
        if (ib == 0 && lane == 0) lds_store(&sm.ychunk[yb], yc);
    };
    // this chain's rows of a checkpoint: written to its LDS rows in the
    // register layout, read back at once as whole rows (lane l: 16-byte
    // units l and l + 64, row u / 8, columns 8 (u % 8) ..) and stored in the
    // next iteration, at element offset ckp (ckp < 0: none pending)
    CkRows& ckr = sm.ck[ib];
    int64_t ckp = -1;
    uint4 ckd0 = {}, ckd1 = {};
    auto store_ck = [&]() {
        bf16_t* const dst =
            A.ckpt + ckp + (16 * ib + (lane >> 3)) * WN + 8 * (lane & 7);
        *reinterpret_cast<uint4*>(dst) = ckd0;
        *reinterpret_cast<uint4*>(dst + 8 * WN) = ckd1;
    };

    // running counters instead of divisions by the slot count and the
    // checkpoint stride: the slot of chunk c, c modulo the stride, and the
    // element offset of checkpoint c / stride
    int s = 0, cph = 0;
    int64_t ckoff = sbase;
    SlotRegs cur;
    // this workgroup's chunks [c_lo, c_hi); it carries the state through the
    // chunks before c_lo without writing y or checkpoints
    const int sg = seg_of(A);
    const int c_lo = A.seg_lo[sg], c_hi = A.seg_hi[sg];
    const int nrun = c_hi > 0 && take(0, 0, -1, cur) ? c_hi : 0;
    for (int c = 0; c < nrun; ++c) {
        const int64_t t0 = int64_t(c) * WL;
        const int n = int(T - t0 < WL ? T - t0 : WL);
        const int exact = cur.exact;
        const bool own = c >= c_lo;
        const int sn = s + 1 == NSLOT ? 0 : s + 1;  // the next chunk's slot

        // bf16(S_0): the operand of the state step and of y, and the
        // checkpoint's rows
        i16x4_t sb[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) sb[jb] = kq(S[jb]);
        const bf16x8_t Sb0 = pk8(sb[0], sb[1]), Sb1 = pk8(sb[2], sb[3]);
        if (!exact) {
            // X^T_ib = W^ bf16(S_0)^T + U (rows of block ib, as D(X_ib)),
            // then S_L^T = S_0^T diag(2^{g_L}) + B^^T X + K^^T V
            f32x4_t xt = unpack4(__builtin_bit_cast(uint2, cur.U));
            mfma(xt, cur.W0, Sb0);
            mfma(xt, cur.W1, Sb1);
            const i16x4_t X = kq(xt);
#pragma unroll
            for (int jpb = 0; jpb < 4; ++jpb) {
                f32x4_t acc;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[e] = S[jpb][e] * cur.eL[jpb][e];
                mfma16(acc, cur.B[jpb], X);
                mfma16(acc, cur.K[jpb], cur.V);
                S[jpb] = acc;
            }
        }
        // the next chunk's ready word (read for every chunk; unused after
        // the last), used after this chunk's step
        const int word = lds_load(vready + sn);
        if (yc >= 0) store_y();
        yc = -1;
        if (ckp >= 0) store_ck();
        ckp = -1;
        if (A.ckpt && cph == 0 && own) {
            // rows 16 ib .. + 15 of checkpoint c / stride, and at once their
            // whole-row read-back (the same wave's LDS accesses complete in
            // order)
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
                *reinterpret_cast<i16x4_t*>(&ckr[lr][16 * jb + 4 * lq]) =
                    sb[jb];
            ckd0 = *reinterpret_cast<const uint4*>(
                &ckr[lane >> 3][8 * (lane & 7)]);
            ckd1 = *reinterpret_cast<const uint4*>(
                &ckr[8 + (lane >> 3)][8 * (lane & 7)]);
            ckp = ckoff;
        }
        if (!exact && own) {
            // Y^T_ib = bf16(S_0) Q^^T + U^T Arb^T + V^T Ark^T, lane:
            // y[t0 + lr][16 ib + 4 lq ..] (added and stored in the next
            // iteration)
            yp = zero4();
            yq = zero4();
            mfma16(yp, cur.U, cur.Arb);
            mfma16(yp, cur.V, cur.Ark);
            mfma(yq, Sb0, cur.Q0);
            mfma(yq, Sb1, cur.Q1);
            yc = c;
        } else {
            lds_drain();  // the slot's reads (some unused) have completed
        }
        // the slot goes back to the producers: its reads completed before
        // their values were used
        if (lane == 0)
            __hip_atomic_fetch_add(&sm.done[s], 1, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_WORKGROUP);
        s = sn;
        if (++cph == A.cstride) {
            cph = 0;
            ckoff += A.BH * NN;
        }
        if (c + 1 < c_hi &&
            !take(c + 1, s, __builtin_amdgcn_readfirstlane(word), cur))
            break;
        if (exact) {
            // exact fp32 sequential pass over the chunk for the rows of
            // block ib (a chunk outside the factored form's range, far
            // beyond the model's clamped decays): sums over the lane's 16
            // columns, then over the four lanes of the row (lq = 0..3)
            for (int t = 0; t < n; ++t) {
                const int64_t off = (t0 + t) * A.lay.ts + hoff;
                float sa = 0.f;
#pragma unroll
                for (int jb = 0; jb < 4; ++jb)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        sa += S[jb][e] *
                              bf16_to_f32(A.a[off + 16 * jb + 4 * lq + e]);
                sa += __shfl_xor(sa, 16);
                sa += __shfl_xor(sa, 32);
                const float vi = bf16_to_f32(A.v[off + row]);
                float acc = 0.f;
#pragma unroll
                for (int jb = 0; jb < 4; ++jb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int64_t j = off + 16 * jb + 4 * lq + e;
                        const float d = expf(-expf(bf16_to_f32(A.w[j])));
                        S[jb][e] = S[jb][e] * d + sa * bf16_to_f32(A.b[j]) +
                                   vi * bf16_to_f32(A.k[j]);
                        acc += S[jb][e] * bf16_to_f32(A.r[j]);
                    }
                acc += __shfl_xor(acc, 16);
                acc += __shfl_xor(acc, 32);
                if (lq == 0 && own) A.y[off + row] = to_bf16(acc);
            }
        }
    }
    if (yc >= 0) store_y();
    if (ckp >= 0) store_ck();

    // final state (fp32) and the last checkpoint, from the segment that
    // ends the sequence
    if (c_hi < nch) return;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        *reinterpret_cast<float4*>(A.s_t + sbase + row * WN + 16 * jb +
                                   4 * lq) =
            make_float4(S[jb][0], S[jb][1], S[jb][2], S[jb][3]);
        if (A.ckpt)
            *reinterpret_cast<uint2*>(A.ckpt +
                                      ((nch + A.cstride - 1) / A.cstride) *
                                          A.BH * NN +
                                      sbase +
                                      row * WN + 16 * jb + 4 * lq) =
                pack4(S[jb]);
    }
}

// A workgroup whose hand-over failed overwrites every output it writes --
// y and the checkpoints of its segment's chunks, and S_T if its segment ends
// the sequence -- with NaN, so that a lost hand-over can never pass as a
// result.
__device__ __forceinline__ void poison(const FwdArgs& A, int tid) {
    const int64_t bh = head_of(A);
    const int sg = seg_of(A);
    const int64_t hoff = A.lay.head(bh, WN);
    const int64_t NN = WN * WN;
    const int64_t nch = (A.T + WL - 1) / WL;
    const int64_t t_lo = int64_t(A.seg_lo[sg]) * WL;
    int64_t t_hi = int64_t(A.seg_hi[sg]) * WL;
    if (t_hi > A.T) t_hi = A.T;
    const bool last = A.seg_hi[sg] == nch;
    const bf16_t nan16 = 0x7fc0;
    for (int64_t e = t_lo * WN + tid; e < t_hi * WN; e += WTHREADS)
        A.y[(e / WN) * A.lay.ts + hoff + e % WN] = nan16;
    if (last)
        for (int e = tid; e < WN * WN; e += WTHREADS)
            A.s_t[bh * NN + e] = __builtin_nanf("");
    if (A.ckpt) {
        // checkpoint k holds the state before chunk k * stride (the last
        // one S_T): those of this segment's chunks, and S_T's if last
        const int64_t nck = (nch + A.cstride - 1) / A.cstride + 1;
        for (int64_t k = 0; k < nck; ++k) {
            const int64_t c = k * A.cstride;
            const bool mine = (c >= A.seg_lo[sg] && c < A.seg_hi[sg]) ||
                              (last && k == nck - 1);
            if (!mine) continue;
            for (int e = tid; e < WN * WN; e += WTHREADS)
                A.ckpt[k * A.BH * NN + bh * NN + e] = nan16;
        }
    }
}

__global__ void __launch_bounds__(WTHREADS)
wkv7_wave_fwd_kernel(FwdArgs A) {
    __shared__ WaveFwdSmem sm;
    const int tid = threadIdx.x, lane = tid & 63;
    // the wave index, in a scalar register: every chunk index, token offset
    // and base address derived from it stays scalar
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (tid < NSLOT) {
        sm.ready[tid] = -1;
        sm.done[tid] = 0;
    }
    if (tid < NYBUF) sm.ychunk[tid] = -1;

    if (tid == 0) sm.failed = 0;
    __syncthreads();
    if (wv < NCHAIN)
        chain(A, sm, wv, lane);
    else
        produce(A, sm, wv - NCHAIN, lane);
    // every wait is bounded, so every wave arrives here (with no LDS DMA
    // in flight)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (lds_load(&sm.failed) != 0) {
        poison(A, tid);
        return;
    }
    // the y of the last chunks, which no later producer stored: wave b
    // stores buffer b
    if (wv < NYBUF) {
        const int ych = __builtin_amdgcn_readfirstlane(lds_load(&sm.ychunk[wv]));
        if (ych >= 0)
            store_y_rows(A, sm, wv, ych, A.lay.head(head_of(A), WN), lane);
    }
}

}  // namespace

namespace {

// Cost of a chunk whose workgroup only carries the state through it (no y,
// no checkpoint), relative to a chunk it writes.  A chain wave takes about
// 1,190 against 1,850 cycles per chunk, but the whole workgroup's time also
// has the producers' start and the chain's end; 0.8 gave the shortest
// forwards of 0.5 .. 0.95 measured at B8 T512 H12, B4 T512 H12 and
// B1 T2048 H8.
constexpr double kFwdPassCost = 0.8;

std::atomic<int> g_force_fwd_segments{0};
std::atomic<int> g_fwd_cu_count[64];

int fwd_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = g_fwd_cu_count[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                                  dev) != hipSuccess)
            return 0;
        g_fwd_cu_count[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Splits a head's nch chunks over k workgroups (at most kMaxFwdSegments):
// segment j owns chunks [lo[j], hi[j]) and first carries the state through
// every earlier chunk.  Equal finishing times give segment j the weight
// 1 - kFwdPassCost * (the weights before it).  Returns the number of
// segments (1 when a segment would own no chunk).
int plan_fwd_segments(int nch, int k, int* lo, int* hi) {
    lo[0] = 0;
    hi[0] = nch;
    if (k > kMaxFwdSegments) k = kMaxFwdSegments;
    for (; k >= 2; --k) {
        double wt[kMaxFwdSegments], tot = 0, before = 0;
        for (int j = 0; j < k; ++j) {
            wt[j] = 1.0 - kFwdPassCost * before;
            if (wt[j] < 0.1) wt[j] = 0.1;
            before += wt[j];
            tot += wt[j];
        }
        int b[kMaxFwdSegments + 1];
        b[0] = 0;
        b[k] = nch;
        bool ok = true;
        double cum = 0;
        for (int j = 1; j < k && ok; ++j) {
            cum += wt[j - 1];
            b[j] = int(nch * cum / tot + 0.5);
            if (b[j] <= b[j - 1] || b[j] >= nch) ok = false;
        }
        if (!ok) continue;
        for (int j = 0; j < k; ++j) {
            lo[j] = b[j];
            hi[j] = b[j + 1];
        }
        return k;
    }
    return 1;
}

}  // namespace

void set_forward_segments(int k) {
    g_force_fwd_segments.store(k < 0 ? 0 : k, std::memory_order_relaxed);
}

hipError_t launch_wave_forward(const ChunkFwdArgs& p, hipStream_t stream) {
    // p.L: the checkpoint interval, a multiple of the 16-token chunk
    if (p.L % WL != 0 || p.L / WL < 1 || p.L / WL > 4)
        return hipErrorInvalidValue;
    FwdArgs A;
    A.T = p.T;
    A.BH = p.B * p.H;
    A.lay = p.lay;
    A.r = static_cast<const bf16_t*>(p.r);
    A.w = static_cast<const bf16_t*>(p.w);
    A.k = static_cast<const bf16_t*>(p.k);
    A.v = static_cast<const bf16_t*>(p.v);
    A.a = static_cast<const bf16_t*>(p.a);
    A.b = static_cast<const bf16_t*>(p.b);
    A.s0 = p.s0;
    A.y = static_cast<bf16_t*>(p.y);
    A.s_t = p.s_t;
    A.ckpt = static_cast<bf16_t*>(p.ckpt);
    A.cstride = p.L / WL;
    A.cshift = A.cstride == 4 ? 2 : A.cstride == 2 ? 1 : 0;
    A.wait = p.wait;
    if (A.BH <= 0) return hipSuccess;
    // workgroups per head: as many as fit beside the other heads' on the
    // device's CUs (one workgroup per CU), at most kMaxFwdSegments
    int k = g_force_fwd_segments.load(std::memory_order_relaxed);
    if (k == 0) {
        const int cus = fwd_cu_count();
        k = cus > 0 && A.BH < cus ? int(cus / A.BH) : 1;
    }
    for (int g = 0; g < kMaxFwdSegments; ++g) A.seg_lo[g] = A.seg_hi[g] = 0;
    A.nseg = plan_fwd_segments(int((A.T + WL - 1) / WL), k, A.seg_lo,
                               A.seg_hi);
    if (A.BH * A.nseg > int64_t(UINT32_MAX)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(wkv7_wave_fwd_kernel, dim3(unsigned(A.BH * A.nseg)),
                       dim3(WTHREADS), 0, stream, A);
    return hipGetLastError();
}

}  // namespace rwkv7m
