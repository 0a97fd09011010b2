// Wave-specialised WKV-7 backward for gfx950: bf16 vectors, fp32 state,
// N = 64, 16-token chunks, bf16 checkpoints every L = 16 m tokens
// (m = 1, 2 or 4).
//
// Per 16-token chunk with start state S_0 and end-state cotangent D (the
// chunk's closed form; g = running log2-decay, g_ref its value at token 7,
// A~ = a 2^{g_{t-1}-g_ref}, R~ = r 2^{g_t-g_ref},
// B~ = b 2^{g_ref-g_t}, K~ = k 2^{g_ref-g_t}, A^ = A~ 2^{g_ref},
// B^ = B~ 2^{g_L-g_ref}, K^ = K~ 2^{g_L-g_ref}; Aab = A~ B~^T and
// Aak = A~ K~^T strictly lower, Arb = R~ B~^T and Ark = R~ K~^T lower with
// the diagonal; Minv = (I - Aab)^{-1}):
//
//   U  = A^ S_0^T + Aak V        X = Minv U   (X_t = S_{t-1} a_t)
//   dX = B^ D^T + Arb^T dY       dU = Minv^T dX
//   dV = K^ D^T + Ark^T dY + Aak^T dU
//   dArb = lower(dY X^T), dArk = lower(dY V^T), dAab = slower(dU X^T),
//   dAak = slower(dU V^T)
//   dR~ = (dY S_0) 2^{g_ref} + dArb B~ + dArk K~
//   dA~ = (dU S_0) 2^{g_ref} + dAab B~ + dAak K~
//   dB~ = dAab^T A~ + dArb^T R~ + (X D) 2^{g_L-g_ref}
//   dK~ = dAak^T A~ + dArk^T R~ + (V D) 2^{g_L-g_ref}
//   D_0 = D 2^{g_L} + bf16(D) B^^T W^ + dY^T Q^      (the cotangent of S_0)
//
// with W^ = Minv A^ and Q^ = R~ 2^{g_ref} + Arb W^.  The decay gradient
// uses the chunk-start identity (S_0 and D_0 fixed; exact for the chunk)
//
//   dlog d_t = sum_{t' < t} (b db + k dk - r dr)_{t'} - sum_{t' <= t} (a da)_{t'}
//              + E_0,   E_0 = sum_i D_0[i, :] S_0[i, :]
//
// and dw = dlog d * (-e^w).  E is needed at every other chunk boundary
// only: a start member (a position of the reverse order of parity tpar, or
// position 0) takes it at its start; the chunk at the next position, one
// chunk earlier in time, takes the same value as its end value E_L and
// recovers its own start value through the same identity,
// E_0 = E_L - sum over the chunk of (b db + k dk - r dr - a da).  With an
// interval of two chunks the start members are the checkpoint chunks, so
// that the chains never wait for a recomputed start state.  These are the
// reference's reverse equations (src/rwkv7m/kernels/wkv_pallas_gpu.py:
// 221-257) summed over a chunk; states come from checkpoints, never from
// dividing by the decay.  Inside an
// interval of m chunks, the start state of chunk c + 1 is recomputed from
// chunk c's: S_L = S_0 2^{g_L} + X^T B^ + V^T K^.
//
// One workgroup of 8 waves per (batch, head):
//   * waves 0..3, the chains: chain ib holds rows 16 ib .. 16 ib + 15 of the
//     fp32 cotangent D in registers and walks the chunks in reverse.  Per
//     chunk it writes bf16(D) into the chunk's worker's D buffer, takes the
//     worker's map (B^, W^, Q^, dY), advances D_0 (2 + 4 MFMAs: D_0 depends
//     only on rows of D, so the four chains are independent) and, at even
//     positions, adds its rows' share of sum_i D_0 S_0 for the two workers
//     that use it;
//   * waves 4..7, the workers: worker w takes chunks nch - 1 - w,
//     nch - 1 - w - 4, ...  It loads the chunk's vectors, forms the factors,
//     the 16 x 16 matrices and the inverse in registers, publishes the map,
//     recomputes the next chunk's start state if the interval continues
//     (at an interval of two chunks it hands X, V, B^ and K^ to the chains,
//     which form that state between their steps), then, once D has arrived, forms every gradient in registers and writes
//     them.  Four chunks are in flight at once; only D is serial.
// Register layouts are those of wkv7_wave_common.h.  The S and D buffers are
// bf16 64 x 64 in 16-byte units (sd_off), read as row fragments (plain
// reads) or column fragments (gfx950 transposing reads).
//
// A chunk outside the factored form's range (log-decay span beyond +-40
// around the reference point) stops the workgroup: it leaves
// kExactPassMark in dS0[b][h][0][0] and the exact sequential backward
// recomputes that head.  Every wait is bounded (wkv7_status.hip); a wait
// that gives up sets every output of the head to NaN and raises the
// device's failure counter.

#include <atomic>

#include "wkv7_wave_bwd_common.h"

namespace rwkv7m {
namespace {

using namespace wave;

constexpr int NCHAIN = 4;
constexpr int NWORK = 4;
constexpr int BTHREADS = 64 * (NCHAIN + NWORK);
constexpr int NN = WN * WN;

// A chunk's hand-over from its worker to the chains, as register images
// (element [..][lane] is that lane's operand).
struct BMap {
    bf16x8_t Bh[2][64];  // B~ (T layout pairs): x32 A operands (m = t, k = j)
    bf16x8_t QW[4][64];  // D(Q^_jb) (slots 0..3), D(W^_jb) (slots 4..7)
    i16x4_t dY[4][64];   // D(dY_ib)
};

struct BwdFlags {
    int map_ready[NWORK];  // maps the worker has published (count)
    int map_taken[NWORK];  // chain reads of its maps (NCHAIN per map)
    int d_cnt[NWORK];      // chain writes into its D buffer (NCHAIN per chunk)
    int d_done[NWORK];     // chunks whose D buffer the worker has finished
    int tail_cnt[NWORK];   // chain tail partials (NCHAIN per chunk)
    int tail_used[NWORK];  // odd workers' reads of the even tail (count)
    int s_ready[NWORK];    // chunk whose start state the S buffer holds
    int s_free[NWORK];     // chunk whose start state the S buffer takes next
    // interval of two chunks: the chains form the odd chunk's start state
    int h_ready[NWORK];    // chunk whose step operands the buffers hold
    int h_read[NWORK];     // chain reads of the worker's shared operands
    int s_cnt[NWORK];      // chain writes of start-state rows (NCHAIN each)
    int abort;             // a chunk needs the exact pass: every wave stops
    int failed;            // a bounded wait gave up
};

// LDS, as separate objects: the vector stage (the only LDS DMA target read
// after a DMA is issued in the same chunk) is then provably distinct from
// every other array, and the compiler inserts no vmcnt wait before their
// reads while a prefetch is in flight.
// lds_stage[w][v][h][s][u]: 16-byte segment s (columns 8s .. 8s + 7) of
// token 8h + u of vector v (r, w, k, v, neg_kk, kka, dy)
__shared__ uint4 lds_stage[NWORK][7][2][8][8];
__shared__ bf16_t lds_S[NWORK][NN];  // the chunk's start state (sd_off)
__shared__ bf16_t lds_D[NWORK][NN];  // the cotangent of its end state
__shared__ BMap lds_map[NWORK];
// sum_i D_0 S_0 per chain, for the start members' workers (tail_start)
__shared__ float lds_tail[NWORK][NCHAIN][WN];
// per-column factors of the chunk: [0] 2^{g_L - g_ref}, [1] 2^{g_ref},
// [2] 2^{g_L} (written by lanes 0, 1, 2 of each 16-lane row in one store)
__shared__ float lds_fac[NWORK][3][WN];
__shared__ BwdFlags lds_flags;

// Wait until pred(*p) holds: 1 when it does, 0 when the workgroup aborted
// first, -1 when the poll budget ran out (then the workgroup is marked
// failed and aborted).  A chain (raised issue priority) that has to wait
// drops to normal priority until pred holds, so that its polls do not take
// issue slots from the worker sharing its SIMD.  The abort word is read on
// every eighth poll.
template <typename Pred>
__device__ __forceinline__ int wait_for(const WaitCfg& wc, int* p, int lane,
                                        Pred pred, bool chain = false) {
    if (pred(__builtin_amdgcn_readfirstlane(lds_load(p)))) {
        asm volatile("" ::: "memory");
        return 1;
    }
    if (chain) __builtin_amdgcn_s_setprio(0);
    for (int it = 1; it < wc.limit; ++it) {  // wc.limit polls in all
        if (pred(__builtin_amdgcn_readfirstlane(lds_load(p)))) {
            asm volatile("" ::: "memory");
            if (chain) __builtin_amdgcn_s_setprio(2);
            return 1;
        }
        if ((it & 7) == 7 &&
            __builtin_amdgcn_readfirstlane(lds_load(&lds_flags.abort)) != 0)
            return 0;
        __builtin_amdgcn_s_sleep(1);
    }
    wait_failed(&lds_flags.failed, wc.failures, lane);
    if (lane == 0) lds_store(&lds_flags.abort, 1);
    return -1;
}


// Whether the chunk at reverse position p takes the decay gradient's
// boundary sum sum_i D_0 S_0 at its start (a start member; the chains form it
// there) or at its end, from the start member one position earlier (an end
// member, one chunk earlier in time).  Start members are the positions of
// parity A.tpar, and position 0 (whose end is the sequence's end).
__device__ __forceinline__ bool tail_start(const BwdArgs& A, int p) {
    return (p & 1) == A.tpar || p == 0;
}

// ---------------------------------------------------------------------------
// Chain ib: rows 16 ib .. 16 ib + 15 of the cotangent through every chunk.
// Intervals of two chunks: at the odd chunk c it also forms rows 16 ib ..
// + 15 of that chunk's start state from chunk c - 1's checkpoint and step
// operands (see work()).
template <int M>
__device__ __forceinline__ void chain(const BwdArgs& A, int ib, int lane) {
    const int lr = lane & 15, lq = lane >> 4;
    const int64_t bh = head_of(A);
    const int nch = int((A.T + WL - 1) / WL);
    // this workgroup's chunks [c_lo, c_hi); the later ones it only passes
    // the cotangent through
    const int sg = seg_of(A);
    const int c_lo = A.seg_lo[sg], c_hi = A.seg_hi[sg];
    const int row = 16 * ib + lr;
    BwdFlags& fl = lds_flags;
    __builtin_amdgcn_s_setprio(2);  // the serial path
    // the identity and a matrix of ones as bf16 operands (B and A)
    i16x4_t kI, kOne;
    {
        f32x4_t id, one;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            id[e] = (4 * lq + e == lr) ? 1.f : 0.f;
            one[e] = 1.f;
        }
        kI = kq(id);
        kOne = kq(one);
    }
    // tiles D(D^T_{j'b, ib}): lane holds D[row][16 j'b + 4 lq + e]
    f32x4_t Dt[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        Dt[jb] = zero4();
        if (A.ds_t)
            Dt[jb] = *reinterpret_cast<const f32x4_t*>(
                A.ds_t + bh * NN + row * WN + 16 * jb + 4 * lq);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)

    bool done = true;
    for (int p = 0; p < nch - c_lo; ++p) {
        const int c = nch - 1 - p;
        const int w = p % NWORK, kord = p / NWORK;

        // the chunk's map (its per-column factors are in LDS by then)
        if (wait_for(A.wait, &fl.d_done[w], lane,
                     [&](int x) { return x >= kord; }, true) <= 0 ||
            wait_for(A.wait, &fl.map_ready[w], lane,
                     [&](int x) { return x >= kord + 1; }, true) <= 0) {
            done = false;
            break;
        }
        // bf16(D diag(2^{g_L - g_ref})): the step's operand and the
        // worker's D buffer (folding the per-column factor in here takes it
        // out of every product of D with B~ and K~)
        i16x4_t sb[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const f32x4_t elr = *reinterpret_cast<const f32x4_t*>(
                &lds_fac[w][0][16 * jb + 4 * lq]);
            f32x4_t x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = Dt[jb][e] * elr[e];
            sb[jb] = kq(x);
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
            sd_write4(lds_D[w], row, 16 * jb + 4 * lq,
                      __builtin_bit_cast(uint2, sb[jb]));
        lds_drain();
        if (lane == 0) lds_add(&fl.d_cnt[w], 1);
        const BMap& mp = lds_map[w];
        const bf16x8_t Bh0 = mp.Bh[0][lane], Bh1 = mp.Bh[1][lane];
        bf16x8_t QW[4];
        f32x4_t eL[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            QW[jb] = mp.QW[jb][lane];
            eL[jb] = *reinterpret_cast<const f32x4_t*>(
                &lds_fac[w][2][16 * jb + 4 * lq]);
        }
        const i16x4_t dYt = mp.dY[ib][lane];
        lds_drain();
        if (lane == 0) lds_add(&fl.map_taken[w], 1);

        // Z = B~ bf16(D diag(2^{g_L - g_ref}))^T = B^ D^T ([t][i]), then
        // D_0^T = 2^{g_L} D^T + Q^^T dY + W^^T Z (rows of block ib), the
        // two products over t as one K = 32 product: (Q^ | W^)^T (dY ; Z)
        f32x4_t z = zero4();
        mfma(z, Bh0, pk8(sb[0], sb[1]));
        mfma(z, Bh1, pk8(sb[2], sb[3]));
        const bf16x8_t dYZ = pk8(dYt, kq(z));
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            f32x4_t acc;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = Dt[jb][e] * eL[jb][e];
            mfma(acc, QW[jb], dYZ);
            Dt[jb] = acc;
        }

        // An odd chunk of an interval of two: its start state, rows 16 ib ..
        // + 15, S_L = S_0 2^{g_L} + X^T B^ + V^T K^ of chunk c - 1 (worker
        // we, position p + 1).  B^ and K^ (J layout, all key blocks) are in
        // that worker's D buffer, which the chains write only after its map
        // (published once every chain has read them); X and V of value block
        // ib (J layout) in this chain's own 16 rows of this worker's S
        // buffer, which it reads before writing its rows there.
        const bool fed = M == 2 && (c & 1) && c < c_hi;
        if (fed) {
            const int we = (w + 1) % NWORK;
            if (wait_for(A.wait, &fl.h_ready[w], lane,
                         [&](int x) { return x == c; }, true) <= 0) {
                done = false;
                break;
            }
            const i16x4_t* const hs = reinterpret_cast<const i16x4_t*>(lds_D[we]);
            const i16x4_t* const hp = reinterpret_cast<const i16x4_t*>(lds_S[w]);
            i16x4_t kB[4], kK[4];
            uint2 s0r[4];
            f32x4_t el[4];
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                kB[jb] = hs[64 * jb + lane];
                kK[jb] = hs[64 * (4 + jb) + lane];
                s0r[jb] = sd_read4(lds_S[we], row, 16 * jb + 4 * lq);
                el[jb] = *reinterpret_cast<const f32x4_t*>(
                    &lds_fac[we][2][16 * jb + 4 * lq]);
            }
            const bf16x8_t XV = pk8(hp[64 * (4 * ib) + lane],
                                    hp[64 * (4 * ib + 1) + lane]);
            lds_drain();
            if (lane == 0) lds_add(&fl.h_read[we], 1);
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                const f32x4_t s0 = unpack4(s0r[jb]);
                f32x4_t acc;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[e] = s0[e] * el[jb][e];
                mfma(acc, pk8(kB[jb], kK[jb]), XV);
                sd_write4(lds_S[w], row, 16 * jb + 4 * lq, pack4(acc));
            }
            lds_drain();
            if (lane == 0) lds_add(&fl.s_cnt[w], 1);
        }

        // The decay gradient needs sum_i D_0[i][j] S_0[i][j] at every other
        // chunk boundary only: a start member's worker takes it as its
        // chunk's start value, and the worker of the next position, one
        // chunk earlier in time, as its chunk's end value (tail_start).
        if (!tail_start(A, p)) continue;
        if (c >= c_hi) {
            // a chunk past this workgroup's own: no gradients, so no share,
            // but the count stays in step with the worker's chunk order
            if (lane == 0) lds_add(&fl.tail_cnt[w], 1);
            continue;
        }
        // this block's share for the worker.  P = D_0 * S_0 on the block's
        // tiles D(P^T) is split into bf16 parts P = P_hi + P_lo (16
        // significant bits); each part is turned into D(P) by P I and summed
        // over i by a product with ones (exact for bf16 values, fp32
        // accumulation)
        // (rows of a start state this chain formed itself need no wait)
        if ((!fed && wait_for(A.wait, &fl.s_ready[w], lane,
                              [&](int x) { return x == c; }, true) <= 0) ||
            (kord > 0 && wait_for(A.wait, &fl.tail_used[(w + 1) % NWORK], lane,
                                  [&](int x) { return x >= kord; },
                                  true) <= 0)) {
            done = false;
            break;
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const f32x4_t s0 =
                unpack4(sd_read4(lds_S[w], row, 16 * jb + 4 * lq));
            f32x4_t pt, plo;
#pragma unroll
            for (int e = 0; e < 4; ++e) pt[e] = Dt[jb][e] * s0[e];
            const i16x4_t khi = kq(pt);
            const f32x4_t phi = unpack_i16(khi);
#pragma unroll
            for (int e = 0; e < 4; ++e) plo[e] = pt[e] - phi[e];
            f32x4_t ph = zero4(), pl = zero4(), cs = zero4();
            mfma16(ph, khi, kI);       // D(P_hi)
            mfma16(pl, kq(plo), kI);   // D(P_lo)
            mfma16(cs, kOne, kq(ph));  // every row: sum_i P[i][j]
            mfma16(cs, kOne, kq(pl));
            if (lq == 0) lds_tail[w][ib][16 * jb + lr] = cs[0];
        }
        lds_drain();
        if (lane == 0) lds_add(&fl.tail_cnt[w], 1);
    }
    if (done && c_lo == 0) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
            *reinterpret_cast<f32x4_t*>(A.ds0 + bh * NN + row * WN + 16 * jb +
                                        4 * lq) = Dt[jb];
    }
}

// ---------------------------------------------------------------------------
// Worker w: chunks nch - 1 - w, nch - 1 - w - NWORK, ...
// The vectors of chunk c straight to worker w's stage (global_load_lds
// writes lane l's 16 bytes at 16 l): lane l of load (vector, h) fetches
// segment l / 8 of token 8h + l % 8; tokens past the end re-read the last
// token.
// cb2: byte offset of the chunk's first token of this head; n: its tokens.
__device__ __forceinline__ void fetch_vecs(const BwdArgs& A, int w,
                                           uint32_t cb2, int n, int lane) {
    const VecPtrs src{A.r, A.w, A.k, A.v, A.a, A.b, A.dy};
    const int ldu = lane & 7, ldseg = lane >> 3;
    // the stage's LDS address, formed here and opaque to the compiler: the
    // fourteen destinations are then sums formed at each load, instead of
    // fourteen scalar registers held (and spilled) across the whole loop
    uint32_t base = lds_addr(&lds_stage[w][0][0][0][0]);
    asm volatile("" : "+s"(base));
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int t = 8 * h + ldu;
        const uint32_t off =
            cb2 + uint32_t(t < n ? t : n - 1) * A.ts2 + 16 * ldseg;
#pragma unroll
        for (int vv = 0; vv < 7; ++vv)
            dma16(src.get(vv), off,
                  base + uint32_t(sizeof(lds_stage[0][0])) * vv +
                      uint32_t(sizeof(lds_stage[0][0][0])) * h);
    }
}

// Checkpoint c / M (chunk c starts an interval) straight to worker w's S
// buffer: load g fills rows 8g .. 8g + 7 (lane l: row 8g + l % 8, segment
// l / 8).
template <int M>
__device__ __forceinline__ void fetch_state(const BwdArgs& A, int w, int c,
                                            int lane) {
    const uint32_t off =
        (uint32_t(c / M) * uint32_t(A.BH) + uint32_t(head_of(A))) *
            uint32_t(NN * 2) +
        uint32_t(((lane & 7) * WN + 8 * (lane >> 3)) * 2);
    uint32_t base = lds_addr(&lds_S[w][0]);
    asm volatile("" : "+s"(base));
#pragma unroll
    for (int g = 0; g < 8; ++g)
        dma16(A.ckpt, off + 8 * g * WN * 2, base + 1024 * g);
}

// The T layout read of vector vv from worker w's stage: token lr, columns
// 16 kb + 4 lq .. + 3 (segment 2 kb + lq / 2, half lq % 2).
__device__ __forceinline__ uint2 read_t(int w, int vv, int kb, int lane) {
    const int lr = lane & 15, lq = lane >> 4;
    const bf16_t* p = reinterpret_cast<const bf16_t*>(
        &lds_stage[w][vv][lr >> 3][2 * kb + (lq >> 1)][lr & 7]);
    return *reinterpret_cast<const uint2*>(p + 4 * (lq & 1));
}

// The J layout tile D(X_jb) of vector vv from worker w's stage by one
// transposing read: lane s of each 16-lane group addresses token 4 lq + s / 4,
// columns 16 jb + 4 (s % 4) .. + 3 (segment 2 jb + (s % 4) / 2, half s % 2),
// and receives X[4 lq + e][16 jb + s].
__device__ __forceinline__ i16x4_t stage_j(int w, int vv, int jb, int lane) {
    const int s = lane & 15, q = lane >> 4;
    const int t = 4 * q + (s >> 2);
    const bf16_t* p = reinterpret_cast<const bf16_t*>(
        &lds_stage[w][vv][t >> 3][2 * jb + ((s & 3) >> 1)][t & 7]);
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(p + 4 * (s & 1)));
}

// ---------------------------------------------------------------------------
// Worker w: chunks nch - 1 - w, nch - 1 - w - NWORK, ...; checkpoints every
// M chunks.  ACC: the cotangents add_dr, add_dk, add_dv are added to dr, dk,
// dv before they are rounded; their 12 loads are issued just before the next
// chunk's vector loads (so that waiting for them does not wait for those)
// and count in the waits below.
template <int M, bool ACC>
__device__ __forceinline__ void work(const BwdArgs& A, int w, int lane0) {
    const int64_t bh = head_of(A);
    const uint32_t hoff2 = uint32_t(A.lay.head(bh, WN)) * 2;
    const int T = int(A.T);
    const int nch = (T + WL - 1) / WL;
    const uint32_t ts2 = A.ts2;
    constexpr int m = M;
    // Blocks of four independent 16-column tiles go through some phases
    // stage by stage, GW blocks at a time: all four for the plain instances
    // at intervals 16 and 32; one at a time where the registers of four in
    // flight would spill (interval 64, the summing instance).
    constexpr int GW = (M <= 2 && !ACC) ? 4 : 1;
    // the worker of chunk c + 1 (one position earlier in the reverse order),
    // whose start state chunk c's end state is
    const int wfeed = (w + NWORK - 1) % NWORK;
    BwdFlags& fl = lds_flags;
    bf16_t* const S = lds_S[w];
    bf16_t* const D = lds_D[w];
    BMap& map = lds_map[w];
    // this workgroup's chunks [c_lo, c_hi) (segment boundaries are interval
    // boundaries); for a chunk at or past c_hi it only publishes the map
    // that carries the cotangent through
    const int sg = seg_of(A);
    const int c_lo = A.seg_lo[sg], c_hi = A.seg_hi[sg];

    if (nch - 1 - w >= c_lo) {
        const int c0 = nch - 1 - w;
        fetch_vecs(A, w, uint32_t(c0) * WL * ts2 + hoff2,
                   T - c0 * WL < WL ? T - c0 * WL : WL, lane0);
        if (c0 < c_hi && c0 % m == 0) fetch_state<M>(A, w, c0, lane0);
    }

    // interval of two: this worker's chunks so far whose start states the
    // chains formed, and whose successors' step operands it handed over
    int nfed = 0, nfeed = 0;
    for (int kord = 0, p = w; p < nch - c_lo; ++kord, p += NWORK) {
        // lane-derived addresses and masks are formed inside each iteration:
        // hoisted out of the loop they would each hold a register for the
        // whole run
        int lane_it = threadIdx.x;
        asm volatile("" : "+v"(lane_it));
        const int lane = lane_it & 63, lr = lane & 15, lq = lane >> 4;
        // the identity as a B operand (for to_j)
        i16x4_t kI;
        {
            f32x4_t id;
#pragma unroll
            for (int e = 0; e < 4; ++e) id[e] = (4 * lq + e == lr) ? 1.f : 0.f;
            kI = kq(id);
        }
        // the zero half of a K = 16 product run as a K = 32 one
        const i16x4_t kZero = {0, 0, 0, 0};
        const int c = nch - 1 - p;
        const int cn = c - NWORK;  // this worker's next chunk
        const int n = T - c * WL < WL ? T - c * WL : WL;
        const bool valid = lr < n;
        // byte offset of the chunk's first token, and of this lane's token
        // row of the token-major outputs (kNoLane past the end: dropped)
        const uint32_t cb2 = uint32_t(c) * WL * ts2 + hoff2;
        const uint32_t row2 = valid ? cb2 + uint32_t(lr) * ts2 : kNoLane;
        const bool skim = c >= c_hi;  // only the map (past the segment)
        const bool more = cn >= c_lo;  // the worker has a next chunk
        // S_0 is checkpoint c / m; S_0 of c + 1 is formed here
        const bool starts = !skim && c % m == 0;
        const bool feeds = !skim && c % m != m - 1 && c + 1 < c_hi;
        if (M == 2 && !skim && !starts) ++nfed;
        // the decay gradient's boundary sum (tail_start): a start member
        // takes it at its own start (worker tw = w, round tk = kord); an end
        // member at its end, from the start member one position earlier
        // (worker w - 1; round kord - 1 when that is worker NWORK - 1)
        const bool endm = !tail_start(A, p);
        const int tw = endm ? (w + NWORK - 1) % NWORK : w;
        const int tk = (endm && w == 0) ? kord - 1 : kord;
        // the vectors.  Vector memory operations complete in issue order, and
        // since the vectors' loads this worker issued the previous chunk's 12
        // gradient stores (2 of dv, 10 of the column blocks, 16 bytes per
        // lane; none after a chunk that only published its map) and, when
        // this chunk starts an interval, its start state's 8 loads, whose
        // wait comes only before S_0's first use
        if (kord == 0 || c + NWORK >= c_hi) {
            if (starts)
                __builtin_amdgcn_s_waitcnt(0x0f78);  // vmcnt(8)
            else
                __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
        } else {
            if (starts)
                __builtin_amdgcn_s_waitcnt(0x4f74);  // vmcnt(20)
            else
                __builtin_amdgcn_s_waitcnt(0x0f7c);  // vmcnt(12)
        }
        asm volatile("" ::: "memory");

        uint2 raw[7][4];
#pragma unroll
        for (int vv = 0; vv < 7; ++vv)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) raw[vv][kb] = read_t(w, vv, kb, lane);
        // v and dy in the J layout (products over t), straight from the stage
        i16x4_t jV[4], jdY[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            jV[jb] = stage_j(w, 3, jb, lane);
            jdY[jb] = stage_j(w, 6, jb, lane);
        }
        lds_drain();
        // the cotangents added to this chunk's dv (value blocks ib) and dr,
        // dk (key blocks jb), at the lanes' own output offsets
        uint2 adv[4], adr[4], adk[4];
        if (ACC && !skim) {
            const __amdgpu_buffer_rsrc_t rv = in_rsrc(A.add_dv),
                                         rr = in_rsrc(A.add_dr),
                                         rk = in_rsrc(A.add_dk);
            const uint32_t lo0 = row2 + 8 * lq;
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) adv[ib] = load8(rv, lo0 + 32 * ib);
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
                adr[jb] = load8(rr, lo0 + 32 * jb);
                adk[jb] = load8(rk, lo0 + 32 * jb);
            }
        }
        // the stage is free: the next chunk's vectors load during this one
        if (more) fetch_vecs(A, w, cb2 - NWORK * WL * ts2, WL, lane);
        if (n < WL) {
            // (a branch, not selects: only a head's last chunk is short)
            asm volatile("" ::: "memory");
            // padding tokens: zero vectors and w = -inf (bf16), so that
            // they decay by nothing
#pragma unroll
            for (int vv = 0; vv < 7; ++vv) {
                const uint2 pad = vv == 1 ? make_uint2(0xff80ff80u, 0xff80ff80u)
                                          : make_uint2(0, 0);
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    raw[vv][kb] = valid ? raw[vv][kb] : pad;
            }
            // the J tiles hold tokens 4 lq + e
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * lq + e >= n) {
                        jV[jb][e] = 0;
                        jdY[jb][e] = 0;
                    }
        }

        // ---- factors (T layout) ------------------------------------------
        // The per-column factors and the map of this worker's previous chunk
        // are read by every chain at that chunk's position (the factors
        // before the map's hand-over count): overwrite neither before the
        // count says all have been read.
        if (wait_for(A.wait, &fl.map_taken[w], lane,
                     [&](int x) { return x >= NCHAIN * kord; }) <= 0)
            break;
        // lam = log2 d_t, g its running sum over the chunk, g_ref = g at
        // token 7, g_L = g at token 15 (padding tokens decay by nothing)
        i16x4_t tA[4], tR[4], tB[4], tK[4], tAh[4];
        // kept for the input gradients: 2^{g_t - g_ref}, 2^{g_ref - g_t},
        // 2^{g_{t-1} - g_ref} (bf16) and -e^w (the decay gradient's factor)
        i16x4_t keg[4], keng[4], kep[4];
        f32x4_t lam4[4], facv[4];
        float lo = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const f32x4_t wr = unpack4(raw[1][kb]);
            const f32x4_t ar = unpack4(raw[4][kb]), br = unpack4(raw[5][kb]);
            const f32x4_t rr = unpack4(raw[0][kb]), kr = unpack4(raw[2][kb]);
            f32x4_t sp4, lr4, fA, fR, fB, fK, eh, eg4, eng4, ep4;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ew = __builtin_amdgcn_exp2f(wr[e] * kLog2e);
                const float g = scan16(-ew * kLog2e);
                lam4[kb][e] = -ew;
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
                eg4[e] = eg;
                eng4[e] = eng;
                ep4[e] = eprev;
                sp4[e] = sp;
                const float sLR = pin_lanes(row_bcast<15>(eg));
                lr4[e] = sLR;
                fA[e] = ar[e] * eprev;
                fR[e] = rr[e] * eg;
                fB[e] = br[e] * eng;
                fK[e] = kr[e] * eng;
                eh[e] = fA[e] * pin_lanes(row_bcast<1>(sp));
            }
            tA[kb] = kq(fA);
            tR[kb] = kq(fR);
            tB[kb] = kq(fB);
            tK[kb] = kq(fK);
            tAh[kb] = kq(eh);
            keg[kb] = kq(eg4);
            keng[kb] = kq(eng4);
            kep[kb] = kq(ep4);
            if constexpr (GW == 4)
                facv[kb] = lr == 0 ? lr4 : sp4;
            else if (lr < 3)
                *reinterpret_cast<f32x4_t*>(&lds_fac[w][lr][16 * kb + 4 * lq]) =
                    lr == 0 ? lr4 : sp4;
        }
        if constexpr (GW == 4) {
            // (stored after the loop: a store under a lane condition inside
            // it splits the four column blocks' chains into separate blocks;
            // the other instances keep it inside, where its registers fit)
            if (lr < 3) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    *reinterpret_cast<f32x4_t*>(
                        &lds_fac[w][lr][16 * kb + 4 * lq]) = facv[kb];
            }
        }
        // the factored form needs g_ref >= -H and g_L - g_ref >= -H
        if (__builtin_amdgcn_ballot_w64(lo < -kHalfRange * kLog2e) != 0) {
            // hand the head to the exact pass: every wave stops
            if (lane == 0) {
                lds_store(&fl.abort, 1);
                *reinterpret_cast<uint32_t*>(A.ds0 + bh * NN) = kExactPassMark;
            }
            break;
        }
        // kept for the rest of the chunk: v, dy as T layout pairs (products
        // over the value index)
        bf16x8_t Vp[2], dYp[2];
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            Vp[kp] = pk8(as_i16x4(raw[3][2 * kp]), as_i16x4(raw[3][2 * kp + 1]));
            dYp[kp] =
                pk8(as_i16x4(raw[6][2 * kp]), as_i16x4(raw[6][2 * kp + 1]));
        }

        // ---- the 16 x 16 matrices (K = 64) ---------------------------------
        f32x4_t mA = zero4(), mAT = zero4(), mAak = zero4(), mAakT = zero4(),
                mArb = zero4(), mArbT = zero4(), mArk = zero4();
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            const bf16x8_t a8 = pk8(tA[2 * kp], tA[2 * kp + 1]);
            const bf16x8_t b8 = pk8(tB[2 * kp], tB[2 * kp + 1]);
            const bf16x8_t k8 = pk8(tK[2 * kp], tK[2 * kp + 1]);
            const bf16x8_t r8 = pk8(tR[2 * kp], tR[2 * kp + 1]);
            mfma(mA, a8, b8);     // Aab[t][s] = A~_t . B~_s
            mfma(mAT, b8, a8);    // Aab^T
            mfma(mAak, a8, k8);   // Aak[t][s] = A~_t . K~_s
            mfma(mAakT, k8, a8);  // Aak^T
            mfma(mArb, r8, b8);   // Arb[t][s] = R~_t . B~_s
            mfma(mArbT, b8, r8);  // Arb^T
            mfma(mArk, r8, k8);   // Ark[t][s] = R~_t . K~_s
        }
        mA = mask4(mA, lr, lq, true, true);          // s < t
        mAT = mask4(mAT, lr, lq, true, false);
        mAak = mask4(mAak, lr, lq, true, true);
        mAakT = mask4(mAakT, lr, lq, true, false);
        mArb = mask4(mArb, lr, lq, false, true);     // s <= t
        mArbT = mask4(mArbT, lr, lq, false, false);
        mArk = mask4(mArk, lr, lq, false, true);
        const i16x4_t kAakA = kq(mAakT);  // A operand: Aak
        const i16x4_t kAakB = kq(mAak);   // B operand: Aak
        const i16x4_t kArbTA = kq(mArb);  // A operand: Arb^T
        const i16x4_t kArbA = kq(mArbT);  // A operand: Arb
        const i16x4_t kArkB = kq(mArk);   // B operand: Ark

        // ---- Minv = (I - Aab)^{-1} = (I + A)(I + A^2)(I + A^4)(I + A^8) ----
        // kMinv = kq(D(Minv^T)): A operand Minv, B operand Minv^T;
        // kMinvT = kq(D(Minv)): A operand Minv^T, B operand Minv
        i16x4_t kMinv, kMinvT;
        {
            const i16x4_t pA = kq(mA), pT = kq(mAT);
            f32x4_t x2 = zero4(), t2 = zero4();
            mfma16(x2, pT, pA);  // A A
            mfma16(t2, pA, pT);  // (A A)^T
            const i16x4_t px2 = kq(x2), pt2 = kq(t2);
            f32x4_t q1, q1t;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float one = (4 * lq + e == lr) ? 1.f : 0.f;
                q1[e] = one + mA[e] + x2[e];
                q1t[e] = one + mAT[e] + t2[e];
            }
            mfma16(q1, pT, px2);   // + A A^2
            mfma16(q1t, px2, pT);  // + (A A^2)^T
            f32x4_t x4 = zero4(), t4 = zero4();
            mfma16(x4, pt2, px2);  // A^4
            mfma16(t4, px2, pt2);  // (A^4)^T
            const i16x4_t pq1t = kq(q1t), px4 = kq(x4), pt4 = kq(t4);
            f32x4_t q2 = q1, q2t = q1t, x8 = zero4();
            mfma16(q2, pq1t, px4);   // + Q1 A^4
            mfma16(q2t, px4, pq1t);  // + (Q1 A^4)^T
            mfma16(x8, pt4, px4);    // A^8
            const i16x4_t pq2t = kq(q2t), px8 = kq(x8);
            f32x4_t dM = q2, dMT = q2t;
            mfma16(dM, pq2t, px8);   // Minv = Q2 + Q2 A^8
            mfma16(dMT, px8, pq2t);  // Minv^T = Q2^T + (A^8)^T Q2^T
            kMinv = kq(dMT);
            kMinvT = kq(dM);
        }

        // The phases after the factors, as calls: the map (the chains'
        // operands), U and X (need S_0), and dX, dU, dV (need D).  At an
        // interval of two chunks the even (checkpoint) chunk forms U, X and
        // hands its successor's start-state operands to the chains first,
        // and the odd chunk, whose start state that is, forms dX, dU, dV
        // before waiting for it; otherwise the odd chunk's worker waits most
        // of a chunk for it.
        bf16x8_t Bhp0, Bhp1;
        i16x4_t kXT[4], kdUT[4];
        auto publish_map = [&]() -> bool {
            // ---- W^ = Minv A^, Q^ = R~ 2^{g_ref} + Arb W^ (J layout); map
            // (each stage for GW key blocks before the next)
#pragma unroll
            for (int jb0 = 0; jb0 < 4; jb0 += GW) {
                float erj[GW];
                f32x4_t xa[GW], xr[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    erj[g] = lds_fac[w][1][16 * (jb0 + g) + lr];
                    xa[g] = zero4();
                    xr[g] = zero4();
                    mfma16(xa[g], tA[jb0 + g], kI);  // D(A~_jb), J layout
                    mfma16(xr[g], tR[jb0 + g], kI);  // D(R~_jb)
                }
                i16x4_t jAt[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) jAt[g] = kq(xa[g]);
                f32x4_t xw[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    xw[g] = zero4();
                    mfma16(xw[g], kMinv, jAt[g]);
                }
                i16x4_t kW[GW];
                f32x4_t yq[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    // R~ as the products take it (bf16), times 2^{g_ref}
                    const f32x4_t rj = unpack_i16(kq(xr[g]));
                    f32x4_t xs = xw[g];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        xs[e] *= erj[g];
                        yq[g][e] = rj[e] * erj[g];
                    }
                    kW[g] = kq(xs);
                }
#pragma unroll
                for (int g = 0; g < GW; ++g) mfma16(yq[g], kArbA, kW[g]);
#pragma unroll
                for (int g = 0; g < GW; ++g)
                    map.QW[jb0 + g][lane] = pk8(kq(yq[g]), kW[g]);
            }
            Bhp0 = pk8(tB[0], tB[1]);
            Bhp1 = pk8(tB[2], tB[3]);
            map.Bh[0][lane] = Bhp0;
            map.Bh[1][lane] = Bhp1;
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) map.dY[ib][lane] = jdY[ib];
            lds_drain();
            // (interval of two: the chains write D into the buffer that
            // holds their step operands only after this map; every chain
            // has read them first)
            if constexpr (M == 2) {
                if (feeds && wait_for(A.wait, &fl.h_read[w], lane,
                                      [&](int x) { return x >= NCHAIN * nfeed; }) <= 0)
                    return false;
            }
            if (lane == 0) lds_store(&fl.map_ready[w], kord + 1);
            return true;
        };
        auto do_ux = [&]() -> bool {
            // ---- U = A^ S_0^T + Aak V, X = Minv U --------------------------
            if (starts) {
                // the start state: since its loads, only the next chunk's 14
                // vector loads (if any) were issued
                if constexpr (ACC) {
                    // and the 12 cotangent loads
                    if (more)
                        __builtin_amdgcn_s_waitcnt(0x4f7a);  // vmcnt(26)
                    else
                        __builtin_amdgcn_s_waitcnt(0x0f7c);  // vmcnt(12)
                } else {
                    if (more)
                        __builtin_amdgcn_s_waitcnt(0x0f7e);  // vmcnt(14)
                    else
                        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
                }
                asm volatile("" ::: "memory");
                if (lane == 0) lds_store(&fl.s_ready[w], c);
            } else if constexpr (M == 2) {
                // formed by the four chains
                if (wait_for(A.wait, &fl.s_cnt[w], lane,
                             [&](int x) { return x >= NCHAIN * nfed; }) <= 0)
                    return false;
            } else if (wait_for(A.wait, &fl.s_ready[w], lane,
                                [&](int x) { return x == c; }) <= 0) {
                return false;
            }
            // the next chunk's start state, S_L = S_0 2^{g_L} + X^T B^ +
            // V^T K^,
            // goes to the worker of chunk c + 1 (tiles of S_L^T, formed per i
            // block as X is)
            i16x4_t kBh[4], kKh[4];
            if (feeds) {
                if (wait_for(A.wait, &fl.s_free[wfeed], lane,
                             [&](int x) { return x == c + 1; }) <= 0)
                    return false;
#pragma unroll
                for (int jb = 0; jb < 4; ++jb) {
                    const float elr = lds_fac[w][0][16 * jb + lr];
                    f32x4_t bj = unpack_i16(to_j(tB[jb], kI));
                    f32x4_t kj = unpack_i16(to_j(tK[jb], kI));
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        bj[e] *= elr;
                        kj[e] *= elr;
                    }
                    kBh[jb] = kq(bj);
                    kKh[jb] = kq(kj);
                }
                if constexpr (M == 2) {
                    // the chains' shared step operands, in this worker's
                    // D buffer (free until its map is published)
                    i16x4_t* const hs = reinterpret_cast<i16x4_t*>(D);
#pragma unroll
                    for (int jb = 0; jb < 4; ++jb) {
                        hs[64 * jb + lane] = kBh[jb];
                        hs[64 * (4 + jb) + lane] = kKh[jb];
                    }
                }
            }
            const bf16x8_t Ahp0 = pk8(tAh[0], tAh[1]),
                           Ahp1 = pk8(tAh[2], tAh[3]);
            if constexpr (GW == 4) {
                // (each stage for all four value blocks before the next, as
                // for dX, dU, dV)
                f32x4_t u[4], xt[4];
#pragma unroll
                for (int ib = 0; ib < 4; ++ib) {
                    u[ib] = zero4();
                    mfma(u[ib], Ahp0, frag_rows(S, ib, 0, lane));
                    mfma(u[ib], Ahp1, frag_rows(S, ib, 1, lane));
                    mfma(u[ib], pk8(kAakA, kZero), pk8(jV[ib], jV[ib]));
                }
                i16x4_t kU[4];
#pragma unroll
                for (int ib = 0; ib < 4; ++ib) kU[ib] = kq(u[ib]);
#pragma unroll
                for (int ib = 0; ib < 4; ++ib) {
                    xt[ib] = zero4();
                    mfma16(xt[ib], kU[ib], kMinv);  // X^T = U^T Minv^T
                }
#pragma unroll
                for (int ib = 0; ib < 4; ++ib) kXT[ib] = kq(xt[ib]);
                if (M == 2 && feeds) {
                    // X and V of value block ib for chain ib, in its own
                    // rows of the S buffer of chunk c + 1's worker
                    f32x4_t xj[4];
#pragma unroll
                    for (int ib = 0; ib < 4; ++ib) {
                        xj[ib] = zero4();
                        mfma16(xj[ib], kMinv, kU[ib]);  // X = Minv U
                    }
                    i16x4_t* const hp = reinterpret_cast<i16x4_t*>(lds_S[wfeed]);
#pragma unroll
                    for (int ib = 0; ib < 4; ++ib) {
                        hp[64 * (4 * ib) + lane] = kq(xj[ib]);
                        hp[64 * (4 * ib + 1) + lane] = jV[ib];
                    }
                    lds_drain();
                    ++nfeed;
                    if (lane == 0) lds_store(&fl.h_ready[wfeed], c + 1);
                }
                return true;
            }
#pragma unroll
            for (int ib = 0; ib < 4; ++ib) {
                // Aak V as a K = 32 product with a zero half, accumulated with
                // the K = 64 products
                f32x4_t u = zero4();
                mfma(u, Ahp0, frag_rows(S, ib, 0, lane));
                mfma(u, Ahp1, frag_rows(S, ib, 1, lane));
                mfma(u, pk8(kAakA, kZero), pk8(jV[ib], jV[ib]));
                const i16x4_t kU = kq(u);  // D(U_ib): B = U, A = U^T
                f32x4_t xt = zero4();
                mfma16(xt, kU, kMinv);  // X^T = U^T Minv^T
                kXT[ib] = kq(xt);
                if (feeds && M == 2) {
                    // X and V of value block ib for chain ib, in its own
                    // rows of the S buffer of chunk c + 1's worker
                    f32x4_t xj = zero4();
                    mfma16(xj, kMinv, kU);  // X = Minv U
                    i16x4_t* const hp = reinterpret_cast<i16x4_t*>(lds_S[wfeed]);
                    hp[64 * (4 * ib) + lane] = kq(xj);
                    hp[64 * (4 * ib + 1) + lane] = jV[ib];
                } else if (feeds) {
                    f32x4_t xj = zero4();
                    mfma16(xj, kMinv, kU);  // X = Minv U
                    const i16x4_t kXJ = kq(xj);
                    bf16_t* const Sn = lds_S[wfeed];
                    // lane: S_L[16 ib + lr][16 jpb + 4 lq + e].  The block's
                    // four S_0 tiles are read before any S_L tile is
                    // written: the compiler cannot tell the two buffers
                    // apart, and read after each write the sixteen tiles
                    // would take one LDS round trip each.
                    // (The summing instance, short of registers, goes tile
                    // by tile.)
                    constexpr int GS = ACC ? 1 : 4;
#pragma unroll
                    for (int jp0 = 0; jp0 < 4; jp0 += GS) {
                        uint2 s0r[GS];
                        f32x4_t el[GS];  // 2^{g_L} per column
#pragma unroll
                        for (int g = 0; g < GS; ++g) {
                            const int jpb = jp0 + g;
                            s0r[g] =
                                sd_read4(S, 16 * ib + lr, 16 * jpb + 4 * lq);
                            el[g] = *reinterpret_cast<const f32x4_t*>(
                                &lds_fac[w][2][16 * jpb + 4 * lq]);
                        }
                        f32x4_t acc[GS];
#pragma unroll
                        for (int g = 0; g < GS; ++g) {
                            const int jpb = jp0 + g;
                            const f32x4_t s0 = unpack4(s0r[g]);
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                acc[g][e] = s0[e] * el[g][e];
                            mfma(acc[g], pk8(kBh[jpb], kKh[jpb]),
                                 pk8(kXJ, jV[ib]));
                        }
#pragma unroll
                        for (int g = 0; g < GS; ++g)
                            sd_write4(Sn, 16 * ib + lr,
                                      16 * (jp0 + g) + 4 * lq,
                                      pack4(acc[g]));
                    }
                }
            }
            if (feeds) {
                lds_drain();
                if constexpr (M == 2) {
                    ++nfeed;
                    if (lane == 0) lds_store(&fl.h_ready[wfeed], c + 1);
                } else {
                    if (lane == 0) lds_store(&fl.s_ready[wfeed], c + 1);
                }
            }

            return true;
        };
        auto do_dx = [&]() -> bool {
            // ---- D arrives: dX = B^ D^T + Arb^T dY, dU = Minv^T dX (J and T),
            // dV^T = D K^^T + dY^T Ark + dU^T Aak.  The buffer holds
            // D' = bf16(D diag(2^{g_L - g_ref})), so B^ D^T = B~ D'^T and
            // K^ D^T = K~ D'^T ---------------------------------------------
            if (wait_for(A.wait, &fl.d_cnt[w], lane,
                         [&](int x) { return x >= NCHAIN * (kord + 1); }) <= 0)
                return false;
            const bf16x8_t Khp0 = pk8(tK[0], tK[1]), Khp1 = pk8(tK[2], tK[3]);
            const __amdgpu_buffer_rsrc_t rs_dv = whole_rsrc(A.dv);
            if constexpr (ACC) {
                // the dv cotangents: the 8 dr, dk loads and the next chunk's 14
                // vector loads (if any) came after them
                if (more)
                    __builtin_amdgcn_s_waitcnt(0x4f76);  // vmcnt(22)
                else
                    __builtin_amdgcn_s_waitcnt(0x0f78);  // vmcnt(8)
                asm volatile("" ::: "memory");
            }
            // The four value blocks are independent: each stage is issued
            // for GW of them before the next, so that one block's products
            // cover another's latency (block by block, the compiler keeps
            // each block's chain of products and conversions in sequence).
            uint2 held_dv;
#pragma unroll
            for (int ib0 = 0; ib0 < 4; ib0 += GW) {
                f32x4_t dx[GW], dv[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    const int ib = ib0 + g;
                    const bf16x8_t d0 = frag_rows(D, ib, 0, lane);
                    const bf16x8_t d1 = frag_rows(D, ib, 1, lane);
                    dx[g] = zero4();
                    mfma(dx[g], Bhp0, d0);
                    mfma(dx[g], Bhp1, d1);
                    mfma(dx[g], pk8(kArbTA, kZero), pk8(jdY[ib], jdY[ib]));
                    // D K^^T (dY^T Ark + dU^T Aak follow, once dU is formed)
                    dv[g] = zero4();
                    mfma(dv[g], d0, Khp0);
                    mfma(dv[g], d1, Khp1);
                }
                i16x4_t kdX[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) kdX[g] = kq(dx[g]);
                f32x4_t du[GW], dut[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    du[g] = zero4();
                    dut[g] = zero4();
                    mfma16(du[g], kMinvT, kdX[g]);   // dU = Minv^T dX (J)
                    mfma16(dut[g], kdX[g], kMinvT);  // dU^T = dX^T Minv (T)
                }
                i16x4_t kdUJ[GW];
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    kdUT[ib0 + g] = kq(dut[g]);
                    kdUJ[g] = kq(du[g]);
                }
                // + dY^T Ark + dU^T Aak as one K = 32 product
#pragma unroll
                for (int g = 0; g < GW; ++g)
                    mfma(dv[g], pk8(jdY[ib0 + g], kdUJ[g]),
                         pk8(kArkB, kAakB));
#pragma unroll
                for (int g = 0; g < GW; ++g) {
                    const int ib = ib0 + g;
                    f32x4_t o = dv[g];
                    if constexpr (ACC) {
                        const f32x4_t ad = unpack4(adv[ib]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) o[e] += ad[e];
                    }
                    // lane: dV[t0 + lr][16 ib + 4 lq + e]; value blocks in
                    // pairs, 16 bytes per lane (pair_rows)
                    const uint2 pv = pack4(o);
                    if ((ib & 1) == 0)
                        held_dv = pv;
                    else
                        store16(rs_dv, row2 + 32 * (ib - 1) + pair_off(lq),
                                pair_rows(held_dv, pv));
                }
            }

            return true;
        };
        if constexpr (M == 2) {
            if (starts && !do_ux()) break;
        }
        if (!publish_map()) break;
        if (skim) {
            // the cotangent passes through this chunk; nothing else is
            // formed here.  Its D buffer and tail are not read: release them
            // at once (the chains' counts stay in step), and start the next
            // chunk's start state if it is this segment's first.
            if (lane == 0) {
                lds_store(&fl.d_done[w], kord + 1);
                lds_store(&fl.s_free[w], cn);
                if (endm) lds_store(&fl.tail_used[w], tk + 1);
            }
            if (more && cn < c_hi && cn % m == 0)
                fetch_state<M>(A, w, cn, lane);
            continue;
        }

        if constexpr (M != 2) {
            if (!do_ux()) break;
        }
        if (!do_dx()) break;
        if constexpr (M == 2) {
            if (!starts && !do_ux()) break;
        }

        // ---- cotangents of the 16 x 16 matrices (K = 64 over i) -----------
        bf16x8_t Xp[2], dUp[2];
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            Xp[kp] = pk8(kXT[2 * kp], kXT[2 * kp + 1]);
            dUp[kp] = pk8(kdUT[2 * kp], kdUT[2 * kp + 1]);
        }
        f32x4_t gArb = zero4(), gArbT = zero4(), gArk = zero4(),
                gArkT = zero4(), gAab = zero4(), gAabT = zero4(),
                gAak = zero4(), gAakT = zero4();
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            mfma(gArb, dYp[kp], Xp[kp]);    // dArb[t][s] = dY_t . X_s
            mfma(gArbT, Xp[kp], dYp[kp]);
            mfma(gArk, dYp[kp], Vp[kp]);    // dArk[t][s] = dY_t . V_s
            mfma(gArkT, Vp[kp], dYp[kp]);
            mfma(gAab, dUp[kp], Xp[kp]);    // dAab[t][s] = dU_t . X_s
            mfma(gAabT, Xp[kp], dUp[kp]);
            mfma(gAak, dUp[kp], Vp[kp]);    // dAak[t][s] = dU_t . V_s
            mfma(gAakT, Vp[kp], dUp[kp]);
        }
        const i16x4_t kgArb = kq(mask4(gArb, lr, lq, false, true));
        const i16x4_t kgArbT = kq(mask4(gArbT, lr, lq, false, false));
        const i16x4_t kgArk = kq(mask4(gArk, lr, lq, false, true));
        const i16x4_t kgArkT = kq(mask4(gArkT, lr, lq, false, false));
        const i16x4_t kgAab = kq(mask4(gAab, lr, lq, true, true));
        const i16x4_t kgAabT = kq(mask4(gAabT, lr, lq, true, false));
        const i16x4_t kgAak = kq(mask4(gAak, lr, lq, true, true));
        const i16x4_t kgAakT = kq(mask4(gAakT, lr, lq, true, false));

        // the B operands of the K = 32 products that add the 16 x 16
        // cotangents' terms to dR~, dA~, dB~, dK~
        const bf16x8_t kgR2 = pk8(kgArbT, kgArkT), kgA2 = pk8(kgAabT, kgAakT);
        const bf16x8_t kgB2 = pk8(kgAab, kgArb), kgK2 = pk8(kgAak, kgArk);

        // ---- the chains' shares of sum_i D_0 S_0 at the boundary they
        // formed it: this chunk's start (even positions, worker tw = w) or
        // its end, the start of chunk c + 1 (odd positions, tw = w - 1) ----
        const float oddf = endm ? 1.f : 0.f;
        if (wait_for(A.wait, &fl.tail_cnt[tw], lane,
                     [&](int x) { return x >= NCHAIN * (tk + 1); }) <= 0)
            break;

        // ---- per column block: dR~, dA~, dB~, dK~ and the input gradients -
        // (tiles of the transposes: lane holds token lr, columns
        // 16 jb + 4 lq + e, the T layout)
        const uint32_t goff = row2 + pair_off(lq);
        uint2 held[5];
        const __amdgpu_buffer_rsrc_t rs_dr = whole_rsrc(A.dr),
                                     rs_dw = whole_rsrc(A.dw),
                                     rs_dk = whole_rsrc(A.dk),
                                     rs_da = whole_rsrc(A.da),
                                     rs_db = whole_rsrc(A.db);
        // the products over i of column block jb, issued one block ahead
        // of their use: their latency is hidden by the previous block's
        // element-wise work
        struct Acc4 {
            f32x4_t R, A, B, K;
        };
        auto products = [&](int jb) {
            Acc4 g;
            g.R = g.A = g.B = g.K = zero4();
            const bf16x8_t s0 = frag_cols(S, jb, 0, lane);
            const bf16x8_t s1 = frag_cols(S, jb, 1, lane);
            mfma(g.R, s0, dYp[0]);  // S_0^T dY^T
            mfma(g.R, s1, dYp[1]);
            mfma(g.A, s0, dUp[0]);  // S_0^T dU^T
            mfma(g.A, s1, dUp[1]);
            const bf16x8_t d0 = frag_cols(D, jb, 0, lane);
            const bf16x8_t d1 = frag_cols(D, jb, 1, lane);
            mfma(g.B, d0, Xp[0]);   // D'^T X^T = (D^T X^T) 2^{g_L - g_ref}
            mfma(g.B, d1, Xp[1]);
            mfma(g.K, d0, Vp[0]);   // D'^T V^T
            mfma(g.K, d1, Vp[1]);
            return g;
        };
        if constexpr (ACC) {
            // the dr and dk cotangents: the next chunk's vector loads (if
            // any) and the 2 dv stores came after them
            if (more)
                __builtin_amdgcn_s_waitcnt(0x4f70);  // vmcnt(16)
            else
                __builtin_amdgcn_s_waitcnt(0x0f72);  // vmcnt(2)
            asm volatile("" ::: "memory");
        }
        Acc4 cur = products(0);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const f32x4_t er = *reinterpret_cast<const f32x4_t*>(
                &lds_fac[w][1][16 * jb + 4 * lq]);
            f32x4_t tl[NCHAIN];
#pragma unroll
            for (int ch = 0; ch < NCHAIN; ++ch)
                tl[ch] = *reinterpret_cast<const f32x4_t*>(
                    &lds_tail[tw][ch][16 * jb + 4 * lq]);
            Acc4 nxt;
            if (jb < 3) nxt = products(jb + 1);
            f32x4_t tail = zero4();
#pragma unroll
            for (int ch = 0; ch < NCHAIN; ++ch)
#pragma unroll
                for (int e = 0; e < 4; ++e) tail[e] += tl[ch][e];
            f32x4_t gR = cur.R, gA = cur.A, gB = cur.B, gK = cur.K;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                gR[e] *= er[e];
                gA[e] *= er[e];
            }
            const i16x4_t jA = to_j(tA[jb], kI), jB = to_j(tB[jb], kI);
            const i16x4_t jK = to_j(tK[jb], kI), jR = to_j(tR[jb], kI);
            const bf16x8_t jBK = pk8(jB, jK), jAR = pk8(jA, jR);
            mfma(gR, jBK, kgR2);  // + B~^T dArb^T + K~^T dArk^T
            mfma(gA, jBK, kgA2);  // + B~^T dAab^T + K~^T dAak^T
            mfma(gB, jAR, kgB2);  // + A~^T dAab + R~^T dArb
            mfma(gK, jAR, kgK2);  // + A~^T dAak + R~^T dArk

            // input gradients.  The decay gradient's terms r dr, b db, k dk,
            // a da are R~ dR~, B~ dB~, K~ dK~, A~ dA~, and
            // dlog d_t = S_t - f1_t + E_0 with S the inclusive prefix sum of
            // f1 - A~ dA~ (f1 = B~ dB~ + K~ dK~ - R~ dR~) and E_0 the
            // chunk's sum_i D_0 S_0 at its start.  The end value E_L gives
            // it through the same identity: E_0 = E_L - S_15 (the chunk-end
            // identity, dlog d_t = E_L - sum_{t' > t} (f1 - a da)_{t'} - f1_t)
            const f32x4_t fA = unpack_i16(tA[jb]), fR = unpack_i16(tR[jb]);
            const f32x4_t fB = unpack_i16(tB[jb]), fK = unpack_i16(tK[jb]);
            const f32x4_t eg = unpack_i16(keg[jb]), eng = unpack_i16(keng[jb]);
            const f32x4_t ep = unpack_i16(kep[jb]);
            f32x4_t drv, dwv, dkv, dav, dbv;
            float f1[4], sc[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                drv[e] = gR[e] * eg[e];
                dav[e] = gA[e] * ep[e];
                dbv[e] = gB[e] * eng[e];
                dkv[e] = gK[e] * eng[e];
                f1[e] = fB[e] * gB[e] + fK[e] * gK[e] - fR[e] * gR[e];
                sc[e] = f1[e] - fA[e] * gA[e];
            }
            scan16x4(sc);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // odd positions: E_0 = E_L - S_15 (the scan's last token)
                const float e0 =
                    tail[e] - oddf * pin_lanes(row_bcast<15>(sc[e]));
                dwv[e] = (sc[e] - f1[e] + e0) * lam4[jb][e];  // dlog d (-e^w)
            }
            if constexpr (ACC) {
                const f32x4_t ar = unpack4(adr[jb]), ak = unpack4(adk[jb]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    drv[e] += ar[e];
                    dkv[e] += ak[e];
                }
            }
            // column blocks in pairs, 16 bytes per lane (pair_rows)
            const uint2 pv[5] = {pack4(drv), pack4(dwv), pack4(dkv),
                                 pack4(dav), pack4(dbv)};
            if ((jb & 1) == 0) {
#pragma unroll
                for (int g = 0; g < 5; ++g) held[g] = pv[g];
            } else {
                const uint32_t o = goff + 32 * (jb - 1);
                store16(rs_dr, o, pair_rows(held[0], pv[0]));
                store16(rs_dw, o, pair_rows(held[1], pv[1]));
                store16(rs_dk, o, pair_rows(held[2], pv[2]));
                store16(rs_da, o, pair_rows(held[3], pv[3]));
                store16(rs_db, o, pair_rows(held[4], pv[4]));
            }
            if (jb < 3) cur = nxt;
        }

        // ---- release the buffers; the next chunk's start state ------------
        lds_drain();
        if (lane == 0) {
            lds_store(&fl.d_done[w], kord + 1);
            lds_store(&fl.s_free[w], cn);
            if (endm) lds_store(&fl.tail_used[w], tk + 1);
        }
        if (more && cn % m == 0) fetch_state<M>(A, w, cn, lane);
    }
}

template <int M, bool ACC>
__global__ void __launch_bounds__(BTHREADS)
wkv7_wave_bwd_kernel(BwdArgs A) {
    BwdFlags& fl = lds_flags;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nch = int((A.T + WL - 1) / WL);
    if (tid < NWORK) {
        fl.map_ready[tid] = 0;
        fl.map_taken[tid] = 0;
        fl.d_cnt[tid] = 0;
        fl.d_done[tid] = 0;
        fl.tail_cnt[tid] = 0;
        fl.tail_used[tid] = 0;
        fl.s_ready[tid] = -1;
        fl.s_free[tid] = nch - 1 - tid;
        fl.h_ready[tid] = -1;
        fl.h_read[tid] = 0;
        fl.s_cnt[tid] = 0;
    }
    if (tid == 0) {
        fl.abort = 0;
        fl.failed = 0;
    }
    __syncthreads();
    if (wv < NCHAIN)
        chain<M>(A, wv, lane);
    else
        work<M, ACC>(A, wv - NCHAIN, lane);
    // every wait is bounded, so every wave arrives here
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (lds_load(&fl.failed) != 0) poison(A, tid, BTHREADS);
}

}  // namespace

namespace {

// Cost of a chunk whose workgroup only publishes its map (the cotangent
// passes through it), relative to a chunk whose gradients it forms: the
// factors, the inverse and the map, about 7,300 of 19,600 cycles per worker.
constexpr double kPassCost = 0.4;

std::atomic<int> g_force_segments{0};
std::atomic<int> g_cu_count[64];

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = g_cu_count[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount,
                                  dev) != hipSuccess)
            return 0;
        g_cu_count[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Splits a head's nch chunks (interval m chunks) over k workgroups when the
// heads alone leave CUs idle.  Segment j owns chunks [lo[j], hi[j]) and first
// carries the cotangent through every later chunk, so the later segments
// own fewer chunks: with costs 1 (own) and kPassCost (passed through), equal
// finishing times give segment j the weight 1 - kPassCost * (the weights
// before it).  Every boundary b is an interval boundary (b % m == 0) and
// leaves an even number of chunks after it, so that the chunk-boundary
// pairs of the decay gradient's identity stay inside a segment.  Returns the
// number of segments (1 when no split satisfies that).
int plan_segments(int nch, int m, int k, int* lo, int* hi) {
    lo[0] = 0;
    hi[0] = nch;
    // (an interval of two chunks is not split: one workgroup per head puts
    // the decay gradient's boundary sums at the checkpoint chunks (tpar),
    // which a segment's first own chunk cannot follow, and every count must
    // give the same bits)
    if (k < 2 || m == 2 || (m > 1 && nch % 2 != 0)) return 1;
    if (k > kMaxSegments) k = kMaxSegments;
    for (; k >= 2; --k) {
        double wt[kMaxSegments], tot = 0, before = 0;
        for (int j = 0; j < k; ++j) {
            wt[j] = 1.0 - kPassCost * before;
            if (wt[j] < 0.15) wt[j] = 0.15;
            before += wt[j];
            tot += wt[j];
        }
        int b[kMaxSegments + 1];
        b[0] = nch;
        b[k] = 0;
        bool ok = true;
        double cum = 0;
        for (int j = 1; j < k && ok; ++j) {
            cum += wt[j - 1];
            const double target = nch * (1.0 - cum / tot);
            // the nearest allowed boundary: nch - 2i (m = 1) or a multiple
            // of m (m even, nch even)
            int v;
            if (m == 1) {
                const int i = int((nch - target) / 2.0 + 0.5);
                v = nch - 2 * i;
            } else {
                v = int(target / m + 0.5) * m;
            }
            const int step = m > 1 ? m : 2;
            if (v > b[j - 1] - step) v = b[j - 1] - step;
            if (v < step) ok = false;
            b[j] = v;
        }
        if (!ok) continue;
        for (int j = 0; j < k; ++j) {
            hi[j] = b[j];
            lo[j] = b[j + 1];
        }
        return k;
    }
    return 1;
}

}  // namespace

void set_backward_segments(int k) {
    g_force_segments.store(k < 0 ? 0 : k, std::memory_order_relaxed);
}

hipError_t launch_wave_backward(const WaveBwdArgs& p, hipStream_t stream) {
    if (p.L % WL != 0 || p.L / WL < 1 || p.L / WL > 4 || p.L / WL == 3)
        return hipErrorInvalidValue;
    BwdArgs A = bwd_args(p);
    if (A.BH <= 0 || A.T <= 0) return hipSuccess;
    // workgroups per head: as many as fit beside the other heads' on the
    // device's CUs (one workgroup per CU), at most kMaxSegments
    int k = g_force_segments.load(std::memory_order_relaxed);
    if (k == 0) {
        const int cus = cu_count();
        k = cus > 0 && A.BH < cus ? int(cus / A.BH) : 1;
    }
    const int nch = int((A.T + WL - 1) / WL);
    A.nseg = plan_segments(nch, p.L / WL, k, A.seg_lo, A.seg_hi);
    if (A.BH * A.nseg > int64_t(UINT32_MAX)) return hipErrorInvalidValue;
    // an interval of two chunks (never split): the boundary sums at the even
    // (checkpoint) chunks, reverse positions of parity nch - 1
    A.tpar = (p.L / WL == 2) ? ((nch - 1) & 1) : 0;
    const bool acc = A.add_dr || A.add_dk || A.add_dv;
    const dim3 grid(unsigned(A.BH * A.nseg)), block(BTHREADS);
    switch (p.L / WL) {
        case 1:
            if (acc)
                hipLaunchKernelGGL((wkv7_wave_bwd_kernel<1, true>), grid,
                                   block, 0, stream, A);
            else
                hipLaunchKernelGGL((wkv7_wave_bwd_kernel<1, false>), grid,
                                   block, 0, stream, A);
            break;
        case 2:
            if (acc)
                hipLaunchKernelGGL((wkv7_wave_bwd_kernel<2, true>), grid,
                                   block, 0, stream, A);
            else
                hipLaunchKernelGGL((wkv7_wave_bwd_kernel<2, false>), grid,
                                   block, 0, stream, A);
            break;
        default:
            if (acc)
                hipLaunchKernelGGL((wkv7_wave_bwd_kernel<4, true>), grid,
                                   block, 0, stream, A);
            else
                hipLaunchKernelGGL((wkv7_wave_bwd_kernel<4, false>), grid,
                                   block, 0, stream, A);
            break;
    }
    return hipGetLastError();
}

}  // namespace rwkv7m
