// Pieces shared by the chunked WKV-7 forward and backward kernels (gfx950,
// bf16 vectors, N = 64, one 8-wave workgroup per (batch, head), chunks of
// L = 16 or 32 tokens).
//
// Conventions.  Token-major arrays are [t][j] with row pitch PN.  An L x L
// matrix X is stored transposed: memory [s][t] holds X(t, s), pitch PL.
// Operand fragments come from frag_rk (rows stored [row][k]) or frag_kr
// (rows stored [k][row], transposing LDS load), so every product reads its
// operands in whichever order they are stored.
#pragma once

#include "wkv7_common.h"
#include "wkv7_mfma.h"

namespace rwkv7m {
namespace chunk {

constexpr int CN = 64;        // head size served by the chunked kernels
constexpr int PN = CN + 8;    // LDS row pitch of 64-wide rows
constexpr int NWAVES = 8;
constexpr int NTHREADS = NWAVES * 64;
// Largest log-decay span on either side of the chunk's reference point that
// the factored form represents (e^40 keeps every factor finite in bf16).
constexpr float kHalfRange = 40.f;
constexpr float kLog2e = 1.4426950408889634f;

// The chunk kernels' input vectors.  Pointers are picked by a switch over
// kernel arguments (never from an indexed array) so that the compiler keeps
// them in the global address space: flat loads would also count against the
// LDS wait counter and stall every LDS access behind in-flight HBM loads.
struct VecPtrs {
    const bf16_t *p0, *p1, *p2, *p3, *p4, *p5, *p6;
    __device__ __forceinline__ const bf16_t* get(int vec) const {
        switch (vec) {
            case 0: return p0;
            case 1: return p1;
            case 2: return p2;
            case 3: return p3;
            case 4: return p4;
            case 5: return p5;
            default: return p6;
        }
    }
};

// Fragments of a contraction over K = 16 or 32 tokens.
template <int K>
__device__ __forceinline__ bf16x8_t fkr(const bf16_t* M, int ld, int lane) {
    if constexpr (K == 16) return frag_kr16(M, ld, lane);
    else return frag_kr(M, ld, lane);
}
template <int K>
__device__ __forceinline__ bf16x8_t frk(const bf16_t* M, int ld, int lane) {
    if constexpr (K == 16) return frag_rk16(M, ld, lane);
    else return frag_rk(M, ld, lane);
}

// LDS writes of a wave made visible to the same wave's later reads.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// s_waitcnt vmcnt(0): every vector memory access of this wave has completed.
// Placed where the loads of a conditional prefetch are known to be consumed:
// the compiler's wait insertion does not correlate the prefetch's condition
// with the consumer's, and would otherwise treat the registers those loads
// wrote as still pending and wait for all outstanding loads and stores
// (a full HBM round trip) when it next reuses them.
__device__ __forceinline__ void wait_vmem() {
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt 0, expcnt 7, lgkmcnt 15
}

// Keeps a cross-lane result (DPP, ds_swizzle) where it is computed, with
// every lane active.  A cross-lane value consumed only under a condition,
// such as select(first token, v, previous lane's value), may otherwise be
// moved into a branch, where the lanes outside the branch no longer supply
// their values.
__device__ __forceinline__ float pin_lanes(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Inclusive prefix sum over groups of L consecutive lanes (L = 16 or 32).
template <int L>
__device__ __forceinline__ float scan_lanes(float x) {
#define RWKV7M_SHR(n)                                                       \
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), \
                                                    0x110 + (n), 0xF, 0xF, \
                                                    true))
    RWKV7M_SHR(1);
    RWKV7M_SHR(2);
    RWKV7M_SHR(4);
    RWKV7M_SHR(8);
#undef RWKV7M_SHR
    if constexpr (L == 32) {
        // row_bcast:15 into rows 1 and 3 (from lane 15 of rows 0 and 2)
        x += __int_as_float(__builtin_amdgcn_update_dpp(
            0, __float_as_int(x), 0x142, 0xA, 0xF, false));
    }
    return x;
}

// Inclusive suffix sum over groups of L consecutive lanes (L = 16 or 32).
template <int L>
__device__ __forceinline__ float suffix_scan_lanes(float x, int lane) {
#define RWKV7M_SHL(n)                                                       \
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), \
                                                    0x100 + (n), 0xF, 0xF, \
                                                    true))
    RWKV7M_SHL(1);
    RWKV7M_SHL(2);
    RWKV7M_SHL(4);
    RWKV7M_SHL(8);
#undef RWKV7M_SHL
    if constexpr (L == 32) {
        // rows 0 and 2 add the total of rows 1 and 3 (lane 16 of each
        // 32-lane half, by ds_swizzle in bitmask mode: lane | 16)
        const float hi = pin_lanes(__int_as_float(
            __builtin_amdgcn_ds_swizzle(__float_as_int(x), 16 << 5)));
        x += (lane & 16) ? 0.f : hi;
    }
    return x;
}

// Sum over each row of 16 lanes, in every lane of the row (DPP row_ror).
__device__ __forceinline__ float row_sum16(float x) {
#define RWKV7M_ROR(n)                                                       \
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), \
                                                    0x120 + (n), 0xF, 0xF, \
                                                    false))
    RWKV7M_ROR(8);
    RWKV7M_ROR(4);
    RWKV7M_ROR(2);
    RWKV7M_ROR(1);
#undef RWKV7M_ROR
    return x;
}

// Value of lane t + 1 of the same group of L lanes (0 for the group's last
// lane), by wave_shl:1.
template <int L>
__device__ __forceinline__ float next_token(float x, int lane) {
    const float y = pin_lanes(__int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(x), 0x130, 0xF, 0xF, true)));
    return (lane % L == L - 1) ? 0.f : y;
}

// Value of lane l - 1 (wave_shr:1; lane 0 receives 0).  Lanes at the start
// of a group of L lanes receive the previous group's last value, which
// callers replace.
__device__ __forceinline__ float prev_lane(float x) {
    return pin_lanes(__int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(x), 0x138, 0xF, 0xF, true)));
}

// ---------------------------------------------------------------------------
// Decayed factors of one chunk, computed by NW waves.  Lane = (token
// t = lane % L, CPL = L * CN / (64 * NW) columns j0 .. j0+CPL-1 with
// j0 = (CN / NW) * wave + CPL * (lane / L)).  The log-decay is kept in base
// 2 (lam = log2 d_t, g its running sum over the chunk) and the reference
// point is g_ref = g at token L/2 - 1.  Writes the token-major factors
//   A~_t = a_t 2^{g_{t-1}-g_ref}, R~_t = r_t 2^{g_t-g_ref},
//   B~_t = b_t 2^{g_ref-g_t},     K~_t = k_t 2^{g_ref-g_t},
// and per column 2^{g_L}, 2^{g_ref}, 2^{g_L-g_ref}; raises *flag when the
// factored form cannot represent the chunk.  raw: the chunk's vectors
// (r, w, k, v, neg_kk, kka, ...) as [vec][t][j]; tokens t >= n are padding.
template <int L, int NW>
struct LaneFactors {
    static constexpr int CPL = L * CN / (64 * NW);
    static_assert(CPL == 1 || CPL == 2 || CPL == 4, "columns per lane");
    int t, j0;
    float lam[CPL], eg[CPL], eng[CPL], eprev[CPL];
    float r[CPL], k[CPL], a[CPL], b[CPL];
};

template <int CPL>
__device__ __forceinline__ void load_cols(const bf16_t* p, float* dst) {
    if constexpr (CPL == 4) {
        const uint2 u = *reinterpret_cast<const uint2*>(p);
        dst[0] = __uint_as_float(u.x << 16);
        dst[1] = __uint_as_float(u.x & 0xffff0000u);
        dst[2] = __uint_as_float(u.y << 16);
        dst[3] = __uint_as_float(u.y & 0xffff0000u);
    } else if constexpr (CPL == 2) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
        dst[0] = __uint_as_float(u << 16);
        dst[1] = __uint_as_float(u & 0xffff0000u);
    } else {
        dst[0] = bf16_to_f32(*p);
    }
}

template <int CPL>
__device__ __forceinline__ void store_cols(bf16_t* p, const float* x) {
    if constexpr (CPL == 4) {
        uint2 u;
        u.x = pack_bf16x2(x[0], x[1]);
        u.y = pack_bf16x2(x[2], x[3]);
        *reinterpret_cast<uint2*>(p) = u;
    } else if constexpr (CPL == 2) {
        *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(x[0], x[1]);
    } else {
        *p = to_bf16(x[0]);
    }
}

// CPL consecutive floats (aligned to their size) in one LDS write.
template <int CPL>
__device__ __forceinline__ void store_f32(float* p, const float* x) {
    if constexpr (CPL == 4)
        *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    else if constexpr (CPL == 2)
        *reinterpret_cast<float2*>(p) = make_float2(x[0], x[1]);
    else
        *p = x[0];
}

template <int L, int NW>
__device__ __forceinline__ void chunk_factors(
    const bf16_t (*raw)[L][PN], int n, int wv, int lane, bf16_t (*At)[PN],
    bf16_t (*Rt)[PN], bf16_t (*Bt)[PN], bf16_t (*Kt)[PN], float* eL,
    float* eRef, float* eLR, int* flag, LaneFactors<L, NW>& F) {
    constexpr int CPL = LaneFactors<L, NW>::CPL;
    const int t = lane % L, grp = lane / L;
    const int j0 = (CN / NW) * wv + CPL * grp;
    F.t = t;
    F.j0 = j0;
    float wl[CPL];
    load_cols<CPL>(&raw[0][t][j0], F.r);
    load_cols<CPL>(&raw[1][t][j0], wl);
    load_cols<CPL>(&raw[2][t][j0], F.k);
    load_cols<CPL>(&raw[4][t][j0], F.a);
    load_cols<CPL>(&raw[5][t][j0], F.b);
    float g[CPL];
    const bool valid = t < n;
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
        // log2 d_t = -e^{w} log2(e); padding tokens (t >= n) decay by nothing
        const float ew = __builtin_amdgcn_exp2f(
            valid ? wl[e] * kLog2e : -__builtin_inff());
        F.lam[e] = -ew * kLog2e;
        g[e] = scan_lanes<L>(F.lam[e]);
    }
    // Four exponentials per element.  A~'s factor 2^{g_{t-1}-g_ref} is the
    // previous token's 2^{g_t-g_ref} (one lane over), except at t = 0 where
    // it is 2^{-g_ref}.  That value comes from a fourth exponential whose
    // argument depends on the token: t = 0 takes -g_ref, t = 1 and t = 2
    // take the per-column g_ref and g_L.  2^{g_L-g_ref} is 2^{g_t-g_ref} at
    // t = L - 1.
    float lo = 0.f;  // min over columns of g_ref and g_L - g_ref
    float fA[CPL], fR[CPL], fB[CPL], fK[CPL], sp[CPL];
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
        // g at tokens L/2 - 1 and L - 1 of this lane group (ds_swizzle in
        // bitmask mode within 32 lanes: (lane & and_mask) | or_mask)
        float gref, gL;
        if constexpr (L == 32) {
            gref = __int_as_float(
                __builtin_amdgcn_ds_swizzle(__float_as_int(g[e]), 15 << 5));
            gL = __int_as_float(
                __builtin_amdgcn_ds_swizzle(__float_as_int(g[e]), 31 << 5));
        } else {
            gref = __int_as_float(__builtin_amdgcn_ds_swizzle(
                __float_as_int(g[e]), 0x10 | (7 << 5)));
            gL = __int_as_float(__builtin_amdgcn_ds_swizzle(
                __float_as_int(g[e]), 0x10 | (15 << 5)));
        }
        lo = fminf(lo, fminf(gref, gL - gref));
        const float dg = g[e] - gref;
        F.eg[e] = __builtin_amdgcn_exp2f(dg);
        F.eng[e] = __builtin_amdgcn_exp2f(-dg);
        sp[e] = __builtin_amdgcn_exp2f(t == 0 ? -gref : t == 1 ? gref : gL);
        const float pe = prev_lane(F.eg[e]);  // every lane takes part
        F.eprev[e] = t == 0 ? sp[e] : pe;
        fA[e] = F.a[e] * F.eprev[e];
        fR[e] = F.r[e] * F.eg[e];
        fB[e] = F.b[e] * F.eng[e];
        fK[e] = F.k[e] * F.eng[e];
    }
    // the factored form needs g_ref >= -H and g_L - g_ref >= -H
    if (lo < -kHalfRange * kLog2e) *flag = 1;
    store_cols<CPL>(&At[t][j0], fA);
    store_cols<CPL>(&Rt[t][j0], fR);
    store_cols<CPL>(&Bt[t][j0], fB);
    store_cols<CPL>(&Kt[t][j0], fK);
    if (t == 1) store_f32<CPL>(&eRef[j0], sp);
    if (t == 2) store_f32<CPL>(&eL[j0], sp);
    if (t == L - 1) store_f32<CPL>(&eLR[j0], F.eg);
}

// ---------------------------------------------------------------------------
// The four L x L matrices (stored transposed, pitch PL = L + 8):
//   Aab = A~ B~^T, Aak = A~ K~^T (strictly lower), Arb = R~ B~^T,
//   Ark = R~ K~^T (lower with diagonal).
// Aab is consumed only by the inverse (minv_regs), which forms it in
// registers; the other three are stored by lower_tile.

// A masked lower tile (tb, sb) of X Y^T over K = 64 (X, Y token-major),
// stored transposed into dst.
template <int L>
__device__ __forceinline__ void lower_tile(const bf16_t (*X)[PN],
                                           const bf16_t (*Y)[PN],
                                           bf16_t (*dst)[L + 8], int tb,
                                           int sb, bool strict, int lane) {
    const int lr = lane & 15, lq = lane >> 4;
    f32x4_t acc = zero4();
#pragma unroll
    for (int k0 = 0; k0 < CN; k0 += 32)
        mfma(acc, frag_rk(&X[16 * tb][k0], PN, lane),
             frag_rk(&Y[16 * sb][k0], PN, lane));
    if (sb == tb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int tt = 4 * lq + e;
            const bool keep = strict ? (lr < tt) : (lr <= tt);
            acc[e] = keep ? acc[e] : 0.f;
        }
    }
    store_tile_bf16_t(acc, &dst[16 * sb][16 * tb], L + 8, lane);
}

// Lower tile number rem (of NB (NB + 1) / 2) -> (tb, sb).
__device__ __forceinline__ void lower_tile_index(int rem, int& tb, int& sb) {
    tb = rem < 1 ? 0 : 1;
    sb = rem - tb;
}

// ---------------------------------------------------------------------------
// A 16 x 16 matrix as an operand of v_mfma_f32_16x16x16_bf16, straight from
// an accumulator tile.  D(M), the accumulator layout, has lane l holding
// M[4 (l/16) + e][l % 16] (e = 0..3); the 16x16x16 operands take, in lane l,
// A[l % 16][4 (l/16) + e] and B[4 (l/16) + e][l % 16].  So kq(D(M)), the
// lane's four values as bf16, is M as the B operand and M^T as the A
// operand:
//   mfma16(acc, kq(D(N)), kq(D(M))) accumulates N^T M.
// Products then chain in registers; a transpose costs a second product.
// These products never accumulate onto a 16x16x32 result (their
// accumulators start from zero, from VALU sums or from 16x16x16 results).
__device__ __forceinline__ i16x4_t kq(const f32x4_t& d) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t u = {pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])};
    return __builtin_bit_cast(i16x4_t, u);
}

__device__ __forceinline__ void mfma16(f32x4_t& acc, const i16x4_t& a,
                                       const i16x4_t& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
}

// Minv = (I - Aab)^{-1} of a chunk on one wave, entirely in registers, from
// the token-major factors A~, B~; stored transposed into MinvT (whose blocks
// above the diagonal must hold zeros).  Per diagonal block p, A = Aab_pp is
// strictly lower (A^16 = 0) and
//   Minv_pp = (I + A)(I + A^2)(I + A^4)(I + A^8)
//           = Q2 + Q2 A^8,  Q2 = Q1 + Q1 A^4,  Q1 = I + A + A^2 + A A^2,
// each product carried together with its transpose (the A operand of a kq
// product is a transpose).  For L = 32, Minv_10 = Minv_11 (Aab_10 Minv_00).
// Every product is bf16 x bf16 with fp32 accumulation, as in the rest of
// the chunk.
template <int L>
__device__ __forceinline__ void minv_regs(const bf16_t (*At)[PN],
                                          const bf16_t (*Bt)[PN],
                                          bf16_t (*MinvT)[L + 8], int lane) {
    constexpr int NB = L / 16, PL = L + 8;
    const int lr = lane & 15, lq = lane >> 4;
    // A and A^T of each diagonal block (masked products over K = 64) and,
    // for L = 32, Aab_10^T = B~_0 A~_1^T
    f32x4_t dA[NB], dAT[NB], dA10T = zero4();
#pragma unroll
    for (int p = 0; p < NB; ++p) {
        dA[p] = zero4();
        dAT[p] = zero4();
#pragma unroll
        for (int k0 = 0; k0 < CN; k0 += 32) {
            const bf16x8_t fa = frag_rk(&At[16 * p][k0], PN, lane);
            const bf16x8_t fb = frag_rk(&Bt[16 * p][k0], PN, lane);
            mfma(dA[p], fa, fb);
            mfma(dAT[p], fb, fa);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int row = 4 * lq + e;
            dA[p][e] = row > lr ? dA[p][e] : 0.f;
            dAT[p][e] = lr > row ? dAT[p][e] : 0.f;
        }
    }
    if constexpr (NB == 2) {
#pragma unroll
        for (int k0 = 0; k0 < CN; k0 += 32)
            mfma(dA10T, frag_rk(&Bt[0][k0], PN, lane),
                 frag_rk(&At[16][k0], PN, lane));
    }
    f32x4_t dM[NB], dM1T = zero4();
#pragma unroll
    for (int p = 0; p < NB; ++p) {
        const i16x4_t pA = kq(dA[p]), pT = kq(dAT[p]);
        f32x4_t x2 = zero4(), t2 = zero4();
        mfma16(x2, pT, pA);  // A A
        mfma16(t2, pA, pT);  // A^T A^T
        const i16x4_t px2 = kq(x2), pt2 = kq(t2);
        f32x4_t q1, q1t;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float one = (4 * lq + e == lr) ? 1.f : 0.f;
            q1[e] = one + dA[p][e] + x2[e];
            q1t[e] = one + dAT[p][e] + t2[e];
        }
        mfma16(q1, pT, px2);   // + A A^2
        mfma16(q1t, px2, pT);  // + (A^2)^T A^T
        f32x4_t x4 = zero4(), t4 = zero4();
        mfma16(x4, pt2, px2);  // A^2 A^2
        mfma16(t4, px2, pt2);  // (A^2)^T (A^2)^T
        const i16x4_t pq1t = kq(q1t), px4 = kq(x4), pt4 = kq(t4);
        f32x4_t q2 = q1, q2t = q1t, x8 = zero4();
        mfma16(q2, pq1t, px4);   // + Q1 A^4
        mfma16(q2t, px4, pq1t);  // + (A^4)^T Q1^T
        mfma16(x8, pt4, px4);    // A^4 A^4
        const i16x4_t pq2t = kq(q2t), px8 = kq(x8);
        dM[p] = q2;
        mfma16(dM[p], pq2t, px8);  // + Q2 A^8
        if (NB == 2 && p == 1) {
            dM1T = q2t;
            mfma16(dM1T, px8, pq2t);  // + (A^8)^T Q2^T
        }
        store_tile_bf16_t(dM[p], &MinvT[16 * p][16 * p], PL, lane);
    }
    if constexpr (NB == 2) {
        f32x4_t z = zero4(), m10 = zero4();
        mfma16(z, kq(dA10T), kq(dM[0]));  // Aab_10 Minv_00
        mfma16(m10, kq(dM1T), kq(z));     // Minv_11 (Aab_10 Minv_00)
        store_tile_bf16_t(m10, &MinvT[0][16], PL, lane);
    }
}

// Zero the blocks above the diagonal of n L x L matrices (stored transposed:
// memory rows s, columns t, block s > block t).  Called once per kernel.
template <int L>
__device__ __forceinline__ void zero_upper(bf16_t (*const* mats)[L + 8], int n,
                                           int tid, int nth) {
    for (int e = tid; e < L * L; e += nth) {
        const int s = e / L, t = e % L;
        if ((s >> 4) > (t >> 4))
            for (int m = 0; m < n; ++m) mats[m][s][t] = 0;
    }
}

}  // namespace chunk
}  // namespace rwkv7m
