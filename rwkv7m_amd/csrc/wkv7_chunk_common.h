// Pieces shared by the chunked WKV-7 forward and backward kernels (gfx950,
// bf16 vectors, N = 64, one 4-wave workgroup per (batch, head)).
#pragma once

#include "wkv7_common.h"
#include "wkv7_mfma.h"

namespace rwkv7m {
namespace chunk {

constexpr int CN = 64;          // head size served by the chunked kernels
constexpr int PN = CN + 8;      // LDS row pitch of K = N operands
constexpr int NTHREADS = 256;   // 4 waves
// Largest log-decay span on either side of the chunk's reference point that
// the factored form represents (e^40 keeps every factor finite in bf16).
constexpr float kHalfRange = 40.f;

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

// Stage NV time-major [T][BH][64] bf16 vectors of one chunk (L tokens from
// t0) into dst[NV][L][64].  Rows past the end of the sequence, and vectors
// whose pointer is null, are zeros.
template <int L, int NV>
__device__ __forceinline__ void load_rows(bf16_t (*dst)[L][CN],
                                          const VecPtrs& src, int64_t t0,
                                          int64_t T, int64_t BH, int64_t bh,
                                          int tid) {
    constexpr int ROWS = NV * L;
#pragma unroll
    for (int p = 0; p < (ROWS + 31) / 32; ++p) {
        const int row = p * 32 + (tid >> 3), seg = tid & 7;
        if (row < ROWS) {
            const int vec = row / L, t = row % L;
            const bf16_t* base = src.get(vec);
            uint4 val = make_uint4(0, 0, 0, 0);
            if (t0 + t < T && base != nullptr)
                val = *reinterpret_cast<const uint4*>(
                    base + ((t0 + t) * BH + bh) * CN + seg * 8);
            *reinterpret_cast<uint4*>(&dst[vec][t][seg * 8]) = val;
        }
    }
}

// Write n (1, 2, 4, 8 or 16) consecutive bf16 values to LDS with the widest
// aligned stores (dst must be aligned to 2 * n bytes, up to 16).
template <int n>
__device__ __forceinline__ void put_row(bf16_t* dst, const bf16_t* v) {
    if constexpr (n == 1) {
        dst[0] = v[0];
    } else if constexpr (n == 2) {
        *reinterpret_cast<uint32_t*>(dst) = uint32_t(v[0]) | (uint32_t(v[1]) << 16);
    } else if constexpr (n == 4) {
        *reinterpret_cast<uint2*>(dst) =
            make_uint2(uint32_t(v[0]) | (uint32_t(v[1]) << 16),
                       uint32_t(v[2]) | (uint32_t(v[3]) << 16));
    } else {
        static_assert(n % 8 == 0, "row length");
#pragma unroll
        for (int q = 0; q < n / 8; ++q)
            *reinterpret_cast<uint4*>(dst + 8 * q) = make_uint4(
                uint32_t(v[8 * q]) | (uint32_t(v[8 * q + 1]) << 16),
                uint32_t(v[8 * q + 2]) | (uint32_t(v[8 * q + 3]) << 16),
                uint32_t(v[8 * q + 4]) | (uint32_t(v[8 * q + 5]) << 16),
                uint32_t(v[8 * q + 6]) | (uint32_t(v[8 * q + 7]) << 16));
    }
}

// Minv = (I - Aab)^{-1} for the strictly lower-triangular L x L matrix Aab.
// Inputs: Aab (bf16, [t][s], pitch PL) and its 16x16 diagonal blocks
// transposed (AabTD, pitch 24).  Outputs Minv ([t][s]) and MinvT ([s][t]),
// bf16, pitch PL.  Z is a per-wave 16 x 24 scratch (L/16 - 1 waves use it),
// W a per-block scratch of five 16 x 24 tiles.  All NTH threads of the
// workgroup must call it; it ends with a barrier.  Waves L/16 and up, which
// have no diagonal block, run overlap() while waves 0 .. L/16-1 invert.
//
// Diagonal block p (wave p): A is nilpotent (A^16 = 0), so
//   (I - A)^{-1} = (I + A)(I + A^2)(I + A^4)(I + A^8)
// = P + P A^4 + (P + P A^4) A^8 with P = I + A + A^2 + A^3: four dependent
// MFMA steps (bf16 operands, fp32 accumulation).  Off-diagonal blocks:
// Minv[p][q] = Minv[p][p] * sum_{m=q}^{p-1} Aab[p][m] Minv[m][q], by block
// distance p - q.
template <int L, int NTH, typename Overlap>
__device__ __forceinline__ void build_minv(const bf16_t* Aab,
                                           const bf16_t (*AabTD)[16][24],
                                           bf16_t* Minv, bf16_t* MinvT,
                                           bf16_t (*Z)[16][24],
                                           bf16_t (*W)[5][16][24], int tid,
                                           Overlap overlap) {
    constexpr int PL = L + 8, NB = L / 16;
    const int wv = tid >> 6, lane = tid & 63;
    const int lr = lane & 15, lq = lane >> 4;
    if (wv < NB) {
        const int p = wv;
        const bf16_t* Ap = Aab + 16 * p * PL + 16 * p;
        const bf16_t* ApT = &AabTD[p][0][0];
        bf16_t(*Bf)[16][24] = W[p];
        // A^2
        f32x4_t a2 = zero4();
        mma_nt<16>(a2, Ap, PL, ApT, 24, lane);
        store_tile_bf16(a2, &Bf[0][0][0], 24, lane);    // A^2
        store_tile_bf16_t(a2, &Bf[1][0][0], 24, lane);  // (A^2)^T
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // A^4 and P = I + A + A^2 + A^3
        f32x4_t a4 = zero4(), pp = zero4();
        mma_nt<16>(a4, &Bf[0][0][0], 24, &Bf[1][0][0], 24, lane);
        mma_nt<16>(pp, Ap, PL, &Bf[1][0][0], 24, lane);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = 4 * lq + e;
            pp[e] += ((t == lr) ? 1.f : 0.f) + bf16_to_f32(Ap[t * PL + lr]) +
                     a2[e];
        }
        store_tile_bf16(a4, &Bf[2][0][0], 24, lane);    // A^4
        store_tile_bf16_t(a4, &Bf[3][0][0], 24, lane);  // (A^4)^T
        store_tile_bf16(pp, &Bf[4][0][0], 24, lane);    // P
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // A^8 and P2 = P + P A^4
        f32x4_t a8 = zero4();
        mma_nt<16>(a8, &Bf[2][0][0], 24, &Bf[3][0][0], 24, lane);
        mma_nt<16>(pp, &Bf[4][0][0], 24, &Bf[3][0][0], 24, lane);
        store_tile_bf16_t(a8, &Bf[0][0][0], 24, lane);  // (A^8)^T
        store_tile_bf16(pp, &Bf[1][0][0], 24, lane);    // P2
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        // Minv_pp = P2 + P2 A^8
        mma_nt<16>(pp, &Bf[1][0][0], 24, &Bf[0][0][0], 24, lane);
        store_tile_bf16(pp, Minv + 16 * p * PL + 16 * p, PL, lane);
        store_tile_bf16_t(pp, MinvT + 16 * p * PL + 16 * p, PL, lane);
    } else {
        overlap();
    }
    if (NB > 1) {
        // zero blocks: Minv above the block diagonal, MinvT below it
        for (int e = tid; e < L * L; e += NTH) {
            const int a = e / L, b = e % L;
            if ((b >> 4) > (a >> 4)) {
                Minv[a * PL + b] = 0;
                MinvT[b * PL + a] = 0;
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 1; kk < NB; ++kk) {
        const int q = wv, p = wv + kk;
        if (p < NB) {
            f32x4_t z = zero4();
            mma_nt_k<48>(z, &Aab[16 * p * PL + 16 * q], PL,
                         &MinvT[16 * q * PL + 16 * q], PL, 16 * kk, lane);
            store_tile_bf16_t(z, &Z[wv][0][0], 24, lane);
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            f32x4_t mq = zero4();
            mma_nt<16>(mq, &Minv[16 * p * PL + 16 * p], PL, &Z[wv][0][0], 24,
                       lane);
            store_tile_bf16(mq, &Minv[16 * p * PL + 16 * q], PL, lane);
            store_tile_bf16_t(mq, &MinvT[16 * q * PL + 16 * p], PL, lane);
        }
        __syncthreads();
    }
}

}  // namespace chunk
}  // namespace rwkv7m
