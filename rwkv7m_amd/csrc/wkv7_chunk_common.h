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

// Stage NV time-major [T][BH][64] bf16 vectors of one chunk (L tokens from
// t0) into dst[NV][L][64].  Rows past the end of the sequence, and vectors
// whose pointer is null, are zeros.
template <int L, int NV>
__device__ __forceinline__ void load_rows(bf16_t (*dst)[L][CN],
                                          const bf16_t* const* src,
                                          int64_t t0, int64_t T, int64_t BH,
                                          int64_t bh, int tid) {
    constexpr int ROWS = NV * L;
#pragma unroll
    for (int p = 0; p < (ROWS + 31) / 32; ++p) {
        const int row = p * 32 + (tid >> 3), seg = tid & 7;
        if (ROWS % 32 != 0 && row >= ROWS) break;
        const int vec = row / L, t = row % L;
        uint4 val = make_uint4(0, 0, 0, 0);
        if (t0 + t < T && src[vec] != nullptr)
            val = *reinterpret_cast<const uint4*>(
                src[vec] + ((t0 + t) * BH + bh) * CN + seg * 8);
        *reinterpret_cast<uint4*>(&dst[vec][t][seg * 8]) = val;
    }
}

// Minv = (I - Aab)^{-1} for the strictly lower-triangular L x L matrix Aab.
// Inputs: Aab (bf16, [t][s], pitch PL) and its 16x16 diagonal blocks in fp32
// (AabD).  Outputs Minv ([t][s]) and MinvT ([s][t]), bf16, pitch PL; Z is a
// per-wave 16 x 24 scratch.  Every thread of the workgroup must call it; it
// ends with a barrier.
//
// Diagonal blocks: forward substitution in fp32, one lane per column
// (lane = 16 * block + column, all blocks in wave 0).  Off-diagonal blocks:
// Minv[p][q] = Minv[p][p] * sum_{m=q}^{p-1} Aab[p][m] Minv[m][q], by block
// distance p - q, with bf16 MFMA.
template <int L>
__device__ __forceinline__ void build_minv(const float (*AabD)[16][17],
                                           const bf16_t* Aab, bf16_t* Minv,
                                           bf16_t* MinvT, bf16_t (*Z)[16][24],
                                           int tid) {
    constexpr int PL = L + 8, NB = L / 16;
    const int wv = tid >> 6, lane = tid & 63;
    if (wv == 0 && lane < 16 * NB) {
        const int p = lane >> 4, col = lane & 15;
        float x[16];
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            float s = (t == col) ? 1.f : 0.f;
#pragma unroll
            for (int ss = 0; ss < t; ++ss) s += AabD[p][t][ss] * x[ss];
            x[t] = s;
        }
#pragma unroll
        for (int t = 0; t < 16; ++t)
            Minv[(16 * p + t) * PL + 16 * p + col] = to_bf16(x[t]);
        uint32_t pk[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) pk[q] = pack_bf16x2(x[2 * q], x[2 * q + 1]);
        *reinterpret_cast<uint4*>(&MinvT[(16 * p + col) * PL + 16 * p]) =
            make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *reinterpret_cast<uint4*>(&MinvT[(16 * p + col) * PL + 16 * p + 8]) =
            make_uint4(pk[4], pk[5], pk[6], pk[7]);
    }
    if (NB > 1) {
        // zero blocks: Minv above the block diagonal, MinvT below it
        for (int e = tid; e < L * L; e += NTHREADS) {
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
