// MFMA tile helpers for gfx950 (CDNA4, wave64).
//
// A tile is a 16x16 fp32 accumulator held by one wave: lane l holds rows
// 4*(l/16) + e (e = 0..3) of column l%16.  Operands are bf16 matrices in LDS
// stored with the contraction index K contiguous: A as [m][k], B as [n][k]
// (so every GEMM here computes A * B^T), row pitch a multiple of 8 elements
// and rows 16-byte aligned.
//
// Lane layout (checked on gfx950 hardware):
//   v_mfma_f32_16x16x32_bf16: A lane l holds A[l%16][8*(l/16) + 0..7],
//     B lane l holds B[8*(l/16) + 0..7][l%16], D as above.
// Tile products from LDS use this instruction.  A K step of 16 is a
// 16x16x32 step whose lanes 32..63 (k = 16..31) carry zeros: accumulating a
// v_mfma_f32_16x16x16_bf16 onto the result of a 16x16x32 in the same
// registers gave nondeterministic results on gfx950 with this toolchain
// (no wait states are emitted between the two opcodes).  The 16x16x16 form
// is used only for products chained in registers whose accumulators never
// hold a 16x16x32 result (the triangular inverse).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7_common.h"

namespace rwkv7m {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t zero4() {
    f32x4_t z = {0.f, 0.f, 0.f, 0.f};
    return z;
}

// Hardware round-to-nearest-even conversion (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t to_bf16(float x) {
    return __builtin_bit_cast(bf16_t, static_cast<__bf16>(x));
}

// Two floats to a packed bf16 pair in one v_cvt_pk_bf16_f32 (round to
// nearest even); lo in the low half.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t f = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// The 4 values of a tile lane as 4 contiguous bf16 (one 8-byte store).
__device__ __forceinline__ uint2 pack4(const f32x4_t& x) {
    uint2 p;
    p.x = pack_bf16x2(x[0], x[1]);
    p.y = pack_bf16x2(x[2], x[3]);
    return p;
}

// Inverse of pack4 (bf16 -> fp32 is exact).
__device__ __forceinline__ f32x4_t unpack4(uint2 p) {
    f32x4_t x;
    x[0] = __uint_as_float(p.x << 16);
    x[1] = __uint_as_float(p.x & 0xffff0000u);
    x[2] = __uint_as_float(p.y << 16);
    x[3] = __uint_as_float(p.y & 0xffff0000u);
    return x;
}

// ---------------------------------------------------------------------------
// Operand fragments of one v_mfma_f32_16x16x32_bf16 step (32 values of the
// contraction index k, starting at the pointer's k): lane l holds operand row
// l%16 at k = 8*(l/16) + 0..7.  Two storage orders are served:
//
//   frag_rk: rows stored [row][k] (k contiguous), one 16-byte read;
//   frag_kr: rows stored [k][row] (row contiguous), two ds_read_b64_tr_b16.
//
// ds_read_b64_tr_b16 (gfx950), checked on hardware: within each 16-lane
// group, lane 4a+b receives element b of the 8 bytes addressed by lanes
// a, a+4, a+8 and a+12 (in that order).  So lane s = a + 4e of the group
// addresses row k0 + e at columns 4a..4a+3, and lane 4a+b ends up with
// column 4a+b at k0 + 0..3.
// The *16 variants cover k = 0..15 only (lanes 32..63 carry zeros).
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

__device__ __forceinline__ bf16x8_t frag_rk(const bf16_t* M, int ld,
                                            int lane) {
    return *reinterpret_cast<const bf16x8_t*>(M + (lane & 15) * ld +
                                              8 * (lane >> 4));
}

__device__ __forceinline__ bf16x8_t frag_kr(const bf16_t* M, int ld,
                                            int lane) {
    const int s = lane & 15;
    const bf16_t* p = M + (8 * (lane >> 4) + (s >> 2)) * ld + 4 * (s & 3);
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(p));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(p + 4 * ld));
    const i16x4_t v0 = lo, v1 = hi;
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    const i16x8_t v = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, v);
}

// Every lane loads (lanes 32..63 repeat the addresses of lanes 0..31) and
// the upper half is then cleared with a select: no load sits under a
// divergent branch.
__device__ __forceinline__ bf16x8_t keep_lower_half(bf16x8_t v, int lane) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    u32x4_t u = __builtin_bit_cast(u32x4_t, v);
    const bool keep = lane < 32;
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = keep ? u[e] : 0u;
    return __builtin_bit_cast(bf16x8_t, u);
}

__device__ __forceinline__ bf16x8_t frag_rk16(const bf16_t* M, int ld,
                                              int lane) {
    return keep_lower_half(frag_rk(M, ld, lane & 31), lane);
}

__device__ __forceinline__ bf16x8_t frag_kr16(const bf16_t* M, int ld,
                                              int lane) {
    return keep_lower_half(frag_kr(M, ld, lane & 31), lane);
}

__device__ __forceinline__ void mfma(f32x4_t& acc, const bf16x8_t& a,
                                     const bf16x8_t& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

// Store a tile transposed as bf16 into D[n][m] (pitch ld, a multiple of 4):
// the 4 rows a lane holds are contiguous there, one 8-byte write.
__device__ __forceinline__ void store_tile_bf16_t(const f32x4_t& acc,
                                                  bf16_t* D, int ld,
                                                  int lane) {
    const int r = lane & 15, q = lane >> 4;
    *reinterpret_cast<uint2*>(D + r * ld + 4 * q) = pack4(acc);
}

}  // namespace rwkv7m
