// Shared device helpers for the gfx950 WKV-7 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rwkv7m {

using bf16_t = uint16_t;  // bfloat16 bit pattern

__device__ __forceinline__ float bf16_to_f32(bf16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN maps to the canonical quiet NaN 0x7FC0.
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
}

__device__ __forceinline__ float load_f(const float* p) { return *p; }
__device__ __forceinline__ float load_f(const bf16_t* p) {
    return bf16_to_f32(*p);
}
__device__ __forceinline__ void store_f(float* p, float x) { *p = x; }
__device__ __forceinline__ void store_f(bf16_t* p, float x) {
    *p = f32_to_bf16(x);
}

// Element layout of the token vectors [T, B, H, N] or [B, T, H, N]: element
// (t, b, h, j) sits at t * ts + b * bs + h * N + j.  Time-major (the
// reference's layout): ts = B*H*N, bs = H*N.  Batch-major: ts = H*N,
// bs = T*H*N.  States are [B][H][N][N] in both.
struct VecLayout {
    int64_t ts, bs, H;
    __device__ __forceinline__ int64_t head(int64_t bh, int64_t N) const {
        return (bh / H) * bs + (bh % H) * N;
    }
};

// x plus the x of lane l ^ M.  Within a row of 16 lanes (M < 16) a DPP
// row rotation by M gives the partner, or one whose value equals it after
// the larger steps of a butterfly over the row (sums over lanes l ^ 8, then
// l ^ 4, ...); across rows, the two halves of a permlane swap of x with
// itself are x and its partner.  Each lane adds the same two values as with
// a shuffle, so the sums are bit-identical to a shuffle butterfly in the same
// order.  No LDS traffic, unlike the shuffle's ds_bpermute.
template <int M>
__device__ __forceinline__ float add_ror(float x) {
    const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + M,
                                              0xf, 0xf, false);
    return x + __int_as_float(y);
}
template <int M>
__device__ __forceinline__ float add_swap(float x) {
    const unsigned u = __float_as_uint(x);
    if constexpr (M == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __uint_as_float(p[0]) + __uint_as_float(p[1]);
    } else {
        const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
}

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64),
// butterfly steps l ^ G/2, ..., l ^ 1.
template <int G>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (G == 16) {
        return add_ror<1>(add_ror<2>(add_ror<4>(add_ror<8>(x))));
    } else {
#pragma unroll
        for (int m = G / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m);
        return x;
    }
}

// Sum over the lanes of one wave that share (lane % G), across the
// WAVE_LANES / G row groups of the wave (steps l ^ G, l ^ 2G, ...).
template <int G, int WAVE_LANES>
__device__ __forceinline__ float cross_group_sum(float x) {
    if constexpr (WAVE_LANES == 64 && (G == 16 || G == 8)) {
        if constexpr (G == 8) x = add_ror<8>(x);
        return add_swap<32>(add_swap<16>(x));
    } else {
#pragma unroll
        for (int m = G; m < WAVE_LANES; m <<= 1) x += __shfl_xor(x, m);
        return x;
    }
}

}  // namespace rwkv7m
