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

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float x) {
#pragma unroll
    for (int m = G / 2; m >= 1; m >>= 1) x += __shfl_xor(x, m);
    return x;
}

// Sum over the lanes of one wave that share (lane % G), across the
// WAVE_LANES / G row groups of the wave.
template <int G, int WAVE_LANES>
__device__ __forceinline__ float cross_group_sum(float x) {
#pragma unroll
    for (int m = G; m < WAVE_LANES; m <<= 1) x += __shfl_xor(x, m);
    return x;
}

}  // namespace rwkv7m
