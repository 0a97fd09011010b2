// Single-token WKV-7 step for N = 64 (decode): one state read and one state
// write per (batch, head), at HBM rate.
//
// Math (reference src/rwkv7m/model/rwkv_core.py:54-86, one step):
//   d = exp(-exp(w));  sa = S a;  S' = S diag(d) + sa b^T + v k^T;  y = S' r
//
// The reference's eager decode loop (src/rwkv7m/infer/generate.py:74-99)
// calls the WKV once per token with the whole [B, H, N, N] state, so a step
// is a pass over 2 * B*H*N*N*4 bytes of state (268 MB each way at B = 256,
// H = 64) against 7 * B*H*N vector elements.  The sequential kernel's
// one-workgroup-of-1024-threads-per-head shape keeps only two heads' states
// in flight per CU; this kernel uses 256 threads per head, so eight
// workgroups (128 KB of state) are in flight per CU.
//
// Thread t of a head's workgroup owns the four float4 groups t + 256 m
// (m = 0..3) of the row-major 64 x 64 state: rows t/16 + 16 m, columns
// 4 (t % 16) .. + 3.  The 16 lanes holding one row are one DPP row, so the
// row sums S a and S' r are row_ror reductions; every state load and store
// is a fully coalesced 16-byte access.  The state may be updated in place
// (s_t == s0): each thread reads its elements before writing them.

#include "wkv7_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace {

constexpr int DN = 64;         // head size served
constexpr int DTHREADS = 256;  // threads per head

// Sum over each row of 16 lanes, in every lane of the row (DPP row_ror).
__device__ __forceinline__ float dec_row_sum16(float x) {
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

// Four consecutive vector elements as floats.
__device__ __forceinline__ void load4(const float* p, float* x) {
    const float4 u = *reinterpret_cast<const float4*>(p);
    x[0] = u.x; x[1] = u.y; x[2] = u.z; x[3] = u.w;
}
__device__ __forceinline__ void load4(const bf16_t* p, float* x) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    x[0] = __uint_as_float(u.x << 16);
    x[1] = __uint_as_float(u.x & 0xffff0000u);
    x[2] = __uint_as_float(u.y << 16);
    x[3] = __uint_as_float(u.y & 0xffff0000u);
}

template <typename VT>
__global__ void __launch_bounds__(DTHREADS)
wkv7_decode_kernel(const VT* __restrict__ r, const VT* __restrict__ w,
                   const VT* __restrict__ k, const VT* __restrict__ v,
                   const VT* __restrict__ a, const VT* __restrict__ b,
                   const float* s0, VT* __restrict__ y, float* s_t) {
    const int t = threadIdx.x;
    const int64_t bh = blockIdx.x;
    const int c0 = 4 * (t & 15);   // the thread's four columns
    const int row0 = t >> 4;       // rows row0 + 16 m
    const int64_t vbase = bh * DN;
    const int64_t sbase = bh * DN * DN;

    // the state first (its loads are the long ones), then the vectors
    float4 S[4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
        S[m] = *reinterpret_cast<const float4*>(s0 + sbase + 4 * (t + 256 * m));
    float rr[4], ww[4], kk[4], aa[4], bb[4], vv[4];
    load4(r + vbase + c0, rr);
    load4(w + vbase + c0, ww);
    load4(k + vbase + c0, kk);
    load4(a + vbase + c0, aa);
    load4(b + vbase + c0, bb);
#pragma unroll
    for (int m = 0; m < 4; ++m) vv[m] = load_f(v + vbase + row0 + 16 * m);
    float d[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) d[e] = expf(-expf(ww[e]));

#pragma unroll
    for (int m = 0; m < 4; ++m) {
        float s[4] = {S[m].x, S[m].y, S[m].z, S[m].w};
        float sa = s[0] * aa[0] + s[1] * aa[1] + s[2] * aa[2] + s[3] * aa[3];
        sa = dec_row_sum16(sa);
        float acc = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            s[e] = s[e] * d[e] + sa * bb[e] + vv[m] * kk[e];
            acc += s[e] * rr[e];
        }
        acc = dec_row_sum16(acc);
        *reinterpret_cast<float4*>(s_t + sbase + 4 * (t + 256 * m)) =
            make_float4(s[0], s[1], s[2], s[3]);
        if ((t & 15) == m) store_f(y + vbase + row0 + 16 * m, acc);
    }
}

}  // namespace

hipError_t launch_decode(const SeqFwdArgs& p, hipStream_t stream) {
    if (p.N != DN || p.T != 1 || p.ckpt) return hipErrorInvalidValue;
    const int64_t BH = p.B * p.H;
    if (BH <= 0) return hipSuccess;
    if (p.bf16)
        hipLaunchKernelGGL(wkv7_decode_kernel<bf16_t>, dim3(unsigned(BH)),
                           dim3(DTHREADS), 0, stream,
                           static_cast<const bf16_t*>(p.r),
                           static_cast<const bf16_t*>(p.w),
                           static_cast<const bf16_t*>(p.k),
                           static_cast<const bf16_t*>(p.v),
                           static_cast<const bf16_t*>(p.a),
                           static_cast<const bf16_t*>(p.b), p.s0,
                           static_cast<bf16_t*>(p.y), p.s_t);
    else
        hipLaunchKernelGGL(wkv7_decode_kernel<float>, dim3(unsigned(BH)),
                           dim3(DTHREADS), 0, stream,
                           static_cast<const float*>(p.r),
                           static_cast<const float*>(p.w),
                           static_cast<const float*>(p.k),
                           static_cast<const float*>(p.v),
                           static_cast<const float*>(p.a),
                           static_cast<const float*>(p.b), p.s0,
                           static_cast<float*>(p.y), p.s_t);
    return hipGetLastError();
}

}  // namespace rwkv7m
