// Pieces of the MFMA backward (wkv7_wave_bwd.hip) that do not depend on its
// wave roles: its arguments, 32-bit buffer addressing and the failure path.
#pragma once

#include "wkv7_wave_common.h"

namespace rwkv7m {
namespace wave {

// Most workgroups one head's backward is split over (see BwdArgs::nseg).
constexpr int kMaxSegments = 4;

// Every byte offset into the vectors and the checkpoints is below 2^31
// (checked by the host): addresses are a kernel-constant base plus a 32-bit
// per-lane offset, and a lane with nothing to store or load uses the offset
// kNoLane, past every buffer's 2^31-byte range.
constexpr uint32_t kNoLane = 0x80000000u;
struct BwdArgs {
    int64_t T, BH;
    VecLayout lay;
    uint32_t ts2;  // bytes per token step of the vectors
    const bf16_t *r, *w, *k, *v, *a, *b, *dy;
    const float* ds_t;
    const bf16_t* ckpt;
    bf16_t *dr, *dw, *dk, *dv, *da, *db;
    float* ds0;
    WaitCfg wait;
    // cotangents added to dr, dk, dv (the accumulating kernel; null: zeros)
    const bf16_t *add_dr, *add_dk, *add_dv;
    // Workgroups per head and, per segment s, the chunks [seg_lo[s],
    // seg_hi[s]) whose gradients that workgroup writes (segment 0 ends the
    // sequence).  Workgroup blockIdx.x serves head blockIdx.x / nseg,
    // segment blockIdx.x % nseg.
    int nseg;
    int seg_lo[kMaxSegments], seg_hi[kMaxSegments];
    // Parity of the reverse positions whose chunks take the decay
    // gradient's boundary sum at their start (see tail_start): 0, or, for
    // an interval of two chunks in one workgroup per head, the parity that
    // puts those sums at the checkpoint chunks, whose start states are
    // loaded, not recomputed by a neighbouring worker.
    int tpar;
};

__device__ __forceinline__ int64_t head_of(const BwdArgs& A) {
    return int64_t(blockIdx.x) / A.nseg;
}
__device__ __forceinline__ int seg_of(const BwdArgs& A) {
    return int(blockIdx.x % unsigned(A.nseg));
}

__host__ inline BwdArgs bwd_args(const WaveBwdArgs& p) {
    BwdArgs A;
    A.T = p.T;
    A.BH = p.B * p.H;
    A.lay = p.lay;
    A.ts2 = uint32_t(p.lay.ts * 2);
    A.r = static_cast<const bf16_t*>(p.r);
    A.w = static_cast<const bf16_t*>(p.w);
    A.k = static_cast<const bf16_t*>(p.k);
    A.v = static_cast<const bf16_t*>(p.v);
    A.a = static_cast<const bf16_t*>(p.a);
    A.b = static_cast<const bf16_t*>(p.b);
    A.dy = static_cast<const bf16_t*>(p.dy);
    A.ds_t = p.ds_t;
    A.ckpt = static_cast<const bf16_t*>(p.ckpt);
    A.dr = static_cast<bf16_t*>(p.dr);
    A.dw = static_cast<bf16_t*>(p.dw);
    A.dk = static_cast<bf16_t*>(p.dk);
    A.dv = static_cast<bf16_t*>(p.dv);
    A.da = static_cast<bf16_t*>(p.da);
    A.db = static_cast<bf16_t*>(p.db);
    A.ds0 = p.ds0;
    A.wait = p.wait;
    A.add_dr = static_cast<const bf16_t*>(p.add_dr);
    A.add_dk = static_cast<const bf16_t*>(p.add_dk);
    A.add_dv = static_cast<const bf16_t*>(p.add_dv);
    A.nseg = 1;
    A.tpar = 0;
    for (int g = 0; g < kMaxSegments; ++g) A.seg_lo[g] = A.seg_hi[g] = 0;
    A.seg_lo[0] = 0;
    A.seg_hi[0] = int((p.T + WL - 1) / WL);
    return A;
}

__device__ __forceinline__ f32x4_t unpack_i16(const i16x4_t& x) {
    return unpack4(__builtin_bit_cast(uint2, x));
}

// A buffer resource over a whole input tensor (null p: an empty range, so
// every load returns zeros); loads at offset kNoLane return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t in_rsrc(const bf16_t* p) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(p), 0,
                                             p ? int(kNoLane) : 0,
                                             0x00020000);
}

// A buffer resource over a whole output tensor: stores at offset kNoLane
// are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t whole_rsrc(bf16_t* p) {
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, int(kNoLane), 0x00020000);
}

// 8 bytes at byte offset `off` of the buffer.
__device__ __forceinline__ uint2 load8(__amdgpu_buffer_rsrc_t rs,
                                       uint32_t off) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t x = __builtin_amdgcn_raw_buffer_load_b64(rs, int(off), 0, 0);
    return make_uint2(x[0], x[1]);
}

// The J layout tile D(X_kb) of a T layout tile of X: X_kb I, with the
// identity as the B operand (exact for bf16 values).
__device__ __forceinline__ i16x4_t to_j(const i16x4_t& t, const i16x4_t& kI) {
    f32x4_t x = zero4();
    mfma16(x, t, kI);
    return kq(x);
}

// A workgroup whose wait gave up overwrites every output it writes with NaN:
// the gradients of its segment's tokens of its head, and dS0 if its segment
// starts the sequence (all `nthreads` threads of the workgroup take part).
__device__ __forceinline__ void poison(const BwdArgs& A, int tid,
                                       int nthreads) {
    const int64_t bh = head_of(A);
    const int sg = seg_of(A);
    const int64_t hoff = A.lay.head(bh, WN);
    const int64_t t_lo = int64_t(A.seg_lo[sg]) * WL;
    int64_t t_hi = int64_t(A.seg_hi[sg]) * WL;
    if (t_hi > A.T) t_hi = A.T;
    const bf16_t nan16 = 0x7fc0;
    bf16_t* const outs[6] = {A.dr, A.dw, A.dk, A.dv, A.da, A.db};
    for (int g = 0; g < 6; ++g)
        for (int64_t e = t_lo * WN + tid; e < t_hi * WN; e += nthreads)
            outs[g][(e / WN) * A.lay.ts + hoff + e % WN] = nan16;
    if (A.seg_lo[sg] == 0)
        for (int e = tid; e < WN * WN; e += nthreads)
            A.ds0[bh * WN * WN + e] = __builtin_nanf("");
}

}  // namespace wave
}  // namespace rwkv7m
