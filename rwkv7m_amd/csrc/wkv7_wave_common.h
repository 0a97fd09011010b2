// Pieces shared by the wave-specialised WKV-7 kernels (wkv7_wave_fwd.hip,
// wkv7_wave_bwd.hip): bf16 vectors, N = 64, 16-token chunks, register-
// resident 16 x 16 tiles, and bounded LDS hand-overs between waves.
//
// Register layouts (lane l, r = l % 16, q = l / 16).  A 16 x 16 accumulator
// tile D(X) holds X[4q + e][r] (e = 0..3).  As operands of
// v_mfma_f32_16x16x16_bf16, the lane's four values as bf16 (kq) are X as the
// B operand and X^T as the A operand.  A token-major matrix X[t][j]
// (16 x 64) is held two ways:
//   T layout: lane holds X[r][16 kb + 4q + e] (kb = 0..3): the tiles
//             D((X^T)_kb), for products contracting over j;
//   J layout: lane holds X[4q + e][16 jb + r]: the tiles D(X_jb), for
//             products contracting over t.
// Products over K = 64 pair two T tiles (kb = 2p, 2p + 1) into one
// v_mfma_f32_16x16x32_bf16 operand: slots 0..3 hold k = 32p + 4q + e and
// slots 4..7 k = 32p + 16 + 4q + e, the same on both operands.  A 16x16x16
// product never accumulates onto a 16x16x32 result or the other way round:
// every such hand-over goes through a VALU operation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7_common.h"
#include "wkv7_launch.h"

namespace rwkv7m {
namespace wave {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// Largest log2-decay span on either side of a chunk's reference point that
// the factored form represents (2^{40 log2 e} keeps every factor finite in
// bf16).
constexpr float kHalfRange = 40.f;
constexpr float kLog2e = 1.4426950408889634f;

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

// A 16 x 16 accumulator tile as bf16 operand registers of
// v_mfma_f32_16x16x16_bf16.  D(M) holds M[4q + e][r]; the 16x16x16 operands
// take, in lane l, A[r][4q + e] and B[4q + e][r].  So kq(D(M)) is M as the B
// operand and M^T as the A operand: mfma16(acc, kq(D(N)), kq(D(M)))
// accumulates N^T M, and products chain in registers.
__device__ __forceinline__ i16x4_t kq(const f32x4_t& d) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t u = {pack_bf16x2(d[0], d[1]), pack_bf16x2(d[2], d[3])};
    return __builtin_bit_cast(i16x4_t, u);
}

__device__ __forceinline__ void mfma16(f32x4_t& acc, const i16x4_t& a,
                                       const i16x4_t& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: lane l holds A[l % 16][8 (l / 16) + 0..7] and
// B[8 (l / 16) + 0..7][l % 16] (the pairing of pk8 below is one such
// assignment of the contraction index).
__device__ __forceinline__ void mfma(f32x4_t& acc, const bf16x8_t& a,
                                     const bf16x8_t& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

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

// LDS writes of a wave made visible to the same wave's later reads.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
}

// Keeps a cross-lane result (DPP, ds_swizzle) where it is computed, with
// every lane active.  A cross-lane value consumed only under a condition may
// otherwise be moved into a branch, where the lanes outside the branch no
// longer supply their values.
__device__ __forceinline__ float pin_lanes(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Inclusive prefix sum over each row of 16 lanes (DPP row_shr).
__device__ __forceinline__ float scan16(float x) {
#define RWKV7M_SHR(n)                                                       \
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), \
                                                    0x110 + (n), 0xF, 0xF, \
                                                    true))
    RWKV7M_SHR(1);
    RWKV7M_SHR(2);
    RWKV7M_SHR(4);
    RWKV7M_SHR(8);
#undef RWKV7M_SHR
    return x;
}

// scan16 of four independent values in lock step: each DPP step is issued
// for all four before the next, so the steps' read-after-write distance is
// covered by the other values' instructions instead of wait states.
__device__ __forceinline__ void scan16x4(float (&x)[4]) {
#define RWKV7M_SHR4(n)                                                      \
    for (int e = 0; e < 4; ++e)                                             \
        x[e] += __int_as_float(__builtin_amdgcn_update_dpp(                 \
            0, __float_as_int(x[e]), 0x110 + (n), 0xF, 0xF, true))
    RWKV7M_SHR4(1);
    RWKV7M_SHR4(2);
    RWKV7M_SHR4(4);
    RWKV7M_SHR4(8);
#undef RWKV7M_SHR4
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

constexpr int WN = 64;          // head size
constexpr int WL = 16;          // tokens per chunk
constexpr int XPITCH = WN + 8;  // bf16 transpose buffer row pitch

typedef short i16x8_t __attribute__((ext_vector_type(8)));

__device__ __forceinline__ bf16x8_t pk8(const i16x4_t& lo, const i16x4_t& hi) {
    const i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8_t, v);
}

__device__ __forceinline__ i16x4_t as_i16x4(uint2 u) {
    return __builtin_bit_cast(i16x4_t, u);
}

// Value of lane n of each 16-lane row, in every lane of the row (every
// lane reads a valid source, so no old value is needed).
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x),
                                                   0x150 + N, 0xF, 0xF, true));
}

// The previous lane's value within each row; the row's first lane keeps
// `first`.
__device__ __forceinline__ float row_prev(float x, float first) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        __float_as_int(first), __float_as_int(x), 0x111, 0xF, 0xF, false));
}

// X[4q + e][16 jb + r] (e = 0..3) of a [t][j] matrix in LDS (the J layout)
// by one transposing read: lane s of each 16-lane group addresses row
// 4q + s / 4, columns 16 jb + 4 (s % 4) .. + 3.
__device__ __forceinline__ i16x4_t read_j(const bf16_t (*X)[XPITCH], int jb,
                                          int lane) {
    const int s = lane & 15, q = lane >> 4;
    const bf16_t* p = &X[4 * q + (s >> 2)][16 * jb + 4 * (s & 3)];
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
}

// Keep X[4q + e][r] where (row_below: r < 4q + e; else 4q + e < r), with
// equality kept unless strict.
__device__ __forceinline__ f32x4_t mask4(f32x4_t x, int r, int q, bool strict,
                                         bool row_below) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int m = 4 * q + e;
        const bool keep = row_below ? (strict ? r < m : r <= m)
                                    : (strict ? m < r : m <= r);
        x[e] = keep ? x[e] : 0.f;
    }
    return x;
}

// Element (i, j) of a 64 x 64 bf16 S/D buffer: 16-byte unit (i, j / 8) at
// ((i / 8) * 8 + j / 8) * 8 + i % 8, so one global_load_lds of 64 lanes
// (16 bytes each, at consecutive units) fills rows 8g .. 8g + 7.
__device__ __forceinline__ int sd_off(int i, int j) {
    return ((((i >> 3) << 3) + (j >> 3)) * 8 + (i & 7)) * 8 + (j & 7);
}

__device__ __forceinline__ uint2 sd_read4(const bf16_t* buf, int i, int j) {
    return *reinterpret_cast<const uint2*>(buf + sd_off(i, j));
}

__device__ __forceinline__ void sd_write4(bf16_t* buf, int i, int j, uint2 v) {
    *reinterpret_cast<uint2*>(buf + sd_off(i, j)) = v;
}

// x32 fragment of rows 16 rb .. 16 rb + 15 over the 32 columns of pair p:
// lane (q, r) takes row 16 rb + r, columns 32p + 4q .. + 3 (slots 0..3) and
// 32p + 16 + 4q .. + 3 (slots 4..7).  As an A operand: the rows (m = i,
// k = j); as a B operand: their transpose (k = j, n = i).
__device__ __forceinline__ bf16x8_t frag_rows(const bf16_t* buf, int rb,
                                              int p, int lane) {
    const int r = lane & 15, q = lane >> 4;
    const int i = 16 * rb + r, j = 32 * p + 4 * q;
    return pk8(as_i16x4(sd_read4(buf, i, j)),
               as_i16x4(sd_read4(buf, i, j + 16)));
}

// x32 fragment of columns 16 cb .. 16 cb + 15 over the 32 rows of pair p,
// by two transposing reads: lane (q, r) takes column 16 cb + r at rows
// 32p + 4q + e (slots 0..3) and 32p + 16 + 4q + e (slots 4..7).  Lane
// s = a + 4e of each 16-lane group addresses row 32p + 4q + e, columns
// 16 cb + 4a .. + 3.  As an A operand: the transpose (m = j, k = i); as a B
// operand: the matrix (k = i, n = j).
__device__ __forceinline__ bf16x8_t frag_cols(const bf16_t* buf, int cb,
                                              int p, int lane) {
    const int s = lane & 15, q = lane >> 4;
    const int i = 32 * p + 4 * q + (s >> 2), j = 16 * cb + 4 * (s & 3);
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(buf + sd_off(i, j)));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_i16x4_t*)(buf + sd_off(i + 16, j)));
    return pk8(lo, hi);
}

// LDS DMA (global_load_lds_dwordx4): lane l's 16 bytes at gbase + voff (a
// byte offset) land at LDS byte address lds + 16 l; gbase and lds are
// wave-uniform.  Written as inline assembly so that the compiler does not
// treat every later LDS access as a possible reader of the DMA's data (it
// would wait for all outstanding vector memory operations, this load's and
// every earlier store's, before each one): the caller orders the data's
// use with explicit vmcnt waits.  M0 is set in the same statement; no other
// code of these kernels uses it.  `lds` is wave-uniform; the readfirstlane
// only tells the compiler so where its uniformity analysis cannot see it
// (after a loop with an early exit) and costs nothing otherwise.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* gbase, uint32_t voff,
                                      uint32_t lds) {
    asm volatile(
        "s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(gbase), "s"(__builtin_amdgcn_readfirstlane(lds))
        : "memory", "m0");
}
#pragma clang diagnostic pop

// A raw buffer resource over `bytes` bytes at `base`: stores through it at
// byte offsets at or past `bytes` are dropped by the hardware, so masked
// lanes need no branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t out_rsrc(void* base,
                                                         uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(base, 0, int(bytes), 0x00020000);
}

// 8 bytes at byte offset `off` of the buffer.
__device__ __forceinline__ void store8(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                       uint2 v) {
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t x = {v.x, v.y};
    __builtin_amdgcn_raw_buffer_store_b64(x, rs, int(off), 0, 0);
}

// 16 bytes at byte offset `off` of the buffer.
__device__ __forceinline__ void store16(__amdgpu_buffer_rsrc_t rs,
                                        uint32_t off, uint4 v) {
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t x = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(x, rs, int(off), 0, 0);
}

// Two 16-column blocks of a token-major tile as 16-byte pieces.  Lane (q, r)
// holds 8 bytes of block p (columns 16 p + 4 q .. + 3) in `a` and of block
// p + 1 in `b`.  v_permlane16_swap exchanges the odd 16-lane rows of its
// first operand with the even rows of its second, so after one swap per
// dword an even-row lane holds columns 16 p + 4 q .. + 7 (its own and its
// odd neighbour's `a`) and an odd-row lane columns 16 (p + 1) + 4 (q - 1)
// .. + 7 (its even neighbour's `b` and its own): every lane then stores 16
// contiguous bytes, at byte 32 p + pair_off(q) of the token's row, instead
// of two 8-byte pieces (a half-line write per instruction and lane, which
// the memory path serves at about two thirds of the rate of 16-byte ones).
__device__ __forceinline__ uint4 pair_rows(uint2 a, uint2 b) {
    const auto lo = __builtin_amdgcn_permlane16_swap(a.x, b.x, false, false);
    const auto hi = __builtin_amdgcn_permlane16_swap(a.y, b.y, false, false);
    return make_uint4(lo[0], hi[0], lo[1], hi[1]);
}
__device__ __forceinline__ uint32_t pair_off(int q) {
    return uint32_t(8 * q + ((q & 1) ? 24 : 0));
}

// The LDS byte address of a __shared__ object.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// Hand-over words in LDS are read and written as relaxed workgroup-scope
// atomics: a volatile access would also make the wave wait for all its
// outstanding global stores.  Ordering against the data they guard comes
// from an explicit lgkmcnt(0) before each write and from the polling
// reads' own completion before the guarded reads are issued.
__device__ __forceinline__ int lds_load(int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_store(int* p, int x) {
    __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_add(int* p, int x) {
    __hip_atomic_fetch_add(p, x, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
}

// s_waitcnt lgkmcnt(0): this wave's LDS accesses have completed (issued
// before a hand-over word is written).
__device__ __forceinline__ void lds_drain() {
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("" ::: "memory");
}

// Poll an LDS word until pred(value) holds: 1 when it does, 0 when the word
// *stop turned nonzero first (read on every eighth poll: another wave of
// the workgroup gave up), -1 after `limit` polls.
template <typename Pred>
__device__ __forceinline__ int poll_or_stop(int* p, int limit, int* stop,
                                            Pred pred) {
    for (int it = 0; it < limit; ++it) {
        if (pred(__builtin_amdgcn_readfirstlane(lds_load(p)))) {
            asm volatile("" ::: "memory");
            return 1;
        }
        if ((it & 7) == 7 &&
            __builtin_amdgcn_readfirstlane(lds_load(stop)) != 0) {
            asm volatile("" ::: "memory");
            return 0;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    asm volatile("" ::: "memory");
    return -1;
}

// A wait gave up: mark the workgroup failed (LDS) and count it on the device
// (a per-lane global atomic from lane 0).
__device__ __forceinline__ void wait_failed(int* failed, unsigned int* counter,
                                            int lane) {
    if (lane == 0) {
        lds_store(failed, 1);
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace wave
}  // namespace rwkv7m
