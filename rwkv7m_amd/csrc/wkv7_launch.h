// Internal launcher interface between the C ABI (wkv7_capi.hip) and the
// kernel translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7_common.h"

namespace rwkv7m {

struct SeqFwdArgs {
    bool bf16;
    int64_t T, B, H, N;
    VecLayout lay;  // token vectors' layout
    const void *r, *w, *k, *v, *a, *b;
    const float* s0;
    void* y;
    float* s_t;
    void* ckpt;           // nullptr: no checkpoints
    bool ckpt_bf16;       // checkpoint element type: bf16 (else fp32)
    int64_t ci;           // checkpoint interval (when ckpt != nullptr)
};

struct SeqBwdArgs {
    bool bf16;
    int64_t T, B, H, N;
    VecLayout lay;
    const void *r, *w, *k, *v, *a, *b, *dy;
    const float* ds_t;
    const void* ckpt;
    bool ckpt_bf16;
    int64_t ci;
    void *dr, *dw, *dk, *dv, *da, *db;
    float* ds0;
};

// MFMA forward: bf16 vectors, N = 64; L is the checkpoint interval.
struct ChunkFwdArgs {
    int L;
    int64_t T, B, H;
    VecLayout lay;
    const void *r, *w, *k, *v, *a, *b;
    const float* s0;
    void* y;
    float* s_t;
    void* ckpt;  // nullptr: no checkpoints; else bf16, one per chunk (every L)
};

// The forward runs in 16-token chunks (wkv7_wave_fwd.hip); L in {16, 32, 64}
// is the checkpoint interval (checkpoints every L / 16 chunks).
hipError_t launch_wave_forward(const ChunkFwdArgs& p, hipStream_t stream);

// Chunked backward: L in {16, 32}; ckpt holds a state every L tokens.
struct ChunkBwdArgs {
    int L;
    int64_t T, B, H;
    VecLayout lay;
    const void *r, *w, *k, *v, *a, *b, *dy;
    const float* ds_t;
    const void* ckpt;  // bf16, one state every L tokens
    void *dr, *dw, *dk, *dv, *da, *db;
    float* ds0;
};

hipError_t launch_chunk_backward(const ChunkBwdArgs& p, hipStream_t stream);

hipError_t launch_seq_forward(const SeqFwdArgs& p, hipStream_t stream);

// Fused time-mix producers and consumer (wkv7_timemix.hip).  Activations are
// [rows][C] of the launch dtype; parameters fp32 [C]; N in {8, ..., 128}.
struct TmInputsArgs {
    int64_t rows, C;
    const void *w_raw, *k, *a;
    const float *k_k, *k_a;
    void *w, *k_out, *neg_kk, *kka;
};

struct TmInputsBwdArgs {
    int64_t rows, C;
    const void *w_raw, *k, *a;
    const float *k_k, *k_a;
    const void *dw, *dk_out, *dk_out2, *dneg_kk, *dkka;  // dk_out2 may be 0
    void *dw_raw, *dk, *da;
    float *dk_k, *dk_a;
    float* workspace;  // timemix_workspace_floats(rows, C) floats
};

struct TmOutputArgs {
    int64_t rows, C;
    float eps;
    const void *y, *r, *k, *v, *g;
    const float *r_k, *scale, *bias;
    void* out;
};

struct TmOutputBwdArgs {
    int64_t rows, C;
    float eps;
    const void *y, *r, *k, *v, *g, *dout;
    const float *r_k, *scale, *bias;
    void *dy, *dr, *dk, *dv, *dg;
    float *dr_k, *dscale, *dbias;
    float* workspace;
};

int64_t timemix_workspace_floats(int64_t rows, int64_t C);
hipError_t launch_timemix_inputs(bool bf16, int N, const TmInputsArgs& A,
                                 hipStream_t stream);
hipError_t launch_timemix_inputs_backward(bool bf16, int N,
                                          const TmInputsBwdArgs& A,
                                          hipStream_t stream);
hipError_t launch_timemix_output(bool bf16, int N, const TmOutputArgs& A,
                                 hipStream_t stream);
hipError_t launch_timemix_output_backward(bool bf16, int N,
                                          const TmOutputBwdArgs& A,
                                          hipStream_t stream);

// One token (T = 1) for N = 64 without checkpoints; s_t may alias s0.
hipError_t launch_decode(const SeqFwdArgs& p, hipStream_t stream);
hipError_t launch_seq_backward(const SeqBwdArgs& p, hipStream_t stream);

}  // namespace rwkv7m
