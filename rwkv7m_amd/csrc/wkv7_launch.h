// Internal launcher interface between the C ABI (wkv7_capi.hip) and the
// kernel translation units.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wkv7_common.h"

namespace rwkv7m {

// Bounded waits (wkv7_status.hip): the poll budget of one hand-over and this
// device's failure counter.
constexpr int kDefaultWaitPolls = 1 << 20;
struct WaitCfg {
    int limit;                // polls per wait before it gives up
    unsigned int* failures;   // device address of the failure counter
};
// The current device's configuration (looks the counter up once per device).
hipError_t wait_config(WaitCfg* out);
// Poll budget for later launches (0: the default); a hook for tests of the
// failure path.
void set_wait_limit(int64_t polls);
// Exchanges the current device's count for zero (atomically, after the
// stream's queued work), synchronises the stream and returns what was taken.
hipError_t take_wait_failures(hipStream_t stream, unsigned int* count);

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
    // only the heads whose ds0[b][h][0][0] holds kExactPassMark (left by the
    // wave backward to this exact pass); others are untouched
    bool marked_only;
    // nullptr, or cotangents (vector layout and dtype) added to dr, dk, dv
    // in fp32 before they are rounded and stored
    const void *add_dr, *add_dk, *add_dv;
};

// Bit pattern (a NaN no arithmetic produces) that the wave backward leaves in
// dS0[b][h][0][0] of a head it hands to the exact sequential pass.
constexpr uint32_t kExactPassMark = 0x7fa5a5a5u;

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
    WaitCfg wait;
};

// The forward runs in 16-token chunks (wkv7_wave_fwd.hip); L in {16, 32, 64}
// is the checkpoint interval (checkpoints every L / 16 chunks).
hipError_t launch_wave_forward(const ChunkFwdArgs& p, hipStream_t stream);
// Workgroups per head for later wave forward launches (0: as many as the
// device's idle CUs allow, at most 2).  A hook for tests.
void set_forward_segments(int k);

// Wave-specialised backward (wkv7_wave_bwd.hip): 16-token chunks, bf16
// checkpoints every L in {16, 32, 64} tokens.  A head with a chunk outside
// the factored form's range is left with kExactPassMark in dS0[b][h][0][0]
// for the exact pass (launch_seq_backward with marked_only).
struct WaveBwdArgs {
    int L;
    int64_t T, B, H;
    VecLayout lay;
    const void *r, *w, *k, *v, *a, *b, *dy;
    const float* ds_t;
    const void* ckpt;
    void *dr, *dw, *dk, *dv, *da, *db;
    float* ds0;
    WaitCfg wait;
    // nullptr, or bf16 cotangents added to dr, dk, dv (as SeqBwdArgs); any
    // non-null one selects the accumulating kernel, which takes all three
    // (a null one reads as zeros)
    const void *add_dr, *add_dk, *add_dv;
};

hipError_t launch_wave_backward(const WaveBwdArgs& p, hipStream_t stream);
// Workgroups per head for later wave backward launches (0: as many as the
// device's idle CUs allow, at most 4).  A hook for tests.
void set_backward_segments(int k);

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

// State-level screening read path (screen_kernels.hip).  Slot recurrence:
// base [B][T][ds] and slots_seq / d_slots_seq [B][T][M][ds] of the launch
// dtype; everything else fp32.
struct ScreenScanArgs {
    int64_t B, T, M, ds;
    const void* base;
    const float *slot_term, *mu, *slots0;  // [M][ds], [M], [B][M][ds]
    void* slots_seq;                        // S_t, the slots step t reads
    float *slots_T, *upd2;                  // [B][M][ds], [B][T][M][ds/64]
    const void* d_slots_seq;                // backward inputs
    const float* d_slots_T;                 // may be 0
    float *d_pre, *d_slots0, *d_mu_part;    // [B][T][M][ds], [B][M][ds] x2
    float* workspace;  // screen_scan_workspace_floats(B, T, M, ds) floats
};

int64_t screen_scan_workspace_floats(int64_t B, int64_t T, int64_t M,
                                     int64_t ds);

// Per-token read: q fp32 [B][T][dk]; proj [B][T][M][dk + dv] (keys then
// values, launch dtype); u / du [B][T][dv] (launch dtype).
struct ScreenReadArgs {
    int64_t B, T;
    int M, dk, dv;
    const float* q;
    const void* proj;
    const float* tau;  // one fp32 on the device
    float trim_eps;
    const float* age_w;  // [B][M] or [B][T][M] (see the strides) or 0
    int64_t age_bstride, age_tstride;  // M, 0 or T * M, M
    int value_unit_norm, leaky;
    float leaky_alpha, leaky_gamma, cap, eps;
    void* u;
    float *rel, *z_norm, *u_norm;  // [B][T][M], [B][T], [B][T]
    const void* du;                // backward inputs
    const float* d_rel;            // [B][T][M] or 0
    float* dq;
    void* d_proj;
    float *d_tau, *g_age;  // [B][T], [B][T][M]
};

// Write phase (read_write): one workgroup per (b, m) walks the steps.
struct ScreenWriteArgs {
    int64_t B, T, M, ds;
    int dk;
    const void* base;                           // [B][T][ds]
    const float *slot_term, *slot_embed, *kw;  // [M][ds] x2, [ds][dk]
    const float *q_w, *tau_w, *mu;             // [B][T][dk], 1, [M]
    float floor, eps;
    const float *slots0, *ages0;               // [B][M][ds], [B][M]
    void* slots_seq;                           // S_t rounded, [B][T][M][ds]
    float *slots32, *ages_seq, *rel_w, *upd2;  // S_t fp32, [B][T][M] x2, ..
    float *slots_T, *ages_T;
    const void* d_slots_seq;                   // backward inputs
    const float *d_slots_T, *d_rel_w, *d_ages_seq, *d_ages_T;  // may be 0
    float *d_pre, *d_slots0, *d_ages0, *d_embed_part, *d_mu_bm;
    float *d_kraw, *dq_w, *d_tau_w;            // [B][T][M][dk] x2, [B][T][M]
};

hipError_t launch_screen_write(bool bf16, bool backward,
                               const ScreenWriteArgs& A, hipStream_t stream);

hipError_t launch_screen_scan(bool bf16, bool backward,
                              const ScreenScanArgs& A, hipStream_t stream);
hipError_t launch_screen_read(bool bf16, bool backward,
                              const ScreenReadArgs& A, hipStream_t stream);

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
