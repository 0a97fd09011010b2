/*
 * rwkv7m_wkv.h -- C ABI of the MI355X (gfx950) WKV-7 recurrence library
 * (librwkv7m_wkv.so).
 *
 * The entry points replace the three callables of the reference's FFI
 * plugin contract, WKVFFIBackend (src/rwkv7m/kernels/wkv_ffi.py:21-34),
 * as called by the dispatcher at src/rwkv7m/model/wkv.py:172-175 and
 * :215-216:
 *
 *   forward(r, w, k, v, neg_kk, kka, S0)            -> (y, S_T)
 *   forward_with_aux(r, w, k, v, neg_kk, kka, S0)   -> ((y, S_T), aux)
 *   backward(r, ..., S0, dy, dS_T, *aux)            -> (dr, dw, dk, dv,
 *                                                       dneg_kk, dkka, dS0)
 *
 * Conventions (the reference's layout contract, wkv.py:19-57):
 *   - vectors r, w, k, v, neg_kk, kka, y, dy and the six vector gradients are
 *     time-major [T][B][H][N], contiguous, all of one dtype (bf16 or fp32);
 *   - states S0, S_T, dS_T, dS0 are [B][H][N][N] fp32, row i = value index,
 *     column j = key index;
 *   - w is log(-log(decay)): the recurrence applies exp(-exp(w))
 *     (rwkv_core.py:74);
 *   - all arithmetic on the state is fp32; y and the vector gradients are
 *     rounded to the vector dtype (round to nearest even) once, at the store.
 *   - aux is one buffer of checkpoints [ceil(T/ci)+1][B][H][N][N]:
 *     entry 0 = S0, entry c = the state after token c*ci - 1, the last entry
 *     = S_T (the layout of wkv_pallas_gpu.py:83-120, :319-343).  Its element
 *     type is rwkv7m_wkv7_checkpoint_dtype(dtype, N, ci): bf16 for bf16
 *     vectors with N == 64 and ci in {16, 32, 64} (the MFMA path, which
 *     only reads them as bf16 operands), fp32 otherwise.
 *
 * Every pointer is a device pointer; every call only enqueues work on
 * `stream` (a hipStream_t, NULL = the null stream) and never synchronises.
 * Calls are stateless and reentrant.  On failure a call returns a nonzero
 * rwkv7m_status and rwkv7m_last_error() describes it (thread-local).
 * Supported head sizes N: 1, 2, 4, 8, 16, 32, 64, 128.  The MFMA chunked
 * kernels serve bf16 with N == 64; every other case runs the sequential
 * kernels, with identical results to the tolerance of the contract.
 */
#ifndef RWKV7M_WKV_H
#define RWKV7M_WKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum rwkv7m_dtype {
    RWKV7M_DTYPE_F32 = 0,
    RWKV7M_DTYPE_BF16 = 1
} rwkv7m_dtype;

typedef enum rwkv7m_status {
    RWKV7M_OK = 0,
    RWKV7M_ERR_INVALID_ARGUMENT = 1, /* bad shape, dtype, pointer or size */
    RWKV7M_ERR_UNSUPPORTED = 2,      /* valid request this build cannot run */
    RWKV7M_ERR_HIP = 3,              /* a HIP runtime call or launch failed */
    RWKV7M_ERR_DEVICE = 4            /* a kernel's bounded wait gave up */
} rwkv7m_status;

/* Version of this ABI; bumped on any incompatible change. */
int rwkv7m_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char *rwkv7m_last_error(void);

/*
 * Device status of the kernels' bounded waits.  The MFMA kernels hand data
 * between their waves through LDS and wait for each hand-over a bounded
 * number of times, so every wave always exits.  A wait that gives up does
 * not pass silently: the workgroup overwrites every output of its
 * (batch, head) -- y, S_T, checkpoints, gradients -- with NaN and raises a
 * per-device failure counter.  This call takes the current device's
 * counter in one atomic exchange with zero, ordered after the work already
 * queued on `stream`, then synchronises `stream`: RWKV7M_OK if no wait gave
 * up since the last call, RWKV7M_ERR_DEVICE (with the count in
 * rwkv7m_last_error()) otherwise.  A failure that a kernel on another
 * stream records while this call runs is kept for the next call, never lost.  No counterpart in the reference (its
 * Pallas kernels have no inter-wave hand-over); for callers that check a
 * run's health, and for the failure-path tests.
 */
int rwkv7m_device_status(void *stream);

/*
 * Poll budget of every bounded wait in later launches; 0 restores the
 * default (2^20 polls, about 70 ms at the lowest clock, orders of magnitude
 * above any real hand-over).  A hook for tests of the failure path: a budget
 * of 1 makes the waits give up without any kernel hanging or faulting.  Not
 * thread-safe against launches on other threads.  No counterpart in the
 * reference.
 */
void rwkv7m_debug_set_wait_limit(int64_t polls);

/*
 * Workgroups per (batch, head) of the MFMA backward in later launches; 0
 * restores the default.  By default a head's backward is split over as many
 * workgroups as the device's CUs leave room for beside the other heads (at
 * most 4): each takes a run of chunks and first carries the cotangent
 * through the chunks after its own, so a call with few heads (B * H well
 * below the CU count) uses the idle CUs.  The split changes no arithmetic:
 * results are bit-identical for every count.  A hook for tests; not
 * thread-safe against launches on other threads.  No counterpart in the
 * reference.
 */
void rwkv7m_debug_set_backward_segments(int workgroups_per_head);

/*
 * The same for the MFMA forward (at most 2 workgroups per head by default):
 * each writes y and the checkpoints of its run of chunks and first carries
 * the state through the chunks before them.  Bit-identical results for
 * every count.  A hook for tests; no counterpart in the reference.
 */
void rwkv7m_debug_set_forward_segments(int workgroups_per_head);

/*
 * Name of the kernel path the last successful WKV-7 call on this thread
 * launched: "wave_forward" (MFMA chunked forward), "decode" (single-token
 * kernel), "seq_forward", "wave_backward" (MFMA chunked backward, with the
 * exact sequential pass for any head outside the factored form's range),
 * "seq_backward", or "" (nothing launched).  A diagnostic for tests that
 * must prove which kernel served a request; no counterpart in the
 * reference.
 */
const char *rwkv7m_wkv7_last_path(void);

/* Number of aux checkpoints for T tokens at interval ci: ceil(T/ci) + 1. */
int64_t rwkv7m_wkv7_checkpoint_count(int64_t T, int64_t checkpoint_interval);

/* Checkpoint interval the library uses when the caller passes 0. */
int64_t rwkv7m_wkv7_default_checkpoint_interval(int dtype, int64_t N);

/* Element type (an rwkv7m_dtype) of the checkpoints forward_with_aux writes
 * and backward reads for these vectors and this interval (0 = default). */
int rwkv7m_wkv7_checkpoint_dtype(int dtype, int64_t N,
                                 int64_t checkpoint_interval);

/*
 * forward: y = WKV(r, w, k, v, neg_kk, kka; S0) and S_T.
 * Replaces WKVFFIBackend.forward (wkv_ffi.py:32; called at wkv.py:175) and
 * the reference's inference kernel (wkv_pallas_gpu.py:123-164, :378-430).
 * final_state may alias initial_state (in-place carry of the state).
 */
int rwkv7m_wkv7_forward(int dtype, int64_t T, int64_t B, int64_t H, int64_t N,
                        const void *r, const void *w, const void *k,
                        const void *v, const void *neg_kk, const void *kka,
                        const float *initial_state, void *y,
                        float *final_state, void *stream);

/*
 * forward_with_aux: as forward, and also writes the checkpoints the backward
 * needs.  Replaces WKVFFIBackend.forward_with_aux (wkv_ffi.py:33; called at
 * wkv.py:174) and the reference's fwd+aux kernel (wkv_pallas_gpu.py:66-120,
 * :303-375).  checkpoint_interval = 0 selects the library default; the
 * MFMA path serves bf16, N = 64 and an interval of 16, 32 or 64; other
 * intervals run the sequential kernels.
 * checkpoints: [rwkv7m_wkv7_checkpoint_count(T, ci)][B][H][N][N] of
 * rwkv7m_wkv7_checkpoint_dtype(dtype, N, ci).
 */
int rwkv7m_wkv7_forward_with_aux(int dtype, int64_t T, int64_t B, int64_t H,
                                 int64_t N, const void *r, const void *w,
                                 const void *k, const void *v,
                                 const void *neg_kk, const void *kka,
                                 const float *initial_state, void *y,
                                 float *final_state, void *checkpoints,
                                 int64_t checkpoint_interval, void *stream);

/*
 * backward: the seven input cotangents from (dy, dS_T) and the aux of
 * forward_with_aux (which must have used the same checkpoint_interval).
 * Replaces WKVFFIBackend.backward (wkv_ffi.py:34; called at wkv.py:216) and
 * the reference's backward kernel (wkv_pallas_gpu.py:167-282, :433-530).
 * Vector gradients are written in the vector dtype, dS0 in fp32.
 * dy may be NULL (treated as zeros) and so may ds_t.  ds0 may not share a
 * byte with ds_t (RWKV7M_ERR_INVALID_ARGUMENT): a head that needs the exact
 * sequential pass reads dS_T again after its dS0 holds the pass's mark.
 * At N = 128 the backward takes up to 128 MiB of stream-ordered device
 * memory for the row-split workgroups' partial column sums, from a pool
 * of the library's own that keeps it reserved for later calls.
 */
int rwkv7m_wkv7_backward(int dtype, int64_t T, int64_t B, int64_t H,
                         int64_t N, const void *r, const void *w,
                         const void *k, const void *v, const void *neg_kk,
                         const void *kka, const float *initial_state,
                         const void *dy, const float *ds_t,
                         const void *checkpoints,
                         int64_t checkpoint_interval, void *dr, void *dw,
                         void *dk, void *dv, void *dneg_kk, void *dkka,
                         float *ds0, void *stream);

/*
 * Batch-major variants: the same three calls, with the token vectors (r,
 * w, k, v, neg_kk, kka, y, dy and the six vector gradients) laid out
 * [B][T][H][N] instead of [T][B][H][N].  States and checkpoints keep their
 * layouts.  The reference's model keeps its activations batch-major and
 * transposes to and from the time-major WKV layout around every call
 * (src/rwkv7m/model/nnx_model.py:695-698 before, :709-711 after); these
 * entry points take the batch-major tensors as they are.  Results equal
 * those of the time-major calls on the transposed tensors.
 */
int rwkv7m_wkv7_forward_bthn(int dtype, int64_t T, int64_t B, int64_t H,
                             int64_t N, const void *r, const void *w,
                             const void *k, const void *v, const void *neg_kk,
                             const void *kka, const float *initial_state,
                             void *y, float *final_state, void *stream);

int rwkv7m_wkv7_forward_with_aux_bthn(
    int dtype, int64_t T, int64_t B, int64_t H, int64_t N, const void *r,
    const void *w, const void *k, const void *v, const void *neg_kk,
    const void *kka, const float *initial_state, void *y, float *final_state,
    void *checkpoints, int64_t checkpoint_interval, void *stream);

int rwkv7m_wkv7_backward_bthn(int dtype, int64_t T, int64_t B, int64_t H,
                              int64_t N, const void *r, const void *w,
                              const void *k, const void *v, const void *neg_kk,
                              const void *kka, const float *initial_state,
                              const void *dy, const float *ds_t,
                              const void *checkpoints,
                              int64_t checkpoint_interval, void *dr, void *dw,
                              void *dk, void *dv, void *dneg_kk, void *dkka,
                              float *ds0, void *stream);

/*
 * decode_inplace: one token (T = 1) for B*H states, with the fp32 state
 * read and overwritten in place in HBM.  The T == 1 case of forward
 * (the eager decode loop at src/rwkv7m/infer/generate.py:74-99 reaches
 * wkv.py:175 with T = 1), with the state buffer donated.
 * Vectors are [B][H][N] (the [1][B][H][N] slice), state [B][H][N][N].
 */
int rwkv7m_wkv7_decode_inplace(int dtype, int64_t B, int64_t H, int64_t N,
                               const void *r, const void *w, const void *k,
                               const void *v, const void *neg_kk,
                               const void *kka, float *state, void *y,
                               void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV7M_WKV_H */
