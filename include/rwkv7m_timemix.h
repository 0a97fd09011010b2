/*
 * rwkv7m_timemix.h -- C ABI of the fused producers and consumer of the WKV-7
 * call in the RWKV-7 time mix (part of librwkv7m_wkv.so; status codes, dtype
 * codes and rwkv7m_last_error() are those of rwkv7m_wkv.h).
 *
 * The reference computes these as plain JAX inside
 * NNXRWKV7TimeMix.__call__ (src/rwkv7m/model/nnx_model.py:592-730), fused
 * by XLA, with jax autodiff for the backward:
 *
 *   producers (nnx_model.py:630, :683-694)
 *     w      = -softplus(-w_raw) - 0.5
 *     kk     = (k*k_k) / sqrt(sum_head (k*k_k)^2 + 1e-24)
 *     k'     = k * (1 + (a - 1) * k_a)
 *     neg_kk = -kk,  kka = kk * a
 *   consumer (nnx_model.py:709-727; GroupNorm ln_x with epsilon eps, fp32
 *   statistics, variance E[y^2] - E[y]^2 clamped at 0 as flax's GroupNorm
 *   with use_fast_variance computes it)
 *     out = (GroupNorm(y) + (sum_head r * k' * r_k) * v) * g
 *
 * Conventions:
 *   - activations are [rows][H][N] contiguous (rows = token rows in any
 *     order; the model's own batch-major [B][T] needs no transpose and its
 *     outputs feed the rwkv7m_wkv7_*_bthn entry points directly), all of one
 *     dtype (bf16 or fp32);
 *   - parameters k_k, k_a, r_k, ln_scale, ln_bias and their gradients are
 *     fp32 [H*N] (r_k's [H][N] flattened);
 *   - N is 8, 16, 32, 64 or 128;
 *   - every pointer is a 16-byte aligned device pointer; arithmetic is fp32
 *     and each output is rounded to the activation dtype once;
 *   - parameter gradients are the sums over all rows, written (not
 *     accumulated), in an order that does not depend on scheduling;
 *   - calls only enqueue work on `stream` and never allocate or synchronise.
 */
#ifndef RWKV7M_TIMEMIX_H
#define RWKV7M_TIMEMIX_H

#include <stdint.h>

#include "rwkv7m_wkv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Floats of device workspace each backward call needs for `rows` token rows
 * of H heads of size N (-1 for invalid sizes).  No counterpart in the
 * reference (XLA allocates its reduction buffers itself). */
int64_t rwkv7m_timemix_workspace_floats(int64_t rows, int64_t H, int64_t N);

/*
 * Producers: (w_raw, k, a) -> (w, k_out, neg_kk, kka), the six-vector WKV
 * inputs besides r and v.  Replaces nnx_model.py:630 (w clamp) and :683-694
 * (kk normalisation, k scaling, neg_kk and kka).
 */
int rwkv7m_timemix_wkv_inputs(int dtype, int64_t rows, int64_t H, int64_t N,
                              const void *w_raw, const void *k, const void *a,
                              const float *k_k, const float *k_a, void *w,
                              void *k_out, void *neg_kk, void *kka,
                              void *stream);

/*
 * Backward of the producers: cotangents of (w, k_out, neg_kk, kka) ->
 * cotangents of (w_raw, k, a) and of the parameters k_k, k_a.  dk_out2
 * (may be NULL) is a second cotangent of k_out, added to dk_out: k' feeds
 * both the WKV call and the consumer's bonus.  The jax.vjp of the same
 * expressions (the reference's training step differentiates them with
 * jax autodiff).
 */
int rwkv7m_timemix_wkv_inputs_backward(
    int dtype, int64_t rows, int64_t H, int64_t N, const void *w_raw,
    const void *k, const void *a, const float *k_k, const float *k_a,
    const void *dw, const void *dk_out, const void *dk_out2,
    const void *dneg_kk, const void *dkka, void *dw_raw, void *dk, void *da,
    float *dk_k, float *dk_a, float *workspace, int64_t workspace_floats,
    void *stream);

/*
 * Consumer: out = (GroupNorm(y; ln_scale, ln_bias, eps) + (sum_head r*k*r_k)
 * * v) * g, where y is the WKV output and k the scaled key k'.  Replaces
 * nnx_model.py:709-727 up to the output projection.
 */
int rwkv7m_timemix_wkv_output(int dtype, int64_t rows, int64_t H, int64_t N,
                              const void *y, const void *r, const void *k,
                              const void *v, const void *g, const float *r_k,
                              const float *ln_scale, const float *ln_bias,
                              double eps, void *out, void *stream);

/*
 * Backward of the consumer: dout -> cotangents of (y, r, k, v, g) and of the
 * parameters r_k, ln_scale, ln_bias.
 */
int rwkv7m_timemix_wkv_output_backward(
    int dtype, int64_t rows, int64_t H, int64_t N, const void *y,
    const void *r, const void *k, const void *v, const void *g,
    const float *r_k, const float *ln_scale, const float *ln_bias, double eps,
    const void *dout, void *dy, void *dr, void *dk, void *dv, void *dg,
    float *dr_k, float *dln_scale, float *dln_bias, float *workspace,
    int64_t workspace_floats, void *stream);

/*
 * Backward of the consumer that allocates nothing: rwkv7m_timemix_wkv_
 * output_backward without the workspace arguments.  No counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The parameter gradients' partial rows go to a scratch array built into
 * the library, 24 MiB per device, held by each device the library runs on
 * until the process ends.  Limit: rwkv7m_timemix_workspace_floats(rows, H,
 * N) <= 3 * 1024 * 2048 floats, which holds for every H * N up to 2^21
 * channels; larger requests fail with RWKV7M_ERR_INVALID_ARGUMENT.  Every
 * call on a device shares that device's scratch: calls that overlap on one
 * device (concurrent streams, other threads) race and must be serialised by
 * the caller.  Each call writes every scratch entry it reads, so nothing
 * carries over from an earlier call.  Results are bit-identical to
 * rwkv7m_timemix_wkv_output_backward.
 */
int rwkv7m_timemix_wkv_output_backward_noalloc(
    int dtype, int64_t rows, int64_t H, int64_t N, const void *y,
    const void *r, const void *k, const void *v, const void *g,
    const float *r_k, const float *ln_scale, const float *ln_bias, double eps,
    const void *dout, void *dy, void *dr, void *dk, void *dv, void *dg,
    float *dr_k, float *dln_scale, float *dln_bias, void *stream);

/*
 * The WKV-7 backward as the time mix needs it: rwkv7m_wkv7_backward_bthn
 * (batch-major vectors, the same arguments and checks) with the consumer's
 * cotangents of r, k' and v (dr_add, dk_add, dv_add, each batch-major in
 * the vector dtype, or NULL for none) added to dr, dk and dv.  r, k' and v
 * feed both the WKV call and the consumer's bonus term, so jax autodiff
 * sums the two cotangents of each (nnx_model.py:695-727; the reference's
 * training step differentiates the time mix as a whole).  The sums are
 * formed in fp32 and rounded once, inside the backward's own stores, so no
 * separate pass re-reads the three gradients.  An added cotangent may not
 * share a byte with an output buffer (RWKV7M_ERR_INVALID_ARGUMENT, checked
 * over the buffers' byte ranges), and ds0 may not share a byte with ds_t.
 */
int rwkv7m_timemix_wkv_backward(
    int dtype, int64_t T, int64_t B, int64_t H, int64_t N, const void *r,
    const void *w, const void *k, const void *v, const void *neg_kk,
    const void *kka, const float *initial_state, const void *dy,
    const float *ds_t, const void *checkpoints, int64_t checkpoint_interval,
    const void *dr_add, const void *dk_add, const void *dv_add, void *dr,
    void *dw, void *dk, void *dv, void *dneg_kk, void *dkka, float *ds0,
    void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV7M_TIMEMIX_H */
