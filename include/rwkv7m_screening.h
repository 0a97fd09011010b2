/*
 * rwkv7m_screening.h -- C ABI of the state-level screening module (phases
 * read_screening_only and read_write) in librwkv7m_wkv.so; status codes,
 * dtype codes and rwkv7m_last_error() are those of rwkv7m_wkv.h.
 *
 * The reference runs NNXStateLevelScreening.__call__
 * (src/rwkv7m/model/nnx_model.py:999-1160) as one jax.lax.scan step per
 * token, each step projecting all slots.  With writes disabled the slot
 * update does not depend on the read, so the call splits into:
 *   1. projections of the whole sequence (library GEMMs, the caller's);
 *   2. rwkv7m_screen_slot_scan: the slots every step reads,
 *        delta_t[m] = tanh(base_t + slot_term[m])         (rounded to dtype)
 *        S_{t+1}[m] = S_t[m] + mu[m] (delta_t[m] - S_t[m])
 *      (compute_slot_delta, screening.py:61-88, and nnx_model.py:1098-1102);
 *   3. the keys and values of those slots (one GEMM, the caller's);
 *   4. rwkv7m_screen_read: per token, unit-normalised keys (and values),
 *      sim = q . k, relevance trim_square(sim, tau) (or the leaky blend)
 *      times the age weight, z = sum_m rel_m v_m, u = tanh_norm(z, cap)
 *      (nnx_model.py:1063-1086, screening.py:21-52).
 * The backward entry points are the adjoints of 2 and 4.
 *
 * Layouts (row-major, contiguous): base [B][T][ds]; slots_seq and its
 * cotangent [B][T][M][ds], both of `dtype`; slot_term [M][ds], mu [M],
 * slots0 / slots_T / their cotangents [B][M][ds], fp32.  q [B][T][dk] fp32;
 * proj [B][T][M][dk + dv] (keys then values) and u [B][T][dv] of `dtype`;
 * rel [B][T][M], z_norm and u_norm [B][T], age_w [B][M] fp32.
 * Limits: M <= 64, dk <= 128, dv <= 512.  Calls only enqueue work on
 * `stream`, never allocate, never synchronise.  The slot scan runs in
 * chunks of 32 steps (each chunk's contribution from a zero start, a serial
 * pass over the chunk ends, then every chunk from its true start), with a
 * caller-provided fp32 workspace.
 */
#ifndef RWKV7M_SCREENING_H
#define RWKV7M_SCREENING_H

#include <stdint.h>

#include "rwkv7m_wkv.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Floats of fp32 device workspace each slot-scan call needs (-1 for
 * invalid sizes).  No counterpart in the reference (XLA allocates its scan
 * buffers itself). */
int64_t rwkv7m_screen_slot_scan_workspace_floats(int64_t B, int64_t T,
                                                 int64_t M, int64_t ds);

/* Slots read at each step (S_t, t = 0..T-1, rounded to dtype), the final
 * slots S_T, and upd2[b][t][m][g] = sum over channels 64g..64g+63 of
 * (mu (delta - S_t))^2 (for the slot_update_norm statistic).  Replaces the
 * slot half of the scan step, nnx_model.py:1087-1102. */
int rwkv7m_screen_slot_scan(int dtype, int64_t B, int64_t T, int64_t M,
                            int64_t ds, const void *base,
                            const float *slot_term, const float *mu,
                            const float *slots0, void *slots_seq,
                            float *slots_T, float *upd2, float *workspace,
                            int64_t workspace_floats, void *stream);

/* Adjoint of rwkv7m_screen_slot_scan: from the cotangents of slots_seq and
 * of slots_T (NULL = zero) to d_pre[b][t][m][d] (the cotangent of the tanh
 * argument; its sum over m is d base, over b and t d slot_term),
 * d_slots0 and d_mu_part[b][m][d] (summed over b and d it is d mu). */
int rwkv7m_screen_slot_scan_backward(
    int dtype, int64_t B, int64_t T, int64_t M, int64_t ds, const void *base,
    const float *slot_term, const float *mu, const void *slots_seq,
    const void *d_slots_seq, const float *d_slots_T, float *d_pre,
    float *d_slots0, float *d_mu_part, float *workspace,
    int64_t workspace_floats, void *stream);

/* Per-token read.  tau is one fp32 on the device, in (-1, 1) (the
 * reference's bounded_tau), read by the kernel so that a caller can capture
 * the call in a HIP graph.  leaky = 0: rel = trim_square(sim, tau,
 * trim_eps) * age;
 * leaky = 1: ((1 - alpha) trim_square + alpha sigmoid(gamma (sim - tau)))
 * * age.  age_w may be NULL (no age mask); it is [B][M], or [B][T][M] with
 * age_per_step = 1 (the write phase's ages change at every step).  Replaces nnx_model.py:1063-1086
 * for every step at once. */
int rwkv7m_screen_read(int dtype, int64_t B, int64_t T, int64_t M,
                       int64_t dk, int64_t dv, const float *q,
                       const void *proj, const float *tau, double trim_eps,
                       const float *age_w, int age_per_step,
                       int value_unit_norm, int leaky, double leaky_alpha,
                       double leaky_gamma, double cap, double eps, void *u,
                       float *rel, float *z_norm, float *u_norm,
                       void *stream);

/* Adjoint of rwkv7m_screen_read: from du (and d_rel, the cotangent of rel,
 * may be NULL) to dq, d_proj, d_tau[b][t] (summed it is d tau) and
 * g_age[b][t][m] = d rel * rel / age (summed over t it is d age_w). */
int rwkv7m_screen_read_backward(
    int dtype, int64_t B, int64_t T, int64_t M, int64_t dk, int64_t dv,
    const float *q, const void *proj, const float *tau, double trim_eps,
    const float *age_w, int age_per_step, int value_unit_norm, int leaky,
    double leaky_alpha, double leaky_gamma, double cap, double eps,
    const void *du, const float *d_rel, float *dq, void *d_proj,
    float *d_tau, float *g_age, void *stream);

/* Write phase (read_write, nnx_model.py:1040-1047 and :1103-1115): the slot
 * recurrence whose update strength is mu * max(rel_w, floor), rel_w the
 * trim-square relevance of the write query q_w [B][T][dk] (fp32, unit
 * norm) against the write keys unit_norm(round(S_t + slot_embed) kw)
 * (kw [ds][dk] fp32), with ages reset where rel_w > 1e-3.  One workgroup
 * per (b, m) walks the steps.  Outputs: slots_seq (S_t rounded to dtype,
 * for the read), slots32 (S_t fp32, for the backward), ages_seq [B][T][M]
 * (the ages step t reads), rel_w [B][T][M], upd2 as the read-only scan,
 * slots_T, ages_T.  Limits: ds <= 1024, 1 <= dk <= 128. */
int rwkv7m_screen_write(int dtype, int64_t B, int64_t T, int64_t M,
                        int64_t ds, int64_t dk, const void *base,
                        const float *slot_term, const float *slot_embed,
                        const float *kw, const float *q_w, const float *tau_w,
                        const float *mu, double floor, double eps,
                        const float *slots0, const float *ages0,
                        void *slots_seq, float *slots32, float *ages_seq,
                        float *rel_w, float *upd2, float *slots_T,
                        float *ages_T, void *stream);

/* Adjoint of rwkv7m_screen_write.  Cotangents in: d_slots_seq (dtype),
 * d_slots_T, d_rel_w, d_ages_seq, d_ages_T (fp32; each may be NULL = 0).
 * Out: d_pre [B][T][M][ds] (as the read-only scan), d_slots0, d_ages0,
 * d_embed_part [B][M][ds] (summed over b: d slot_embed through the write
 * keys), d_mu_bm [B][M] (summed over b: d mu), d_kraw [B][T][M][dk] (the
 * cotangent of the write keys before normalisation: d kw is the sum over
 * (b, t, m) of round(S_t + slot_embed)^T d_kraw), dq_w [B][T][M][dk]
 * (summed over m: d q_w) and d_tau_w [B][T][M] (summed: d tau_w). */
int rwkv7m_screen_write_backward(
    int dtype, int64_t B, int64_t T, int64_t M, int64_t ds, int64_t dk,
    const void *base, const float *slot_term, const float *slot_embed,
    const float *kw, const float *q_w, const float *tau_w, const float *mu,
    double floor, double eps, const float *slots32, const void *d_slots_seq,
    const float *d_slots_T, const float *d_rel_w, const float *d_ages_seq,
    const float *d_ages_T, float *d_pre, float *d_slots0, float *d_ages0,
    float *d_embed_part, float *d_mu_bm, float *d_kraw, float *dq_w,
    float *d_tau_w, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* RWKV7M_SCREENING_H */
