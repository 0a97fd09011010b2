/*
 * TEST INFRASTRUCTURE ONLY: the CPU oracle for the WKV-7 recurrence.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker; no product code path calls into it.
 *
 * This body is included twice by wkv_oracle.c, once with REAL=double (the
 * parity oracle) and once with REAL=float (the reference's own fp32
 * arithmetic, used as the timed CPU baseline).  SUFFIX names the variant.
 *
 * Layout (matches the reference's time-major contract, wkv.py:19-57):
 *   vectors r,w,k,v,a(=neg_kk),b(=kka): [T][B][H][N]
 *   state S:                            [B][H][N][N], S[i][j] with i = row
 *                                       (value index), j = column (key index)
 */

#define CAT2(a, b) a##b
#define CAT(a, b) CAT2(a, b)
#define FN(name) CAT(name, SUFFIX)

/* One recurrence step on one (b, h) state, in place.
 * Follows wkv_step, src/rwkv7m/model/rwkv_core.py:54-86:
 *   d = exp(-exp(w));  sa = S @ a;  S = S*d[j] + sa (x) b + v (x) k;  y = S @ r
 * sa_out (may be NULL) receives sa for the backward pass. */
static void FN(step_)(int64_t n, REAL *s, const REAL *r, const REAL *w,
                      const REAL *k, const REAL *v, const REAL *a,
                      const REAL *b, REAL *y, REAL *sa_out, REAL *decay)
{
    for (int64_t j = 0; j < n; ++j)
        decay[j] = EXP(-EXP(w[j]));
    for (int64_t i = 0; i < n; ++i) {
        REAL *row = s + i * n;
        REAL sa = 0;
        for (int64_t j = 0; j < n; ++j)
            sa += row[j] * a[j];
        if (sa_out)
            sa_out[i] = sa;
        REAL acc = 0;
        for (int64_t j = 0; j < n; ++j) {
            row[j] = row[j] * decay[j] + sa * b[j] + v[i] * k[j];
            acc += row[j] * r[j];
        }
        y[i] = acc;
    }
}

/* Forward scan over T (wkv.py:60-67 lax.scan of wkv_step), for every (b, h).
 * ckpt (may be NULL) receives the reference aux checkpoint format of
 * wkv_pallas_gpu.py:83-120 / :319-343: ckpt[0] = S0, ckpt[c] = state after
 * token c*ci - 1, last entry = S_T.  Shape [ceil(T/ci)+1][B][H][N][N]. */
void FN(oracle_wkv7_forward_)(int64_t T, int64_t B, int64_t H, int64_t N,
                              const REAL *r, const REAL *w, const REAL *k,
                              const REAL *v, const REAL *a, const REAL *b,
                              const REAL *s0, REAL *y, REAL *s_t, REAL *ckpt,
                              int64_t ci, int threads)
{
    const int64_t BH = B * H, NN = N * N;
    const int64_t nck = ci > 0 ? (T + ci - 1) / ci + 1 : 0;
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t bh = 0; bh < BH; ++bh) {
        REAL *s = s_t + bh * NN;
        REAL *decay = (REAL *)malloc(sizeof(REAL) * N);
        memcpy(s, s0 + bh * NN, sizeof(REAL) * NN);
        if (ckpt)
            memcpy(ckpt + bh * NN, s, sizeof(REAL) * NN);
        for (int64_t t = 0; t < T; ++t) {
            const int64_t off = (t * BH + bh) * N;
            FN(step_)(N, s, r + off, w + off, k + off, v + off, a + off,
                      b + off, y + off, NULL, decay);
            if (ckpt && ((t + 1) % ci == 0 || t + 1 == T)) {
                int64_t c = (t + ci) / ci;
                memcpy(ckpt + (c * BH + bh) * NN, s, sizeof(REAL) * NN);
            }
        }
        (void)nck;
        free(decay);
    }
}

/* Reverse-mode pass.  The per-token equations follow the Pallas backward,
 * wkv_pallas_gpu.py:221-257, which is the transpose of wkv_step:
 *   G  = dS + dy (x) r
 *   dr[j] = sum_i S_t[i,j] dy[i]      dd[j] = sum_i G[i,j] S_{t-1}[i,j]
 *   dsa[i] = sum_j G[i,j] b[j]        db[j] = sum_i G[i,j] sa[i]
 *   dv[i] = sum_j G[i,j] k[j]         dk[j] = sum_i G[i,j] v[i]
 *   da[j] = sum_i S_{t-1}[i,j] dsa[i] dw[j] = dd[j] * (-exp(w[j]) * d[j])
 *   dS_{t-1} = G * d[j] + dsa (x) a
 * States S_{t-1}, S_t are recomputed forward from every 16th state instead of
 * the reference kernel's division by the decay (no loss for tiny decays). */
void FN(oracle_wkv7_backward_)(int64_t T, int64_t B, int64_t H, int64_t N,
                               const REAL *r, const REAL *w, const REAL *k,
                               const REAL *v, const REAL *a, const REAL *b,
                               const REAL *s0, const REAL *dy,
                               const REAL *ds_t, REAL *dr, REAL *dw,
                               REAL *dk, REAL *dv, REAL *da, REAL *db,
                               REAL *ds0, int threads)
{
    const int64_t BH = B * H, NN = N * N, SEG = 16;
    (void)threads;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (int64_t bh = 0; bh < BH; ++bh) {
        const int64_t nseg = (T + SEG - 1) / SEG;
        /* seg_start[s] = state before token s*SEG */
        REAL *seg_start = (REAL *)malloc(sizeof(REAL) * NN * (nseg + 1));
        REAL *states = (REAL *)malloc(sizeof(REAL) * NN * (SEG + 1));
        REAL *sas = (REAL *)malloc(sizeof(REAL) * N * SEG);
        REAL *ytmp = (REAL *)malloc(sizeof(REAL) * N);
        REAL *decay = (REAL *)malloc(sizeof(REAL) * N);
        REAL *ds = (REAL *)malloc(sizeof(REAL) * NN);
        REAL *g = (REAL *)malloc(sizeof(REAL) * NN);
        REAL *dsa = (REAL *)malloc(sizeof(REAL) * N);

        memcpy(seg_start, s0 + bh * NN, sizeof(REAL) * NN);
        {
            REAL *s = states;
            memcpy(s, s0 + bh * NN, sizeof(REAL) * NN);
            for (int64_t t = 0; t < T; ++t) {
                const int64_t off = (t * BH + bh) * N;
                FN(step_)(N, s, r + off, w + off, k + off, v + off, a + off,
                          b + off, ytmp, NULL, decay);
                if ((t + 1) % SEG == 0)
                    memcpy(seg_start + ((t + 1) / SEG) * NN, s,
                           sizeof(REAL) * NN);
            }
        }
        memcpy(ds, ds_t + bh * NN, sizeof(REAL) * NN);

        for (int64_t sg = nseg - 1; sg >= 0; --sg) {
            const int64_t t0 = sg * SEG;
            const int64_t t1 = (t0 + SEG < T) ? t0 + SEG : T;
            /* states[u] = state before token t0+u; states[u+1] after it */
            memcpy(states, seg_start + sg * NN, sizeof(REAL) * NN);
            for (int64_t t = t0; t < t1; ++t) {
                const int64_t u = t - t0, off = (t * BH + bh) * N;
                memcpy(states + (u + 1) * NN, states + u * NN,
                       sizeof(REAL) * NN);
                FN(step_)(N, states + (u + 1) * NN, r + off, w + off,
                          k + off, v + off, a + off, b + off, ytmp,
                          sas + u * N, decay);
            }
            for (int64_t t = t1 - 1; t >= t0; --t) {
                const int64_t u = t - t0, off = (t * BH + bh) * N;
                const REAL *sp = states + u * NN;      /* S_{t-1} */
                const REAL *sc = states + (u + 1) * NN; /* S_t */
                const REAL *sa = sas + u * N;
                const REAL *rt = r + off, *wt = w + off, *kt = k + off;
                const REAL *vt = v + off, *at = a + off, *bt = b + off;
                const REAL *dyt = dy + off;
                for (int64_t j = 0; j < N; ++j)
                    decay[j] = EXP(-EXP(wt[j]));
                for (int64_t i = 0; i < N; ++i) {
                    REAL acc_dsa = 0, acc_dv = 0;
                    for (int64_t j = 0; j < N; ++j) {
                        REAL gij = ds[i * N + j] + dyt[i] * rt[j];
                        g[i * N + j] = gij;
                        acc_dsa += gij * bt[j];
                        acc_dv += gij * kt[j];
                    }
                    dsa[i] = acc_dsa;
                    dv[off + i] = acc_dv;
                }
                for (int64_t j = 0; j < N; ++j) {
                    REAL acc_dr = 0, acc_dd = 0, acc_db = 0, acc_dk = 0,
                         acc_da = 0;
                    for (int64_t i = 0; i < N; ++i) {
                        REAL gij = g[i * N + j];
                        acc_dr += sc[i * N + j] * dyt[i];
                        acc_dd += gij * sp[i * N + j];
                        acc_db += gij * sa[i];
                        acc_dk += gij * vt[i];
                        acc_da += sp[i * N + j] * dsa[i];
                    }
                    dr[off + j] = acc_dr;
                    dw[off + j] = acc_dd * (-EXP(wt[j]) * decay[j]);
                    db[off + j] = acc_db;
                    dk[off + j] = acc_dk;
                    da[off + j] = acc_da;
                }
                for (int64_t i = 0; i < N; ++i)
                    for (int64_t j = 0; j < N; ++j)
                        ds[i * N + j] =
                            g[i * N + j] * decay[j] + dsa[i] * at[j];
            }
        }
        memcpy(ds0 + bh * NN, ds, sizeof(REAL) * NN);
        free(seg_start);
        free(states);
        free(sas);
        free(ytmp);
        free(decay);
        free(ds);
        free(g);
        free(dsa);
    }
}

#undef FN
#undef CAT
#undef CAT2
