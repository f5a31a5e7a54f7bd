/*
 * ldlq_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Plain-C restatement of the LDLQ block error feedback of the TCQ matrix quantizer
 * (src/liqk_v2.py:948-980, row-scale branch), in the summation order the MI355X kernels define:
 *
 *   ltq_oracle_ldlq_sub     src/liqk_v2.py:957-967: after sub-block ib of a 256-column block,
 *                             G[:, s0:s1] = g, resid = w - fl(d g),
 *                             err = resid @ U_inv[s0:s1, s0:s1]      (fma chain over k = 0..15 from 0)
 *                             w[:, s1:] -= err @ U[s0:s1, s1:]       (fma chain over k = 0..15 from 0, then w - acc)
 *                             x_next = w[:, s1:s1+16] * fl(1 / d)    (the next sub-block's tiles, t = 16 r + c)
 *                           and the value each Viterbi saw, fed[:, s0:s1] = w[:, s0:s1].
 *   ltq_oracle_ldlq_err     src/liqk_v2.py:972-978: W_hat = fl(d G), E = (W_start - W_hat) @ U_blk_inv
 *                           (fma chain over k = 0..255 from 0).
 *   ltq_oracle_ldlq_update  src/liqk_v2.py:979: W[:, c1:] -= E @ U[c0:c1, c1:] (fma chain over k = 0..255 from 0,
 *                           then W - acc).
 *
 * The chains are the reference's matrix products evaluated in one fixed order: ascending k, one correctly
 * rounded fused multiply-add per term (fmaf; built with -ffp-contract=off so nothing else is fused).
 */
#include <math.h>
#include <stdint.h>

void ltq_oracle_ldlq_sub(float* wk, long ldw, const float* rec, const float* d, long ldd, const float* uinv, long ldi,
                         const float* ublk, long ldu, int ib, float* G, long ldg, float* xnext, long M, float* fed,
                         long ld_fed)
{
    const int s0 = 16 * ib, s1 = s0 + 16;
#pragma omp parallel for schedule(static)
    for (long n = 0; n < M / 16; n++) {
        float err[16][16];
        for (int r = 0; r < 16; r++) {
            const long row = 16 * n + r;
            const float dr = d[row * ldd];
            float resid[16];
            for (int c = 0; c < 16; c++) {
                const float g = rec[n * 256 + 16 * r + c];
                const float w = wk[row * ldw + s0 + c];
                G[row * ldg + s0 + c] = g;
                if (fed) fed[row * ld_fed + s0 + c] = w;
                resid[c] = w - dr * g;
            }
            for (int c = 0; c < 16; c++) {
                float e = 0.f;
                for (int k = 0; k < 16; k++) e = fmaf(resid[k], uinv[(long)(s0 + k) * ldi + s0 + c], e);
                err[r][c] = e;
            }
            for (int j = s1; j < 256; j++) {
                float acc = 0.f;
                for (int k = 0; k < 16; k++) acc = fmaf(err[r][k], ublk[(long)(s0 + k) * ldu + j], acc);
                wk[row * ldw + j] -= acc;
            }
            if (xnext && s1 < 256) {
                const float inv = 1.0f / dr;
                for (int c = 0; c < 16; c++) xnext[n * 256 + 16 * r + c] = wk[row * ldw + s1 + c] * inv;
            }
        }
    }
}

void ltq_oracle_ldlq_err(const float* ws, long ldw, const float* G, long ldg, const float* d, long ldd,
                         const float* uinv, long ldi, float* E, long ldE, float* what, long ldh, long M)
{
#pragma omp parallel for schedule(static)
    for (long i = 0; i < M; i++) {
        float a[256];
        const float di = d[i * ldd];
        for (int k = 0; k < 256; k++) {
            const float dg = di * G[i * ldg + k];
            if (what) what[i * ldh + k] = dg;
            a[k] = ws[i * ldw + k] - dg;
        }
        for (int j = 0; j < 256; j++) {
            float acc = 0.f;
            for (int k = 0; k < 256; k++) acc = fmaf(a[k], uinv[(long)k * ldi + j], acc);
            E[i * ldE + j] = acc;
        }
    }
}

void ltq_oracle_ldlq_update(float* W, long ldw, const float* E, long ldE, const float* U, long ldu, long M, long N)
{
#pragma omp parallel for schedule(static)
    for (long i = 0; i < M; i++) {
        const float* e = E + i * ldE;
        for (long j = 0; j < N; j++) {
            float acc = 0.f;
            for (int k = 0; k < 256; k++) acc = fmaf(e[k], U[(long)k * ldu + j], acc);
            W[i * ldw + j] -= acc;
        }
    }
}
