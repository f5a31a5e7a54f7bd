/*
 * ltq_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Plain-C restatement of the reference TCQ Viterbi quantizer, used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg. The product path
 * (ltq-research_amd/) never links or loads this file.
 *
 * What it restates (reference file:line):
 *   - labels, branch metrics     src/cuda/tcq_viterbi.cu:46-95, src/tcq_proto.py:363-387
 *   - tile load / rot / ld       src/cuda/tcq_viterbi.cu:133-137
 *   - gain-candidate prologue    src/cuda/tcq_viterbi.cu:155-180
 *   - sub-block gain merge       src/cuda/tcq_viterbi.cu:184-201, src/tcq_proto.py:393-396
 *   - integer ACS step           src/cuda/tcq_viterbi.cu:501-554, src/tcq_proto.py:327-332
 *   - D2 pair (pp=1)             src/cuda/tcq_viterbi.cu:268-313, 444-500
 *   - D4 / EQ group (pp=2/3)     src/cuda/tcq_viterbi.cu:217-267, 322-443
 *   - free / given start          src/cuda/tcq_viterbi.cu:151-153, 314-321
 *   - final argmin (tail)        src/cuda/tcq_viterbi.cu:561-578
 *   - traceback (mid, planes)    src/cuda/tcq_viterbi.cu:580-661
 *   - reconstruction / code      src/cuda/tcq_viterbi.cu:662-682
 *   - ABI validation             src/cuda/tcq_viterbi.cu:748-763
 *   - FWHT-256                   src/iqk_format.py:153-170
 *
 * Arithmetic: fp32, no FP contraction (built with -ffp-contract=off), the same
 * order of operations as the torch reference viterbi_ub (x - fl(g*tab), squared,
 * min over u, times w). Every "best = 3.4e38; if (v < best)" selection is kept
 * verbatim, including the sentinel initialisation.
 *
 * Decision storage is per (step, gain slot, state) bytes -- simple, not fast.
 */
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define SENT 3.4e38f
#define MAX_G 16
#define MAX_U 128
#define MAX_SUBS 32
#define MAX_T 512

/* Planted-mistake switch for the oracle's own tests (never set elsewhere): 1 = integer-step predecessor
 * ties go to p1 instead of p0. Used to show that the tie-heavy golden vectors detect a wrong tie rule. */
int ltq_oracle_plant = 0;

static inline int par32(uint32_t v) { return __builtin_popcount(v) & 1; }

static inline int label_x(int s, int m, int m2, int m3, int m4, int nl)
{
    int lb = (par32((uint32_t)((s >> 1) & m)) << 1) | (s & 1);
    if (nl >= 8) lb |= par32((uint32_t)((s >> 1) & m2)) << 2;
    if (nl >= 16) lb |= par32((uint32_t)((s >> 1) & m3)) << 3;
    if (nl >= 32) lb |= par32((uint32_t)((s >> 1) & m4)) << 4;
    return lb;
}

/* min over u (stride du, from u0) of fl(fl(x - fl(g*tab[u]))^2), sentinel start (tcq_viterbi.cu:46-54, 75-83) */
static inline float branch_err(float xt, float gain, const float* tab, int u0, int U, int du)
{
    float e = SENT;
    for (int u = u0; u < U; u += du) {
        float v = gain * tab[u];
        float d = xt - v;
        float dd = d * d;
        e = fminf(e, dd);
    }
    return e;
}

typedef struct {
    const float *x, *w, *tab, *gains, *tab_hi, *gains_hi;
    float* rec;
    const int* init_st;
    int *end_st, *best, *code, *mid_st;
    uint8_t* gcand;
    uint8_t* gsel_out; /* optional [N, T/sub, S] */
    int mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pp;
} OArgs;

typedef struct {
    float *cur, *tmp;            /* [G][S] */
    float *I, *C, *J;            /* D2/D4 intermediates: I [2][G][S], C [2][G][S], J [4][G][S] */
    uint8_t* dec;                /* [T][G][S] predecessor bits */
    uint8_t* par;                /* [T/2][G][S] D2 class bits */
    uint8_t* pl;                 /* [T/4][G][9][S] D4 planes */
    uint8_t* gsel;               /* [T/sub][S] */
    float* err;                  /* [G][nl][2] metrics of one step */
} Work;

static int validate(int N, int T, int S, int U, int G, int Gfull, int sub, int U_hi, int mix, int nl, int ld, int pp,
                    int has_gcand)
{
    (void)N;
    if (G > MAX_G || Gfull > MAX_G || (!has_gcand && Gfull != G) || U > MAX_U || U_hi > MAX_U || sub <= 0 ||
        T % sub != 0 || (sub & 1) || T / sub > MAX_SUBS || T > MAX_T || sub > 32 ||
        sub * G * nl * (pp ? 2 : 1) > 4096 || (pp && (S != 1024 || mix > 0 || (T & 1))) ||
        (pp >= 2 && ((T & 3) || (sub & 3))) || pp > 3 || pp < 0 ||
        (nl != 4 && nl != 8 && nl != 16 && nl != 32) || ld < T || (S != 1024 && nl != 4) || nl * U > 4 * MAX_U ||
        nl * U_hi > 4 * MAX_U)
        return -1;
    if (S != 1024 && S != 256) return -1;
    if (G != 1 && G != 2 && G != 3 && G != 4 && G != 8) return -1;
    if (T <= 0 || G <= 0) return -1;
    return 0;
}

/* metrics of step t for every (slot g, label, parity class) -> wk->err */
static void step_metrics(const OArgs* a, const float* xs, const float* ws, const uint8_t* gc, int t, float* err)
{
    const int NP = a->pp ? 2 : 1;
    const int cand = a->gcand != NULL;
    for (int g = 0; g < a->G; g++) {
        const int gi = cand ? (int)gc[(t / a->sub) * a->G + g] : g;
        const int hi = a->mix > 0 && ((t / a->mix) & 1);
        for (int lb = 0; lb < a->nl; lb++)
            for (int p = 0; p < NP; p++) {
                float e;
                if (a->pp) e = branch_err(xs[t], a->gains[gi], a->tab + lb * a->U, p, a->U, 2);
                else if (hi) e = branch_err(xs[t], a->gains_hi[gi], a->tab_hi + lb * a->U_hi, 0, a->U_hi, 1);
                else e = branch_err(xs[t], a->gains[gi], a->tab + lb * a->U, 0, a->U, 1);
                err[(g * a->nl + lb) * 2 + p] = e * ws[t];
            }
    }
}

#define E(g, lb, p) err[((g) * nl + (lb)) * 2 + (p)]

static void run_tile(const OArgs* a, int n, Work* wk, int* labs)
{
    const int T = a->T, S = a->S, G = a->G, sub = a->sub, nl = a->nl, pp = a->pp;
    const int HALF = S / 2;
    const int EQ = pp == 3, G4 = pp >= 2;
    const int cand = a->gcand != NULL;
    const int nsub = T / sub, Gf = a->Gfull;
    float xs[MAX_T], ws[MAX_T];
    uint8_t gc[MAX_SUBS * MAX_G];
    float* err = wk->err;

    for (int i = 0; i < T; i++) {
        const size_t j = (size_t)n * a->ld + (size_t)((i + a->rot) % a->ld);
        xs[i] = a->x[j];
        ws[i] = a->w[j];
    }
    const int s0 = a->init_st ? a->init_st[n] : -1;

    if (cand) { /* tcq_viterbi.cu:155-180 */
        float ce[MAX_SUBS * MAX_G];
        for (int j = 0; j < nsub; j++)
            for (int gi = 0; gi < Gf; gi++) {
                float e = 0.f;
                for (int t = j * sub; t < (j + 1) * sub; t++) {
                    const int hi = a->mix > 0 && ((t / a->mix) & 1);
                    float be = hi ? branch_err(xs[t], a->gains_hi[gi], a->tab_hi, 0, nl * a->U_hi, 1)
                                  : branch_err(xs[t], a->gains[gi], a->tab, 0, nl * a->U, 1);
                    float prod = be * ws[t];
                    e = e + prod;
                }
                ce[j * Gf + gi] = e;
            }
        for (int j = 0; j < nsub; j++) {
            uint32_t used = 0;
            for (int c = 0; c < G; c++) {
                int bg = 0;
                float be = SENT;
                for (int gi = 0; gi < Gf; gi++)
                    if (!((used >> gi) & 1) && ce[j * Gf + gi] < be) { be = ce[j * Gf + gi]; bg = gi; }
                used |= 1u << bg;
                gc[j * G + c] = (uint8_t)bg;
                a->gcand[((size_t)n * nsub + j) * G + c] = (uint8_t)bg;
            }
        }
    }

    float* cur = wk->cur;
    float* I = wk->I; /* I[b][g][s] */
    float* C = wk->C; /* C[c][g][s] */
    float* J = wk->J; /* J[c*2+b][g][s] */
    uint8_t* dec = wk->dec;
    uint8_t* parb = wk->par;
    uint8_t* pl = wk->pl;
    uint8_t* gsel = wk->gsel;
    const size_t GS = (size_t)G * S;
#define DEC(t, g, s) dec[((size_t)(t) * G + (g)) * S + (s)]
#define PAR(i, g, s) parb[((size_t)(i) * G + (g)) * S + (s)]
#define PL(q, g, k, s) pl[(((size_t)(q) * G + (g)) * 9 + (k)) * S + (s)]

    int t = 0;
    while (t < T) {
        if (t > 0 && (t % sub) == 0 && G > 1) { /* gain merge, tcq_viterbi.cu:185-201 */
            for (int s = 0; s < S; s++) {
                float bv = cur[s];
                int bg = 0;
                for (int g = 1; g < G; g++) {
                    float v = cur[g * S + s];
                    if (v < bv) { bv = v; bg = g; }
                }
                gsel[(size_t)(t / sub) * S + s] = (uint8_t)bg;
                for (int g = 0; g < G; g++) cur[g * S + s] = bv;
            }
        }
        if (pp == 0) {
            step_metrics(a, xs, ws, gc, t, err);
            if (t == 0) { /* tcq_viterbi.cu:314-321 */
                for (int s = 0; s < S; s++) {
                    const int ok = s0 < 0 || (s >> 1) == (s0 & (HALF - 1));
                    for (int g = 0; g < G; g++) cur[g * S + s] = ok ? E(g, labs[s], 0) : SENT;
                }
            } else { /* tcq_viterbi.cu:540-554 */
                float* nx = wk->tmp;
                for (int g = 0; g < G; g++)
                    for (int s = 0; s < S; s++) {
                        const float va = cur[g * S + (s >> 1)], vb = cur[g * S + HALF + (s >> 1)];
                        const int h = ltq_oracle_plant == 1 ? vb <= va : vb < va;
                        nx[g * S + s] = (h ? vb : va) + E(g, labs[s], 0);
                        DEC(t, g, s) = (uint8_t)h;
                    }
                memcpy(cur, nx, GS * sizeof(float));
            }
            t += 1;
        } else if (pp == 1) {
            /* step t: intermediates per parity class p */
            step_metrics(a, xs, ws, gc, t, err);
            for (int g = 0; g < G; g++)
                for (int s = 0; s < S; s++)
                    for (int p = 0; p < 2; p++) {
                        float v;
                        if (t == 0) {
                            const int ok = s0 < 0 || (s >> 1) == (s0 & (HALF - 1));
                            v = ok ? E(g, labs[s], p) : SENT;
                        } else {
                            const float va = cur[g * S + (s >> 1)], vb = cur[g * S + HALF + (s >> 1)];
                            const int h = vb < va;
                            v = (h ? vb : va) + E(g, labs[s], p);
                            if (p == 0) DEC(t, g, s) = (uint8_t)h;
                        }
                        I[p * GS + g * S + s] = v;
                    }
            /* step t+1: best class (p ascending, strict <) */
            step_metrics(a, xs, ws, gc, t + 1, err);
            for (int g = 0; g < G; g++)
                for (int s = 0; s < S; s++) {
                    const int q0 = s >> 1, q1 = HALF + (s >> 1);
                    float best = SENT;
                    int bh = 0, bp = 0;
                    for (int p = 0; p < 2; p++) {
                        const float va = I[p * GS + g * S + q0], vb = I[p * GS + g * S + q1];
                        const int h = vb < va;
                        const float v = (h ? vb : va) + E(g, labs[s], p);
                        if (v < best) { best = v; bh = h; bp = p; }
                    }
                    cur[g * S + s] = best;
                    DEC(t + 1, g, s) = (uint8_t)bh;
                    PAR(t / 2, g, s) = (uint8_t)bp;
                }
            t += 2;
        } else {
            const int q = t / 4;
            /* phase A, step t: intermediates per low bit b */
            step_metrics(a, xs, ws, gc, t, err);
            for (int g = 0; g < G; g++)
                for (int s = 0; s < S; s++)
                    for (int b = 0; b < 2; b++) {
                        float v;
                        if (t == 0) {
                            const int ok = s0 < 0 || (s >> 1) == (s0 & (HALF - 1));
                            v = ok ? E(g, labs[s], b) : SENT;
                        } else {
                            const float va = cur[g * S + (s >> 1)], vb = cur[g * S + HALF + (s >> 1)];
                            const int h = vb < va;
                            v = (h ? vb : va) + E(g, labs[s], b);
                            if (b == 0) DEC(t, g, s) = (uint8_t)h;
                        }
                        I[b * GS + g * S + s] = v;
                    }
            /* phase A, step t+1: class c = XOR of the pair's low bits */
            step_metrics(a, xs, ws, gc, t + 1, err);
            for (int g = 0; g < G; g++)
                for (int s = 0; s < S; s++) {
                    const int q0 = s >> 1, q1 = HALF + (s >> 1);
                    for (int c = 0; c < 2; c++) {
                        float best = SENT;
                        int bh = 0, bb = 0;
                        for (int b = EQ ? c : 0; b < (EQ ? c + 1 : 2); b++) {
                            const float va = I[b * GS + g * S + q0], vb = I[b * GS + g * S + q1];
                            const int h = vb < va;
                            const float v = (h ? vb : va) + E(g, labs[s], EQ ? c : (b ^ c));
                            if (v < best) { best = v; bh = h; bb = b; }
                        }
                        C[c * GS + g * S + s] = best;
                        PL(q, g, c, s) = (uint8_t)bh;
                        PL(q, g, 2 + c, s) = (uint8_t)bb;
                    }
                }
            /* phase B, step t+2: intermediates per (class, low bit) */
            step_metrics(a, xs, ws, gc, t + 2, err);
            for (int g = 0; g < G; g++)
                for (int s = 0; s < S; s++)
                    for (int c = 0; c < 2; c++) {
                        const float va = C[c * GS + g * S + (s >> 1)], vb = C[c * GS + g * S + HALF + (s >> 1)];
                        const int h = vb < va;
                        const float mn = h ? vb : va;
                        PL(q, g, 4 + c, s) = (uint8_t)h;
                        for (int b = 0; b < 2; b++) J[(c * 2 + b) * GS + g * S + s] = mn + E(g, labs[s], b);
                    }
            /* phase B, step t+3: best (c, b) in order 00, 01, 10, 11 */
            step_metrics(a, xs, ws, gc, t + 3, err);
            for (int g = 0; g < G; g++)
                for (int s = 0; s < S; s++) {
                    const int q0 = s >> 1, q1 = HALF + (s >> 1);
                    float best = SENT;
                    int oc = 0, oh = 0, ob = 0;
                    for (int c = 0; c < 2; c++)
                        for (int b = EQ ? c : 0; b < (EQ ? c + 1 : 2); b++) {
                            const float va = J[(c * 2 + b) * GS + g * S + q0], vb = J[(c * 2 + b) * GS + g * S + q1];
                            const int h = vb < va;
                            const float v = (h ? vb : va) + E(g, labs[s], EQ ? c : (b ^ c));
                            if (v < best) { best = v; oc = c; oh = h; ob = b; }
                        }
                    cur[g * S + s] = best;
                    PL(q, g, 6, s) = (uint8_t)oc;
                    PL(q, g, 7, s) = (uint8_t)oh;
                    PL(q, g, 8, s) = (uint8_t)ob;
                }
            t += 4;
        }
    }
    if (a->gsel_out) memcpy(a->gsel_out + (size_t)n * nsub * S, gsel, (size_t)nsub * S);

    /* argmin over (g, s), lowest index on ties (tcq_viterbi.cu:561-578) */
    float bv = SENT;
    int bi = INT_MAX;
    const int s_end = a->tail ? s0 : -1;
    for (int g = 0; g < G; g++)
        for (int s = 0; s < S; s++) {
            const int idx = g * S + s;
            const float v = (s_end < 0 || s == s_end) ? cur[idx] : SENT;
            if (v < bv || (v == bv && idx < bi)) { bv = v; bi = idx; }
        }
    if (bi == INT_MAX) bi = 0; /* every candidate above the sentinel: the reference reads out of range here */
    a->best[n] = bi;
    if (a->end_st) a->end_st[n] = bi % S;

    /* traceback (tcq_viterbi.cu:601-661) */
    uint16_t s_st[MAX_T];
    uint8_t s_g[MAX_T], s_par[MAX_T];
    memset(s_par, 0, sizeof(s_par));
    int st = bi % S, g = bi / S, pcur = 0, cstar = 0;
    for (int tt = T - 1; tt >= 0; tt--) {
        s_st[tt] = (uint16_t)st;
        s_g[tt] = (uint8_t)g;
        if (pp == 1) {
            if (tt & 1) pcur = PAR(tt >> 1, g, st);
            s_par[tt] = (uint8_t)pcur;
        }
        if (a->mid_st && tt == a->mid_t - 1) {
            a->mid_st[n] = st;
            return; /* first tail-biting pass: only the state before mid_t (tcq_viterbi.cu:623, 660) */
        }
        if (G4 && (tt & 3)) {
            const int qq = tt >> 2;
            int hh;
            if ((tt & 3) == 3) {
                cstar = PL(qq, g, 6, st);
                hh = PL(qq, g, 7, st);
                if (EQ) {
                    s_par[tt] = s_par[tt - 1] = s_par[tt - 2] = s_par[tt - 3] = (uint8_t)cstar;
                } else {
                    const int bb = PL(qq, g, 8, st);
                    s_par[tt] = (uint8_t)(bb ^ cstar);
                    s_par[tt - 1] = (uint8_t)bb;
                }
            } else if ((tt & 3) == 2) {
                hh = PL(qq, g, 4 + cstar, st);
            } else {
                hh = PL(qq, g, 0 + cstar, st);
                if (!EQ) {
                    const int bb = PL(qq, g, 2 + cstar, st);
                    s_par[tt] = (uint8_t)(bb ^ cstar);
                    s_par[tt - 1] = (uint8_t)bb;
                }
            }
            st = hh * HALF + (st >> 1);
        } else if (tt > 0) {
            st = DEC(tt, g, st) * HALF + (st >> 1);
            if (G > 1 && (tt % sub) == 0) g = gsel[(size_t)(tt / sub) * S + st];
        }
    }

    /* reconstruction and code (tcq_viterbi.cu:662-682) */
    float* rn = a->rec + (size_t)n * a->ld;
    for (int tt = 0; tt < T; tt++) {
        const int stt = s_st[tt], gg = s_g[tt];
        const int lb = labs[stt];
        const int hi = a->mix > 0 && ((tt / a->mix) & 1);
        const int Ut = hi ? a->U_hi : a->U;
        const int gi = cand ? (int)gc[(tt / sub) * G + gg] : gg;
        const float gt = hi ? a->gains_hi[gi] : a->gains[gi];
        const float* tb = (hi ? a->tab_hi : a->tab) + lb * Ut;
        const float xt = xs[tt];
        float bestd = SENT, val = 0.f;
        int bu = 0;
        for (int u = pp ? s_par[tt] : 0; u < Ut; u += pp ? 2 : 1) {
            const float v = gt * tb[u];
            const float d = xt - v;
            const float dd = d * d;
            if (dd < bestd) { bestd = dd; val = v; bu = u; }
        }
        const int tp = (tt + a->rot) % a->ld;
        rn[tp] = val;
        if (a->code) a->code[(size_t)n * a->ld + tp] = (gi << 16) | (lb * Ut + bu);
    }
#undef DEC
#undef PAR
#undef PL
}
#undef E

/* Same argument list as the reference export tcq_viterbi (tcq_viterbi.cu:743-746) minus the three
 * caller-provided scratch buffers (bp, gsel, pbits), plus an optional gsel output and a thread count. */
int ltq_oracle_tcq_viterbi(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                           const int* init_st, int* end_st, const float* tab_hi, const float* gains_hi, uint8_t* gcand,
                           int* best, int* code, int* mid_st, int mid_t, int tail, int N, int T, int S, int U, int G,
                           int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3, int m4, int nl, int ld, int rot,
                           int pp, uint8_t* gsel_out, int nthreads)
{
    if (validate(N, T, S, U, G, Gfull, sub, U_hi, mix, nl, ld, pp, gcand != NULL)) return -1;
    OArgs a = {x, w, tab, gains, tab_hi, gains_hi, rec, init_st, end_st, best, code, mid_st, gcand, gsel_out,
               mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pp};
    int* labs = (int*)malloc(sizeof(int) * S);
    for (int s = 0; s < S; s++) labs[s] = label_x(s, m, m2, m3, m4, nl);
    int rc = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel
    {
        const size_t GS = (size_t)G * S;
        Work wk;
        wk.cur = (float*)malloc(GS * sizeof(float));
        wk.tmp = (float*)malloc(GS * sizeof(float));
        wk.I = (float*)malloc(2 * GS * sizeof(float));
        wk.C = (float*)malloc(2 * GS * sizeof(float));
        wk.J = (float*)malloc(4 * GS * sizeof(float));
        wk.dec = (uint8_t*)calloc((size_t)T * GS, 1);
        wk.par = (uint8_t*)calloc((size_t)(T / 2 + 1) * GS, 1);
        wk.pl = (uint8_t*)calloc((size_t)(T / 4 + 1) * GS * 9, 1);
        wk.gsel = (uint8_t*)calloc((size_t)(T / sub + 1) * S, 1);
        wk.err = (float*)malloc(sizeof(float) * G * nl * 2);
        if (!wk.cur || !wk.tmp || !wk.I || !wk.C || !wk.J || !wk.dec || !wk.par || !wk.pl || !wk.gsel || !wk.err) {
#pragma omp atomic write
            rc = -2;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int n = 0; n < N; n++) run_tile(&a, n, &wk, labs);
        }
        free(wk.cur); free(wk.tmp); free(wk.I); free(wk.C); free(wk.J);
        free(wk.dec); free(wk.par); free(wk.pl); free(wk.gsel); free(wk.err);
    }
    free(labs);
    return rc;
}

/* label of every state, as the reference's lab_of / tcq_label_x (tcq_proto.py:370, tcq_viterbi.cu:85-95) */
void ltq_oracle_labels(int S, int m, int m2, int m3, int m4, int nl, int* out)
{
    for (int s = 0; s < S; s++) out[s] = label_x(s, m, m2, m3, m4, nl);
}

/* normalized FWHT over contiguous blocks of 256 (iqk_format.py:153-170): stages h = 1..128 of
 * (a + b, a - b), then x 0.0625 */
void ltq_oracle_fwht256(float* x, long n_blocks)
{
    for (long b = 0; b < n_blocks; b++) {
        float* y = x + b * 256;
        for (int h = 1; h < 256; h <<= 1)
            for (int i = 0; i < 256; i++)
                if (!(i & h)) {
                    const float p = y[i], q = y[i + h];
                    y[i] = p + q;
                    y[i + h] = p - q;
                }
        for (int i = 0; i < 256; i++) y[i] = y[i] * 0.0625f;
    }
}

/* lut_subs_kernel (tcq_viterbi.cu:771-800): per sub-block of 16 weights, bucket b_j = clamp(rint(x_j inv_step +
 * half_b), 0, nb - 1), err_c = sum_j d_j (x_j - lut[b_j][c])^2 over 64 candidates in order j = 0..15, the first
 * minimal c wins (strict '<' scan), out_j = lut[b_j][c]. The products and sums are written with fmaf as nvcc's
 * default contraction (--fmad=true) forms them: fma(x, inv_step, half_b) and err = fma(d e, e, err). A NaN
 * bucket argument gives bucket 0, as the device's float-to-int conversion does. */
static int lut_bucket(float x, float inv_step, float half_b, int nb)
{
    const float r = rintf(fmaf(x, inv_step, half_b));
    if (r != r) return 0;
    if (r < 0.f) return 0;
    if (r > (float)(nb - 1)) return nb - 1;
    return (int)r;
}

void ltq_oracle_lut_subs(const float* xs, const float* dh, const float* lut, float* out, long S, float inv_step,
                         float half_b, int nb)
{
#pragma omp parallel for schedule(static)
    for (long i = 0; i < S; i++) {
        float err[64];
        int b[16];
        for (int c = 0; c < 64; c++) err[c] = 0.f;
        for (int j = 0; j < 16; j++) {
            const float x = xs[i * 16 + j], d = dh[i * 16 + j];
            b[j] = lut_bucket(x, inv_step, half_b, nb);
            for (int c = 0; c < 64; c++) {
                const float e = x - lut[(long)b[j] * 64 + c];
                err[c] = fmaf(d * e, e, err[c]);
            }
        }
        int best = 0;
        float be = err[0];
        for (int c = 1; c < 64; c++)
            if (err[c] < be) {
                be = err[c];
                best = c;
            }
        for (int j = 0; j < 16; j++) out[i * 16 + j] = lut[(long)b[j] * 64 + best];
    }
}
