/*
 * ltq_brute.c -- TEST INFRASTRUCTURE ONLY: exhaustive search that pins the oracle's dynamic program.
 *
 * For a tiny tile it enumerates every state path s_0 .. s_{T-1} of the shift-register trellis
 * (s_t = ((s_{t-1} << 1) | c_t) mod S, with s_0 restricted by `init` as in tcq_viterbi.cu:314-321
 * and s_{T-1} == init when `tail`, tcq_viterbi.cu:564), and for each path takes, per sub-block,
 * the best gain and, per pair / group, the best admissible low-bit pattern:
 *   pp = 0: none; pp = 1 (D2): both low bits of a pair equal; pp = 2 (D4): even sum over a group
 *   of 4; pp = 3 (EQ): all 4 equal (tcq_proto.py:575-579 docstring, ltq_format.py:171-174).
 * Branch metrics are the same fp32 values the Viterbi uses; path costs are summed in double, so the
 * result is the true optimum of the problem the Viterbi solves -- a different computation from the
 * DP recursion, not a retyping of it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline int bpar(uint32_t v) { return __builtin_popcount(v) & 1; }

static int lab(int s, int m, int m2, int m3, int m4, int nl)
{
    int lb = (bpar((uint32_t)((s >> 1) & m)) << 1) | (s & 1);
    if (nl >= 8) lb |= bpar((uint32_t)((s >> 1) & m2)) << 2;
    if (nl >= 16) lb |= bpar((uint32_t)((s >> 1) & m3)) << 3;
    if (nl >= 32) lb |= bpar((uint32_t)((s >> 1) & m4)) << 4;
    return lb;
}

typedef struct {
    int T, S, G, sub, nl, pp, init, tail;
    const float* E;     /* [T][G][nl][2] fp32 metrics (parity class 0 only when pp == 0) */
    int labs[1024];
    int st[64];
    double best;
    int best_st[64];
} BF;

#define EM(t, g, l, p) b->E[((((size_t)(t) * b->G + (g)) * b->nl + (l)) * 2) + (p)]

/* cost of the unit ending at position t (a position, a pair or a group) for gain g, and the best low bits */
static double unit_cost(const BF* b, int t, int g, int* lowbits)
{
    if (b->pp == 0) {
        if (lowbits) lowbits[0] = 0;
        return EM(t, g, b->labs[b->st[t]], 0);
    }
    if (b->pp == 1) {
        double best = INFINITY;
        for (int p = 0; p < 2; p++) {
            double v = (double)EM(t - 1, g, b->labs[b->st[t - 1]], p) + (double)EM(t, g, b->labs[b->st[t]], p);
            if (v < best) { best = v; if (lowbits) lowbits[0] = lowbits[1] = p; }
        }
        return best;
    }
    double best = INFINITY;
    for (int pat = 0; pat < 16; pat++) {
        const int b0 = pat & 1, b1 = (pat >> 1) & 1, b2 = (pat >> 2) & 1, b3 = (pat >> 3) & 1;
        if (b->pp == 2 && ((b0 + b1 + b2 + b3) & 1)) continue;
        if (b->pp == 3 && !(b0 == b1 && b1 == b2 && b2 == b3)) continue;
        double v = 0.0;
        const int bits[4] = {b0, b1, b2, b3};
        for (int i = 0; i < 4; i++) v += (double)EM(t - 3 + i, g, b->labs[b->st[t - 3 + i]], bits[i]);
        if (v < best) {
            best = v;
            if (lowbits) for (int i = 0; i < 4; i++) lowbits[i] = bits[i];
        }
    }
    return best;
}

static int unit_end(const BF* b, int t)
{
    if (b->pp == 0) return 1;
    if (b->pp == 1) return t & 1;
    return (t & 3) == 3;
}

/* total cost of the current full path: sum over sub-blocks of the min over gains */
static double path_cost(const BF* b)
{
    double total = 0.0;
    for (int j = 0; j < b->T / b->sub; j++) {
        double bj = INFINITY;
        for (int g = 0; g < b->G; g++) {
            double v = 0.0;
            for (int t = j * b->sub; t < (j + 1) * b->sub; t++)
                if (unit_end(b, t)) v += unit_cost(b, t, g, NULL);
            if (v < bj) bj = v;
        }
        total += bj;
    }
    return total;
}

static void dfs(BF* b, int t)
{
    if (t == b->T) {
        if (b->tail && b->st[b->T - 1] != b->init) return;
        const double c = path_cost(b);
        if (c < b->best) { b->best = c; memcpy(b->best_st, b->st, sizeof(int) * b->T); }
        return;
    }
    for (int c = 0; c < 2; c++) {
        b->st[t] = ((b->st[t - 1] << 1) | c) & (b->S - 1);
        dfs(b, t + 1);
    }
}

/* Returns the optimal cost; writes the optimal states, the per-sub-block best gain and the low bits. */
double ltq_brute_force(const float* E, int T, int S, int G, int sub, int m, int m2, int m3, int m4, int nl, int pp,
                       int init, int tail, int* out_states, int* out_g, int* out_low)
{
    BF* b = (BF*)calloc(1, sizeof(BF));
    b->T = T; b->S = S; b->G = G; b->sub = sub; b->nl = nl; b->pp = pp; b->init = init; b->tail = tail; b->E = E;
    for (int s = 0; s < S; s++) b->labs[s] = lab(s, m, m2, m3, m4, nl);
    b->best = INFINITY;
    for (int s = 0; s < S; s++) {
        if (init >= 0 && (s >> 1) != (init & (S / 2 - 1))) continue;
        b->st[0] = s;
        dfs(b, 1);
    }
    const double best = b->best;
    memcpy(b->st, b->best_st, sizeof(int) * T);
    for (int t = 0; t < T; t++) out_states[t] = b->st[t];
    for (int j = 0; j < T / sub; j++) {
        double bj = INFINITY;
        int bg = 0;
        for (int g = 0; g < G; g++) {
            double v = 0.0;
            for (int t = j * sub; t < (j + 1) * sub; t++)
                if (unit_end(b, t)) v += unit_cost(b, t, g, NULL);
            if (v < bj) { bj = v; bg = g; }
        }
        out_g[j] = bg;
        for (int t = j * sub; t < (j + 1) * sub; t++)
            if (unit_end(b, t)) {
                int lowb[4] = {0, 0, 0, 0};
                unit_cost(b, t, bg, lowb);
                const int w = pp == 0 ? 1 : (pp == 1 ? 2 : 4);
                for (int i = 0; i < w; i++) out_low[t - w + 1 + i] = lowb[i];
            }
    }
    free(b);
    return best;
}
