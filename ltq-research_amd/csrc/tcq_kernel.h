// Portable body of the MI355X TCQ Viterbi kernel (one workgroup per 256-weight tile).
//
// The same source is compiled two ways:
//   - for gfx950 by tcq_viterbi.hip (X = GpuX: threadIdx, __syncthreads, LDS, v_addc decision packing);
//   - for the host by the CPU emulation used in tests (X = CpuX: one std::thread per lane, barriers),
//     so layout / indexing bugs show up on the CPU, under AddressSanitizer, before any GPU run.
//
// Semantics follow the reference kernel (src/cuda/tcq_viterbi.cu:97-683): Ungerboeck trellis with
// S = 2^NU states, predecessors p_h = h*S/2 + (s >> 1), labels from parities of (s >> 1) & masks, a gain
// slot per wavefront, sub-block gain merge, integer / D2 (pp=1) / D4 (pp=2) / EQ (pp=3) parity modes,
// gain candidates, free / given start, tail-biting end, mid-state pass, cyclic shift, traceback and
// reconstruction. Ties: strict "<" everywhere, predecessor p0, lowest gain slot, lowest (g, s) index,
// lowest class / low bit, lowest u -- identical choices to the reference given identical fp32 inputs.
//
// MI355X mapping (see DESIGN.md for the derivation):
//   - wavefront w of the workgroup owns gain slot g = w and all S states of that slot: R = S/64 path
//     metrics per lane in VGPRs. No cross-wave traffic except at sub-block gain merges.
//   - a "group" = RB = log2(R) trellis steps done entirely in registers: each step is an in-place
//     butterfly between two register slots. The logical state of (slot r, lane l) after k steps of the
//     group is Lay::state(k, r, l); after RB steps the lane / slot roles of the state bits are
//     exchanged through LDS (one write + one read per metric per group).
//   - a group is two 2-step "phases" (radix-4 blocks of 4 slots), which is exactly a D4 group (phase A,
//     phase B) and two D2 pairs.
//   - branch metrics: per group each wave builds a compact table E[k][label][parity] and expands it to
//     one row per lane class (label bits carried by the lane part of the state), so that a lane reads its
//     R x NP metrics for a step with 128-bit LDS loads at compile-time offsets.
//   - decisions: one bit per lane per compare, pushed into 32-bit words with v_addc (acc = 2 acc + bit),
//     stored per group with coalesced writes into the caller's bp / pbits scratch.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifndef LTQ_DEV
#define LTQ_DEV __device__ __forceinline__
#endif
#ifndef LTQ_HD
#define LTQ_HD __host__ __device__ __forceinline__
#endif

namespace ltq {

constexpr float kSent = 3.4e38f;
constexpr int kMaxG = 16, kMaxU = 128, kMaxSubs = 32, kMaxT = 512;

// Arguments of the reference C ABI tcq_viterbi (tcq_viterbi.cu:743-746), same meaning.
struct TcqArgs {
    const float* x;        // [N, ld]
    const float* w;        // [N, ld]
    const float* tab;      // [nl * U]
    const float* gains;    // [Gfull]
    float* rec;            // [N, ld]
    uint32_t* bp;          // scratch (caller-allocated, reference size [N, T, G, S/32] u32)
    uint8_t* gsel;         // scratch, unused here (gain-merge choices stay in LDS)
    const int* init_st;    // [N] or null
    int* end_st;           // [N] or null
    const float* tab_hi;   // [nl * U_hi]
    const float* gains_hi; // [Gfull]
    uint8_t* gcand;        // [N, T/sub, G] or null
    int* best;             // [N]
    int* code;             // [N, ld] or null
    int* mid_st;           // [N] or null
    int mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot;
    uint32_t* pbits;       // scratch (reference size [N, T/2, G, S/32] for pp=1, [N, T/4, G, 9, S/32] for pp>=2)
    int pp;
};

LTQ_DEV int parity32(uint32_t v)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_popcount(v) & 1;
#else
    return __builtin_popcount(v) & 1;
#endif
}

// label of state s: (s & 1) | par((s>>1)&m) << 1 | par((s>>1)&m2) << 2 | ... (tcq_viterbi.cu:85-95)
struct Masks {
    int m, m2, m3, m4, nl;
    LTQ_DEV int label(int s) const
    {
        int lb = (parity32((uint32_t)((s >> 1) & m)) << 1) | (s & 1);
        if (nl >= 8) lb |= parity32((uint32_t)((s >> 1) & m2)) << 2;
        if (nl >= 16) lb |= parity32((uint32_t)((s >> 1) & m3)) << 3;
        if (nl >= 32) lb |= parity32((uint32_t)((s >> 1) & m4)) << 4;
        return lb;
    }
};

// Register layout of one wavefront's S = 2^NU states.
template <int NU>
struct Lay {
    static constexpr int RB = NU - 6, R = 1 << RB, S = 1 << NU, HALF = S / 2;
    // state held by (slot r, lane l) after k in-register steps of a group (0 <= k <= RB): the k newest code
    // bits sit in the top k bits of r (oldest highest), the remaining RB-k slot bits and the lane bits are
    // the older state bits.
    static LTQ_DEV int state(int k, int r, int l)
    {
        const int rlow = r & ((1 << (RB - k)) - 1);
        return (((rlow << 6) | l) << k) | (r >> (RB - k));
    }
    static LTQ_DEV int slot(int k, int s) { return ((s & ((1 << k) - 1)) << (RB - k)) | (s >> (k + 6)); }
    static LTQ_DEV int lane(int k, int s) { return (s >> k) & 63; }
};

// Decision-word layout per parity mode (MD: 0 integer, 1 D2, 2 D4, 3 EQ).
// Per phase ph (2 steps on slot bits hb = RB-1-2ph and lb = hb-1), R/4 blocks of 4 slots; per block two
// step-a butterflies (PA pushes each) then two step-b butterflies (PB pushes each).
template <int NU, int MD>
struct Mode {
    static constexpr int RB = NU - 6, R = 1 << RB, NPH = RB / 2, NB = R / 4;
    static constexpr int NP = MD ? 2 : 1;
    static constexpr int PA(int ph) { return (MD >= 2 && ph == 1) ? 2 : 1; }
    static constexpr int PB(int ph)
    {
        return MD == 0 ? 1 : MD == 1 ? 4 : MD == 2 ? (ph == 0 ? 6 : 10) : (ph == 0 ? 2 : 4);
    }
    static constexpr int PBLK(int ph) { return 2 * (PA(ph) + PB(ph)); }
    static constexpr int PPH(int ph) { return NB * PBLK(ph); }
    static constexpr int BASE(int ph) { return ph == 0 ? 0 : PPH(0); }
    static constexpr int PG = PPH(0) + (NPH > 1 ? PPH(1) : 0);     // pushes per group
    static constexpr int FG = PG >= 32 ? 1 : 32 / PG;              // groups per stored chunk
    static constexpr int NW = (FG * PG + 31) / 32;                  // words per lane per chunk
    static constexpr int WB = NW < 2 ? NW : 2;                      // words of a chunk kept in bp (rest: pbits)
    // bit position of push P (within a chunk) inside its word
    static LTQ_DEV int word_of(int P) { return P >> 5; }
    static LTQ_DEV int bit_of(int P)
    {
        const int w = P >> 5;
        const int nb = (FG * PG - 32 * w) < 32 ? (FG * PG - 32 * w) : 32;
        return nb - 1 - (P & 31);
    }
};

// dynamic LDS layout (byte offsets), identical on host (launch size) and device
struct Smem {
    int x, w, tab, tab_hi, gain, gain_hi, gc, ce, lbr, exch, tabs, gsel, st, g, par, red_v, red_i, ctl, total;
    int tabs_per_wave;  // floats
    int ec_floats;      // compact part of a wave's tables
};

LTQ_HD int align16(int v) { return (v + 15) & ~15; }

template <int NU, int MD>
LTQ_HD Smem smem_layout(int T, int G, int nl, int Gfull, int sub)
{
    using M = Mode<NU, MD>;
    constexpr int R = Lay<NU>::R, S = Lay<NU>::S, RB = Lay<NU>::RB, NP = M::NP;
    Smem L;
    int o = 0;
    L.x = o; o = align16(o + 4 * T);
    L.w = o; o = align16(o + 4 * T);
    L.tab = o; o = align16(o + 4 * 4 * kMaxU);
    L.tab_hi = o; o = align16(o + 4 * 4 * kMaxU);
    L.gain = o; o = align16(o + 4 * kMaxG);
    L.gain_hi = o; o = align16(o + 4 * kMaxG);
    L.gc = o; o = align16(o + kMaxSubs * kMaxG);
    L.ce = o; o = align16(o + 4 * kMaxSubs * kMaxG);
    L.lbr = o; o = align16(o + 4 * RB * R);
    L.ec_floats = align16(4 * RB * nl * NP) / 4;
    L.tabs_per_wave = L.ec_floats + RB * (nl / 2) * R * NP;
    L.exch = o; o = align16(o + 4 * G * S);
    L.tabs = o; o = align16(o + 4 * G * L.tabs_per_wave);
    L.gsel = o; o = align16(o + (T / sub) * S);
    L.st = o; o = align16(o + 2 * T);
    L.g = o; o = align16(o + T);
    L.par = o; o = align16(o + T + 4);
    L.red_v = o; o = align16(o + 4 * 64 * G);
    L.red_i = o; o = align16(o + 4 * 64 * G);
    L.ctl = o; o = align16(o + 4 * 8);
    L.total = o;
    return L;
}

// bytes of decision words one traceback window stages (reuses the exch + tabs region)
template <int NU, int MD>
constexpr int stage_chunks()
{
    return Mode<NU, MD>::FG == 1 ? 4 : 1;
}

LTQ_DEV int exch_index(int s) { return s ^ (((s >> 5) & 3) << 2); }

// squared-error minimum over levels u0, u0+du, ... < Ut of fl(x - fl(g * tab[u]))^2 (tcq_viterbi.cu:46-54, 75-83)
LTQ_DEV float level_err(float xt, float gain, const float* tb, int u0, int Ut, int du)
{
    float e = kSent;
    for (int u = u0; u < Ut; u += du) {
        const float v = gain * tb[u];
        const float d = xt - v;
        const float dd = d * d;
        e = dd < e ? dd : e;
    }
    return e;
}

// pointer to decision word w of (chunk c, gain slot g) of tile n (64 consecutive u32, one per lane)
template <int NU, int MD>
LTQ_DEV uint32_t* dec_words(const TcqArgs& a, int n, int c, int g, int w)
{
    using M = Mode<NU, MD>;
    constexpr int S = Lay<NU>::S;
    const int G = a.G;
    if (w < M::WB) {
        uint32_t* base = a.bp + (size_t)n * a.T * G * (S / 32);
        return base + ((size_t)(c * G + g) * M::WB + w) * 64;
    }
    const size_t per_tile = MD == 1 ? (size_t)(a.T / 2) * G * (S / 32) : (size_t)(a.T / 4) * G * 9 * (S / 32);
    uint32_t* base = a.pbits + (size_t)n * per_tile;
    return base + ((size_t)(c * G + g) * (M::NW - M::WB) + (w - M::WB)) * 64;
}

// ------------------------------------------------------------------------------------------------
// One 2-step phase of a group, all in registers. PH = phase index in the group (steps 2PH, 2PH+1 on
// slot bits HB = RB-1-2PH and LB = HB-1). Blocks of 4 slots {x, x|L, x|H, x|H|L}; local index j = 2*hbit + lbit.
// Step a (bit HB): butterflies (j=e, j=2+e); step b (bit LB): butterflies (j=2f, j=2f+1). The output with new
// code bit c of a butterfly goes to the slot whose butterfly bit is c.
// ------------------------------------------------------------------------------------------------
template <int NU, int MD, int PH, class X>
LTQ_DEV void run_phase(bool init, int s0, int lane, float (&D)[Lay<NU>::R], float* C0, float* C1, const float* Ma,
                       const float* Mb, uint32_t* acc, X& X_)
{
    using LY = Lay<NU>;
    using M = Mode<NU, MD>;
    constexpr int R = LY::R, RB = LY::RB, NB = R / 4, NP = M::NP;
    constexpr int HB = RB - 1 - 2 * PH, LB = HB - 1, H = 1 << HB, L = 1 << LB;
    constexpr int PA = M::PA(PH), PB = M::PB(PH), PBLK = M::PBLK(PH), BASE = M::BASE(PH);
    constexpr bool EQ = MD == 3;
    (void)NP;
#define LTQ_PUSH(P, bit) acc[(P) >> 5] = X_.push(acc[(P) >> 5], (bit))
#pragma unroll
    for (int be = 0; be < NB; be++) {
        const int x = ((be >> LB) << (HB + 1)) | (be & (L - 1));
        int sl[4];
#pragma unroll
        for (int j = 0; j < 4; j++) sl[j] = x | ((j >> 1) ? H : 0) | ((j & 1) ? L : 0);
        const int P0 = BASE + be * PBLK;
        if constexpr (MD == 0) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j0 = e, j1 = 2 + e;
                if (init) {
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int jj = q ? j1 : j0;
                        const int s = LY::state(1, sl[jj], lane);
                        const bool ok = s0 < 0 || (s >> 1) == (s0 & (LY::HALF - 1));
                        v[jj] = ok ? Ma[sl[jj]] : kSent;
                    }
                    LTQ_PUSH(P0 + e, false);
                } else {
                    const float va = D[sl[j0]], vb = D[sl[j1]];
                    const bool h = vb < va;
                    const float m = h ? vb : va;
                    LTQ_PUSH(P0 + e, h);
                    v[j0] = m + Ma[sl[j0]];
                    v[j1] = m + Ma[sl[j1]];
                }
            }
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const int j0 = 2 * f, j1 = 2 * f + 1;
                const float va = v[j0], vb = v[j1];
                const bool h = vb < va;
                const float m = h ? vb : va;
                LTQ_PUSH(P0 + 2 + f, h);
                D[sl[j0]] = m + Mb[sl[j0]];
                D[sl[j1]] = m + Mb[sl[j1]];
            }
        } else if constexpr (MD == 1 || PH == 0) {
            // D2 pair, or phase A of a D4 / EQ group: intermediates per low bit b of the first sample
            float I0[4], I1[4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j0 = e, j1 = 2 + e;
                if (init) {
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int jj = q ? j1 : j0;
                        const int s = LY::state(1, sl[jj], lane);
                        const bool ok = s0 < 0 || (s >> 1) == (s0 & (LY::HALF - 1));
                        I0[jj] = ok ? Ma[sl[jj] * 2 + 0] : kSent;
                        I1[jj] = ok ? Ma[sl[jj] * 2 + 1] : kSent;
                    }
                    LTQ_PUSH(P0 + e, false);
                } else {
                    const float va = D[sl[j0]], vb = D[sl[j1]];
                    const bool h = vb < va;
                    const float m = h ? vb : va;
                    LTQ_PUSH(P0 + e, h);
                    I0[j0] = m + Ma[sl[j0] * 2 + 0];
                    I1[j0] = m + Ma[sl[j0] * 2 + 1];
                    I0[j1] = m + Ma[sl[j1] * 2 + 0];
                    I1[j1] = m + Ma[sl[j1] * 2 + 1];
                }
            }
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 2 * PA + f * PB;
                const bool h0 = I0[j1] < I0[j0];
                const float m0 = h0 ? I0[j1] : I0[j0];
                const bool h1 = I1[j1] < I1[j0];
                const float m1 = h1 ? I1[j1] : I1[j0];
                LTQ_PUSH(PF + 0, h0);
                LTQ_PUSH(PF + 1, h1);
                if constexpr (MD == 1) {  // D2: best class p of the pair (ties: p = 0)
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int r = sl[q ? j1 : j0];
                        const float v0 = m0 + Mb[r * 2 + 0], v1 = m1 + Mb[r * 2 + 1];
                        const bool sel = v1 < v0;
                        D[r] = sel ? v1 : v0;
                        LTQ_PUSH(PF + 2 + q, sel);
                    }
                } else if constexpr (!EQ) {  // D4 phase A: per class c the best b (ties: b = 0), parity b ^ c
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int r = sl[q ? j1 : j0];
                        {
                            const float v0 = m0 + Mb[r * 2 + 0], v1 = m1 + Mb[r * 2 + 1];
                            const bool sel = v1 < v0;
                            C0[r] = sel ? v1 : v0;
                            LTQ_PUSH(PF + 2 + 2 * q + 0, sel);
                        }
                        {
                            const float v0 = m0 + Mb[r * 2 + 1], v1 = m1 + Mb[r * 2 + 0];
                            const bool sel = v1 < v0;
                            C1[r] = sel ? v1 : v0;
                            LTQ_PUSH(PF + 2 + 2 * q + 1, sel);
                        }
                    }
                } else {  // EQ phase A: class c keeps b = c
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int r = sl[q ? j1 : j0];
                        C0[r] = m0 + Mb[r * 2 + 0];
                        C1[r] = m1 + Mb[r * 2 + 1];
                    }
                }
            }
        } else if constexpr (!EQ) {
            // D4 phase B: J[c][b] = min over predecessors of C_c + E(b); output = best (c, b) in order 00,01,10,11
            float J[4][4];  // [2c+b][j]
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j0 = e, j1 = 2 + e;
                const bool hc0 = C0[sl[j1]] < C0[sl[j0]];
                const float mc0 = hc0 ? C0[sl[j1]] : C0[sl[j0]];
                const bool hc1 = C1[sl[j1]] < C1[sl[j0]];
                const float mc1 = hc1 ? C1[sl[j1]] : C1[sl[j0]];
                LTQ_PUSH(P0 + e * PA + 0, hc0);
                LTQ_PUSH(P0 + e * PA + 1, hc1);
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int jj = q ? j1 : j0, r = sl[jj];
                    J[0][jj] = mc0 + Ma[r * 2 + 0];
                    J[1][jj] = mc0 + Ma[r * 2 + 1];
                    J[2][jj] = mc1 + Ma[r * 2 + 0];
                    J[3][jj] = mc1 + Ma[r * 2 + 1];
                }
            }
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 2 * PA + f * PB;
                float mm[4];
#pragma unroll
                for (int cb = 0; cb < 4; cb++) {
                    const bool h = J[cb][j1] < J[cb][j0];
                    mm[cb] = h ? J[cb][j1] : J[cb][j0];
                    LTQ_PUSH(PF + cb, h);
                }
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int r = sl[q ? j1 : j0];
                    float v = mm[0] + Mb[r * 2 + 0];
                    const float w1 = mm[1] + Mb[r * 2 + 1];
                    const bool s1 = w1 < v;
                    v = s1 ? w1 : v;
                    LTQ_PUSH(PF + 4 + 3 * q + 0, s1);
                    const float w2 = mm[2] + Mb[r * 2 + 1];
                    const bool s2 = w2 < v;
                    v = s2 ? w2 : v;
                    LTQ_PUSH(PF + 4 + 3 * q + 1, s2);
                    const float w3 = mm[3] + Mb[r * 2 + 0];
                    const bool s3 = w3 < v;
                    v = s3 ? w3 : v;
                    LTQ_PUSH(PF + 4 + 3 * q + 2, s3);
                    D[r] = v;
                }
            }
        } else {
            // EQ phase B: classes keep b = c; output = best class (ties: c = 0)
            float Jc[2][4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j0 = e, j1 = 2 + e;
                const bool hc0 = C0[sl[j1]] < C0[sl[j0]];
                const float mc0 = hc0 ? C0[sl[j1]] : C0[sl[j0]];
                const bool hc1 = C1[sl[j1]] < C1[sl[j0]];
                const float mc1 = hc1 ? C1[sl[j1]] : C1[sl[j0]];
                LTQ_PUSH(P0 + e * PA + 0, hc0);
                LTQ_PUSH(P0 + e * PA + 1, hc1);
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int jj = q ? j1 : j0, r = sl[jj];
                    Jc[0][jj] = mc0 + Ma[r * 2 + 0];
                    Jc[1][jj] = mc1 + Ma[r * 2 + 1];
                }
            }
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 2 * PA + f * PB;
                const bool h0 = Jc[0][j1] < Jc[0][j0];
                const float m0 = h0 ? Jc[0][j1] : Jc[0][j0];
                const bool h1 = Jc[1][j1] < Jc[1][j0];
                const float m1 = h1 ? Jc[1][j1] : Jc[1][j0];
                LTQ_PUSH(PF + 0, h0);
                LTQ_PUSH(PF + 1, h1);
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int r = sl[q ? j1 : j0];
                    const float v0 = m0 + Mb[r * 2 + 0], v1 = m1 + Mb[r * 2 + 1];
                    const bool sel = v1 < v0;
                    D[r] = sel ? v1 : v0;
                    LTQ_PUSH(PF + 2 + q, sel);
                }
            }
        }
    }
#undef LTQ_PUSH
}

// zero pushes for a phase that lies beyond the tile end (keeps every decision bit at its fixed position)
template <int NU, int MD, int PH, class X>
LTQ_DEV void pad_phase(uint32_t* acc, X& X_)
{
    using M = Mode<NU, MD>;
#pragma unroll
    for (int i = 0; i < M::PPH(PH); i++) {
        const int P = M::BASE(PH) + i;
        acc[P >> 5] = X_.push(acc[P >> 5], false);
    }
}

// ------------------------------------------------------------------------------------------------
// The per-tile kernel body.
// ------------------------------------------------------------------------------------------------
template <int NU, int MD, class X>
LTQ_DEV void tcq_tile(const TcqArgs& a, X& X_)
{
    using LY = Lay<NU>;
    using M = Mode<NU, MD>;
    constexpr int RB = LY::RB, R = LY::R, S = LY::S, NP = M::NP, NW = M::NW, FG = M::FG;
    constexpr bool G4 = MD >= 2, EQ = MD == 3;

    const int n = X_.tile(), tid = X_.tid(), nthr = X_.nthreads();
    const int lane = tid & 63, g = tid >> 6;
    const int T = a.T, G = a.G, sub = a.sub, nl = a.nl, U = a.U, U_hi = a.U_hi, mix = MD ? 0 : a.mix;
    const int nl2 = nl >> 1, Gf = a.Gfull, nsub = T / sub;
    const bool cand = a.gcand != nullptr;
    const Masks mk{a.m, a.m2, a.m3, a.m4, nl};
    const Smem SM = smem_layout<NU, MD>(T, G, nl, Gf, sub);
    char* sm = (char*)X_.smem();
    float* s_x = (float*)(sm + SM.x);
    float* s_w = (float*)(sm + SM.w);
    float* s_tab = (float*)(sm + SM.tab);
    float* s_tab_hi = (float*)(sm + SM.tab_hi);
    float* s_gain = (float*)(sm + SM.gain);
    float* s_gain_hi = (float*)(sm + SM.gain_hi);
    uint8_t* s_gc = (uint8_t*)(sm + SM.gc);
    float* s_ce = (float*)(sm + SM.ce);
    float* s_exch = (float*)(sm + SM.exch);
    float* s_tabs = (float*)(sm + SM.tabs) + (size_t)g * SM.tabs_per_wave;
    float* s_ec = s_tabs;
    float* s_ex = s_tabs + SM.ec_floats;
    uint8_t* s_gsel = (uint8_t*)(sm + SM.gsel);
    uint16_t* s_st = (uint16_t*)(sm + SM.st);
    uint8_t* s_g = (uint8_t*)(sm + SM.g);
    uint8_t* s_par = (uint8_t*)(sm + SM.par);
    float* s_rv = (float*)(sm + SM.red_v);
    int* s_ri = (int*)(sm + SM.red_i);
    int* s_ctl = (int*)(sm + SM.ctl);

    // ---- tile load (tcq_viterbi.cu:133-140) -----------------------------------------------------
    for (int i = tid; i < T; i += nthr) {
        const size_t j = (size_t)n * a.ld + (size_t)((i + a.rot) % a.ld);
        s_x[i] = a.x[j];
        s_w[i] = a.w[j];
    }
    for (int i = tid; i < nl * U; i += nthr) s_tab[i] = a.tab[i];
    for (int i = tid; i < nl * U_hi; i += nthr) s_tab_hi[i] = a.tab_hi[i];
    if (tid < Gf) {
        s_gain[tid] = a.gains[tid];
        s_gain_hi[tid] = a.gains_hi[tid];
    }
    const int s0 = a.init_st ? a.init_st[n] : -1;
    X_.sync();

    // ---- gain candidates: the G gains of lowest scalar error per sub-block (tcq_viterbi.cu:155-180) ----
    if (cand) {
        for (int i = tid; i < nsub * Gf; i += nthr) {
            const int j = i / Gf, gi = i % Gf;
            float e = 0.f;
            for (int t = j * sub; t < (j + 1) * sub; t++) {
                const bool hi = mix > 0 && ((t / mix) & 1);
                const float be = hi ? level_err(s_x[t], s_gain_hi[gi], s_tab_hi, 0, nl * U_hi, 1)
                                    : level_err(s_x[t], s_gain[gi], s_tab, 0, nl * U, 1);
                const float prod = be * s_w[t];
                e = e + prod;
            }
            s_ce[i] = e;
        }
        X_.sync();
        if (tid < nsub) {
            uint32_t used = 0;
            for (int c = 0; c < G; c++) {
                int bg = 0;
                float be = kSent;
                for (int gi = 0; gi < Gf; gi++)
                    if (!((used >> gi) & 1) && s_ce[tid * Gf + gi] < be) {
                        be = s_ce[tid * Gf + gi];
                        bg = gi;
                    }
                used |= 1u << bg;
                s_gc[tid * G + c] = (uint8_t)bg;
                a.gcand[((size_t)n * nsub + tid) * G + c] = (uint8_t)bg;
            }
        }
        X_.sync();
    }

    // ---- per-lane layout constants ----------------------------------------------------------------
    // row of the expanded metric table this lane reads at step k: label bits of the lane part of its states
    int rowk[RB];
    // fixed (slot, parity) this lane fills in table expansions, and that slot's label offset per step
    constexpr int RP = R * NP, LG = 64 / RP;
    const int re = (lane % RP) / NP, pe = lane % NP, rsub = lane / RP;
    int lbr[RB];
#pragma unroll
    for (int k = 0; k < RB; k++) {
        rowk[k] = mk.label(LY::state(k + 1, 0, lane)) >> 1;
        lbr[k] = mk.label(LY::state(k + 1, re, 0));
    }

    float D[R];
    uint32_t acc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) acc[w] = 0;
    float C0[G4 ? R : 1], C1[G4 ? R : 1];

    const int NG = (T + RB - 1) / RB;
    for (int gr = 0; gr < NG; gr++) {
        const int tb = gr * RB;
        // ---- exchange into the group-start layout (+ gain merge at a sub-block boundary) --------------
        if (gr > 0) {
            const bool merge = G > 1 && (tb % sub) == 0;
#pragma unroll
            for (int r = 0; r < R; r++) s_exch[g * S + exch_index(LY::state(RB, r, lane))] = D[r];
            if (merge) X_.sync();
            else X_.wave_sync();
            if (!merge) {
#pragma unroll
                for (int r = 0; r < R; r++) D[r] = s_exch[g * S + exch_index(LY::state(0, r, lane))];
            } else {
                const int j = tb / sub;
#pragma unroll
                for (int r = 0; r < R; r++) {
                    const int s = LY::state(0, r, lane);
                    float bv = s_exch[exch_index(s)];
                    int bg = 0;
                    for (int gg = 1; gg < G; gg++) {
                        const float v = s_exch[gg * S + exch_index(s)];
                        if (v < bv) { bv = v; bg = gg; }
                    }
                    D[r] = bv;
                    if (g == 0) s_gsel[j * S + s] = (uint8_t)bg;
                }
            }
            if (merge) X_.sync();
            else X_.wave_sync();
        }
        // ---- metric tables of the group's steps (wave-local) --------------------------------------------
        {
            const int ne = RB * nl * NP;
            for (int e = lane; e < ne; e += 64) {
                const int k = e / (nl * NP), rem = e % (nl * NP), lb = rem / NP, p = rem % NP;
                const int t = tb + k;
                float E = 0.f;
                if (t < T) {
                    const int gi = cand ? (int)s_gc[(t / sub) * G + g] : g;
                    const bool hi = mix > 0 && ((t / mix) & 1);
                    float be;
                    if (MD) be = level_err(s_x[t], s_gain[gi], s_tab + lb * U, p, U, 2);
                    else if (hi) be = level_err(s_x[t], s_gain_hi[gi], s_tab_hi + lb * U_hi, 0, U_hi, 1);
                    else be = level_err(s_x[t], s_gain[gi], s_tab + lb * U, 0, U, 1);
                    E = be * s_w[t];
                }
                s_ec[e] = E;
            }
            X_.wave_sync();
#pragma unroll
            for (int k = 0; k < RB; k++)
                for (int row = rsub; row < nl2; row += LG)
                    s_ex[((k * nl2 + row) * R + re) * NP + pe] = s_ec[(k * nl + ((row << 1) ^ lbr[k])) * NP + pe];
            X_.wave_sync();
        }
        // ---- the group's phases ------------------------------------------------------------------------
#pragma unroll
        for (int ph = 0; ph < M::NPH; ph++) {
            const int ka = 2 * ph;
            const int ta = tb + ka;
            if (ta < T) {
                if (ph > 0 && G > 1 && (ta % sub) == 0) {  // sub-block boundary inside a group (sub % 4 == 2)
                    const int j = ta / sub;
#pragma unroll
                    for (int r = 0; r < R; r++) s_exch[g * S + exch_index(LY::state(ka, r, lane))] = D[r];
                    X_.sync();
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const int s = LY::state(ka, r, lane);
                        float bv = s_exch[exch_index(s)];
                        int bg = 0;
                        for (int gg = 1; gg < G; gg++) {
                            const float v = s_exch[gg * S + exch_index(s)];
                            if (v < bv) { bv = v; bg = gg; }
                        }
                        D[r] = bv;
                        if (g == 0) s_gsel[j * S + s] = (uint8_t)bg;
                    }
                    X_.sync();
                }
                float Ma[R * NP], Mb[R * NP];
                const float* pa = s_ex + (ka * nl2 + rowk[ka]) * RP;
                const float* pb = s_ex + ((ka + 1) * nl2 + rowk[ka + 1]) * RP;
#pragma unroll
                for (int i = 0; i < R * NP; i++) {
                    Ma[i] = pa[i];
                    Mb[i] = pb[i];
                }
                const bool init = ta == 0;
                if (ph == 0) run_phase<NU, MD, 0>(init, s0, lane, D, C0, C1, Ma, Mb, acc, X_);
                else if constexpr (M::NPH > 1) run_phase<NU, MD, M::NPH - 1>(init, s0, lane, D, C0, C1, Ma, Mb, acc, X_);
            } else {
                if (ph == 0) pad_phase<NU, MD, 0>(acc, X_);
                else if constexpr (M::NPH > 1) pad_phase<NU, MD, M::NPH - 1>(acc, X_);
            }
        }
        // ---- store the chunk's decision words -----------------------------------------------------------
        if ((gr % FG) == FG - 1 || gr == NG - 1) {
            const int have = gr % FG + 1;
            if (have < FG) {
                const int miss = (FG - have) * M::PG;  // pad missing groups (only FG > 1, single word)
#pragma unroll
                for (int w = 0; w < NW; w++) acc[w] = miss >= 32 ? 0u : (acc[w] << miss);
            }
            const int c = gr / FG;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                dec_words<NU, MD>(a, n, c, g, w)[lane] = acc[w];
                acc[w] = 0;
            }
        }
    }

    // ---- argmin over (g, s), lowest index on ties (tcq_viterbi.cu:561-578) ---------------------------
    {
        const int kf = ((T - 1) % RB) + 1;
        const int s_end = a.tail ? s0 : -1;
        float bv = kSent;
        int bi = 0x7fffffff;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int s = LY::state(kf, r, lane);
            const int idx = g * S + s;
            const float v = (s_end < 0 || s == s_end) ? D[r] : kSent;
            if (v < bv || (v == bv && idx < bi)) { bv = v; bi = idx; }
        }
        s_rv[tid] = bv;
        s_ri[tid] = bi;
        X_.sync();
        for (int off = 1; off < nthr; off <<= 1) {
            float ov = 0.f;
            int oi = 0;
            const bool act = (tid % (2 * off)) == 0 && tid + off < nthr;
            if (act) {
                ov = s_rv[tid + off];
                oi = s_ri[tid + off];
            }
            X_.sync();
            if (act) {
                const float cv = s_rv[tid];
                const int ci = s_ri[tid];
                if (ov < cv || (ov == cv && oi < ci)) {
                    s_rv[tid] = ov;
                    s_ri[tid] = oi;
                }
            }
            X_.sync();
        }
        if (tid == 0) {
            int b = s_ri[0];
            if (b == 0x7fffffff) b = 0;  // no candidate at or below the sentinel: the reference reads out of range
            a.best[n] = b;
            if (a.end_st) a.end_st[n] = b % S;
            s_ctl[0] = b % S;  // walker state
            s_ctl[1] = b / S;  // walker gain slot
            s_ctl[2] = 0;      // mid reached
            s_ctl[3] = T - 1;  // next position to walk
            s_ctl[4] = 0;      // class of the current D4 / EQ group
        }
        X_.sync();
    }

    // ---- traceback in windows of staged decision words (tcq_viterbi.cu:601-661) -----------------------
    {
        constexpr int WCH = stage_chunks<NU, MD>();
        uint32_t* stg = (uint32_t*)(sm + SM.exch);  // reuses the exchange + table region
        const int steps_per_chunk = FG * RB;
        const int c_last = (T - 1) / steps_per_chunk;
        for (int chi = c_last; chi >= 0; chi -= WCH) {
            const int clo = chi - WCH + 1 < 0 ? 0 : chi - WCH + 1;
            const int nch = chi - clo + 1;
            const int nwords = nch * G * NW * 64;
            for (int i = tid; i < nwords; i += nthr) {
                const int ln = i & 63, q = i >> 6;
                const int w = q % NW, gg = (q / NW) % G, cr = q / (NW * G);
                stg[i] = dec_words<NU, MD>(a, n, clo + cr, gg, w)[ln];
            }
            X_.sync();
            if (tid == 0) {
                int st = s_ctl[0], gs = s_ctl[1], t = s_ctl[3], cstar = s_ctl[4];
                const int t_lo = clo * steps_per_chunk;
                bool hit = false;
                for (; t >= t_lo; t--) {
                    s_st[t] = (uint16_t)st;
                    s_g[t] = (uint8_t)gs;
                    const int k = t % RB;
                    const int c = t / steps_per_chunk;
                    const int pc = ((t / RB) % FG) * M::PG;
                    const uint32_t* wb = stg + ((size_t)((c - clo) * G + gs) * NW) * 64;
                    const int ln = LY::lane(k + 1, st);
                    auto bit = [&](int P) -> int {
                        const int PP = pc + P;
                        return (int)((wb[M::word_of(PP) * 64 + ln] >> M::bit_of(PP)) & 1u);
                    };
                    const int r = LY::slot(k + 1, st);
                    const int ph = k >> 1, hb = RB - 1 - 2 * ph, lbt = hb - 1;
                    const int beta = ((r >> (hb + 1)) << lbt) | (r & ((1 << lbt) - 1));
                    const int cout = st & 1;
                    const bool stepb = k & 1;
                    const int pa = ph == 0 ? M::PA(0) : M::PA(1), pbb = ph == 0 ? M::PB(0) : M::PB(1);
                    const int base = (ph == 0 ? M::BASE(0) : M::BASE(1)) + beta * 2 * (pa + pbb) +
                                     (stepb ? 2 * pa + ((r >> hb) & 1) * pbb : ((r >> lbt) & 1) * pa);
                    int h = 0;
                    if (MD == 0) {
                        h = bit(base);
                    } else if (MD == 1) {
                        if (stepb) {
                            const int p = bit(base + 2 + cout);
                            h = bit(base + p);
                            s_par[t] = (uint8_t)p;
                            s_par[t - 1] = (uint8_t)p;
                        } else {
                            h = bit(base);
                        }
                    } else if (!EQ) {
                        if (k == 3) {
                            const int s1 = bit(base + 4 + 3 * cout), s2 = bit(base + 5 + 3 * cout),
                                      s3 = bit(base + 6 + 3 * cout);
                            const int idx = s3 ? 3 : s2 ? 2 : s1 ? 1 : 0;
                            cstar = idx >> 1;
                            const int b = idx & 1;
                            h = bit(base + idx);
                            s_par[t] = (uint8_t)(b ^ cstar);
                            s_par[t - 1] = (uint8_t)b;
                        } else if (k == 2) {
                            h = bit(base + cstar);
                        } else if (k == 1) {
                            const int b = bit(base + 2 + 2 * cout + cstar);
                            h = bit(base + b);
                            s_par[t] = (uint8_t)(b ^ cstar);
                            s_par[t - 1] = (uint8_t)b;
                        } else {
                            h = bit(base);
                        }
                    } else {
                        if (k == 3) {
                            cstar = bit(base + 2 + cout);
                            h = bit(base + cstar);
                            s_par[t] = s_par[t - 1] = s_par[t - 2] = s_par[t - 3] = (uint8_t)cstar;
                        } else if (k == 2 || k == 1) {
                            h = bit(base + cstar);
                        } else {
                            h = bit(base);
                        }
                    }
                    if (a.mid_st && t == a.mid_t - 1) {
                        a.mid_st[n] = st;
                        hit = true;
                        break;
                    }
                    if (t > 0) {
                        st = (h << (NU - 1)) | (st >> 1);
                        if (G > 1 && (t % sub) == 0) gs = s_gsel[(t / sub) * S + st];
                    }
                }
                s_ctl[0] = st;
                s_ctl[1] = gs;
                s_ctl[2] = hit ? 1 : 0;
                s_ctl[3] = t;
                s_ctl[4] = cstar;
            }
            X_.sync();
            if (s_ctl[2]) return;  // first tail-biting pass: only the state before mid_t is needed
        }
    }

    // ---- reconstruction and code (tcq_viterbi.cu:662-682) -------------------------------------------
    float* rn = a.rec + (size_t)n * a.ld;
    for (int t = tid; t < T; t += nthr) {
        const int stt = s_st[t], gg = s_g[t];
        const int lb = mk.label(stt);
        const bool hi = mix > 0 && ((t / mix) & 1);
        const int Ut = hi ? U_hi : U;
        const int gi = cand ? (int)s_gc[(t / sub) * G + gg] : gg;
        const float gt = hi ? s_gain_hi[gi] : s_gain[gi];
        const float* tt = (hi ? s_tab_hi : s_tab) + lb * Ut;
        const float xt = s_x[t];
        float bestd = kSent, val = 0.f;
        int bu = 0;
        for (int u = MD ? (int)s_par[t] : 0; u < Ut; u += MD ? 2 : 1) {
            const float v = gt * tt[u];
            const float d = xt - v;
            const float dd = d * d;
            if (dd < bestd) { bestd = dd; val = v; bu = u; }
        }
        const int tp = (t + a.rot) % a.ld;
        rn[tp] = val;
        if (a.code) a.code[(size_t)n * a.ld + tp] = (gi << 16) | (lb * Ut + bu);
    }
}

}  // namespace ltq
