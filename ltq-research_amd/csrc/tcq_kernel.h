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
//   - decisions: one bit per lane per compare -- the sign bit of the difference of the two candidates --
//     shifted into 32-bit words with v_alignbit (acc = 2 acc + bit), stored per group with coalesced writes
//     into the caller's bp / pbits scratch.
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
    // pushes into the last word of a chunk; the word is left-aligned when stored, so push P of a chunk is
    // bit 31 - (P & 31) of word P >> 5
    static constexpr int LAST = FG * PG - 32 * (NW - 1);
    static LTQ_DEV int word_of(int P) { return P >> 5; }
    static LTQ_DEV int bit_of(int P) { return 31 - (P & 31); }
    // first / last push index of any butterfly of in-group step k (0 <= k < RB)
    static constexpr int pmin(int k)
    {
        return BASE(k >> 1) + ((k & 1) ? 2 * PA(k >> 1) : 0);
    }
    static constexpr int pmax(int k)
    {
        return BASE(k >> 1) + (NB - 1) * PBLK(k >> 1) + ((k & 1) ? 2 * PA(k >> 1) + 2 * PB(k >> 1) : 2 * PA(k >> 1)) - 1;
    }
};

// Traceback windows: 16 trellis steps (4 groups at S = 1024, one 8-group chunk at S = 256).
template <int NU, int MD>
struct Tb {
    using M = Mode<NU, MD>;
    static constexpr int WS = 16;                                  // steps per window
    static constexpr int CPW = WS / (M::FG * (NU - 6));            // stored chunks per window
    static constexpr int NWW = CPW * M::NW;                        // words per lane per window per gain slot
    static constexpr int LW = (NWW + 3) / 4;                       // 16-byte loads per lane per window (each wave)
};

// dynamic LDS layout (byte offsets), identical on host (launch size) and device
struct Smem {
    int x, w, tab, tab_hi, gain, gain_hi, gc, ce, lbr, exch, tabs, gsel, st, g, par, red_v, red_i, ctl, total;
    int tabs_per_wave;  // floats
    int ec_floats;      // compact part of a wave's tables
    int ring, nslot, slot_words;  // traceback window ring (overlaps exch + tabs, dead after the forward pass)
};

LTQ_HD int align16(int v) { return (v + 15) & ~15; }

struct alignas(16) F4 {
    float x, y, z, w;
};

template <int NU, int MD, int NL>
LTQ_HD Smem smem_layout(int T, int G, int Gfull, int sub, int lds_max)
{
    using M = Mode<NU, MD>;
    using TB = Tb<NU, MD>;
    constexpr int R = Lay<NU>::R, S = Lay<NU>::S, RB = Lay<NU>::RB, NP = M::NP;
    constexpr int RPP = R * NP + 4;  // padded row: lane classes start on different LDS banks
    (void)Gfull;
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
    L.gsel = o; o = align16(o + (T / sub) * S);
    L.st = o; o = align16(o + 2 * T + 32);
    L.g = o; o = align16(o + T + 16);
    L.par = o; o = align16(o + T + 16);
    L.red_v = o; o = align16(o + 4 * 64 * G);
    L.red_i = o; o = align16(o + 4 * 64 * G);
    L.ctl = o; o = align16(o + 4 * 8);
    L.ec_floats = align16(4 * RB * NL * NP) / 4;
    L.tabs_per_wave = L.ec_floats + 2 * RB * (NL / 2) * RPP;  // compact table + two expanded tables
    L.exch = o;
    L.tabs = align16(L.exch + 4 * G * S);
    const int fwd_end = align16(L.tabs + 4 * G * L.tabs_per_wave);
    // ring slots: one window of decision words of every gain slot, padded to whole 1 KB wave loads
    L.slot_words = TB::LW * G * 256;
    L.ring = L.exch;
    // two workgroups per CU (two waves per SIMD) whenever the forward state fits half of the LDS: a single
    // wave per SIMD issues at most every other VALU cycle, so occupancy is worth more than ring depth
    const int budget = 2 * fwd_end <= lds_max ? lds_max / 2 : lds_max;
    int ns = 4;
    while (ns > 2 && L.ring + ns * 4 * L.slot_words > budget && L.ring + ns * 4 * L.slot_words > fwd_end) ns--;
    L.nslot = ns;
    const int ring_end = L.ring + ns * 4 * L.slot_words;
    L.total = fwd_end > ring_end ? fwd_end : ring_end;
    return L;
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
// Compare-select-push: for candidates (x, y) with "x wins when x < y" the kernel computes
//   m = min(x, y)          (v_min_f32: equals x < y ? x : y)
//   d = x - y              (sign bit = [x < y]: no metric is -0, NaN or infinite, see level_err and below)
//   acc = 2 acc + sign(d)  (v_alignbit_b32 acc, acc, d, 31)
// three VGPR-only instructions per decision, no lane masks in scalar registers.
#define LTQ_CSP(P, x, y, m)                                                              \
    do {                                                                                 \
        const float d_ = (x) - (y);                                                      \
        m = X_.fmin((x), (y));                                                           \
        acc[(P) >> 5] = X_.push_sign(acc[(P) >> 5], d_);                                 \
    } while (0)
// decision only (the caller keeps the value of its own sequential min)
#define LTQ_PUSH0(P) acc[(P) >> 5] = X_.push_sign(acc[(P) >> 5], 0.f)

// ------------------------------------------------------------------------------------------------
// One 2-step phase of a group, all in registers. PH = phase index in the group (steps 2PH, 2PH+1 on
// slot bits HB = RB-1-2PH and LB = HB-1). Blocks of 4 slots {x, x|L, x|H, x|H|L}; local index j = 2*hbit + lbit.
// Step a (bit HB): butterflies (j=e, j=2+e); step b (bit LB): butterflies (j=2f, j=2f+1). The output with new
// code bit c of a butterfly goes to the slot whose butterfly bit is c. The predecessor with the high state
// bit (slot j1) wins only when strictly smaller, as in the reference (p0 on ties).
// ------------------------------------------------------------------------------------------------
template <int NU, int MD, int PH, class X>
LTQ_DEV void run_phase(bool init, int s0, int lane, float (&D)[Lay<NU>::R], float* C0, float* C1, const float* Ma,
                       const float* Mb, uint32_t* acc, X& X_)
{
    using LY = Lay<NU>;
    using M = Mode<NU, MD>;
    constexpr int R = LY::R, RB = LY::RB, NB = R / 4;
    constexpr int HB = RB - 1 - 2 * PH, LB = HB - 1, H = 1 << HB, L = 1 << LB;
    constexpr int PA = M::PA(PH), PB = M::PB(PH), PBLK = M::PBLK(PH), BASE = M::BASE(PH);
    constexpr bool EQ = MD == 3;
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
                    LTQ_PUSH0(P0 + e);
                } else {
                    float m;
                    LTQ_CSP(P0 + e, D[sl[j1]], D[sl[j0]], m);
                    v[j0] = m + Ma[sl[j0]];
                    v[j1] = m + Ma[sl[j1]];
                }
            }
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const int j0 = 2 * f, j1 = 2 * f + 1;
                float m;
                LTQ_CSP(P0 + 2 + f, v[j1], v[j0], m);
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
                    LTQ_PUSH0(P0 + e);
                } else {
                    float m;
                    LTQ_CSP(P0 + e, D[sl[j1]], D[sl[j0]], m);
                    I0[j0] = m + Ma[sl[j0] * 2 + 0];
                    I1[j0] = m + Ma[sl[j0] * 2 + 1];
                    I0[j1] = m + Ma[sl[j1] * 2 + 0];
                    I1[j1] = m + Ma[sl[j1] * 2 + 1];
                }
            }
#pragma unroll
            for (int f = 0; f < 2; f++) {
                const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 2 * PA + f * PB;
                float m0, m1;
                LTQ_CSP(PF + 0, I0[j1], I0[j0], m0);
                LTQ_CSP(PF + 1, I1[j1], I1[j0], m1);
                if constexpr (MD == 1) {  // D2: best class p of the pair (ties: p = 0)
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int r = sl[q ? j1 : j0];
                        float o;
                        LTQ_CSP(PF + 2 + q, m1 + Mb[r * 2 + 1], m0 + Mb[r * 2 + 0], o);
                        D[r] = o;
                    }
                } else if constexpr (!EQ) {  // D4 phase A: per class c the best b (ties: b = 0), parity b ^ c
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const int r = sl[q ? j1 : j0];
                        float o0, o1;
                        LTQ_CSP(PF + 2 + 2 * q + 0, m1 + Mb[r * 2 + 1], m0 + Mb[r * 2 + 0], o0);
                        LTQ_CSP(PF + 2 + 2 * q + 1, m1 + Mb[r * 2 + 0], m0 + Mb[r * 2 + 1], o1);
                        C0[r] = o0;
                        C1[r] = o1;
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
                float mc0, mc1;
                LTQ_CSP(P0 + e * PA + 0, C0[sl[j1]], C0[sl[j0]], mc0);
                LTQ_CSP(P0 + e * PA + 1, C1[sl[j1]], C1[sl[j0]], mc1);
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
                for (int cb = 0; cb < 4; cb++) LTQ_CSP(PF + cb, J[cb][j1], J[cb][j0], mm[cb]);
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int r = sl[q ? j1 : j0];
                    float v = mm[0] + Mb[r * 2 + 0];
                    LTQ_CSP(PF + 4 + 3 * q + 0, mm[1] + Mb[r * 2 + 1], v, v);
                    LTQ_CSP(PF + 4 + 3 * q + 1, mm[2] + Mb[r * 2 + 1], v, v);
                    LTQ_CSP(PF + 4 + 3 * q + 2, mm[3] + Mb[r * 2 + 0], v, v);
                    D[r] = v;
                }
            }
        } else {
            // EQ phase B: classes keep b = c; output = best class (ties: c = 0)
            float Jc[2][4];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int j0 = e, j1 = 2 + e;
                float mc0, mc1;
                LTQ_CSP(P0 + e * PA + 0, C0[sl[j1]], C0[sl[j0]], mc0);
                LTQ_CSP(P0 + e * PA + 1, C1[sl[j1]], C1[sl[j0]], mc1);
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
                float m0, m1;
                LTQ_CSP(PF + 0, Jc[0][j1], Jc[0][j0], m0);
                LTQ_CSP(PF + 1, Jc[1][j1], Jc[1][j0], m1);
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int r = sl[q ? j1 : j0];
                    float o;
                    LTQ_CSP(PF + 2 + q, m1 + Mb[r * 2 + 1], m0 + Mb[r * 2 + 0], o);
                    D[r] = o;
                }
            }
        }
    }
}

// zero pushes for a phase that lies beyond the tile end (keeps every decision bit at its fixed position)
template <int NU, int MD, int PH, class X>
LTQ_DEV void pad_phase(uint32_t* acc, X& X_)
{
    using M = Mode<NU, MD>;
#pragma unroll
    for (int i = 0; i < M::PPH(PH); i++) {
        const int P = M::BASE(PH) + i;
        acc[P >> 5] = X_.push_sign(acc[P >> 5], 0.f);
    }
}

// ------------------------------------------------------------------------------------------------
// The per-tile kernel body.
// X provides: tid(), wave() (tid / 64 as a uniform value), tile(), nthreads(), smem(), sync() (full barrier incl. global memory), lds_sync()
// (barrier for LDS only), wave_sync(), push_sign(acc, d), fmin(x, y), readlane(v, lane), load16(global src, LDS wave
// base) (asynchronous 16-byte global -> LDS copy landing at base + 16 * lane), wait_loads<N>() (at most N
// such copies of this wave still outstanding).
// ------------------------------------------------------------------------------------------------
template <int NU, int MD, int NL, class X>
LTQ_DEV void tcq_tile(const TcqArgs& a, X& X_, int lds_max)
{
    using LY = Lay<NU>;
    using M = Mode<NU, MD>;
    using TB = Tb<NU, MD>;
    constexpr int RB = LY::RB, R = LY::R, S = LY::S, NP = M::NP, NW = M::NW, FG = M::FG;
    constexpr bool G4 = MD >= 2, EQ = MD == 3;
    constexpr int NL2 = NL / 2, RP = R * NP, RPP = RP + 4;

    const int n = X_.tile(), tid = X_.tid(), nthr = X_.nthreads();
    const int lane = tid & 63, g = X_.wave();  // wave index, provably uniform (scalar registers)
    const int T = a.T, G = a.G, sub = a.sub, U = a.U, U_hi = a.U_hi, mix = MD ? 0 : a.mix;
    const int Gf = a.Gfull, nsub = T / sub;
    const bool cand = a.gcand != nullptr;
    const Masks mk{a.m, a.m2, a.m3, a.m4, NL};
    const Smem SM = smem_layout<NU, MD, NL>(T, G, Gf, sub, lds_max);
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
    float* s_ec = (float*)(sm + SM.tabs) + (size_t)g * SM.tabs_per_wave;
    float* s_ex = s_ec + SM.ec_floats;
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
    for (int i = tid; i < NL * U; i += nthr) s_tab[i] = a.tab[i];
    for (int i = tid; i < NL * U_hi; i += nthr) s_tab_hi[i] = a.tab_hi[i];
    if (tid < Gf) {
        s_gain[tid] = a.gains[tid];
        s_gain_hi[tid] = a.gains_hi[tid];
    }
    const int s0 = a.init_st ? a.init_st[n] : -1;
    X_.lds_sync();

    // ---- gain candidates: the G gains of lowest scalar error per sub-block (tcq_viterbi.cu:155-180) ----
    if (cand) {
        for (int i = tid; i < nsub * Gf; i += nthr) {
            const int j = i / Gf, gi = i % Gf;
            float e = 0.f;
            for (int t = j * sub; t < (j + 1) * sub; t++) {
                const bool hi = mix > 0 && ((t / mix) & 1);
                const float be = hi ? level_err(s_x[t], s_gain_hi[gi], s_tab_hi, 0, NL * U_hi, 1)
                                    : level_err(s_x[t], s_gain[gi], s_tab, 0, NL * U, 1);
                const float prod = be * s_w[t];
                e = e + prod;
            }
            s_ce[i] = e;
        }
        X_.lds_sync();
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
        X_.lds_sync();
    }

    // ---- per-lane layout constants ----------------------------------------------------------------
    // row offset of the expanded metric table this lane reads at in-group step k: the label bits of the lane
    // part of its states select the row
    int rowoff[RB];
    // expansion: this lane fills the (slot re, parity pe) column of EPK rows per step
    constexpr int LG = 64 / RP;
    constexpr int EPK = (NL2 + LG - 1) / LG;
    const int re = (lane % RP) / NP, pe = lane % NP, rsub = lane / RP;
    int lbr[RB];
#pragma unroll
    for (int k = 0; k < RB; k++) {
        rowoff[k] = (k * NL2 + (mk.label(LY::state(k + 1, 0, lane)) >> 1)) * RPP;
        lbr[k] = mk.label(LY::state(k + 1, re, 0));
    }
    // compact table E[k][label][parity]: entry e = lane + 64 i has fixed (k, label, parity); its gain-scaled
    // levels fl(g * tab[u]) are cached in registers for a sub-block (fast path)
    constexpr int NE = RB * NL * NP, EPL = (NE + 63) / 64;
    constexpr int CMAX = 16 / EPL < 1 ? 1 : 16 / EPL;      // cached levels per entry
    const int nlev_max = (U + NP - 1) / NP;                  // levels of a parity class (upper bound)
    const bool fast = mix == 0 && (sub % RB) == 0 && nlev_max <= CMAX;
    float cl[EPL][CMAX];
    int ek[EPL], elb[EPL], ep[EPL], enl[EPL];
#pragma unroll
    for (int i = 0; i < EPL; i++) {
        const int e = lane + 64 * i;
        const int ee = e < NE ? e : 0;
        ek[i] = ee / (NL * NP);
        elb[i] = (ee % (NL * NP)) / NP;
        ep[i] = ee % NP;
        enl[i] = (U - ep[i] + NP - 1) / NP;
    }
    float* const s_exb[2] = {s_ex, s_ex + RB * NL2 * RPP};

    // compact table of the group starting at step tb2 -> s_ec
    auto compact = [&](int tb2) {
        if (fast) {
            if (tb2 % sub == 0) {  // gain slot's gain for this sub-block
                const int gi = cand ? (int)s_gc[(tb2 / sub) * G + g] : g;
                const float gn = s_gain[gi];
#pragma unroll
                for (int i = 0; i < EPL; i++)
#pragma unroll
                    for (int j = 0; j < CMAX; j++) {
                        const int idx = elb[i] * U + ep[i] + NP * j;
                        cl[i][j] = gn * s_tab[idx < NL * U ? idx : 0];
                    }
            }
#pragma unroll
            for (int i = 0; i < EPL; i++) {
                const int e = lane + 64 * i;
                if (NE % 64 == 0 || e < NE) {
                    const int t0 = tb2 + ek[i];
                    const int t = t0 < T ? t0 : T - 1;
                    const float xt = s_x[t];
                    float m = kSent;
#pragma unroll
                    for (int j = 0; j < CMAX; j++) {
                        const float d = xt - cl[i][j];
                        const float dd = d * d;
                        m = (j < enl[i] && dd < m) ? dd : m;
                    }
                    float E = m * s_w[t];
                    E = E + 0.0f;  // -0 -> +0: no metric is -0, so sign(x - y) is exactly [x < y]
                    s_ec[e] = E;
                }
            }
        } else {  // general path: half-integer tables, sub-blocks inside a group, many levels
#pragma unroll
            for (int i = 0; i < EPL; i++) {
                const int e = lane + 64 * i;
                if (NE % 64 == 0 || e < NE) {
                    const int k = ek[i], lb = elb[i], p = ep[i];
                    const int t = tb2 + k;
                    float E = 0.f;
                    if (t < T) {
                        const int gi = cand ? (int)s_gc[(t / sub) * G + g] : g;
                        const bool hi = mix > 0 && ((t / mix) & 1);
                        float be;
                        if (MD) be = level_err(s_x[t], s_gain[gi], s_tab + lb * U, p, U, 2);
                        else if (hi) be = level_err(s_x[t], s_gain_hi[gi], s_tab_hi + lb * U_hi, 0, U_hi, 1);
                        else be = level_err(s_x[t], s_gain[gi], s_tab + lb * U, 0, U, 1);
                        E = be * s_w[t];
                        E = E + 0.0f;
                    }
                    s_ec[e] = E;
                }
            }
        }
    };
    // expanded table rows: row (k, c) holds, for slot r and parity p, the metric of label (2c) ^ label(slot r)
    float ev[RB][EPK];
    auto expand_read = [&]() {
#pragma unroll
        for (int k = 0; k < RB; k++)
#pragma unroll
            for (int it = 0; it < EPK; it++) {
                const int row = rsub + it * LG;
                const int rr = (NL2 % LG == 0 || row < NL2) ? row : 0;
                ev[k][it] = s_ec[(k * NL + ((rr << 1) ^ lbr[k])) * NP + pe];
            }
    };
    auto expand_write = [&](float* ex) {
#pragma unroll
        for (int k = 0; k < RB; k++)
#pragma unroll
            for (int it = 0; it < EPK; it++) {
                const int row = rsub + it * LG;
                if (NL2 % LG == 0 || row < NL2) ex[(k * NL2 + row) * RPP + re * NP + pe] = ev[k][it];
            }
    };
    auto load_metrics = [&](const float* ex, int k, float* M) {
        const F4* p4 = (const F4*)(ex + rowoff[k]);
#pragma unroll
        for (int i = 0; i < RP / 4; i++) {
            const F4 v = p4[i];
            M[4 * i] = v.x;
            M[4 * i + 1] = v.y;
            M[4 * i + 2] = v.z;
            M[4 * i + 3] = v.w;
        }
    };
    // gain merge at a sub-block boundary, in the layout after k0 in-group steps (tcq_viterbi.cu:185-201)
    auto merge_read = [&](int k0, int j, float (&Dm)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int s = LY::state(k0, r, lane);
            const int ix = exch_index(s);
            float bv = s_exch[ix];
            int bg = 0;
#pragma unroll
            for (int gg = 1; gg < 8; gg++) {
                const float v = gg < G ? s_exch[gg * S + ix] : kSent;
                if (gg < G && v < bv) { bv = v; bg = gg; }
            }
            Dm[r] = bv;
            if (g == 0) s_gsel[j * S + s] = (uint8_t)bg;
        }
    };

    float D[R];
    uint32_t acc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) acc[w] = 0;
    float C0[G4 ? R : 1], C1[G4 ? R : 1];

    const int NG = (T + RB - 1) / RB;
    // tables of group 0
    compact(0);
    X_.wave_sync();
    expand_read();
    expand_write(s_exb[0]);
    X_.wave_sync();
    bool pend = false;  // another wave may still read this wave's exchange region (after a gain merge)
    for (int gr = 0; gr < NG; gr++) {
        const int tb = gr * RB;
        const bool has_next = gr + 1 < NG;
        const float* exc = s_exb[gr & 1];
        // ---- phase 0 (steps tb, tb+1); the next group's compact table is computed meanwhile -------------
        {
            float Ma[RP], Mb[RP];
            load_metrics(exc, 0, Ma);
            load_metrics(exc, 1, Mb);
            if (has_next) compact(tb + RB);
            run_phase<NU, MD, 0>(tb == 0, s0, lane, D, C0, C1, Ma, Mb, acc, X_);
        }
        X_.wave_sync();  // compact table of the next group visible to every lane of the wave
        if (has_next) expand_read();
        // ---- phase 1 (steps tb+2, tb+3) ---------------------------------------------------------------
        if constexpr (M::NPH > 1) {
            const int ta = tb + 2;
            if (ta < T) {
                if (G > 1 && (ta % sub) == 0) {  // sub-block boundary inside a group (sub % 4 == 2)
                    if (pend) X_.lds_sync();
#pragma unroll
                    for (int r = 0; r < R; r++) s_exch[g * S + exch_index(LY::state(2, r, lane))] = D[r];
                    X_.lds_sync();
                    merge_read(2, ta / sub, D);
                    pend = true;
                }
                float Ma[RP], Mb[RP];
                load_metrics(exc, 2, Ma);
                load_metrics(exc, 3, Mb);
                run_phase<NU, MD, M::NPH - 1>(false, s0, lane, D, C0, C1, Ma, Mb, acc, X_);
            } else {
                pad_phase<NU, MD, M::NPH - 1>(acc, X_);
            }
        }
        if (has_next) expand_write(s_exb[(gr + 1) & 1]);
        // ---- store the chunk's decision words (left-aligned) ---------------------------------------------
        if ((gr % FG) == FG - 1 || gr == NG - 1) {
            const int have = gr % FG + 1;
            if (have < FG) {
                const int miss = (FG - have) * M::PG;  // pad missing groups (only FG > 1, single word)
#pragma unroll
                for (int w = 0; w < NW; w++) acc[w] = miss >= 32 ? 0u : (acc[w] << miss);
            }
            if (M::LAST < 32) acc[NW - 1] <<= (32 - M::LAST) & 31;
            const int c = gr / FG;
#pragma unroll
            for (int w = 0; w < NW; w++) {
                dec_words<NU, MD>(a, n, c, g, w)[lane] = acc[w];
                acc[w] = 0;
            }
        }
        // ---- exchange into the next group's start layout (+ gain merge at a sub-block boundary) ---------
        if (has_next) {
            const bool merge = G > 1 && ((tb + RB) % sub) == 0;
            if (pend) X_.lds_sync();
            pend = false;
#pragma unroll
            for (int q = 0; q < R / 4; q++) {  // lane l holds states (l << RB) | r: 4 consecutive per 16 bytes
                F4 v4;
                v4.x = D[4 * q];
                v4.y = D[4 * q + 1];
                v4.z = D[4 * q + 2];
                v4.w = D[4 * q + 3];
                *(F4*)(s_exch + g * S + exch_index(LY::state(RB, 4 * q, lane))) = v4;
            }
            if (merge) {
                X_.lds_sync();
                merge_read(0, (tb + RB) / sub, D);
                pend = true;
            } else {
                X_.wave_sync();
#pragma unroll
                for (int r = 0; r < R; r++) D[r] = s_exch[g * S + exch_index(LY::state(0, r, lane))];
            }
        }
        X_.wave_sync();
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
        X_.sync();  // full barrier: also completes every wave's decision-word stores before the traceback
        for (int off = 1; off < nthr; off <<= 1) {
            float ov = 0.f;
            int oi = 0;
            const bool act = (tid % (2 * off)) == 0 && tid + off < nthr;
            if (act) {
                ov = s_rv[tid + off];
                oi = s_ri[tid + off];
            }
            X_.lds_sync();
            if (act) {
                const float cv = s_rv[tid];
                const int ci = s_ri[tid];
                if (ov < cv || (ov == cv && oi < ci)) {
                    s_rv[tid] = ov;
                    s_ri[tid] = oi;
                }
            }
            X_.lds_sync();
        }
    }
    int bi_all = s_ri[0];
    if (bi_all == 0x7fffffff) bi_all = 0;  // no candidate at or below the sentinel: the reference reads out of range
    if (tid == 0) {
        a.best[n] = bi_all;
        if (a.end_st) a.end_st[n] = bi_all % S;
    }

    // ---- traceback (tcq_viterbi.cu:601-661) ----------------------------------------------------------
    // Windows of 16 steps; the decision words of every gain slot of a window are copied global -> LDS
    // asynchronously, nslot windows ahead, into a ring that reuses the forward pass's LDS. Wavefront 0 walks:
    // the path state is wave-uniform (scalar registers), each step reads its decision word with v_readlane
    // from the window's words held in VGPRs.
    {
        constexpr int WS = TB::WS, NWW = TB::NWW, LW = TB::LW, CPW = TB::CPW;
        uint32_t* ring = (uint32_t*)(sm + SM.ring);
        const int nslot = SM.nslot, slot_words = SM.slot_words;
        const int nwin = (T + WS - 1) / WS;
        const int nchunk = (NG + FG - 1) / FG;
        const int lines = G * NWW * 16;  // 16-byte lines of one window (all gain slots)
        // per load i of this lane: the (gain slot, chunk-in-window, word, quarter) it copies is fixed; only the
        // window changes, so keep a base pointer and a per-chunk stride
        const uint32_t* dummy = a.bp + (size_t)n * a.T * G * (S / 32);  // valid source for padding lanes
        const uint32_t* lbase[LW];
        size_t lstride[LW];
        int lcr[LW];
#pragma unroll
        for (int i = 0; i < LW; i++) {
            const int L = (i * G + g) * 64 + lane;
            lcr[i] = -1;
            lbase[i] = dummy;
            lstride[i] = 0;
            if (L < lines) {
                const int gg = L / (NWW * 16), row = (L / 16) % NWW, q = L % 16;
                const int cr = row / NW, w = row % NW;
                lcr[i] = cr;
                lbase[i] = dec_words<NU, MD>(a, n, cr, gg, w) + 4 * q;
                lstride[i] = (size_t)(dec_words<NU, MD>(a, n, cr + 1, gg, w) - dec_words<NU, MD>(a, n, cr, gg, w));
            }
        }
        auto issue = [&](int win) {
            uint32_t* slot = ring + (win % nslot) * slot_words;
#pragma unroll
            for (int i = 0; i < LW; i++) {
                const int ch = win * CPW + (lcr[i] < 0 ? 0 : lcr[i]);
                const uint32_t* src = (lcr[i] >= 0 && ch < nchunk) ? lbase[i] + (size_t)win * CPW * lstride[i] : dummy;
                X_.load16(src, slot + (i * G + g) * 256);
            }
        };
        for (int j = 0; j < nslot; j++)
            if (nwin - 1 - j >= 0) issue(nwin - 1 - j);
        int st = bi_all % S, gs = bi_all / S, cstar = 0;
        bool hit = false;
        const int midpos = a.mid_st ? a.mid_t - 1 : -1;
        int nextb = ((T - 1) / sub) * sub;  // largest sub-block start <= current position (gain switch point)
        for (int iw = nwin - 1; iw >= 0; iw--) {
            // this window's copies are done when at most the later-issued windows' copies are outstanding
            const int later = iw < nslot - 1 ? iw : nslot - 1;
            if (later >= 3) X_.template wait_loads<3 * LW>();
            else if (later == 2) X_.template wait_loads<2 * LW>();
            else if (later == 1) X_.template wait_loads<LW>();
            else X_.template wait_loads<0>();
            X_.lds_sync();
            if (g == 0) {
                const uint32_t* slot = ring + (iw % nslot) * slot_words;
                uint32_t wv[NWW];
                int gl = gs;
#pragma unroll
                for (int j = 0; j < NWW; j++) wv[j] = slot[(gs * NWW + j) * 64 + lane];
                uint32_t vrec = 0, vpar = 0;
                const int t0 = iw * WS;
#pragma unroll
                for (int jj = WS - 1; jj >= 0; jj--) {
                    const int t = t0 + jj;
                    if (t >= T || hit) continue;
                    if (gs != gl) {  // gain slot changed inside the window (sub-block boundary off a window edge)
#pragma unroll
                        for (int j = 0; j < NWW; j++) wv[j] = slot[(gs * NWW + j) * 64 + lane];
                        gl = gs;
                    }
                    const int k = jj % RB;                      // compile-time after unrolling
                    const int cr = jj / (FG * RB);
                    const int pc = ((jj / RB) % FG) * M::PG;
                    const int wlo = (pc + M::pmin(k)) >> 5, whi = (pc + M::pmax(k)) >> 5;
                    // this step's decision words of the lane that holds state st
                    const int ln = LY::lane(k + 1, st);
                    uint32_t wr[NW];
#pragma unroll
                    for (int w = 0; w < NW; w++) wr[w] = (w >= wlo && w <= whi) ? X_.readlane(wv[cr * NW + w], ln) : 0u;
                    const int r = LY::slot(k + 1, st);
                    const int ph = k >> 1, hb = RB - 1 - 2 * ph, lbt = hb - 1;
                    const int beta = ((r >> (hb + 1)) << lbt) | (r & ((1 << lbt) - 1));
                    const int cout = st & 1;
                    const bool stepb = k & 1;
                    const int pa = M::PA(ph), pbb = M::PB(ph);
                    const int base = pc + M::BASE(ph) + beta * 2 * (pa + pbb) +
                                     (stepb ? 2 * pa + ((r >> hb) & 1) * pbb : ((r >> lbt) & 1) * pa);
                    // 64-bit view of words base >> 5 and base >> 5 + 1 (a butterfly's pushes span at most two)
                    const int w0 = base >> 5;
                    uint32_t W0 = wr[wlo], W1 = wlo + 1 < NW ? wr[wlo + 1] : 0u;
#pragma unroll
                    for (int w = 1; w < NW; w++)
                        if (w > wlo && w <= whi && w == w0) {
                            W0 = wr[w];
                            W1 = w + 1 < NW ? wr[w + 1] : 0u;
                        }
                    const uint64_t V = ((uint64_t)W0 << 32) | W1;
                    auto bits = [&](int P, int nbit) -> int {  // nbit bits starting at push P, first push highest
                        return (int)((V >> (64 - (P - 32 * w0) - nbit)) & ((1u << nbit) - 1u));
                    };
                    int h = 0;
                    if (MD == 0) {
                        h = bits(base, 1);
                    } else if (MD == 1) {
                        if (stepb) {
                            const int p = bits(base + 2 + cout, 1);
                            h = bits(base + p, 1);
                            vpar = (lane == jj || lane == jj - 1) ? (uint32_t)p : vpar;
                        } else {
                            h = bits(base, 1);
                        }
                    } else if (!EQ) {
                        if (k == 3) {
                            // three sequential-min bits (s1 s2 s3) -> winner (c, b): 0xEDEC maps s1s2s3 to 2c + b
                            const int v3 = bits(base + 4 + 3 * cout, 3);
                            const int idx = (0xEDEC >> (2 * v3)) & 3;
                            cstar = idx >> 1;
                            const int b = idx & 1;
                            h = bits(base + idx, 1);
                            vpar = lane == jj ? (uint32_t)(b ^ cstar) : lane == jj - 1 ? (uint32_t)b : vpar;
                        } else if (k == 2) {
                            h = bits(base + cstar, 1);
                        } else if (k == 1) {
                            const int b = bits(base + 2 + 2 * cout + cstar, 1);
                            h = bits(base + b, 1);
                            vpar = lane == jj ? (uint32_t)(b ^ cstar) : lane == jj - 1 ? (uint32_t)b : vpar;
                        } else {
                            h = bits(base, 1);
                        }
                    } else {
                        if (k == 3) {
                            cstar = bits(base + 2 + cout, 1);
                            h = bits(base + cstar, 1);
                            vpar = (lane <= jj && lane >= jj - 3) ? (uint32_t)cstar : vpar;
                        } else if (k == 2 || k == 1) {
                            h = bits(base + cstar, 1);
                        } else {
                            h = bits(base, 1);
                        }
                    }
                    vrec = lane == jj ? (uint32_t)(st | (gs << 10)) : vrec;
                    if (t == midpos) {
                        if (lane == 0) a.mid_st[n] = st;
                        hit = true;
                        continue;
                    }
                    if (t > 0) {
                        st = (h << (NU - 1)) | (st >> 1);
                        if (t == nextb) {
                            if (G > 1) gs = s_gsel[(t / sub) * S + st];
                            nextb -= sub;
                        }
                    }
                }
                const int tpos = t0 + lane;
                if (lane < WS && tpos < T) {
                    s_st[tpos] = (uint16_t)(vrec & 1023u);
                    s_g[tpos] = (uint8_t)(vrec >> 10);
                    s_par[tpos] = (uint8_t)vpar;
                }
                if (lane == 0) s_ctl[2] = hit ? 1 : 0;
            }
            X_.lds_sync();
            if (s_ctl[2]) {
                X_.template wait_loads<0>();
                return;  // first tail-biting pass: only the state before mid_t is needed
            }
            if (iw - nslot >= 0) issue(iw - nslot);
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
