// Portable body of the MI355X TCQ Viterbi kernel (one workgroup per 256-weight tile).
//
// The same source is compiled two ways:
//   - for gfx950 by tcq_viterbi.hip (X = GpuX: threadIdx, s_barrier, LDS, v_alignbit decision packing);
//   - for the host by the CPU emulation used in tests (X = CpuX: one std::thread per lane, barriers),
//     so layout / indexing bugs show up on the CPU, under AddressSanitizer, before any GPU run.
//
// Semantics follow the reference kernel (src/cuda/tcq_viterbi.cu:97-683): Ungerboeck trellis with
// S = 2^NU states, predecessors p_h = h*S/2 + (s >> 1), labels from parities of (s >> 1) & masks, joint gain
// slots with a sub-block gain merge, integer / D2 (pp=1) / D4 (pp=2) / EQ (pp=3) parity modes, gain
// candidates, free / given start, tail-biting end, mid-state pass, cyclic shift, traceback and reconstruction.
// Ties: strict "<" everywhere, predecessor p0, lowest gain slot, lowest (g, s) index, lowest class / low bit,
// lowest u -- identical choices to the reference given identical fp32 inputs.
//
// MI355X mapping:
//   - a tile's G gain slots each own Q = S / (64 R) wavefronts; a lane holds R = 4 (R = 8 when G = 8) path
//     metrics, so G = 4 gives 16 wavefronts: four per SIMD, enough to hide LDS and VALU latency.
//   - a "phase" is two trellis steps done in registers as one radix-4 block per 4 slots. Between phases the
//     metrics go through LDS in natural state order (one 16-byte store per block, one 4-byte load per slot,
//     both conflict-free) and come back in the phase-start layout
//         state = (r << (6 + QB)) | (q << 6) | lane        (r: register slot, q: wave of the gain slot)
//     so each lane's states, labels and metric-table offsets are the same in every phase.
//   - labels are linear over GF(2) in the state bits, so a lane's label for (phase step, slot) is a per-lane
//     constant XOR; branch metrics E[g][step][label][class] are tabulated per 16-step chunk by all threads
//     and read with one LDS load per (slot, step).
//   - decisions: one bit per compare-select -- the sign bit of the difference of the two candidates --
//     shifted into 32-bit words with v_alignbit (acc = 2 acc + bit), stored per chunk per lane into the
//     caller's bp / pbits scratch.
//   - traceback: wavefront 0 walks one phase (two steps) per LDS lookup with its state in scalar registers;
//     the decision words of the chunks ahead are copied global -> LDS asynchronously by every wavefront.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

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
    int scratch_T = 0;     // > 0: the step count bp / pbits / gcand are sized for per tile (fused pass 1), else T
    long tile_words = 0;   // > 0: compact scratch, tile n's decision words at bp + n * tile_words (pbits unused)
};

LTQ_DEV int parity32(uint32_t v) { return __builtin_popcount(v) & 1; }

// label of state s: (s & 1) | par((s>>1)&m) << 1 | par((s>>1)&m2) << 2 | ... (tcq_viterbi.cu:85-95)
struct Masks {
    int m, m2, m3, m4, nl;
    LTQ_HD int label(int s) const
    {
        int lb = (__builtin_popcount((uint32_t)((s >> 1) & m)) & 1) << 1 | (s & 1);
        if (nl >= 8) lb |= (__builtin_popcount((uint32_t)((s >> 1) & m2)) & 1) << 2;
        if (nl >= 16) lb |= (__builtin_popcount((uint32_t)((s >> 1) & m3)) & 1) << 3;
        if (nl >= 32) lb |= (__builtin_popcount((uint32_t)((s >> 1) & m4)) & 1) << 4;
        return lb;
    }
};

// Geometry: NU state bits = RB register bits (top) + QB wave bits + 6 lane bits at a phase start.
template <int NU, int RB>
struct Geo {
    static constexpr int S = 1 << NU, HALF = S / 2, R = 1 << RB, NB = R / 4, QB = NU - 6 - RB, Q = 1 << QB;
    static_assert(RB >= 2 && QB >= 0, "geometry");
    // state of register slot r of (wave q, lane l) at a phase start
    static LTQ_HD int start(int r, int q, int l) { return (r << (6 + QB)) | (q << 6) | l; }
    // state after step a of block b, slot jj = 2 ca + e (e: the block's second input bit)
    static LTQ_HD int mid(int b, int jj, int q, int l)
    {
        return ((jj & 1) << (NU - 1)) | (b << (7 + QB)) | (q << 7) | (l << 1) | (jj >> 1);
    }
    // state after step b of block b, output j = 2 ca + cb
    static LTQ_HD int end(int b, int j, int q, int l) { return (b << (8 + QB)) | (q << 8) | (l << 2) | j; }
};

// Decision-bit layout per parity mode (MD: 0 integer, 1 D2, 2 D4, 3 EQ). Phase types: 0 (integer pair,
// D2 pair, D4 / EQ phase A) and 1 (D4 / EQ phase B); D4 / EQ alternate A, B from step 0.
template <int MD, int RB>
struct Md {
    static constexpr int NB = (1 << RB) / 4, NP = MD ? 2 : 1, XF = MD >= 2 ? 2 : 1;
    static constexpr bool TWO = MD >= 2;
    static constexpr int PBLK(int pt) { return MD == 0 ? 4 : MD == 1 ? 10 : MD == 2 ? (pt ? 24 : 14) : (pt ? 12 : 6); }
    static constexpr int PPH(int pt) { return NB * PBLK(pt); }
    static constexpr int NPC = (MD == 1 && NB == 1) ? 16 : 8;   // phases per chunk
    static constexpr int CK = 2 * NPC;                          // steps per chunk
    static constexpr int PT(int pi) { return TWO ? (pi & 1) : 0; }
    // pushes before in-chunk phase pi
    static constexpr int OFF(int pi) { return TWO ? (pi / 2) * (PPH(0) + PPH(1)) + (pi & 1) * PPH(0) : pi * PPH(0); }
    static constexpr int CB = OFF(NPC);       // pushes per full chunk
    static constexpr int NW = (CB + 31) / 32; // words per lane per chunk
    static constexpr int LAST = CB - 32 * (NW - 1);
};

LTQ_HD int align16(int v) { return (v + 15) & ~15; }

// f(integral_constant<I>), ..., f(integral_constant<N-1>): a loop whose index is a compile-time constant
template <int I, int N, class F>
LTQ_DEV void static_for(F&& f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

struct alignas(16) F4 {
    float x, y, z, w;
};

// dynamic LDS layout (byte offsets), identical on host (launch size) and device
struct Smem {
    int x, w, tab, tab_hi, gain, gain_hi, gc, ce, gix, gsel, st, g, par, red, ctl, tabs, exch, total;
    int tab_floats;   // one chunk table (all gain slots)
    int exch_floats;  // one exchange buffer (all gain slots)
    int dbl;          // exchange double-buffered
    int ring, nslot, slot_words;  // traceback ring (overlaps tables + exchange, dead after the forward pass)
};

template <int NU, int RB, int MD, int NL>
LTQ_HD Smem smem_layout(int T, int G, int Gfull, int sub, int lds_max)
{
    using GE = Geo<NU, RB>;
    using MM = Md<MD, RB>;
    Smem L;
    int o = 0;
    const int nsub = T / sub;
    L.x = o; o = align16(o + 4 * T);
    L.w = o; o = align16(o + 4 * T);
    L.tab = o; o = align16(o + 4 * 4 * kMaxU);
    L.tab_hi = o; o = align16(o + 4 * 4 * kMaxU);
    L.gain = o; o = align16(o + 4 * kMaxG);
    L.gain_hi = o; o = align16(o + 4 * kMaxG);
    L.gc = o; o = align16(o + nsub * kMaxG);
    L.ce = o; o = align16(o + 4 * nsub * kMaxG);
    L.gix = o; o = align16(o + T * G);                     // gain index per (step, slot); bit 7: hi table
    L.gsel = o; o = align16(o + (G > 1 ? nsub * GE::S : 0));
    L.st = o; o = align16(o + 2 * T + 32);
    L.g = o; o = align16(o + T + 32);
    L.par = o; o = align16(o + T + 32);
    L.red = o; o = align16(o + 8 * 64);
    L.ctl = o; o = align16(o + 4 * 8);
    L.tab_floats = G * MM::CK * NL * MM::NP;
    L.exch_floats = G * MM::XF * GE::S;
    L.tabs = o;
    L.exch = align16(L.tabs + 2 * 4 * L.tab_floats);
    const int one = align16(L.exch + 4 * L.exch_floats), two = align16(L.exch + 2 * 4 * L.exch_floats);
    L.dbl = two <= lds_max ? 1 : 0;
    const int fwd_end = L.dbl ? two : one;
    // ring slots: one chunk of decision words of every (gain slot, wave, lane), whole 1 KB wave loads + pad
    const int cw = G * GE::Q * 64 * MM::NW;
    L.slot_words = ((cw + 255) / 256) * 256 + 256;  // + pad: the walker reads word w + 1 of any lane
    L.ring = L.tabs;
    // the copying wavefront keeps nslot - 1 chunks of copies in flight: at most 63 outstanding (vmcnt)
    const int nl = (cw / 4 + 63) / 64;
    int ns = 4;
    while (ns > 2 && ((L.ring + ns * 4 * L.slot_words > lds_max && L.ring + ns * 4 * L.slot_words > fwd_end) ||
                      (ns - 1) * nl > 63))
        ns--;
    L.nslot = ns;
    const int ring_end = L.ring + ns * 4 * L.slot_words;
    L.total = fwd_end > ring_end ? fwd_end : ring_end;
    return L;
}

// words of decision scratch of one tile available in bp + pbits
LTQ_HD long scratch_words(int T, int G, int S, int pp)
{
    const long bp = (long)T * G * (S / 32);
    const long pb = pp == 1 ? (long)(T / 2) * G * (S / 32) : pp >= 2 ? (long)(T / 4) * G * 9 * (S / 32) : 0;
    return bp + pb;
}

// words of decision scratch one tile needs (full chunks of NW words per lane, the last chunk only the words
// holding its real decisions)
template <int NU, int RB, int MD>
LTQ_HD long needed_words(int T, int G)
{
    using MM = Md<MD, RB>;
    const int nph = T / 2, full = nph / MM::NPC, rem = nph % MM::NPC;
    const int rbits = MM::TWO ? (rem / 2) * (MM::PPH(0) + MM::PPH(1)) + (rem & 1) * MM::PPH(0) : rem * MM::PPH(0);
    const long w = (long)full * MM::NW + (rbits + 31) / 32;
    return w * G * Geo<NU, RB>::Q * 64;
}

// squared-error minimum over levels u0, u0+du, ... < Ut of fl(x - fl(g * tab[u]))^2 (tcq_viterbi.cu:46-54, 75-83)
LTQ_DEV float level_err(float xt, float gain, const float* tb, int u0, int Ut, int du)
{
    float e = kSent;
    for (int u = u0; u < Ut; u += du) {
        const float v = gain * tb[u];
        const float d = xt - v;
        const float dd = d * d;
        e = dd < e ? dd : e;  // v_min_f32: dd and e are never NaN
    }
    return e;
}

// Compare-select-push: for candidates (x, y) with "x wins when x < y" the kernel computes
//   m = min(x, y)          (v_min_f32: equals x < y ? x : y)
//   d = x - y              (sign bit = [x < y]: no metric is -0, NaN or infinite)
//   acc = 2 acc + sign(d)  (v_alignbit_b32 acc, acc, d, 31)
#define LTQ_CSP(P, x, y, m)                                         \
    do {                                                            \
        const float d_ = (x) - (y);                                 \
        m = X_.fmin((x), (y));                                      \
        acc[(P) >> 5] = X_.push_sign(acc[(P) >> 5], d_);            \
    } while (0)
#define LTQ_PUSH0(P) acc[(P) >> 5] = X_.push_sign(acc[(P) >> 5], 0.f)

// ------------------------------------------------------------------------------------------------
// One radix-4 block of a phase (two trellis steps). Inputs: slot j = 2 hbit + lbit (hbit: the state's top
// bit, consumed by step a; lbit: consumed by step b). Step a: butterflies (e, 2+e) -> intermediate slot
// jj = 2 ca + e; step b: butterflies (2f, 2f+1) -> output j = 2 f + cb with f = ca. The predecessor with the
// high state bit wins only when strictly smaller (p0 on ties), as in the reference.
// ma[jj][p]: metric of intermediate jj (step a), mb[j][p]: metric of output j (step b), p = parity class.
// ------------------------------------------------------------------------------------------------
template <int MD, int PT, int P0, bool init, class X, class HA, class HB>
LTQ_DEV void run_block(const bool (&ok)[4], const float (&I)[2][4], const float (&ma)[4][2],
                       const float (&mb)[4][2], float (&O)[2][4], uint32_t* acc, X& X_, HA&& ha, HB&& hb)
{
    constexpr bool EQ = MD == 3;
    if constexpr (MD == 0) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int j0 = e, j1 = 2 + e;
            if constexpr (init) {
                v[j0] = ok[j0] ? ma[j0][0] : kSent;
                v[j1] = ok[j1] ? ma[j1][0] : kSent;
                LTQ_PUSH0(P0 + e);
            } else {
                float m;
                LTQ_CSP(P0 + e, I[0][j1], I[0][j0], m);
                v[j0] = m + ma[j0][0];
                v[j1] = m + ma[j1][0];
            }
            ha(e);
        }
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int j0 = 2 * f, j1 = 2 * f + 1;
            float m;
            LTQ_CSP(P0 + 2 + f, v[j1], v[j0], m);
            O[0][j0] = m + mb[j0][0];
            O[0][j1] = m + mb[j1][0];
            hb(f);
        }
    } else if constexpr (PT == 0) {
        // D2 pair, or phase A of a D4 / EQ group: intermediates per low bit b of the first sample
        float I0[4], I1[4];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int j0 = e, j1 = 2 + e;
            if constexpr (init) {
#pragma unroll
                for (int qq = 0; qq < 2; qq++) {
                    const int jj = qq ? j1 : j0;
                    I0[jj] = ok[jj] ? ma[jj][0] : kSent;
                    I1[jj] = ok[jj] ? ma[jj][1] : kSent;
                }
                LTQ_PUSH0(P0 + e);
            } else {
                float m;
                LTQ_CSP(P0 + e, I[0][j1], I[0][j0], m);
                I0[j0] = m + ma[j0][0];
                I1[j0] = m + ma[j0][1];
                I0[j1] = m + ma[j1][0];
                I1[j1] = m + ma[j1][1];
            }
            ha(e);
        }
        constexpr int PB = MD == 1 ? 4 : MD == 2 ? 6 : 2;
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 2 + f * PB;
            float m0, m1;
            LTQ_CSP(PF + 0, I0[j1], I0[j0], m0);
            LTQ_CSP(PF + 1, I1[j1], I1[j0], m1);
            if constexpr (MD == 1) {  // D2: best class p of the pair (ties: p = 0)
#pragma unroll
                for (int qq = 0; qq < 2; qq++) {
                    const int r = qq ? j1 : j0;
                    float o;
                    LTQ_CSP(PF + 2 + qq, m1 + mb[r][1], m0 + mb[r][0], o);
                    O[0][r] = o;
                }
            } else if constexpr (!EQ) {  // D4 phase A: per class c the best b (ties: b = 0), parity b ^ c
#pragma unroll
                for (int qq = 0; qq < 2; qq++) {
                    const int r = qq ? j1 : j0;
                    float o0, o1;
                    LTQ_CSP(PF + 2 + 2 * qq + 0, m1 + mb[r][1], m0 + mb[r][0], o0);
                    LTQ_CSP(PF + 2 + 2 * qq + 1, m1 + mb[r][0], m0 + mb[r][1], o1);
                    O[0][r] = o0;
                    O[1][r] = o1;
                }
            } else {  // EQ phase A: class c keeps b = c
#pragma unroll
                for (int qq = 0; qq < 2; qq++) {
                    const int r = qq ? j1 : j0;
                    O[0][r] = m0 + mb[r][0];
                    O[1][r] = m1 + mb[r][1];
                }
            }
            hb(f);
        }
    } else if constexpr (!EQ) {
        // D4 phase B: J[c][b] = min over predecessors of C_c + E(b); output = best (c, b) in order 00,01,10,11
        float J[4][4];  // [2c+b][jj]
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int j0 = e, j1 = 2 + e;
            float mc0, mc1;
            LTQ_CSP(P0 + 2 * e + 0, I[0][j1], I[0][j0], mc0);
            LTQ_CSP(P0 + 2 * e + 1, I[1][j1], I[1][j0], mc1);
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int jj = qq ? j1 : j0;
                J[0][jj] = mc0 + ma[jj][0];
                J[1][jj] = mc0 + ma[jj][1];
                J[2][jj] = mc1 + ma[jj][0];
                J[3][jj] = mc1 + ma[jj][1];
            }
            ha(e);
        }
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 4 + f * 10;
            float mm[4];
#pragma unroll
            for (int cb = 0; cb < 4; cb++) LTQ_CSP(PF + cb, J[cb][j1], J[cb][j0], mm[cb]);
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int r = qq ? j1 : j0;
                float v = mm[0] + mb[r][0];
                LTQ_CSP(PF + 4 + 3 * qq + 0, mm[1] + mb[r][1], v, v);
                LTQ_CSP(PF + 4 + 3 * qq + 1, mm[2] + mb[r][1], v, v);
                LTQ_CSP(PF + 4 + 3 * qq + 2, mm[3] + mb[r][0], v, v);
                O[0][r] = v;
            }
            hb(f);
        }
    } else {
        // EQ phase B: classes keep b = c; output = best class (ties: c = 0)
        float Jc[2][4];
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int j0 = e, j1 = 2 + e;
            float mc0, mc1;
            LTQ_CSP(P0 + 2 * e + 0, I[0][j1], I[0][j0], mc0);
            LTQ_CSP(P0 + 2 * e + 1, I[1][j1], I[1][j0], mc1);
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int jj = qq ? j1 : j0;
                Jc[0][jj] = mc0 + ma[jj][0];
                Jc[1][jj] = mc1 + ma[jj][1];
            }
            ha(e);
        }
#pragma unroll
        for (int f = 0; f < 2; f++) {
            const int j0 = 2 * f, j1 = 2 * f + 1, PF = P0 + 4 + f * 4;
            float m0, m1;
            LTQ_CSP(PF + 0, Jc[0][j1], Jc[0][j0], m0);
            LTQ_CSP(PF + 1, Jc[1][j1], Jc[1][j0], m1);
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {
                const int r = qq ? j1 : j0;
                float o;
                LTQ_CSP(PF + 2 + qq, m1 + mb[r][1], m0 + mb[r][0], o);
                O[0][r] = o;
            }
            hb(f);
        }
    }
}

// Location of decision word (tile n, linear word L): bp holds the first scratch_words(bp part) words of a
// tile, pbits the rest.
struct DecMap {
    uint32_t* bp;
    uint32_t* pb;
    long cap_bp;
    LTQ_DEV uint32_t* at(long L) const { return L < cap_bp ? bp + L : pb + (L - cap_bp); }
};

// ------------------------------------------------------------------------------------------------
// The per-tile kernel body.
// X provides: tid(), wave() (tid / 64, uniform), tile(), nthreads(), smem(), sync() (full barrier incl. global
// memory), lds_sync() (barrier for LDS only), push_sign(acc, d), fmin(x, y), wave_min(v, i) (the wavefront's
// (value, index) minimum, lowest index on ties, in lane 63), readlane(v, l) (lane l's value, l uniform), uni(v)
// (a uniform value in a scalar register), pin(v) (v computed at this point), sched_fence() (no instruction
// moved across), load_coherent(p) (a global int written by this workgroup before a sync()), acquire()
// (device-scope acquire: invalidates this CU's L1), load16(global src, LDS wave base) (asynchronous 16-byte
// global -> LDS copy landing at base + 16 * lane), wait_loads(n) (at most n such copies of this wave still
// outstanding, n <= 63).
// ------------------------------------------------------------------------------------------------
// init_val >= 0: the start (and tail) state of the tile in place of init_st (the fused closing pass)
template <int NU, int RB, int MD, int NL, class X>
LTQ_DEV void tcq_tile(const TcqArgs& a, X& X_, int lds_max, int init_val = -1)
{
    using GE = Geo<NU, RB>;
    using MM = Md<MD, RB>;
    constexpr int S = GE::S, HALF = GE::HALF, R = GE::R, NB = GE::NB, QB = GE::QB, Q = GE::Q;
    constexpr int NP = MM::NP, NPC = MM::NPC, CK = MM::CK, NW = MM::NW, XF = MM::XF;
    constexpr bool TWO = MM::TWO, EQ = MD == 3;

    const int n = X_.tile(), tid = X_.tid(), nthr = X_.nthreads();
    const int lane = tid & 63, wv = X_.wave();
    const int g = wv / Q, q = wv % Q;  // gain slot and wave of the slot (uniform)
    const int T = a.T, G = a.G, sub = a.sub, U = a.U, U_hi = a.U_hi, mix = MD ? 0 : a.mix;
    const int Gf = a.Gfull, nsub = T / sub;
    const bool cand = a.gcand != nullptr;
    const int Ts = a.scratch_T > 0 ? a.scratch_T : T;  // per-tile scratch layout (a fused pass 1 shares pass 2's)
    const Masks mk{a.m, a.m2, a.m3, a.m4, NL};
    const Smem SM = smem_layout<NU, RB, MD, NL>(T, G, Gf, sub, lds_max);
    char* sm = (char*)X_.smem();
    float* s_x = (float*)(sm + SM.x);
    float* s_w = (float*)(sm + SM.w);
    float* s_tab = (float*)(sm + SM.tab);
    float* s_tab_hi = (float*)(sm + SM.tab_hi);
    float* s_gain = (float*)(sm + SM.gain);
    float* s_gain_hi = (float*)(sm + SM.gain_hi);
    uint8_t* s_gc = (uint8_t*)(sm + SM.gc);
    float* s_ce = (float*)(sm + SM.ce);
    uint8_t* s_gix = (uint8_t*)(sm + SM.gix);
    uint8_t* s_gsel = (uint8_t*)(sm + SM.gsel);
    uint16_t* s_st = (uint16_t*)(sm + SM.st);
    uint8_t* s_g = (uint8_t*)(sm + SM.g);
    uint8_t* s_par = (uint8_t*)(sm + SM.par);
    float* s_rv = (float*)(sm + SM.red);
    int* s_ri = (int*)(sm + SM.red + 4 * 64);
    int* s_ctl = (int*)(sm + SM.ctl);
    float* s_tabs = (float*)(sm + SM.tabs);
    float* s_exch = (float*)(sm + SM.exch);

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
    const int s0 = init_val >= 0 ? init_val : (a.init_st ? a.init_st[n] : -1);
    X_.lds_sync();

    // ---- gain candidates: the G gains of lowest scalar error per sub-block (tcq_viterbi.cu:155-180) ----
    if (cand) {
        // The (step, gain) products fl(level_err * w) are independent: every thread computes some of them into
        // the forward pass's LDS (free until tables(0)), then each (sub-block, gain) sums its steps in order, as
        // the reference's loop does (identical fp32 operations). A tile too large for that LDS (never a
        // production shape) runs the loop as written.
        const int nprod = nsub * sub * Gf;
        const int room = (SM.exch - SM.tabs) / 4 + (SM.dbl ? 2 : 1) * SM.exch_floats;
        auto prod_of = [&](int t, int gi) {
            const bool hi = mix > 0 && ((t / mix) & 1);
            const float be = hi ? level_err(s_x[t], s_gain_hi[gi], s_tab_hi, 0, NL * U_hi, 1)
                                : level_err(s_x[t], s_gain[gi], s_tab, 0, NL * U, 1);
            return be * s_w[t];
        };
        if (nprod <= room) {
            float* s_prod = s_tabs;  // [t][gi]
            for (int i = tid; i < nprod; i += nthr) s_prod[i] = prod_of(i / Gf, i % Gf);
            X_.lds_sync();
            for (int i = tid; i < nsub * Gf; i += nthr) {
                const int j = i / Gf, gi = i % Gf;
                float e = 0.f;
                for (int t = j * sub; t < (j + 1) * sub; t++) e = e + s_prod[t * Gf + gi];
                s_ce[i] = e;
            }
        } else {
            for (int i = tid; i < nsub * Gf; i += nthr) {
                const int j = i / Gf, gi = i % Gf;
                float e = 0.f;
                for (int t = j * sub; t < (j + 1) * sub; t++) e = e + prod_of(t, gi);
                s_ce[i] = e;
            }
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
                a.gcand[((size_t)n * (Ts / sub) + tid) * G + c] = (uint8_t)bg;
            }
        }
        X_.lds_sync();
    }
    // gain index of every (step, slot), bit 7 = the step uses the hi table (mix)
    for (int i = tid; i < T * G; i += nthr) {
        const int t = i / G, gg = i % G;
        const int gi = cand ? (int)s_gc[(t / sub) * G + gg] : gg;
        const bool hi = mix > 0 && ((t / mix) & 1);
        s_gix[i] = (uint8_t)(gi | (hi ? 0x80 : 0));
    }
    X_.lds_sync();

    // metric table of chunk cc -> buffer (cc & 1): E[g][k][label][p] for steps cc*CK + k (0 beyond T)
    const int TF = SM.tab_floats;
    auto tables = [&](int cc) {
        float* tb = s_tabs + (cc & 1) * TF;
        // one entry per thread (the table has 64 Q entries per gain slot: D4 and EQ with 8 labels, D2 with 4, at
        // four wavefronts per slot), the slot's own gain (no candidates), two levels per parity class at most:
        // straight-line, the level loop of level_err unrolled; any other launch shape takes the loop below
        if constexpr (MD != 0 && CK * NL * NP == 64 * Q) {
            if (!cand && (U == 2 || U == 4) && nthr == TF) {
                const int e = tid;
                const int p = e & 1, lb = (e / NP) % NL, k = (e / (NP * NL)) % CK, gg = e / (NP * NL * CK);
                const int t = cc * CK + k;
                float E = 0.f;
                if (t < T) {
                    const float gain = s_gain[gg];
                    const float xt = s_x[t];
                    const float* tl = s_tab + lb * U + p;  // levels p and p + 2 of label lb
                    const float l0 = tl[0], l1 = tl[2];   // tl[2] lies inside s_tab (4 kMaxU floats) also for U = 2
                    float be = kSent;
                    {
                        const float v = gain * l0;
                        const float d = xt - v;
                        const float dd = d * d;
                        be = dd < be ? dd : be;
                    }
                    if (U == 4) {
                        const float v = gain * l1;
                        const float d = xt - v;
                        const float dd = d * d;
                        be = dd < be ? dd : be;
                    }
                    E = be * s_w[t];
                    E = E + 0.0f;
                }
                tb[e] = E;
                return;
            }
        }
        for (int e = tid; e < TF; e += nthr) {
            const int p = NP == 2 ? (e & 1) : 0;
            const int lb = (e / NP) % NL, k = (e / (NP * NL)) % CK, gg = e / (NP * NL * CK);
            const int t = cc * CK + k;
            float E = 0.f;
            if (t < T) {
                const int gx = s_gix[t * G + gg], gi = gx & 0x7f;
                float be;
                if (MD) be = level_err(s_x[t], s_gain[gi], s_tab + lb * U, p, U, 2);
                else if (gx & 0x80) be = level_err(s_x[t], s_gain_hi[gi], s_tab_hi + lb * U_hi, 0, U_hi, 1);
                else be = level_err(s_x[t], s_gain[gi], s_tab + lb * U, 0, U, 1);
                E = be * s_w[t];
                E = E + 0.0f;  // -0 -> +0: no metric is -0, so sign(x - y) is exactly [x < y]
            }
            tb[e] = E;
        }
    };

    // ---- per-lane constants: table offsets of each (block, slot) at step a / b, start check -----------
    const int la_lane = mk.label(GE::mid(0, 0, q, lane)), lb_lane = mk.label(GE::end(0, 0, q, lane));
    int offa[NB][4], offb[NB][4];
    bool ok[NB][4];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            offa[b][j] = (g * CK * NL + (la_lane ^ mk.label(GE::mid(b, j, 0, 0)))) * NP;
            offb[b][j] = (g * CK * NL + (lb_lane ^ mk.label(GE::end(b, j, 0, 0)))) * NP;
            const int sm1 = GE::mid(b, j, q, lane);
            ok[b][j] = s0 < 0 || (sm1 >> 1) == (s0 & (HALF - 1));
        }

    const DecMap dm = a.tile_words > 0
                          ? DecMap{a.bp + (size_t)n * a.tile_words, nullptr, a.tile_words}
                          : DecMap{a.bp + (size_t)n * Ts * G * (S / 32),
                                   a.pbits ? a.pbits + (size_t)n * (scratch_words(Ts, G, S, a.pp) - (long)Ts * G * (S / 32))
                                           : nullptr,
                                   (long)Ts * G * (S / 32)};
    const int nph = T / 2;
    const int nchunk = (nph + NPC - 1) / NPC;
    const long chunk_words = (long)G * Q * 64 * NW;

    float I[2][NB][4];  // phase inputs (class planes for phase B)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) I[c][b][j] = 0.f;
    float O[2][NB][4];
    uint32_t acc[NW];

    // metrics of in-chunk phase PI (steps 2 PI, 2 PI + 1 of the chunk) for every (block, slot), read through
    // per-lane pointers into a chunk's table (set once per chunk; the phase and class are immediate offsets)
    float ma[NB][4][2], mb[NB][4][2];
    const float* pma[NB][4];
    const float* pmb[NB][4];
    auto point_metrics = [&](const float* tb) {
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                pma[b][j] = tb + offa[b][j];
                pmb[b][j] = tb + offb[b][j];
            }
    };
    auto load_metrics = [&](auto PIc) {
        constexpr int pi = decltype(PIc)::value;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int p = 0; p < NP; p++) {
                    ma[b][j][p] = pma[b][j][(2 * pi) * NL * NP + p];
                    mb[b][j][p] = pmb[b][j][(2 * pi + 1) * NL * NP + p];
                }
    };

    tables(0);
    X_.lds_sync();
    point_metrics(s_tabs);
    load_metrics(std::integral_constant<int, 0>{});
    // exchange addresses of this lane in buffer 0 / 1 (phases alternate, and every chunk has an even number of
    // phases, so in-chunk phase pi uses buffer pi & 1): store at block 0 of the phase-end layout, loads at
    // slot 0 of the phase-start layout (own gain slot, and gain slot 0 for the merge); blocks, slots, class
    // planes and gain slots are immediate offsets
    float* const xs_st0 = s_exch + (g * XF) * S + GE::end(0, 0, q, lane);
    const float* const xs_ld0 = s_exch + (g * XF) * S + GE::start(0, q, lane);
    const float* const xs_mg0 = s_exch + GE::start(0, q, lane);
    const int xs_1 = SM.dbl ? SM.exch_floats : 0;
    int next_merge = sub, merge_j = 1;   // next sub-block boundary and its index
    // chunk c; FIRST: chunk 0, whose phase 0 starts the trellis (compile-time, so no other phase carries the
    // start-state selects)
    // streamlined traceback (whole chunks, one block per lane, a second wavefront, a ring of at least 3 chunks,
    // sub-blocks of 16 or 32): the last chunk's decision words then go straight from registers to the traceback's
    // LDS ring
    bool fast = false;
    if constexpr (RB == 2) fast = T % CK == 0 && nthr >= 128 && SM.nslot >= 3 && (sub == 16 || sub == 32);
    uint32_t last_acc[NW];
#pragma unroll
    for (int w = 0; w < NW; w++) last_acc[w] = 0;
    // AL (whole chunks, sub-blocks a multiple of 16 steps): a sub-block can only end where the phase's end step is
    // a multiple of 16, so every other phase is compiled without the tile-end and merge tests (and without the
    // register copies a runtime merge branch costs in every phase)
    auto chunk = [&](int c, auto FIRSTc, auto ALc) {
        constexpr bool FIRST = decltype(FIRSTc)::value;
        constexpr bool AL = decltype(ALc)::value;
#pragma unroll
        for (int w = 0; w < NW; w++) acc[w] = 0;
        const float* tbn = s_tabs + ((c + 1) & 1) * TF;
        int real = 0;  // phases of this chunk inside the tile
        static_for<0, NPC>([&](auto PIc) {
            constexpr int pi = decltype(PIc)::value;
            constexpr int PT = MM::PT(pi);
            const int ta = c * CK + 2 * pi;
            if (!AL && ta >= T) {  // beyond the tile end: zero pushes keep every decision bit at its fixed position
#pragma unroll
                for (int i = 0; i < MM::PPH(PT); i++) LTQ_PUSH0(MM::OFF(pi) + i);
                return;
            }
            real++;
            if constexpr (AL) X_.sched_fence();  // one scheduling region per phase, as the runtime tests give the other build
            constexpr bool init = FIRST && pi == 0;
            // The next phase's metrics are loaded while this phase computes, each pair of slots as soon as its
            // step has consumed it (the LDS reads then stream beside the compare-selects instead of queueing
            // with the exchange stores at the barrier). The last phase of a chunk reads the next chunk's table
            // (written in this chunk's phase 0, visible since phase 1's barrier); loads past the tile's last
            // phase stay inside the table and are unused.
            constexpr int PN = (pi + 1) % NPC;
            if constexpr (pi + 1 == NPC) point_metrics(tbn);
            static_for<0, NB>([&](auto Bc) {
                constexpr int b = decltype(Bc)::value;
                float Ib[2][4], Ob[2][4];
#pragma unroll
                for (int cc2 = 0; cc2 < 2; cc2++)
#pragma unroll
                    for (int j = 0; j < 4; j++) Ib[cc2][j] = I[cc2][b][j];
                // (scheduling fences keep the compiler from sinking the loads to the end of the phase)
                auto ha = [&](int e) {  // step a used slots e, 2 + e of ma
                    X_.sched_fence();
#pragma unroll
                    for (int p = 0; p < NP; p++) {
                        ma[b][e][p] = pma[b][e][(2 * PN) * NL * NP + p];
                        ma[b][2 + e][p] = pma[b][2 + e][(2 * PN) * NL * NP + p];
                    }
                    X_.sched_fence();
                };
                auto hb = [&](int f) {  // step b used slots 2 f, 2 f + 1 of mb
                    X_.sched_fence();
#pragma unroll
                    for (int p = 0; p < NP; p++) {
                        mb[b][2 * f][p] = pmb[b][2 * f][(2 * PN + 1) * NL * NP + p];
                        mb[b][2 * f + 1][p] = pmb[b][2 * f + 1][(2 * PN + 1) * NL * NP + p];
                    }
                    X_.sched_fence();
                };
                run_block<MD, PT, MM::OFF(pi) + b * MM::PBLK(PT), init>(ok[b], Ib, ma[b], mb[b], Ob, acc, X_, ha,
                                                                        hb);
#pragma unroll
                for (int cc2 = 0; cc2 < 2; cc2++)
#pragma unroll
                    for (int j = 0; j < 4; j++) O[cc2][b][j] = Ob[cc2][j];
            });
            if constexpr (AL) {  // the phase's decision bits are pushed now, not sunk to the chunk's word stores
                constexpr int w0 = MM::OFF(pi) >> 5, w1 = (MM::OFF(pi + 1) - 1) >> 5;
#pragma unroll
                for (int w = w0; w <= w1; w++) X_.pin(acc[w]);
            }
            const int tn = ta + 2;
            constexpr bool MAYB = !AL || (2 * (pi + 1)) % 16 == 0;  // this phase may end the tile or a sub-block
            if (MAYB && tn >= T) return;  // last phase: outputs stay in registers for the argmin
            // ---- exchange into the next phase's start layout (+ gain merge at a sub-block boundary) ----
            constexpr bool carry2 = TWO && PT == 0;  // phase A -> B carries two class planes
            const int xo = (pi & 1) ? xs_1 : 0;
            float* const xst = xs_st0 + xo;
            const float* const xld = xs_ld0 + xo;
            const float* const xmg = xs_mg0 + xo;
            if (!SM.dbl) X_.lds_sync();  // single buffer: every wave has read the previous exchange
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int cp = 0; cp < (carry2 ? 2 : 1); cp++) {
                    F4 v4;
                    v4.x = O[cp][b][0];
                    v4.y = O[cp][b][1];
                    v4.z = O[cp][b][2];
                    v4.w = O[cp][b][3];
                    *(F4*)(xst + cp * S + (b << (8 + QB))) = v4;
                }
            X_.lds_sync();
            const bool at_sub = MAYB && tn == next_merge;
            const int jm = merge_j;
            if (at_sub) {
                next_merge += sub;
                merge_j++;
            }
            if (!carry2 && G > 1 && at_sub) {
                // gain merge: per state the lowest metric over the slots, lowest slot on ties (slots >= G read
                // slot 0's value again, which never wins the strict compare). The slot bases are formed here, from
                // an opaque zero, so they are not hoisted out of the chunk loop.
                constexpr int GM = 16 / Q < 8 ? 16 / Q : 8;  // most gain slots this geometry serves
                const float* xm[GM];
                const int z0 = X_.opaque_zero();
#pragma unroll
                for (int gg = 0; gg < GM; gg++) xm[gg] = xmg + z0 + (gg < G ? gg * XF * S : 0);
                if (g == 0) {  // slot 0's wavefronts also record the merge choice for the traceback
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int s = GE::start((j << (RB - 2)) | b, q, lane);
                            const int so = ((j << (RB - 2)) | b) << (6 + QB);  // s - start(0, q, lane)
                            float v[GM];
#pragma unroll
                            for (int gg = 0; gg < GM; gg++) v[gg] = xm[gg][so];
                            float bv = v[0];
                            int bg = 0;
#pragma unroll
                            for (int gg = 1; gg < GM; gg++)
                                if (v[gg] < bv) {
                                    bv = v[gg];
                                    bg = gg;
                                }
                            I[0][b][j] = bv;
                            s_gsel[jm * S + s] = (uint8_t)bg;
                        }
                } else {  // the merged metric alone: the minimum over the slots (the value the lowest-slot rule
                          // selects, as no metric is NaN or -0), a third of the VALU on three of four SIMD slots
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const int so = ((j << (RB - 2)) | b) << (6 + QB);
                            float bv = xm[0][so];
#pragma unroll
                            for (int gg = 1; gg < GM; gg++) bv = X_.fmin(bv, xm[gg][so]);
                            I[0][b][j] = bv;
                        }
                }
            } else {
#pragma unroll
                for (int cp = 0; cp < (carry2 ? 2 : 1); cp++)
#pragma unroll
                    for (int b = 0; b < NB; b++)
#pragma unroll
                        for (int j = 0; j < 4; j++)  // slot j of block b is register (j << (RB - 2)) | b
                            I[cp][b][j] = xld[cp * S + (((j << (RB - 2)) | b) << (6 + QB))];
            }
            // next chunk's table (its buffer was last read in chunk c-1), built while the exchange loads fly
            if (pi == 0 && c + 1 < nchunk) tables(c + 1);
        });
        // ---- store this chunk's decision words (left-aligned), only the words holding real bits -------
        if (MM::LAST < 32) acc[NW - 1] <<= (32 - MM::LAST) & 31;
        const int rbits = TWO ? (real / 2) * (MM::PPH(0) + MM::PPH(1)) + (real & 1) * MM::PPH(0) : real * MM::PPH(0);
        const int nwc = real == NPC ? NW : (rbits + 31) / 32;
        // word-major: word w of every lane of (slot g, wave q) is 64 consecutive u32 (coalesced stores)
        const long Lb = (long)c * chunk_words + (long)(g * Q + q) * nwc * 64;  // uniform: the wave's first word
        const long L0 = Lb + lane;
        if (fast && c == nchunk - 1) {
#pragma unroll
            for (int w = 0; w < NW; w++) last_acc[w] = acc[w];
        } else if (Lb + 64L * nwc <= dm.cap_bp || Lb >= dm.cap_bp) {
            // the wave's words lie in one buffer: a scalar base, the lane offset and immediate word offsets
            uint32_t* const wb = Lb < dm.cap_bp ? dm.bp + Lb : dm.pb + (Lb - dm.cap_bp);
#pragma unroll
            for (int w = 0; w < NW; w++)
                if (w < nwc) wb[lane + 64 * w] = acc[w];
        } else {
#pragma unroll
            for (int w = 0; w < NW; w++)
                if (w < nwc) *dm.at(L0 + 64L * w) = acc[w];
        }
    };
    if (T % CK == 0 && sub % 16 == 0) {
        chunk(0, std::true_type{}, std::true_type{});
        for (int c = 1; c < nchunk; c++) chunk(c, std::false_type{}, std::true_type{});
    } else {
        chunk(0, std::true_type{}, std::false_type{});
        for (int c = 1; c < nchunk; c++) chunk(c, std::false_type{}, std::false_type{});
    }

    // ---- argmin over (g, s), lowest index on ties (tcq_viterbi.cu:561-578) ---------------------------
    int bi_sel = 0;
    const int s_end = a.tail ? s0 : -1;
    if (s_end >= 0 && s_end < S) {
        // Closing pass: every (slot, state) but state s_end of each slot enters the argmin at the sentinel, so the
        // lexicographic minimum is the one over the G candidates (value of s_end in slot g, index g S + s_end)
        // and the lowest-index sentinel entry (kSent, s_end ? 0 : 1). The lane holding s_end in each slot stores
        // its value; one reduction over G + 1 lanes follows the barrier (no per-wavefront reduction before it).
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (GE::end(b, j, q, lane) == s_end) s_rv[g] = O[0][b][j];
        X_.sync();  // full barrier: also completes every wave's decision-word stores before the traceback
        if (wv == 0) {  // only the walking wavefront uses the result (the others keep an in-range 0)
            float bv = lane < G ? s_rv[lane] : kSent;
            int bi = lane < G ? lane * S + s_end : lane == 63 ? (s_end != 0 ? 0 : 1) : 0x7fffffff;
            X_.wave_min(bv, bi);
            bi_sel = (int)X_.readlane((uint32_t)bi, 63);
        }
    } else {
        float bv = kSent;
        int bi = 0x7fffffff;
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int s = GE::end(b, j, q, lane);
                const int idx = g * S + s;
                const float v = (s_end < 0 || s == s_end) ? O[0][b][j] : kSent;
                if (v < bv || (v == bv && idx < bi)) {
                    bv = v;
                    bi = idx;
                }
            }
        X_.wave_min(bv, bi);  // in lane 63
        if (lane == 63) {
            s_rv[wv] = bv;
            s_ri[wv] = bi;
        }
        X_.sync();  // full barrier: also completes every wave's decision-word stores before the traceback
        // the walking wavefront reduces the per-wavefront results across its lanes (no second barrier); the
        // others keep an in-range 0
        if (wv == 0) {
            const int nw = nthr / 64;
            bv = lane < nw ? s_rv[lane] : kSent;
            bi = lane < nw ? s_ri[lane] : 0x7fffffff;
            X_.wave_min(bv, bi);
            bi_sel = (int)X_.readlane((uint32_t)bi, 63);
            if (bi_sel == 0x7fffffff) bi_sel = 0;  // no candidate at or below the sentinel: the reference reads out of range
        }
    }
    const int bi_all = X_.uni(bi_sel);  // uniform: scalar registers

    // ---- traceback (tcq_viterbi.cu:601-661) ----------------------------------------------------------
    // One LDS lookup per phase: the phase's output state names the (wave, lane) that computed it and the
    // block; that lane's decision bits give the phase's input state, the intermediate state and the parity
    // classes. Lanes of the walking wavefront fetch the possible next lookups one phase ahead; v_readlane
    // picks the true one.
    uint16_t* s_rec = (uint16_t*)s_st;  // per phase: output state | slot << 10 | e << 13 | classes << 14
    // Streamlined walk (whole chunks, one block per lane, a second wavefront, a ring of at least 3 chunks,
    // sub-blocks of 16 or 32; every matrix-path tile): wavefront 0 walks, wavefront 1 copies the decision words of the chunks ahead
    // global -> LDS, one barrier per chunk hands them over, and every thread writes the outputs. Otherwise
    // wavefront 0 alone walks (copying its own words) and writes the outputs, and the others are done.
    if (!fast && wv != 0) return;
    int out_t0 = lane, out_dt = 64;
    if constexpr (RB == 2) {
        // No per-phase control flow but one uniform stop check. Bit positions are compile-time (one block per
        // lane); at the start of each phase, lane L + 4 gp fetches the decision words of the phase below for
        // the input-state hypothesis L (the phase's two decision bits h e) and, when the phase starts a
        // sub-block, for every gain slot gp the merge may choose, together with the merge choice of hypothesis
        // L, so neither the next chunk nor a slot change ever waits on an LDS round trip.
        if (fast) {
            out_t0 = tid;
            out_dt = nthr;
            uint32_t* ring = (uint32_t*)(sm + SM.ring);
            const int nslot = SM.nslot, slot_words = SM.slot_words;
            const int nloads = (G * Q * 16 * NW + 63) / 64;  // wave loads per chunk
            // copies of chunk cc: 16-byte units u = 64 i + lane; a chunk lies in bp or in pbits as a whole except
            // at most one, so the source is a uniform base plus the lane's offset (the last unit repeated past the
            // end: the copy then stays inside the chunk and lands in the slot's pad)
            auto issue = [&](int cc) {
                const int units = G * Q * 16 * NW;
                uint32_t* slot = ring + (cc % nslot) * slot_words;
                const long base = (long)cc * chunk_words;
                if (base + chunk_words <= dm.cap_bp || base >= dm.cap_bp) {
                    const uint32_t* src = dm.at(base);
                    for (int i = 0; i < nloads; i++) {
                        const int u = i * 64 + lane;
                        X_.load16(src + 4L * (u < units ? u : units - 1), slot + i * 256);
                    }
                } else {
                    for (int i = 0; i < nloads; i++) {
                        const int u = i * 64 + lane;
                        X_.load16(dm.at(base + 4L * (u < units ? u : units - 1)), slot + i * 256);
                    }
                }
            };
            auto min_i = [](int x, int y) { return x < y ? x : y; };
            auto max_i = [](int x, int y) { return x > y ? x : y; };
            auto count = [](int lo, int hi) { return hi >= lo ? hi - lo + 1 : 0; };
            const int mid_ph = a.mid_st ? (a.mid_t - 1) >> 1 : -1;
            const int kmax = a.mid_st ? nchunk - mid_ph / NPC : nchunk;  // chunks walked
            // copier: chunks nchunk-2 .. nchunk-nslot+1 now (the last one is written from registers); before the
            // first barrier the two the walk reads first (its chunk and, from its last phase on, the one below)
            // are in LDS
            {  // the last chunk's words from registers (the forward pass's LDS is free since the argmin barrier)
                uint32_t* slot = ring + ((nchunk - 1) % nslot) * slot_words;
#pragma unroll
                for (int w = 0; w < NW; w++) slot[((g * Q + q) * NW + w) * 64 + lane] = last_acc[w];
            }
            if (wv == 1) {
                for (int j = 1; j < nslot - 1 && nchunk - 1 - j >= 0; j++) issue(nchunk - 1 - j);
                X_.wait_loads(count(max_i(0, nchunk - nslot + 1), nchunk - 3) * nloads);
            }
            X_.lds_sync();
            // per-lane hypothesis: L = lane & 3 (input-state bits h e), gp = lane >> 2 (gain slot at a boundary)
            const int hypL = lane & 3;
            const int gp = min_i(lane >> 2, G - 1);
            const int sxL = GE::start(hypL, 0, 0);
            const int wL = (sxL >> 8) & (Q - 1), lL = (sxL >> 2) & 63;
            int st = bi_all % S, gs = bi_all / S, cstar = 0;
            uint32_t c0, c1, gv = 0;
            {  // exact words of the walk's first phase, in every lane
                constexpr int P0 = MM::OFF(NPC - 1);
                const uint32_t* slot = ring + ((nchunk - 1) % nslot) * slot_words;
                const int wi = ((gs * Q + ((st >> 8) & (Q - 1))) * NW + (P0 >> 5)) * 64 + ((st >> 2) & 63);
                c0 = slot[wi];
                c1 = slot[wi + 64];
            }
            int sel = 0, mid_val = 0;
            const int lsub = sub == 16 ? 4 : 5;  // the fast walk serves sub 16 and 32
            // word offset of this lane's hypothesis (wave and lane bits of start(hypL, 0, 0), disjoint from those of
            // start(0, q, l)) in a ring slot, for the phases that cannot start a sub-block
            const int lane_off = wL * NW * 64 + lL;
            // The walk over chunks kmax .. : MIDW (first tail-biting pass) stops at the phase holding mid_t and writes
            // no records; the full walk keeps every phase's 16-bit record in scalar registers and stores a chunk's
            // records, two a word, at the end of the chunk. A sub-block can only start at a phase with 2 pi a
            // multiple of 16 (sub is 16 or 32), so every other phase carries no boundary test, no merge-choice fetch
            // and a scalar word address.
            auto walk = [&](auto midw) {
                constexpr bool MIDW = decltype(midw)::value;
                bool stop = false;
                for (int k = 0; k < kmax; k++) {
                    const int cc = nchunk - 1 - k;
                    if (wv == 1) {  // chunk cc - nslot + 1 into the slot chunk cc + 1 left; chunk cc - 2 lands first
                        if (cc - nslot + 1 >= 0) issue(cc - nslot + 1);
                        X_.wait_loads(count(max_i(0, cc - nslot + 1), cc - 3) * nloads);
                    }
                    if (wv == 0) {
                        const uint32_t* slot = ring + (cc % nslot) * slot_words;
                        const uint32_t* slot_next = ring + ((cc + nslot - 1) % nslot) * slot_words;  // chunk cc - 1
                        uint32_t recs[NPC];
                        static_for<0, NPC>([&](auto Kc) {
                            constexpr int pi = NPC - 1 - decltype(Kc)::value;
                            constexpr int PT = MM::PT(pi);
                            constexpr int P = MM::OFF(pi);
                            constexpr int o = P - 32 * (P >> 5);
                            constexpr int NB_ = MM::PBLK(PT);  // the phase's decision bits, first push highest
                            constexpr bool TWO_WORDS = o + NB_ > 32;
                            constexpr bool BC = (2 * pi) % 16 == 0;
                            if constexpr (MIDW) {
                                if (stop) return;
                            }
                            const int ta = cc * CK + 2 * pi, ph = ta >> 1;
                            bool bnd = false;
                            if constexpr (BC) bnd = G > 1 && ta > 0 && (ta & (sub - 1)) == 0;
                            const int qq = (st >> 8) & (Q - 1), ll = (st >> 2) & 63, jo = st & 3;
                            const uint32_t W0 = X_.readlane(c0, sel);
                            const uint32_t W1 = TWO_WORDS ? X_.readlane(c1, sel) : 0u;
                            X_.sched_fence();
                            // prefetch the words of the phase below for every hypothesis (and, where a sub-block may
                            // start, every slot, with the merge choice of every hypothesis: an in-bounds byte even
                            // where it is not used). The addresses need only this phase's state: the loads go out
                            // after this phase's words are read (so the wait for those does not cover them) and
                            // before the decode, which they overlap; the fences keep the compiler from moving them.
                            uint32_t n0 = c0, n1 = c1;
                            if (pi > 0 || cc > 0) {
                                constexpr int PN = pi > 0 ? pi - 1 : NPC - 1;
                                constexpr int PNw = MM::OFF(PN) >> 5;
                                const int su = GE::start(0, qq, ll);
                                const uint32_t* tsl = pi > 0 ? slot : slot_next;
                                if constexpr (BC) {
                                    const int gsl = bnd ? gp : gs;
                                    const int wi = ((gsl * Q + (((su >> 8) & (Q - 1)) | wL)) * NW + PNw) * 64 + (((su >> 2) & 63) | lL);
                                    n0 = tsl[wi];
                                    n1 = tsl[wi + 64];
                                    gv = s_gsel[G > 1 ? (ta >> lsub) * S + (su | sxL) : 0];
                                } else {
                                    const uint32_t* tb = tsl + X_.uni(((gs * Q + ((su >> 8) & (Q - 1))) * NW + PNw) * 64 + ((su >> 2) & 63));
                                    n0 = tb[lane_off];
                                    n1 = tb[lane_off + 64];
                                }
                            }
                            X_.sched_fence();
                            c0 = n0;
                            c1 = n1;
                            const uint32_t F = TWO_WORDS ? (uint32_t)(((((uint64_t)W0 << 32) | W1) >> (64 - o - NB_)) & ((1u << NB_) - 1u))
                                                         : (W0 >> (32 - o - NB_)) & ((1u << NB_) - 1u);
                            // n bits of F from position k on; the shift NB_ - k - n comes from tables indexed by jo
                            auto fld = [&](int sh, int nbit) -> int { return (int)((F >> sh) & ((1u << nbit) - 1u)); };
                            auto tab8 = [](uint32_t t, int i) -> int { return (int)((t >> (8 * i)) & 0xFFu); };
                            int h = 0, e = 0, pa = 0, pb = 0;
                            if constexpr (MD == 0) {  // e at 2 + ca, h at e
                                e = fld(tab8(((NB_ - 3) << 0) | ((NB_ - 3) << 8) | ((NB_ - 4) << 16) | ((NB_ - 4) << 24), jo), 1);
                                h = fld(NB_ - 1 - e, 1);
                            } else if constexpr (MD == 1) {  // p at 4 + 4 ca + cb, e at 2 + 4 ca + p, h at e
                                const int p = fld(tab8(((NB_ - 5) << 0) | ((NB_ - 6) << 8) | ((NB_ - 9) << 16) | ((NB_ - 10) << 24), jo), 1);
                                e = fld(tab8(((NB_ - 3) << 0) | ((NB_ - 3) << 8) | ((NB_ - 7) << 16) | ((NB_ - 7) << 24), jo) - p, 1);
                                h = fld(NB_ - 1 - e, 1);
                                pa = pb = p;
                            } else if constexpr (!EQ) {
                                if constexpr (PT == 1) {  // v3 at 8 + 10 ca + 3 cb (3 bits); e at 4 + 10 ca + idx; h at 2 e + c
                                    const int v3 = fld(tab8(((NB_ - 11) << 0) | ((NB_ - 14) << 8) | ((NB_ - 21) << 16) | ((NB_ - 24) << 24), jo), 3);
                                    const int idx = (0xEDEC >> (2 * v3)) & 3;
                                    cstar = idx >> 1;
                                    const int bsel = idx & 1;
                                    e = fld(tab8(((NB_ - 5) << 0) | ((NB_ - 5) << 8) | ((NB_ - 15) << 16) | ((NB_ - 15) << 24), jo) - idx, 1);
                                    h = fld(NB_ - 1 - 2 * e - cstar, 1);
                                    pb = bsel ^ cstar;
                                    pa = bsel;
                                } else {  // bsel at 4 + 6 ca + 2 cb + c; e at 2 + 6 ca + bsel; h at e
                                    const int bsel = fld(tab8(((NB_ - 5) << 0) | ((NB_ - 7) << 8) | ((NB_ - 11) << 16) | ((NB_ - 13) << 24), jo) - cstar, 1);
                                    e = fld(tab8(((NB_ - 3) << 0) | ((NB_ - 3) << 8) | ((NB_ - 9) << 16) | ((NB_ - 9) << 24), jo) - bsel, 1);
                                    h = fld(NB_ - 1 - e, 1);
                                    pb = bsel ^ cstar;
                                    pa = bsel;
                                }
                            } else {
                                if constexpr (PT == 1) {  // c at 6 + 4 ca + cb; e at 4 + 4 ca + c; h at 2 e + c
                                    cstar = fld(tab8(((NB_ - 7) << 0) | ((NB_ - 8) << 8) | ((NB_ - 11) << 16) | ((NB_ - 12) << 24), jo), 1);
                                    e = fld(tab8(((NB_ - 5) << 0) | ((NB_ - 5) << 8) | ((NB_ - 9) << 16) | ((NB_ - 9) << 24), jo) - cstar, 1);
                                    h = fld(NB_ - 1 - 2 * e - cstar, 1);
                                } else {  // e at 2 + 2 ca + c; h at e
                                    e = fld(tab8(((NB_ - 3) << 0) | ((NB_ - 3) << 8) | ((NB_ - 5) << 16) | ((NB_ - 5) << 24), jo) - cstar, 1);
                                    h = fld(NB_ - 1 - e, 1);
                                }
                                pa = pb = cstar;
                            }
                            if constexpr (MIDW) {
                                if (ph == mid_ph) {  // first tail-biting pass: only the state before mid_t is needed
                                    mid_val = (a.mid_t - 1) & 1 ? st : GE::mid(0, 2 * (jo >> 1) + e, qq, ll);
                                    stop = true;
                                    return;
                                }
                            } else {
                                recs[pi] = (uint32_t)(st | (gs << 10) | (e << 13) | (pa << 14) | (pb << 15));
                            }
                            const int Ln = X_.uni(2 * h + e);
                            st = X_.uni(GE::start(Ln, qq, ll));  // state at step ta - 1
                            sel = Ln;
                            cstar = X_.uni(cstar);
                            if (bnd) {  // sub-block start: the path came from the slot the merge chose
                                gs = (int)X_.readlane(gv, Ln);
                                sel = Ln + 4 * gs;
                            }
                        });
                        if constexpr (!MIDW) {
                            if (lane == 0) {
                                uint32_t* dst = (uint32_t*)s_rec + cc * (NPC / 2);
                                static_for<0, NPC / 2>([&](auto Wc) {
                                    constexpr int w = decltype(Wc)::value;
                                    dst[w] = recs[2 * w] | (recs[2 * w + 1] << 16);
                                });
                            }
                        }
                    }
                    X_.lds_sync();  // the records of chunk cc are written; chunk cc - 2 is in LDS; slot of cc + 1 free
                }
            };
            if (a.mid_st)
                walk(std::true_type{});
            else
                walk(std::false_type{});
            if (wv == 1) X_.wait_loads(0);  // no copy may still land in this workgroup's LDS after it ends
            if (wv == 0 && lane == 0) {
                if (a.mid_st) a.mid_st[n] = mid_val;
                a.best[n] = bi_all;
                if (a.end_st) a.end_st[n] = bi_all % S;
            }
            if (a.mid_st) return;
        }
    }
    if (!fast) {
        uint32_t* ring = (uint32_t*)(sm + SM.ring);
        const int nslot = SM.nslot, slot_words = SM.slot_words;
        const uint32_t* dummy = dm.bp;
        auto chunk_nwc = [&](int cc) {
            const int rp = (cc + 1) * NPC <= nph ? NPC : nph - cc * NPC;
            const int rb = TWO ? (rp / 2) * (MM::PPH(0) + MM::PPH(1)) + (rp & 1) * MM::PPH(0) : rp * MM::PPH(0);
            return rp == NPC ? NW : (rb + 31) / 32;
        };
        // copies of one chunk: 16-byte units u = i * 64 + lane for wave loads i = 0 .. nl-1
        auto nloads = [&](int cc) { return (G * Q * 16 * chunk_nwc(cc) + 63) / 64; };
        auto issue = [&](int cc) {
            const int units = G * Q * 16 * chunk_nwc(cc), nl = (units + 63) / 64;
            uint32_t* slot = ring + (cc % nslot) * slot_words;
            const long base = (long)cc * chunk_words;
            for (int i = 0; i < nl; i++) {
                const int u = i * 64 + lane;
                X_.load16(u < units ? dm.at(base + 4L * u) : dummy, slot + i * 256);
            }
        };
        for (int j = 0; j < nslot; j++)
            if (nchunk - 1 - j >= 0) issue(nchunk - 1 - j);
        int st = bi_all % S, gs = bi_all / S, cstar = 0;
        const int mid_ph = a.mid_st ? (a.mid_t - 1) >> 1 : -1;  // phase holding the step before mid_t
        int nbnd = ((T - 1) / sub) * sub, jb = (T - 1) / sub;  // largest sub-block start <= the walk position
        bool done = false;
        for (int cc = nchunk - 1; cc >= 0 && !done; cc--) {
            // this chunk's copies are done when only the copies of later-issued chunks are outstanding
            int later = 0;
            for (int j = 1; j < nslot && cc - j >= 0; j++) later += nloads(cc - j);
            X_.wait_loads(later);
            const uint32_t* slot = ring + (cc % nslot) * slot_words;
            const int nwc = chunk_nwc(cc);
            // word index of the first decision word of phase PI for output state sx
            auto word_at = [&](int sx, int PI) -> int {
                const int P = MM::OFF(PI) + (sx >> (8 + QB)) * MM::PBLK(MM::PT(PI));
                return ((gs * Q + ((sx >> 8) & (Q - 1))) * nwc + (P >> 5)) * 64 + ((sx >> 2) & 63);
            };
            uint32_t c0 = 0, c1 = 0;  // lane i: the two words of hypothesis i for the phase about to be walked
            int sel = 0;
            bool need = true;  // candidates not loaded (chunk start, or the gain slot changed)
            static_for<0, NPC>([&](auto Kc) {
                constexpr int pi = NPC - 1 - decltype(Kc)::value;
                constexpr int PT = MM::PT(pi);
                const int ta = cc * CK + 2 * pi;
                if (done || ta >= T) return;
                if (need) {  // exact words of this phase into every lane
                    const int wi = word_at(st, pi);
                    c0 = slot[wi];
                    c1 = slot[wi + 64];
                    sel = 0;
                    need = false;
                }
                const uint32_t W0 = X_.readlane(c0, sel), W1 = X_.readlane(c1, sel);
                const int qq = (st >> 8) & (Q - 1), ll = (st >> 2) & 63, bb = st >> (8 + QB), jo = st & 3;
                if constexpr (pi > 0) {  // the next phase's four candidates (inputs h e = 0..3 of this one)
                    const int sx = GE::start(((lane & 3) << (RB - 2)) | bb, qq, ll);
                    const int wi = word_at(sx, pi - 1);
                    c0 = slot[wi];
                    c1 = slot[wi + 64];
                }
                const int ca = jo >> 1, cb = jo & 1;
                const int P = MM::OFF(pi) + bb * MM::PBLK(PT);
                const int w0 = P >> 5;
                const uint64_t V = ((uint64_t)W0 << 32) | W1;
                auto bits = [&](int Pp, int nbit) -> int {  // nbit bits from push Pp on, first push highest
                    return (int)((V >> (64 - (Pp - 32 * w0) - nbit)) & ((1u << nbit) - 1u));
                };
                int h = 0, e = 0, pa = 0, pb = 0;  // pa / pb: parity class of steps ta / ta + 1
                if constexpr (MD == 0) {
                    e = bits(P + 2 + ca, 1);
                    h = bits(P + e, 1);
                } else if constexpr (MD == 1) {
                    const int PF = P + 2 + ca * 4;
                    const int p = bits(PF + 2 + cb, 1);
                    e = bits(PF + p, 1);
                    h = bits(P + e, 1);
                    pa = pb = p;
                } else if constexpr (!EQ) {
                    if constexpr (PT == 1) {  // D4 phase B: three sequential-min bits -> winner (c, b) = 0xEDEC map
                        const int PF = P + 4 + ca * 10;
                        const int v3 = bits(PF + 4 + 3 * cb, 3);
                        const int idx = (0xEDEC >> (2 * v3)) & 3;
                        cstar = idx >> 1;
                        const int bsel = idx & 1;
                        e = bits(PF + idx, 1);
                        h = bits(P + 2 * e + cstar, 1);
                        pb = bsel ^ cstar;
                        pa = bsel;
                    } else {  // D4 phase A, with the class chosen by the phase B that follows it
                        const int PF = P + 2 + ca * 6;
                        const int bsel = bits(PF + 2 + 2 * cb + cstar, 1);
                        e = bits(PF + bsel, 1);
                        h = bits(P + e, 1);
                        pb = bsel ^ cstar;
                        pa = bsel;
                    }
                } else {
                    if constexpr (PT == 1) {  // EQ phase B
                        const int PF = P + 4 + ca * 4;
                        cstar = bits(PF + 2 + cb, 1);
                        e = bits(PF + cstar, 1);
                        h = bits(P + 2 * e + cstar, 1);
                    } else {  // EQ phase A
                        const int PF = P + 2 + ca * 2;
                        e = bits(PF + cstar, 1);
                        h = bits(P + e, 1);
                    }
                    pa = pb = cstar;
                }
                const int ph = ta >> 1;
                // the phase's output state, slot, intermediate bit and classes (the step-ta state follows from them)
                s_rec[ph] = (uint16_t)(st | (gs << 10) | (e << 13) | (pa << 14) | (pb << 15));
                if (ph == mid_ph) {  // first tail-biting pass: only the state before mid_t is needed
                    if (lane == 0) a.mid_st[n] = (a.mid_t - 1) & 1 ? st : GE::mid(bb, 2 * ca + e, qq, ll);
                    done = true;
                    return;
                }
                if (ta == 0) return;
                sel = 2 * h + e;
                st = GE::start((h << (RB - 1)) | (e << (RB - 2)) | bb, qq, ll);  // state at step ta - 1
                if (ta == nbnd) {  // sub-block start: the path came from the slot the merge chose
                    if (G > 1) {
                        const int gn = (int)X_.readlane(s_gsel[jb * S + st], 0);
                        need = gn != gs;
                        gs = gn;
                    }
                    nbnd -= sub;
                    jb--;
                }
            });
            if (!done && cc - nslot >= 0) issue(cc - nslot);
        }
        X_.wait_loads(0);  // no copy may still land in this workgroup's LDS after it ends
        if (lane == 0) {
            a.best[n] = bi_all;
            if (a.end_st) a.end_st[n] = bi_all % S;
        }
        if (done) return;
    }

    // ---- reconstruction and code (tcq_viterbi.cu:662-682) -------------------------------------------
    float* rn = a.rec + (size_t)n * a.ld;
    for (int t = out_t0; t < T; t += out_dt) {
        const uint32_t rr = s_rec[t >> 1];
        const int so = rr & 1023, gg = (rr >> 10) & 7;
        // odd step: the phase's output state; even step: its intermediate state (block bits, e, ca, q, lane of so)
        const int stt = (t & 1) ? so
                                : GE::mid(so >> (8 + QB), 2 * ((so >> 1) & 1) + ((rr >> 13) & 1), (so >> 8) & (Q - 1),
                                          (so >> 2) & 63);
        const int par = (rr >> ((t & 1) ? 15 : 14)) & 1;
        const int lb = mk.label(stt);
        const bool hi = mix > 0 && ((t / mix) & 1);
        const int Ut = hi ? U_hi : U;
        const int gi = cand ? (int)s_gc[(t / sub) * G + gg] : gg;
        const float gt = hi ? s_gain_hi[gi] : s_gain[gi];
        const float* tt = (hi ? s_tab_hi : s_tab) + lb * Ut;
        const float xt = s_x[t];
        float bestd = kSent, val = 0.f;
        int bu = 0;
        for (int u = MD ? par : 0; u < Ut; u += MD ? 2 : 1) {
            const float v = gt * tt[u];
            const float d = xt - v;
            const float dd = d * d;
            if (dd < bestd) {
                bestd = dd;
                val = v;
                bu = u;
            }
        }
        const int tp = (t + a.rot) % a.ld;
        rn[tp] = val;
        if (a.code) a.code[(size_t)n * a.ld + tp] = (gi << 16) | (lb * Ut + bu);
    }
}

#undef LTQ_CSP
#undef LTQ_PUSH0


// Both tail-biting passes of one tile in one workgroup (the two tcq_viterbi calls of src/tcq_proto.py:584-609
// with tb_passes = 2, same gain slots): pass 1 leaves the state before its mid_t in a1.mid_st; after a full
// barrier (the pass-1 walk done, the store visible) every thread reads it back coherently and pass 2 starts and
// closes there. The two passes lay LDS out independently; the barrier ends every use of pass 1's layout.
template <int NU, int RB, int MD, int NL, class X>
LTQ_DEV void tcq_tile_tb(const TcqArgs& a1, const TcqArgs& a2, X& X_, int lds_max)
{
    int init = -1;
    // one copy of the tile body, run twice (two inlined copies would double the code the instruction cache holds)
#pragma nounroll
    for (int p = 0; p < 2; p++) {
        tcq_tile<NU, RB, MD, NL>(p == 0 ? a1 : a2, X_, lds_max, init);
        if (p == 0) {
            X_.sync();
            // pass 1's traceback pulled its decision words through this CU's L1; pass 2 rewrites the same
            // scratch (stores bypass L1), so the stale lines must go before pass 2's traceback reads them back
            X_.acquire();
            init = X_.uni(X_.load_coherent(a1.mid_st + X_.tile()));
        }
    }
}

// ---- host side: argument validation and dispatch, shared by the gfx950 entry point and the CPU emulation ----

// The reference's validation (tcq_viterbi.cu:748-751, 762-763) plus this implementation's limits.
inline int tcq_check(const TcqArgs& a)
{
    const int G = a.G, Gfull = a.Gfull, U = a.U, U_hi = a.U_hi, sub = a.sub, T = a.T, S = a.S, pp = a.pp, nl = a.nl;
    if (G > kMaxG || Gfull > kMaxG || (!a.gcand && Gfull != G) || U > kMaxU || U_hi > kMaxU || sub <= 0 ||
        T % sub != 0 || (sub & 1) || T / sub > kMaxSubs || T > kMaxT || sub > 32 || sub * G * nl * (pp ? 2 : 1) > 4096 ||
        (pp && (S != 1024 || a.mix > 0 || (T & 1))) || (pp >= 2 && ((T & 3) || (sub & 3))) || pp > 3 || pp < 0 ||
        (nl != 4 && nl != 8 && nl != 16 && nl != 32) || a.ld < T || (S != 1024 && nl != 4) || nl * U > 4 * kMaxU ||
        nl * U_hi > 4 * kMaxU)
        return -1;
    if ((S != 1024 && S != 256) || (G != 1 && G != 2 && G != 3 && G != 4 && G != 8)) return -1;
    // buffers are checked only when there are tiles: with none, torch hands over null pointers and the call must
    // reach the zero-tile return code, as the reference's unchecked zero-block launch does
    if (T <= 0 || (a.N > 0 && (!a.bp || (pp && !a.pbits && a.tile_words <= 0) || !a.best || !a.rec))) return -1;
    return 0;
}

// decision words one tile of this configuration needs (the instance tcq_dispatch selects), -1 if none serves it
inline long tcq_needed_words(const TcqArgs& a)
{
    if (a.S == 256) return needed_words<8, 2, 0>(a.T, a.G);
    const bool r3 = a.G > 4;
    switch (a.pp) {
        case 0: return r3 ? needed_words<10, 3, 0>(a.T, a.G) : needed_words<10, 2, 0>(a.T, a.G);
        case 1: return r3 ? needed_words<10, 3, 1>(a.T, a.G) : needed_words<10, 2, 1>(a.T, a.G);
        case 2: return r3 ? needed_words<10, 3, 2>(a.T, a.G) : needed_words<10, 2, 2>(a.T, a.G);
        case 3: return r3 ? needed_words<10, 3, 3>(a.T, a.G) : needed_words<10, 2, 3>(a.T, a.G);
        default: return -1;
    }
}

// decision words available per tile: the compact window, or bp + pbits in the reference's shapes
inline long tcq_capacity_words(const TcqArgs& a)
{
    return a.tile_words > 0 ? a.tile_words : scratch_words(a.scratch_T > 0 ? a.scratch_T : a.T, a.G, a.S, a.pp);
}

// Calls f.template run<NU, RB, MD, NL>() for the instance serving a (RB = 3 when G = 8 at S = 1024, so that a
// workgroup stays at 16 wavefronts), after checking that the packed decisions fit the caller's scratch.
template <class F>
int tcq_dispatch(const TcqArgs& a, const F& f)
{
    auto go = [&](auto nu, auto rb, auto md) -> int {
        constexpr int NU = decltype(nu)::value, RB = decltype(rb)::value, MD = decltype(md)::value;
        if (needed_words<NU, RB, MD>(a.T, a.G) > tcq_capacity_words(a)) return -1;
        switch (a.nl) {
            case 4: return f.template run<NU, RB, MD, 4>();
            case 8: return f.template run<NU, RB, MD, 8>();
            case 16: return f.template run<NU, RB, MD, 16>();
            default: return f.template run<NU, RB, MD, 32>();
        }
    };
    using I8 = std::integral_constant<int, 8>;
    using I10 = std::integral_constant<int, 10>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    if (a.S == 256) {
        if (needed_words<8, 2, 0>(a.T, a.G) > tcq_capacity_words(a)) return -1;
        return f.template run<8, 2, 0, 4>();
    }
    const bool r3 = a.G > 4;
    auto by_md = [&](auto rb) -> int {
        switch (a.pp) {
            case 0: return go(I10{}, rb, std::integral_constant<int, 0>{});
            case 1: return go(I10{}, rb, std::integral_constant<int, 1>{});
            case 2: return go(I10{}, rb, std::integral_constant<int, 2>{});
            default: return go(I10{}, rb, std::integral_constant<int, 3>{});
        }
    };
    (void)sizeof(I8);
    return r3 ? by_md(I3{}) : by_md(I2{});
}

}  // namespace ltq
