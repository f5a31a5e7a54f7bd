// TEST INFRASTRUCTURE: host (CPU) emulation of the gfx950 TCQ Viterbi kernel.
//
// Compiles the product kernel body (ltq-research_amd/csrc/tcq_trellis.h) for the host with one std::thread
// per lane and std::barrier for workgroup / wavefront synchronisation, so that layout, indexing and
// synchronisation bugs of the kernel show up on the CPU (optionally under AddressSanitizer) and can be
// compared with the oracle before a GPU run. The decision-word packing is acc = 2 * acc + bit, as the
// kernel's v_alignbit does.
#define LTQ_DEV inline
#define LTQ_HD inline
#include "../../ltq-research_amd/csrc/tcq_trellis.h"

#include <barrier>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <memory>
#include <thread>
#include <type_traits>
#include <vector>

using namespace ltq;

struct CpuX {
    int tid_, tile_, nthr_;
    char* smem_;
    std::barrier<>* blk_;
    std::barrier<>** waves_;
    uint32_t* xch_;  // per-wave lane exchange for shuffles
    int tid() const { return tid_; }
    int wave() const { return tid_ >> 6; }
    int tile() const { return tile_; }
    int nthreads() const { return nthr_; }
    void* smem() const { return smem_; }
    void sync() const { blk_->arrive_and_wait(); }
    void lds_sync() const { blk_->arrive_and_wait(); }
    uint32_t push_sign(uint32_t acc, float d) const
    {
        uint32_t b;
        std::memcpy(&b, &d, 4);
        return (acc << 1) | (b >> 31);
    }
    float fmin(float x, float y) const { return std::fmin(x, y); }
    uint32_t xor_lane(uint32_t v, int m) const
    {
        const int w = tid_ >> 6;
        xch_[tid_] = v;
        waves_[w]->arrive_and_wait();
        const uint32_t r = xch_[w * 64 + ((tid_ & 63) ^ m)];
        waves_[w]->arrive_and_wait();
        return r;
    }
    float shfl_xor(float v, int m) const
    {
        uint32_t b;
        std::memcpy(&b, &v, 4);
        b = xor_lane(b, m);
        float r;
        std::memcpy(&r, &b, 4);
        return r;
    }
    int shfl_xor(int v, int m) const { return (int)xor_lane((uint32_t)v, m); }
    int uni(int v) const { return v; }
    int load_coherent(const int* p) const { return *p; }
    void acquire() const {}
    void sched_fence() const {}
    int opaque_zero() const { return 0; }
    void pin(uint32_t&) const {}
    void pin_s(uint32_t&) const {}
    // (value, index) minimum over the wavefront, lowest index on ties, in every lane (the GPU leaves it in lane 63)
    void wave_min(float& bv, int& bi) const
    {
        for (int off = 1; off < 64; off <<= 1) {
            const float ov = shfl_xor(bv, off);
            const int oi = shfl_xor(bi, off);
            if (ov < bv || (ov == bv && oi < bi)) {
                bv = ov;
                bi = oi;
            }
        }
    }
    uint32_t readlane(uint32_t v, int l) const
    {
        const int w = tid_ >> 6;
        xch_[tid_] = v;
        waves_[w]->arrive_and_wait();
        const uint32_t r = xch_[w * 64 + l];
        waves_[w]->arrive_and_wait();
        return r;
    }
    // the GPU copy is asynchronous; here it completes at once
    void load16(const uint32_t* src, uint32_t* lds_wave_base) const
    {
        std::memcpy(lds_wave_base + 4 * (tid_ & 63), src, 16);
    }
    // a wave's copies have landed for every lane once the wave has waited: model that with a wave barrier
    void wait_loads(int) const { waves_[tid_ >> 6]->arrive_and_wait(); }
};

constexpr int kLdsMax = 160 * 1024;  // gfx950 LDS per workgroup

struct CpuRun {
    const TcqArgs& a;
    template <int NU, int RB, int MD, int NL>
    int run() const
    {
        const Smem L = smem_layout<NU, RB, MD, NL>(a.T, a.G, a.Gfull, a.sub, kLdsMax);
        if (L.total > kLdsMax) return -1;
        const int nthr = 64 * a.G * Geo<NU, RB>::Q;
        const int nw = nthr / 64;
        std::vector<char> smem(L.total + 64);
        for (int n = 0; n < a.N; n++) {
            std::memset(smem.data(), 0xA5, smem.size());  // garbage, like uninitialised LDS
            std::barrier<> blk(nthr);
            std::vector<std::unique_ptr<std::barrier<>>> wv;
            std::vector<std::barrier<>*> ptrs;
            for (int g = 0; g < nw; g++) {
                wv.emplace_back(new std::barrier<>(64));
                ptrs.push_back(wv.back().get());
            }
            std::vector<uint32_t> xch(nthr);
            std::vector<std::thread> th;
            for (int t = 0; t < nthr; t++) {
                th.emplace_back([&, t]() {
                    CpuX x{t, n, nthr, smem.data(), &blk, ptrs.data(), xch.data()};
                    tcq_tile<NU, RB, MD, NL>(a, x, kLdsMax);
                });
            }
            for (auto& t : th) t.join();
        }
        return 0;
    }
};

struct CpuRunTb {
    const TcqArgs& a1;
    const TcqArgs& a2;
    template <int NU, int RB, int MD, int NL>
    int run() const
    {
        const Smem L1 = smem_layout<NU, RB, MD, NL>(a1.T, a1.G, a1.Gfull, a1.sub, kLdsMax);
        const Smem L2 = smem_layout<NU, RB, MD, NL>(a2.T, a2.G, a2.Gfull, a2.sub, kLdsMax);
        const int total = L1.total > L2.total ? L1.total : L2.total;
        if (total > kLdsMax) return -1;
        const int nthr = 64 * a2.G * Geo<NU, RB>::Q;
        const int nw = nthr / 64;
        std::vector<char> smem(total + 64);
        for (int n = 0; n < a2.N; n++) {
            std::memset(smem.data(), 0xA5, smem.size());
            std::barrier<> blk(nthr);
            std::vector<std::unique_ptr<std::barrier<>>> wv;
            std::vector<std::barrier<>*> ptrs;
            for (int g = 0; g < nw; g++) {
                wv.emplace_back(new std::barrier<>(64));
                ptrs.push_back(wv.back().get());
            }
            std::vector<uint32_t> xch(nthr);
            std::vector<std::thread> th;
            for (int t = 0; t < nthr; t++) {
                th.emplace_back([&, t]() {
                    CpuX x{t, n, nthr, smem.data(), &blk, ptrs.data(), xch.data()};
                    tcq_tile_tb<NU, RB, MD, NL>(a1, a2, x, kLdsMax);
                });
            }
            for (auto& t : th) t.join();
        }
        return 0;
    }
};

struct CpuCheck {
    template <int NU, int RB, int MD, int NL>
    int run() const
    {
        return 0;
    }
};

extern "C" int tcq_viterbi_tb_emu(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                                  uint32_t* bp, uint8_t* gsel, int* mid_buf, int* end_st, const float* tab_hi,
                                  const float* gains_hi, uint8_t* gcand, int* best, int* code, int tail, int N, int T,
                                  int S, int U, int G, int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3,
                                  int m4, int nl, int ld, int rot, uint32_t* pbits, int pp, int steps1, int rot1,
                                  int mid_t1)
{
    TcqArgs a2{x, w, tab, gains, rec, bp, gsel, mid_buf, end_st, tab_hi, gains_hi, gcand, best, code, nullptr,
               0, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pbits, pp};
    TcqArgs a1{x, w, tab, gains, rec, bp, gsel, nullptr, nullptr, tab_hi, gains_hi, gcand, best, nullptr, mid_buf,
               mid_t1, 0, N, steps1, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot1, pbits, pp};
    a1.scratch_T = T;  // pass 1 works inside the scratch sized for the closing pass
    if (!mid_buf || steps1 <= 0 || steps1 > T || mid_t1 <= 0 || mid_t1 > steps1) return -1;
    if (tcq_check(a1) != 0 || tcq_check(a2) != 0) return -1;
    if (N <= 0) return N == 0 ? 0 : -1;
    const int rc = tcq_dispatch(a1, CpuCheck{});
    if (rc != 0) return rc;
    return tcq_dispatch(a2, CpuRunTb{a1, a2});
}

extern "C" int tcq_viterbi_emu(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                               uint32_t* bp, uint8_t* gsel, const int* init_st, int* end_st, const float* tab_hi,
                               const float* gains_hi, uint8_t* gcand, int* best, int* code, int* mid_st, int mid_t,
                               int tail, int N, int T, int S, int U, int G, int Gfull, int m, int sub, int U_hi, int mix,
                               int m2, int m3, int m4, int nl, int ld, int rot, uint32_t* pbits, int pp)
{
    TcqArgs a{x, w, tab, gains, rec, bp, gsel, init_st, end_st, tab_hi, gains_hi, gcand, best, code, mid_st,
              mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pbits, pp};
    if (tcq_check(a) != 0) return -1;
    if (N <= 0) return N == 0 ? 0 : -1;
    return tcq_dispatch(a, CpuRun{a});
}

// the compact scratch window of the allocation-free entry point: tile n's decision words at bp + n * tile_words
extern "C" long tcq_needed_words_emu(int T, int S, int G, int pp)
{
    TcqArgs a{};
    a.T = T;
    a.S = S;
    a.G = G;
    a.pp = pp;
    return tcq_needed_words(a);
}

extern "C" int tcq_viterbi_compact_emu(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                                       uint32_t* bp, const int* init_st, int* end_st, uint8_t* gcand, int* best,
                                       int* code, int* mid_st, int mid_t, int tail, int N, int T, int S, int U, int G,
                                       int Gfull, int m, int sub, int nl, int m2, int m3, int ld, int rot, int pp,
                                       long tile_words)
{
    TcqArgs a{x, w, tab, gains, rec, bp, nullptr, init_st, end_st, tab, gains, gcand, best, code, mid_st,
              mid_t, tail, N, T, S, U, G, Gfull, m, sub, U, 0, m2, m3, 0, nl, ld, rot, nullptr, pp};
    a.tile_words = tile_words;
    if (tile_words <= 0 || tcq_check(a) != 0) return -1;
    if (N <= 0) return N == 0 ? 0 : -1;
    return tcq_dispatch(a, CpuRun{a});
}
