// TEST INFRASTRUCTURE: host (CPU) emulation of the gfx950 TCQ Viterbi kernel.
//
// Compiles the product kernel body (ltq-research_amd/csrc/tcq_kernel.h) for the host with one std::thread
// per lane and std::barrier for workgroup / wavefront synchronisation, so that layout, indexing and
// synchronisation bugs of the kernel show up on the CPU (optionally under AddressSanitizer) and can be
// compared with the oracle before a GPU run. The decision-word packing is acc = 2 * acc + bit, as the
// kernel's v_addc does.
#define LTQ_DEV inline
#define LTQ_HD inline
#include "../../ltq-research_amd/csrc/tcq_kernel.h"

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
    uint32_t* xch_;  // per-wave lane exchange for readlane
    int tid() const { return tid_; }
    int wave() const { return tid_ >> 6; }
    int tile() const { return tile_; }
    int nthreads() const { return nthr_; }
    void* smem() const { return smem_; }
    void sync() const { blk_->arrive_and_wait(); }
    void lds_sync() const { blk_->arrive_and_wait(); }
    void wave_sync() const { waves_[tid_ >> 6]->arrive_and_wait(); }
    uint32_t push_sign(uint32_t acc, float d) const
    {
        uint32_t b;
        std::memcpy(&b, &d, 4);
        return (acc << 1) | (b >> 31);
    }
    float fmin(float x, float y) const { return std::fmin(x, y); }
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
    template <int N>
    void wait_loads() const {}
};

constexpr int kLdsMax = 160 * 1024;  // gfx950 LDS per workgroup

template <int NU, int MD, int NL>
static int run(const TcqArgs& a)
{
    const Smem L = smem_layout<NU, MD, NL>(a.T, a.G, a.Gfull, a.sub, kLdsMax);
    if (L.total > kLdsMax) return -1;
    const int nthr = 64 * a.G;
    std::vector<char> smem(L.total + 64);
    for (int n = 0; n < a.N; n++) {
        std::memset(smem.data(), 0xA5, smem.size());  // garbage, like uninitialised LDS
        std::barrier<> blk(nthr);
        std::vector<std::unique_ptr<std::barrier<>>> wv;
        std::vector<std::barrier<>*> ptrs;
        for (int g = 0; g < a.G; g++) {
            wv.emplace_back(new std::barrier<>(64));
            ptrs.push_back(wv.back().get());
        }
        std::vector<uint32_t> xch(nthr);
        std::vector<std::thread> th;
        for (int t = 0; t < nthr; t++) {
            th.emplace_back([&, t]() {
                CpuX x{t, n, nthr, smem.data(), &blk, ptrs.data(), xch.data()};
                tcq_tile<NU, MD, NL>(a, x, kLdsMax);
            });
        }
        for (auto& t : th) t.join();
    }
    return 0;
}

extern "C" int tcq_viterbi_emu(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                               uint32_t* bp, uint8_t* gsel, const int* init_st, int* end_st, const float* tab_hi,
                               const float* gains_hi, uint8_t* gcand, int* best, int* code, int* mid_st, int mid_t,
                               int tail, int N, int T, int S, int U, int G, int Gfull, int m, int sub, int U_hi, int mix,
                               int m2, int m3, int m4, int nl, int ld, int rot, uint32_t* pbits, int pp)
{
    if (G > kMaxG || Gfull > kMaxG || (!gcand && Gfull != G) || U > kMaxU || U_hi > kMaxU || sub <= 0 || T % sub != 0 ||
        (sub & 1) || T / sub > kMaxSubs || T > kMaxT || sub > 32 || sub * G * nl * (pp ? 2 : 1) > 4096 ||
        (pp && (S != 1024 || mix > 0 || (T & 1))) || (pp >= 2 && ((T & 3) || (sub & 3))) || pp > 3 || pp < 0 ||
        (nl != 4 && nl != 8 && nl != 16 && nl != 32) || ld < T || (S != 1024 && nl != 4) || nl * U > 4 * kMaxU ||
        nl * U_hi > 4 * kMaxU)
        return -1;
    if ((S != 1024 && S != 256) || (G != 1 && G != 2 && G != 3 && G != 4 && G != 8)) return -1;
    if (pp == 1 && (T & 3)) return -1;
    if (S == 256 && T < 8) return -1;
    TcqArgs a{x, w, tab, gains, rec, bp, gsel, init_st, end_st, tab_hi, gains_hi, gcand, best, code, mid_st,
              mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pbits, pp};
    if (S == 256) return run<8, 0, 4>(a);
    auto by_nl = [&](auto md) -> int {
        constexpr int MD = decltype(md)::value;
        switch (nl) {
            case 4: return run<10, MD, 4>(a);
            case 8: return run<10, MD, 8>(a);
            case 16: return run<10, MD, 16>(a);
            default: return run<10, MD, 32>(a);
        }
    };
    if (pp == 0) return by_nl(std::integral_constant<int, 0>{});
    if (pp == 1) return by_nl(std::integral_constant<int, 1>{});
    if (pp == 2) return by_nl(std::integral_constant<int, 2>{});
    return by_nl(std::integral_constant<int, 3>{});
}
