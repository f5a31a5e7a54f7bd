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
#include <cstring>
#include <memory>
#include <thread>
#include <vector>

using namespace ltq;

struct CpuX {
    int tid_, tile_, nthr_;
    char* smem_;
    std::barrier<>* blk_;
    std::barrier<>** waves_;
    int tid() const { return tid_; }
    int tile() const { return tile_; }
    int nthreads() const { return nthr_; }
    void* smem() const { return smem_; }
    void sync() const { blk_->arrive_and_wait(); }
    void wave_sync() const { waves_[tid_ >> 6]->arrive_and_wait(); }
    uint32_t push(uint32_t acc, bool bit) const { return acc + acc + (uint32_t)bit; }
};

template <int NU, int MD>
static int run(const TcqArgs& a)
{
    const Smem L = smem_layout<NU, MD>(a.T, a.G, a.nl, a.Gfull, a.sub);
    constexpr int WCH = Mode<NU, MD>::FG == 1 ? 4 : 1;
    if (WCH * a.G * Mode<NU, MD>::NW * 64 * 4 > L.gsel - L.exch) return -1;
    if (L.total > 160 * 1024) return -1;
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
        std::vector<std::thread> th;
        for (int t = 0; t < nthr; t++) {
            th.emplace_back([&, t]() {
                CpuX x{t, n, nthr, smem.data(), &blk, ptrs.data()};
                tcq_tile<NU, MD>(a, x);
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
    if (S == 256) return run<8, 0>(a);
    if (pp == 0) return run<10, 0>(a);
    if (pp == 1) return run<10, 1>(a);
    if (pp == 2) return run<10, 2>(a);
    return run<10, 3>(a);
}
