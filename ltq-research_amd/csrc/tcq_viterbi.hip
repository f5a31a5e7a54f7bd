// gfx950 build of the TCQ Viterbi kernel and the drop-in C ABI (tcq_viterbi, lut_subs_quant).
//
// C ABI replaced: src/cuda/tcq_viterbi.cu:743-766 (tcq_viterbi) and :806-811 (lut_subs_quant); the argument
// lists, buffer shapes and return codes are the reference's (0 = ok, -1 = rejected configuration, otherwise
// the HIP error code of the launch). The caller allocates every buffer, as in the reference; bp / pbits are
// used as opaque scratch for this kernel's own decision-word format, gsel is not touched. A configuration
// whose packed decisions do not fit bp + pbits is rejected with -1.
#include <hip/hip_runtime.h>
#include <stdlib.h>

#include <mutex>

#include "ltq_timing.h"
#include "tcq_launch.h"

#include "ltq_hip.h"

namespace ltq {

// instantiated in tcq_inst_*.hip (compiled in parallel)
#define LTQ_EXT(NU, RB, MD, NL)                                                \
    extern template int launch<NU, RB, MD, NL>(const TcqArgs&, hipStream_t); \
    extern template int launch_tb<NU, RB, MD, NL>(const TcqArgs&, const TcqArgs&, hipStream_t);
#define LTQ_EXT_MD(MD)                                                                                \
    LTQ_EXT(10, 2, MD, 4) LTQ_EXT(10, 2, MD, 8) LTQ_EXT(10, 2, MD, 16) LTQ_EXT(10, 2, MD, 32)        \
    LTQ_EXT(10, 3, MD, 4) LTQ_EXT(10, 3, MD, 8) LTQ_EXT(10, 3, MD, 16) LTQ_EXT(10, 3, MD, 32)
LTQ_EXT(8, 2, 0, 4)
LTQ_EXT_MD(0) LTQ_EXT_MD(1) LTQ_EXT_MD(2) LTQ_EXT_MD(3)
#undef LTQ_EXT_MD
#undef LTQ_EXT

// per-device attributes of the current device, cached per device ordinal (a process may drive several GPUs)
constexpr int kMaxDevices = 64;

static int device_attr(hipDeviceAttribute_t attr, int (&cache)[kMaxDevices])
{
    int dev = 0, x = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return -1;
    if (dev < kMaxDevices && cache[dev] > 0) return cache[dev];
    if (hipDeviceGetAttribute(&x, attr, dev) != hipSuccess) return -1;
    if (dev < kMaxDevices) cache[dev] = x;
    return x;
}

int device_lds_max()
{
    static int cache[kMaxDevices] = {};
    return device_attr(hipDeviceAttributeMaxSharedMemoryPerBlock, cache);
}

int device_cu_count()
{
    static int cache[kMaxDevices] = {};
    return device_attr(hipDeviceAttributeMultiprocessorCount, cache);
}

struct GpuLaunch {
    const TcqArgs& a;
    hipStream_t st;
    template <int NU, int RB, int MD, int NL>
    int run() const
    {
        return launch<NU, RB, MD, NL>(a, st);
    }
};

// capacity check only (tcq_dispatch rejects what does not fit the scratch before calling run)
struct GpuLaunchTbCheck {
    template <int NU, int RB, int MD, int NL>
    int run() const
    {
        return 0;
    }
};

struct GpuLaunchTb {
    const TcqArgs& a1;
    const TcqArgs& a2;
    hipStream_t st;
    template <int NU, int RB, int MD, int NL>
    int run() const
    {
        return launch_tb<NU, RB, MD, NL>(a1, a2, st);
    }
};

}  // namespace ltq

using ltq::TcqArgs;

extern "C" int tcq_viterbi(const float* x, const float* w, const float* tab, const float* gains, float* rec, uint32_t* bp,
                           uint8_t* gsel, const int* init_st, int* end_st, const float* tab_hi, const float* gains_hi,
                           uint8_t* gcand, int* best, int* code, int* mid_st, int mid_t, int tail, int N, int T, int S,
                           int U, int G, int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3, int m4, int nl,
                           int ld, int rot, uint32_t* pbits, int pp, void* stream)
{
    using namespace ltq;
    TcqArgs a{x, w, tab, gains, rec, bp, gsel, init_st, end_st, tab_hi, gains_hi, gcand, best, code, mid_st,
              mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pbits, pp};
    // the reference also rejects any label count but 4 when TCQ_BLOCK is set (tcq_viterbi.cu:750)
    if (tcq_check(a) != 0 || (getenv("TCQ_BLOCK") && nl != 4)) return -1;
    if (N <= 0) return N == 0 ? (int)hipErrorInvalidConfiguration : -1;  // a 0-block launch, as the reference gets
    const int rc = tcq_dispatch(a, GpuLaunch{a, (hipStream_t)stream});
    if (rc != 0) return rc;
    return (int)hipGetLastError();
}

// Both tail-biting passes in one launch (the two calls of src/tcq_proto.py:584-609 with tb_passes = 2 and the
// same gain slots): the arguments of the closing pass (init_st: the [N] buffer pass 1 leaves its middle states
// in, read back by the same workgroup) and pass 1's steps, rotation and mid_t.
extern "C" int tcq_viterbi_tb(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                              uint32_t* bp, uint8_t* gsel, int* mid_buf, int* end_st, const float* tab_hi,
                              const float* gains_hi, uint8_t* gcand, int* best, int* code, int tail, int N, int T, int S,
                              int U, int G, int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3, int m4,
                              int nl, int ld, int rot, uint32_t* pbits, int pp, int steps1, int rot1, int mid_t1,
                              void* stream)
{
    using namespace ltq;
    TcqArgs a2{x, w, tab, gains, rec, bp, gsel, mid_buf, end_st, tab_hi, gains_hi, gcand, best, code, nullptr,
               0, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pbits, pp};
    TcqArgs a1{x, w, tab, gains, rec, bp, gsel, nullptr, nullptr, tab_hi, gains_hi, gcand, best, nullptr, mid_buf,
               mid_t1, 0, N, steps1, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot1, pbits, pp};
    a1.scratch_T = T;  // pass 1 works inside the scratch sized for the closing pass
    if (!mid_buf || steps1 <= 0 || steps1 > T || mid_t1 <= 0 || mid_t1 > steps1) return -1;
    if (tcq_check(a1) != 0 || tcq_check(a2) != 0 || (getenv("TCQ_BLOCK") && nl != 4)) return -1;
    if (N <= 0) return N == 0 ? (int)hipErrorInvalidConfiguration : -1;
    // pass 1 must fit the scratch of the instance pass 2 selects (it has fewer steps)
    int rc = tcq_dispatch(a1, GpuLaunchTbCheck{});
    if (rc != 0) return rc;
    rc = tcq_dispatch(a2, GpuLaunchTb{a1, a2, (hipStream_t)stream});
    if (rc != 0) return rc;
    return (int)hipGetLastError();
}

// ---- the allocation-free entry point ---------------------------------------------------------------------
// Decision scratch in a file-scope device array. Each GPU that loads the library holds its own copy until the
// process ends; host code reaches a device's copy only through the address hipGetSymbolAddress returns while
// that device is current (the array's name is a host-side stand-in), kept per device.
namespace {

constexpr size_t kStaticScratchBytes = size_t(96) << 20;
static __device__ __align__(256) uint32_t scratch[kStaticScratchBytes / 4];

std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// this device's copy of the array, looked up once per device
int static_scratch(void** out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= 64) return -1;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!ptr) return -1;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

extern "C" long tcq_viterbi_static_bytes(void) { return (long)kStaticScratchBytes; }

extern "C" int tcq_viterbi_static(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                                  const int* init_st, int* end_st, const float* tab_hi, const float* gains_hi, int* best,
                                  int* code, int* mid_st, int mid_t, int tail, int N, int T, int S, int U, int G,
                                  int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3, int m4, int nl, int ld,
                                  int rot, int pp, void* stream)
{
    using namespace ltq;
    // validation runs on stand-in scratch pointers (tcq_check only tests them for null; they are replaced before
    // the launch): the sizes come first, so an oversized call is refused before any device is touched
    uint32_t* const probe = reinterpret_cast<uint32_t*>(uintptr_t(256));
    const bool cand = G < Gfull;
    TcqArgs a{x, w, tab, gains, rec, probe, nullptr, init_st, end_st, tab_hi, gains_hi,
              cand ? reinterpret_cast<uint8_t*>(probe) : nullptr, best, code, mid_st, mid_t, tail, N, T, S, U, G,
              Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, nullptr, pp};
    if (N <= 0 || T <= 0 || G <= 0 || sub <= 0) return -1;
    const long need = tcq_needed_words(a);
    if (need <= 0) return -1;
    a.tile_words = (need + 63) / 64 * 64;  // 256-byte aligned tile windows
    const size_t dec_bytes = (size_t)N * (size_t)a.tile_words * 4;
    const size_t cand_bytes = cand ? ((size_t)N * (T / sub) * G + 255) / 256 * 256 : 0;
    if (dec_bytes + cand_bytes > kStaticScratchBytes) return -2;
    if (tcq_check(a) != 0 || (getenv("TCQ_BLOCK") && nl != 4)) return -1;
    void* base = nullptr;
    if (const int rc = static_scratch(&base)) return rc;
    a.bp = static_cast<uint32_t*>(base);
    a.gcand = cand ? static_cast<uint8_t*>(base) + dec_bytes : nullptr;
    const int rc = tcq_dispatch(a, GpuLaunch{a, (hipStream_t)stream});
    if (rc != 0) return rc;
    return (int)hipGetLastError();
}

extern "C" int ltq_viterbi_timing(void* start_event, void* stop_event, int launches)
{
    if (launches < 0) return -1;
    ltq::viterbi_timing.arm((hipEvent_t)start_event, (hipEvent_t)stop_event, launches);
    return 0;
}

extern "C" int ltq_kernel_timing(void* start_event, void* stop_event, int launches)
{
    if (launches < 0) return -1;
    ltq::kernel_timing.arm((hipEvent_t)start_event, (hipEvent_t)stop_event, launches);
    return 0;
}
