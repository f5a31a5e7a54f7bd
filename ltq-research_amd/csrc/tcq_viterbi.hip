// gfx950 build of the TCQ Viterbi kernel and the drop-in C ABI (tcq_viterbi, lut_subs_quant).
//
// C ABI replaced: src/cuda/tcq_viterbi.cu:743-766 (tcq_viterbi) and :806-811 (lut_subs_quant); the argument
// lists, buffer shapes and return codes are the reference's (0 = ok, -1 = rejected configuration, otherwise
// the HIP error code of the launch). The caller allocates every buffer, as in the reference; bp / pbits are
// used as opaque scratch for this kernel's own decision-word format, gsel is not touched.
#include <hip/hip_runtime.h>
#include <stdlib.h>

#include "tcq_launch.h"

#include "ltq_hip.h"

namespace ltq {

// instantiated in tcq_inst_*.hip (compiled in parallel)
extern template int launch<8, 0, 4>(const TcqArgs&, hipStream_t);
extern template int launch<10, 0, 4>(const TcqArgs&, hipStream_t);
extern template int launch<10, 0, 8>(const TcqArgs&, hipStream_t);
extern template int launch<10, 0, 16>(const TcqArgs&, hipStream_t);
extern template int launch<10, 0, 32>(const TcqArgs&, hipStream_t);
extern template int launch<10, 1, 4>(const TcqArgs&, hipStream_t);
extern template int launch<10, 1, 8>(const TcqArgs&, hipStream_t);
extern template int launch<10, 1, 16>(const TcqArgs&, hipStream_t);
extern template int launch<10, 1, 32>(const TcqArgs&, hipStream_t);
extern template int launch<10, 2, 4>(const TcqArgs&, hipStream_t);
extern template int launch<10, 2, 8>(const TcqArgs&, hipStream_t);
extern template int launch<10, 2, 16>(const TcqArgs&, hipStream_t);
extern template int launch<10, 2, 32>(const TcqArgs&, hipStream_t);
extern template int launch<10, 3, 4>(const TcqArgs&, hipStream_t);
extern template int launch<10, 3, 8>(const TcqArgs&, hipStream_t);
extern template int launch<10, 3, 16>(const TcqArgs&, hipStream_t);
extern template int launch<10, 3, 32>(const TcqArgs&, hipStream_t);

int device_lds_max()
{
    static int v = -1;
    if (v < 0) {
        int dev = 0, x = 0;
        if (hipGetDevice(&dev) != hipSuccess) return -1;
        if (hipDeviceGetAttribute(&x, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return -1;
        v = x;
    }
    return v;
}

template <int NU, int MD>
static int launch_nl(const TcqArgs& a, hipStream_t st)
{
    switch (a.nl) {
        case 4: return launch<NU, MD, 4>(a, st);
        case 8: return launch<NU, MD, 8>(a, st);
        case 16: return launch<NU, MD, 16>(a, st);
        case 32: return launch<NU, MD, 32>(a, st);
        default: return -1;
    }
}

}  // namespace ltq

using ltq::TcqArgs;

extern "C" int tcq_viterbi(const float* x, const float* w, const float* tab, const float* gains, float* rec, uint32_t* bp,
                           uint8_t* gsel, const int* init_st, int* end_st, const float* tab_hi, const float* gains_hi,
                           uint8_t* gcand, int* best, int* code, int* mid_st, int mid_t, int tail, int N, int T, int S,
                           int U, int G, int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3, int m4, int nl,
                           int ld, int rot, uint32_t* pbits, int pp, void* stream)
{
    using namespace ltq;
    // the reference's validation (tcq_viterbi.cu:748-751, 762-763)
    if (G > kMaxG || Gfull > kMaxG || (!gcand && Gfull != G) || U > kMaxU || U_hi > kMaxU || sub <= 0 || T % sub != 0 ||
        (sub & 1) || T / sub > kMaxSubs || T > kMaxT || sub > 32 || sub * G * nl * (pp ? 2 : 1) > 4096 ||
        (pp && (S != 1024 || mix > 0 || (T & 1))) || (pp >= 2 && ((T & 3) || (sub & 3))) || pp > 3 || pp < 0 ||
        (nl != 4 && nl != 8 && nl != 16 && nl != 32) || ld < T || ((S != 1024 || getenv("TCQ_BLOCK")) && nl != 4) ||
        nl * U > 4 * kMaxU || nl * U_hi > 4 * kMaxU)
        return -1;
    if (S != 1024 && S != 256) return -1;
    if (G != 1 && G != 2 && G != 3 && G != 4 && G != 8) return -1;
    // limits of this implementation's decision-word storage inside the reference-sized scratch
    if (pp == 1 && (T & 3)) return -1;
    if (S == 256 && T < 8) return -1;
    if (T <= 0 || !bp || (pp && !pbits) || !best || !rec) return -1;
    if (N <= 0) return N == 0 ? (int)hipErrorInvalidConfiguration : -1;  // a 0-block launch, as the reference gets
    TcqArgs a{x, w, tab, gains, rec, bp, gsel, init_st, end_st, tab_hi, gains_hi, gcand, best, code, mid_st,
              mid_t, tail, N, T, S, U, G, Gfull, m, sub, U_hi, mix, m2, m3, m4, nl, ld, rot, pbits, pp};
    hipStream_t st = (hipStream_t)stream;
    int rc;
    if (S == 256) rc = launch<8, 0, 4>(a, st);
    else if (pp == 0) rc = launch_nl<10, 0>(a, st);
    else if (pp == 1) rc = launch_nl<10, 1>(a, st);
    else if (pp == 2) rc = launch_nl<10, 2>(a, st);
    else rc = launch_nl<10, 3>(a, st);
    if (rc != 0) return rc;
    return (int)hipGetLastError();
}
