// Benchmark timing hooks. A host thread arms the next `launches` launches of one kernel family with a start /
// stop event pair: the first launch carries start, the last stop, and each goes out through
// hipExtLaunchKernelGGL, which stamps the events with the dispatch's own start and end times (no event packet
// sits between two kernels). Unarmed launches carry null events. Results are not affected.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace ltq {

struct TimingHook {
    hipEvent_t start = nullptr, stop = nullptr;
    int left = 0;  // launches still to go; the last one carries stop

    void arm(hipEvent_t s, hipEvent_t e, int launches)
    {
        start = s;
        stop = e;
        left = launches;
    }

    // events for the next launch (null when unarmed)
    void take(hipEvent_t* s, hipEvent_t* e)
    {
        *s = *e = nullptr;
        if (left <= 0) return;
        *s = start;
        start = nullptr;
        if (--left == 0) {
            *e = stop;
            stop = nullptr;
        }
    }
};

inline thread_local TimingHook viterbi_timing;  // Viterbi launches (tcq_viterbi, tcq_viterbi_tb, tcq_viterbi_static)
inline thread_local TimingHook kernel_timing;   // FWHT, row scale, pack, LDLQ err / update launches

// hipExtLaunchKernelGGL with the armed events of `hook`, then the launch status
template <typename... KArgs, typename... Args>
int timed_launch(TimingHook& hook, void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t shmem, hipStream_t st,
                 Args... args)
{
    hipEvent_t e0, e1;
    hook.take(&e0, &e1);
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, st, e0, e1, 0, static_cast<KArgs>(args)...);
    return (int)hipGetLastError();
}

}  // namespace ltq
