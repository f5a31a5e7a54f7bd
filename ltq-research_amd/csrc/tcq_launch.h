// gfx950 launch plumbing for the TCQ Viterbi kernel: the wavefront primitives the portable body uses, the
// __global__ entry and a launcher. Each tcq_inst_*.hip instantiates the launcher for one parity mode, so the
// 17 (S, mode, label-count) variants compile in parallel.
#pragma once
#include <hip/hip_runtime.h>

#include "tcq_kernel.h"

namespace ltq {

extern "C" __shared__ __align__(16) char ltq_dyn_smem[];

struct GpuX {
    __device__ __forceinline__ int tid() const { return (int)threadIdx.x; }
    __device__ __forceinline__ int wave() const { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }
    __device__ __forceinline__ int tile() const { return (int)blockIdx.x; }
    __device__ __forceinline__ int nthreads() const { return (int)blockDim.x; }
    __device__ __forceinline__ void* smem() const { return ltq_dyn_smem; }
    // full workgroup barrier: LDS and global memory (waits for this wave's outstanding stores)
    __device__ __forceinline__ void sync() const { __syncthreads(); }
    // workgroup barrier for LDS data only: outstanding global loads / stores keep flying
    __device__ __forceinline__ void lds_sync() const
    {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    __device__ __forceinline__ void wave_sync() const
    {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // acc = 2 * acc + sign bit of d (v_alignbit_b32 acc, acc, d, 31)
    __device__ __forceinline__ uint32_t push_sign(uint32_t acc, float d) const
    {
        return __builtin_amdgcn_alignbit(acc, __builtin_bit_cast(uint32_t, d), 31);
    }
    __device__ __forceinline__ float fmin(float x, float y) const { return __builtin_fminf(x, y); }
    __device__ __forceinline__ uint32_t readlane(uint32_t v, int l) const
    {
        return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
    }
    // asynchronous 16-byte copy global -> LDS; lane l's bytes land at lds_wave_base + 16 l
    __device__ __forceinline__ void load16(const uint32_t* src, uint32_t* lds_wave_base) const
    {
        __builtin_amdgcn_global_load_lds((const void*)src, (__attribute__((address_space(3))) void*)lds_wave_base,
                                         16, 0, 0);
    }
    template <int N>
    __device__ __forceinline__ void wait_loads() const
    {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0xF70);  // vmcnt(N) only
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
};

// WG = most wavefronts (gain slots) per workgroup the instance serves: 4 lets the compiler use the whole
// 512-entry register file of a SIMD (one wave per SIMD), 8 halves it.
template <int NU, int MD, int NL, int WG>
__global__ __launch_bounds__(64 * WG) void tcq_viterbi_kernel(TcqArgs a, int lds_max)
{
    GpuX x;
    tcq_tile<NU, MD, NL>(a, x, lds_max);
}

int device_lds_max();

template <int NU, int MD, int NL>
int launch(const TcqArgs& a, hipStream_t stream)
{
    const int lds_max = device_lds_max();
    if (lds_max <= 0) return -1;
    const Smem L = smem_layout<NU, MD, NL>(a.T, a.G, a.Gfull, a.sub, lds_max);
    if (L.total > lds_max) return -1;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)tcq_viterbi_kernel<NU, MD, NL, 4>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds_max);
        (void)hipFuncSetAttribute((const void*)tcq_viterbi_kernel<NU, MD, NL, 8>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, lds_max);
        attr = true;
    }
    if (a.G <= 4)
        hipLaunchKernelGGL((tcq_viterbi_kernel<NU, MD, NL, 4>), dim3(a.N), dim3(64 * a.G), L.total, stream, a, lds_max);
    else
        hipLaunchKernelGGL((tcq_viterbi_kernel<NU, MD, NL, 8>), dim3(a.N), dim3(64 * a.G), L.total, stream, a, lds_max);
    return 0;
}

}  // namespace ltq
