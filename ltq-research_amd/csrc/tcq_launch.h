// gfx950 launch plumbing for the TCQ Viterbi kernel: the wavefront primitives the portable body uses, the
// __global__ entry and a launcher. Each tcq_inst_*.hip instantiates the launcher for one parity mode, so the
// variants compile in parallel.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "ltq_timing.h"
#include "tcq_trellis.h"

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
    // acc = 2 * acc + sign bit of d (v_alignbit_b32 acc, acc, d, 31)
    __device__ __forceinline__ uint32_t push_sign(uint32_t acc, float d) const
    {
        return __builtin_amdgcn_alignbit(acc, __builtin_bit_cast(uint32_t, d), 31);
    }
    __device__ __forceinline__ float fmin(float x, float y) const { return __builtin_fminf(x, y); }
    // instruction-scheduling barrier: nothing is moved across it (keeps loads issued ahead of the code they overlap)
    __device__ __forceinline__ void sched_fence() const { __builtin_amdgcn_sched_barrier(0); }
    // 0, computed where it is used: offsets derived from it stay there instead of being hoisted out of loops
    // (and held in registers across them)
    __device__ __forceinline__ int opaque_zero() const
    {
        int z;
        asm volatile("v_mov_b32 %0, 0" : "=v"(z));
        return z;
    }
    // v is computed at this point (not sunk past it), held in a vector register
    __device__ __forceinline__ void pin(uint32_t& v) const { asm volatile("" : "+v"(v)); }
    // v (uniform) is computed at this point, held in a scalar register
    __device__ __forceinline__ void pin_s(uint32_t& v) const { asm volatile("" : "+s"(v)); }
    // (value, index) minimum over the wavefront, lowest index on ties, left in lane 63: DPP row operations
    // (quad swaps, half-row and row mirrors, then row broadcasts 15 and 31) instead of LDS permutes. The
    // lexicographic minimum does not depend on the order of the combines.
    template <int CTRL, int ROWS>
    __device__ __forceinline__ static void dpp_min(float& bv, int& bi)
    {
        const int vb = __builtin_bit_cast(int, bv);
        const float ov = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(vb, vb, CTRL, ROWS, 0xF, false));
        const int oi = __builtin_amdgcn_update_dpp(bi, bi, CTRL, ROWS, 0xF, false);
        if (ov < bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    __device__ __forceinline__ void wave_min(float& bv, int& bi) const
    {
        dpp_min<0xB1, 0xF>(bv, bi);   // quad_perm [1, 0, 3, 2]
        dpp_min<0x4E, 0xF>(bv, bi);   // quad_perm [2, 3, 0, 1]
        dpp_min<0x141, 0xF>(bv, bi);  // row_half_mirror
        dpp_min<0x140, 0xF>(bv, bi);  // row_mirror: every lane of a row holds the row's minimum
        dpp_min<0x142, 0xA>(bv, bi);  // row_bcast:15 into rows 1 and 3
        dpp_min<0x143, 0xC>(bv, bi);  // row_bcast:31 into rows 2 and 3: lane 63 holds the wavefront's minimum
    }
    // a value every lane holds equally, pinned to a scalar register
    __device__ __forceinline__ int uni(int v) const { return __builtin_amdgcn_readfirstlane(v); }
    // acquire at device scope: drops this CU's L1 lines, so global data rewritten since it was last read (by
    // stores, which bypass L1) is fetched again
    __device__ __forceinline__ void acquire() const { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
    // a global int another thread of the workgroup stored before the last sync(), read past the L1 cache
    __device__ __forceinline__ int load_coherent(const int* p) const
    {
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // lane l's value (l uniform), into a scalar register
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
    // at most n (<= 63) of this wave's vector memory operations still outstanding (vmcnt: bits 3:0, 15:14)
    __device__ __forceinline__ void wait_loads(int n) const
    {
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        switch (n) {
#define LTQ_W(k) \
    case k: __builtin_amdgcn_s_waitcnt(((k) & 15) | (((k) >> 4) << 14) | 0xF70); break;
#define LTQ_W8(k) LTQ_W(k) LTQ_W(k + 1) LTQ_W(k + 2) LTQ_W(k + 3) LTQ_W(k + 4) LTQ_W(k + 5) LTQ_W(k + 6) LTQ_W(k + 7)
            LTQ_W(1) LTQ_W(2) LTQ_W(3) LTQ_W(4) LTQ_W(5) LTQ_W(6) LTQ_W(7)
            LTQ_W8(8) LTQ_W8(16) LTQ_W8(24) LTQ_W8(32) LTQ_W8(40) LTQ_W8(48) LTQ_W8(56)
#undef LTQ_W8
#undef LTQ_W
            default: __builtin_amdgcn_s_waitcnt(0xF70); break;  // vmcnt(0)
        }
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
};

// Up to 16 wavefronts (1024 threads): G gain slots x Q waves. WMIN = 8 (waves per SIMD) builds the integer-mode
// instance for two workgroups per CU (64 VGPRs), used with half the LDS when a launch has at least two tiles per
// CU: its phases are bound by barrier and LDS latency rather than VALU, which a second workgroup overlaps
// (ring tables); with one tile per CU the 83-VGPR build (WMIN = 1) is faster.
template <int NU, int RB, int MD, int NL, int WMIN = 1>
__global__ __launch_bounds__(1024, WMIN) void tcq_viterbi_kernel(TcqArgs a, int lds_max)
{
    GpuX x;
    tcq_tile<NU, RB, MD, NL>(a, x, lds_max);
}

int device_lds_max();
int device_cu_count();

// hipFuncSetAttribute(f, max dynamic LDS, bytes) once per (kernel, device): done[] is the caller's per-kernel
// flag array; a failed call is returned and retried at the next launch
template <class K>
int set_max_lds_once(K* kernel, int bytes, bool (&done)[64])
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return -1;
    if (dev >= 0 && dev < 64 && done[dev]) return 0;
    const hipError_t e = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return (int)e;
    if (dev >= 0 && dev < 64) done[dev] = true;
    return 0;
}

// Both tail-biting passes of every tile in one launch.
template <int NU, int RB, int MD, int NL>
__global__ __launch_bounds__(1024) void tcq_viterbi_tb_kernel(TcqArgs a1, TcqArgs a2, int lds_max)
{
    GpuX x;
    tcq_tile_tb<NU, RB, MD, NL>(a1, a2, x, lds_max);
}

template <int NU, int RB, int MD, int NL>
int launch(const TcqArgs& a, hipStream_t stream)
{
    const int lds_max = device_lds_max();
    if (lds_max <= 0) return -1;
    if constexpr (MD == 0 && RB == 2) {
        const int cus = device_cu_count();
        const int half = lds_max / 2;
        const Smem H = smem_layout<NU, RB, MD, NL>(a.T, a.G, a.Gfull, a.sub, half);
        if (cus > 0 && a.N >= 2 * cus && H.total <= half) {
            static bool attr2[64] = {};
            if (const int e = set_max_lds_once(tcq_viterbi_kernel<NU, RB, MD, NL, 8>, half, attr2)) return e;
            const int threads = 64 * a.G * Geo<NU, RB>::Q;
            hipEvent_t e0 = nullptr, e1 = nullptr;
            viterbi_timing.take(&e0, &e1);
            hipExtLaunchKernelGGL((tcq_viterbi_kernel<NU, RB, MD, NL, 8>), dim3(a.N), dim3(threads), H.total, stream,
                                  e0, e1, 0, a, half);
            return 0;
        }
    }
    const Smem L = smem_layout<NU, RB, MD, NL>(a.T, a.G, a.Gfull, a.sub, lds_max);
    if (L.total > lds_max) return -1;
    static bool attr[64] = {};
    if (const int e = set_max_lds_once(tcq_viterbi_kernel<NU, RB, MD, NL>, lds_max, attr)) return e;
    const int threads = 64 * a.G * Geo<NU, RB>::Q;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    viterbi_timing.take(&e0, &e1);
    hipExtLaunchKernelGGL((tcq_viterbi_kernel<NU, RB, MD, NL>), dim3(a.N), dim3(threads), L.total, stream, e0, e1, 0,
                          a, lds_max);
    return 0;
}

template <int NU, int RB, int MD, int NL>
int launch_tb(const TcqArgs& a1, const TcqArgs& a2, hipStream_t stream)
{
    const int lds_max = device_lds_max();
    if (lds_max <= 0) return -1;
    const Smem L1 = smem_layout<NU, RB, MD, NL>(a1.T, a1.G, a1.Gfull, a1.sub, lds_max);
    const Smem L2 = smem_layout<NU, RB, MD, NL>(a2.T, a2.G, a2.Gfull, a2.sub, lds_max);
    const int total = L1.total > L2.total ? L1.total : L2.total;
    if (total > lds_max) return -1;
    static bool attr[64] = {};
    if (const int e = set_max_lds_once(tcq_viterbi_tb_kernel<NU, RB, MD, NL>, lds_max, attr)) return e;
    const int threads = 64 * a2.G * Geo<NU, RB>::Q;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    viterbi_timing.take(&e0, &e1);
    hipExtLaunchKernelGGL((tcq_viterbi_tb_kernel<NU, RB, MD, NL>), dim3(a2.N), dim3(threads), total, stream, e0, e1,
                          0, a1, a2, lds_max);
    return 0;
}

}  // namespace ltq
