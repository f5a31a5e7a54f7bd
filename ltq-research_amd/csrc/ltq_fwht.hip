// Normalized block FWHT-256 for gfx950, along rows (optionally fused with a per-column divide / multiply and
// a bf16 / fp16 -> fp32 widening) and along columns (256-row blocks, for the second side of H).
//
// Arithmetic follows src/iqk_format.py:153-170 operation by operation: stages h = 1, 2, 4, ..., 128, each
// (a, b) -> (a + b, a - b) with a the element whose index bit h is clear, then one multiply by 0.0625 (exact).
// A fused scale is applied first, as the callers write it: x / s (src/liqk_v2.py:438) or x * s (:439-440).
// The transform is bit-identical to the reference's torch code on the same fp32 input.
//
// Roofline: HBM. Row mode moves (input bytes + 4) per element, column mode 8 per element.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "ltq_hip.h"

namespace {

constexpr int kWaves = 4;  // waves per workgroup

template <int DT>
__device__ __forceinline__ void load4(const void* base, long off, float v[4])
{
    if constexpr (DT == 0) {
        const float4 f = *(const float4*)((const float*)base + off);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
        const uint2 u = *(const uint2*)((const uint16_t*)base + off);
        const uint32_t h[4] = {u.x & 0xFFFFu, u.x >> 16, u.y & 0xFFFFu, u.y >> 16};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (DT == 1) v[i] = __uint_as_float(h[i] << 16);                  // bf16: exact widening
            else v[i] = __half2float(__ushort_as_half((unsigned short)h[i]));           // fp16: exact widening
        }
    }
}

// the 256-point transform of the 4 elements a lane holds (elements 4 * lane .. 4 * lane + 3 of the block)
__device__ __forceinline__ void fwht_wave(float v[4], int lane)
{
    // h = 1 and h = 2 inside the lane
    float a0 = v[0] + v[1], a1 = v[0] - v[1], a2 = v[2] + v[3], a3 = v[2] - v[3];
    v[0] = a0 + a2; v[2] = a0 - a2; v[1] = a1 + a3; v[3] = a1 - a3;
    // h = 4 .. 128: the partner element sits in lane ^ (h / 4)
#pragma unroll
    for (int j = 0; j < 6; j++) {
        const bool upper = (lane >> j) & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float p = __shfl_xor(v[i], 1 << j, 64);
            v[i] = upper ? p - v[i] : v[i] + p;  // upper lane: a - b with a = partner; lower: a + b
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] *= 0.0625f;
}

// one wave per (row, 256-column block); SM: 0 none, 1 x / s[col], 2 x * s[col]
template <int DT, int SM>
__global__ __launch_bounds__(64 * kWaves) void fwht_rows_kernel(const void* __restrict__ x, float* __restrict__ y,
                                                               long rows, long nblk, long ldx, long ldy,
                                                               const float* __restrict__ s)
{
    const int lane = threadIdx.x & 63;
    const long total = rows * nblk;
    for (long u = (long)blockIdx.x * kWaves + (threadIdx.x >> 6); u < total; u += (long)gridDim.x * kWaves) {
        const long r = u / nblk, c = (u - r * nblk) * 256 + 4 * lane;
        float v[4];
        load4<DT>(x, r * ldx + c, v);
        if constexpr (SM == 1) {
            const float4 d = *(const float4*)(s + c);
            v[0] = v[0] / d.x; v[1] = v[1] / d.y; v[2] = v[2] / d.z; v[3] = v[3] / d.w;
        } else if constexpr (SM == 2) {
            const float4 d = *(const float4*)(s + c);
            v[0] = v[0] * d.x; v[1] = v[1] * d.y; v[2] = v[2] * d.z; v[3] = v[3] * d.w;
        }
        fwht_wave(v, lane);
        *(float4*)(y + r * ldy + c) = make_float4(v[0], v[1], v[2], v[3]);
    }
}

// column mode: a workgroup transforms a [256 rows, 32 columns] tile through LDS (coalesced 128-byte row
// segments in and out); SM scales by s[row] before the transform
constexpr int kColTile = 32;
constexpr int kColPitch = 257;  // words per column in LDS: consecutive columns start on consecutive banks

template <int SM>
__global__ __launch_bounds__(64 * kWaves) void fwht_cols_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                               long rows, long cols, long ldx, long ldy,
                                                               const float* __restrict__ s)
{
    __shared__ float t[kColTile * kColPitch];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const long ctiles = (cols + kColTile - 1) / kColTile;
    const long total = (rows / 256) * ctiles;
    for (long u = blockIdx.x; u < total; u += gridDim.x) {
        const long r0 = (u / ctiles) * 256, c0 = (u % ctiles) * kColTile;
        const int cc = tid & (kColTile - 1);
        const bool in = c0 + cc < cols;
        for (int i = tid / kColTile; i < 256; i += 64 * kWaves / kColTile) {
            float v = in ? x[(r0 + i) * ldx + c0 + cc] : 0.f;
            if constexpr (SM == 1) v = v / s[r0 + i];
            else if constexpr (SM == 2) v = v * s[r0 + i];
            t[cc * kColPitch + i] = v;
        }
        __syncthreads();
        for (int c = wv; c < kColTile; c += kWaves) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = t[c * kColPitch + 4 * lane + i];
            fwht_wave(v, lane);
#pragma unroll
            for (int i = 0; i < 4; i++) t[c * kColPitch + 4 * lane + i] = v[i];
        }
        __syncthreads();
        if (in)
            for (int i = tid / kColTile; i < 256; i += 64 * kWaves / kColTile) y[(r0 + i) * ldy + c0 + cc] = t[cc * kColPitch + i];
        __syncthreads();
    }
}

int grid_for(long work_items)
{
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    const long g = (work_items + kWaves - 1) / kWaves;
    const long cap = (long)cus * 16;  // enough resident waves to cover HBM latency; the kernels stride the rest
    return (int)(g < cap ? (g > 0 ? g : 1) : cap);
}

template <int DT>
int rows_dispatch(const void* x, float* y, long rows, long cols, long ldx, long ldy, const float* s, int smode,
                  hipStream_t st)
{
    const long nblk = cols / 256;
    const int grid = grid_for(rows * nblk);
    switch (smode) {
        case 0: hipLaunchKernelGGL((fwht_rows_kernel<DT, 0>), dim3(grid), dim3(64 * kWaves), 0, st, x, y, rows, nblk, ldx, ldy, s); break;
        case 1: hipLaunchKernelGGL((fwht_rows_kernel<DT, 1>), dim3(grid), dim3(64 * kWaves), 0, st, x, y, rows, nblk, ldx, ldy, s); break;
        default: hipLaunchKernelGGL((fwht_rows_kernel<DT, 2>), dim3(grid), dim3(64 * kWaves), 0, st, x, y, rows, nblk, ldx, ldy, s); break;
    }
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int ltq_fwht256_rows(const void* x, int dtype, float* y, long rows, long cols, long ldx, long ldy,
                                const float* s, int smode, void* stream)
{
    if (rows < 0 || cols < 0 || cols % 256 || ldx < cols || ldy < cols || (ldx & 3) || (ldy & 3) || smode < 0 ||
        smode > 2 || (smode && !s) || dtype < 0 || dtype > 2)
        return -1;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !y || ((uintptr_t)x & (dtype ? 7 : 15)) || ((uintptr_t)y & 15) || ((uintptr_t)s & 15))
        return -1;  // vector loads: 16-byte fp32 / 8-byte 16-bit groups of 4 (ldx, ldy are multiples of 4)
    hipStream_t st = (hipStream_t)stream;
    if (dtype == 0) return rows_dispatch<0>(x, y, rows, cols, ldx, ldy, s, smode, st);
    if (dtype == 1) return rows_dispatch<1>(x, y, rows, cols, ldx, ldy, s, smode, st);
    return rows_dispatch<2>(x, y, rows, cols, ldx, ldy, s, smode, st);
}

extern "C" int ltq_fwht256_cols(const float* x, float* y, long rows, long cols, long ldx, long ldy, const float* s,
                                int smode, void* stream)
{
    if (rows < 0 || cols < 0 || rows % 256 || ldx < cols || ldy < cols || smode < 0 || smode > 2 || (smode && !s))
        return -1;
    if (rows == 0 || cols == 0) return 0;
    if (!x || !y || ((uintptr_t)s & 3)) return -1;  // in place is fine: a tile is read whole before it is written
    hipStream_t st = (hipStream_t)stream;
    const long tiles = (rows / 256) * ((cols + kColTile - 1) / kColTile);
    int grid = grid_for(tiles * kWaves);
    switch (smode) {
        case 0: hipLaunchKernelGGL((fwht_cols_kernel<0>), dim3(grid), dim3(64 * kWaves), 0, st, x, y, rows, cols, ldx, ldy, s); break;
        case 1: hipLaunchKernelGGL((fwht_cols_kernel<1>), dim3(grid), dim3(64 * kWaves), 0, st, x, y, rows, cols, ldx, ldy, s); break;
        default: hipLaunchKernelGGL((fwht_cols_kernel<2>), dim3(grid), dim3(64 * kWaves), 0, st, x, y, rows, cols, ldx, ldy, s); break;
    }
    return (int)hipGetLastError();
}
