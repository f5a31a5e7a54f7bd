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
#include "ltq_timing.h"

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

// one wave per four consecutive (row, 256-column block) units, loads of all four issued before the first
// transform; SM: 0 none, 1 x / s[col], 2 x * s[col]
constexpr int kRowUnits = 4;

template <int DT, int SM>
__global__ __launch_bounds__(64 * kWaves) void fwht_rows_kernel(const void* __restrict__ x, float* __restrict__ y,
                                                               long rows, long nblk, long ldx, long ldy,
                                                               const float* __restrict__ s)
{
    const int lane = threadIdx.x & 63;
    const long total = rows * nblk;
    const long stride = (long)gridDim.x * kWaves * kRowUnits;
    for (long u0 = ((long)blockIdx.x * kWaves + (threadIdx.x >> 6)) * kRowUnits; u0 < total; u0 += stride) {
        float v[kRowUnits][4];
        long r[kRowUnits], c[kRowUnits];
#pragma unroll
        for (int j = 0; j < kRowUnits; j++) {
            const long u = u0 + j < total ? u0 + j : total - 1;  // a short last group repeats its last unit
            r[j] = u / nblk;
            c[j] = (u - r[j] * nblk) * 256 + 4 * lane;
            load4<DT>(x, r[j] * ldx + c[j], v[j]);
        }
#pragma unroll
        for (int j = 0; j < kRowUnits; j++) {
            if constexpr (SM == 1) {
                const float4 d = *(const float4*)(s + c[j]);
                v[j][0] = v[j][0] / d.x; v[j][1] = v[j][1] / d.y; v[j][2] = v[j][2] / d.z; v[j][3] = v[j][3] / d.w;
            } else if constexpr (SM == 2) {
                const float4 d = *(const float4*)(s + c[j]);
                v[j][0] = v[j][0] * d.x; v[j][1] = v[j][1] * d.y; v[j][2] = v[j][2] * d.z; v[j][3] = v[j][3] * d.w;
            }
            fwht_wave(v[j], lane);
        }
#pragma unroll
        for (int j = 0; j < kRowUnits; j++)
            if (u0 + j < total) *(float4*)(y + r[j] * ldy + c[j]) = make_float4(v[j][0], v[j][1], v[j][2], v[j][3]);
    }
}

// column mode: a workgroup transforms a [256 rows, 64 columns] tile (64 KB of LDS, two workgroups per CU; 128
// columns with one workgroup per CU measured 1.6x slower). Rows come in and go out as 256-byte float4 segments
// through a row-major LDS tile; the transform runs with lane = column (every LDS access conflict-free)
// in two register passes: stages h = 1, 2, 4, 8 over 16 consecutive rows, then h = 16, 32, 64, 128 over 16 rows
// spaced 16 apart (the same stage order and pairs as the reference, so the same bits). SM scales by s[row]
// before the transform.
constexpr int kColTile = 64;

template <int SM, bool VEC>
__global__ __launch_bounds__(64 * kWaves) void fwht_cols_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                               long rows, long cols, long ldx, long ldy,
                                                               const float* __restrict__ s)
{
    __shared__ __align__(16) float t[256][kColTile];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const long ctiles = (cols + kColTile - 1) / kColTile;
    const long total = (rows / 256) * ctiles;
    const int c4 = 4 * (tid & 15), i0 = tid >> 4;  // rows i0 + 16 k, columns c4 .. c4 + 3
    for (long u = blockIdx.x; u < total; u += gridDim.x) {
        const long r0 = (u / ctiles) * 256, cg = (u % ctiles) * kColTile + c4;
        float4 f[16];  // all 16 row segments in flight before the first LDS store
        if (VEC) {
#pragma unroll
            for (int k = 0; k < 16; k++) f[k] = *(const float4*)(x + (r0 + i0 + 16 * k) * ldx + cg);
        } else {
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float* src = x + (r0 + i0 + 16 * k) * ldx + cg;
                f[k] = make_float4(cg < cols ? src[0] : 0.f, cg + 1 < cols ? src[1] : 0.f, cg + 2 < cols ? src[2] : 0.f,
                                   cg + 3 < cols ? src[3] : 0.f);
            }
        }
        if constexpr (SM != 0) {
            float sr[16];
#pragma unroll
            for (int k = 0; k < 16; k++) sr[k] = s[r0 + i0 + 16 * k];
#pragma unroll
            for (int k = 0; k < 16; k++) {
                if constexpr (SM == 1) {
                    f[k].x = f[k].x / sr[k]; f[k].y = f[k].y / sr[k]; f[k].z = f[k].z / sr[k]; f[k].w = f[k].w / sr[k];
                } else {
                    f[k].x = f[k].x * sr[k]; f[k].y = f[k].y * sr[k]; f[k].z = f[k].z * sr[k]; f[k].w = f[k].w * sr[k];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 16; k++) *(float4*)&t[i0 + 16 * k][c4] = f[k];
        __syncthreads();
        // pass 1: wave w, row groups 4 w .. 4 w + 3 of 16 consecutive rows; stages h = 1, 2, 4, 8
        for (int gq = 0; gq < 4; gq++) {
            const int rb = 16 * (4 * wv + gq);
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = t[rb + k][lane];
#pragma unroll
            for (int h = 1; h < 16; h <<= 1)
#pragma unroll
                for (int k = 0; k < 16; k++)
                    if (!(k & h)) {
                        const float a = v[k], b = v[k + h];
                        v[k] = a + b;
                        v[k + h] = a - b;
                    }
#pragma unroll
            for (int k = 0; k < 16; k++) t[rb + k][lane] = v[k];
        }
        __syncthreads();
        // pass 2: wave w, rows r_lo + 16 k for r_lo = 4 w .. 4 w + 3; stages h = 16 .. 128, then x 0.0625
        for (int gq = 0; gq < 4; gq++) {
            const int rl = 4 * wv + gq;
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = t[rl + 16 * k][lane];
#pragma unroll
            for (int h = 1; h < 16; h <<= 1)
#pragma unroll
                for (int k = 0; k < 16; k++)
                    if (!(k & h)) {
                        const float a = v[k], b = v[k + h];
                        v[k] = a + b;
                        v[k + h] = a - b;
                    }
#pragma unroll
            for (int k = 0; k < 16; k++) t[rl + 16 * k][lane] = v[k] * 0.0625f;
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float4 o = *(const float4*)&t[i0 + 16 * k][c4];
            float* dst = y + (r0 + i0 + 16 * k) * ldy + cg;
            if (VEC) {
                *(float4*)dst = o;
            } else {
                if (cg < cols) dst[0] = o.x;
                if (cg + 1 < cols) dst[1] = o.y;
                if (cg + 2 < cols) dst[2] = o.z;
                if (cg + 3 < cols) dst[3] = o.w;
            }
        }
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
    const dim3 grid(grid_for((rows * nblk + kRowUnits - 1) / kRowUnits)), block(64 * kWaves);
    auto& hook = ltq::kernel_timing;
    if (smode == 0) return ltq::timed_launch(hook, fwht_rows_kernel<DT, 0>, grid, block, 0, st, x, y, rows, nblk, ldx, ldy, s);
    if (smode == 1) return ltq::timed_launch(hook, fwht_rows_kernel<DT, 1>, grid, block, 0, st, x, y, rows, nblk, ldx, ldy, s);
    return ltq::timed_launch(hook, fwht_rows_kernel<DT, 2>, grid, block, 0, st, x, y, rows, nblk, ldx, ldy, s);
}

template <bool VEC>
int cols_dispatch(const float* x, float* y, long rows, long cols, long ldx, long ldy, const float* s, int smode,
                  int grid, hipStream_t st)
{
    const dim3 g(grid), block(64 * kWaves);
    auto& hook = ltq::kernel_timing;
    if (smode == 0) return ltq::timed_launch(hook, fwht_cols_kernel<0, VEC>, g, block, 0, st, x, y, rows, cols, ldx, ldy, s);
    if (smode == 1) return ltq::timed_launch(hook, fwht_cols_kernel<1, VEC>, g, block, 0, st, x, y, rows, cols, ldx, ldy, s);
    return ltq::timed_launch(hook, fwht_cols_kernel<2, VEC>, g, block, 0, st, x, y, rows, cols, ldx, ldy, s);
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
    const int grid = grid_for(tiles * kWaves);
    // whole float4 row segments: aligned rows and every 64-column tile full
    const bool vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)y % 16 == 0) && ldx % 4 == 0 && ldy % 4 == 0 &&
                     cols % kColTile == 0;
    if (vec) return cols_dispatch<true>(x, y, rows, cols, ldx, ldy, s, smode, grid, st);
    return cols_dispatch<false>(x, y, rows, cols, ldx, ldy, s, smode, grid, st);
}
