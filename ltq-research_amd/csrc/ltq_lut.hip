// LUT sub-block quantization of the diagonal profile (the second export of the reference C ABI,
// src/cuda/tcq_viterbi.cu:768-811, called from src/liqk_v2.py:497-500 through src/tcq_proto.py:537-548).
//
// Per sub-block i of 16 weights x_j with weights d_j: bucket b_j = clamp(rint(x_j * inv_step + half_b), 0, nb-1)
// selects a row of 64 candidate values lut[b_j][0..63]; candidate c has the error
//     err_c = sum_j d_j (x_j - lut[b_j][c])^2        (j = 0 .. 15 in order)
// and the sub-block takes the first candidate with the lowest error: out[i][j] = lut[b_j][c*].
// Rounding is the one nvcc's default contraction gives the reference's expressions: the bucket argument is
// fma(x, inv_step, half_b) and the accumulation err = fma(d e, e, err).
//
// MI355X mapping: one wavefront per sub-block, lane c = candidate c, so every LUT row is one coalesced 256-byte
// load (the 2 MB table stays in L2) and the 64 errors are an argmin across lanes (lowest error, then lowest lane).
// Roofline: VALU (~150 wave instructions per sub-block); 192 bytes of HBM traffic per sub-block.
#include <hip/hip_runtime.h>
#include <math.h>

#include "ltq_hip.h"

namespace {

constexpr int kWaves = 4;

__device__ inline int bucket(float x, float inv_step, float half_b, int nb)
{
    int b = (int)rintf(__builtin_fmaf(x, inv_step, half_b));
    return b < 0 ? 0 : (b > nb - 1 ? nb - 1 : b);
}

__global__ __launch_bounds__(64 * kWaves) void lut_subs_kernel(const float* __restrict__ xs,
                                                               const float* __restrict__ dh,
                                                               const float* __restrict__ lut, float* __restrict__ out,
                                                               long S, float inv_step, float half_b, int nb)
{
    const int lane = threadIdx.x & 63;
    for (long i = (long)blockIdx.x * kWaves + (threadIdx.x >> 6); i < S; i += (long)gridDim.x * kWaves) {
        const float xl = lane < 16 ? xs[i * 16 + lane] : 0.f;
        const float dl = lane < 16 ? dh[i * 16 + lane] : 0.f;
        float xv[16], dv[16], v[16];
#pragma unroll
        for (int j = 0; j < 16; j++) {
            xv[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xl), j));
            dv[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dl), j));
            v[j] = lut[(long)bucket(xv[j], inv_step, half_b, nb) * 64 + lane];
        }
        float err = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const float e = xv[j] - v[j];
            err = __builtin_fmaf(dv[j] * e, e, err);
        }
        // first minimum over c = 0..63 with the reference's strict '<' scan: a NaN error is never chosen, and a
        // NaN error of candidate 0 keeps candidate 0
        const bool nan0 = __builtin_isnan(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(err), 0)));
        float be = __builtin_isnan(err) ? __builtin_inff() : err;
        int bi = lane;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float oe = __shfl_xor(be, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (oe < be || (oe == be && oi < bi)) {
                be = oe;
                bi = oi;
            }
        }
        const int best = nan0 ? 0 : bi;
        if (lane < 16) out[i * 16 + lane] = lut[(long)bucket(xl, inv_step, half_b, nb) * 64 + best];
    }
}

}  // namespace

extern "C" int lut_subs_quant(const float* xs, const float* dh, const float* lut, float* out, int S, float inv_step,
                              float half_b, int nb, void* stream)
{
    if (S < 0 || nb < 1) return -1;
    // no sub-blocks: the error of the zero-block launch the reference makes (its caller raises on it)
    if (S == 0) return (int)hipErrorInvalidConfiguration;
    if (!xs || !dh || !lut || !out) return -1;
    long grid = ((long)S + kWaves - 1) / kWaves;
    if (grid > 1L << 20) grid = 1L << 20;
    hipLaunchKernelGGL(lut_subs_kernel, dim3((unsigned)grid), dim3(64 * kWaves), 0, (hipStream_t)stream, xs, dh, lut, out,
                       (long)S, inv_step, half_b, nb);
    return (int)hipGetLastError();
}
