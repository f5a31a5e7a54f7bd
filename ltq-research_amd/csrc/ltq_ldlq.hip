// Row scale fitting and the LDLQ sub-block error feedback of the TCQ matrix quantizer, gfx950.
//
// ltq_row_scale (src/liqk_v2.py:938-946): per row, the rms of every 256-column block (clamped at 1e-10, times
// the format scale), d_row = fp16(exp(mean over blocks of log rms)) clamped at 1e-8, the block exponent
// e = clamp(round(log2(rms / d_row) / e_step), -2^(bits-1), 2^(bits-1) - 1) and d = d_row * 2^(e_step e).
// The result is defined to the bit, so that a CPU restatement reproduces it exactly:
//   - block sum of squares: lane l holds ((x[4l]^2 + x[4l+1]^2) + x[4l+2]^2) + x[4l+3]^2, then a butterfly over
//     lane offsets 32, 16, 8, 4, 2, 1 (s_l + s_(l^o): every lane ends with the same bits); rms = sqrt(s / 256),
//     all fp32, correctly rounded;
//   - log, mean and exp in float64 (the logs one block per lane, their sum sequential over the blocks), rounded
//     to fp32 and then to fp16; the
//     exponent from the fp32 ratio rms / d_row as round-half-even of log2(ratio) / e_step in float64: float64
//     keeps every value far from the fp16 / half-step rounding boundaries the fp32 functions can straddle;
//   - 2^(e_step e) is read from a host-computed table (float64, rounded once to fp32), the same table the PACK
//     tail, the .ltq decoder and the CPU oracle use.
// One wavefront per row. Roofline: HBM, 4 bytes read per weight.
//
// ltq_ldlq_sub (src/liqk_v2.py:957-967): after the Viterbi of sub-block ib of a 256-column block, for the 16
// rows of every tile
//     G[:, s0:s1]      = g                                   (the tile's reconstruction, unscaled)
//     err              = (w[:, s0:s1] - d * g) @ U_inv[s0:s1, s0:s1]
//     w[:, s1:]       -= err @ U[s0:s1, s1:]
//     x_next           = w[:, s1:s1+16] * (1 / d)             (next sub-block's Viterbi tiles, t = 16 r + c)
//     idx[:, s0:s1]    = code & 0xFFFF, gi[:, s0:s1] = code >> 16   (optional: the PACK fields, src/liqk_v2.py:919-921)
// with the element-wise products and the division rounded as the reference's torch code rounds them; the two
// small contractions are fma chains over k = 0..15 in ascending order from 0 (then w - acc), and the value each
// element had when its Viterbi ran is optionally recorded (fed).
// One workgroup per tile; roofline: L2 (the block's working copy and U rows are re-read per sub-block).
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdint.h>

#include "ltq_hip.h"
#include "ltq_timing.h"

namespace {

__global__ __launch_bounds__(256) void row_scale_kernel(const float* __restrict__ w, long M, int nblk, long ldw,
                                                        float scale, double e_step, int e_max,
                                                        const float* __restrict__ exp2_tab, float* __restrict__ d_row,
                                                        int8_t* __restrict__ e_out, long lde, float* __restrict__ d_out,
                                                        long ldd)
{
    extern __shared__ double s_dyn[];  // [4 waves][nblk] log(rms) (float64), then [4 waves][nblk] rms (fp32)
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const long row = (long)blockIdx.x * 4 + wv;
    if (row >= M) return;
    double* lg = s_dyn + wv * nblk;
    float* rms = (float*)(s_dyn + 4 * nblk) + wv * nblk;
    const float* wr = w + row * ldw;
    constexpr int kAhead = 8;  // blocks whose loads are in flight together
    // rows start at different blocks (row * 13 mod nblk) so that the waves streaming their rows side by side do
    // not all address the same offsets of equally spaced rows; each block's rms is independent of the order
    const int rot = (int)((row * 13) % nblk);
    for (int b0 = 0; b0 < nblk; b0 += kAhead) {
        float4 v[kAhead];
#pragma unroll
        for (int j = 0; j < kAhead; j++)
            if (b0 + j < nblk) {
                const int bj = b0 + j + rot < nblk ? b0 + j + rot : b0 + j + rot - nblk;
                v[j] = *(const float4*)(wr + bj * 256 + 4 * lane);
            }
        float s[kAhead];
#pragma unroll
        for (int j = 0; j < kAhead; j++) s[j] = v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1)
#pragma unroll
            for (int j = 0; j < kAhead; j++) s[j] += __shfl_xor(s[j], o, 64);
#pragma unroll
        for (int j = 0; j < kAhead; j++) {
            if (b0 + j >= nblk) break;
            const float r = fmaxf(sqrtf(s[j] / 256.f), 1e-10f) * scale;
            if (lane == 0) rms[b0 + j + rot < nblk ? b0 + j + rot : b0 + j + rot - nblk] = r;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // the float64 logs one block per lane, then their sum in block order (the same values and order as one lane
    // summing log(rms) block by block)
    for (int b = lane; b < nblk; b += 64) lg[b] = log((double)rms[b]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    double lsum = 0.0;
    for (int b = 0; b < nblk; b++) lsum += lg[b];
    const float d = fmaxf(__half2float(__float2half((float)exp(lsum / (double)nblk))), 1e-8f);
    if (lane == 0) d_row[row] = d;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int b = lane; b < nblk; b += 64) {
        const float ratio = rms[b] / d;
        double e = rint(log2((double)ratio) / e_step);
        e = fmin(fmax(e, (double)-e_max), (double)(e_max - 1));
        const int ei = (int)e;
        e_out[row * lde + b] = (int8_t)ei;
        d_out[row * ldd + b] = fmaxf(d * exp2_tab[ei + e_max], 1e-8f);
    }
}

// One workgroup per 16-row tile. Every global load of the tile is issued first (its Viterbi output and codes, the
// weights it saw and the ones it updates, the diagonal block of U_inv, the block's 16 U rows into LDS), so the
// workgroup waits for memory about once; written as a loop over the updated columns the compiler had waited for
// each column group's loads in turn.
__global__ __launch_bounds__(256) void ldlq_sub_kernel(float* __restrict__ wk, long ldw, const float* __restrict__ rec,
                                                       const float* __restrict__ d, long ldd,
                                                       const float* __restrict__ uinv, long ldi,
                                                       const float* __restrict__ ublk, long ldu, int s0,
                                                       float* __restrict__ G, long ldg,
                                                       float* __restrict__ xnext, long M,
                                                       const int* __restrict__ code, int16_t* __restrict__ idx,
                                                       long ld_idx, uint8_t* __restrict__ gi, long ld_gi,
                                                       float* __restrict__ fed, long ld_fed, long tiles_per_mat,
                                                       long uinv_ms, long ublk_ms)
{
    __shared__ float s_err[16][17];
    __shared__ float s_d[16];
    __shared__ __align__(16) float s_u[16][256];  // U rows s0 .. s0 + 15 of the block, columns s1 .. 255
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    const long row0 = (long)blockIdx.x * 16, row = row0 + r;
    if (row0 >= M) return;
    const int s1 = s0 + 16, nj = (256 - s1) / 16;  // this thread updates columns s1 + c + 16 m, m < nj
    if (tiles_per_mat > 0) {  // stacked matrices: this tile's rows belong to matrix blockIdx.x / tiles_per_mat
        const long mat = (long)blockIdx.x / tiles_per_mat;
        uinv += mat * uinv_ms;
        ublk += mat * ublk_ms;
    }
    // tile element t = 16 r + c is row r, sub-block column c
    const float g = rec[(long)blockIdx.x * 256 + tid];
    const int cv = code ? code[(long)blockIdx.x * 256 + tid] : 0;
    const float wv = wk[row * ldw + s0 + c];  // the value this sub-block's Viterbi saw (times 1 / d)
    float wj[15];
#pragma unroll
    for (int m = 0; m < 15; m++) wj[m] = m < nj ? wk[row * ldw + s1 + c + 16 * m] : 0.f;
    float ui[16];
#pragma unroll
    for (int k = 0; k < 16; k++) ui[k] = uinv[(long)(s0 + k) * ldi + s0 + c];
    {  // thread (k, group q) copies U[s0 + k][16 q .. 16 q + 15] when those columns are updated
        const int k = tid >> 4, c0 = (tid & 15) * 16;
        if (c0 >= s1) {
            const float* src = ublk + (long)(s0 + k) * ldu + c0;
#pragma unroll
            for (int v = 0; v < 16; v++) s_u[k][c0 + v] = src[v];
        }
    }
    if (tid < 16) s_d[tid] = d[(row0 + tid) * ldd];
    G[row * ldg + s0 + c] = g;
    if (code) {
        idx[row * ld_idx + s0 + c] = (int16_t)(cv & 0xFFFF);
        gi[row * ld_gi + s0 + c] = (uint8_t)(cv >> 16);
    }
    if (fed) fed[row * ld_fed + s0 + c] = wv;
    __syncthreads();
    const float dr = s_d[r];
    // residual of this element, then err[r][c] = sum_k resid[r][k] * uinv[s0+k][s0+c] (fma chain, k ascending)
    const float resid = wv - dr * g;
    s_err[r][c] = resid;
    __syncthreads();
    float e = 0.f;
#pragma unroll
    for (int k = 0; k < 16; k++) e = __fmaf_rn(s_err[r][k], ui[k], e);
    __syncthreads();
    s_err[r][c] = e;
    __syncthreads();
    // w[r][j] -= sum_k err[r][k] * U[s0+k][j] for j >= s1 (fma chain, k ascending); column s1 + c (m = 0) also
    // gives the next sub-block's tile value
    const float inv = 1.0f / dr;
#pragma unroll
    for (int m = 0; m < 15; m++) {
        if (m < nj) {
            const int j = s1 + c + 16 * m;
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < 16; k++) acc = __fmaf_rn(s_err[r][k], s_u[k][j], acc);
            const float nv = wj[m] - acc;
            wk[row * ldw + j] = nv;
            if (m == 0 && xnext) xnext[(long)blockIdx.x * 256 + tid] = nv * inv;
        }
    }
}

// first sub-block's tiles of a block: x[t = 16 r + c] = w[r][c] * (1 / d[r])
__global__ __launch_bounds__(256) void ldlq_prep_kernel(const float* __restrict__ wk, long ldw, const float* __restrict__ d,
                                                        long ldd, float* __restrict__ x, long M)
{
    const int tid = threadIdx.x, r = tid >> 4, c = tid & 15;
    const long row = (long)blockIdx.x * 16 + r;
    if (row >= M) return;
    const float inv = 1.0f / d[row * ldd];
    x[(long)blockIdx.x * 256 + tid] = wk[row * ldw + c] * inv;
}

}  // namespace

extern "C" int ltq_row_scale(const float* w, long M, long K, long ldw, float scale, float e_step, int e_bits,
                             const float* exp2_tab, float* d_row, int8_t* e, long lde, float* d, long ldd, void* stream)
{
    if (M < 0 || K < 0 || K % 256 || ldw < K || (ldw & 3) || e_bits < 1 || e_bits > 8 || !(e_step > 0.f) || !(scale > 0.f))
        return -1;
    const int nblk = (int)(K / 256);
    if (M == 0 || nblk == 0) return 0;
    if (!w || !exp2_tab || !d_row || !e || !d || lde < nblk || ldd < nblk || ((uintptr_t)w & 15) || nblk > 1024)
        return -1;
    const long grid = (M + 3) / 4;
    return ltq::timed_launch(ltq::kernel_timing, row_scale_kernel, dim3((unsigned)grid), dim3(256),
                             (uint32_t)(4 * 12 * nblk), (hipStream_t)stream, w, M, nblk, ldw, scale, (double)e_step,
                             1 << (e_bits - 1), exp2_tab, d_row, e, lde, d, ldd);
}

extern "C" int ltq_ldlq_prep(const float* wk, long ldw, const float* d, long ldd, float* x, long M, void* stream)
{
    if (M < 0 || M % 16 || ldw < 16 || ldd < 1) return -1;
    if (M == 0) return 0;
    if (!wk || !d || !x) return -1;
    hipLaunchKernelGGL(ldlq_prep_kernel, dim3((unsigned)(M / 16)), dim3(256), 0, (hipStream_t)stream, wk, ldw, d, ldd, x, M);
    return (int)hipGetLastError();
}

extern "C" int ltq_ldlq_sub(float* wk, long ldw, const float* rec, const float* d, long ldd, const float* uinv,
                            long ldi, const float* ublk, long ldu, int ib, float* G, long ldg, float* xnext, long M,
                            const int* code, int16_t* idx, long ld_idx, uint8_t* gi, long ld_gi, float* fed,
                            long ld_fed, long rows_per_mat, long uinv_ms, long ublk_ms, void* stream)
{
    if (M < 0 || M % 16 || ib < 0 || ib > 15 || ldw < 256 || ldi < 256 || ldu < 256 || ldg < 256 || ldd < 1) return -1;
    if (code && (!idx || !gi || ld_idx < 256 || ld_gi < 256)) return -1;
    if (fed && ld_fed < 256) return -1;
    if (rows_per_mat < 0 || (rows_per_mat > 0 && (rows_per_mat % 16 || M % rows_per_mat))) return -1;
    if (M == 0) return 0;
    if (!wk || !rec || !d || !uinv || !ublk || !G) return -1;
    hipLaunchKernelGGL(ldlq_sub_kernel, dim3((unsigned)(M / 16)), dim3(256), 0, (hipStream_t)stream, wk, ldw, rec, d, ldd,
                       uinv, ldi, ublk, ldu, 16 * ib, G, ldg, xnext, M, code, idx, ld_idx, gi, ld_gi, fed, ld_fed,
                       rows_per_mat / 16, uinv_ms, ublk_ms);
    return (int)hipGetLastError();
}
