// Input-covariance (Hessian) accumulation for the matrix quantizer, gfx950: the _CovAccumulator of
// src/liqk_v2.py:207-231.
//
// ltq_cov_accumulate: H += X^T X for one batch X [n, K] of bf16 or fp16 activations (row stride ldx). The
// products are exact in fp32, the batch sum accumulates in fp32 on the matrix cores (the reference's half-
// precision GEMM with fp32 output, src/liqk_v2.py:221) and the batch result is added into the fp64 running sum
// (src/liqk_v2.py:226). Only the tiles on and below the diagonal of H are computed and updated (H is
// symmetric; ltq_cov_finalize reads the lower triangle), which halves both the MFMA work and the fp64
// read-modify-write traffic.
//
//   tiles   128 x 128 of H per workgroup (tile row I >= tile column J), 4 wavefronts of 64 x 64 each, every
//           wavefront 2 x 2 v_mfma_f32_32x32x16 (bf16 or f16) with 64 fp32 accumulators per lane
//   chunks  32 rows of X at a time: each thread loads 4 rows x 8 columns (four 16-byte loads) of one of the two
//           column slices (I or J) and stores them as they are into a row-major LDS tile (16-byte stores, the
//           16-byte column groups of each row XOR-swizzled by the row); the MFMA operands (8 consecutive rows of
//           one column per lane) come out of it with the transposing LDS read ds_read_b64_tr_b16, which gives
//           lane j of a 16-lane group element e = word j % 4 of the address lane 4 e + j / 4 supplied: lanes
//           pointing at rows k .. k + 3, 4 columns each, receive one column and 4 consecutive rows. Both the stores
//           and the transposing reads spread over all 64 LDS banks. Four register sets: a chunk is loaded three
//           chunks before its LDS store, so the global-load latency overlaps the MFMAs of three chunks.
//   epilog  H[i][j] += (double)acc, coalesced along j.
// Roofline: MFMA (bf16 dense 2.5 PFLOP/s) for batches of more than a few hundred rows: n K (K + 128) flop per
// batch (lower-triangle tiles); below that, HBM: 16 bytes per lower-triangle element of H (fp64 read + write).
//
// ltq_cov_finalize: out[i][j] = (float)(H[max(i,j)][min(i,j)] * inv_n) in 64 x 64 tiles through LDS (the upper
// triangle is read transposed from the lower), the get() of src/liqk_v2.py:230-231 with its fp64 scaling
// (torch's device kernel multiplies by the fp64 reciprocal of the integer count) and round to fp32.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ltq_hip.h"

namespace {

constexpr int kTile = 128;  // edge of an H tile
constexpr int kChunk = 32;  // rows of X per LDS chunk
constexpr int kThreads = 256;
constexpr int kSliceBytes = kTile * kChunk * 2;  // one column slice of a chunk: 32 rows x 128 columns

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

// byte offset in a column slice (32 rows x 128 columns of 16-bit values, 256 bytes a row) of the 16-byte column
// group g (columns 8 g .. 8 g + 7) of row r: the groups of a row are permuted by r % 4
__device__ __forceinline__ int slice_offset(int r, int g) { return 256 * r + 16 * (g ^ (4 * (r & 3))); }

template <bool F16>
__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
}

// Lower-triangle tile t (I >= J) in panel order: panels of 8 tile rows, each panel's tiles column by column
// (J outer, I inner), so consecutive tiles share their column slices of X. Panel P starts at tile
// 8P (8P + 1) / 2 = 32 P^2 + 4 P.
__device__ __forceinline__ void tile_of(int t, int nt, int& I, int& J)
{
    int P = (int)((__builtin_sqrtf(8.f * (float)t + 1.f) - 1.f) / 16.f);
    while (P > 0 && 32 * P * P + 4 * P > t) P--;
    while (32 * (P + 1) * (P + 1) + 4 * (P + 1) <= t) P++;
    const int r0 = 8 * P, h = (nt - r0) < 8 ? nt - r0 : 8;
    int loc = t - (32 * P * P + 4 * P);
    if (loc < r0 * h) {  // full columns left of the diagonal block
        J = loc / h;
        I = r0 + loc % h;
        return;
    }
    loc -= r0 * h;  // lower triangle of the h x h diagonal block, column by column
    int j = 0;
    while (loc >= h - j) {
        loc -= h - j;
        j++;
    }
    J = r0 + j;
    I = r0 + j + loc;
}

// Four rows (r .. r + 3) x 8 columns (c .. c + 7) of X. Element loads (VEC false): zeros outside [n, K]. 16-byte
// loads: rows past n are loaded from row n - 1 and zeroed by store_block.
template <bool VEC>
__device__ __forceinline__ void load_block(const uint16_t* __restrict__ X, long n, int K, long ldx, long r, int c,
                                           u32x4 (&v)[4])
{
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const long row = r + q;
        if constexpr (VEC) {
            // unconditional load from a clamped address (no branch around it, so the compiler can count the
            // loads in flight), rows past n then zeroed; columns past K keep whatever the clamped address
            // holds: column i only enters row and column i of the tile, which are not stored for i >= K
            const long rc = row < n ? row : n - 1;
            const int cc = c < K ? c : K - 8;
            v[q] = *(const u32x4*)(X + rc * ldx + cc);
        } else {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t lo = (row < n && c + 2 * e < K) ? X[row * ldx + c + 2 * e] : 0u;
                const uint32_t hi = (row < n && c + 2 * e + 1 < K) ? X[row * ldx + c + 2 * e + 1] : 0u;
                w[e] = lo | (hi << 16);
            }
            v[q] = u32x4{w[0], w[1], w[2], w[3]};
        }
    }
}

// The 4 x 8 block (rows rq .. rq + 3, column group g) into a column slice; rows q >= nvalid as zeros.
__device__ __forceinline__ void store_block(char* slice, int g, int rq, const u32x4 (&raw)[4], long nvalid)
{
#pragma unroll
    for (int q = 0; q < 4; q++)
        *(u32x4*)(slice + slice_offset(rq + q, g)) = q < nvalid ? raw[q] : u32x4{0u, 0u, 0u, 0u};
}

typedef __attribute__((ext_vector_type(4))) short i16x4;

// MFMA operand of lane l for the 32 columns c0 .. c0 + 31 of a slice and rows k0 .. k0 + 15: column
// c0 + l % 32, rows k0 + 8 (l / 32) .. + 7, as two transposing reads of 4 rows each
__device__ __forceinline__ u32x4 operand(const char* slice, int c0, int k0, int lane)
{
    const int i = lane & 15, grp = lane >> 4;
    const int g = (c0 + 16 * (grp & 1)) / 8 + ((i & 3) >> 1);  // column group of this lane's 4 columns
    const int r = k0 + 8 * (grp >> 1) + (i >> 2);
    const char* p0 = slice + slice_offset(r, g) + 8 * (i & 1);
    const char* p1 = slice + slice_offset(r + 4, g) + 8 * (i & 1);
    const i16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p0);
    const i16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p1);
    const u32x2 ua = __builtin_bit_cast(u32x2, a), ub = __builtin_bit_cast(u32x2, b);
    return u32x4{ua[0], ua[1], ub[0], ub[1]};
}

template <bool F16, bool VEC>
__device__ __forceinline__ void cov_tile(const uint16_t* __restrict__ X, long n, int K, long ldx, int nt, int per_xcd,
                                         double* __restrict__ H, long ldh)
{
    __shared__ __align__(16) char lds[2][2][kSliceBytes];  // [buffer][slice I / J][...], 32 KB
    // workgroup b runs on XCD b % 8 (round-robin dispatch): XCD x takes the contiguous tile range
    // [x per_xcd, (x + 1) per_xcd) of the panel order, so the workgroups resident on one XCD share slices in its L2
    const int t = ((int)blockIdx.x & 7) * per_xcd + ((int)blockIdx.x >> 3);
    if (t >= nt * (nt + 1) / 2) return;
    int I, J;
    tile_of(t, nt, I, J);
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // loader role: slice s (0: columns of tile row I, 1: of tile column J), 4 rows x 8 columns
    const int s = tid >> 7, u = tid & 127, cg = u & 15, rg = u >> 4;
    const int col0 = (s ? J : I) * kTile + 8 * cg;

    // MFMA role: wavefront (wm, wn) owns rows 64 wm .. of the I slice and columns 64 wn .. of the J slice
    const int wm = wave & 1, wn = wave >> 1;
    f32x16 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[a][b][e] = 0.f;

    auto ld = [&](u32x4 (&v)[4], long ch) { load_block<VEC>(X, n, K, ldx, ch * kChunk + 4 * rg, col0, v); };
    auto mma = [&](const char* sa, const char* sb) {
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            u32x4 a[2], b[2];
#pragma unroll
            for (int q = 0; q < 2; q++) {
                a[q] = operand(sa, 64 * wm + 32 * q, 16 * ks, lane);
                b[q] = operand(sb, 64 * wn + 32 * q, 16 * ks, lane);
            }
#pragma unroll
            for (int ta = 0; ta < 2; ta++)
#pragma unroll
                for (int tb = 0; tb < 2; tb++) acc[ta][tb] = mfma<F16>(a[ta], b[tb], acc[ta][tb]);
        }
    };
    // four register sets: chunk c + 1 is loaded three chunks ahead of its LDS store, so the global-load latency
    // overlaps the MFMAs of three chunks; chunks past the end load as zeros without touching memory
    const long nchunks = (n + kChunk - 1) / kChunk;
    u32x4 r0[4], r1[4], r2[4], r3[4];
    ld(r0, 0);
    ld(r1, 1);
    ld(r2, 2);
    ld(r3, 3);
    store_block(lds[0][s], cg, 4 * rg, r0, n - 4 * rg);
    __syncthreads();
    // the scheduling barriers keep the masking and packing of a register set after the MFMAs, so its loads are
    // waited for only when they are stored
    auto step = [&](long ch, u32x4 (&cur)[4], u32x4 (&nxt)[4]) {
        ld(cur, ch + 4);  // cur held chunk ch, already in LDS
        __builtin_amdgcn_sched_barrier(0);
        mma(lds[ch & 1][0], lds[ch & 1][1]);
        __builtin_amdgcn_sched_barrier(0);
        store_block(lds[(ch + 1) & 1][s], cg, 4 * rg, nxt, n - (ch + 1) * kChunk - 4 * rg);
        __syncthreads();
    };
    // whole groups of 4 chunks (the padding chunks are zeros and add nothing): no exit inside the group, so the
    // accumulators stay in place
    for (long ch = 0; ch < nchunks; ch += 4) {
        step(ch, r0, r1);
        step(ch + 1, r1, r2);
        step(ch + 2, r2, r3);
        step(ch + 3, r3, r0);
    }

    // accumulator e of lane l in the 32 x 32 block: row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
#pragma unroll
    for (int ta = 0; ta < 2; ta++)
#pragma unroll
        for (int tb = 0; tb < 2; tb++) {
            const int j = J * kTile + 64 * wn + 32 * tb + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int i = I * kTile + 64 * wm + 32 * ta + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (i < K && j < K) {
                    double* h = H + (long)i * ldh + j;
                    *h = *h + (double)acc[ta][tb][e];
                }
            }
        }
}

// 16-byte loads: 168 registers, three workgroups per CU (96 KB of LDS)
template <bool F16>
__global__ __launch_bounds__(kThreads, 3) void cov_kernel(const uint16_t* __restrict__ X, long n, int K, long ldx,
                                                          int nt, int per_xcd, double* __restrict__ H, long ldh)
{
    cov_tile<F16, true>(X, n, K, ldx, nt, per_xcd, H, ldh);
}

// element loads (rows not 16-byte aligned or K % 8 != 0)
template <bool F16>
__global__ __launch_bounds__(kThreads) void cov_kernel_elem(const uint16_t* __restrict__ X, long n, int K, long ldx,
                                                            int nt, int per_xcd, double* __restrict__ H, long ldh)
{
    cov_tile<F16, false>(X, n, K, ldx, nt, per_xcd, H, ldh);
}

constexpr int kFin = 64;

__global__ __launch_bounds__(256) void cov_finalize_kernel(const double* __restrict__ H, int K, long ldh,
                                                           double inv_n, float* __restrict__ out, long ldo)
{
    __shared__ double t[kFin][kFin + 1];
    const int bi = (int)blockIdx.y, bj = (int)blockIdx.x;
    const int si = bi > bj ? bi : bj, sj = bi > bj ? bj : bi;  // the source tile, on or below the diagonal
    const int tx = (int)threadIdx.x & 63, ty = (int)threadIdx.x >> 6;
    for (int r = ty; r < kFin; r += 4) {
        const int i = si * kFin + r, j = sj * kFin + tx;
        t[r][tx] = (i < K && j < K) ? H[(long)i * ldh + j] : 0.0;
    }
    __syncthreads();
    for (int r = ty; r < kFin; r += 4) {
        const int i = bi * kFin + r, j = bj * kFin + tx;
        if (i >= K || j >= K) continue;
        // element (max(i, j), min(i, j)) of H, relative to the source tile
        const int gi = i > j ? i : j, gj = i > j ? j : i;
        out[(long)i * ldo + j] = (float)(t[gi - si * kFin][gj - sj * kFin] * inv_n);
    }
}

}  // namespace

extern "C" int ltq_cov_accumulate(const void* X, long n, int K, long ldx, int f16, double* H, long ldh, void* stream)
{
    if (n < 0 || K < 1 || ldx < K || ldh < K || !H || (f16 != 0 && f16 != 1)) return -1;
    if (n == 0) return 0;
    if (!X) return -1;
    const long nt = (K + kTile - 1) / kTile;
    const long tiles = nt * (nt + 1) / 2;
    if (tiles > 0x3FFFFFFFL) return -1;
    const int per_xcd = (int)((tiles + 7) / 8);
    const bool vec = ldx % 8 == 0 && K % 8 == 0 && ((uintptr_t)X & 15) == 0;
    const dim3 grid((unsigned)(8 * per_xcd)), block(kThreads);
    const hipStream_t st = (hipStream_t)stream;
    const uint16_t* x = (const uint16_t*)X;
    if (f16) {
        if (vec)
            hipLaunchKernelGGL((cov_kernel<true>), grid, block, 0, st, x, n, K, ldx, (int)nt, per_xcd, H, ldh);
        else
            hipLaunchKernelGGL((cov_kernel_elem<true>), grid, block, 0, st, x, n, K, ldx, (int)nt, per_xcd, H, ldh);
    } else {
        if (vec)
            hipLaunchKernelGGL((cov_kernel<false>), grid, block, 0, st, x, n, K, ldx, (int)nt, per_xcd, H, ldh);
        else
            hipLaunchKernelGGL((cov_kernel_elem<false>), grid, block, 0, st, x, n, K, ldx, (int)nt, per_xcd, H,
                               ldh);
    }
    return (int)hipGetLastError();
}

extern "C" int ltq_cov_finalize(const double* H, int K, long ldh, double inv_n, float* out, long ldo, void* stream)
{
    if (K < 1 || ldh < K || ldo < K || !H || !out) return -1;
    const unsigned nt = (unsigned)((K + kFin - 1) / kFin);
    hipLaunchKernelGGL(cov_finalize_kernel, dim3(nt, nt), dim3(256), 0, (hipStream_t)stream, H, K, ldh, inv_n, out,
                       ldo);
    return (int)hipGetLastError();
}
