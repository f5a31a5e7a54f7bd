// The two dense contractions of the LDLQ block error feedback on the matrix cores (gfx950 fp32 MFMA).
//
// After the 16 sub-blocks of a 256-column block [c0, c1) (src/liqk_v2.py:972-979):
//   ltq_ldlq_err:     E = (W_start - d * G) @ U_blk_inv          [M, 256] @ [256, 256], stored transposed (E^T)
//                     (and W_hat[:, c0:c1] = d * G, the block's reconstruction)
//   ltq_ldlq_update:  W[:, c1:] -= E @ U[c0:c1, c1:]             [M, 256] @ [256, K - c1]
//                     (and the next block's working copy and first Viterbi tiles from the updated columns)
// with the element-wise products and differences rounded as the reference's torch code rounds them.
//
// Summation order. Every output is the fp32 fused multiply-add chain over k = 0, 1, ..., 255 in ascending order
// starting from 0, i.e. acc = fma(a[k], b[k], acc), then (update) w - acc. v_mfma_f32_16x16x4_f32 computes
// exactly that chain over its four k (measured on gfx950: every output of random and cancelling inputs equals
// the ascending correctly rounded FMA chain, no other ordering or single rounding does), and the kernels issue
// the instructions of an output in ascending k, so the result is a defined function of the inputs that a CPU
// restatement with fmaf reproduces bit for bit. (A library GEMM's split-k and blocking orders are not fixed.)
//
// Tiling. A workgroup of 4 wavefronts computes a 128 x 128 output tile; wavefront (wr, wc) a 64 x 64 quarter
// as 4 x 4 MFMA blocks of 16 x 16. k advances in stages of 16: the stage's A (128 x 16) and B (16 x 128)
// operands go global -> registers -> LDS (k-major, row pitch 144 floats: each half-wavefront's operand reads
// hit 32 distinct banks), double-buffered, one barrier per stage, the next stage's loads in flight during the
// current stage's 64 MFMAs per wavefront. Workgroups are dealt to the 8 XCDs in contiguous tile ranges with
// the row tile fastest, so the workgroups on one XCD share the U column panels in its L2. Launch bounds ask for
// three workgroups per CU: the compiler then keeps the accumulators in ordinary VGPRs (116 / 124, no AGPRs) and
// four fit. The update's epilogue reads each row block's 16 old values of W at once before storing (the loop
// that read, subtracted and stored one value at a time waited for every load in turn): 11.0 -> 8.8 ms per C3
// step, 0.48 -> 0.60 of the fp32 MFMA peak.
// Roofline: MFMA fp32 (157.3 TFLOP/s dense), 2 M 256 N flops per update.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ltq_hip.h"
#include "ltq_timing.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, KC = 16, LDP = 144, KD = 256;

struct GemmArgs {
    // A operand: AMODE 0 -> at[k * ld_a + i] (k-major E^T); AMODE 1 -> ws[i * ld_a + k] - d[i * ldd] * g[i * ldg + k]
    const float* a;
    long ld_a;
    const float* g;
    long ldg;
    const float* d;
    long ldd;
    const float* b;  // B operand b[k * ldb + j], k < 256
    long ldb;
    long M, N;       // output rows, columns (N % 128 == 0)
    long rows_per_mat, b_ms;  // stacked matrices: rows [m R, (m + 1) R) use the B operand b + m * b_ms
    // EPI 0: out[j * ld_out + i] = acc (transposed), what[i * ld_what + j] = d g (column tile 0's A values)
    // EPI 1: out[i * ld_out + j] -= acc; wsub[i * ld_wsub + j] = new value for j < 256; xnext for j < 16
    float* out;
    long ld_out;
    float* what;
    long ld_what;
    float* wsub;
    long ld_wsub;
    float* xnext;
    const float* dnext;
    long ld_dnext;
    int tiles_m, tiles_n;
};

// XCD-aware tile order: block b runs on XCD b % 8; XCD x takes a contiguous range of tiles, row tile fastest
__device__ __forceinline__ void tile_of(int b, int tiles_m, int tiles_n, int& tm, int& tn)
{
    const int nt = tiles_m * tiles_n, q = nt / 8, r = nt % 8;
    const int xcd = b % 8, slot = b / 8;
    const int t = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + slot;
    tm = t % tiles_m;
    tn = t / tiles_m;
}

template <int AMODE, int EPI>
__global__ __launch_bounds__(256, 3) void ldlq_gemm_kernel(GemmArgs p)
{
    __shared__ __align__(16) float sA[2][KC][LDP];
    __shared__ __align__(16) float sB[2][KC][LDP];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    int tm, tn;
    tile_of((int)blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const long row0 = (long)tm * BM, col0 = (long)tn * BN;
    if (p.rows_per_mat > 0) p.b += (row0 / p.rows_per_mat) * p.b_ms;  // a tile never straddles two matrices
    const bool write_what = EPI == 0 && p.what != nullptr && tn == 0;

    // staging registers of one stage: 2 float4 of A and 2 of B per thread. AMODE 1 keeps its raw operands
    // (ws, g, d) until store_stage, after the stage's MFMAs: no arithmetic or store sits between the loads and the
    // MFMAs, so the next stage's loads fly while they run.
    v4f ra[2], rb[2], rw[2], rg[2];
    float rd[2];
    int k_st = 0;  // k0 of the staged stage
    auto load_stage = [&](int k0) {
        k_st = k0;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int e = tid + 256 * q;
            // B: row k = e / 32, columns 4 (e % 32) .. + 3
            const int kb = e >> 5, jb = (e & 31) * 4;
            rb[q] = *(const v4f*)(p.b + (long)(k0 + kb) * p.ldb + col0 + jb);
            if constexpr (AMODE == 0) {
                // A^T: row k = e / 32, output rows 4 (e % 32) .. + 3
                const long i = row0 + (e & 31) * 4;
                ra[q] = i < p.M ? *(const v4f*)(p.a + (long)(k0 + kb) * p.ld_a + i) : v4f{0.f, 0.f, 0.f, 0.f};
            } else {
                // A: output row r = e / 4, k = 4 (e % 4) .. + 3, later ws - d * g
                const long i = row0 + (e >> 2);
                const int k = k0 + (e & 3) * 4;
                const bool in = i < p.M;
                rw[q] = in ? *(const v4f*)(p.a + i * p.ld_a + k) : v4f{0.f, 0.f, 0.f, 0.f};
                rg[q] = in ? *(const v4f*)(p.g + i * p.ldg + k) : v4f{0.f, 0.f, 0.f, 0.f};
                rd[q] = in ? p.d[i * p.ldd] : 0.f;
            }
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int e = tid + 256 * q;
            const int kb = e >> 5, jb = (e & 31) * 4;
            *(v4f*)&sB[buf][kb][jb] = rb[q];
            if constexpr (AMODE == 0) {
                *(v4f*)&sA[buf][kb][(e & 31) * 4] = ra[q];
            } else {
                const int r = e >> 2, k = (e & 3) * 4;
                const float dd = rd[q];
                const v4f dg = v4f{dd * rg[q].x, dd * rg[q].y, dd * rg[q].z, dd * rg[q].w};
                const long i = row0 + r;
                if (write_what && i < p.M) *(v4f*)(p.what + i * p.ld_what + k_st + k) = dg;
                const v4f a = rw[q] - dg;
                sA[buf][k + 0][r] = a.x;
                sA[buf][k + 1][r] = a.y;
                sA[buf][k + 2][r] = a.z;
                sA[buf][k + 3][r] = a.w;
            }
        }
    };

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

    load_stage(0);
    store_stage(0);
    __syncthreads();
    constexpr int NST = KD / KC;
    const int kl = lane >> 4, il = lane & 15;
    for (int s = 0; s < NST; s++) {
        const int buf = s & 1;
        if (s + 1 < NST) load_stage((s + 1) * KC);
#pragma unroll
        for (int kk = 0; kk < KC; kk += 4) {
            float av[4], bv[4];
#pragma unroll
            for (int r = 0; r < 4; r++) av[r] = sA[buf][kk + kl][wr * 64 + r * 16 + il];
#pragma unroll
            for (int c = 0; c < 4; c++) bv[c] = sB[buf][kk + kl][wc * 64 + c * 16 + il];
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    acc[r][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[r], bv[c], acc[r][c], 0, 0, 0);
        }
        if (s + 1 < NST) {
            store_stage(buf ^ 1);
            __syncthreads();
        }
    }

    // epilogue: block (r, c) register v is output row 16 r + 4 (lane / 16) + v, column 16 c + lane % 16
    if constexpr (EPI == 0) {
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const long i = row0 + wr * 64 + r * 16 + 4 * kl + v;
                if (i >= p.M) continue;
#pragma unroll
                for (int c = 0; c < 4; c++) p.out[(col0 + wc * 64 + c * 16 + il) * p.ld_out + i] = acc[r][c][v];
            }
    } else {
        // per row block r: its 16 old values in flight at once, before any store (the stores go to other buffers
        // or to the same elements, so no load waits on a store), then the new values out
        const bool xn = p.xnext != nullptr && col0 == 0 && wc == 0;  // the tile holding columns 0..15
#pragma unroll
        for (int r = 0; r < 4; r++) {
            float wv[4][4], inv[4];
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const long i = row0 + wr * 64 + r * 16 + 4 * kl + v;
#pragma unroll
                for (int c = 0; c < 4; c++)
                    wv[v][c] = i < p.M ? p.out[i * p.ld_out + col0 + wc * 64 + c * 16 + il] : 0.f;
                inv[v] = xn && i < p.M ? 1.0f / p.dnext[i * p.ld_dnext] : 0.f;
            }
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const long i = row0 + wr * 64 + r * 16 + 4 * kl + v;
                if (i >= p.M) continue;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const long j = col0 + wc * 64 + c * 16 + il;
                    const float nv = wv[v][c] - acc[r][c][v];
                    p.out[i * p.ld_out + j] = nv;
                    if (p.wsub && j < KD) p.wsub[i * p.ld_wsub + j] = nv;
                    if (xn && c == 0) p.xnext[(i >> 4) * 256 + (i & 15) * 16 + il] = nv * inv[v];
                }
            }
        }
    }
}

int launch_gemm(int amode, int epi, GemmArgs p, hipStream_t st)
{
    p.tiles_m = (int)((p.M + BM - 1) / BM);
    p.tiles_n = (int)(p.N / BN);
    const unsigned grid = (unsigned)(p.tiles_m * p.tiles_n);
    if (grid == 0) return 0;
    if (amode == 0 && epi == 1) return ltq::timed_launch(ltq::kernel_timing, ldlq_gemm_kernel<0, 1>, dim3(grid), dim3(256), 0, st, p);
    if (amode == 1 && epi == 0) return ltq::timed_launch(ltq::kernel_timing, ldlq_gemm_kernel<1, 0>, dim3(grid), dim3(256), 0, st, p);
    return -1;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

static bool bad_stack(long M, long rows_per_mat, long b_ms)
{
    return rows_per_mat < 0 || (rows_per_mat > 0 && (rows_per_mat % BM || M % rows_per_mat || (b_ms & 3)));
}

extern "C" int ltq_ldlq_err(const float* wstart, long ldw, const float* G, long ldg, const float* d, long ldd,
                            const float* uinv, long ldi, float* et, long ld_et, float* what, long ld_what, long M,
                            long rows_per_mat, long uinv_ms, void* stream)
{
    if (M < 0 || M % 16 || ldw < 256 || ldg < 256 || ldd < 1 || ldi < 256 || ld_et < M || (what && ld_what < 256))
        return -1;
    if (bad_stack(M, rows_per_mat, uinv_ms)) return -1;
    if (M == 0) return 0;
    if (!wstart || !G || !d || !uinv || !et) return -1;
    if ((ldw | ldg | ldi | ld_et | (what ? ld_what : 0)) & 3) return -1;
    if (!aligned16(wstart) || !aligned16(G) || !aligned16(uinv) || !aligned16(et) || (what && !aligned16(what)))
        return -1;
    GemmArgs p{};
    p.a = wstart;
    p.ld_a = ldw;
    p.g = G;
    p.ldg = ldg;
    p.d = d;
    p.ldd = ldd;
    p.b = uinv;
    p.ldb = ldi;
    p.M = M;
    p.N = KD;
    p.out = et;
    p.ld_out = ld_et;
    p.what = what;
    p.ld_what = ld_what;
    p.rows_per_mat = rows_per_mat;
    p.b_ms = uinv_ms;
    return launch_gemm(1, 0, p, (hipStream_t)stream);
}

extern "C" int ltq_ldlq_update(float* w, long ldw, const float* et, long ld_et, const float* u, long ldu, long M, long N,
                               float* wsub, long ld_wsub, float* xnext, const float* dnext, long ld_dnext,
                               long rows_per_mat, long u_ms, void* stream)
{
    if (bad_stack(M, rows_per_mat, u_ms)) return -1;
    if (M < 0 || N < 0 || M % 16 || N % BN || ldw < N || ld_et < M || ldu < N || (wsub && (ld_wsub < KD || N < KD)) ||
        (xnext && (!dnext || ld_dnext < 1 || N < 16)))
        return -1;
    if (M == 0 || N == 0) return 0;
    if (!w || !et || !u) return -1;
    if ((ld_et | ldu) & 3) return -1;
    if (!aligned16(et) || !aligned16(u)) return -1;
    GemmArgs p{};
    p.a = et;
    p.ld_a = ld_et;
    p.b = u;
    p.ldb = ldu;
    p.M = M;
    p.N = N;
    p.out = w;
    p.ld_out = ldw;
    p.wsub = wsub;
    p.ld_wsub = ld_wsub;
    p.xnext = xnext;
    p.dnext = dnext;
    p.ld_dnext = ld_dnext;
    p.rows_per_mat = rows_per_mat;
    p.b_ms = u_ms;
    return launch_gemm(0, 1, p, (hipStream_t)stream);
}
