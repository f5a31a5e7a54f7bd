// .ltq tile bit-packing for gfx950 (src/ltq_format.py:104-124, src/ltq_file.py:67-96).
//
// A row slice [R, K] of codes (label * U + u, int16) and gain indices (uint8) becomes four structure-of-arrays
// regions, each starting on a 64-byte boundary of the output:
//   codes  [T, 16] u16          bit j of word w = code bit (label & 1) of tile position 16 w + j
//   planes [T, K-2, 16] u16     uncoded bits 1 .. K-2 of u, same layout
//   lsb    [T, 16 | 8 | 12]     lowest uncoded bit: every position / one per pair (D2) / three per quad (D4)
//   gains  [T, ceil(256/sub*h/16)] u16   gain index of each sub-block, h bits LSB first, back to back
// Tiles are ordered by row group then 16-column block; tile position t = 16 r + c is row 16 rg + r, column
// 16 kb + c. One wavefront packs one tile: it stages the tile's 256 codes in LDS, then each lane assembles
// whole 16-bit words.
//
// Roofline: HBM, 3 bytes in per weight (int16 code + uint8 gain index) plus the tile bytes out.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ltq_hip.h"

namespace {

constexpr int kWaves = 4;

struct PackGeo {
    int K, frac, h, sub, U;
    int n[4];      // u16 words per tile of each region
    long off[4];   // byte offset of each region
    long total;    // bytes of the slice
};

__host__ __device__ inline long align64(long v) { return (v + 63) & ~63L; }

__host__ __device__ inline PackGeo pack_geo(int R, int Kc, int K, int frac, int h, int sub)
{
    PackGeo g;
    g.K = K;
    g.frac = frac;
    g.h = h;
    g.sub = sub;
    g.U = 1 << (K - 1);
    const long T = (long)(R / 16) * (Kc / 16);
    const int lsb_bits = frac == 0 ? 256 : frac == 1 ? 128 : 192;
    g.n[0] = 16;
    g.n[1] = 16 * (K > 2 ? K - 2 : 0);
    g.n[2] = K > 1 ? (lsb_bits + 15) / 16 : 0;
    g.n[3] = h ? (256 / sub * h + 15) / 16 : 0;
    long o = 0;
    for (int r = 0; r < 4; r++) {
        o = align64(o);
        g.off[r] = o;
        o += 2 * T * g.n[r];
    }
    g.total = o;
    return g;
}

__global__ __launch_bounds__(64 * kWaves) void pack_kernel(const int16_t* __restrict__ idx, long ld_idx,
                                                           const uint8_t* __restrict__ gi, long ld_gi, int R, int Kc,
                                                           PackGeo g, uint8_t* __restrict__ out)
{
    __shared__ int16_t s_ix[kWaves][256];
    __shared__ uint8_t s_g[kWaves][256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kbs = Kc / 16;
    const long T = (long)(R / 16) * kbs;
    // zero the gaps between regions (the reference pads with zero bytes)
    if (blockIdx.x == 0) {
        for (int r = 1; r < 4; r++) {
            const long end_prev = g.off[r - 1] + 2 * T * g.n[r - 1];
            for (long b = end_prev + threadIdx.x; b < g.off[r]; b += blockDim.x) out[b] = 0;
        }
    }
    for (long tile = (long)blockIdx.x * kWaves + wv; tile < T; tile += (long)gridDim.x * kWaves) {
        const long rg = tile / kbs, kb = tile - rg * kbs;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 4 * lane + i, r = t >> 4, c = t & 15;
            const long row = rg * 16 + r, col = kb * 16 + c;
            s_ix[wv][t] = idx[row * ld_idx + col];
            s_g[wv][t] = gi[row * ld_gi + col];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int W = g.n[0] + g.n[1] + g.n[2] + g.n[3];
        for (int w = lane; w < W; w += 64) {
            int reg = 0, wr = w;
            while (wr >= g.n[reg]) {
                wr -= g.n[reg];
                reg++;
            }
            uint32_t word = 0;
            for (int j = 0; j < 16; j++) {
                const int i = 16 * wr + j;  // bit index within the region's stream of this tile
                uint32_t bit = 0;
                if (reg == 0) {
                    bit = ((uint32_t)s_ix[wv][i] >> (g.K - 1)) & 1;  // label & 1
                } else if (reg == 1) {
                    const int p = 1 + wr / 16, t = 16 * (wr % 16) + j;
                    bit = (((uint32_t)s_ix[wv][t] & (g.U - 1)) >> p) & 1;
                } else if (reg == 2) {
                    const int nb = g.frac == 0 ? 256 : g.frac == 1 ? 128 : 192;
                    if (i < nb) {
                        const int t = g.frac == 0 ? i : g.frac == 1 ? 2 * i : 4 * (i / 3) + i % 3;
                        bit = (uint32_t)s_ix[wv][t] & 1;
                    }
                } else {
                    const int nb = 256 / g.sub * g.h;
                    if (i < nb) bit = ((uint32_t)s_g[wv][g.sub * (i / g.h)] >> (i % g.h)) & 1;
                }
                word |= bit << j;
            }
            *(uint16_t*)(out + g.off[reg] + 2 * (tile * g.n[reg] + wr)) = (uint16_t)word;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

}  // namespace

extern "C" long ltq_slice_bytes(int R, int K, int fmt_K, int frac, int h, int sub)
{
    if (R < 0 || K < 0 || R % 16 || K % 16 || fmt_K < 1 || fmt_K > 8 || frac < 0 || frac > 2 || h < 0 || h > 8 || sub <= 0 ||
        256 % sub)
        return -1;
    return pack_geo(R, K, fmt_K, frac, h, sub).total;
}

extern "C" int ltq_pack_slice(const int16_t* idx, long ld_idx, const uint8_t* gi, long ld_gi, int R, int K, int fmt_K,
                              int frac, int h, int sub, uint8_t* out, long out_bytes, void* stream)
{
    const long need = ltq_slice_bytes(R, K, fmt_K, frac, h, sub);
    if (need < 0 || out_bytes < need || ld_idx < K || ld_gi < K) return -1;
    if (R == 0 || K == 0) return 0;
    if (!idx || !gi || !out) return -1;
    const PackGeo g = pack_geo(R, K, fmt_K, frac, h, sub);
    const long T = (long)(R / 16) * (K / 16);
    long grid = (T + kWaves - 1) / kWaves;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(pack_kernel, dim3((unsigned)grid), dim3(64 * kWaves), 0, (hipStream_t)stream, idx, ld_idx, gi, ld_gi,
                       R, K, g, out);
    return (int)hipGetLastError();
}
