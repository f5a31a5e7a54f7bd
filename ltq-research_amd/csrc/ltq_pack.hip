// .ltq tile bit-packing for gfx950 (src/ltq_format.py:104-124, src/ltq_file.py:67-96).
//
// A row slice [R, K] of codes (label * U + u, int16) and gain indices (uint8) becomes four structure-of-arrays
// regions, each starting on a 64-byte boundary of the output:
//   codes  [T, 16] u16          bit j of word w = code bit (label & 1) of tile position 16 w + j
//   planes [T, K-2, 16] u16     uncoded bits 1 .. K-2 of u, same layout
//   lsb    [T, 16 | 8 | 12]     lowest uncoded bit: every position / one per pair (D2) / three per quad (D4)
//   gains  [T, ceil(256/sub*h/16)] u16   gain index of each sub-block, h bits LSB first, back to back
// Tiles are ordered by row group then 16-column block; tile position t = 16 r + c is row 16 rg + r, column
// 16 kb + c. A workgroup packs a strip of 16 consecutive tiles of one row group: contiguous row loads into LDS,
// every 64 bits of a field's stream from one wavefront ballot, each region's run of the strip written at once.
//
// Row rings (src/ltq_format.py:42-50, 104-124 with L instead of 256; the ring tables of src/ple_quant.py): a
// ring of L positions (L % 16 == 0, L <= 512) packs into one record of the same four fields back to back,
// 2 (L/16 + L/16 (K-2) + lsb words + gain words) bytes; rings are consecutive records.
//
// Roofline: HBM, 3 bytes in per weight (int16 code + uint8 gain index) plus the tile bytes out.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ltq_hip.h"
#include "ltq_timing.h"

namespace {

constexpr int kWaves = 4;
constexpr int kMaxL = 512;

// Field sizes of one tile / ring of L positions (src/ltq_format.py:42-50): u16 words per field and where each
// field starts -- region offsets of a slice (structure of arrays) or word offsets inside a ring record.
struct PackGeo {
    int K, frac, h, sub, U, L;
    int n[4];      // u16 words per tile / ring: codes, planes, lsb, gains
    long off[4];   // slice: byte offset of each region; rings: word offset of each field inside a record
    long total;    // slice: bytes of the slice; rings: bytes of one record
};

__host__ __device__ inline long align64(long v) { return (v + 63) & ~63L; }

__host__ __device__ inline int lsb_bits(int frac, int L) { return frac == 0 ? L : frac == 1 ? L / 2 : 3 * L / 4; }

__host__ __device__ inline void field_words(PackGeo& g, int K, int frac, int h, int sub, int L)
{
    g.K = K;
    g.frac = frac;
    g.h = h;
    g.sub = sub;
    g.U = 1 << (K - 1);
    g.L = L;
    g.n[0] = L / 16;
    g.n[1] = L / 16 * (K > 2 ? K - 2 : 0);
    g.n[2] = K > 1 ? (lsb_bits(frac, L) + 15) / 16 : 0;
    g.n[3] = h ? (L / sub * h + 15) / 16 : 0;
}

__host__ __device__ inline PackGeo pack_geo(int R, int Kc, int K, int frac, int h, int sub)
{
    PackGeo g;
    field_words(g, K, frac, h, sub, 256);
    const long T = (long)(R / 16) * (Kc / 16);
    long o = 0;
    for (int r = 0; r < 4; r++) {
        o = align64(o);
        g.off[r] = o;
        o += 2 * T * g.n[r];
    }
    g.total = o;
    return g;
}

__host__ __device__ inline PackGeo ring_geo(int L, int K, int frac, int h, int sub)
{
    PackGeo g;
    field_words(g, K, frac, h, sub, L);
    long o = 0;
    for (int r = 0; r < 4; r++) {
        g.off[r] = o;
        o += g.n[r];
    }
    g.total = 2 * o;
    return g;
}

__device__ inline void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Bit streams of the four fields of one tile / ring of L positions, as wave ballots: the bit of stream element
// e = 64 q + lane is computed by lane `lane`, ballot(bit) is 64 consecutive stream bits = 4 consecutive u16
// words, and lanes 0..3 hand one word each to store(field, word, value).
//   codes   e = position t:                       bit K-1 of the code (= label & 1)
//   planes  e = position t, plane p = 1 .. K-2:   bit p of u (= code & (U - 1))
//   lsb     frac 0: e = t; 1 (D2): t = 2 e; 2 (D4): t = 4 (e / 3) + e % 3 (the first three of each quad): bit 0
//   gains   e < (L / sub) h: bit e % h of the gain index at the first position of sub-block e / h
// ixat(t) / gat(t) read the code / gain index of position t; bits past a stream's end are 0.
template <class IX, class GG, class ST>
__device__ inline void ballot_fields(const PackGeo& g, int lane, IX ixat, GG gat, ST store)
{
    const int L = g.L, W = L / 16;
    auto put = [&](int field, int w0, int nw, unsigned long long m) {
        if (lane < 4 && w0 + lane < nw) store(field, w0 + lane, (uint16_t)(m >> (16 * lane)));
    };
    for (int q = 0; q < (L + 63) / 64; q++) {
        const int t = 64 * q + lane;
        const uint32_t v = t < L ? (uint32_t)(uint16_t)ixat(t) : 0u;
        put(0, 4 * q, W, __ballot((v >> (g.K - 1)) & 1u));
        for (int p = 1; p < g.K - 1; p++) put(1, (p - 1) * W + 4 * q, p * W, __ballot(((v & (g.U - 1)) >> p) & 1u));
        if (g.K > 1 && g.frac == 0) put(2, 4 * q, W, __ballot(v & 1u));
    }
    if (g.K > 1 && g.frac != 0) {
        const int nb = lsb_bits(g.frac, L);
        for (int q = 0; q < (nb + 63) / 64; q++) {
            const int e = 64 * q + lane;
            const int t = g.frac == 1 ? 2 * e : 4 * (e / 3) + e % 3;
            const uint32_t b = e < nb ? ((uint32_t)(uint16_t)ixat(t) & 1u) : 0u;
            put(2, 4 * q, g.n[2], __ballot(b));
        }
    }
    if (g.h) {
        const int nb = L / g.sub * g.h;
        for (int q = 0; q < (nb + 63) / 64; q++) {
            const int e = 64 * q + lane;
            const uint32_t b = e < nb ? ((uint32_t)gat(g.sub * (e / g.h)) >> (e % g.h)) & 1u : 0u;
            put(3, 4 * q, g.n[3], __ballot(b));
        }
    }
}

// field and word within it of word w of a tile / ring's concatenated fields
__device__ inline void word_region(const PackGeo& g, int w, int& reg, int& wr)
{
    reg = 0;
    wr = w;
    while (wr >= g.n[reg]) {
        wr -= g.n[reg];
        reg++;
    }
}

constexpr int kStrip = 16;             // tiles per workgroup: one row group, 16 consecutive 16-column blocks
constexpr int kMaxTileWords = 256;     // codes 16 + planes 16 (K-2) <= 96 + lsb <= 16 + gains 256 / sub h / 16 <= 128

// One workgroup (4 wavefronts) per strip of 16 consecutive tiles of one row group: the strip's 16 rows x 256
// columns of codes and gain indices come in as contiguous 16-byte row loads into LDS, each wavefront turns tiles
// j = wave, wave + 4, ... into their words (ballot_fields) staged field by field, and each field's words of the
// strip -- contiguous in the output, tiles being consecutive -- are written as one run of u16 stores. (A
// wavefront per 4 tiles without workgroup barriers, or per whole strip, measured slower: 137 and 246 us
// against 128 us for the C3 slice.) Dynamic LDS: the staging, 16 x tile words x 2 bytes.
__global__ __launch_bounds__(256) void pack_strip_kernel(const int16_t* __restrict__ idx, long ld_idx,
                                                         const uint8_t* __restrict__ gi, long ld_gi, int R, int Kc,
                                                         PackGeo g, int vec, uint8_t* __restrict__ out)
{
    __shared__ __align__(16) int16_t s_ix[16][kStrip * 16];
    __shared__ __align__(16) uint8_t s_g[16][kStrip * 16];
    extern __shared__ uint16_t s_w[];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int kbs = Kc / 16, spr = (kbs + kStrip - 1) / kStrip;
    const long T = (long)(R / 16) * kbs;
    // zero the gaps between regions (the reference pads with zero bytes)
    if (blockIdx.x == 0) {
        for (int r = 1; r < 4; r++) {
            const long end_prev = g.off[r - 1] + 2 * T * g.n[r - 1];
            for (long b = end_prev + tid; b < g.off[r]; b += blockDim.x) out[b] = 0;
        }
    }
    const long rg = (long)blockIdx.x / spr;
    const int kb0 = (int)((long)blockIdx.x % spr) * kStrip;
    const int nt = kbs - kb0 < kStrip ? kbs - kb0 : kStrip;
    {  // thread (row r, chunk c) loads the strip's columns 16 c .. 16 c + 15 of row r
        const int r = tid >> 4, c = tid & 15;
        if (c < nt) {
            const long row = rg * 16 + r, col = (long)(kb0 + c) * 16;
            const int16_t* src = idx + row * ld_idx + col;
            const uint8_t* gsrc = gi + row * ld_gi + col;
            if (vec) {
                *(uint4*)&s_ix[r][16 * c] = *(const uint4*)src;
                *(uint4*)&s_ix[r][16 * c + 8] = *(const uint4*)(src + 8);
                *(uint4*)&s_g[r][16 * c] = *(const uint4*)gsrc;
            } else {
                for (int k = 0; k < 16; k++) {
                    s_ix[r][16 * c + k] = src[k];
                    s_g[r][16 * c + k] = gsrc[k];
                }
            }
        }
    }
    __syncthreads();
    int base[4];
    base[0] = 0;
    for (int f = 1; f < 4; f++) base[f] = base[f - 1] + kStrip * g.n[f - 1];
    for (int j = wv; j < nt; j += 4) {
        ballot_fields(
            g, lane, [&](int t) { return s_ix[t >> 4][16 * j + (t & 15)]; },
            [&](int t) { return s_g[t >> 4][16 * j + (t & 15)]; },
            [&](int f, int w, uint16_t v) { s_w[base[f] + j * g.n[f] + w] = v; });
    }
    __syncthreads();
    const long T0 = rg * kbs + kb0;
    for (int f = 0; f < 4; f++) {
        uint16_t* dst = (uint16_t*)(out + g.off[f]) + T0 * g.n[f];
        const int cnt = nt * g.n[f];
        for (int w = tid; w < cnt; w += 256) dst[w] = s_w[base[f] + w];
    }
}

// Sub-blocks of 16 positions or more (every production format). One wavefront per 16 consecutive tiles of one
// row group, no LDS and no barrier: lane (j = lane / 4, q = lane % 4) loads rows 4 q .. 4 q + 3 of tile j (four
// 32-byte code runs and the gain index at each row's first position) and writes those rows' share of every
// field. Each field stream is row-major with a fixed bit count per tile row (16 for codes and planes, 16 | 8 | 12
// for lsb), so the share is a contiguous run of the tile's words and goes out as one 8 / 4 / 6-byte store; gains
// (h bits per sub-block start) are assembled across the four lanes of the tile with quad broadcasts.
// Bit gather: dword d of a row holds codes 2 d (low half) and 2 d + 1 (high half); rotating it right by
// (b - 2 d) puts bit b of code 2 d at 2 d and of code 2 d + 1 at 16 + 2 d, so 8 rotate + mask-or steps collect
// a row's even codes in the low half and odd codes in the high half, one shift interleaves them.
__device__ inline uint32_t row_bits(const uint32_t (&x)[8], int b)
{
    uint32_t acc = 0;
#pragma unroll
    for (int d = 0; d < 8; d++)
        acc |= __builtin_amdgcn_alignbit(x[d], x[d], (uint32_t)(b - 2 * d) & 31u) & (0x10001u << (2 * d));
    return (acc & 0xffffu) | ((acc >> 15) & 0xfffeu);
}

// bit 0 of the first three codes of each quad (D4): code 4 m + k -> bit 3 m + k, 12 bits
__device__ inline uint32_t row_lsb_d4(const uint32_t (&x)[8])
{
    uint32_t v = 0;
#pragma unroll
    for (int m = 0; m < 4; m++)
        v |= ((x[2 * m] & 1u) << (3 * m)) | (((x[2 * m] >> 16) & 1u) << (3 * m + 1)) | ((x[2 * m + 1] & 1u) << (3 * m + 2));
    return v;
}

// bit 0 of the even codes (D2): code 2 d -> bit d, 8 bits
__device__ inline uint32_t row_lsb_d2(const uint32_t (&x)[8])
{
    uint32_t v = 0;
#pragma unroll
    for (int d = 0; d < 8; d++) v |= (x[d] & 1u) << d;
    return v;
}

template <int Q>
__device__ inline uint32_t quad_lane(uint32_t v)  // lane Q of this lane's quad
{
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, Q * 0x55, 0xf, 0xf, false);
}

__global__ __launch_bounds__(256) void pack_quads_kernel(const int16_t* __restrict__ idx, long ld_idx,
                                                         const uint8_t* __restrict__ gi, long ld_gi, int R, int Kc,
                                                         PackGeo g, int vec, uint8_t* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int kbs = Kc / 16, spr = (kbs + 15) / 16;
    const long T = (long)(R / 16) * kbs;
    if (blockIdx.x == 0) {  // zero the gaps between regions (the reference pads with zero bytes)
        for (int r = 1; r < 4; r++) {
            const long end_prev = g.off[r - 1] + 2 * T * g.n[r - 1];
            for (long b = end_prev + threadIdx.x; b < g.off[r]; b += blockDim.x) out[b] = 0;
        }
    }
    const long wave = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave >= (long)(R / 16) * spr) return;
    const long rg = wave / spr;
    const int kb = (int)(wave - rg * spr) * 16 + (lane >> 2);
    if (kb >= kbs) return;  // whole quads leave together: the quad broadcasts below see four live lanes
    const int q = lane & 3;
    const long tile = rg * kbs + kb, row = rg * 16 + 4 * q, col = (long)kb * 16;
    uint32_t x[4][8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int16_t* src = idx + (row + i) * ld_idx + col;
        if (vec) {
            const uint4 a = *(const uint4*)src, b = *(const uint4*)(src + 8);
            x[i][0] = a.x, x[i][1] = a.y, x[i][2] = a.z, x[i][3] = a.w;
            x[i][4] = b.x, x[i][5] = b.y, x[i][6] = b.z, x[i][7] = b.w;
        } else {
#pragma unroll
            for (int d = 0; d < 8; d++) x[i][d] = (uint32_t)(uint16_t)src[2 * d] | (uint32_t)(uint16_t)src[2 * d + 1] << 16;
        }
    }
    const int rs = g.sub / 16;  // tile rows per sub-block
    uint32_t gv = 0;            // this lane's gain bits, sub-block starts in row order
    if (g.h) {
        int k = 0;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if ((4 * q + i) % rs == 0) gv |= ((uint32_t)gi[(row + i) * ld_gi + col] & ((1u << g.h) - 1)) << (g.h * k++);
    }
    // rows' words of one plane of bits: 4 words, rows 4 q .. 4 q + 3
    auto put4 = [&](int f, long word, int b) {
        const uint32_t w0 = row_bits(x[0], b) | row_bits(x[1], b) << 16, w1 = row_bits(x[2], b) | row_bits(x[3], b) << 16;
        *(uint2*)(out + g.off[f] + 2 * word) = make_uint2(w0, w1);
    };
    put4(0, tile * 16 + 4 * q, g.K - 1);
    for (int p = 1; p < g.K - 1; p++) put4(1, tile * g.n[1] + (p - 1) * 16 + 4 * q, p);
    if (g.K > 1) {
        if (g.frac == 0) {
            put4(2, tile * 16 + 4 * q, 0);
        } else if (g.frac == 1) {
            const uint32_t v = row_lsb_d2(x[0]) | row_lsb_d2(x[1]) << 8 | row_lsb_d2(x[2]) << 16 | row_lsb_d2(x[3]) << 24;
            *(uint32_t*)(out + g.off[2] + 2 * (tile * 8 + 2 * q)) = v;
        } else {
            const uint64_t v = (uint64_t)(row_lsb_d4(x[0]) | row_lsb_d4(x[1]) << 12) |
                               (uint64_t)(row_lsb_d4(x[2]) | row_lsb_d4(x[3]) << 12) << 24;
            uint16_t* dst = (uint16_t*)(out + g.off[2]) + tile * 12 + 3 * q;
            dst[0] = (uint16_t)v;
            dst[1] = (uint16_t)(v >> 16);
            dst[2] = (uint16_t)(v >> 32);
        }
    }
    if (g.h) {
        // lane k's bits start after the sub-block starts of rows 0 .. 4 k - 1: ceil(4 k / rs) of them
        const uint32_t v[4] = {quad_lane<0>(gv), quad_lane<1>(gv), quad_lane<2>(gv), quad_lane<3>(gv)};
        uint64_t lo = 0, hi = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int o = (4 * k + rs - 1) / rs * g.h;
            if (o < 64) {
                lo |= (uint64_t)v[k] << o;
                if (o > 32) hi |= (uint64_t)v[k] >> (64 - o);
            } else {
                hi |= (uint64_t)v[k] << (o - 64);
            }
        }
        uint16_t* dst = (uint16_t*)(out + g.off[3]) + tile * g.n[3];
        for (int w = q; w < g.n[3]; w += 4) dst[w] = (uint16_t)((w < 4 ? lo >> (16 * w) : hi >> (16 * (w - 4))) & 0xffff);
    }
}

constexpr int kMaxRingWords = 512;  // codes 32 + planes <= 192 + lsb 32 + gains <= 256 for L <= 512

// one wavefront per ring: record i = fields codes, planes, lsb, gains back to back (g.total bytes)
__global__ __launch_bounds__(64 * kWaves) void pack_rings_kernel(const int16_t* __restrict__ idx, long ld_idx,
                                                                 const uint8_t* __restrict__ gi, long ld_gi, long n,
                                                                 PackGeo g, uint8_t* __restrict__ out)
{
    __shared__ int16_t s_ix[kWaves][kMaxL];
    __shared__ uint8_t s_g[kWaves][kMaxL];
    __shared__ uint16_t s_w[kWaves][kMaxRingWords];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int W = g.n[0] + g.n[1] + g.n[2] + g.n[3];
    for (long ring = (long)blockIdx.x * kWaves + wv; ring < n; ring += (long)gridDim.x * kWaves) {
        for (int t = lane; t < g.L; t += 64) {
            s_ix[wv][t] = idx[ring * ld_idx + t];
            s_g[wv][t] = gi[ring * ld_gi + t];
        }
        wave_sync();
        ballot_fields(
            g, lane, [&](int t) { return s_ix[wv][t]; }, [&](int t) { return s_g[wv][t]; },
            [&](int f, int w, uint16_t v) { s_w[wv][g.off[f] + w] = v; });
        wave_sync();
        uint16_t* rec = (uint16_t*)(out + ring * g.total);
        for (int w = lane; w < W; w += 64) rec[w] = s_w[wv][w];
        wave_sync();
    }
}

bool fmt_ok(int fmt_K, int frac, int h, int sub)
{
    return fmt_K >= 1 && fmt_K <= 8 && frac >= 0 && frac <= 2 && h >= 0 && h <= 8 && sub > 0;
}

}  // namespace

extern "C" long ltq_slice_bytes(int R, int K, int fmt_K, int frac, int h, int sub)
{
    if (R < 0 || K < 0 || R % 16 || K % 16 || !fmt_ok(fmt_K, frac, h, sub) || 256 % sub) return -1;
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
    if (g.n[0] + g.n[1] + g.n[2] + g.n[3] > kMaxTileWords) return -1;
    const long kbs = K / 16, spr = (kbs + kStrip - 1) / kStrip;
    const int vec = ((uintptr_t)idx % 16 == 0) && ((uintptr_t)gi % 16 == 0) && ld_idx % 8 == 0 && ld_gi % 16 == 0;
    if (sub >= 16) {  // 256 % sub == 0: at most one sub-block start per tile row
        const long grid = ((long)(R / 16) * spr + 3) / 4;
        if (grid > 0x7fffffffL) return -1;
        return ltq::timed_launch(ltq::kernel_timing, pack_quads_kernel, dim3((unsigned)grid), dim3(256), 0,
                                 (hipStream_t)stream, idx, ld_idx, gi, ld_gi, R, K, g, vec, out);
    }
    const long grid = (long)(R / 16) * spr;
    if (grid > 0x7fffffffL) return -1;
    const size_t stage = (size_t)kStrip * (g.n[0] + g.n[1] + g.n[2] + g.n[3]) * sizeof(uint16_t);  // <= 8 KB
    return ltq::timed_launch(ltq::kernel_timing, pack_strip_kernel, dim3((unsigned)grid), dim3(256), (uint32_t)stage,
                             (hipStream_t)stream, idx, ld_idx, gi, ld_gi, R, K, g, vec, out);
}

extern "C" long ltq_ring_bytes(int L, int fmt_K, int frac, int h, int sub)
{
    if (L <= 0 || L > kMaxL || L % 16 || !fmt_ok(fmt_K, frac, h, sub) || L % sub) return -1;
    return ring_geo(L, fmt_K, frac, h, sub).total;
}

extern "C" int ltq_pack_rings(const int16_t* idx, long ld_idx, const uint8_t* gi, long ld_gi, long n_rings, int L,
                              int fmt_K, int frac, int h, int sub, uint8_t* out, long out_bytes, void* stream)
{
    const long rb = ltq_ring_bytes(L, fmt_K, frac, h, sub);
    if (rb < 0 || n_rings < 0 || ld_idx < L || ld_gi < L || out_bytes < rb * n_rings) return -1;
    if (n_rings == 0) return 0;
    if (!idx || !gi || !out) return -1;
    const PackGeo g = ring_geo(L, fmt_K, frac, h, sub);
    if (g.n[0] + g.n[1] + g.n[2] + g.n[3] > kMaxRingWords) return -1;
    long grid = (n_rings + kWaves - 1) / kWaves;
    if (grid > 65536) grid = 65536;
    return ltq::timed_launch(ltq::kernel_timing, pack_rings_kernel, dim3((unsigned)grid), dim3(64 * kWaves), 0,
                             (hipStream_t)stream, idx, ld_idx, gi, ld_gi, n_rings, g, out);
}

// ---- decoding (src/ltq_file.py:119-147, the spec decoder) ------------------------------------------------
// One wavefront per tile; lane l decodes positions 4 l .. 4 l + 3. The code bits give the tail-biting state of
// every position (s_t = sum_j c_((t - j) mod 256) 2^j, j < 10), the state its label (bit 0 | parities of
// (s >> 1) & mask_i), the lsb stream and the planes the level u, the gain stream the gain index of the sub-block:
// value = gain[g] * lut[label * U + u] (the product the quantizer rounds its reconstruction with).
namespace {

__global__ __launch_bounds__(64 * kWaves) void unpack_kernel(const uint8_t* __restrict__ data, int R, int Kc, PackGeo g,
                                                             int m0, int m1, int m2, int m3, int nm,
                                                             const float* __restrict__ lut,
                                                             const float* __restrict__ gains, float* __restrict__ out,
                                                             long ld_out)
{
    constexpr int kMaxWords = 16 + 16 * 6 + 16 + 16;  // codes, planes (K <= 8), lsb, gains (h <= 8, sub >= 16)
    __shared__ uint16_t s_w[kWaves][kMaxWords];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int kbs = Kc / 16;
    const long T = (long)(R / 16) * kbs;
    const int W = g.n[0] + g.n[1] + g.n[2] + g.n[3];
    const int U = g.U;
    for (long tile = (long)blockIdx.x * kWaves + wv; tile < T; tile += (long)gridDim.x * kWaves) {
        for (int w = lane; w < W; w += 64) {
            int reg, wr;
            word_region(g, w, reg, wr);
            s_w[wv][w] = *(const uint16_t*)(data + g.off[reg] + 2 * (tile * g.n[reg] + wr));
        }
        wave_sync();
        const uint16_t* cw = s_w[wv];
        const uint16_t* pw = cw + g.n[0];
        const uint16_t* lw = pw + g.n[1];
        const uint16_t* gw = lw + g.n[2];
        auto bit = [](const uint16_t* ws, int i) -> uint32_t { return ((uint32_t)ws[i >> 4] >> (i & 15)) & 1u; };
        const long rg = tile / kbs, kb = tile - rg * kbs;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int t = 4 * lane + i;
            uint32_t s = 0;
#pragma unroll
            for (int j = 0; j < 10; j++) s |= bit(cw, (t - j) & 255) << j;
            const uint32_t sh = s >> 1;
            uint32_t lb = (s & 1u) | ((uint32_t)(__builtin_popcount(sh & (uint32_t)m0) & 1) << 1);
            if (nm > 1) lb |= (uint32_t)(__builtin_popcount(sh & (uint32_t)m1) & 1) << 2;
            if (nm > 2) lb |= (uint32_t)(__builtin_popcount(sh & (uint32_t)m2) & 1) << 3;
            if (nm > 3) lb |= (uint32_t)(__builtin_popcount(sh & (uint32_t)m3) & 1) << 4;
            uint32_t u = 0;
            if (g.K > 1) {
                if (g.frac == 0) {
                    u = bit(lw, t);
                } else if (g.frac == 1) {
                    u = bit(lw, t >> 1);
                } else {  // three bits per quad, the fourth makes the quad's sum even
                    const int q3 = 3 * (t >> 2), r = t & 3;
                    u = r < 3 ? bit(lw, q3 + r) : (bit(lw, q3) ^ bit(lw, q3 + 1) ^ bit(lw, q3 + 2));
                }
                for (int p = 1; p < g.K - 1; p++) u |= bit(pw + (p - 1) * 16, t) << p;
            }
            float gain = 1.0f;
            if (g.h) {
                const int jb = (t / g.sub) * g.h;
                uint32_t gi = 0;
                for (int k = 0; k < g.h; k++) gi |= bit(gw, jb + k) << k;
                gain = gains[gi];
            }
            out[(rg * 16 + (t >> 4)) * ld_out + kb * 16 + (t & 15)] = gain * lut[lb * U + u];
        }
        wave_sync();
    }
}

}  // namespace

extern "C" int ltq_unpack_slice(const uint8_t* data, long data_bytes, int R, int K, int fmt_K, int frac, int h, int sub,
                                int m0, int m1, int m2, int m3, int n_masks, const float* lut, const float* gains,
                                float* out, long ld_out, void* stream)
{
    const long need = ltq_slice_bytes(R, K, fmt_K, frac, h, sub);
    if (need < 0 || data_bytes < need || ld_out < K || n_masks < 1 || n_masks > 4 || sub < 16 || fmt_K > 8)
        return -1;
    if (R == 0 || K == 0) return 0;
    if (!data || !lut || (h && !gains) || !out) return -1;
    const PackGeo g = pack_geo(R, K, fmt_K, frac, h, sub);
    const long T = (long)(R / 16) * (K / 16);
    long grid = (T + kWaves - 1) / kWaves;
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)grid), dim3(64 * kWaves), 0, (hipStream_t)stream, data, R, K, g, m0,
                       m1, m2, m3, n_masks, lut, gains, out, ld_out);
    return (int)hipGetLastError();
}
