/* C ABI of libltq_hip.so: the MI355X (gfx950) kernels of the LTQ TCQ quantizer.
 *
 * Plain pointers and sizes only. Every device pointer is a HIP device address; `stream` is a hipStream_t
 * (NULL = the default stream). Return codes follow the reference C ABI: 0 = launched, -1 = rejected
 * arguments (nothing launched), any other value = the HIP error code of the launch. Calls are asynchronous
 * on `stream`; no entry point allocates or synchronizes.
 */
#ifndef LTQ_HIP_H
#define LTQ_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Joint (gain, trellis) Viterbi over N tiles of T steps.
 * Replaces src/cuda/tcq_viterbi.cu:743-766 (`tcq_viterbi`), bound by ctypes at src/tcq_proto.py:529
 * (15 pointers, 18 ints, pbits, pp, stream) and driven by src/tcq_proto.py:567-657.
 * Same arguments, shapes and validation as the reference. bp [N, T, G, S/32] and pbits (pp = 1:
 * [N, T/2, G, S/32], pp >= 2: [N, T/4, G, 9, S/32]) are caller-allocated scratch that this implementation
 * fills with its own decision-word layout; gsel is not written. Limits beyond the reference's: S is 256 or
 * 1024, G is 1, 2, 3, 4 or 8, pp = 1 needs T % 4 == 0, S = 256 needs T >= 8. */
int tcq_viterbi(const float* x, const float* w, const float* tab, const float* gains, float* rec, uint32_t* bp,
                uint8_t* gsel, const int* init_st, int* end_st, const float* tab_hi, const float* gains_hi,
                uint8_t* gcand, int* best, int* code, int* mid_st, int mid_t, int tail, int N, int T, int S, int U,
                int G, int Gfull, int m, int sub, int U_hi, int mix, int m2, int m3, int m4, int nl, int ld, int rot,
                uint32_t* pbits, int pp, void* stream);

/* Normalized block FWHT-256 along rows: y[r, :] = FWHT256 of (x[r, :] op s), fp32 out.
 * Replaces the torch function src/iqk_format.py:153-170 (`fwht_inplace`) as called with a fused scale at
 * src/liqk_v2.py:438-439 (smode 1: x / s[col], smode 2: x * s[col], 0: none).
 * dtype of x: 0 fp32, 1 bf16, 2 fp16 (widened exactly). cols % 256 == 0; ldx, ldy (elements) multiples
 * of 4; x 16-byte (fp32) or 8-byte (16-bit) aligned, y and s 16-byte aligned. In place allowed for fp32. */
int ltq_fwht256_rows(const void* x, int dtype, float* y, long rows, long cols, long ldx, long ldy, const float* s,
                     int smode, void* stream);

/* Normalized FWHT-256 along columns (256-row blocks), scale s indexed by row applied first.
 * Replaces fwht_inplace(X.T * s).T (src/liqk_v2.py:440) and _fwht_rows (src/liqk_v2.py:1023-1026);
 * bit-identical to them. rows % 256 == 0. In place allowed. */
int ltq_fwht256_cols(const float* x, float* y, long rows, long cols, long ldx, long ldy, const float* s, int smode,
                     void* stream);

/* Bytes of a packed row slice [R, K] of format (fmt_K, frac, h, sub): four regions, each on a 64-byte
 * boundary (src/ltq_file.py:67-96). Host-only arithmetic; -1 for an invalid shape. */
long ltq_slice_bytes(int R, int K, int fmt_K, int frac, int h, int sub);

/* Packs codes idx [R, K] (int16 label * U + u, row stride ld_idx) and gain indices gi [R, K] (uint8, row
 * stride ld_gi) into the .ltq tile regions codes / planes / lsb / gains. Replaces the torch function
 * src/ltq_file.py:79-96 (`pack_slice`, which returns the same bytes on the host) and the per-tile layout of
 * src/ltq_format.py:104-124 (`pack_tile`). R, K multiples of 16; out holds ltq_slice_bytes(...) bytes, every
 * one of which is written (region gaps are zero). */
int ltq_pack_slice(const int16_t* idx, long ld_idx, const uint8_t* gi, long ld_gi, int R, int K, int fmt_K, int frac,
                   int h, int sub, uint8_t* out, long out_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LTQ_HIP_H */
