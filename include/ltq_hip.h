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

/* tcq_viterbi without any caller workspace, for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the reference: its C ABI
 * takes bp / gsel / gcand / pbits from the caller. Same arguments, meaning and results as tcq_viterbi with those
 * four dropped; the decision words and gain-candidate choices live in a static device array of
 * tcq_viterbi_static_bytes() bytes (96 MiB) that every GPU running the library holds until the process ends
 * (enough for 300 TCQ275X2 tiles of 256 steps). Returns -2, before touching any device, when a call needs more
 * than that; -1 / HIP error codes as tcq_viterbi. The entry point allocates nothing. Calls on one GPU share its
 * array: calls that overlap on one GPU (different streams or host threads) race; calls in one stream do not.
 * Nothing in the array needs clearing between calls (every word is written before it is read). */
int tcq_viterbi_static(const float* x, const float* w, const float* tab, const float* gains, float* rec,
                       const int* init_st, int* end_st, const float* tab_hi, const float* gains_hi, int* best,
                       int* code, int* mid_st, int mid_t, int tail, int N, int T, int S, int U, int G, int Gfull,
                       int m, int sub, int U_hi, int mix, int m2, int m3, int m4, int nl, int ld, int rot, int pp,
                       void* stream);

/* Size in bytes of tcq_viterbi_static's per-device scratch array. Host-only. */
long tcq_viterbi_static_bytes(void);

/* Timing hook for benchmarks; no counterpart in the reference. Arms the calling host thread's next `launches`
 * Viterbi kernel launches (tcq_viterbi, tcq_viterbi_tb, tcq_viterbi_static): the first carries start_event, the
 * last stop_event (hipEvent_t created by the caller, either may be null). They are launched with
 * hipExtLaunchKernelGGL, which stamps the events with the dispatch's own start and end times, so no event
 * packet sits between two kernels. launches = 0 disarms. Returns 0, or -1 for launches < 0. Results are not
 * affected. */
int ltq_viterbi_timing(void* start_event, void* stop_event, int launches);

/* The same hook for the library's other kernels (no counterpart in the reference): the next `launches` launches
 * of ltq_fwht256_rows / ltq_fwht256_cols, ltq_row_scale, ltq_pack_slice / ltq_pack_rings and ltq_ldlq_err /
 * ltq_ldlq_update on the calling host thread carry start_event (first) and stop_event (last). Each of those
 * entry points launches one kernel. launches = 0 disarms. Returns 0, or -1 for launches < 0. */
int ltq_kernel_timing(void* start_event, void* stop_event, int launches);

/* LUT sub-block quantization of the diagonal profile: for S sub-blocks of 16 weights xs[S, 16] with weights
 * dh[S, 16], bucket b = clamp(rint(x * inv_step + half_b), 0, nb - 1) picks a row of 64 candidates of lut[nb, 64];
 * the first candidate with the lowest sum_j dh (xs - lut[b_j][c])^2 gives out[S, 16] = lut[b_j][c]. Same
 * signature, argument meaning and results as src/cuda/tcq_viterbi.cu:806-811 (bound at src/tcq_proto.py:530-532),
 * with the rounding of nvcc's default contraction written out (fma for the bucket argument and the sums).
 * S = 0 returns hipErrorInvalidConfiguration (9), the reference's zero-block launch error; S < 0 or nb < 1: -1. */
int lut_subs_quant(const float* xs, const float* dh, const float* lut, float* out, int S, float inv_step, float half_b,
                   int nb, void* stream);

/* Both passes of the two-pass tail-biting Viterbi in one launch: the tcq_viterbi calls of
 * src/tcq_proto.py:584-609 (tb_passes = 2, pass 1 with the same gain slots) fused, with identical results. The
 * arguments are those of the closing pass (tail, T, rot, code, ...), with mid_buf [N] in the place of init_st:
 * pass 1 (steps1 steps from rotation rot1, free start, no codes) leaves the state before its mid_t1 there and
 * each workgroup starts its closing pass from it. Same return codes as tcq_viterbi. No counterpart in the
 * reference, which launches the two passes separately. */
int tcq_viterbi_tb(const float* x, const float* w, const float* tab, const float* gains, float* rec, uint32_t* bp,
                   uint8_t* gsel, int* mid_buf, int* end_st, const float* tab_hi, const float* gains_hi,
                   uint8_t* gcand, int* best, int* code, int tail, int N, int T, int S, int U, int G, int Gfull, int m,
                   int sub, int U_hi, int mix, int m2, int m3, int m4, int nl, int ld, int rot, uint32_t* pbits, int pp,
                   int steps1, int rot1, int mid_t1, void* stream);

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

/* Decodes a packed row slice [R, K] (the bytes ltq_pack_slice writes) into unscaled values out[R, K] (row
 * stride ld_out): per position the tail-biting state from the code bits, its label from the masks m0 .. m3
 * (n_masks of them), the level from the lsb stream and bit planes, the gain index of its sub-block, and
 * value = gains[g] * lut[label * U + u]. Replaces the torch decoder src/ltq_file.py:119-147 (`decode_slice`). */
int ltq_unpack_slice(const uint8_t* data, long data_bytes, int R, int K, int fmt_K, int frac, int h, int sub, int m0,
                     int m1, int m2, int m3, int n_masks, const float* lut, const float* gains, float* out, long ld_out,
                     void* stream);

/* Bytes of one packed row ring of L positions (src/ltq_format.py:48-50, `tile_bytes(L)`, the ring's fp16 scale
 * excluded). L % 16 == 0, L <= 512, L % sub == 0; -1 otherwise. Host-only arithmetic. */
long ltq_ring_bytes(int L, int fmt_K, int frac, int h, int sub);

/* Packs n_rings rings of L positions, codes idx [n_rings, L] (int16 label * U + u, row stride ld_idx) and gain
 * indices gi (uint8, row stride ld_gi), into consecutive records of ltq_ring_bytes(...) bytes, each the fields
 * codes / planes / lsb / gains of src/ltq_format.py:104-124 (`pack_tile` with L instead of 256) back to back.
 * Serves the ring tables of src/ple_quant.py:36-67. */
int ltq_pack_rings(const int16_t* idx, long ld_idx, const uint8_t* gi, long ld_gi, long n_rings, int L, int fmt_K,
                   int frac, int h, int sub, uint8_t* out, long out_bytes, void* stream);

/* Row scale of a rotated weight matrix w [M, K] (K % 256 == 0, row stride ldw, 16-byte aligned):
 * rms of every 256-column block (clamped at 1e-10, times scale), d_row[M] = fp16-rounded geometric mean of
 * the row's block rms (clamped at 1e-8), e[M, K/256] (int8, row stride lde) = clamp(round(log2(rms / d_row)
 * / e_step), -2^(e_bits-1), 2^(e_bits-1) - 1) and d[M, K/256] (row stride ldd) = max(d_row * exp2_tab[e +
 * 2^(e_bits-1)], 1e-8). exp2_tab: device array of 2^e_bits floats, entry k = 2^(e_step (k - 2^(e_bits-1)))
 * rounded once to fp32 on the host (the table the .ltq decoder uses). Replaces the torch code
 * src/liqk_v2.py:938-946 (and the clamp of :959); its results are defined to the bit: fixed-order block sums
 * (per 4-element group left to right, then a lane butterfly over offsets 32..1), correctly rounded fp32 sqrt,
 * log / mean / exp and log2 in float64, round half to even. K <= 262144. */
int ltq_row_scale(const float* w, long M, long K, long ldw, float scale, float e_step, int e_bits,
                  const float* exp2_tab, float* d_row, int8_t* e, long lde, float* d, long ldd, void* stream);

/* First Viterbi input of a 256-column block: x[T, 256] tiles (t = 16 r + c) = wk[:, 0:16] * (1 / d[row])
 * (src/liqk_v2.py:955-958, the `w_sub_orig * inv_d` of sub-block 0). M % 16 == 0; d has row stride ldd. */
int ltq_ldlq_prep(const float* wk, long ldw, const float* d, long ldd, float* x, long M, void* stream);

/* LDLQ error feedback after sub-block ib (0..15) of a 256-column block (src/liqk_v2.py:957-967): G[:, 16ib..]
 * = rec tiles, err = (wk[:, s0:s1] - d * rec) @ uinv[s0:s1, s0:s1], wk[:, s1:256] -= err @ ublk[s0:s1, s1:256],
 * and, if xnext is not null and ib < 15, the next sub-block's Viterbi tiles xnext = wk[:, s1:s1+16] * (1 / d).
 * Both products are fma chains over k ascending from 0 (then wk - acc). wk, G: [M, 256] working copy /
 * reconstruction of the block; uinv: the block's inverse factor (row stride ldi); ublk: the block's factor
 * U[c0:c1, c0:c1] (row stride ldu). If code (the Viterbi's int32 codes [M/16, 256], gain index << 16 | level
 * index) is not null, the PACK fields of the sub-block are written as well: idx[:, s0:s1] = code & 0xFFFF (int16,
 * row stride ld_idx) and gi[:, s0:s1] = code >> 16 (uint8, row stride ld_gi), the torch scatter of
 * src/liqk_v2.py:919-921; idx and gi point at the block's first column. If fed is not null, fed[:, s0:s1] (row
 * stride ld_fed, pointing at the block's first column) receives wk[:, s0:s1] as the sub-block's Viterbi saw it.
 * Stacked matrices (rows_per_mat > 0, a multiple of 16 dividing M; 0 = one matrix): rows [m R, (m + 1) R) belong
 * to matrix m, whose factors are uinv + m * uinv_ms and ublk + m * ublk_ms (the MoE expert batch). */
int ltq_ldlq_sub(float* wk, long ldw, const float* rec, const float* d, long ldd, const float* uinv, long ldi,
                 const float* ublk, long ldu, int ib, float* G, long ldg, float* xnext, long M, const int* code,
                 int16_t* idx, long ld_idx, uint8_t* gi, long ld_gi, float* fed, long ld_fed, long rows_per_mat,
                 long uinv_ms, long ublk_ms, void* stream);

/* Error of a finished 256-column block (src/liqk_v2.py:972-978): what[:, 0:256] = d * G (the block's
 * reconstruction, if what is not null) and E = (wstart - d * G) @ uinv, stored transposed: et[j * ld_et + i]
 * = E[i][j] (et is [256, M]). Each E entry is the fma chain over k = 0..255 ascending from 0 (fp32 MFMA, whose
 * four-term steps are that chain). wstart, G: [M, 256] (row strides ldw, ldg); d: [M] (stride ldd); uinv:
 * [256, 256]. M % 16 == 0; every matrix pointer 16-byte aligned and every row stride a multiple of 4. Stacked
 * matrices: rows_per_mat > 0 (a multiple of 128 dividing M) gives rows [m R, (m + 1) R) the factor uinv + m *
 * uinv_ms (uinv_ms a multiple of 4); 0 = one matrix. */
int ltq_ldlq_err(const float* wstart, long ldw, const float* G, long ldg, const float* d, long ldd, const float* uinv,
                 long ldi, float* et, long ld_et, float* what, long ld_what, long M, long rows_per_mat, long uinv_ms,
                 void* stream);

/* Update of the columns right of a finished block (src/liqk_v2.py:979): w[:, 0:N] -= E @ u[0:256, 0:N] with E
 * given transposed (et [256, M], row stride ld_et), each product the fma chain over k = 0..255 ascending from 0
 * (fp32 MFMA), then w - acc. Replaces the reference's cuBLAS GEMM, whose order is not fixed. Optionally also the
 * next block's working copy wsub[:, 0:256] = the updated w[:, 0:256] and its first Viterbi tiles xnext [M/16, 256]
 * (t = 16 r + c) = w[:, 0:16] * (1 / dnext). M % 16 == 0, N % 128 == 0 (N >= 256 with wsub); et and u 16-byte
 * aligned with row strides a multiple of 4. Stacked matrices as ltq_ldlq_err: rows [m R, (m + 1) R) are updated
 * with u + m * u_ms. */
int ltq_ldlq_update(float* w, long ldw, const float* et, long ld_et, const float* u, long ldu, long M, long N,
                    float* wsub, long ld_wsub, float* xnext, const float* dnext, long ld_dnext, long rows_per_mat,
                    long u_ms, void* stream);

/* Input-covariance accumulation, the _CovAccumulator.add of src/liqk_v2.py:218-228 for bf16 (f16 = 0) or fp16
 * (f16 = 1) activations: H += X^T X for X [n, K] (element type 16-bit, row stride ldx >= K), fp32 accumulation
 * over the batch on the matrix cores, added into the fp64 running sum H [K, K] (row stride ldh). Only the
 * 128 x 128 tiles on and below the diagonal of H are updated; ltq_cov_finalize reads the lower triangle.
 * n == 0 is a no-op. The reference's fp32 path (torch GEMM) has no counterpart here. */
int ltq_cov_accumulate(const void* X, long n, int K, long ldx, int f16, double* H, long ldh, void* stream);

/* The get() of src/liqk_v2.py:230-231: out[i][j] (fp32, row stride ldo) = (float)(H[max(i,j)][min(i,j)] * inv_n)
 * with inv_n = 1.0 / max(count, 1) in fp64 (torch's device division of an fp64 tensor by an integer). */
int ltq_cov_finalize(const double* H, int K, long ldh, double inv_n, float* out, long ldo, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LTQ_HIP_H */
