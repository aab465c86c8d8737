/*
 * hako_oracle.h — CPU restatement of hako's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, the smoke check and bench.py's CPU
 * baseline leg may load this library, and only as the checker: no product code
 * links, loads or calls it, and it is never the thing measured.
 *
 * Every function restates one reference function (file:line relative to the
 * hako source tree) from its semantics, in this file's own code. How each one
 * is pinned (golden vectors from the compiled reference, closed forms, brute
 * force) is recorded in the tests that exercise it.
 */
#pragma once
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK_K 256
#define ORC_Q4K_BYTES 144   /* quant.h:12-17 */
#define ORC_Q6K_BYTES 210   /* quant.h:19-24 */

/* quant.c:31-54 — exact binary16 → binary32 (subnormals normalised). */
float orc_f16_to_f32(uint16_t h);

/* quant.c:57-66 — 6-bit scale/min of Q4_K sub-block j ∈ [0,8). */
void orc_scale_min_k4(int j, const uint8_t *sc, uint8_t *s, uint8_t *m);

/* quant.c:68-92 / 94-123 — dequantize nelem (multiple of 256) values. */
void orc_dequant_q4_K(const void *blocks, float *out, int64_t nelem);
void orc_dequant_q6_K(const void *blocks, float *out, int64_t nelem);

/* quant.c:234-248 — type dispatch (0 F32, 1 F16, 12 Q4_K, 14 Q6_K); -1 on
 * any other type. */
int orc_dequant_tensor(int type, const void *src, float *out, int64_t nelem);

/* quant.c:127-144 in the form the reference build compiles it to
 * (-O3 -ffast-math, Makefile:7-8): xs = amax·RN(1/127), inv = 127/amax when
 * xs > 0, xq = clamp(rint_even(x·inv), ±127), where a product that does not
 * convert (±inf or NaN, only possible when 127/amax overflows) yields 0. */
void orc_quantize_row_q8_32(const float *x, int n, int8_t *xq, float *xs);

/* Per 32-wide sub-block integer sums of q4k_vec_dot (quant.c:214-220) for one
 * row: iqx[sb] = Σ q·xq, ix[sb] = Σ xq, sb ∈ [0, n_in/32). */
void orc_q4k_isums(const void *w_row, int n_in, const int8_t *xq,
                   int32_t *iqx, int32_t *ix);

/* quant.c:150-232 with the fp32 fold of :222-225 applied in source order. */
float orc_q4k_vec_dot(const void *w_row, int n_in, const int8_t *xq, const float *xs);

/* The same dot, folded in double precision from the exact integer sums. */
double orc_q4k_vec_dot_f64(const void *w_row, int n_in, const int8_t *xq, const float *xs);

/* nn.c:179-210 — out[n_out] = W·x (+bias) for W of the given type, rows of
 * n_in elements (row-major, verbatim block bytes). Q4_K quantizes x with the
 * q8_32 scheme and uses the integer dot (nn.c:76-82, 191-198); every other
 * type dequantizes a row to fp32 and takes an fp32 dot with x (nn.c:84-95).
 * `f64` != 0 accumulates in double (a tighter yardstick than the reference's
 * own reassociated fp32 order). Rows are split over `nthreads` threads.
 * Returns 0, or -1 on an unsupported type. */
int orc_matmul(float *out, const float *x, int type, const void *w,
               const float *bias, int n_out, int n_in, int f64, int nthreads);

/* The same matmul over M activation rows (x is [M][n_in], out is [M][n_out]),
 * i.e. M independent calls of orc_matmul, as the reference runs a prompt
 * token by token (cli/main.c:56-60). */
int orc_matmul_batch(float *out, const float *x, int M, int type, const void *w,
                     const float *bias, int n_out, int n_in, int f64, int nthreads);

/* nn.c:45-53 — bytes in one row of n_in elements of `type`; 0 if unknown. */
size_t orc_row_nbytes(int type, int n_in);

/* sample.c:28-32 — greedy argmax, lowest index wins ties. */
int orc_argmax(const float *logits, int n);

#ifdef __cplusplus
}
#endif
