/*
 * hako_quant.h — drop-in for the reference's quant.h (src/quant.h:9-46),
 * backed by the gfx950 kernels of libhako_gpu.
 *
 * Same names, signatures and argument meaning as the reference. Host pointers
 * in, host results out; a block pointer inside a model uploaded with
 * hako_model_upload (or by the first matmul on that model) is read from HBM
 * without a copy. A GPU failure inside a void function prints the library's
 * error and aborts, since the reference signature has no way to report it.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QK_K 256

/* Super-block layouts, byte for byte (reference src/quant.h:12-24). */
typedef struct {
	uint16_t d;
	uint16_t dmin;
	uint8_t  scales[12];
	uint8_t  qs[128];
} block_q4_K;                /* 144 bytes */

typedef struct {
	uint8_t  ql[128];
	uint8_t  qh[64];
	int8_t   scales[16];
	uint16_t d;
} block_q6_K;                /* 210 bytes */

/* reference src/quant.c:31-54 (host bit conversion; no device round trip). */
float f16_to_f32(uint16_t h);

/* reference src/quant.c:68-92 and :94-123; nelem % 256 == 0. */
void dequant_q4_K(const void *blocks, float *out, int nelem);
void dequant_q6_K(const void *blocks, float *out, int nelem);

/* reference src/quant.c:234-248: 0 on success, -1 on an unsupported type
 * (and, here, on a GPU failure). */
int dequant_tensor(int type, const void *src, float *out, int nelem);

/* reference src/quant.c:127-144; n % 32 == 0. */
void quantize_row_q8_32(const float *x, int n, int8_t *xq, float *xs);

/* reference src/quant.c:150-232; n_in % 256 == 0. */
float q4k_vec_dot(const void *w_row, int n_in, const int8_t *xq, const float *xs);

/* The ggml names of the two dequantizers, for callers written against ggml
 * (same arguments as dequant_q4_K / dequant_q6_K). */
void dequantize_row_q4_K(const void *blocks, float *out, int64_t nelem);
void dequantize_row_q6_K(const void *blocks, float *out, int64_t nelem);

#ifdef __cplusplus
}
#endif
