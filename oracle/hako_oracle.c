/*
 * hako_oracle.c — CPU restatement of hako's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, the smoke check and bench.py's
 * CPU baseline leg as the checker, never by product code.
 *
 * Built without -ffast-math and with -ffp-contract=off so that every rounding
 * below is the one written. Where the reference's compiled behaviour differs
 * from its source text (the q8 quantizer under -ffast-math, see
 * orc_quantize_row_q8_32) the compiled behaviour is what is restated, since
 * that is what the reference actually computes.
 */
#include "hako_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* quant.c:31-54. Restated from IEEE 754 binary16: zero, subnormal (value
 * mant·2^-24, renormalised into binary32), normal (rebias 15→127),
 * inf/nan (payload kept in the top mantissa bits). */
float orc_f16_to_f32(uint16_t h) {
	uint32_t sign = (uint32_t)(h >> 15) << 31;
	uint32_t e = (h >> 10) & 31u, f = h & 1023u, out;
	if (e == 31u) {
		out = sign | 0x7F800000u | (f << 13);
	} else if (e != 0u) {
		out = sign | ((e + 112u) << 23) | (f << 13);
	} else if (f == 0u) {
		out = sign;
	} else {
		/* f·2^-24 with f in [1,1023]: shift the leading one up to bit 10. */
		int shift = 0;
		while (!(f & 1024u)) { f <<= 1; shift++; }
		out = sign | ((uint32_t)(113 - shift) << 23) | ((f & 1023u) << 13);
	}
	float r;
	memcpy(&r, &out, 4);
	return r;
}

/* quant.c:57-66. The 12 scale bytes hold eight (scale, min) 6-bit pairs:
 * sub-blocks 0-3 in the low six bits of bytes 0-3 (scale) and 4-7 (min);
 * sub-blocks 4-7 take their low nibble from bytes 8-11 (scale: low nibble,
 * min: high nibble) and their top two bits from the spare top bits of
 * bytes 0-3 (scale) and 4-7 (min). */
void orc_scale_min_k4(int j, const uint8_t *sc, uint8_t *s, uint8_t *m) {
	if (j < 4) {
		*s = sc[j] & 0x3F;
		*m = sc[4 + j] & 0x3F;
	} else {
		uint8_t lo = sc[8 + (j - 4)];
		*s = (uint8_t)((lo & 0x0F) | ((sc[j - 4] >> 6) << 4));
		*m = (uint8_t)((lo >> 4) | ((sc[j] >> 6) << 4));
	}
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* quant.c:68-92. Weight e of a block (e = 64g + 32h + l, g the 64-group,
 * h ∈ {0,1}, l < 32) is the low (h=0) or high (h=1) nibble of qs[32g + l],
 * in sub-block 2g + h; value d·s·q − dmin·m. */
void orc_dequant_q4_K(const void *blocks, float *out, int64_t nelem) {
	const uint8_t *b = (const uint8_t *)blocks;
	for (int64_t blk = 0; blk < nelem / ORC_QK_K; blk++, b += ORC_Q4K_BYTES) {
		const float d = orc_f16_to_f32(rd16(b)), dmin = orc_f16_to_f32(rd16(b + 2));
		const uint8_t *sc = b + 4, *qs = b + 16;
		float *y = out + blk * ORC_QK_K;
		for (int e = 0; e < ORC_QK_K; e++) {
			int g = e >> 6, h = (e >> 5) & 1, l = e & 31;
			uint8_t s, m;
			orc_scale_min_k4(2 * g + h, sc, &s, &m);
			int q = h ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 0x0F);
			const float ds = d * (float)s, dm = dmin * (float)m;
			y[e] = ds * (float)q - dm;
		}
	}
}

/* quant.c:94-123. Weight e = 128n + 32k + l (n the 128-half, k ∈ [0,4),
 * l < 32): low nibble of ql[64n + l] (k=0), of ql[64n + 32 + l] (k=1), high
 * nibble of ql[64n + l] (k=2), of ql[64n + 32 + l] (k=3); bits 2k..2k+1 of
 * qh[32n + l] on top; minus 32; scaled by d·scales[8n + 2k + l/16]. */
void orc_dequant_q6_K(const void *blocks, float *out, int64_t nelem) {
	const uint8_t *b = (const uint8_t *)blocks;
	for (int64_t blk = 0; blk < nelem / ORC_QK_K; blk++, b += ORC_Q6K_BYTES) {
		const uint8_t *ql = b, *qh = b + 128;
		const int8_t *sc = (const int8_t *)(b + 192);
		const float d = orc_f16_to_f32(rd16(b + 208));
		float *y = out + blk * ORC_QK_K;
		for (int e = 0; e < ORC_QK_K; e++) {
			int n = e >> 7, k = (e >> 5) & 3, l = e & 31;
			uint8_t lbyte = ql[64 * n + (k & 1) * 32 + l];
			int lo = (k & 2) ? (lbyte >> 4) : (lbyte & 0x0F);
			int hi = (qh[32 * n + l] >> (2 * k)) & 3;
			int q = (lo | (hi << 4)) - 32;
			y[e] = d * (float)sc[8 * n + 2 * k + l / 16] * (float)q;
		}
	}
}

int orc_dequant_tensor(int type, const void *src, float *out, int64_t nelem) {
	switch (type) {
	case 0: memcpy(out, src, (size_t)nelem * 4); return 0;
	case 1: {
		const uint8_t *h = (const uint8_t *)src;
		for (int64_t i = 0; i < nelem; i++) out[i] = orc_f16_to_f32(rd16(h + 2 * i));
		return 0;
	}
	case 12: orc_dequant_q4_K(src, out, nelem); return 0;
	case 14: orc_dequant_q6_K(src, out, nelem); return 0;
	default: return -1;
	}
}

/* Flush a binary32 subnormal to (signed) zero: the reference executable and
 * library run with FTZ/DAZ set, because -ffast-math links gcc's crtfastmath
 * (Makefile:7-8), so subnormal operands read as zero and subnormal results
 * are written as zero. */
static float ftz(float v) { return (fabsf(v) < 1.17549435e-38f) ? copysignf(0.0f, v) : v; }

/* quant.c:127-144. The source text says scale = amax/127, inv = 1/scale;
 * under -ffast-math the reference compiles this to the two roundings
 * xs = amax·RN(1/127) and inv = RN(127/amax) (taken only when xs > 0), which
 * differ from the literal reading in a few percent of blocks. The conversion
 * is round-half-even into a 64-bit integer whose low 32 bits are clamped
 * to ±127; a ±inf or NaN product converts to the 64-bit "indefinite" value,
 * whose low 32 bits are 0. */
void orc_quantize_row_q8_32(const float *x, int n, int8_t *xq, float *xs) {
	const float rcp127 = 0x1.020408p-7f;   /* RN(1/127) = 0x3C010204 */
	for (int b = 0; b < n / 32; b++) {
		float amax = 0.0f;
		for (int l = 0; l < 32; l++) {
			float a = fabsf(ftz(x[32 * b + l]));
			if (a > amax) amax = a;
		}
		float scale = ftz(amax * rcp127);
		float inv = scale > 0.0f ? 127.0f / amax : 0.0f;
		xs[b] = scale;
		for (int l = 0; l < 32; l++) {
			float p = ftz(ftz(x[32 * b + l]) * inv);
			long long v;
			if (!isfinite(p)) {
				v = 0;
			} else {
				v = (long long)nearbyintf(p);   /* default mode: half-even */
			}
			int v32 = (int)(uint32_t)(unsigned long long)v;
			if (v32 > 127) v32 = 127;
			if (v32 < -127) v32 = -127;
			xq[32 * b + l] = (int8_t)v32;
		}
	}
}

/* Per-sub-block integer sums, restated from the scalar kernel
 * (quant.c:214-220): in super-block i, 64-group g, the 32 bytes qs[32g..]
 * give sub-block 2g (low nibbles, activations xq[256i + 64g + l]) and
 * sub-block 2g+1 (high nibbles, activations xq[256i + 64g + 32 + l]). */
void orc_q4k_isums(const void *w_row, int n_in, const int8_t *xq,
                   int32_t *iqx, int32_t *ix) {
	const uint8_t *b = (const uint8_t *)w_row;
	for (int i = 0; i < n_in / ORC_QK_K; i++, b += ORC_Q4K_BYTES) {
		const uint8_t *qs = b + 16;
		for (int g = 0; g < 4; g++) {
			int32_t a = 0, ax = 0, c = 0, cx = 0;
			const int8_t *xa = xq + ORC_QK_K * i + 64 * g, *xb = xa + 32;
			for (int l = 0; l < 32; l++) {
				a += (qs[32 * g + l] & 0x0F) * xa[l]; ax += xa[l];
				c += (qs[32 * g + l] >> 4) * xb[l];   cx += xb[l];
			}
			int sb = 8 * i + 2 * g;
			iqx[sb] = a; ix[sb] = ax; iqx[sb + 1] = c; ix[sb + 1] = cx;
		}
	}
}

/* quant.c:222-225: acc += xs[sb]·(d·s·iqx − dmin·m·ix), sb in order. */
float orc_q4k_vec_dot(const void *w_row, int n_in, const int8_t *xq, const float *xs) {
	const uint8_t *b = (const uint8_t *)w_row;
	int nsb = n_in / 32;
	int32_t *iqx = malloc((size_t)nsb * 8), *ix = iqx + nsb;
	orc_q4k_isums(w_row, n_in, xq, iqx, ix);
	float acc = 0.0f;
	for (int sb = 0; sb < nsb; sb++) {
		const uint8_t *blk = b + (size_t)(sb / 8) * ORC_Q4K_BYTES;
		float d = orc_f16_to_f32(rd16(blk)), dmin = orc_f16_to_f32(rd16(blk + 2));
		uint8_t s, m;
		orc_scale_min_k4(sb % 8, blk + 4, &s, &m);
		float t1 = d * (float)s * (float)iqx[sb];
		float t2 = dmin * (float)m * (float)ix[sb];
		acc += xs[sb] * (t1 - t2);
	}
	free(iqx);
	return acc;
}

double orc_q4k_vec_dot_f64(const void *w_row, int n_in, const int8_t *xq, const float *xs) {
	const uint8_t *b = (const uint8_t *)w_row;
	int nsb = n_in / 32;
	int32_t *iqx = malloc((size_t)nsb * 8), *ix = iqx + nsb;
	orc_q4k_isums(w_row, n_in, xq, iqx, ix);
	double acc = 0.0;
	for (int sb = 0; sb < nsb; sb++) {
		const uint8_t *blk = b + (size_t)(sb / 8) * ORC_Q4K_BYTES;
		double d = orc_f16_to_f32(rd16(blk)), dmin = orc_f16_to_f32(rd16(blk + 2));
		uint8_t s, m;
		orc_scale_min_k4(sb % 8, blk + 4, &s, &m);
		acc += (double)xs[sb] * (d * s * iqx[sb] - dmin * m * ix[sb]);
	}
	free(iqx);
	return acc;
}

size_t orc_row_nbytes(int type, int n_in) {
	switch (type) {
	case 0:  return (size_t)n_in * 4;
	case 1:  return (size_t)n_in * 2;
	case 12: return (size_t)(n_in / ORC_QK_K) * ORC_Q4K_BYTES;
	case 14: return (size_t)(n_in / ORC_QK_K) * ORC_Q6K_BYTES;
	default: return 0;
	}
}

typedef struct {
	float *out; const float *x; const uint8_t *w; const float *bias;
	const int8_t *xq; const float *xs;
	int type, n_in, f64, r0, r1; size_t rb;
} orc_job;

/* nn.c:70-97 for one contiguous row range. */
static void *orc_rows(void *arg) {
	orc_job *j = (orc_job *)arg;
	float *row = (j->type == 12) ? NULL : malloc((size_t)j->n_in * 4);
	for (int r = j->r0; r < j->r1; r++) {
		const uint8_t *wr = j->w + (size_t)r * j->rb;
		float acc;
		if (j->type == 12) {
			acc = j->f64 ? (float)orc_q4k_vec_dot_f64(wr, j->n_in, j->xq, j->xs)
			             : orc_q4k_vec_dot(wr, j->n_in, j->xq, j->xs);
		} else {
			orc_dequant_tensor(j->type, wr, row, j->n_in);
			if (j->f64) {
				double a = 0.0;
				for (int i = 0; i < j->n_in; i++) a += (double)row[i] * (double)j->x[i];
				acc = (float)a;
			} else {
				float a = 0.0f;
				for (int i = 0; i < j->n_in; i++) a += row[i] * j->x[i];
				acc = a;
			}
		}
		j->out[r] = j->bias ? acc + j->bias[r] : acc;
	}
	free(row);
	return NULL;
}

int orc_matmul(float *out, const float *x, int type, const void *w,
               const float *bias, int n_out, int n_in, int f64, int nthreads) {
	size_t rb = orc_row_nbytes(type, n_in);
	if (rb == 0) return -1;
	int8_t *xq = NULL; float *xs = NULL;
	if (type == 12) {
		xq = malloc((size_t)n_in);
		xs = malloc((size_t)(n_in / 32) * 4);
		orc_quantize_row_q8_32(x, n_in, xq, xs);
	}
	if (nthreads < 1) nthreads = 1;
	if (nthreads > 64) nthreads = 64;
	if (n_out < nthreads) nthreads = 1;
	orc_job jobs[64];
	pthread_t th[64];
	int per = (n_out + nthreads - 1) / nthreads;
	for (int t = 0; t < nthreads; t++) {
		int r0 = t * per, r1 = r0 + per > n_out ? n_out : r0 + per;
		jobs[t] = (orc_job){ out, x, (const uint8_t *)w, bias, xq, xs, type, n_in, f64,
		                     r0 < n_out ? r0 : n_out, r1, rb };
	}
	for (int t = 1; t < nthreads; t++) pthread_create(&th[t], NULL, orc_rows, &jobs[t]);
	orc_rows(&jobs[0]);
	for (int t = 1; t < nthreads; t++) pthread_join(th[t], NULL);
	free(xq); free(xs);
	return 0;
}

int orc_matmul_batch(float *out, const float *x, int M, int type, const void *w,
                     const float *bias, int n_out, int n_in, int f64, int nthreads) {
	for (int t = 0; t < M; t++) {
		int rc = orc_matmul(out + (size_t)t * n_out, x + (size_t)t * n_in, type, w,
		                    bias, n_out, n_in, f64, nthreads);
		if (rc) return rc;
	}
	return 0;
}

int orc_argmax(const float *logits, int n) {
	int best = 0;
	for (int i = 1; i < n; i++) if (logits[i] > logits[best]) best = i;
	return best;
}
