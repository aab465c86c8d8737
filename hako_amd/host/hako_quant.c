/*
 * hako_quant.c — the reference's quant.h surface (src/quant.h:26-46) over the
 * hako_gpu C ABI, plus the layer's shared host plumbing (device bring-up,
 * staging buffers, failure reporting).
 */
#include "hako_quant.h"
#include "hako_host.h"
#include "hako_mlf2.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

_Static_assert(sizeof(block_q4_K) == 144, "block_q4_K is 144 bytes");
_Static_assert(sizeof(block_q6_K) == 210, "block_q6_K is 210 bytes");
_Static_assert(sizeof(mlf2_header) == 128, "mlf2_header is 128 bytes");
_Static_assert(sizeof(mlf2_tensor) == 104, "mlf2_tensor is 104 bytes");

static pthread_mutex_t g_mu = PTHREAD_MUTEX_INITIALIZER;
static int g_ready = 0;
static void *g_slot[HK_NSLOTS];
static size_t g_slot_bytes[HK_NSLOTS];

void hk_lock(void) { pthread_mutex_lock(&g_mu); }
void hk_unlock(void) { pthread_mutex_unlock(&g_mu); }

int hk_ensure_device(void) {
	if (g_ready) return 0;
	const char *env = getenv("HAKO_DEVICE");
	int dev = env ? atoi(env) : 0;
	int rc = hako_gpu_init(dev);
	if (rc == 0) g_ready = 1;
	return rc;
}

void *hk_stage(int slot, size_t bytes) {
	if (slot < 0 || slot >= HK_NSLOTS) return NULL;
	if (g_slot_bytes[slot] < bytes) {
		if (g_slot[slot]) {
			hako_gpu_sync();
			hako_gpu_free(g_slot[slot]);
		}
		g_slot[slot] = NULL;
		g_slot_bytes[slot] = 0;
		size_t want = bytes < 4096 ? 4096 : bytes;
		if (hako_gpu_malloc(&g_slot[slot], want) != 0) return NULL;
		g_slot_bytes[slot] = want;
	}
	return g_slot[slot];
}

const void *hk_dev_view(const void *p, size_t bytes, size_t align, int slot) {
	if (bytes == 0) bytes = 1;
	const unsigned char *d0 = hako_gpu_mirror_lookup(p);
	const unsigned char *d1 = hako_gpu_mirror_lookup((const unsigned char *)p + bytes - 1);
	if (d0 && d1 && (size_t)(d1 - d0) == bytes - 1 && ((uintptr_t)d0 % align) == 0) return d0;
	void *s = hk_stage(slot, bytes);
	if (!s || hako_gpu_memcpy_h2d(s, p, bytes) != 0) return NULL;
	return s;
}

void hk_die(const char *what) {
	fprintf(stderr, "hako: %s failed: %s\n", what, hako_gpu_last_error());
	fflush(stderr);
	abort();
}

size_t hk_row_nbytes(int type, int n_in) {
	switch (type) {
	case MLF2_TYPE_F32:  return (size_t)n_in * 4;
	case MLF2_TYPE_F16:  return (size_t)n_in * 2;
	case MLF2_TYPE_Q4_K: return (size_t)(n_in / QK_K) * 144;
	case MLF2_TYPE_Q6_K: return (size_t)(n_in / QK_K) * 210;
	default:             return 0;
	}
}

/* IEEE binary16 -> binary32 by bit manipulation (reference src/quant.c:31-54):
 * subnormal inputs are renormalised, inf/nan keep their payload. */
float f16_to_f32(uint16_t h) {
	uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu, b;
	if (e == 0x1Fu) {
		b = sign | 0x7F800000u | (f << 13);
	} else if (e) {
		b = sign | ((e + 112u) << 23) | (f << 13);
	} else if (!f) {
		b = sign;
	} else {
		uint32_t ex = 113u;
		while (!(f & 0x400u)) { f <<= 1; ex--; }
		b = sign | (ex << 23) | ((f & 0x3FFu) << 13);
	}
	float r;
	memcpy(&r, &b, 4);
	return r;
}

/* Device dequant of `nelem` values of `type` at host address src into out. */
static int dequant_dev(int type, const void *src, float *out, int64_t nelem) {
	size_t in_bytes = type == MLF2_TYPE_F16 ? (size_t)nelem * 2 : hk_row_nbytes(type, (int)nelem);
	size_t align = type == MLF2_TYPE_Q4_K ? 16 : 2;
	int rc = hk_ensure_device();
	if (rc) return rc;
	const void *d = hk_dev_view(src, in_bytes, align, HK_SLOT_W);
	float *o = hk_stage(HK_SLOT_OUT, (size_t)nelem * 4);
	if (!d || !o) return -1;
	rc = hako_gpu_dequant(type, d, o, nelem);
	if (!rc) rc = hako_gpu_memcpy_d2h(out, o, (size_t)nelem * 4);
	return rc;
}

static void dequant_or_die(int type, const void *blocks, float *out, int64_t nelem, const char *what) {
	if (nelem <= 0) return;
	hk_lock();
	int rc = dequant_dev(type, blocks, out, nelem);
	hk_unlock();
	if (rc) hk_die(what);
}

void dequant_q4_K(const void *blocks, float *out, int nelem) {
	dequant_or_die(MLF2_TYPE_Q4_K, blocks, out, nelem, "dequant_q4_K");
}

void dequant_q6_K(const void *blocks, float *out, int nelem) {
	dequant_or_die(MLF2_TYPE_Q6_K, blocks, out, nelem, "dequant_q6_K");
}

void dequantize_row_q4_K(const void *blocks, float *out, int64_t nelem) {
	dequant_or_die(MLF2_TYPE_Q4_K, blocks, out, nelem, "dequantize_row_q4_K");
}

void dequantize_row_q6_K(const void *blocks, float *out, int64_t nelem) {
	dequant_or_die(MLF2_TYPE_Q6_K, blocks, out, nelem, "dequantize_row_q6_K");
}

int dequant_tensor(int type, const void *src, float *out, int nelem) {
	switch (type) {
	case MLF2_TYPE_F32:
		memcpy(out, src, (size_t)nelem * sizeof(float));   /* a view, no arithmetic */
		return 0;
	case MLF2_TYPE_F16:
	case MLF2_TYPE_Q4_K:
	case MLF2_TYPE_Q6_K: {
		if (nelem <= 0) return 0;
		hk_lock();
		int rc = dequant_dev(type, src, out, nelem);
		hk_unlock();
		if (rc) fprintf(stderr, "hako: dequant_tensor failed: %s\n", hako_gpu_last_error());
		return rc ? -1 : 0;
	}
	default:
		return -1;
	}
}

void quantize_row_q8_32(const float *x, int n, int8_t *xq, float *xs) {
	if (n <= 0) return;
	hk_lock();
	int rc = hk_ensure_device();
	if (!rc) {
		float *dx = hk_stage(HK_SLOT_X, (size_t)n * 4);
		int8_t *dq = hk_stage(HK_SLOT_XQ, (size_t)n);
		float *ds = hk_stage(HK_SLOT_XS, (size_t)(n / 32) * 4);
		rc = (!dx || !dq || !ds) ? -1 : hako_gpu_memcpy_h2d(dx, x, (size_t)n * 4);
		if (!rc) rc = hako_gpu_quantize_q8_32(dx, 1, n, dq, ds);
		if (!rc) rc = hako_gpu_memcpy_d2h(xq, dq, (size_t)n);
		if (!rc) rc = hako_gpu_memcpy_d2h(xs, ds, (size_t)(n / 32) * 4);
	}
	hk_unlock();
	if (rc) hk_die("quantize_row_q8_32");
}

float q4k_vec_dot(const void *w_row, int n_in, const int8_t *xq, const float *xs) {
	float r = 0.0f;
	hk_lock();
	int rc = hk_ensure_device();
	if (!rc) {
		const void *dw = hk_dev_view(w_row, hk_row_nbytes(MLF2_TYPE_Q4_K, n_in), 16, HK_SLOT_W);
		int8_t *dq = hk_stage(HK_SLOT_XQ, (size_t)n_in);
		float *ds = hk_stage(HK_SLOT_XS, (size_t)(n_in / 32) * 4);
		float *o = hk_stage(HK_SLOT_OUT, 4);
		rc = (!dw || !dq || !ds || !o) ? -1 : hako_gpu_memcpy_h2d(dq, xq, (size_t)n_in);
		if (!rc) rc = hako_gpu_memcpy_h2d(ds, xs, (size_t)(n_in / 32) * 4);
		if (!rc) rc = hako_gpu_q4k_gemv(o, dw, dq, ds, NULL, 1, n_in);
		if (!rc) rc = hako_gpu_memcpy_d2h(&r, o, 4);
	}
	hk_unlock();
	if (rc) hk_die("q4k_vec_dot");
	return r;
}
