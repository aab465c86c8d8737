/*
 * hako_nn.c — the reference's nn.h surface (src/nn.h:6-29).
 *
 * matmul / deq_row run on the GPU: the model's whole data section is mirrored
 * into HBM once (verbatim, so tensor t sits at mirror + t->data_off, as it
 * sits at m->data + t->data_off in the mmap, src/loader.c:66-68), and each
 * call ships only the activation in and the result out. The elementwise
 * helpers are the reference's host-side formulas, restated.
 */
#include "hako_nn.h"
#include "hako_host.h"
#include "hako_quant.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

/* ── host elementwise helpers (reference src/nn.c:13-42) ── */

void rmsnorm(float *y, const float *x, const float *w, int n, float eps) {
	float ss = 0.0f;
	for (int i = 0; i < n; i++) ss += x[i] * x[i];
	const float inv = 1.0f / sqrtf(ss / (float)n + eps);
	for (int i = 0; i < n; i++) y[i] = x[i] * inv * w[i];
}

void softmax(float *x, int n) {
	float mx = x[0];
	for (int i = 1; i < n; i++) mx = x[i] > mx ? x[i] : mx;
	float sum = 0.0f;
	for (int i = 0; i < n; i++) {
		x[i] = expf(x[i] - mx);
		sum += x[i];
	}
	const float inv = 1.0f / sum;
	for (int i = 0; i < n; i++) x[i] *= inv;
}

float silu_f(float x) { return x / (1.0f + expf(-x)); }

/* NeoX rotation: element i pairs with i + head_dim/2, angle pos*theta^(-2i/hd). */
void rope_neox(float *vec, int head_dim, int pos, float theta) {
	const int half = head_dim / 2;
	for (int i = 0; i < half; i++) {
		const float freq = powf(theta, -((float)(2 * i) / (float)head_dim));
		const float ang = (float)pos * freq;
		const float c = cosf(ang), s = sinf(ang);
		const float a = vec[i], b = vec[i + half];
		vec[i] = a * c - b * s;
		vec[i + half] = a * s + b * c;
	}
}

/* ── model mirrors ──
 * One entry per mapped model: its data section lives in HBM for as long as
 * the entry does. A different file mapped at the same address is told apart
 * by its size, header and a sampled signature of its data, and replaces the
 * stale mirror; so does one mapped over part of a stale entry's range. */

typedef struct {
	const void *map;
	size_t map_size;
	const unsigned char *data;
	mlf2_header h;
	uint64_t sig;
	int pins;   /* live decoders reading this mirror (hako_decoder_from_model) */
} model_entry;

#define HK_MAX_MODELS 16
static model_entry g_models[HK_MAX_MODELS];
static int g_nmodels = 0;

static size_t data_extent(const hakm_model *m) {
	return (size_t)((const unsigned char *)m->map + m->map_size - m->data);
}

/* FNV-1a over 64 eight-byte samples spread across the data section. */
static uint64_t data_signature(const hakm_model *m) {
	const size_t n = data_extent(m);
	uint64_t hsh = 1469598103934665603ull;
	for (int k = 0; k < 64 && n >= 8; k++) {
		uint64_t v;
		memcpy(&v, m->data + (n - 8) / 63 * (size_t)k, 8);
		hsh = (hsh ^ v) * 1099511628211ull;
	}
	return hsh;
}

static int find_model(const hakm_model *m) {
	for (int i = 0; i < g_nmodels; i++)
		if (g_models[i].map == m->map) return i;
	return -1;
}

static void drop_model(int i) {
	hako_gpu_mirror_release(g_models[i].data);
	g_models[i] = g_models[--g_nmodels];
}

/* A pinned mirror is read by a live decoder: it is never dropped. */
static int refuse_pinned(int i, const char *why) {
	fprintf(stderr, "hako: model mirror at %p is read by %d live decoder(s): %s refused "
	        "(destroy the decoders first)\n", g_models[i].map, g_models[i].pins, why);
	return HAKO_GPU_EINVAL;
}

/* Lock held. */
static int upload_locked(const hakm_model *m) {
	if (!m->map || !m->data) return HAKO_GPU_EINVAL;
	int rc = hk_ensure_device();
	if (rc) return rc;
	const uint64_t sig = data_signature(m);
	int i = find_model(m);
	if (i >= 0) {
		model_entry *e = &g_models[i];
		if (e->map_size == m->map_size && e->data == m->data && e->sig == sig &&
		    memcmp(&e->h, &m->h, sizeof e->h) == 0)
			return 0;
		if (e->pins) return refuse_pinned(i, "replacing it with a different model at that address");
		drop_model(i);
	}
	/* an entry whose bytes overlap this live mapping belongs to a model
	 * unmapped since (two live mappings never overlap): stale, dropped */
	const unsigned char *lo = m->data, *hi = m->data + data_extent(m);
	for (int k = g_nmodels - 1; k >= 0; k--) {
		const unsigned char *elo = g_models[k].data;
		const unsigned char *ehi = (const unsigned char *)g_models[k].map + g_models[k].map_size;
		if (elo < hi && lo < ehi) {
			if (g_models[k].pins) return refuse_pinned(k, "a new mapping over its range");
			drop_model(k);
		}
	}
	if (g_nmodels == HK_MAX_MODELS) {   /* evict the oldest unpinned entry */
		int k = 0;
		while (k < g_nmodels && g_models[k].pins) k++;
		if (k == g_nmodels) {
			fprintf(stderr, "hako: %d model mirrors, all read by live decoders\n", g_nmodels);
			return HAKO_GPU_ENOMEM;
		}
		drop_model(k);
	}
	rc = hako_gpu_mirror_upload(m->data, data_extent(m), NULL);
	if (rc) return rc;
	g_models[g_nmodels++] = (model_entry){ m->map, m->map_size, m->data, m->h, sig, 0 };
	return 0;
}

int hako_model_upload(const hakm_model *m) {
	hk_lock();
	int rc = upload_locked(m);
	hk_unlock();
	return rc;
}

int hako_model_release(const hakm_model *m) {
	hk_lock();
	int i = find_model(m);
	int rc = i >= 0 ? 0 : HAKO_GPU_ENOTFOUND;
	if (i >= 0 && g_models[i].pins) rc = refuse_pinned(i, "release");
	else if (i >= 0) drop_model(i);
	hk_unlock();
	return rc;
}

int hk_model_pin(const hakm_model *m, int delta) {
	hk_lock();
	int i = find_model(m);
	if (i >= 0) g_models[i].pins += delta;
	hk_unlock();
	return i >= 0 ? 0 : HAKO_GPU_ENOTFOUND;
}

/* the decoder's destroy hook: arg is the map address of its model entry */
void hk_model_unpin_map(void *map) {
	hk_lock();
	for (int i = 0; i < g_nmodels; i++)
		if (g_models[i].map == map && g_models[i].pins > 0) {
			g_models[i].pins--;
			break;
		}
	hk_unlock();
}

/* Device address of `bytes` at host address p of model m: the model mirror
 * for a mapped model, a fresh staging copy for a hand-built one (whose
 * buffers the caller may rewrite between calls). Lock held. */
static const void *model_bytes(const hakm_model *m, const void *p, size_t bytes, size_t align, int slot,
                               int *rc) {
	if (m->map) {
		*rc = upload_locked(m);
		if (*rc) return NULL;
	}
	const void *d = m->map ? hk_dev_view(p, bytes, align, slot) : NULL;
	if (!d) {
		void *s = hk_stage(slot, bytes ? bytes : 1);
		if (!s || hako_gpu_memcpy_h2d(s, p, bytes) != 0) {
			*rc = -1;
			return NULL;
		}
		d = s;
	}
	*rc = 0;
	return d;
}

void matmul(float *out, const float *x, const hakm_model *m, const mlf2_tensor *w, const float *bias,
            int n_out, int n_in) {
	hk_lock();
	int rc = hk_ensure_device();
	if (!rc) {
		const int type = (int)w->type;
		const size_t rb = hk_row_nbytes(type, n_in);
		const void *dw = rb ? model_bytes(m, m->data + w->data_off, rb * (size_t)n_out, 16, HK_SLOT_W, &rc)
		                    : NULL;
		if (!rb) rc = HAKO_GPU_ETYPE;
		const float *db = NULL;
		if (!rc && bias) db = model_bytes(m, bias, (size_t)n_out * 4, 4, HK_SLOT_BIAS, &rc);
		float *dx = rc ? NULL : hk_stage(HK_SLOT_X, (size_t)n_in * 4);
		float *dout = rc ? NULL : hk_stage(HK_SLOT_OUT, (size_t)n_out * 4);
		if (!rc && (!dx || !dout)) rc = -1;
		if (!rc) rc = hako_gpu_memcpy_h2d(dx, x, (size_t)n_in * 4);
		if (!rc) rc = hako_gpu_matmul(dout, dx, type, dw, db, n_out, n_in);
		if (!rc) rc = hako_gpu_memcpy_d2h(out, dout, (size_t)n_out * 4);
	}
	hk_unlock();
	if (rc) hk_die("matmul");
}

void deq_row(const hakm_model *m, const mlf2_tensor *w, int r, int n_in, float *out) {
	const int type = (int)w->type;
	const size_t rb = hk_row_nbytes(type, n_in);
	const unsigned char *src = m->data + w->data_off + (size_t)r * rb;
	if (type == MLF2_TYPE_F32) {
		memcpy(out, src, rb);   /* a view, no arithmetic (reference src/quant.c:236-238) */
		return;
	}
	hk_lock();
	int rc = hk_ensure_device();
	if (!rc && !rb) rc = HAKO_GPU_ETYPE;
	if (!rc) {
		const void *d = model_bytes(m, src, rb, type == MLF2_TYPE_Q4_K ? 16 : 2, HK_SLOT_W, &rc);
		float *o = rc ? NULL : hk_stage(HK_SLOT_OUT, (size_t)n_in * 4);
		if (!rc && !o) rc = -1;
		if (!rc) rc = hako_gpu_dequant(type, d, o, n_in);
		if (!rc) rc = hako_gpu_memcpy_d2h(out, o, (size_t)n_in * 4);
	}
	hk_unlock();
	if (rc) hk_die("deq_row");
}
