/*
 * hako_decode.c — a device decoder for a mapped MLF2 model.
 *
 * Resolves the tensors the reference's hakm_ctx_new resolves (src/model.c:
 * 30-57, names from the converter) in the model's directory, mirrors the data
 * section into HBM (verbatim, once) and hands the device addresses of every
 * tensor to hako_gpu_decoder_create. The caller then runs whole decode steps
 * on the device in place of hakm_forward (src/model.c:93-165).
 */
#include "hako_decode.h"
#include "hako_host.h"
#include "hako_nn.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static const mlf2_tensor *find_tensor(const hakm_model *m, const char *name) {
	for (uint32_t i = 0; i < m->h.n_tensors; i++)
		if (strncmp(m->tensors[i].name, name, MLF2_MAX_NAME) == 0) return &m->tensors[i];
	return NULL;
}

/* Device address of tensor `name` inside the model's mirror; NULL (and *rc
 * set) when the tensor is absent and `required`. */
static const void *dev_tensor(const hakm_model *m, const char *name, int required, int *type, int *rc) {
	const mlf2_tensor *t = find_tensor(m, name);
	if (!t) {
		if (required && !*rc) {
			fprintf(stderr, "hako: missing tensor %s\n", name);
			*rc = HAKO_GPU_EINVAL;
		}
		return NULL;
	}
	if (type) *type = (int)t->type;
	const void *d = hako_gpu_mirror_lookup(m->data + t->data_off);
	if (!d && !*rc) *rc = HAKO_GPU_ENOTFOUND;
	return d;
}

int hako_decoder_from_model(const hakm_model *m, int n_seq, int max_seq, hako_gpu_decoder **dec) {
	if (!m || !dec || !m->map) return HAKO_GPU_EINVAL;
	*dec = NULL;
	char why[256];
	if (hako_mlf2_check(m->map, m->map_size, why, sizeof why)) {
		fprintf(stderr, "hako: %s\n", why);
		return HAKO_GPU_EINVAL;
	}
	int rc = hako_model_upload(m);
	if (rc) return rc;
	const mlf2_header *h = &m->h;
	hako_gpu_block *blocks = calloc(h->n_layers ? h->n_layers : 1, sizeof *blocks);
	if (!blocks) return HAKO_GPU_ENOMEM;
	hako_gpu_model g;
	memset(&g, 0, sizeof g);
	g.n_layers = (int)h->n_layers;
	g.d_model = (int)h->d_model;
	g.n_heads = (int)h->n_heads;
	g.n_kv_heads = (int)h->n_kv_heads;
	g.head_dim = (int)h->head_dim;
	g.ffn_dim = (int)h->ffn_dim;
	g.vocab = (int)h->vocab;
	g.rope_theta = h->rope_theta;
	g.rms_eps = h->rms_eps;
	g.tok_embd = dev_tensor(m, "token_embd.weight", 1, &g.t_embd, &rc);
	g.out_norm = dev_tensor(m, "output_norm.weight", 1, NULL, &rc);
	if (h->flags & MLF2_FLAG_TIED_EMBED) {   /* reference src/model.c:33-38 */
		g.out_weight = g.tok_embd;
		g.t_out = g.t_embd;
	} else {
		g.out_weight = dev_tensor(m, "output.weight", 1, &g.t_out, &rc);
	}
	char nm[64];
	for (int l = 0; l < g.n_layers && !rc; l++) {
		hako_gpu_block *B = &blocks[l];
#define HK_T(field, type, suffix, req)                            \
	snprintf(nm, sizeof nm, "blk.%d." suffix, l);                 \
	B->field = dev_tensor(m, nm, req, type, &rc)
		HK_T(attn_norm, NULL, "attn_norm.weight", 1);
		HK_T(wq, &B->t_q, "attn_q.weight", 1);
		HK_T(wk, &B->t_k, "attn_k.weight", 1);
		HK_T(wv, &B->t_v, "attn_v.weight", 1);
		HK_T(wo, &B->t_o, "attn_output.weight", 1);
		HK_T(ffn_norm, NULL, "ffn_norm.weight", 1);
		HK_T(gate, &B->t_gate, "ffn_gate.weight", 1);
		HK_T(up, &B->t_up, "ffn_up.weight", 1);
		HK_T(down, &B->t_down, "ffn_down.weight", 1);
		HK_T(bq, NULL, "attn_q.bias", 0);   /* optional, as src/model.c:51-54 */
		HK_T(bk, NULL, "attn_k.bias", 0);
		HK_T(bv, NULL, "attn_v.bias", 0);
#undef HK_T
	}
	g.blocks = blocks;
	if (!rc) {
		hk_lock();
		rc = hk_ensure_device();
		hk_unlock();
	}
	if (!rc) rc = hako_gpu_decoder_create(&g, n_seq, max_seq, dec);
	free(blocks);
	/* the decoder reads the mirror in place: pinned until it is destroyed */
	if (!rc) rc = hk_model_pin(m, 1);
	if (!rc) {
		rc = hako_gpu_decoder_on_destroy(*dec, hk_model_unpin_map, (void *)m->map);
		if (rc) hk_model_pin(m, -1);
	}
	if (rc && *dec) {
		hako_gpu_decoder_destroy(*dec);
		*dec = NULL;
	}
	return rc;
}
