/*
 * hako_mlf2.c — structural check of an MLF2 image before any of it reaches
 * the GPU.
 *
 * The reference's loader (src/loader.c:12-52) checks the magic, the version
 * and that the directory and section offsets lie inside the file; it trusts
 * everything else, and hakm_ctx_new (src/model.c:30-57) only checks that the
 * tensors it needs exist. A verbatim upload plus device kernels that read
 * rows of n_in/256 blocks need more: every tensor's bytes inside the data
 * section and consistent with its type and dims, the model tensors of the
 * header's shape, the tokenizer blob inside its section. The layout rules
 * are the converter's (tools/gguf2mlf.py:138-190): 104-byte directory
 * entries, 32-byte aligned data section and tensor offsets, dims padded with
 * zeros, names shorter than 48 bytes.
 */
#include "hako_mlf2.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#define QK 256u

static int fail(char *msg, size_t len, const char *fmt, ...) {
	if (msg && len) {
		va_list ap;
		va_start(ap, fmt);
		vsnprintf(msg, len, fmt, ap);
		va_end(ap);
	}
	return -1;
}

/* Bytes of n elements of `type` (0 when n does not fill whole blocks). */
static uint64_t type_bytes(uint32_t type, uint64_t n) {
	switch (type) {
	case MLF2_TYPE_F32: return 4 * n;
	case MLF2_TYPE_F16: return 2 * n;
	case MLF2_TYPE_Q4_K: return n % QK ? 0 : n / QK * 144;
	case MLF2_TYPE_Q6_K: return n % QK ? 0 : n / QK * 210;
	default: return 0;
	}
}

static const mlf2_tensor *find(const mlf2_tensor *t, uint32_t n, const char *name) {
	for (uint32_t i = 0; i < n; i++)
		if (strncmp(t[i].name, name, MLF2_MAX_NAME) == 0) return &t[i];
	return NULL;
}

/* Tensor `name` must exist with dims {d0, d1} (d1 == 0: one dim), of an F32
 * type when `f32_only`, else any matrix type. */
static int need(const mlf2_tensor *t, uint32_t n, const char *name, uint64_t d0, uint64_t d1, int f32_only,
                int optional, char *msg, size_t len) {
	const mlf2_tensor *e = find(t, n, name);
	if (!e) return optional ? 0 : fail(msg, len, "missing tensor %s", name);
	const uint32_t nd = d1 ? 2u : 1u;
	if (e->n_dims != nd || e->dims[0] != d0 || (d1 && e->dims[1] != d1))
		return fail(msg, len, "tensor %s: dims [%llu, %llu] (n_dims %u), expected [%llu, %llu]", name,
		            (unsigned long long)e->dims[0], (unsigned long long)e->dims[1], e->n_dims,
		            (unsigned long long)d0, (unsigned long long)d1);
	if (f32_only && e->type != MLF2_TYPE_F32) return fail(msg, len, "tensor %s: type %u, expected F32", name, e->type);
	return 0;
}

int hako_mlf2_check(const void *map, size_t size, char *msg, size_t len) {
	const unsigned char *b = map;
	if (!b) return fail(msg, len, "null image");
	if (size < sizeof(mlf2_header)) return fail(msg, len, "file too small (%zu bytes)", size);
	mlf2_header h;
	memcpy(&h, b, sizeof h);
	if (memcmp(h.magic, MLF2_MAGIC, 4) != 0) return fail(msg, len, "bad magic (not MLF2)");
	if (h.version != MLF2_VERSION) return fail(msg, len, "unsupported MLF2 version %u", h.version);
	if (h.arch != 0) return fail(msg, len, "unknown architecture %u (qwen2 is 0)", h.arch);

	/* header shape */
	if (!h.n_layers || !h.d_model || !h.n_heads || !h.n_kv_heads || !h.head_dim || !h.ffn_dim || !h.vocab)
		return fail(msg, len, "zero dimension in the header");
	if ((uint64_t)h.n_heads * h.head_dim != h.d_model)
		return fail(msg, len, "n_heads %u x head_dim %u != d_model %u", h.n_heads, h.head_dim, h.d_model);
	if (h.n_heads % h.n_kv_heads) return fail(msg, len, "n_heads %u not a multiple of n_kv_heads %u", h.n_heads,
	                                          h.n_kv_heads);
	if (!(h.rope_theta > 0.0f) || !isfinite(h.rope_theta) || !(h.rms_eps > 0.0f) || !isfinite(h.rms_eps))
		return fail(msg, len, "rope_theta %g / rms_eps %g", (double)h.rope_theta, (double)h.rms_eps);
	if (h.flags & ~(uint32_t)(MLF2_FLAG_QKV_BIAS | MLF2_FLAG_TIED_EMBED))
		return fail(msg, len, "unknown flags 0x%x", h.flags);

	/* sections */
	if (h.tensors_off < sizeof(mlf2_header) || h.tensors_off > size ||
	    (uint64_t)h.n_tensors > (size - h.tensors_off) / sizeof(mlf2_tensor))
		return fail(msg, len, "tensor directory outside the file");
	const uint64_t dir_end = h.tensors_off + (uint64_t)h.n_tensors * sizeof(mlf2_tensor);
	if (h.tokenizer_off < dir_end || h.tokenizer_off > size) return fail(msg, len, "tokenizer offset %llu",
	                                                                     (unsigned long long)h.tokenizer_off);
	if (h.data_off < h.tokenizer_off || h.data_off > size || h.data_off % MLF2_ALIGN)
		return fail(msg, len, "data offset %llu (must be %u-aligned, after the tokenizer, inside the file)",
		            (unsigned long long)h.data_off, MLF2_ALIGN);
	const uint64_t data_size = size - h.data_off;

	/* tokenizer blob: n_tokens, n_merges, then records inside its section */
	{
		const uint64_t end = h.data_off;
		uint64_t p = h.tokenizer_off;
		uint32_t nt, nm;
		if (end - p < 8) return fail(msg, len, "tokenizer blob truncated");
		memcpy(&nt, b + p, 4);
		memcpy(&nm, b + p + 4, 4);
		p += 8;
		for (uint64_t i = 0; i < (uint64_t)nt + nm; i++) {
			const uint64_t hdr = i < nt ? 5 : 4;
			uint32_t l;
			if (end - p < hdr) return fail(msg, len, "tokenizer record %llu truncated", (unsigned long long)i);
			memcpy(&l, b + p + hdr - 4, 4);
			p += hdr;
			if (end - p < l) return fail(msg, len, "tokenizer record %llu truncated", (unsigned long long)i);
			p += l;
		}
	}

	/* directory entries */
	const mlf2_tensor *t = (const mlf2_tensor *)(b + h.tensors_off);
	for (uint32_t i = 0; i < h.n_tensors; i++) {
		mlf2_tensor e;
		memcpy(&e, &t[i], sizeof e);
		if (!memchr(e.name, 0, MLF2_MAX_NAME) || !e.name[0])
			return fail(msg, len, "tensor %u: name empty or not terminated within %u bytes", i, MLF2_MAX_NAME);
		if (type_bytes(e.type, QK) == 0) return fail(msg, len, "tensor %s: unknown type %u", e.name, e.type);
		if (e.n_dims < 1 || e.n_dims > 4) return fail(msg, len, "tensor %s: n_dims %u", e.name, e.n_dims);
		uint64_t nel = 1;
		for (uint32_t d = 0; d < 4; d++) {
			if (d < e.n_dims) {
				if (!e.dims[d] || e.dims[d] > ((uint64_t)1 << 40) / nel)
					return fail(msg, len, "tensor %s: dims[%u] = %llu", e.name, d, (unsigned long long)e.dims[d]);
				nel *= e.dims[d];
			} else if (e.dims[d]) {
				return fail(msg, len, "tensor %s: dims[%u] = %llu past n_dims", e.name, d,
				            (unsigned long long)e.dims[d]);
			}
		}
		if ((e.type == MLF2_TYPE_Q4_K || e.type == MLF2_TYPE_Q6_K) && e.dims[0] % QK)
			return fail(msg, len, "tensor %s: rows of %llu elements are not whole %u-element blocks", e.name,
			            (unsigned long long)e.dims[0], QK);
		if (e.nbytes != type_bytes(e.type, nel))
			return fail(msg, len, "tensor %s: nbytes %llu, type %u and dims give %llu", e.name,
			            (unsigned long long)e.nbytes, e.type, (unsigned long long)type_bytes(e.type, nel));
		if (e.data_off % MLF2_ALIGN) return fail(msg, len, "tensor %s: data offset %llu not %u-aligned", e.name,
		                                         (unsigned long long)e.data_off, MLF2_ALIGN);
		if (e.data_off > data_size || e.nbytes > data_size - e.data_off)
			return fail(msg, len, "tensor %s: bytes [%llu, +%llu) past the data section (%llu bytes)", e.name,
			            (unsigned long long)e.data_off, (unsigned long long)e.nbytes,
			            (unsigned long long)data_size);
		for (uint32_t k = 0; k < i; k++)
			if (strncmp(t[k].name, e.name, MLF2_MAX_NAME) == 0)
				return fail(msg, len, "tensor %s listed twice", e.name);
	}

	/* the tensors of a Qwen2 model of the header's shape (src/model.c:30-57) */
	const uint64_t D = h.d_model, F = h.ffn_dim, KV = (uint64_t)h.n_kv_heads * h.head_dim, V = h.vocab;
	const uint32_t n = h.n_tensors;
	const int bias = (h.flags & MLF2_FLAG_QKV_BIAS) != 0;
	if (need(t, n, "token_embd.weight", D, V, 0, 0, msg, len) || need(t, n, "output_norm.weight", D, 0, 1, 0, msg, len))
		return -1;
	if (!(h.flags & MLF2_FLAG_TIED_EMBED) && need(t, n, "output.weight", D, V, 0, 0, msg, len)) return -1;
	for (uint32_t l = 0; l < h.n_layers; l++) {
		char nm[64];
#define HK_NEED(suffix, d0, d1, f32, opt)                                  \
	snprintf(nm, sizeof nm, "blk.%u." suffix, l);                          \
	if (need(t, n, nm, (d0), (d1), (f32), (opt), msg, len)) return -1;
		HK_NEED("attn_norm.weight", D, 0, 1, 0)
		HK_NEED("attn_q.weight", D, D, 0, 0)
		HK_NEED("attn_k.weight", D, KV, 0, 0)
		HK_NEED("attn_v.weight", D, KV, 0, 0)
		HK_NEED("attn_output.weight", D, D, 0, 0)
		HK_NEED("ffn_norm.weight", D, 0, 1, 0)
		HK_NEED("ffn_gate.weight", D, F, 0, 0)
		HK_NEED("ffn_up.weight", D, F, 0, 0)
		HK_NEED("ffn_down.weight", F, D, 0, 0)
		/* biases: optional in the reference's lookup, required by the flag */
		HK_NEED("attn_q.bias", D, 0, 1, !bias)
		HK_NEED("attn_k.bias", KV, 0, 1, !bias)
		HK_NEED("attn_v.bias", KV, 0, 1, !bias)
#undef HK_NEED
	}
	if (msg && len) msg[0] = 0;
	return 0;
}
