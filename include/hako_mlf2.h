/*
 * hako_mlf2.h — the MLF2 weight container and the loaded-model view that the
 * reference's nn.h functions take.
 *
 * These declarations must stay byte-compatible with the reference's, because
 * the drop-in matmul/deq_row receive pointers to the caller's own structs:
 *   - mlf2_header: reference include/mlf2.h:55-77 (packed, 128 bytes)
 *   - mlf2_tensor: reference include/mlf2.h:80-87 (packed, 104 bytes)
 *   - hakm_model:  reference src/loader.h:6-13
 * Type ids are the reference's (include/mlf2.h:44-49), which are ggml's.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifndef MLF2_MAGIC
#define MLF2_MAGIC     "MLF2"
#define MLF2_VERSION   2u
#define MLF2_ALIGN     32u
#define MLF2_MAX_NAME  48u

enum mlf2_type {
	MLF2_TYPE_F32  = 0,
	MLF2_TYPE_F16  = 1,
	MLF2_TYPE_Q4_K = 12,
	MLF2_TYPE_Q6_K = 14,
};

#define MLF2_FLAG_QKV_BIAS    (1u << 0)
#define MLF2_FLAG_TIED_EMBED  (1u << 1)

typedef struct __attribute__((packed)) {
	char     magic[4];
	uint32_t version;
	uint32_t arch;
	uint32_t n_layers;
	uint32_t d_model;
	uint32_t n_heads;
	uint32_t n_kv_heads;
	uint32_t head_dim;
	uint32_t ffn_dim;
	uint32_t ctx;
	uint32_t vocab;
	float    rope_theta;
	float    rms_eps;
	uint32_t flags;
	uint32_t n_tensors;
	uint64_t tensors_off;
	uint64_t tokenizer_off;
	uint64_t data_off;
	uint32_t bos_id;
	uint32_t eos_id;
	uint8_t  reserved[36];
} mlf2_header;

typedef struct __attribute__((packed)) {
	char     name[MLF2_MAX_NAME];
	uint32_t type;
	uint32_t n_dims;
	uint64_t dims[4];      /* dims[0] = fastest (columns) */
	uint64_t data_off;     /* relative to the data section */
	uint64_t nbytes;
} mlf2_tensor;
#endif /* MLF2_MAGIC */

#ifndef HAKO_HAKM_MODEL_DEFINED
#define HAKO_HAKM_MODEL_DEFINED
typedef struct {
	mlf2_header          h;
	const mlf2_tensor   *tensors;
	const unsigned char *data;      /* base of the data section */
	const unsigned char *tok;
	void   *map;
	size_t  map_size;
} hakm_model;
#endif

/* ── addition (no reference counterpart) ── */

/* Structural check of a whole MLF2 image (`map`, `size` bytes: the mapped
 * file): the reference loader's own checks (src/loader.c:26-43: size, magic,
 * version, section offsets) plus the converter's layout rules
 * (tools/gguf2mlf.py:138-190: 32-byte aligned data section and tensor
 * offsets, dims padded with zeros), every tensor's type known, nbytes equal
 * to what its type and dims give, its bytes inside the data section, names
 * terminated and unique, the tokenizer records inside their section, and the
 * Qwen2 tensors hakm_ctx_new resolves (src/model.c:30-57) present with the
 * header's dims (norms and biases F32; biases required when the header's
 * QKV_BIAS flag is set). Returns 0, or -1 with a description in msg
 * (msg_len bytes, may be 0). Reads only the image; no device needed. */
#pragma GCC visibility push(default)
int hako_mlf2_check(const void *map, size_t size, char *msg, size_t msg_len);
#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif
