/*
 * hako_nn.h — drop-in for the reference's nn.h (src/nn.h:6-29).
 *
 * matmul and deq_row run on the gfx950 kernels of libhako_gpu; the model's
 * data section is mirrored into HBM verbatim, once, on first use (the upload
 * point the reference's mmap loader, src/loader.c:12-52, leaves open).
 * rmsnorm, softmax, silu_f and rope_neox are the reference's host-side
 * elementwise helpers, kept on the host with the reference's formulas so that
 * a caller linking this library in place of nn.c (src/model.c, src/sample.c)
 * resolves every symbol it used.
 */
#pragma once
#include "hako_decode.h"
#include "hako_mlf2.h"

#ifdef __cplusplus
extern "C" {
#endif

/* reference src/nn.c:13-18 */
void rmsnorm(float *y, const float *x, const float *w, int n, float eps);
/* reference src/nn.c:20-27 */
void softmax(float *x, int n);
/* reference src/nn.c:29 */
float silu_f(float x);
/* reference src/nn.c:32-42 */
void rope_neox(float *vec, int head_dim, int pos, float theta);

/* reference src/nn.c:179-210: out[n_out] = W x (+bias), W the MLF2 tensor `w`
 * of model `m` (row-major, dims[0] = n_in). Q4_K weights use the q8_32
 * activation scheme and integer dot; Q6_K, F16 and F32 weights an fp32 dot.
 * Synchronous; host pointers. */
void matmul(float *out, const float *x, const hakm_model *m, const mlf2_tensor *w,
            const float *bias, int n_out, int n_in);

/* reference src/nn.c:55-59: dequantize row r (n_in values) of `w` into out. */
void deq_row(const hakm_model *m, const mlf2_tensor *w, int r, int n_in, float *out);

/* ── additions (no reference counterpart) ── */

/* Mirror m's data section into HBM now (matmul does it on first use).
 * Returns 0 or a negative hako_gpu error code. */
int hako_model_upload(const hakm_model *m);
/* Forget m's HBM mirror; call before unmapping a model whose address range
 * may be reused by another. Refused (HAKO_GPU_EINVAL, nothing released)
 * while a decoder made by hako_decoder_from_model from m is alive: destroy
 * the decoders first. */
int hako_model_release(const hakm_model *m);

/* A device decoder (hako_decode.h) for mapped model m: the tensors
 * hakm_ctx_new resolves (reference src/model.c:30-57) at their mirror
 * addresses, the lm_head tied to token_embd when the header says so. One
 * hako_gpu_decoder_step / _generate call then replaces hakm_forward
 * (src/model.c:93-165) plus the greedy pick for every step. Returns 0 or a
 * negative hako_gpu error code. */
/* The decoder reads m's mirror in place, so the mirror is pinned until
 * hako_gpu_decoder_destroy(dec): release, eviction or replacement of it are
 * refused until then. */
int hako_decoder_from_model(const hakm_model *m, int n_seq, int max_seq, hako_gpu_decoder **dec);

#ifdef __cplusplus
}
#endif
