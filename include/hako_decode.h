/*
 * hako_decode.h — device-resident Qwen2 decode step (C ABI).
 *
 * Replaces, for a whole token step, the reference's hakm_forward
 * (src/model.c:93-165) with its greedy pick (src/sample.c:28-32): embedding
 * row, then per layer rmsnorm, q/k/v projections with bias, NeoX rope,
 * KV-cache append, GQA softmax attention, output projection and residual,
 * rmsnorm, SwiGLU feed-forward and residual; final rmsnorm, lm_head, argmax.
 * Weights stay where they are in HBM (e.g. inside an uploaded MLF2 mirror,
 * include/hako_gpu.h); activations, KV caches and token ids stay on the
 * device between steps, so a greedy loop needs no host round trip per token.
 *
 * Numerics follow the reference's formulas; its matmuls are the library's
 * kernels (Q4_K x q8 with exact integer sums, Q6_K / F16 / F32 x fp32), and
 * the rope angles come from a table computed on the host with the reference's
 * own expression (src/nn.c:31-41). Plain C, no HIP types; every function
 * returns 0 or a negative HAKO_GPU_E* code with hako_gpu_last_error() set.
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

/* One transformer block (reference src/model.h:5-10): device addresses and
 * HAKO_TYPE_* of each matrix (rows of n_in elements, src/nn.h:18-21); norms
 * and biases are F32 (biases may be NULL). */
typedef struct {
	const float *attn_norm, *ffn_norm;
	const void *wq, *wk, *wv, *wo;
	const float *bq, *bk, *bv;
	const void *gate, *up, *down;
	int t_q, t_k, t_v, t_o, t_gate, t_up, t_down;
} hako_gpu_block;

/* A Qwen2 model (reference src/model.h:12-26, mlf2_header fields). `blocks`
 * is read at create time only. out_weight may equal tok_embd (tied). */
typedef struct {
	int n_layers, d_model, n_heads, n_kv_heads, head_dim, ffn_dim, vocab;
	float rope_theta, rms_eps;
	const void *tok_embd;
	int t_embd;
	const float *out_norm;
	const void *out_weight;
	int t_out;
	const hako_gpu_block *blocks;
} hako_gpu_model;

typedef struct hako_gpu_decoder hako_gpu_decoder;

/* A decoder for n_seq independent sequences of up to max_seq positions each
 * (KV caches, activations and the rope table are allocated here, once).
 * Requires head_dim 64 or 128, n_heads % n_kv_heads == 0 with at most 8
 * query heads per KV head, d_model and ffn_dim multiples of 256, and
 * 1 <= n_seq <= 16. Every tensor may be F32, F16, Q4_K or Q6_K, chosen per
 * layer. With n_seq > 1 every step advances all sequences together, each
 * matmul streaming its weights once for all of them; layers of the Q4_K_M
 * mix (Q4_K q/k/v/o/gate/up, Q6_K down) with d_model <= 4096 take fused
 * launches, other layers one launch per matmul. Every sum of a step has a
 * fixed order or is exact (with n_seq == 1 and Q4_K output projections their
 * 256-input block sums meet in a 64-bit fixed-point accumulator on the 2^-32
 * grid), so steps are bit-reproducible. */
int hako_gpu_decoder_create(const hako_gpu_model *m, int n_seq, int max_seq, hako_gpu_decoder **dec);
int hako_gpu_decoder_destroy(hako_gpu_decoder *dec);

/* Device addresses of the fp32 KV caches, laid out as the reference's
 * (src/model.c:71-72, 117-118) once per sequence:
 * [n_seq][n_layers][max_seq][n_kv_heads*head_dim]. A caller may fill
 * positions below the next write position directly (a prefilled context). */
int hako_gpu_decoder_kv(hako_gpu_decoder *dec, float **k_cache, float **v_cache);

/* Set the next write position of every sequence (hakm_ctx.pos); pos[n_seq]. */
int hako_gpu_decoder_set_pos(hako_gpu_decoder *dec, const int *pos);

/* One step for every sequence: tokens[n_seq] in (host); if logits is not NULL
 * the fp32 logits [n_seq][vocab] are copied to it (host), and next[n_seq]
 * (host, may be NULL) receives the greedy ids. Advances every position by
 * one. Synchronous. */
int hako_gpu_decoder_step(hako_gpu_decoder *dec, const int *tokens, float *logits, int *next);

/* n greedy steps from tokens[n_seq]: out[n][n_seq] (host) receives the ids
 * chosen at each step, each fed back as the next step's input on the device.
 * The step is captured once as a HIP graph and replayed n times; one
 * synchronization at the end. Positions advance by n. */
int hako_gpu_decoder_generate(hako_gpu_decoder *dec, const int *tokens, int n, int *out);

/* Feeds n prompt tokens (host) to sequence seq from its current position,
 * as the reference's feed (src/hakm_api.c:105-111, one hakm_forward per
 * token) but through the multi-token matmuls, up to 512 tokens per pass
 * (fewer when max_seq makes the attention records of a pass exceed 1 GiB),
 * with causal attention over the sequence's cache: the keys and values of
 * every prompt position are written, the position advances by n, and the
 * logits of the last prompt token go to logits[vocab] (host, may be NULL)
 * with their greedy id in *next (may be NULL). Synchronous. The other
 * sequences are untouched. */
int hako_gpu_decoder_prefill(hako_gpu_decoder *dec, int seq, const int *tokens, int n, float *logits, int *next);

/* Replays the captured step n times from the current device state (no host
 * transfer, no synchronization): the timed loop of a benchmark. */
int hako_gpu_decoder_replay(hako_gpu_decoder *dec, int n);

/* Registers fn(arg), run once by hako_gpu_decoder_destroy after the decoder's
 * work has finished and before its memory is released: a decoder reads its
 * weights in place, so whoever owns them (e.g. a model mirror) learns here
 * when they are no longer read. A later call replaces the hook; fn NULL
 * removes it. No reference counterpart (the reference's forward reads the
 * mapping it holds, src/model.h:12-26). */
int hako_gpu_decoder_on_destroy(hako_gpu_decoder *dec, void (*fn)(void *arg), void *arg);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif
