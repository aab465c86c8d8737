/*
 * hako_gpu.h — C ABI of the MI355X (gfx950) quantized-matmul library.
 *
 * Plain C: no HIP or torch types cross this boundary. Every function returns
 * 0 on success or a negative HAKO_GPU_E* code, and records a message that
 * hako_gpu_last_error() returns (per calling thread). Device pointers are
 * addresses returned by hako_gpu_malloc (or any HIP allocation on the same
 * device). Unless a function says otherwise, work is enqueued on the
 * library's stream and the call returns without waiting; hako_gpu_sync()
 * waits for it.
 *
 * The weight layouts are the ones the reference stores verbatim: Q4_K
 * super-blocks of 144 bytes and Q6_K super-blocks of 210 bytes per 256
 * weights (reference src/quant.h:9-24), rows of n_in/256 blocks one after the
 * other, row-major over n_out rows (src/nn.h:18-21).
 */
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

/* ── error codes ── */
#define HAKO_GPU_OK          0
#define HAKO_GPU_EINVAL     -1   /* bad argument: size, alignment, type */
#define HAKO_GPU_ENODEV     -2   /* no usable gfx950 device / not initialised */
#define HAKO_GPU_ENOMEM     -3   /* device allocation failed */
#define HAKO_GPU_EHIP       -4   /* a HIP runtime call failed */
#define HAKO_GPU_ENOTFOUND  -5   /* host pointer is not inside an uploaded mirror */
#define HAKO_GPU_ETYPE      -6   /* unsupported tensor type */

/* Tensor type ids: the values of the MLF2 format (reference include/mlf2.h:44-49). */
#define HAKO_TYPE_F32   0
#define HAKO_TYPE_F16   1
#define HAKO_TYPE_Q4_K 12
#define HAKO_TYPE_Q6_K 14

/* ── runtime ── */

/* Select and initialise device `device` (creates the library stream).
 * Idempotent for the same device. No reference counterpart: the reference
 * has no device (its matmul starts a thread pool, src/nn.c:152-157). */
int hako_gpu_init(int device);
/* Release every buffer, mirror and stream the library owns. */
int hako_gpu_shutdown(void);
/* Message of the last failed call on this thread ("" if none). */
const char *hako_gpu_last_error(void);

/* Launch-shape knobs of the GEMV kernels (for sweeps; results do not depend
 * on them): workgroups per compute unit of the persistent grids (1..8) and
 * waves per workgroup (4 or 8). */
#define HAKO_TUNE_Q4K_WGS_PER_CU 1
#define HAKO_TUNE_Q6K_WGS_PER_CU 2
#define HAKO_TUNE_Q4K_WAVES      3
#define HAKO_TUNE_Q6K_WAVES      4
#define HAKO_TUNE_Q4K_FLAT_ITEMS 5   /* -1: by shape (default); 0: persistent grid; 1/2/4/8: flat grid, row items per wave */
/* Skinny (2..16 token) launches: the Q4_K persistent grid's workgroups (0:
 * the default, 256), and the workgroups a Q6_K launch aims for through its K
 * split (0: the default, 512); the Q6_K split count sets the order in which
 * its fp32 partial sums are added. A decoder sizes its split workspace when
 * it is created; a later, larger Q6_K target makes its steps fail with
 * EINVAL. */
#define HAKO_TUNE_SKINNY_Q4K_WGS 6
#define HAKO_TUNE_SKINNY_Q6K_WGS 7
#define HAKO_TUNE_Q6K_FLAT_ITEMS 8   /* -1: by shape (default); 0: persistent grid; 1/2/4/8: flat grid, row items per wave */
#define HAKO_TUNE_DEC_GU_ITEMS   9   /* one-sequence decoder gate/up launch: row items per wave, 4 or 8, or 0 = by shape (default); read when a step is enqueued or captured */
#define HAKO_TUNE_Q6K_FLAT_SEG  10   /* Q6_K flat grid, rows wider than 64 chunks: chunks per part, 64 or 32, or 0 = by shape (default) */
#define HAKO_TUNE_Q6K_ROWS      11   /* Q6_K rows grid: 10 x waves + items in flight (44, 82, 84, 162), 0 = by shape (default), -1 = never */
#define HAKO_TUNE_Q4K_GEMM_RES  12   /* Q4_K multi-token matmul with n_in <= 3840: 1 = resident token tile (default), 0 = 64 x 64 tiles */
#define HAKO_TUNE_Q6K_GEMM_TN   13   /* Q6_K multi-token matmul: rows per workgroup tile, 64 or 128, or 0 = by shape (default) */
#define HAKO_TUNE_Q6K_DIGITS    14   /* Q6_K persistent GEMV grid: 1 = integer activation columns (default), 0 = fp32 product per weight */
#define HAKO_TUNE_Q6K_GEMM_SK   15   /* Q6_K multi-token matmul, stream-K when 128-row tiles leave CUs idle: 1 = in the decoder's prompt pass (default), 2 = also in hako_gpu_matmul_batch / hako_gpu_q6k_gemm, 0 = never */
#define HAKO_TUNE_DEC_GU_GRID   16   /* one-sequence decoder gate/up launch: 1 = flat grid, 2 = persistent grid (one workgroup per CU, the rmsnorm prologue once per workgroup), 0 = by shape (default: persistent); read when a step is enqueued or captured */
#define HAKO_TUNE_DEC_MERGE_ROWS 17  /* one-sequence decoder merge+o launch: rows per workgroup, 64 or 128, or 0 = by shape (default: 128 past d_model 2048); the same bits either way; read when a step is enqueued or captured */
#define HAKO_TUNE_DEC_QKV_ITEMS  18  /* one-sequence decoder q/k/v launch: row items per wave, 2, 4 or 8, or 0 = by shape (default: 8 past d_model 2048, else 2); the same bits either way; read when a step is enqueued or captured */
#define HAKO_TUNE_DEC_ATTN_PARTS 19  /* one-sequence decoder attention: workgroups that share a query-head group, 1..8, or 0 = by shape (default: 2 with 7 heads per group, else up to 4); the same bits either way; read when a step is enqueued or captured */
int hako_gpu_tune(int knob, int value);

typedef struct {
	char     name[64];        /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
	int      compute_units;
	int      clock_khz;
	size_t   hbm_bytes;
	int      l2_bytes;
	int      lds_bytes_per_cu;
} hako_gpu_info;
int hako_gpu_device_info(hako_gpu_info *out);

/* Device memory (plain pointers). */
int hako_gpu_malloc(void **dptr, size_t bytes);
int hako_gpu_free(void *dptr);
int hako_gpu_memcpy_h2d(void *dst, const void *src, size_t bytes);   /* synchronous */
int hako_gpu_memcpy_d2h(void *dst, const void *src, size_t bytes);   /* synchronous */
int hako_gpu_memcpy_d2d(void *dst, const void *src, size_t bytes);   /* on the stream */
int hako_gpu_sync(void);

/* The library stream as an opaque hipStream_t, for callers that interleave
 * their own HIP work with the library's. */
void *hako_gpu_stream(void);

/* Events on the library stream, for timing. */
int hako_gpu_event_create(void **ev);
int hako_gpu_event_record(void *ev);
int hako_gpu_event_elapsed_ms(void *start, void *stop, float *ms);    /* waits for stop */
int hako_gpu_event_destroy(void *ev);

/* Timing marks that also work inside a captured graph (no reference
 * counterpart; measurement only): a one-wave kernel on the library stream
 * writes the device's constant-rate wall clock, in ticks of
 * hako_gpu_timestamp_hz, to the 8-byte device address dst when it runs. */
int hako_gpu_timestamp(void *dst);
int hako_gpu_timestamp_hz(double *hz);

/* HIP graphs by stream capture: library calls made on this thread between
 * capture_begin and capture_end are recorded, not run; graph_launch replays
 * them on the library stream with one submission. Calls that copy from or to
 * host memory or allocate must stay outside a capture: make one call of each
 * shape before capturing it, so that the library workspaces it uses exist.
 * A workspace outgrown by a later, larger call is kept (not freed) until
 * hako_gpu_shutdown, so a graph captured earlier stays valid; graphs that
 * run concurrently with each other or with eager calls share the workspaces
 * and must not overlap in time. */
int hako_gpu_capture_begin(void);
int hako_gpu_capture_end(void **graph);
int hako_gpu_graph_launch(void *graph);
int hako_gpu_graph_destroy(void *graph);

/* ── verbatim weight upload ──
 * Copies host bytes [host, host+bytes) into one device allocation, once, and
 * remembers the range, so that any host pointer p inside it maps to
 * dev + (p - host). This is how an mmap'd MLF2 data section (reference
 * src/loader.c:12-52; tensors at data + data_off, src/loader.c:66-68) is put
 * in HBM byte for byte. A range that overlaps a mirror is refused (EINVAL):
 * release the older mirror first — memory freed or unmapped while mirrored
 * keeps its mirror until hako_gpu_mirror_release, and a later buffer at
 * those addresses holds other bytes. */
int hako_gpu_mirror_upload(const void *host, size_t bytes, void **dev);
int hako_gpu_mirror_release(const void *host);
/* Device address of host pointer p inside a mirror; NULL if none holds it. */
void *hako_gpu_mirror_lookup(const void *p);

/* ── kernels on device pointers (asynchronous, library stream) ── */

/* quantize_row_q8_32 (reference src/quant.c:127-144) over `rows` rows of n
 * floats (n % 32 == 0): xq[rows*n] int8, xs[rows*n/32] fp32 scales, with the
 * rounding the reference build uses (xs = amax*RN(1/127), inv = 127/amax,
 * round-half-even, clamp to +-127, subnormals flushed). */
int hako_gpu_quantize_q8_32(const float *x, int64_t rows, int n, int8_t *xq, float *xs);

/* dequant_tensor (reference src/quant.c:234-248): nelem values of `type`
 * (F32, F16, Q4_K, Q6_K; nelem % 256 == 0 for the k-quants) to fp32. */
int hako_gpu_dequant(int type, const void *src, float *out, int64_t nelem);

/* Q4_K x q8 GEMV on a pre-quantized activation: out[r] = sum over the
 * sub-blocks sb of xs[sb]*(d*s*iqx - dmin*m*ix) (+ bias[r]), i.e.
 * q4k_vec_dot per row (reference src/quant.c:150-232, src/nn.c:76-82).
 * bias may be NULL. n_in % 256 == 0, n_in <= 32768 (the activation is held
 * in LDS; EINVAL past it). */
int hako_gpu_q4k_gemv(float *out, const void *w, const int8_t *xq, const float *xs,
                      const float *bias, int n_out, int n_in);

/* Integer sums of the same GEMV, for bit-exact checking: iqx[r*n_in/32 + sb]
 * = sum q*xq and ix[...] = sum xq over sub-block sb of row r. Uses the GEMV's
 * own load and unpack code. */
int hako_gpu_q4k_isums(int32_t *iqx, int32_t *ix, const void *w, const int8_t *xq,
                       int n_out, int n_in);

/* Q6_K x fp32 GEMV: out[r] = sum_i deq(W[r])[i] * x[i] (+ bias[r]), the
 * reference's generic path for Q6_K rows (src/nn.c:84-95, src/quant.c:94-123).
 * The activation stays fp32. n_in % 256 == 0, n_in <= 32768 (EINVAL past it),
 * the weight under 2 GiB. */
int hako_gpu_q6k_gemv(float *out, const void *w, const float *x, const float *bias,
                      int n_out, int n_in);

/* F32 / F16 weight GEMV (the reference's generic path for those types). */
int hako_gpu_dense_gemv(float *out, int type, const void *w, const float *x,
                        const float *bias, int n_out, int n_in);

/* ── multi-token matmuls (prompt prefill) ──
 * Y[t][r] for tokens t < m: the m independent products the reference computes
 * with one matmul call per token (src/nn.c:179-210, once per prompt token as
 * cli/main.c:56-60 feeds them). y is [m][n_out], x / xq are [m][n_in],
 * xs is [m][n_in/32]. */

/* Q4_K x q8 on int8 matrix cores: per 32-wide sub-block integer sums exactly
 * as q4k_vec_dot (src/quant.c:150-232), folded in fp32. bias may be NULL. */
int hako_gpu_q4k_gemm(float *y, const void *w, const int8_t *xq, const float *xs,
                      const float *bias, int m, int n_out, int n_in);

/* Q6_K x fp32 (the reference's generic row path, src/nn.c:84-95) on fp16
 * matrix cores, the activation carried as two fp16 halves. Uses a library
 * workspace (grown on first use: not inside a graph capture). */
int hako_gpu_q6k_gemm(float *y, const void *w, const float *x, const float *bias,
                      int m, int n_out, int n_in);

/* matmul over m activation rows for any supported type: Q4_K quantizes the
 * rows with the q8_32 scheme (library workspace) then runs the Q4_K GEMM;
 * Q6_K runs the Q6_K GEMM; F32/F16 run one GEMV per row; m == 1 is
 * hako_gpu_matmul. */
int hako_gpu_matmul_batch(float *y, const float *x, int type, const void *w,
                          const float *bias, int m, int n_out, int n_in);

/* hako_gpu_matmul_batch that allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results (bit for bit) as hako_gpu_matmul_batch;
 * its scratch (activation rows in q8_32 or fp16 hi/lo form, split-K partials)
 * is a 48 MiB array that each device holds until the process ends, enough
 * for 512 tokens x 18944 inputs of either type. A call that needs more is
 * refused with HAKO_GPU_EINVAL and a message. Calls on one device share the
 * array: calls that overlap in time on one device (several streams, or
 * graphs replayed concurrently) race. */
int hako_gpu_matmul_batch_noalloc(float *y, const float *x, int type, const void *w,
                                  const float *bias, int m, int n_out, int n_in);

/* matmul (reference src/nn.c:179-210) on device pointers: out[n_out] =
 * W x (+bias) for a weight of any supported type. For Q4_K the activation is
 * quantized with the q8_32 scheme inside the GEMV's workgroups (in LDS), so
 * one launch does the whole call. */
int hako_gpu_matmul(float *out, const float *x, int type, const void *w,
                    const float *bias, int n_out, int n_in);

/* The same on host pointers, for the nn.h drop-in: x, out and (if not inside
 * a mirror) bias are host memory; w must be inside a mirror (uploaded once).
 * Synchronous. */
int hako_gpu_matmul_host(float *out, const float *x, int type, const void *w_host,
                         const float *bias_host, int n_out, int n_in);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif
