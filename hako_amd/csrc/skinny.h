// skinny.h — the skinny (<= 16 token) matmul launches shared by the batch
// matmul entry point and the batched decode step.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hako {

constexpr int kSkMaxTokens = 16;

// Row segments of one launch: rows [row0, row0 + rows) of the launch's row
// space come from weight w (rows of n_in elements) and go to out[t*ld + r]
// for token t and segment row r; bias (F32, may be null) for the Store
// epilogue. Segment starts are multiples of 16 rows.
struct SkSeg {
	const uint8_t *w;
	const float *bias;
	float *out;
	int row0, rows, ld;
};
struct SkSegs {
	SkSeg s[3];
	int n;
};

// Epilogues: Store out = y (+ bias); Add out += y (a residual); SwiGLU
// (Q4_K only): segment 0 (gate, launch rows [0, F)) and segment 1 (up, rows
// [F, 2F)), out (segment 0's) = silu(gate)*up.
// Part leaves the splits' partial sums in `part` ([split][16][rows], every
// split, tokens past m zero) for a consumer that sums them itself.
enum { kSkStore = 0, kSkAdd = 1, kSkSwiGLU = 2, kSkPart = 3 };

// Q6_K: workgroups a launch aims for; K is split over workgroups to reach
// it. Split results go to `part` (the *_part_floats count of floats;
// part_cap is what the caller holds), summed by a second launch that applies
// the epilogue. 2 per CU: the 7B down matmul over 16 tokens then takes 9
// splits, and the kernel after it, which adds each token's partials on one
// CU, reads half of what 18 splits left (16-sequence step 4151-4167 ->
// 4091-4097 us; 8 splits 4118, 10-11 splits 4210-4222). Q4_K: the
// persistent grid's workgroups (one per CU); K is split over launches only
// past 4096. Both are launch-shape knobs (hako_gpu_tune).
constexpr int kSkTargetWgsQ6 = 512;

// Q4_K x q8: xq [m][n_in] int8 and xs [m][n_in/32] (q8_32 rows), m <= 16.
int q4k_skinny_splits(int n_in, int vrows);
size_t q4k_skinny_part_floats(int n_in, int vrows, int epi);
int q4k_skinny(const SkSegs &segs, int epi, const int8_t *xq, const float *xs, int m, int n_in, int vrows,
               float *part, size_t part_cap);
// Q6_K x fp32 as fp16 hi/lo rows [m][n_in] with a power of two per token,
// esc[m] (x = (hi + lo) * esc), or per token and 256-wide block,
// esc[m][n_in/256] (esc_per_block); Store, Add or Part.
int q6k_skinny_splits(int n_in, int vrows);
size_t q6k_skinny_part_floats(int n_in, int vrows, int epi);
int q6k_skinny(const SkSegs &segs, int epi, const _Float16 *xh, const _Float16 *xl, const float *esc, int m,
               int n_in, int vrows, float *part, size_t part_cap, bool esc_per_block = false);
// The gate/up partials of a Part launch over rows [0, 2F) (gate rows r, up
// rows F + r, nsplit splits) to h = silu(gate)*up as fp16 hi/lo rows [m][F]
// with a power of two per token and 256-row block, escb[m][F/256].
int swiglu_split(const float *part, int nsplit, int F, int m, _Float16 *xh, _Float16 *xl, float *escb);
// The fp16 hi/lo split of m fp32 rows of n floats with one power of two per
// row, esc[m] (gemm.hip).
int f16_split(const float *x, _Float16 *xh, _Float16 *xl, float *esc, int m, int n);

// Multi-token (m > 16) matmuls of gemm.hip. Q4_K x q8 over row segments of
// vrows launch rows (segment starts multiples of 64; each segment's out is
// [m][ld]): Store, Add, or SwiGLU (segment 0 gate and segment 1 up, both
// rows [0, F) with F % 32 == 0; out of segment 0 = silu(gate)*up).
int q4k_gemm_segs(const SkSegs &segs, int epi, const int8_t *xq, const float *xs, int m, int n_in, int vrows);
// Q6_K x the fp16 hi/lo rows of f16_split: y[m][n_out] = (or += when add)
// W x (+ bias).
// skp: stream-K slots of q6k_gemm_sk_floats(q6k_gemm_sk_grid()) floats, or
// null (then no stream-K); the launch uses them only when its 128-row tiles
// would leave CUs idle.
int q6k_gemm_split(float *y, const void *w, const _Float16 *xh, const _Float16 *xl, const float *esc,
                   const float *bias, int m, int n_out, int n_in, bool add, float *skp = nullptr,
                   size_t skp_floats = 0);
size_t q6k_gemm_sk_floats(int G);
int q6k_gemm_sk_grid();

}  // namespace hako
