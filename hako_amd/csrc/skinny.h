// skinny.h — the skinny (<= 16 token) matmul launches shared by the batch
// matmul entry point and the batched decode step.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace hako {

constexpr int kSkMaxTokens = 16;
constexpr int kSkMaxQ4In = 4096;   // activations staged in LDS

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
// (Q4_K only): segments 0 (gate) and 1 (up) of `rows` rows each, out
// (segment 0's) = silu(gate)*up.
enum { kSkStore = 0, kSkAdd = 1, kSkSwiGLU = 2 };

// Q4_K x q8: xq [m][n_in] int8 and xs [m][n_in/32] (q8_32 rows), m <= 16,
// n_in <= kSkMaxQ4In (activations staged in LDS).
int q4k_skinny(const SkSegs &segs, int epi, const int8_t *xq, const float *xs, int m, int n_in, int vrows);
size_t q4k_skinny_lds(int n_in);
// Q6_K x fp32 as fp16 hi/lo rows [m][n_in] with per-row powers of two esc[m];
// Store or Add epilogue. Long rows are split along K over several
// workgroups: `part` (q6k_skinny_part_floats floats) holds their results,
// summed by a second launch that applies the epilogue.
constexpr int kSkTargetWgs = 512;
int q6k_skinny_splits(int n_in, int vrows);
size_t q6k_skinny_part_floats(int n_in, int vrows);
int q6k_skinny(const SkSegs &segs, int epi, const _Float16 *xh, const _Float16 *xl, const float *esc, int m,
               int n_in, int vrows, float *part);
// The fp16 hi/lo split of m fp32 rows of n floats (gemm.hip).
int f16_split(const float *x, _Float16 *xh, _Float16 *xl, float *esc, int m, int n);

}  // namespace hako
