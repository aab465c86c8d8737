// decode.hip — device-resident Qwen2 decode step (include/hako_decode.h).
//
// One step is the reference's hakm_forward (src/model.c:93-165) plus its
// greedy pick (src/sample.c:28-32), as a fixed sequence of launches that
// reads the token and position from device memory, so it is captured once as
// a HIP graph and replayed for every token. Per layer, with the Q4_K_M mix:
//
//   1. q/k/v: rmsnorm + q8_32 quantization in the workgroup prologue, the
//      three Q4_K matrices as row segments of one GEMV, biases added;
//   2. attention: NeoX rope of the group's query heads and of the new key,
//      KV-cache append, softmax attention over 64-position chunks of the cache
//      (one workgroup per chunk and KV head), partial results merged by the
//      last workgroup of each head group to finish;
//   3. output projection (q8 prologue) added into the residual stream;
//   4. gate/up: rmsnorm + q8 prologue, gate and up rows interleaved so each
//      wave holds both sums of a row and writes silu(gate)*up;
//   5. down projection (Q6_K x fp32) added into the residual stream.
//
// Then the final rmsnorm, the lm_head GEMV and the argmax, which writes the
// next token, appends it to the output ring and advances the position.
// Other weight types run the same step through the generic matmul and
// separate elementwise launches.
#include <math.h>
#include <string.h>

#include <vector>

#include "../../include/hako_decode.h"
#include "dequant_dev.h"
#include "hako_dev.h"
#include "hako_rt.h"
#include "q4k_dev.h"
#include "skinny.h"

namespace hako {

int q6k_gemv(float *out, const void *w, const float *x, const float *bias, int n_out, int n_in, const float *res);

namespace {

constexpr int kChunk = 64;   // cache positions per attention workgroup
constexpr int kMaxG = 8;     // query heads per KV head
constexpr int kArgBlocks = 64;
constexpr int kArgHoist = 16;   // loads per thread taken up front by argmax_part_kernel (slices up to 4096)
constexpr int kDecItems = 4; // row items per wave of the fused GEMV
constexpr int kDecItemsQkv = 2; // ... of the q/k/v launch (fewer rows: more workgroups)
// ... of the gate/up launch: 0 = by shape (8 when a row item is one row,
// d_model > 2048: half the workgroups, each repeating the rmsnorm prologue
// over the whole activation; 7B step 1781 -> 1744 us, the 3B shape slower
// with 8), else 4 or 8 (tuning knob)
int g_dec_gu_items = 0;
// gate/up launch of the one-sequence step: 1 flat grid, 2 persistent grid, 0 by shape (persistent)
int g_dec_gu_grid = 0;
// rows per merge+o workgroup: 64 or 128, 0 by shape
int g_dec_merge_rows = 0;
// row items per wave of the q/k/v launch: 2, 4 or 8, 0 by shape
int g_dec_qkv_items = 0;
// attention parts per query-head group with one sequence: 1..8, 0 by shape
int g_dec_attn_parts = 0;

// One sequence's output projection adds its per-input-block row sums into a
// residual accumulator of 64-bit fixed-point values (2^-32 units): integer
// addition is associative, so the sum does not depend on the order in which
// the blocks arrive and the step is bit-reproducible. The value a block adds
// is its fp32 sum rounded to the 2^-32 grid; the accumulated sum is
// converted back to fp32 once.
//
// An accumulator row is D int64 sums followed by D int32 flags. A block sum
// that is not finite adds nothing to the sum and ORs its kind into the
// row's flags (NaN, +inf, -inf), and the consumer turns a flagged row back
// into what an fp32 sum of those terms gives: NaN for a NaN or for both
// infinities, else the infinity — as the reference's fp32 fold and residual
// add propagate them (src/quant.c:222-225, src/model.c:146). A finite block
// sum is clamped to +-2^25 (2^57 units), so the sum of up to 64 blocks
// (d_model <= 16384) cannot wrap; the decoder takes this path only within
// that width, and no model's residual comes near 2^25.
constexpr double kFixScale = 4294967296.0;          // 2^32
constexpr double kFixInv = 1.0 / 4294967296.0;      // 2^-32
constexpr double kFixMax = 144115188075855872.0;    // 2^57
constexpr int kFixMaxBlocks = 64;                   // d_model / 256 blocks per row at most
enum : int { kFlagNaN = 1, kFlagPosInf = 2, kFlagNegInf = 4 };
__device__ __forceinline__ long long to_fixed(float f) {
	if (!__builtin_isfinite(f)) return 0;
	double v = (double)f * kFixScale;
	v = __builtin_fmin(__builtin_fmax(v, -kFixMax), kFixMax);
	return (long long)__builtin_rint(v);
}
__device__ __forceinline__ int fixed_flag(float f) {
	return f != f ? kFlagNaN : (__builtin_isinf(f) ? (f > 0.0f ? kFlagPosInf : kFlagNegInf) : 0);
}
__device__ __forceinline__ float from_fixed(long long a, int flags) {
	if (flags == 0) return (float)((double)a * kFixInv);
	if ((flags & kFlagNaN) || (flags & (kFlagPosInf | kFlagNegInf)) == (kFlagPosInf | kFlagNegInf))
		return __builtin_nanf("");
	return (flags & kFlagPosInf) ? __builtin_inff() : -__builtin_inff();
}
// the flags of an accumulator row of n sums
__device__ __forceinline__ int *acc_flags(long long *acc, int n) { return (int *)(acc + n); }
__device__ __forceinline__ const int *acc_flags(const long long *acc, int n) { return (const int *)(acc + n); }

// ── embedding row (deq_row, reference src/nn.c:55-59) ──

__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *__restrict__ emb, int type, size_t row_bytes,
                                                    const int *__restrict__ tok, float *__restrict__ x, int D,
                                                    int vocab) {
	const int sq = blockIdx.x;
	int t = tok[sq];
	t = t < 0 ? 0 : (t >= vocab ? vocab - 1 : t);
	const uint8_t *row = emb + (size_t)t * row_bytes;
	float *y = x + (size_t)sq * D;
	if (type == HAKO_TYPE_Q6_K || type == HAKO_TYPE_Q4_K) {
		for (int c = threadIdx.x; c < D / 32; c += blockDim.x) {
			if (type == HAKO_TYPE_Q6_K)
				dq6_chunk(row, c, y);
			else
				dq4_chunk(row, c, y);
		}
	} else if (type == HAKO_TYPE_F16) {
		for (int i = threadIdx.x; i < D; i += blockDim.x) y[i] = f16_to_f32(((const uint16_t *)row)[i]);
	} else {
		for (int i = threadIdx.x; i < D; i += blockDim.x) y[i] = ((const float *)row)[i];
	}
}

// ── rmsnorm (reference src/nn.c:13-18) and the elementwise fallbacks ──

// ss over the row, scale = 1/sqrt(ss/n + eps), y = x*scale*w.
__device__ __forceinline__ float block_sum256(float v, float *red) {
	v = wave_sum(v);
	if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
	__syncthreads();
	const float t = red[0] + red[1] + red[2] + red[3];
	__syncthreads();
	return t;
}

// Rows up to kNormHoist * 256 wide take every load of the row and of w up
// front (range-checked buffer loads: past n they read zeros, which add
// nothing to ss) instead of one dependent load per loop step; a thread's
// elements are i = tid + 256 j either way, in the same order, so the sums
// and outputs are the same bits.
constexpr int kNormHoist = 32;

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                      float *__restrict__ y, int n, float eps) {
	__shared__ float red[4];
	const float *xr = x + (size_t)blockIdx.x * n;
	float *yr = y + (size_t)blockIdx.x * n;
	const int tid = threadIdx.x;
	if (n <= kNormHoist * 256) {
		const __amdgpu_buffer_rsrc_t xs = stream_rsrc(xr, (uint32_t)n * 4u), ws = stream_rsrc(w, (uint32_t)n * 4u);
		const int nj = (n + 255) >> 8;   // uniform
		float xv[kNormHoist], wv[kNormHoist];
#pragma unroll
		for (int j = 0; j < kNormHoist; j++) {
			const uint32_t off = j < nj ? 4u * (uint32_t)(tid + 256 * j) : kBufNone;
			xv[j] = ld_f32(xs, off);
			wv[j] = ld_f32(ws, off);
		}
		float ss = 0.0f;
#pragma unroll
		for (int j = 0; j < kNormHoist; j++) ss = __builtin_fmaf(xv[j], xv[j], ss);
		ss = block_sum256(ss, red);
		const float scale = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
		for (int j = 0; j < kNormHoist; j++)
			if (tid + 256 * j < n) yr[tid + 256 * j] = xv[j] * scale * wv[j];
		return;
	}
	float ss = 0.0f;
	for (int i = tid; i < n; i += 256) ss = __builtin_fmaf(xr[i], xr[i], ss);
	ss = block_sum256(ss, red);
	const float scale = 1.0f / sqrtf(ss / (float)n + eps);
	for (int i = tid; i < n; i += 256) yr[i] = xr[i] * scale * w[i];
}

// x = a + y (a may be x)
__global__ __launch_bounds__(256) void add_kernel(float *x, const float *a, const float *__restrict__ y, int n) {
	const int i = blockIdx.x * 256 + threadIdx.x;
	if (i < n) x[i] = a[i] + y[i];
}

__global__ __launch_bounds__(256) void silu_mul_kernel(float *__restrict__ h, const float *__restrict__ g,
                                                       const float *__restrict__ u, int n) {
	const int i = blockIdx.x * 256 + threadIdx.x;
	if (i < n) h[i] = silu(g[i]) * u[i];
}

// Prompt prefill, token i of a chunk at position posv[i]: its key heads
// rotated (NeoX, the rope table) and written with its value row into the
// caches, as the reference's steps 2c-2d (src/model.c:113-121) per token.
__global__ __launch_bounds__(256) void rope_append_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                          const float2 *__restrict__ rope,
                                                          const int *__restrict__ posv, float *kc, float *vc,
                                                          int KVH, int HD, int max_seq) {
	const int i = blockIdx.x, KV = KVH * HD, half = HD / 2;
	const int pos = posv[i];
	if (pos < 0 || pos >= max_seq) return;   // the host checks the room first
	const float2 *rp = rope + (size_t)pos * half;
	const float *kr = k + (size_t)i * KV;
	float *kd = kc + (size_t)pos * KV, *vd = vc + (size_t)pos * KV;
	for (int t = threadIdx.x; t < KVH * half; t += 256) {
		const int h = t / half, j = t - h * half;
		const float2 cs = rp[j];
		const float a = kr[h * HD + j], b = kr[h * HD + j + half];
		kd[h * HD + j] = a * cs.x - b * cs.y;
		kd[h * HD + j + half] = a * cs.y + b * cs.x;
	}
	for (int t = threadIdx.x; t < KV; t += 256) vd[t] = v[(size_t)i * KV + t];
}

// Batched decode, row r (token) of the residual stream x (n floats): first
// x += sum over splits of part[split][r][n] (the split partial sums of the
// matmul that feeds the residual, in split order, when part is not null),
// then rmsnorm with weight w (when w is not null), and q8_32 into xq[r][n],
// xs[r][n/32] (the activation of the next Q4_K matmuls). One workgroup of
// 1024 threads per row, a quad of the row per thread, every partial's load
// issued before any is summed; n <= 4096.
constexpr int kRowT = 1024, kRowSplits = 16;
__device__ __forceinline__ float4 load_resid_quad(float *__restrict__ xr, const float *__restrict__ part, int nsplit,
                                                  int r, int n) {
	const int e = min((int)threadIdx.x * 4, n - 4);
	float4 v = *(const float4 *)(xr + e);
	if (!part) return v;
	float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
	for (int s0 = 0; s0 < nsplit; s0 += kRowSplits) {
		float4 p[kRowSplits];
#pragma unroll
		for (int k = 0; k < kRowSplits; k++)
			if (s0 + k < nsplit) p[k] = *(const float4 *)(part + ((size_t)(s0 + k) * 16 + r) * n + e);
#pragma unroll
		for (int k = 0; k < kRowSplits; k++)
			if (s0 + k < nsplit) {
				y.x += p[k].x;
				y.y += p[k].y;
				y.z += p[k].z;
				y.w += p[k].w;
			}
	}
	v.x += y.x;
	v.y += y.y;
	v.z += y.z;
	v.w += y.w;
	if ((int)threadIdx.x * 4 < n) *(float4 *)(xr + e) = v;
	return v;
}

__device__ __forceinline__ float block_sum1024(float v, float *red) {
	v = wave_sum(v);
	if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
	__syncthreads();
	float t = 0.0f;
#pragma unroll
	for (int w = 0; w < kRowT / 64; w++) t += red[w];
	__syncthreads();
	return t;
}

__device__ __forceinline__ float4 rms_scale_quad(float4 v, const float *__restrict__ w, float eps, int n, float *red) {
	const bool on = (int)threadIdx.x * 4 < n;
	const float4 wv = *(const float4 *)(w + min((int)threadIdx.x * 4, n - 4));
	float ss = 0.0f;
	if (on) {
		ss = __builtin_fmaf(v.x, v.x, ss);
		ss = __builtin_fmaf(v.y, v.y, ss);
		ss = __builtin_fmaf(v.z, v.z, ss);
		ss = __builtin_fmaf(v.w, v.w, ss);
	}
	ss = block_sum1024(ss, red);
	const float scale = 1.0f / sqrtf(ss / (float)n + eps);
	return make_float4(v.x * scale * wv.x, v.y * scale * wv.y, v.z * scale * wv.z, v.w * scale * wv.w);
}

__global__ __launch_bounds__(kRowT) void resid_rmsnorm_q8_kernel(float *__restrict__ x, const float *__restrict__ part,
                                                                 int nsplit, const float *__restrict__ w, float eps,
                                                                 int8_t *__restrict__ xq, float *__restrict__ xs,
                                                                 int n) {
	__shared__ float red[kRowT / 64];
	const int r = blockIdx.x;
	float4 v = load_resid_quad(x + (size_t)r * n, part, nsplit, r, n);
	if (w) v = rms_scale_quad(v, w, eps, n, red);
	const int e = threadIdx.x * 4;
	float sc;
	const uint32_t packed = q8_quant4(v, sc);   // every lane takes part in the 8-lane maxima
	if (e < n) {
		*(uint32_t *)(xq + (size_t)r * n + e) = packed;
		if ((threadIdx.x & 7) == 0) xs[(size_t)r * (n >> 5) + (e >> 5)] = sc;
	}
}

// As above, then the fp16 hi/lo split of the normalized row with one power of
// two for the row (the lm_head's Q6_K activation): xh/xl[r][n], esc[r] = 2^e.
__global__ __launch_bounds__(kRowT) void resid_rmsnorm_split_kernel(float *__restrict__ x,
                                                                    const float *__restrict__ part, int nsplit,
                                                                    const float *__restrict__ w, float eps,
                                                                    _Float16 *__restrict__ xh,
                                                                    _Float16 *__restrict__ xl,
                                                                    float *__restrict__ esc, int n) {
	__shared__ float red[kRowT / 64];
	const int r = blockIdx.x;
	float4 v = load_resid_quad(x + (size_t)r * n, part, nsplit, r, n);
	v = rms_scale_quad(v, w, eps, n, red);
	const bool on = (int)threadIdx.x * 4 < n;
	float a = on ? __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(v.x), __builtin_fabsf(v.y)),
	                               __builtin_fmaxf(__builtin_fabsf(v.z), __builtin_fabsf(v.w)))
	             : 0.0f;
	a = wave_max(a);
	if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
	__syncthreads();
	a = red[0];
#pragma unroll
	for (int k = 1; k < kRowT / 64; k++) a = __builtin_fmaxf(a, red[k]);
	const int e = f16_split_exp(a);
	const float s = __builtin_ldexpf(1.0f, -e);
	if (threadIdx.x == 0) esc[r] = __builtin_ldexpf(1.0f, e);
	if (on) {
		const float f[4] = {v.x * s, v.y * s, v.z * s, v.w * s};
#pragma unroll
		for (int q = 0; q < 4; q++) {
			const _Float16 h = (_Float16)f[q];
			xh[(size_t)r * n + threadIdx.x * 4 + q] = h;
			xl[(size_t)r * n + threadIdx.x * 4 + q] = (_Float16)(f[q] - (float)h);
		}
	}
}

// ── fused Q4_K GEMV of the decode step ──

struct DecSeg {
	const uint8_t *w;    // weight rows of the segment
	const float *bias;   // F32 bias or null
	float *out;          // output rows of the segment
	int row0, rows;      // first row in the launch's row space, row count
};
struct DecSegs {
	DecSeg s[3];
	int n;
};

enum { kProQ8 = 0, kProNorm = 1 };
enum { kEpiStore = 0, kEpiAdd = 1, kEpiSwiGLU = 2 };

// Flat grid (as the standalone Q4_K GEMV): a wave owns ITEMS row items of
// rt rows, every weight load issued at once behind the activation loads, as
// raw buffer loads from the item's matrix (idle slots read nothing). Row
// space: segments one after the other (Store, Add; a wave never straddles
// two), or for SwiGLU 2F rows where a wave's even items are gate rows and
// its odd items the same up rows, so the two sums of a row meet in
// neighbouring lanes. The activation x (n_in floats) is quantized with the
// q8_32 scheme in the prologue, after rmsnorm with weight nw for kProNorm.
//
// OACC: the activation is x plus the fixed-point residual accumulator oacc
// (the output projection's sums and their non-finite flags, merge_o_kernel),
// added in the prologue; workgroup 0 stores that sum to xmid (the residual
// the down projection adds to) and clears the accumulator oacc_next (sums and
// flags) for the next layer's projection.
template <int PRO, int EPI, int XP, int ITEMS, bool OACC = false>
__global__ __launch_bounds__(256) void q4k_dec_kernel(DecSegs segs, const float *__restrict__ x,
                                                      const float *__restrict__ nw, float eps, int n_in,
                                                      int vrows, const long long *__restrict__ oacc,
                                                      float *__restrict__ xmid, long long *__restrict__ oacc_next) {
	extern __shared__ __align__(16) uint8_t smem[];
	int8_t *xq_s = (int8_t *)smem;
	float *xs_s = (float *)(smem + n_in);
	float *red_s = xs_s + (n_in >> 5);
	constexpr int T = 256, WAVES = 4;
	constexpr int NG = (ITEMS + 3) / 4;
	static_assert(EPI != kEpiSwiGLU || ITEMS % 2 == 0, "SwiGLU pairs a gate item with the next (up) item");
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int NB = n_in >> 8, C = NB * 4;
	const int seg = next_pow2(C), rt = 64 / seg;
	const int sub = lane & (seg - 1), rsub = lane / seg;
	const size_t rb = (size_t)NB * kQ4Bytes;
	const int wrow0 = (blockIdx.x * WAVES + wave) * ITEMS * rt;   // first launch row of the wave

	// this wave's segment (Store / Add)
	const int si = EPI == kEpiSwiGLU ? 0
	               : (segs.n > 2 && wrow0 >= segs.s[2].row0) ? 2
	               : (segs.n > 1 && wrow0 >= segs.s[1].row0) ? 1 : 0;
	const uint8_t *sw = si == 0 ? segs.s[0].w : (si == 1 ? segs.s[1].w : segs.s[2].w);
	const float *sbias = si == 0 ? segs.s[0].bias : (si == 1 ? segs.s[1].bias : segs.s[2].bias);
	float *sout = si == 0 ? segs.s[0].out : (si == 1 ? segs.s[1].out : segs.s[2].out);
	const int srow0 = si == 0 ? segs.s[0].row0 : (si == 1 ? segs.s[1].row0 : segs.s[2].row0);
	const int srows = si == 0 ? segs.s[0].rows : (si == 1 ? segs.s[1].rows : segs.s[2].rows);

	// item it, this lane: row of its matrix and validity (SwiGLU: item it is
	// gate (even) or up (odd) row wrow0/2 + rt*(it/2) + rsub)
	auto item_row = [&](int it) -> int {
		return EPI == kEpiSwiGLU ? (wrow0 >> 1) + rt * (it >> 1) + rsub : wrow0 + rt * it + rsub - srow0;
	};
	auto item_ok = [&](int it) -> bool {
		return EPI == kEpiSwiGLU ? item_row(it) < segs.s[0].rows
		                         : wrow0 + rt * it + rsub < vrows && item_row(it) < srows;
	};
	const uint32_t mbytes = (uint32_t)(rb * (EPI == kEpiSwiGLU ? segs.s[0].rows : srows));
	const __amdgpu_buffer_rsrc_t wra = stream_rsrc(EPI == kEpiSwiGLU ? segs.s[0].w : sw, mbytes);
	const __amdgpu_buffer_rsrc_t wrb = stream_rsrc(EPI == kEpiSwiGLU ? segs.s[1].w : sw, mbytes);

	// 1. activation (and norm weight) loads, then residual / bias, then weights
	float4 xv[XP], nv[XP];
	uint4 oa[XP][2];
	// the accumulator's non-finite flags: read by workgroup 0 alone (an empty
	// range for the others, no traffic), which stores x + o as the residual
	uint4 of[XP];
	const __amdgpu_buffer_rsrc_t fr =
	    stream_rsrc(OACC ? (const void *)acc_flags(oacc, n_in) : nullptr, (OACC && blockIdx.x == 0) ? 4u * n_in : 0u);
#pragma unroll
	for (int k = 0; k < XP; k++) {
		const int e = min((int)(threadIdx.x + k * T) * 4, n_in - 4);
		xv[k] = *(const float4 *)(x + e);
		if (PRO == kProNorm) nv[k] = *(const float4 *)(nw + e);
		if (OACC) {
			oa[k][0] = *(const uint4 *)(oacc + e);
			oa[k][1] = *(const uint4 *)(oacc + e + 2);
			of[k] = ld_b128(fr, 4u * e);
		}
	}
	float pre[NG];   // bias (Store) or the residual (Add) of the row this lane writes
	if (EPI != kEpiSwiGLU) {
#pragma unroll
		for (int g = 0; g < NG; g++) {
			const int r = min(item_row(4 * g + (sub & 3)), srows - 1);
			const float *src = EPI == kEpiAdd ? sout : (sbias ? sbias : x);
			pre[g] = src[EPI == kEpiAdd || sbias ? r : 0];
		}
	}
	__builtin_amdgcn_sched_barrier(0);
	Q4Buf buf[ITEMS];
#pragma unroll
	for (int j = 0; j < ITEMS; j++) {
		const bool on = item_ok(j) && sub < C;
		const uint32_t blk = on ? (uint32_t)((size_t)item_row(j) * rb + (size_t)(sub >> 2) * kQ4Bytes) : kBufNone;
		const __amdgpu_buffer_rsrc_t r = (EPI == kEpiSwiGLU && (j & 1)) ? wrb : wra;
		buf[j].h = ld_b128(r, blk);
		buf[j].q0 = ld_b128(r, blk + 16 + 32 * (sub & 3));
		buf[j].q1 = ld_b128(r, blk + 32 + 32 * (sub & 3));
		__builtin_amdgcn_sched_barrier(0);
	}

	// 2. prologue: (residual accumulator,) (rmsnorm and) q8_32 quantization into LDS
	// The activation is x + the finite part of o. Where o is not finite (a
	// flag), the residual x + o that workgroup 0 stores carries the NaN or
	// infinity; the activation here need not: a non-finite residual element
	// makes every later rmsnorm scale NaN or 0, so every later q8 code is 0 (the
	// reference's as well) and the logits are NaN, whatever this layer's
	// gate/up sums were.
	if (OACC) {
		auto fx = [](uint32_t lo, uint32_t hi) -> float {
			return from_fixed((long long)(((unsigned long long)hi << 32) | lo), 0);
		};
#pragma unroll
		for (int k = 0; k < XP; k++) {
			xv[k].x += fx(oa[k][0].x, oa[k][0].y);
			xv[k].y += fx(oa[k][0].z, oa[k][0].w);
			xv[k].z += fx(oa[k][1].x, oa[k][1].y);
			xv[k].w += fx(oa[k][1].z, oa[k][1].w);
		}
	}
	float scale = 1.0f;
	if (PRO == kProNorm) {
		float ss = 0.0f;
#pragma unroll
		for (int k = 0; k < XP; k++) {
			if ((int)(threadIdx.x + k * T) * 4 < n_in) {
				ss = __builtin_fmaf(xv[k].x, xv[k].x, ss);
				ss = __builtin_fmaf(xv[k].y, xv[k].y, ss);
				ss = __builtin_fmaf(xv[k].z, xv[k].z, ss);
				ss = __builtin_fmaf(xv[k].w, xv[k].w, ss);
			}
		}
		ss = wave_sum(ss);
		if (lane == 0) red_s[wave] = ss;
		__syncthreads();
		ss = red_s[0] + red_s[1] + red_s[2] + red_s[3];
		scale = 1.0f / sqrtf(ss / (float)n_in + eps);
	}
#pragma unroll
	for (int k = 0; k < XP; k++) {
		const int e = (threadIdx.x + k * T) * 4;
		float4 v = xv[k];
		if (PRO == kProNorm) {
			v.x = v.x * scale * nv[k].x;
			v.y = v.y * scale * nv[k].y;
			v.z = v.z * scale * nv[k].z;
			v.w = v.w * scale * nv[k].w;
		}
		float sc;
		const uint32_t packed = q8_quant4(v, sc);
		if (e < n_in) {
			*(uint32_t *)(xq_s + q8_lds_pos(e)) = packed;
			if ((threadIdx.x & 7) == 0) xs_s[e >> 5] = sc;
		}
	}
	if (OACC && blockIdx.x == 0) {
#pragma unroll
		for (int k = 0; k < XP; k++) {
			const int e = (threadIdx.x + k * T) * 4;
			if (e < n_in) {
				// x + o with the non-finite terms: finite + NaN or +-inf is the
				// same value however the finite part was rounded
				auto nf = [](float v, uint32_t fl) -> float { return fl ? v + from_fixed(0, (int)fl) : v; };
				const float4 xm = make_float4(nf(xv[k].x, of[k].x), nf(xv[k].y, of[k].y), nf(xv[k].z, of[k].z),
				                              nf(xv[k].w, of[k].w));
				*(float4 *)(xmid + e) = xm;
				*(uint4 *)(oacc_next + e) = make_uint4(0u, 0u, 0u, 0u);
				*(uint4 *)(oacc_next + e + 2) = make_uint4(0u, 0u, 0u, 0u);
				*(int4 *)(acc_flags(oacc_next, n_in) + e) = make_int4(0, 0, 0, 0);
			}
		}
	}
	__syncthreads();
	Q4Col col;
	q4_col(xq_s, xs_s, min(sub, C - 1), col);

	// 3. the row sums
	float rsum[4 * NG];
#pragma unroll
	for (int j = 0; j < 4 * NG; j++) {
		rsum[j] = 0.0f;
		if (j >= ITEMS) continue;
		int ia, ib;
		q4_isum(buf[j], col, ia, ib);
		const float f = q4_fold(buf[j], 16u * (sub & 1), (sub & 3) >= 2 ? ~0u : 0u, ia, ib, col);
		rsum[j] = (item_ok(j) && sub < C) ? f : 0.0f;
	}
	// 4. epilogue: lane sub = j (< 4) of each segment holds item 4g + j
#pragma unroll
	for (int g = 0; g < NG; g++) {
		const float tot = seg_sum4(rsum + 4 * g, seg, lane);
		const int j = 4 * g + (sub & 3);
		const bool writer = (sub >> 2) == 0 && j < ITEMS && item_ok(j);
		if (EPI == kEpiSwiGLU) {
			// the up sum of the same row: item j + 1, in the neighbouring lane
			const float other = dpp_f<kDppQuadSwap1>(tot);
			if (writer && (j & 1) == 0) segs.s[0].out[item_row(j)] = silu(tot) * other;
		} else if (writer) {
			sout[item_row(j)] = EPI == kEpiAdd ? pre[g] + tot : (sbias ? tot + pre[g] : tot);
		}
	}
}

// Persistent grid for the gate/up launch (rmsnorm prologue, SwiGLU
// epilogue): one workgroup of WAVES waves per CU, workgroup b owning the row
// pairs [b F / G, (b+1) F / G) of the two F-row matrices. The prologue (x plus
// the residual accumulator, rmsnorm, q8_32) runs once per workgroup instead
// of once per few rows; the waves then walk their row tiles (tile k of wave
// w: rows p0 + rt (w + WAVES k) + rsub) with kDecDepth items in flight, items
// 2k and 2k+1 the gate and up rows of tile k, so the two sums of a row meet
// in neighbouring lanes as in q4k_dec_kernel. Lane work, reductions and the
// epilogue are q4k_dec_kernel's, so h is the same bit for bit.
constexpr int kDecDepth = 4;

template <int XP, int WAVES, bool OACC>
__global__ __launch_bounds__(WAVES * kWave) void q4k_dec_gu_kernel(DecSegs segs, const float *__restrict__ x,
                                                                  const float *__restrict__ nw, float eps, int n_in,
                                                                  const long long *__restrict__ oacc,
                                                                  float *__restrict__ xmid,
                                                                  long long *__restrict__ oacc_next) {
	extern __shared__ __align__(16) uint8_t smem[];
	int8_t *xq_s = (int8_t *)smem;
	float *xs_s = (float *)(smem + n_in);
	float *red_s = xs_s + (n_in >> 5);
	constexpr int T = WAVES * kWave;
	static_assert(kDecDepth % 2 == 0, "a gate item and its up item share a group");
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int NB = n_in >> 8, C = NB * 4;
	const int seg = next_pow2(C), rt = 64 / seg;
	const int sub = lane & (seg - 1), rsub = lane / seg;
	const size_t rb = (size_t)NB * kQ4Bytes;
	const int F = segs.s[0].rows;
	const int p0 = (int)((int64_t)blockIdx.x * F / gridDim.x), p1 = (int)((int64_t)(blockIdx.x + 1) * F / gridDim.x);
	const int ntiles = (p1 - p0 + rt - 1) / rt;
	const int nit = ntiles > wave ? 2 * ((ntiles - wave + WAVES - 1) / WAVES) : 0;
	auto item_row = [&](int it) -> int { return p0 + rt * (wave + WAVES * (it >> 1)) + rsub; };
	const uint32_t mbytes = (uint32_t)(rb * F);
	const __amdgpu_buffer_rsrc_t wra = stream_rsrc(segs.s[0].w, mbytes), wrb = stream_rsrc(segs.s[1].w, mbytes);
	// item it is gate (even) or up (odd): the parity of its slot j in a group
	auto issue = [&](Q4Buf &b, int it, bool up) {
		const int row = item_row(it);
		const bool on = it < nit && row < p1 && sub < C;
		const uint32_t blk = on ? (uint32_t)((size_t)row * rb + (size_t)(sub >> 2) * kQ4Bytes) : kBufNone;
		const __amdgpu_buffer_rsrc_t r = up ? wrb : wra;
		b.h = ld_b128(r, blk);
		b.q0 = ld_b128(r, blk + 16 + 32 * (sub & 3));
		b.q1 = ld_b128(r, blk + 32 + 32 * (sub & 3));
	};

	// 1. activation, norm weight and accumulator loads, then the first items' weights
	float4 xv[XP], nv[XP];
	uint4 oa[XP][2];
	uint4 of[XP];
	const __amdgpu_buffer_rsrc_t fr =
	    stream_rsrc(OACC ? (const void *)acc_flags(oacc, n_in) : nullptr, (OACC && blockIdx.x == 0) ? 4u * n_in : 0u);
#pragma unroll
	for (int k = 0; k < XP; k++) {
		const int e = min((int)(threadIdx.x + k * T) * 4, n_in - 4);
		xv[k] = *(const float4 *)(x + e);
		nv[k] = *(const float4 *)(nw + e);
		if (OACC) {
			oa[k][0] = *(const uint4 *)(oacc + e);
			oa[k][1] = *(const uint4 *)(oacc + e + 2);
			of[k] = ld_b128(fr, 4u * e);
		}
	}
	__builtin_amdgcn_sched_barrier(0);
	Q4Buf buf[kDecDepth];
#pragma unroll
	for (int j = 0; j < kDecDepth; j++) {
		issue(buf[j], j, j & 1);
		__builtin_amdgcn_sched_barrier(0);
	}

	// 2. prologue (as q4k_dec_kernel): x + o, rmsnorm, q8_32 into LDS;
	//    workgroup 0 stores x + o and clears the next layer's accumulator
	if (OACC) {
		auto fx = [](uint32_t lo, uint32_t hi) -> float {
			return from_fixed((long long)(((unsigned long long)hi << 32) | lo), 0);
		};
#pragma unroll
		for (int k = 0; k < XP; k++) {
			xv[k].x += fx(oa[k][0].x, oa[k][0].y);
			xv[k].y += fx(oa[k][0].z, oa[k][0].w);
			xv[k].z += fx(oa[k][1].x, oa[k][1].y);
			xv[k].w += fx(oa[k][1].z, oa[k][1].w);
		}
	}
	float ss = 0.0f;
#pragma unroll
	for (int k = 0; k < XP; k++) {
		if ((int)(threadIdx.x + k * T) * 4 < n_in) {
			ss = __builtin_fmaf(xv[k].x, xv[k].x, ss);
			ss = __builtin_fmaf(xv[k].y, xv[k].y, ss);
			ss = __builtin_fmaf(xv[k].z, xv[k].z, ss);
			ss = __builtin_fmaf(xv[k].w, xv[k].w, ss);
		}
	}
	ss = wave_sum(ss);
	if (lane == 0) red_s[wave] = ss;
	__syncthreads();
	ss = red_s[0];
#pragma unroll
	for (int w = 1; w < WAVES; w++) ss += red_s[w];
	const float scale = 1.0f / sqrtf(ss / (float)n_in + eps);
#pragma unroll
	for (int k = 0; k < XP; k++) {
		const int e = (threadIdx.x + k * T) * 4;
		float4 v = xv[k];
		v.x = v.x * scale * nv[k].x;
		v.y = v.y * scale * nv[k].y;
		v.z = v.z * scale * nv[k].z;
		v.w = v.w * scale * nv[k].w;
		float sc;
		const uint32_t packed = q8_quant4(v, sc);
		if (e < n_in) {
			*(uint32_t *)(xq_s + q8_lds_pos(e)) = packed;
			if ((threadIdx.x & 7) == 0) xs_s[e >> 5] = sc;
		}
	}
	if (OACC && blockIdx.x == 0) {
#pragma unroll
		for (int k = 0; k < XP; k++) {
			const int e = (threadIdx.x + k * T) * 4;
			if (e < n_in) {
				auto nf = [](float v, uint32_t fl) -> float { return fl ? v + from_fixed(0, (int)fl) : v; };
				const float4 xm = make_float4(nf(xv[k].x, of[k].x), nf(xv[k].y, of[k].y), nf(xv[k].z, of[k].z),
				                              nf(xv[k].w, of[k].w));
				*(float4 *)(xmid + e) = xm;
				*(uint4 *)(oacc_next + e) = make_uint4(0u, 0u, 0u, 0u);
				*(uint4 *)(oacc_next + e + 2) = make_uint4(0u, 0u, 0u, 0u);
				*(int4 *)(acc_flags(oacc_next, n_in) + e) = make_int4(0, 0, 0, 0);
			}
		}
	}
	__syncthreads();
	Q4Col col;
	q4_col(xq_s, xs_s, min(sub, C - 1), col);

	// 3. groups of kDecDepth items: consume each slot, reload it with the item
	//    kDecDepth later, then the group's SwiGLU rows
	float *h = segs.s[0].out;
	for (int base = 0; base < nit; base += kDecDepth) {
		float rsum[kDecDepth];
#pragma unroll
		for (int j = 0; j < kDecDepth; j++) {
			const int it = base + j;
			float f = 0.0f;
			if (it < nit) {
				int ia, ib;
				q4_isum(buf[j], col, ia, ib);
				f = q4_fold(buf[j], 16u * (sub & 1), (sub & 3) >= 2 ? ~0u : 0u, ia, ib, col);
			}
			issue(buf[j], it + kDecDepth, j & 1);
			__builtin_amdgcn_sched_barrier(0);
			rsum[j] = (it < nit && item_row(it) < p1 && sub < C) ? f : 0.0f;
		}
		const float tot = seg_sum4(rsum, seg, lane);
		const int j = sub & 3;
		// the up sum of the same row: item j + 1, in the neighbouring lane
		const float other = dpp_f<kDppQuadSwap1>(tot);
		if ((sub >> 2) == 0 && (j & 1) == 0 && base + j < nit && item_row(base + j) < p1)
			h[item_row(base + j)] = silu(tot) * other;
	}
}

// ── attention (reference src/model.c:105-137) ──

// Workgroup (chunk c x head part hg, KV head kvh, sequence sq) of 256
// threads: positions [64c, 64c+64) up to pos, for the group's query heads
// of part hg (hsplit parts: a small grid splits a group's heads over several
// workgroups, which read the same keys and values). Every key and value load of the chunk is issued
// first (thread = position x every fourth float4 of the head dims for keys,
// value dims x 16-position group for values), so the chunk costs one memory
// latency. The
// group's query heads are rotated into LDS (NeoX, the rope table holding
// cos/sin of pos*theta^(-2i/hd)); the workgroup whose chunk holds pos also
// rotates the new key, appends it and the new value to the caches and uses
// them from LDS. Scores, chunk-local softmax (max m, sum l) and the weighted
// value sum o go to `part` for attn_merge_kernel. Without APPEND (prompt
// prefill) the rotated key and the value at pos are already in the caches
// and are read like every other position.
template <int HD, bool APPEND>
__global__ __launch_bounds__(256) void attn_kernel(const float *__restrict__ qkv, const float2 *__restrict__ rope,
                                                   float *kc, float *vc, const int *__restrict__ posv,
                                                   float *part, int H, int KVH,
                                                   int max_seq, int max_chunks, size_t kv_seq_stride,
                                                   int qkv_stride, float scale, int hsplit) {
	constexpr int HALF = HD / 2;
	constexpr int REC = HD + 2;      // partial record: o[HD], m, l
	constexpr int KQ = HD / 16;      // float4 of a key row per thread (4 threads per position)
	constexpr int DV = HD / 64;      // value dims per thread
	constexpr int PG = 16;           // positions per value group (4 groups)
	constexpr int QR = HD;           // query row in LDS
	// LDS: the rotated queries and the scores are dead once the value sums are
	// in registers; their space then holds the four groups' value sums.
	constexpr int QS = kMaxG * QR, SS = kMaxG * kChunk, OS = 4 * kMaxG * HD;
	__shared__ __align__(16) float u_s[QS + SS > OS ? QS + SS : OS];
	float *q_s = u_s;                // [kMaxG][QR]
	float *s_s = u_s + QS;           // [kMaxG][kChunk]: scores, then e^(score - m)
	float *o_s = u_s;                // [4][kMaxG][HD]: value sums per position group
	__shared__ float ml_s[kMaxG][2];
	__shared__ float kn_s[HD], vn_s[HD];
	// block b -> chunk c, head part hg with b % 8 = c % 8: a chunk's parts run
	// on one XCD (workgroups go to the XCDs round robin) and share its L2
	const int hb = blockIdx.x >> 3;
	const int c = (hb / hsplit) * 8 + (blockIdx.x & 7), hg = hb % hsplit, kvh = blockIdx.y, sq = blockIdx.z;
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: value rows in SGPRs
	const int GA = H / KVH, KV = KVH * HD, D = H * HD;
	// this workgroup's query heads of the group: g0 + [0, G)
	const int GH = (GA + hsplit - 1) / hsplit, g0 = hg * GH, G = min(GH, GA - g0);
	if (G <= 0) return;
	const int pos = posv[sq];
	if (pos < 0 || pos >= max_seq) return;   // no room left: the host refuses such steps
	const int nact = pos / kChunk + 1;
	if (c >= nact) return;
	const bool has_pos = APPEND && c == nact - 1;
	const bool writer = has_pos && hg == 0;   // appends the new key and value
	const float *q = qkv + (size_t)sq * qkv_stride;
	float *kcs = kc + (size_t)sq * kv_seq_stride + kvh * HD;
	float *vcs = vc + (size_t)sq * kv_seq_stride + kvh * HD;
	// 1. the query rows, their rope factors and (chunk holding pos) the new
	//    key and value first: the rotation below waits for these only
	const float2 *rp = rope + (size_t)pos * HALF;
	constexpr int QI = (kMaxG * HALF + 255) / 256;   // rotation items per thread
	float qa[QI], qb[QI];
	float2 qcs[QI];
#pragma unroll
	for (int r = 0; r < QI; r++) {
		const int t = min(tid + 256 * r, G * HALF - 1);
		const int g = t / HALF, i = t - g * HALF;
		qcs[r] = rp[i];
		qa[r] = q[(kvh * GA + g0 + g) * HD + i];
		qb[r] = q[(kvh * GA + g0 + g) * HD + i + HALF];
	}
	float na = 0.0f, nb = 0.0f, nv = 0.0f;
	float2 ncs = {0.0f, 0.0f};
	if (has_pos) {
		if (tid < HALF) {
			ncs = rp[tid];
			na = q[D + kvh * HD + tid];
			nb = q[D + kvh * HD + tid + HALF];
		}
		if (tid < HD) nv = q[D + KV + kvh * HD + tid];
	}
	__builtin_amdgcn_sched_barrier(0);

	// 2. every key, then every value load of the chunk (rows past pos read
	//    row pos: in bounds, discarded): raw buffer loads over this
	//    sequence's layer cache. Keys: load j of the position's four threads
	//    reads float4s kq + 4j, so the four cover 64 contiguous bytes and two
	//    consecutive loads whole cache lines. Values: one lane offset plus a
	//    wave-uniform row offset. The scores wait for the keys only.
	const uint32_t cache_bytes = (uint32_t)((size_t)max_seq * KV * 4);
	const __amdgpu_buffer_rsrc_t krs = stream_rsrc(kc + (size_t)sq * kv_seq_stride, cache_bytes);
	const __amdgpu_buffer_rsrc_t vrs = stream_rsrc(vc + (size_t)sq * kv_seq_stride, cache_bytes);
	const int kp = tid >> 2, kq = tid & 3;
	const int ks = c * kChunk + kp;
	const uint32_t koff = ((uint32_t)min(ks, pos) * KV + kvh * HD + 4 * kq) * 4u;
	float4 kr[KQ];
#pragma unroll
	for (int j = 0; j < KQ; j++) kr[j] = __builtin_bit_cast(float4, ld_b128(krs, koff + 64u * j));
	__builtin_amdgcn_sched_barrier(0);
	const int vd = DV * lane, vg = wave;
	const uint32_t voff = (uint32_t)(kvh * HD + vd) * 4u;
	float vr[PG][DV];
#pragma unroll
	for (int j = 0; j < PG; j++) {
		const int row = min(c * kChunk + PG * vg + j, pos);
		const int soff = row * KV * 4;
		if (DV == 2) {
			const float2 t = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(vrs, (int)voff, soff, 0));
			vr[j][0] = t.x;
			vr[j][DV - 1] = t.y;
		} else {
			vr[j][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(vrs, (int)voff, soff, 0));
		}
	}
	__builtin_amdgcn_sched_barrier(0);

	// 3. rotated query heads (and the new key, value) into LDS; the new key
	//    and value appended to the caches
#pragma unroll
	for (int r = 0; r < QI; r++) {
		const int t = tid + 256 * r;
		if (t < G * HALF) {
			const int g = t / HALF, i = t - g * HALF;
			q_s[g * QR + i] = qa[r] * qcs[r].x - qb[r] * qcs[r].y;
			q_s[g * QR + i + HALF] = qa[r] * qcs[r].y + qb[r] * qcs[r].x;
		}
	}
	if (has_pos) {
		if (tid < HALF) {
			const float k0 = na * ncs.x - nb * ncs.y, k1 = na * ncs.y + nb * ncs.x;
			kn_s[tid] = k0;
			kn_s[tid + HALF] = k1;
			if (writer) {
				kcs[(size_t)pos * KV + tid] = k0;
				kcs[(size_t)pos * KV + tid + HALF] = k1;
			}
		}
		if (tid < HD) {
			vn_s[tid] = nv;
			if (writer) vcs[(size_t)pos * KV + tid] = nv;
		}
	}
	__syncthreads();

	// rows past pos carry weight 0; zero them too, so no stale value reaches a sum
#pragma unroll
	for (int j = 0; j < PG; j++)
		if (c * kChunk + PG * vg + j > pos)
#pragma unroll
			for (int u = 0; u < DV; u++) vr[j][u] = 0.0f;

	// 3. scores: 4 threads per position, every fourth float4 of the dims each
	if (APPEND && ks == pos) {
#pragma unroll
		for (int j = 0; j < KQ; j++) kr[j] = *(const float4 *)(kn_s + 4 * kq + 16 * j);
	}
#pragma unroll
	for (int g = 0; g < kMaxG; g++) {
		if (g < G) {
			float a = 0.0f;
			const float *qg = q_s + g * QR + 4 * kq;
#pragma unroll
			for (int j = 0; j < KQ; j++) {
				const float4 qv = *(const float4 *)(qg + 16 * j);
				a = __builtin_fmaf(qv.x, kr[j].x, a);
				a = __builtin_fmaf(qv.y, kr[j].y, a);
				a = __builtin_fmaf(qv.z, kr[j].z, a);
				a = __builtin_fmaf(qv.w, kr[j].w, a);
			}
			a += dpp_f<kDppQuadSwap1>(a);
			a += dpp_f<kDppQuadSwap2>(a);
			if (kq == 0) s_s[g * kChunk + kp] = ks <= pos ? a * scale : -INFINITY;
		}
	}
	__syncthreads();

	// 4. chunk-local softmax: wave w takes heads w, w+4
#pragma unroll
	for (int h = 0; h < kMaxG / 4; h++) {
		const int g = wave + 4 * h;
		if (g < G) {
			const float v = s_s[g * kChunk + lane];
			const float m = wave_max(v);
			const float e = v == -INFINITY ? 0.0f : expf(v - m);
			const float l = wave_sum(e);
			s_s[g * kChunk + lane] = e;
			if (lane == 0) {
				ml_s[g][0] = m;
				ml_s[g][1] = l;
			}
		}
	}
	__syncthreads();

	// 5. weighted values over this thread's 16 positions (kept in registers
	//    until every wave is done with the scores), then over the 4 groups
	if (has_pos) {
		const int j = pos - c * kChunk - PG * vg;
		if (j >= 0 && j < PG) {
#pragma unroll
			for (int jj = 0; jj < PG; jj++)
				if (jj == j)
#pragma unroll
					for (int u = 0; u < DV; u++) vr[jj][u] = vn_s[vd + u];
		}
	}
	float o[kMaxG][DV];
#pragma unroll
	for (int g = 0; g < kMaxG; g++) {
#pragma unroll
		for (int u = 0; u < DV; u++) o[g][u] = 0.0f;
		if (g < G) {
#pragma unroll
			for (int j = 0; j < PG; j++) {
				const float w = s_s[g * kChunk + PG * vg + j];
#pragma unroll
				for (int u = 0; u < DV; u++) o[g][u] = __builtin_fmaf(w, vr[j][u], o[g][u]);
			}
		}
	}
	__syncthreads();   // scores consumed: their space takes the value sums
#pragma unroll
	for (int g = 0; g < kMaxG; g++)
		if (g < G)
#pragma unroll
			for (int u = 0; u < DV; u++) o_s[(vg * kMaxG + g) * HD + vd + u] = o[g][u];
	__syncthreads();
	float *rec0 = part + (((size_t)(sq * KVH + kvh) * max_chunks + c) * kMaxG + g0) * REC;
	for (int t = tid; t < G * HD; t += 256) {
		const int g = t / HD, d = t - g * HD;
		rec0[(size_t)g * REC + d] = o_s[(0 * kMaxG + g) * HD + d] + o_s[(1 * kMaxG + g) * HD + d] +
		                            o_s[(2 * kMaxG + g) * HD + d] + o_s[(3 * kMaxG + g) * HD + d];
	}
	if (tid < G) {
		rec0[(size_t)tid * REC + HD] = ml_s[tid][0];
		rec0[(size_t)tid * REC + HD + 1] = ml_s[tid][1];
	}
}

// Prompt pass on the matrix cores, for passes whose tokens all lie below
// kFlashPos cache positions (every key of a token in one workgroup): workgroup
// (query head, 16·QG-token tile) of 2·QG waves, wave w taking the 16 query
// tokens 16(w%QG).. and key half w/QG of every chunk. A tile's work grows
// with its last position, so the grid runs the last tiles first, and
// 32-token tiles (QG 2, two workgroups per CU) spread the longest tiles'
// keys over twice the CUs of 64-token ones: 7B 512-token prompt, attention
// 51.3 -> 39.2 us per layer (16-token tiles: slower again, each chunk staged
// for fewer queries). The outputs do not depend on QG. The tile's rotated query rows
// are staged through LDS into registers once; then per 64-key chunk (keys and
// values staged in LDS, rows 132 floats apart) each wave forms its half of
// S^T = K Q^T with v_mfma_f32_16x16x4_f32 (2 key tiles x 32 steps, lane l's
// steps taking dims 32(l/16) + s), masks keys past each token's position,
// keeps its own running max and sum per token (online softmax, -inf scores
// weigh 0), and adds V^T P^T into its O^T (8 dim tiles x 8 steps; step
// (t, v) is keys 16t + 4k + v for lane group k, which is where the S^T
// layout left p, and tile dt row i is dim 8i + dt). The two halves of a
// token meet once at the end (max, rescaled sums and outputs through LDS);
// O / sum goes to att and, with xq, each lane's 32 dims (one whole 32-block)
// to q8_32. The math is the reference's (src/model.c:123-142: scores,
// softmax, weighted values) in fp32 with a different order of additions.
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kFlashPos = 512;   // positions a pass may reach for this kernel
constexpr int kFlashQG = 2;      // query groups of 16 tokens per workgroup
constexpr int kFlashRow = 132;   // floats per staged key / value / query row
template <int QG>
__global__ __launch_bounds__(128 * QG, 1) void attn_flash_kernel(const float *__restrict__ q_all,
                                                            const float2 *__restrict__ rope,
                                                            const float *__restrict__ kc, const float *__restrict__ vc,
                                                            const int *__restrict__ posv, float *__restrict__ att,
                                                            int8_t *__restrict__ xq, float *__restrict__ xs, int H,
                                                            int KVH, int max_seq, int ntok, float scale) {
	constexpr int HD = 128, HALF = 64, NT = 128 * QG, QT = 16 * QG;   // threads, query tokens per tile
	// keys of the chunk (first: the tile's queries), then its values; at the
	// end the combine area of the key halves (QG x 64 lanes x 34 floats)
	__shared__ __align__(16) float kv_s[2 * 64 * kFlashRow];
	float *k_s = kv_s, *v_s = kv_s + 64 * kFlashRow;
	static_assert(QG * 64 * 34 <= 2 * 64 * kFlashRow, "combine area inside the chunk rows");
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int qg = wave % QG, kh = wave / QG;   // query group, key half
	const int qi = lane & 15, kg = lane >> 4;
	// grid (head, tile): the last tiles, whose tokens see the most keys, first
	const int ntile = (ntok + QT - 1) / QT;
	const int t0 = (ntile - 1 - (int)blockIdx.y) * QT, h = blockIdx.x, kvh = h / (H / KVH);
	const int KV = KVH * HD, D = H * HD;
	const int tq = t0 + 16 * qg + qi;   // this lane's query token
	int pos_q = tq < ntok ? posv[tq] : -1;
	pos_q = pos_q < max_seq ? pos_q : -1;
	const int plast = posv[min(t0 + QT - 1, ntok - 1)];   // positions rise with the token
	if (plast < 0 || plast >= max_seq) return;        // the host refuses such passes
	const int nch = plast / 64 + 1;

	// 1. the tile's rotated query rows (NeoX rope at each token's position) into k_s
#pragma unroll 4
	for (int r = 0; r < QT * HALF / NT; r++) {
		const int e = tid + NT * r, i = e >> 6, p = e & 63;
		const int tok = min(t0 + i, ntok - 1);
		const int pos = min(max(posv[tok], 0), max_seq - 1);
		const float *q = q_all + (size_t)tok * D + h * HD;
		const float a = q[p], b = q[p + HALF];
		const float2 cs = rope[(size_t)pos * HALF + p];
		k_s[i * kFlashRow + p] = a * cs.x - b * cs.y;
		k_s[i * kFlashRow + p + HALF] = a * cs.y + b * cs.x;
	}
	__syncthreads();
	float qv[32];   // Q[query qi][32 kg + s]
	{
		const float *src = k_s + (16 * qg + qi) * kFlashRow + 32 * kg;
#pragma unroll
		for (int i = 0; i < 8; i++) {
			const float4 t = *(const float4 *)(src + 4 * i);
			qv[4 * i] = t.x; qv[4 * i + 1] = t.y; qv[4 * i + 2] = t.z; qv[4 * i + 3] = t.w;
		}
	}
	__syncthreads();   // the query rows are in registers: k_s takes the keys

	const uint32_t cache_bytes = (uint32_t)((size_t)max_seq * KV * 4);
	const __amdgpu_buffer_rsrc_t krs = stream_rsrc(kc, cache_bytes), vrs = stream_rsrc(vc, cache_bytes);
	v4f acco[8];
#pragma unroll
	for (int dt = 0; dt < 8; dt++) acco[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
	float m_run = -INFINITY, l_run = 0.0f;
	const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
	for (int c = 0; c < nch; c++) {
		// 2. the chunk's keys and values (rows past the tile's last position
		//    read that row: in bounds, masked below)
#pragma unroll
		for (int r = 0; r < 64 * 32 / NT; r++) {
			const int e = tid + NT * r, row = e >> 5, f = e & 31;
			const int key = min(64 * c + row, plast);
			const uint32_t off = ((uint32_t)key * KV + kvh * HD + 4 * f) * 4u;
			*(float4 *)(k_s + row * kFlashRow + 4 * f) = __builtin_bit_cast(float4, ld_b128(krs, off));
			*(float4 *)(v_s + row * kFlashRow + 4 * f) = __builtin_bit_cast(float4, ld_b128(vrs, off));
		}
		__syncthreads();
		// 3. this wave's S^T tiles: keys 32kh + 16t + 4kg + v, query qi
		v4f sc[2];
#pragma unroll
		for (int t = 0; t < 2; t++) {
			v4f a = zero;
			const float *kr = k_s + (32 * kh + 16 * t + qi) * kFlashRow + 32 * kg;
#pragma unroll
			for (int i = 0; i < 8; i++) {
				const float4 kv = *(const float4 *)(kr + 4 * i);
				a = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qv[4 * i], a, 0, 0, 0);
				a = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qv[4 * i + 1], a, 0, 0, 0);
				a = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qv[4 * i + 2], a, 0, 0, 0);
				a = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qv[4 * i + 3], a, 0, 0, 0);
			}
			sc[t] = a;
		}
		// 4. online softmax of query qi over this half's 32 keys (lanes qi,
		//    qi+16, qi+32, qi+48 of the wave)
		float mc = -INFINITY;
#pragma unroll
		for (int t = 0; t < 2; t++)
#pragma unroll
			for (int v = 0; v < 4; v++) {
				const int key = 64 * c + 32 * kh + 16 * t + 4 * kg + v;
				sc[t][v] = key <= pos_q ? sc[t][v] * scale : -INFINITY;
				mc = __builtin_fmaxf(mc, sc[t][v]);
			}
		mc = __builtin_fmaxf(mc, __shfl_xor(mc, 16));
		mc = __builtin_fmaxf(mc, __shfl_xor(mc, 32));
		const float m_new = __builtin_fmaxf(m_run, mc);
		const float alpha = m_run == -INFINITY ? 0.0f : expf(m_run - m_new);
		float ps = 0.0f;
#pragma unroll
		for (int t = 0; t < 2; t++)
#pragma unroll
			for (int v = 0; v < 4; v++) {
				const float p = sc[t][v] == -INFINITY ? 0.0f : expf(sc[t][v] - m_new);
				sc[t][v] = p;
				ps += p;
			}
		ps += __shfl_xor(ps, 16);
		ps += __shfl_xor(ps, 32);
		l_run = l_run * alpha + ps;
		m_run = m_new;
#pragma unroll
		for (int dt = 0; dt < 8; dt++)
#pragma unroll
			for (int v = 0; v < 4; v++) acco[dt][v] *= alpha;
		// 5. O^T += V^T P^T: step (t, v) = keys 32kh + 16t + 4kg + v, tile dt row i = dim 8i + dt
#pragma unroll
		for (int t = 0; t < 2; t++)
#pragma unroll
			for (int v = 0; v < 4; v++) {
				const float *vr = v_s + (32 * kh + 16 * t + 4 * kg + v) * kFlashRow + 8 * qi;
				const float4 va = *(const float4 *)vr, vb = *(const float4 *)(vr + 4);
				const float vv[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
				for (int dt = 0; dt < 8; dt++)
					acco[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[dt], sc[t][v], acco[dt], 0, 0, 0);
			}
		__syncthreads();   // before the next chunk's rows land (and, last, before the combine)
	}
	// 6. the two key halves of each token: half 1 hands (m, l, O) to half 0
	//    through LDS (the chunk rows are free)
	float *x_s = kv_s + (size_t)(qg * 64 + lane) * 34;
	if (kh == 1) {
#pragma unroll
		for (int dt = 0; dt < 8; dt++)
#pragma unroll
			for (int v = 0; v < 4; v++) x_s[4 * dt + v] = acco[dt][v];
		x_s[32] = m_run;
		x_s[33] = l_run;
	}
	__syncthreads();
	if (kh == 1 || tq >= ntok || pos_q < 0) return;
	const float m1 = x_s[32], l1 = x_s[33];
	const float m = __builtin_fmaxf(m_run, m1);
	const float a0 = m_run == -INFINITY ? 0.0f : expf(m_run - m), a1 = m1 == -INFINITY ? 0.0f : expf(m1 - m);
	const float inv_l = 1.0f / (l_run * a0 + l1 * a1);
	// this lane holds dims 32kg + 8v + dt of query qi (one 32-block)
	float o[32];
#pragma unroll
	for (int v = 0; v < 4; v++)
#pragma unroll
		for (int dt = 0; dt < 8; dt++) o[8 * v + dt] = (acco[dt][v] * a0 + x_s[4 * dt + v] * a1) * inv_l;
	const size_t ob = (size_t)tq * D + h * HD + 32 * kg;
#pragma unroll
	for (int i = 0; i < 8; i++) *(float4 *)(att + ob + 4 * i) = make_float4(o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]);
	if (xq) {
		float amax = 0.0f;
#pragma unroll
		for (int i = 0; i < 32; i++) amax = __builtin_fmaxf(amax, __builtin_fabsf(ftz(o[i])));
		const float s = q8_xs(amax), inv = q8_inv(amax, s);
		uint32_t pk[8];
#pragma unroll
		for (int i = 0; i < 8; i++)
			pk[i] = q8_code(ftz(o[4 * i]), inv) | (q8_code(ftz(o[4 * i + 1]), inv) << 8) |
			        (q8_code(ftz(o[4 * i + 2]), inv) << 16) | (q8_code(ftz(o[4 * i + 3]), inv) << 24);
		*(uint4 *)(xq + ob) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
		*(uint4 *)(xq + ob + 16) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
		xs[ob >> 5] = s;
	}
}

// The merge of one query head's chunk records by the HD threads of its waves
// (waves hw0 .. hw0 + HD/64 - 1 of the workgroup; thread ht = value dim):
// M = max m_c, weights e^(m_c - M) / L with L = sum l_c e^(m_c - M), output
// sum over chunks of weight * o_c, in chunk order. grp: the head's record of
// chunk 0 (chunk c at grp + c * kMaxG * (HD + 2)); nact chunks; r_s and ws
// (HD floats) are this head's LDS. Every thread of the workgroup calls it
// with the same nact (it holds barriers).
template <int HD>
__device__ __forceinline__ float merge_head(const float *__restrict__ grp, int nact, int ht, int lane, int wave,
                                            int hw0, float (*r_s)[4], float *ws) {
	constexpr int REC = HD + 2, NWH = HD / 64;
	constexpr int OB = 32;                       // o rows in flight per thread
	constexpr size_t CS = (size_t)kMaxG * REC;   // floats between two chunks' records of one head
	// one round trip for the common case (nact <= HD chunks): every thread's
	// (m, l) of chunk ht and its value dim of the first OB chunks, issued together
	float m0 = -INFINITY, l0 = 0.0f;
	if (ht < nact) {
		m0 = grp[ht * CS + HD];
		l0 = grp[ht * CS + HD + 1];
	}
	float ov[OB];
#pragma unroll
	for (int j = 0; j < OB; j++) ov[j] = j < nact ? grp[j * CS + ht] : 0.0f;
	float mx = m0;
	for (int cc = ht + HD; cc < nact; cc += HD) mx = __builtin_fmaxf(mx, grp[cc * CS + HD]);
	mx = wave_max(mx);
	if (lane == 0) r_s[0][wave] = mx;
	__syncthreads();
	mx = r_s[0][hw0];
#pragma unroll
	for (int w = 1; w < NWH; w++) mx = __builtin_fmaxf(mx, r_s[0][hw0 + w]);
	float lsum = ht < nact ? l0 * expf(m0 - mx) : 0.0f;
	for (int cc = ht + HD; cc < nact; cc += HD) lsum += grp[cc * CS + HD + 1] * expf(grp[cc * CS + HD] - mx);
	lsum = wave_sum(lsum);
	if (lane == 0) r_s[1][wave] = lsum;
	__syncthreads();
	lsum = r_s[1][hw0];
#pragma unroll
	for (int w = 1; w < NWH; w++) lsum += r_s[1][hw0 + w];
	const float inv = 1.0f / lsum;
	float acc = 0.0f;
	for (int c0 = 0; c0 < nact; c0 += HD) {
		const int nc = min(HD, nact - c0);
		if (c0) __syncthreads();   // ws of the previous batch is consumed
		if (ht < nc) ws[ht] = expf((c0 ? grp[(c0 + ht) * CS + HD] : m0) - mx) * inv;
		__syncthreads();
		const float *r = grp + c0 * CS + ht;
		int cc = 0;
		if (c0 == 0) {
#pragma unroll
			for (int j = 0; j < OB; j++)
				if (j < nc) acc = __builtin_fmaf(ov[j], ws[j], acc);
			cc = min(OB, nc);
		}
		for (; cc + OB <= nc; cc += OB) {
			float o[OB];
#pragma unroll
			for (int j = 0; j < OB; j++) o[j] = r[(cc + j) * CS];
#pragma unroll
			for (int j = 0; j < OB; j++) acc = __builtin_fmaf(o[j], ws[cc + j], acc);
		}
		for (; cc < nc; cc++) acc = __builtin_fmaf(r[cc * CS], ws[cc], acc);
	}
	return acc;
}

// q8_32 code of this lane's value a, the 32-block being the lanes of equal
// lane / 32; sc = the block's scale (quantize_row_q8_32, src/quant.c:127-144).
__device__ __forceinline__ int8_t q8_lane32(float a, float &sc) {
	a = ftz(a);
	float amax = __builtin_fabsf(a);
#pragma unroll
	for (int k = 1; k < 32; k <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, k));
	sc = q8_xs(amax);
	return (int8_t)q8_code(a, q8_inv(amax, sc));
}

// Grid (G, n_kv_heads, n_seq), HD threads: query head kvh*G + g of sequence
// sq from its chunks' records (merge_head). A launch of its own: the records of every chunk's workgroup are
// visible at the kernel boundary, with no fence per workgroup. When xq is not
// null the head's outputs are also quantized (q8_32: a head holds whole
// 32-blocks) into xq[sq][H*HD] and xs[sq][H*HD/32], the activation of the
// batched output projection.
template <int HD>
__global__ __launch_bounds__(HD) void attn_merge_kernel(const float *__restrict__ part, const int *__restrict__ posv,
                                                        float *__restrict__ att, int8_t *__restrict__ xq,
                                                        float *__restrict__ xs, int H, int KVH, int max_seq,
                                                        int max_chunks) {
	constexpr int REC = HD + 2;
	__shared__ float w_s[HD];
	__shared__ float r_s[2][4];
	const int g = blockIdx.x, kvh = blockIdx.y, sq = blockIdx.z, tid = threadIdx.x;
	const int G = H / KVH;
	const int pos = posv[sq];
	if (pos < 0 || pos >= max_seq) return;
	const float *grp = part + ((size_t)(sq * KVH + kvh) * max_chunks * kMaxG + g) * REC;
	const float acc = merge_head<HD>(grp, pos / kChunk + 1, tid, tid & 63, tid >> 6, 0, r_s, w_s);
	const size_t o = (size_t)sq * H * HD + (size_t)(kvh * G + g) * HD + tid;
	att[o] = acc;
	if (xq) {
		float sc;
		xq[o] = q8_lane32(acc, sc);
		if ((tid & 31) == 0) xs[o >> 5] = sc;
	}
}

// One sequence: the merge above and the output projection (Q4_K) in one
// launch. Grid (D/256 input blocks, D/64 row chunks), 256 threads: workgroup
// (b, rc) merges the 256/HD query heads whose outputs are input block b of
// the projection (thread t: head 256b/HD + t/HD, dim t % HD, merge_head),
// quantizes them with q8_32 (a block holds whole 32-blocks, so the codes and
// scales are those of the full row), and adds block b's terms of q4k_vec_dot
// (its eight sub-blocks, reference src/quant.c:150-232) for the 64 rows of
// chunk rc to the fixed-point accumulator oacc (zero before the launch) with
// an integer atomic add: the D/256 block sums of a row meet in an order-free
// sum, which the next kernel adds to the residual stream.
template <int HD, int RI>
__global__ __launch_bounds__(256) void merge_o_kernel(const float *__restrict__ part, const int *__restrict__ posv,
                                                      const uint8_t *__restrict__ wo, long long *__restrict__ oacc,
                                                      int H, int KVH, int max_seq, int max_chunks, int D) {
	__shared__ float w_s[256];
	__shared__ float r_s[2][4];
	__shared__ __align__(16) int8_t xq_s[256];
	__shared__ __align__(16) float xs_s[8];
	const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int pos = posv[0];
	if (pos < 0 || pos >= max_seq) return;

	// 1. this lane's weights: rows 64*RI*rc + 64*i + 16*wave + lane/4 (i < RI),
	//    64-weight group g of block b
	const int g = lane & 3;
	const uint32_t rb = (uint32_t)(D / kQK) * kQ4Bytes;
	const __amdgpu_buffer_rsrc_t wr = stream_rsrc(wo, (uint32_t)D * rb);
	int rows[RI];
	Q4Buf wb[RI];
#pragma unroll
	for (int i = 0; i < RI; i++) {
		rows[i] = blockIdx.y * 64 * RI + 64 * i + 16 * wave + (lane >> 2);
		const uint32_t bo = rows[i] < D ? (uint32_t)rows[i] * rb + (uint32_t)b * kQ4Bytes : kBufNone;
		wb[i].h = ld_b128(wr, bo);
		wb[i].q0 = ld_b128(wr, bo + 16 + 32 * g);
		wb[i].q1 = ld_b128(wr, bo + 32 + 32 * g);
	}
	__builtin_amdgcn_sched_barrier(0);

	// 2. merge of head hh (kvh = hh / G, g = hh % G), HD threads per head
	const int hs = tid / HD, hh = b * (256 / HD) + hs, G = H / KVH;
	const float *grp = part + ((size_t)(hh / G) * max_chunks * kMaxG + hh % G) * (HD + 2);
	const float acc =
	    merge_head<HD>(grp, pos / kChunk + 1, tid % HD, lane, wave, hs * (HD / 64), r_s, w_s + hs * HD);

	// 3. q8_32 of the block's 256 outputs (32 lanes per 32-block)
	{
		float sc;
		xq_s[q8_lds_pos(tid)] = q8_lane32(acc, sc);
		if ((tid & 31) == 0) xs_s[tid >> 5] = sc;
	}
	__syncthreads();

	// 4. block b's terms of the lane's rows, each row's four lanes summed, one atomic add per row
	Q4Col col;
	q4_col(xq_s, xs_s, g, col);
#pragma unroll
	for (int i = 0; i < RI; i++) {
		int ia, ib;
		q4_isum(wb[i], col, ia, ib);
		float f = q4_fold(wb[i], 16u * (g & 1), g >= 2 ? ~0u : 0u, ia, ib, col);
		f += __shfl_xor(f, 1);
		f += __shfl_xor(f, 2);
		if (g == 0 && rows[i] < D) {
			__hip_atomic_fetch_add(oacc + rows[i], to_fixed(f), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
			if (const int fl = fixed_flag(f))
				__hip_atomic_fetch_or(acc_flags(oacc, D) + rows[i], fl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
		}
	}
}

// x += the fixed-point accumulator oacc (with its flags), which is then
// cleared (the merged output projection's residual add when no fused gate/up
// kernel takes it), and oacc_next cleared for the next layer.
__global__ __launch_bounds__(256) void oacc_apply_kernel(float *__restrict__ x, long long *__restrict__ oacc,
                                                         long long *__restrict__ oacc_next, int n) {
	const int i = blockIdx.x * 256 + threadIdx.x;
	if (i < n) {
		x[i] += from_fixed(oacc[i], acc_flags(oacc, n)[i]);
		oacc[i] = 0;
		acc_flags(oacc, n)[i] = 0;
		oacc_next[i] = 0;
		acc_flags(oacc_next, n)[i] = 0;
	}
}

// ── greedy pick (reference src/sample.c:28-32) ──

// (value, index) order: larger value first, then lower index (the reference's
// ascending scan with a strict >); NaN never wins.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
	if (v != v) return false;
	if (bv != bv) return true;
	return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void argmax_wave(float &v, int &i) {
#pragma unroll
	for (int off = 1; off < 64; off <<= 1) {
		const float ov = __shfl_xor(v, off);
		const int oi = __shfl_xor(i, off);
		if (better(ov, oi, v, i)) {
			v = ov;
			i = oi;
		}
	}
}

// Grid (kArgBlocks, n_seq): each block's best (value, index) of its slice.
__global__ __launch_bounds__(256) void argmax_part_kernel(const float *__restrict__ logits, int V,
                                                          float2 *__restrict__ part) {
	__shared__ float bv_s[4];
	__shared__ int bi_s[4];
	const int b = blockIdx.x, sq = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const float *lg = logits + (size_t)sq * V;
	const int i0 = (int)((int64_t)b * V / kArgBlocks), i1 = (int)((int64_t)(b + 1) * V / kArgBlocks);
	float bv = NAN;
	int bi = 0x7FFFFFFF;
	if (i1 - i0 <= kArgHoist * 256) {
		// every load of the slice up front (past i1 a range-checked load reads
		// a value no index takes), then the same comparisons in the same order
		const __amdgpu_buffer_rsrc_t ls = stream_rsrc(lg + i0, (uint32_t)(i1 - i0) * 4u);
		float lv[kArgHoist];
#pragma unroll
		for (int j = 0; j < kArgHoist; j++) {
			const int i = i0 + threadIdx.x + 256 * j;
			lv[j] = ld_f32(ls, i < i1 ? 4u * (uint32_t)(i - i0) : kBufNone);
		}
#pragma unroll
		for (int j = 0; j < kArgHoist; j++) {
			const int i = i0 + threadIdx.x + 256 * j;
			if (i < i1 && better(lv[j], i, bv, bi)) {
				bv = lv[j];
				bi = i;
			}
		}
	} else {
		for (int i = i0 + threadIdx.x; i < i1; i += 256)
			if (better(lg[i], i, bv, bi)) {
				bv = lg[i];
				bi = i;
			}
	}
	argmax_wave(bv, bi);
	if (lane == 0) {
		bv_s[wave] = bv;
		bi_s[wave] = bi;
	}
	__syncthreads();
	if (threadIdx.x == 0) {
		for (int w = 1; w < 4; w++)
			if (better(bv_s[w], bi_s[w], bv, bi)) {
				bv = bv_s[w];
				bi = bi_s[w];
			}
		part[sq * kArgBlocks + b] = make_float2(bv, __builtin_bit_cast(float, bi));
	}
}

// Grid (n_seq), one wave: the token of the blocks' best, appended to the ring;
// the position advances. The reference's scan starts from logits[0] and
// only a strictly larger value replaces it, so a NaN at index 0 is never
// replaced (src/sample.c:28-31): token 0 then, whatever follows.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float2 *__restrict__ part,
                                                          const float *__restrict__ logits, int V, int *tok,
                                                          int *posv, int *ring, int ring_len, int *nout) {
	const int sq = blockIdx.x, lane = threadIdx.x;
	const float2 p = part[sq * kArgBlocks + lane];
	const float l0 = logits[(size_t)sq * V];
	float v = p.x;
	int i = __builtin_bit_cast(int, p.y);
	argmax_wave(v, i);
	if (lane == 0) {
		const int t = (i == 0x7FFFFFFF || l0 != l0) ? 0 : i;   // all NaN, or NaN first: index 0
		tok[sq] = t;
		const int n = nout[sq];
		if (n < ring_len) ring[(size_t)sq * ring_len + n] = t;
		nout[sq] = n + 1;
		posv[sq] += 1;
	}
}

size_t row_bytes(int type, int n) {
	switch (type) {
	case HAKO_TYPE_Q4_K: return (size_t)n / kQK * kQ4Bytes;
	case HAKO_TYPE_Q6_K: return (size_t)n / kQK * kQ6Bytes;
	case HAKO_TYPE_F16: return (size_t)n * 2;
	case HAKO_TYPE_F32: return (size_t)n * 4;
	default: return 0;
	}
}

bool known_type(int t) {
	return t == HAKO_TYPE_Q4_K || t == HAKO_TYPE_Q6_K || t == HAKO_TYPE_F16 || t == HAKO_TYPE_F32;
}

}  // namespace

void dec_set_gu_items(int v) { g_dec_gu_items = (v == 4 || v == 8) ? v : 0; }
void dec_set_gu_grid(int v) { g_dec_gu_grid = (v == 1 || v == 2) ? v : 0; }
void dec_set_merge_rows(int v) { g_dec_merge_rows = (v == 64 || v == 128) ? v : 0; }
void dec_set_qkv_items(int v) { g_dec_qkv_items = (v == 2 || v == 4 || v == 8) ? v : 0; }
void dec_set_attn_parts(int v) { g_dec_attn_parts = v > 0 && v <= 8 ? v : 0; }

}  // namespace hako

using namespace hako;

struct hako_gpu_decoder {
	hako_gpu_model m{};
	std::vector<hako_gpu_block> blocks;
	int n_seq = 0, max_seq = 0, max_chunks = 0, kv_dim = 0, qkv_dim = 0;
	// device state
	float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *h = nullptr, *g = nullptr, *u = nullptr,
	      *tmp = nullptr, *logits = nullptr, *part = nullptr, *kc = nullptr, *vc = nullptr;
	float2 *rope = nullptr, *apart = nullptr;
	int *tok = nullptr, *pos = nullptr, *ring = nullptr, *nout = nullptr;
	// one sequence: the output projection's fixed-point residual accumulators
	// (three: by layer parity, and the last layer of an odd count; then one
	// scratch row) and the residual after it (x + o)
	long long *oacc = nullptr;
	float *xa = nullptr;
	// batched steps (n_seq > 1): q8 and fp16 hi/lo activations, split-K state
	int8_t *xq = nullptr;
	float *xs = nullptr, *esc = nullptr, *escb = nullptr, *skpart = nullptr;
	size_t skpart_floats = 0;   // capacity of skpart
	_Float16 *xh = nullptr, *xl = nullptr;
	// prompt prefill (allocated on first use): chunk activations and records
	float *pf_x = nullptr, *pf_xn = nullptr, *pf_q = nullptr, *pf_k = nullptr, *pf_v = nullptr, *pf_att = nullptr,
	      *pf_tmp = nullptr, *pf_g = nullptr, *pf_u = nullptr, *pf_part = nullptr;
	int8_t *pf_xq = nullptr;                    // q8 rows [chunk][max(d_model, ffn)] and their scales
	float *pf_xs = nullptr, *pf_esc = nullptr;  // fp16 split of the SwiGLU rows: hi, lo [chunk][ffn], esc[chunk]
	_Float16 *pf_xh = nullptr, *pf_xl = nullptr;
	float *pf_sk = nullptr;   // stream-K slots of the down matmul
	size_t pf_sk_floats = 0;
	int *pf_tok = nullptr, *pf_pos = nullptr;
	int pf_chunk = 0;   // most tokens per prefill pass
	size_t pf_part_bytes = 0;   // capacity of pf_part
	std::vector<void *> allocs;
	hipGraphExec_t exec = nullptr;
	hipGraph_t graph = nullptr;
	void (*on_destroy)(void *) = nullptr;   // hako_gpu_decoder_on_destroy
	void *on_destroy_arg = nullptr;
};

namespace {

int dalloc(hako_gpu_decoder *d, size_t bytes, void **p) {
	if (hipMalloc(p, bytes < 256 ? 256 : bytes) != hipSuccess) {
		(void)hipGetLastError();
		return set_error(HAKO_GPU_ENOMEM, "decoder allocation of %zu bytes", bytes);
	}
	d->allocs.push_back(*p);
	return HAKO_GPU_OK;
}

// Launch helpers of the fused Q4_K GEMV: XP activation quads per thread.
// With oacc the activation is x + oacc (OACC prologue; see q4k_dec_kernel).
template <int PRO, int EPI, int IT = kDecItems>
int launch_dec(const DecSegs &segs, const float *x, const float *nw, float eps, int n_in, int vrows,
               const long long *oacc = nullptr, float *xmid = nullptr, long long *oacc_next = nullptr) {
	const int C = n_in / kQK * 4;
	const int rt = 64 / next_pow2(C);
	const int rows_wg = 4 * IT * rt;
	for (int i = 0; i < segs.n; i++)   // weights are read through 32-bit buffer offsets
		if ((size_t)segs.s[i].rows * (n_in / kQK) * kQ4Bytes >= kBufNone)
			return set_error(HAKO_GPU_EINVAL, "fused Q4_K GEMV segment of %d x %d exceeds 2 GiB", segs.s[i].rows, n_in);
	const int wgs = (vrows + rows_wg - 1) / rows_wg;
	const size_t lds = (size_t)n_in + (size_t)(n_in / 32) * 4 + 16;
	const int xp = (n_in + 1023) / 1024;
#define HK_DEC(XP, OA) \
	hipLaunchKernelGGL((q4k_dec_kernel<PRO, EPI, XP, IT, OA>), dim3(wgs), dim3(256), lds, stream(), segs, x, nw, eps, \
	                   n_in, vrows, oacc, xmid, oacc_next)
	if constexpr (PRO == kProNorm && EPI == kEpiSwiGLU) {
		if (oacc) {
			if (xp <= 1) HK_DEC(1, true);
			else if (xp <= 2) HK_DEC(2, true);
			else HK_DEC(4, true);
			HK_LAUNCHED("q4k_dec");
			return HAKO_GPU_OK;
		}
	}
	if (oacc) return set_error(HAKO_GPU_EINVAL, "the residual accumulator rides on the gate/up launch");
	{
		if (xp <= 1) HK_DEC(1, false);
		else if (xp <= 2) HK_DEC(2, false);
		else HK_DEC(4, false);
	}
#undef HK_DEC
	HK_LAUNCHED("q4k_dec");
	return HAKO_GPU_OK;
}

// The gate/up launch on the persistent grid (q4k_dec_gu_kernel): one
// workgroup of four waves per CU. segs: gate (out = h) and up, F rows each.
int launch_dec_gu(const DecSegs &segs, const float *x, const float *nw, float eps, int n_in,
                  const long long *oacc = nullptr, float *xmid = nullptr, long long *oacc_next = nullptr) {
	constexpr int W = 4;
	const int F = segs.s[0].rows, rt = 64 / next_pow2(n_in / kQK * 4);
	if ((size_t)F * (n_in / kQK) * kQ4Bytes >= kBufNone)
		return set_error(HAKO_GPU_EINVAL, "fused Q4_K GEMV segment of %d x %d exceeds 2 GiB", F, n_in);
	int wgs = cu_count();
	const int tiles = (F + rt - 1) / rt;
	if (wgs > tiles) wgs = tiles;
	const size_t lds = (size_t)n_in + (size_t)(n_in / 32) * 4 + 4 * W + 16;
	const int xp = (n_in + 4 * W * 64 - 1) / (4 * W * 64);
#define HK_DGU(XP, OA) \
	hipLaunchKernelGGL((q4k_dec_gu_kernel<XP, W, OA>), dim3(wgs), dim3(W * kWave), lds, stream(), segs, x, nw, eps, n_in, \
	                   oacc, xmid, oacc_next)
	if (oacc) {
		if (xp <= 1) HK_DGU(1, true);
		else if (xp <= 2) HK_DGU(2, true);
		else HK_DGU(4, true);
	} else {
		if (xp <= 1) HK_DGU(1, false);
		else if (xp <= 2) HK_DGU(2, false);
		else HK_DGU(4, false);
	}
#undef HK_DGU
	HK_LAUNCHED("q4k_dec_gu");
	return HAKO_GPU_OK;
}

// rows per wave of the fused GEMV at this n_in (segment starts must be multiples)
int dec_rows_per_wave(int n_in, int items = kDecItems) { return items * (64 / next_pow2(n_in / kQK * 4)); }

bool fusable_q4(int n_in) { return n_in % kQK == 0 && n_in / kQK * 4 <= 64; }

int rmsnorm(const float *x, const float *w, float *y, int n, float eps, int rows) {
	hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, stream(), x, w, y, n, eps);
	HK_LAUNCHED("rmsnorm");
	return HAKO_GPU_OK;
}

// rmsnorm (weight w) and q8_32 of `rows` rows of x (n floats, n <= 4096) into
// xq[rows][n], xs[rows][n/32]: the activation of multi-token Q4_K matmuls.
int rmsnorm_q8_rows(const float *x, const float *w, float eps, int8_t *xq, float *xs, int n, int rows) {
	hipLaunchKernelGGL(resid_rmsnorm_q8_kernel, dim3(rows), dim3(kRowT), 0, stream(), const_cast<float *>(x), nullptr,
	                   0, w, eps, xq, xs, n);
	HK_LAUNCHED("rmsnorm_q8");
	return HAKO_GPU_OK;
}

// x = a + y (a may be x)
int add(float *x, const float *a, const float *y, int n) {
	hipLaunchKernelGGL(add_kernel, dim3((n + 255) / 256), dim3(256), 0, stream(), x, a, y, n);
	HK_LAUNCHED("add");
	return HAKO_GPU_OK;
}

// Attention of layer l for every sequence: chunk records, then their merge
// (which also writes the q8 rows of the output to mxq/mxs when not null).
int attention(hako_gpu_decoder *d, int l, int8_t *mxq = nullptr, float *mxs = nullptr, bool merge = true) {
	const hako_gpu_model &m = d->m;
	const int KV = d->kv_dim, HD = m.head_dim, G = m.n_heads / m.n_kv_heads;
	const float scale = 1.0f / sqrtf((float)HD);
	const size_t kv_seq_stride = (size_t)m.n_layers * d->max_seq * KV;
	float *kcl = d->kc + (size_t)l * d->max_seq * KV, *vcl = d->vc + (size_t)l * d->max_seq * KV;
	// one sequence: a grid of chunks x KV heads leaves most CUs idle, so each
	// group's query heads are split over (up to) four workgroups (3B decode at
	// position 1024: 1374 / 1322 / 1304 / 1362 us per token for 1 / 2 / 4 / 8
	// parts). Seven heads per group (7B) take two parts of 4 and 3 heads: four
	// parts of 2, 2, 2, 1 measured 1554 against 1543 us per token, three 1562,
	// seven 1568. (16 sequences: two parts per group made the 7B step 4% slower.)
	const int parts = g_dec_attn_parts ? g_dec_attn_parts : (G == 7 ? 2 : 4);
	const int hsplit = d->n_seq == 1 ? (G < parts ? G : parts) : 1;
	const dim3 ag((d->max_chunks + 7) / 8 * 8 * hsplit, m.n_kv_heads, d->n_seq), mg(G, m.n_kv_heads, d->n_seq);
	if (HD == 128) {
		hipLaunchKernelGGL((attn_kernel<128, true>), ag, dim3(256), 0, stream(), d->qkv, d->rope, kcl, vcl, d->pos, d->part,
		                   m.n_heads, m.n_kv_heads, d->max_seq, d->max_chunks, kv_seq_stride, d->qkv_dim, scale,
		                   hsplit);
		HK_LAUNCHED("attention");
		if (!merge) return HAKO_GPU_OK;
		hipLaunchKernelGGL(attn_merge_kernel<128>, mg, dim3(128), 0, stream(), d->part, d->pos, d->att, mxq, mxs,
		                   m.n_heads, m.n_kv_heads, d->max_seq, d->max_chunks);
	} else {
		hipLaunchKernelGGL((attn_kernel<64, true>), ag, dim3(256), 0, stream(), d->qkv, d->rope, kcl, vcl, d->pos, d->part,
		                   m.n_heads, m.n_kv_heads, d->max_seq, d->max_chunks, kv_seq_stride, d->qkv_dim, scale,
		                   hsplit);
		HK_LAUNCHED("attention");
		if (!merge) return HAKO_GPU_OK;
		hipLaunchKernelGGL(attn_merge_kernel<64>, mg, dim3(64), 0, stream(), d->part, d->pos, d->att, mxq, mxs,
		                   m.n_heads, m.n_kv_heads, d->max_seq, d->max_chunks);
	}
	HK_LAUNCHED("attention merge");
	return HAKO_GPU_OK;
}

int argmax(hako_gpu_decoder *d) {
	hipLaunchKernelGGL(argmax_part_kernel, dim3(kArgBlocks, d->n_seq), dim3(256), 0, stream(), d->logits, d->m.vocab,
	                   d->apart);
	HK_LAUNCHED("argmax");
	hipLaunchKernelGGL(argmax_final_kernel, dim3(d->n_seq), dim3(64), 0, stream(), d->apart, d->logits, d->m.vocab,
	                   d->tok, d->pos, d->ring, d->max_seq, d->nout);
	HK_LAUNCHED("argmax final");
	return HAKO_GPU_OK;
}

// x += the pending split partials (part, nsplit; none when part is null),
// then rmsnorm (w) and q8 rows of x into d->xq / d->xs.
int resid_rmsnorm_q8(hako_gpu_decoder *d, const float *part, int nsplit, const float *w, int n) {
	hipLaunchKernelGGL(resid_rmsnorm_q8_kernel, dim3(d->n_seq), dim3(kRowT), 0, stream(), d->x, part, nsplit, w,
	                   d->m.rms_eps, d->xq, d->xs, n);
	HK_LAUNCHED("resid_rmsnorm_q8");
	return HAKO_GPU_OK;
}

// A layer of the batched step runs fused (the row kernels, q/k/v as one
// skinny launch over three segments, the o and down sums left for the next
// row kernel) when it has the Q4_K_M mix — Q4_K q/k/v/o/gate/up, Q6_K down —
// and d_model <= 4096 (a quad per thread of a 1024-thread workgroup in the
// row kernels), with d_model and kv_dim multiples of 16 (skinny row segments
// start on 16-row boundaries). Any other layer runs generic: one launch per
// matmul and elementwise launches, as the reference's forward
// (src/model.c:102-157) for each sequence.
bool batched_dims_ok(const hako_gpu_model &m, int kv_dim) {
	return kv_dim % 16 == 0 && m.d_model % 16 == 0 && m.d_model <= 4 * kRowT;
}
bool batched_fused_layer(const hako_gpu_model &m, const hako_gpu_block &B, int kv_dim) {
	return batched_dims_ok(m, kv_dim) && B.t_q == HAKO_TYPE_Q4_K && B.t_k == HAKO_TYPE_Q4_K &&
	       B.t_v == HAKO_TYPE_Q4_K && B.t_o == HAKO_TYPE_Q4_K && B.t_gate == HAKO_TYPE_Q4_K &&
	       B.t_up == HAKO_TYPE_Q4_K && B.t_down == HAKO_TYPE_Q6_K;
}

// One matmul of the batched step outside the fused layers, for every
// sequence: y[t * ldy + r] = (W x_t)[r] (+ bias[r]) for t < n_seq, x rows of
// n_in floats. Q4_K: the q8_32 rows in d->xq / d->xs and the skinny int8
// kernel; Q6_K: the fp16 hi/lo rows in d->xh / d->xl and the skinny fp16
// kernel; F16 / F32: one dense GEMV per sequence. Split sums go to the
// decoder's skpart (sized for these shapes when the decoder is created).
int batch_matmul(hako_gpu_decoder *d, float *y, int ldy, const float *x, int type, const void *w,
                 const float *bias, int n_out, int n_in) {
	const int M = d->n_seq;
	SkSegs s{};
	s.n = 1;
	s.s[0] = {(const uint8_t *)w, bias, y, 0, n_out, ldy};
	switch (type) {
	case HAKO_TYPE_Q4_K:
		if (int rc = hako_gpu_quantize_q8_32(x, M, n_in, d->xq, d->xs)) return rc;
		return q4k_skinny(s, kSkStore, d->xq, d->xs, M, n_in, n_out, d->skpart, d->skpart_floats);
	case HAKO_TYPE_Q6_K:
		if (int rc = f16_split(x, d->xh, d->xl, d->esc, M, n_in)) return rc;
		return q6k_skinny(s, kSkStore, d->xh, d->xl, d->esc, M, n_in, n_out, d->skpart, d->skpart_floats);
	default:
		for (int t = 0; t < M; t++)
			if (int rc = hako_gpu_dense_gemv(y + (size_t)t * ldy, type, w, x + (size_t)t * n_in, bias, n_out, n_in))
				return rc;
		return HAKO_GPU_OK;
	}
}

// Split floats the batched step's matmuls need in skpart: the fused layers'
// launches and every generic matmul shape (either quantized type).
size_t batched_part_floats(const hako_gpu_model &m, int kv_dim) {
	const int D = m.d_model, F = m.ffn_dim, qkv_rows = D + 2 * kv_dim;
	size_t need = 0;
	auto take = [&](size_t v) { need = v > need ? v : need; };
	if (batched_dims_ok(m, kv_dim)) {
		take(q4k_skinny_part_floats(D, qkv_rows, kSkStore));
		take(q4k_skinny_part_floats(D, D, kSkPart));
		take(q4k_skinny_part_floats(D, 2 * F, kSkPart));
		take(q6k_skinny_part_floats(F, D, kSkPart));
	}
	const int shapes[6][2] = {{D, D}, {D, kv_dim}, {D, F}, {F, D}, {D, m.vocab}, {D, qkv_rows}};
	for (const auto &sh : shapes) {
		take(q4k_skinny_part_floats(sh[0], sh[1], kSkStore));
		take(q6k_skinny_part_floats(sh[0], sh[1], kSkStore));
	}
	return need;
}

// One step of n_seq > 1 sequences. Fused layers: every matmul a skinny MFMA
// GEMM that streams the weights once for all sequences; the o and down
// matmuls leave their split partial sums for the next kernel, which adds
// them to the residual stream on its way (rmsnorm + q8, or the lm_head's
// split); the gate/up sums go straight into the fp16 form of the down
// matmul. Generic layers first add any pending partials to the residual.
int enqueue_batched_step(hako_gpu_decoder *d) {
	const hako_gpu_model &m = d->m;
	const int D = m.d_model, F = m.ffn_dim, KV = d->kv_dim, M = d->n_seq;
	hipLaunchKernelGGL(embed_kernel, dim3(M), dim3(256), 0, stream(), (const uint8_t *)m.tok_embd, m.t_embd,
	                   row_bytes(m.t_embd, D), d->tok, d->x, D, m.vocab);
	HK_LAUNCHED("embed");
	const bool dims_ok = batched_dims_ok(m, KV);
	const int ns_o = dims_ok ? q4k_skinny_splits(D, D) : 0, ns_gu = dims_ok ? q4k_skinny_splits(D, 2 * F) : 0;
	const int ns_down = dims_ok ? q6k_skinny_splits(F, D) : 0;
	const float *pend = nullptr;   // the previous fused down matmul's partials
	int pend_ns = 0;
	for (int l = 0; l < m.n_layers; l++) {
		const hako_gpu_block &B = d->blocks[l];
		if (!batched_fused_layer(m, B, KV)) {
			// generic layer (x holds the residual of every sequence)
			if (pend) {
				if (int rc = resid_rmsnorm_q8(d, pend, pend_ns, nullptr, D)) return rc;
				pend = nullptr;
			}
			if (int rc = rmsnorm(d->x, B.attn_norm, d->xn, D, m.rms_eps, M)) return rc;
			if (int rc = batch_matmul(d, d->qkv, d->qkv_dim, d->xn, B.t_q, B.wq, B.bq, D, D)) return rc;
			if (int rc = batch_matmul(d, d->qkv + D, d->qkv_dim, d->xn, B.t_k, B.wk, B.bk, KV, D)) return rc;
			if (int rc = batch_matmul(d, d->qkv + D + KV, d->qkv_dim, d->xn, B.t_v, B.wv, B.bv, KV, D)) return rc;
			if (int rc = attention(d, l)) return rc;
			if (int rc = batch_matmul(d, d->tmp, D, d->att, B.t_o, B.wo, nullptr, D, D)) return rc;
			if (int rc = add(d->x, d->x, d->tmp, M * D)) return rc;
			if (int rc = rmsnorm(d->x, B.ffn_norm, d->xn, D, m.rms_eps, M)) return rc;
			if (int rc = batch_matmul(d, d->g, F, d->xn, B.t_gate, B.gate, nullptr, F, D)) return rc;
			if (int rc = batch_matmul(d, d->u, F, d->xn, B.t_up, B.up, nullptr, F, D)) return rc;
			hipLaunchKernelGGL(silu_mul_kernel, dim3((M * F + 255) / 256), dim3(256), 0, stream(), d->h, d->g, d->u,
			                   M * F);
			HK_LAUNCHED("silu_mul");
			if (int rc = batch_matmul(d, d->tmp, D, d->h, B.t_down, B.down, nullptr, D, F)) return rc;
			if (int rc = add(d->x, d->x, d->tmp, M * D)) return rc;
			continue;
		}
		// 1. residual, rmsnorm, q8; q, k, v: rows [q | k | v] of qkv[t][D + 2KV]
		if (int rc = resid_rmsnorm_q8(d, pend, pend_ns, B.attn_norm, D)) return rc;
		SkSegs s{};
		s.n = 3;
		s.s[0] = {(const uint8_t *)B.wq, B.bq, d->qkv, 0, D, d->qkv_dim};
		s.s[1] = {(const uint8_t *)B.wk, B.bk, d->qkv + D, D, KV, d->qkv_dim};
		s.s[2] = {(const uint8_t *)B.wv, B.bv, d->qkv + D + KV, D + KV, KV, d->qkv_dim};
		if (int rc = q4k_skinny(s, kSkStore, d->xq, d->xs, M, D, D + 2 * KV, d->skpart, d->skpart_floats)) return rc;
		// 2. attention, one grid over every sequence; q8 rows of its output
		if (int rc = attention(d, l, d->xq, d->xs)) return rc;
		// 3. output projection: partials, added to the residual by step 4
		s = SkSegs{};
		s.n = 1;
		s.s[0] = {(const uint8_t *)B.wo, nullptr, d->x, 0, D, D};
		if (int rc = q4k_skinny(s, kSkPart, d->xq, d->xs, M, D, D, d->skpart, d->skpart_floats)) return rc;
		// 4. residual, rmsnorm, q8; gate and up partials
		if (int rc = resid_rmsnorm_q8(d, d->skpart, ns_o, B.ffn_norm, D)) return rc;
		s = SkSegs{};
		s.n = 2;
		s.s[0] = {(const uint8_t *)B.gate, nullptr, d->h, 0, F, F};
		s.s[1] = {(const uint8_t *)B.up, nullptr, d->h, F, F, F};
		if (int rc = q4k_skinny(s, kSkPart, d->xq, d->xs, M, D, 2 * F, d->skpart, d->skpart_floats)) return rc;
		// 5. SwiGLU of the gate/up partials, straight to the down matmul's fp16
		//    hi/lo rows with a power of two per 256-row block
		if (int rc = swiglu_split(d->skpart, ns_gu, F, M, d->xh, d->xl, d->escb)) return rc;
		// 6. down projection: partials, added to the residual by the next kernel
		s = SkSegs{};
		s.n = 1;
		s.s[0] = {(const uint8_t *)B.down, nullptr, d->x, 0, D, D};
		if (int rc = q6k_skinny(s, kSkPart, d->xh, d->xl, d->escb, M, F, D, d->skpart, d->skpart_floats, true))
			return rc;
		pend = d->skpart;
		pend_ns = ns_down;
	}
	SkSegs s{};
	s.n = 1;
	s.s[0] = {(const uint8_t *)m.out_weight, nullptr, d->logits, 0, m.vocab, m.vocab};
	if (dims_ok && m.t_out == HAKO_TYPE_Q4_K) {
		if (int rc = resid_rmsnorm_q8(d, pend, pend_ns, m.out_norm, D)) return rc;
		if (int rc = q4k_skinny(s, kSkStore, d->xq, d->xs, M, D, m.vocab, d->skpart, d->skpart_floats)) return rc;
	} else if (dims_ok && m.t_out == HAKO_TYPE_Q6_K) {
		hipLaunchKernelGGL(resid_rmsnorm_split_kernel, dim3(M), dim3(kRowT), 0, stream(), d->x, pend, pend_ns,
		                   m.out_norm, m.rms_eps, d->xh, d->xl, d->esc, D);
		HK_LAUNCHED("resid_rmsnorm_split");
		if (int rc = q6k_skinny(s, kSkStore, d->xh, d->xl, d->esc, M, D, m.vocab, d->skpart, d->skpart_floats)) return rc;
	} else {
		if (pend)
			if (int rc = resid_rmsnorm_q8(d, pend, pend_ns, nullptr, D)) return rc;
		if (int rc = rmsnorm(d->x, m.out_norm, d->xn, D, m.rms_eps, M)) return rc;
		if (int rc = batch_matmul(d, d->logits, m.vocab, d->xn, m.t_out, m.out_weight, nullptr, m.vocab, D)) return rc;
	}
	if (int rc = argmax(d)) return rc;
	return HAKO_GPU_OK;
}

// int64 words of one accumulator row: D sums and D int32 flags
size_t acc_row(int D) { return (size_t)D + (size_t)D / 2; }

// The attention merge joins the Q4_K output projection of one sequence
// (merge_o_kernel) when every layer's projection can take it: each merged
// layer clears the accumulator the next layer adds into, so a layer that
// does not merge would leave the one after it a stale sum.
bool merge_o_all(const hako_gpu_model &m, const std::vector<hako_gpu_block> &blocks) {
	if (m.d_model % kQK || kQK % m.head_dim || m.d_model / kQK > kFixMaxBlocks) return false;
	for (const hako_gpu_block &B : blocks)
		if (B.t_o != HAKO_TYPE_Q4_K) return false;
	return true;
}

// One decode step on the library stream (n_seq == 1).
int enqueue_step(hako_gpu_decoder *d) {
	if (d->n_seq > 1) return enqueue_batched_step(d);
	const hako_gpu_model &m = d->m;
	const int D = m.d_model, F = m.ffn_dim, KV = d->kv_dim;
	const bool merge_o = merge_o_all(m, d->blocks);
	hipLaunchKernelGGL(embed_kernel, dim3(d->n_seq), dim3(256), 0, stream(), (const uint8_t *)m.tok_embd, m.t_embd,
	                   row_bytes(m.t_embd, D), d->tok, d->x, D, m.vocab);
	HK_LAUNCHED("embed");
	for (int l = 0; l < m.n_layers; l++) {
		const hako_gpu_block &B = d->blocks[l];
		float *q = d->qkv, *k = d->qkv + D, *v = d->qkv + D + KV;
		// 1. q, k, v
		// row items per wave: 2, or 8 past d_model 2048 (fewer workgroups, each
		// repeating the rmsnorm prologue: 7B step 1569 -> 1556 us; 4 items
		// 1569, 16 items 1626; at 3B 2 items, 1120 against 1127 / 1181 with 4 / 8)
		const bool qkv8 = D > 2048 && D % dec_rows_per_wave(D, 8) == 0 && KV % dec_rows_per_wave(D, 8) == 0;
		const int qkv_items = g_dec_qkv_items ? g_dec_qkv_items : (qkv8 ? 8 : kDecItemsQkv);
		const int rpw = dec_rows_per_wave(D, qkv_items);
		if (B.t_q == HAKO_TYPE_Q4_K && B.t_k == HAKO_TYPE_Q4_K && B.t_v == HAKO_TYPE_Q4_K && fusable_q4(D) &&
		    D % rpw == 0 && KV % rpw == 0) {
			DecSegs s{};
			s.n = 3;
			s.s[0] = {(const uint8_t *)B.wq, B.bq, q, 0, D};
			s.s[1] = {(const uint8_t *)B.wk, B.bk, k, D, KV};
			s.s[2] = {(const uint8_t *)B.wv, B.bv, v, D + KV, KV};
			const int vr = D + 2 * KV;
			if (int rc = qkv_items == 8   ? launch_dec<kProNorm, kEpiStore, 8>(s, d->x, B.attn_norm, m.rms_eps, D, vr)
			             : qkv_items == 4 ? launch_dec<kProNorm, kEpiStore, 4>(s, d->x, B.attn_norm, m.rms_eps, D, vr)
			                              : launch_dec<kProNorm, kEpiStore, kDecItemsQkv>(s, d->x, B.attn_norm,
			                                                                              m.rms_eps, D, vr))
				return rc;
		} else {
			if (int rc = rmsnorm(d->x, B.attn_norm, d->xn, D, m.rms_eps, 1)) return rc;
			if (int rc = hako_gpu_matmul(q, d->xn, B.t_q, B.wq, B.bq, D, D)) return rc;
			if (int rc = hako_gpu_matmul(k, d->xn, B.t_k, B.wk, B.bk, KV, D)) return rc;
			if (int rc = hako_gpu_matmul(v, d->xn, B.t_v, B.wv, B.bv, KV, D)) return rc;
		}
		// 2. rope, cache append, attention; 3. output projection + residual
		// (merged with the attention records in one launch for Q4_K, its sums
		// into the fixed-point accumulator of this layer, taken up by the
		// gate/up kernel's prologue or by oacc_apply_kernel)
		const bool fused_gu = B.t_gate == HAKO_TYPE_Q4_K && B.t_up == HAKO_TYPE_Q4_K && fusable_q4(D);
		// accumulators alternate by layer; with an odd layer count the last
		// layer takes a third, so that it differs from the next step's layer 0
		// (one layer: the same one, cleared by a launch of its own below).
		// Each merged layer clears the next layer's accumulator, so the merge
		// is taken for all layers or none (merge_o_all).
		auto acc_of = [&](int layer) -> long long * {
			const int i = (m.n_layers & 1) && layer == m.n_layers - 1 && m.n_layers > 1 ? 2 : (layer & 1);
			return d->oacc + (size_t)i * acc_row(D);
		};
		long long *oacc = acc_of(l);
		long long *oacc_next = acc_of(l + 1 == m.n_layers ? 0 : l + 1);
		const bool self_next = oacc_next == oacc;
		if (int rc = attention(d, l, nullptr, nullptr, !merge_o)) return rc;
		if (merge_o) {
			// rows per workgroup: 64, or 128 by shape past d_model 2048 (each
			// workgroup merges its heads' chunk records once for twice the rows:
			// 7B step 1589 -> 1566 us; at 3B, 256 workgroups of 64 rows leave
			// none idle and 128 rows measured 1120 -> 1141 us); the same bits
			const int ri = (g_dec_merge_rows ? g_dec_merge_rows == 128 : D > 2048) ? 2 : 1;
			const dim3 grid(D / kQK, (D + 64 * ri - 1) / (64 * ri));
			if (m.head_dim == 128)
				hipLaunchKernelGGL((ri == 2 ? merge_o_kernel<128, 2> : merge_o_kernel<128, 1>), grid, dim3(256), 0,
				                   stream(), d->part, d->pos, (const uint8_t *)B.wo, oacc, m.n_heads, m.n_kv_heads,
				                   d->max_seq, d->max_chunks, D);
			else
				hipLaunchKernelGGL((ri == 2 ? merge_o_kernel<64, 2> : merge_o_kernel<64, 1>), grid, dim3(256), 0,
				                   stream(), d->part, d->pos, (const uint8_t *)B.wo, oacc, m.n_heads, m.n_kv_heads,
				                   d->max_seq, d->max_chunks, D);
			HK_LAUNCHED("attention merge + o");
			if (!fused_gu) {
				hipLaunchKernelGGL(oacc_apply_kernel, dim3((D + 255) / 256), dim3(256), 0, stream(), d->x, oacc,
				                   oacc_next, D);
				HK_LAUNCHED("residual accumulator");
			}
		} else if (B.t_o == HAKO_TYPE_Q4_K && fusable_q4(D) && D % dec_rows_per_wave(D) == 0) {
			DecSegs s{};
			s.n = 1;
			s.s[0] = {(const uint8_t *)B.wo, nullptr, d->x, 0, D};
			if (int rc = launch_dec<kProQ8, kEpiAdd>(s, d->att, nullptr, 0.0f, D, D)) return rc;
		} else {
			if (int rc = hako_gpu_matmul(d->tmp, d->att, B.t_o, B.wo, nullptr, D, D)) return rc;
			if (int rc = add(d->x, d->x, d->tmp, D)) return rc;
		}
		// 4. gate, up, SwiGLU (after merge_o: on x + the accumulator, that sum
		// kept in xa as the residual of step 5)
		const float *resid = d->x;
		const int gu_items = g_dec_gu_items ? g_dec_gu_items : (D > 2048 ? 8 : kDecItems);
		// the persistent grid by shape (its prologue once per workgroup: 7B
		// step 1665 -> 1571 us, 3B 1138 -> 1117.5 us, the same bits)
		const bool gu_persist = g_dec_gu_grid != 1;
		if (fused_gu) {
			DecSegs s{};
			s.n = 2;
			s.s[0] = {(const uint8_t *)B.gate, nullptr, d->h, 0, F};
			s.s[1] = {(const uint8_t *)B.up, nullptr, d->h, 0, F};
			if (merge_o) {
				// (a workgroup must not clear what the others still read)
				long long *on = self_next ? d->oacc + (size_t)3 * acc_row(D) : oacc_next;
				if (int rc = gu_persist ? launch_dec_gu(s, d->x, B.ffn_norm, m.rms_eps, D, oacc, d->xa, on)
				             : gu_items == 8
				                 ? launch_dec<kProNorm, kEpiSwiGLU, 8>(s, d->x, B.ffn_norm, m.rms_eps, D, 2 * F, oacc,
				                                                       d->xa, on)
				                 : launch_dec<kProNorm, kEpiSwiGLU>(s, d->x, B.ffn_norm, m.rms_eps, D, 2 * F, oacc,
				                                                    d->xa, on))
					return rc;
				if (self_next) {
					hipLaunchKernelGGL(oacc_apply_kernel, dim3((D + 255) / 256), dim3(256), 0, stream(), d->tmp,
					                   oacc, oacc, D);
					HK_LAUNCHED("residual accumulator clear");
				}
				resid = d->xa;
			} else if (int rc = gu_persist ? launch_dec_gu(s, d->x, B.ffn_norm, m.rms_eps, D)
			                    : gu_items == 8
			                        ? launch_dec<kProNorm, kEpiSwiGLU, 8>(s, d->x, B.ffn_norm, m.rms_eps, D, 2 * F)
			                        : launch_dec<kProNorm, kEpiSwiGLU>(s, d->x, B.ffn_norm, m.rms_eps, D, 2 * F)) {
				return rc;
			}
		} else {
			if (int rc = rmsnorm(d->x, B.ffn_norm, d->xn, D, m.rms_eps, 1)) return rc;
			if (int rc = hako_gpu_matmul(d->g, d->xn, B.t_gate, B.gate, nullptr, F, D)) return rc;
			if (int rc = hako_gpu_matmul(d->u, d->xn, B.t_up, B.up, nullptr, F, D)) return rc;
			hipLaunchKernelGGL(silu_mul_kernel, dim3((F + 255) / 256), dim3(256), 0, stream(), d->h, d->g, d->u, F);
			HK_LAUNCHED("silu_mul");
		}
		// 5. down projection + residual: x = resid + W h
		if (B.t_down == HAKO_TYPE_Q6_K) {
			if (int rc = q6k_gemv(d->x, B.down, d->h, nullptr, D, F, resid)) return rc;
		} else {
			if (int rc = hako_gpu_matmul(d->tmp, d->h, B.t_down, B.down, nullptr, D, F)) return rc;
			if (int rc = add(d->x, resid, d->tmp, D)) return rc;
		}
	}
	if (int rc = rmsnorm(d->x, m.out_norm, d->xn, D, m.rms_eps, 1)) return rc;
	if (int rc = hako_gpu_matmul(d->logits, d->xn, m.t_out, m.out_weight, nullptr, m.vocab, D)) return rc;
	if (int rc = argmax(d)) return rc;
	return HAKO_GPU_OK;
}

int capture(hako_gpu_decoder *d) {
	if (d->exec) return HAKO_GPU_OK;
	HK_HIP(hipStreamBeginCapture(stream(), hipStreamCaptureModeThreadLocal));
	const int rc = enqueue_step(d);
	hipGraph_t g = nullptr;
	const hipError_t e = hipStreamEndCapture(stream(), &g);
	if (rc) {
		if (g) (void)hipGraphDestroy(g);
		return rc;
	}
	if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
	d->graph = g;
	HK_HIP(hipGraphInstantiate(&d->exec, g, nullptr, nullptr, 0));
	return HAKO_GPU_OK;
}

int set_tokens(hako_gpu_decoder *d, const int *tokens) {
	for (int s = 0; s < d->n_seq; s++)
		if (tokens[s] < 0 || tokens[s] >= d->m.vocab)
			return set_error(HAKO_GPU_EINVAL, "token %d of sequence %d outside the vocabulary", tokens[s], s);
	HK_HIP(hipMemcpyAsync(d->tok, tokens, sizeof(int) * d->n_seq, hipMemcpyHostToDevice, stream()));
	return HAKO_GPU_OK;
}

// positions must leave room for n more steps
int check_room(hako_gpu_decoder *d, int n) {
	std::vector<int> pos(d->n_seq);
	HK_HIP(hipMemcpyAsync(pos.data(), d->pos, sizeof(int) * d->n_seq, hipMemcpyDeviceToHost, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	for (int s = 0; s < d->n_seq; s++)
		if (pos[s] < 0 || pos[s] + n > d->max_seq)
			return set_error(HAKO_GPU_EINVAL, "sequence %d at position %d has no room for %d steps (max_seq %d)", s,
			                 pos[s], n, d->max_seq);
	return HAKO_GPU_OK;
}

// ── prompt prefill: the reference's feed (src/hakm_api.c:105-111), one
// hakm_forward per prompt token, as passes of up to pf_chunk tokens
// through the multi-token matmuls ──

// Tokens per pass: up to 512 (64-token GEMM tiles fill the chip and the
// weights stream once per 512 tokens), halved while the pass's attention
// records (tokens x KV heads x the chunks its last position reaches x heads
// per KV head) exceed the record buffer, at most 1 GiB.
constexpr int kPrefillMax = 512;
constexpr size_t kPrefillRecordBytes = (size_t)1 << 30;

// Attention chunks a pass ending at position `last` spans (the grid width and
// the record stride of its launches): rounded up to an odd count, since
// workgroups go to the 8 XCDs in turn and an even width would pin a chunk to
// a few of them (with 8, chunk c to XCD c, while the causal span gives chunk
// 0 every token).
int prefill_chunks(int last) { return (last / kChunk + 1) | 1; }
size_t prefill_rec_bytes(const hako_gpu_model &m, int tokens, int chunks) {
	return (size_t)tokens * m.n_kv_heads * chunks * kMaxG * (m.head_dim + 2) * 4;
}

int prefill_alloc(hako_gpu_decoder *d) {
	if (d->pf_x) return HAKO_GPU_OK;
	const hako_gpu_model &m = d->m;
	const size_t C = kPrefillMax;
	d->pf_chunk = (int)C;
	size_t rec = prefill_rec_bytes(m, kPrefillMax, prefill_chunks(d->max_seq - 1));
	d->pf_part_bytes = rec < kPrefillRecordBytes ? rec : kPrefillRecordBytes;
	const size_t D = m.d_model, F = m.ffn_dim, KV = d->kv_dim;
	int rc = 0;
#define HK_ALLOC(ptr, bytes) \
	if (!rc) rc = dalloc(d, (bytes), (void **)&(ptr))
	HK_ALLOC(d->pf_x, 4 * C * D);
	HK_ALLOC(d->pf_xn, 4 * C * D);
	HK_ALLOC(d->pf_q, 4 * C * D);
	HK_ALLOC(d->pf_k, 4 * C * KV);
	HK_ALLOC(d->pf_v, 4 * C * KV);
	HK_ALLOC(d->pf_att, 4 * C * D);
	HK_ALLOC(d->pf_tmp, 4 * C * D);
	HK_ALLOC(d->pf_g, 4 * C * F);
	HK_ALLOC(d->pf_u, 4 * C * F);
	HK_ALLOC(d->pf_part, d->pf_part_bytes);
	HK_ALLOC(d->pf_xq, C * (D > F ? D : F));
	HK_ALLOC(d->pf_xs, 4 * C * (D > F ? D : F) / 32);
	HK_ALLOC(d->pf_xh, 2 * C * F);
	HK_ALLOC(d->pf_xl, 2 * C * F);
	HK_ALLOC(d->pf_esc, 4 * C);
	d->pf_sk_floats = q6k_gemm_sk_floats(q6k_gemm_sk_grid());
	HK_ALLOC(d->pf_sk, 4 * d->pf_sk_floats);
	HK_ALLOC(d->pf_tok, 4 * C);
	HK_ALLOC(d->pf_pos, 4 * C);
#undef HK_ALLOC
	if (rc) d->pf_x = nullptr;   // retried on the next call; the others stay tracked for destroy
	return rc;
}

// Tokens [0, n) of sequence seq at positions pos0.. (n <= pf_chunk):
// every layer for all of them, each matmul one multi-token launch, causal
// attention over the cache (the chunk's keys and values appended first).
int prefill_chunk(hako_gpu_decoder *d, int seq, const int *tokens, int n, int pos0) {
	const hako_gpu_model &m = d->m;
	const int D = m.d_model, F = m.ffn_dim, KV = d->kv_dim, HD = m.head_dim, KVH = m.n_kv_heads;
	const int G = m.n_heads / KVH;
	std::vector<int> posv(n);
	for (int i = 0; i < n; i++) posv[i] = pos0 + i;
	HK_HIP(hipMemcpyAsync(d->pf_tok, tokens, sizeof(int) * n, hipMemcpyHostToDevice, stream()));
	HK_HIP(hipMemcpyAsync(d->pf_pos, posv.data(), sizeof(int) * n, hipMemcpyHostToDevice, stream()));
	HK_HIP(hipStreamSynchronize(stream()));   // posv is this frame's
	hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(256), 0, stream(), (const uint8_t *)m.tok_embd, m.t_embd,
	                   row_bytes(m.t_embd, D), d->pf_tok, d->pf_x, D, m.vocab);
	HK_LAUNCHED("embed");
	const float scale = 1.0f / sqrtf((float)HD);
	const size_t seq_off = (size_t)seq * m.n_layers * d->max_seq * KV;
	for (int l = 0; l < m.n_layers; l++) {
		const hako_gpu_block &B = d->blocks[l];
		float *kcl = d->kc + seq_off + (size_t)l * d->max_seq * KV;
		float *vcl = d->vc + seq_off + (size_t)l * d->max_seq * KV;
		// Q4_K matmuls of more than 16 tokens run fused: one rmsnorm+q8 launch
		// per input, q/k/v as one launch over three row segments, gate/up as
		// one launch writing silu(gate)*up, the residual added by the o and
		// down launches; other types and short passes take one call per matmul.
		const bool multi = n > kSkMaxTokens && D <= 4 * kRowT;
		const bool f_qkv = multi && B.t_q == HAKO_TYPE_Q4_K && B.t_k == HAKO_TYPE_Q4_K && B.t_v == HAKO_TYPE_Q4_K;
		const bool f_o = multi && B.t_o == HAKO_TYPE_Q4_K;
		const bool f_gu = multi && B.t_gate == HAKO_TYPE_Q4_K && B.t_up == HAKO_TYPE_Q4_K;
		if (f_qkv) {
			if (int rc = rmsnorm_q8_rows(d->pf_x, B.attn_norm, m.rms_eps, d->pf_xq, d->pf_xs, D, n)) return rc;
			SkSegs s{};
			s.n = 3;
			s.s[0] = {(const uint8_t *)B.wq, B.bq, d->pf_q, 0, D, D};
			s.s[1] = {(const uint8_t *)B.wk, B.bk, d->pf_k, D, KV, KV};
			s.s[2] = {(const uint8_t *)B.wv, B.bv, d->pf_v, D + KV, KV, KV};
			if (int rc = q4k_gemm_segs(s, kSkStore, d->pf_xq, d->pf_xs, n, D, D + 2 * KV)) return rc;
		} else {
			if (int rc = rmsnorm(d->pf_x, B.attn_norm, d->pf_xn, D, m.rms_eps, n)) return rc;
			if (int rc = hako_gpu_matmul_batch(d->pf_q, d->pf_xn, B.t_q, B.wq, B.bq, n, D, D)) return rc;
			if (int rc = hako_gpu_matmul_batch(d->pf_k, d->pf_xn, B.t_k, B.wk, B.bk, n, KV, D)) return rc;
			if (int rc = hako_gpu_matmul_batch(d->pf_v, d->pf_xn, B.t_v, B.wv, B.bv, n, KV, D)) return rc;
		}
		hipLaunchKernelGGL(rope_append_kernel, dim3(n), dim3(256), 0, stream(), d->pf_k, d->pf_v, d->rope, d->pf_pos,
		                   kcl, vcl, KVH, HD, d->max_seq);
		HK_LAUNCHED("rope_append");
		// token i attends over positions [0, pos0 + i] of the sequence's cache;
		// the merge also writes the q8 rows of its output for a fused o
		int8_t *mxq = f_o ? d->pf_xq : nullptr;
		float *mxs = f_o ? d->pf_xs : nullptr;
		// chunks up to the pass's last position (not max_seq's: the rest would
		// exit at once), also the record stride of the pass
		const int pchunks = prefill_chunks(pos0 + n - 1);
		const dim3 ag(pchunks, KVH, n), mg(G, KVH, n);
		if (HD == 128 && pos0 + n <= kFlashPos) {
			// every token's keys in one workgroup: matrix cores, no merge pass
			hipLaunchKernelGGL(attn_flash_kernel<kFlashQG>, dim3(m.n_heads, (n + 16 * kFlashQG - 1) / (16 * kFlashQG)),
			                   dim3(128 * kFlashQG), 0, stream(), d->pf_q,
			                   d->rope, kcl, vcl, d->pf_pos, d->pf_att, mxq, mxs, m.n_heads, KVH, d->max_seq, n, scale);
			HK_LAUNCHED("attention");
		} else if (HD == 128) {
			hipLaunchKernelGGL((attn_kernel<128, false>), ag, dim3(256), 0, stream(), d->pf_q, d->rope, kcl, vcl,
			                   d->pf_pos, d->pf_part, m.n_heads, KVH, d->max_seq, pchunks, (size_t)0, D, scale,
			                   1);
			HK_LAUNCHED("attention");
			hipLaunchKernelGGL(attn_merge_kernel<128>, mg, dim3(128), 0, stream(), d->pf_part, d->pf_pos, d->pf_att,
			                   mxq, mxs, m.n_heads, KVH, d->max_seq, pchunks);
			HK_LAUNCHED("attention merge");
		} else {
			hipLaunchKernelGGL((attn_kernel<64, false>), ag, dim3(256), 0, stream(), d->pf_q, d->rope, kcl, vcl,
			                   d->pf_pos, d->pf_part, m.n_heads, KVH, d->max_seq, pchunks, (size_t)0, D, scale,
			                   1);
			HK_LAUNCHED("attention");
			hipLaunchKernelGGL(attn_merge_kernel<64>, mg, dim3(64), 0, stream(), d->pf_part, d->pf_pos, d->pf_att,
			                   mxq, mxs, m.n_heads, KVH, d->max_seq, pchunks);
			HK_LAUNCHED("attention merge");
		}
		if (f_o) {
			SkSegs s{};
			s.n = 1;
			s.s[0] = {(const uint8_t *)B.wo, nullptr, d->pf_x, 0, D, D};
			if (int rc = q4k_gemm_segs(s, kSkAdd, d->pf_xq, d->pf_xs, n, D, D)) return rc;
		} else {
			if (int rc = hako_gpu_matmul_batch(d->pf_tmp, d->pf_att, B.t_o, B.wo, nullptr, n, D, D)) return rc;
			if (int rc = add(d->pf_x, d->pf_x, d->pf_tmp, n * D)) return rc;
		}
		if (f_gu) {
			if (int rc = rmsnorm_q8_rows(d->pf_x, B.ffn_norm, m.rms_eps, d->pf_xq, d->pf_xs, D, n)) return rc;
			SkSegs s{};
			s.n = 2;
			s.s[0] = {(const uint8_t *)B.gate, nullptr, d->pf_g, 0, F, F};
			s.s[1] = {(const uint8_t *)B.up, nullptr, d->pf_g, 0, F, F};
			if (int rc = q4k_gemm_segs(s, kSkSwiGLU, d->pf_xq, d->pf_xs, n, D, 2 * F)) return rc;
		} else {
			if (int rc = rmsnorm(d->pf_x, B.ffn_norm, d->pf_xn, D, m.rms_eps, n)) return rc;
			if (int rc = hako_gpu_matmul_batch(d->pf_g, d->pf_xn, B.t_gate, B.gate, nullptr, n, F, D)) return rc;
			if (int rc = hako_gpu_matmul_batch(d->pf_u, d->pf_xn, B.t_up, B.up, nullptr, n, F, D)) return rc;
			hipLaunchKernelGGL(silu_mul_kernel, dim3((n * F + 255) / 256), dim3(256), 0, stream(), d->pf_g, d->pf_g,
			                   d->pf_u, n * F);
			HK_LAUNCHED("silu_mul");
		}
		// down + residual: h = pf_g
		if (n > kSkMaxTokens && B.t_down == HAKO_TYPE_Q6_K) {
			if (int rc = f16_split(d->pf_g, d->pf_xh, d->pf_xl, d->pf_esc, n, F)) return rc;
			if (int rc = q6k_gemm_split(d->pf_x, B.down, d->pf_xh, d->pf_xl, d->pf_esc, nullptr, n, D, F, true, d->pf_sk,
			                             d->pf_sk_floats))
				return rc;
		} else if (n > kSkMaxTokens && B.t_down == HAKO_TYPE_Q4_K) {
			if (int rc = hako_gpu_quantize_q8_32(d->pf_g, n, F, d->pf_xq, d->pf_xs)) return rc;
			SkSegs s{};
			s.n = 1;
			s.s[0] = {(const uint8_t *)B.down, nullptr, d->pf_x, 0, D, D};
			if (int rc = q4k_gemm_segs(s, kSkAdd, d->pf_xq, d->pf_xs, n, F, D)) return rc;
		} else {
			if (int rc = hako_gpu_matmul_batch(d->pf_tmp, d->pf_g, B.t_down, B.down, nullptr, n, D, F)) return rc;
			if (int rc = add(d->pf_x, d->pf_x, d->pf_tmp, n * D)) return rc;
		}
	}
	return HAKO_GPU_OK;
}

}  // namespace

extern "C" {

int hako_gpu_decoder_create(const hako_gpu_model *m, int n_seq, int max_seq, hako_gpu_decoder **out) {
	if (int rc = require_device()) return rc;
	if (!m || !out || !m->blocks) return set_error(HAKO_GPU_EINVAL, "null model or output");
	*out = nullptr;
	if (n_seq < 1 || n_seq > kSkMaxTokens)
		return set_error(HAKO_GPU_EINVAL, "decoder runs 1 to %d sequences per step (got %d)", kSkMaxTokens, n_seq);
	if (m->n_layers <= 0 || m->n_heads <= 0 || m->n_kv_heads <= 0 || m->n_heads % m->n_kv_heads != 0 ||
	    m->n_heads / m->n_kv_heads > kMaxG || (m->head_dim != 64 && m->head_dim != 128) ||
	    m->d_model != m->n_heads * m->head_dim || m->d_model % kQK != 0 || m->ffn_dim % kQK != 0 || m->vocab <= 0 ||
	    max_seq <= 0)
		return set_error(HAKO_GPU_EINVAL,
		                 "unsupported decoder shape: layers %d d_model %d heads %d/%d head_dim %d ffn %d vocab %d "
		                 "max_seq %d",
		                 m->n_layers, m->d_model, m->n_heads, m->n_kv_heads, m->head_dim, m->ffn_dim, m->vocab,
		                 max_seq);
	// one sequence's layer cache is read through 32-bit buffer offsets
	if ((size_t)max_seq * m->n_kv_heads * m->head_dim * 4 >= kBufNone)
		return set_error(HAKO_GPU_EINVAL, "max_seq %d x kv_dim %d: a layer's cache of one sequence exceeds 2 GiB",
		                 max_seq, m->n_kv_heads * m->head_dim);
	if (!known_type(m->t_embd) || !known_type(m->t_out) || !m->tok_embd || !m->out_weight || !m->out_norm)
		return set_error(HAKO_GPU_ETYPE, "embedding / output types %d / %d", m->t_embd, m->t_out);
	for (int l = 0; l < m->n_layers; l++) {
		const hako_gpu_block &B = m->blocks[l];
		const int ts[7] = {B.t_q, B.t_k, B.t_v, B.t_o, B.t_gate, B.t_up, B.t_down};
		for (int t : ts)
			if (!known_type(t)) return set_error(HAKO_GPU_ETYPE, "layer %d: unsupported tensor type %d", l, t);
		if (!B.attn_norm || !B.ffn_norm || !B.wq || !B.wk || !B.wv || !B.wo || !B.gate || !B.up || !B.down)
			return set_error(HAKO_GPU_EINVAL, "layer %d: missing tensor", l);
	}
	hako_gpu_decoder *d = new hako_gpu_decoder();
	d->m = *m;
	d->blocks.assign(m->blocks, m->blocks + m->n_layers);
	d->m.blocks = nullptr;
	d->n_seq = n_seq;
	d->max_seq = max_seq;
	d->max_chunks = (max_seq + kChunk - 1) / kChunk;
	d->kv_dim = m->n_kv_heads * m->head_dim;
	d->qkv_dim = m->d_model + 2 * d->kv_dim;
	const int D = m->d_model, F = m->ffn_dim, HD = m->head_dim;
	const size_t kvn = (size_t)n_seq * m->n_layers * max_seq * d->kv_dim;
	int rc = 0;
#define HK_ALLOC(ptr, bytes) \
	if (!rc) rc = dalloc(d, (bytes), (void **)&(ptr))
	HK_ALLOC(d->x, sizeof(float) * n_seq * D);
	HK_ALLOC(d->xn, sizeof(float) * n_seq * D);
	HK_ALLOC(d->qkv, sizeof(float) * n_seq * d->qkv_dim);
	HK_ALLOC(d->att, sizeof(float) * n_seq * D);
	HK_ALLOC(d->h, sizeof(float) * n_seq * F);
	HK_ALLOC(d->g, sizeof(float) * n_seq * F);
	HK_ALLOC(d->u, sizeof(float) * n_seq * F);
	HK_ALLOC(d->tmp, sizeof(float) * n_seq * D);
	HK_ALLOC(d->logits, sizeof(float) * n_seq * m->vocab);
	HK_ALLOC(d->part, sizeof(float) * n_seq * m->n_kv_heads * d->max_chunks * kMaxG * (HD + 2));
	HK_ALLOC(d->kc, sizeof(float) * kvn);
	HK_ALLOC(d->vc, sizeof(float) * kvn);
	HK_ALLOC(d->rope, sizeof(float2) * (size_t)max_seq * (HD / 2));
	HK_ALLOC(d->apart, sizeof(float2) * n_seq * kArgBlocks);
	HK_ALLOC(d->tok, sizeof(int) * n_seq);
	HK_ALLOC(d->pos, sizeof(int) * n_seq);
	HK_ALLOC(d->ring, sizeof(int) * n_seq * max_seq);
	HK_ALLOC(d->nout, sizeof(int) * n_seq);
	HK_ALLOC(d->oacc, sizeof(long long) * 4 * acc_row(D));   // three accumulators and a scratch row
	HK_ALLOC(d->xa, sizeof(float) * D);
	const int DF = F > D ? F : D;
	// split-K partials of the largest skinny matmul of a step
	const size_t skpart = batched_part_floats(d->m, d->kv_dim);
	if (n_seq > 1) {
		// q8 rows of the widest matmul input (generic layers quantize h too)
		HK_ALLOC(d->xq, (size_t)n_seq * DF);
		HK_ALLOC(d->xs, sizeof(float) * n_seq * (DF / 32));
		HK_ALLOC(d->xh, sizeof(_Float16) * n_seq * DF);
		HK_ALLOC(d->xl, sizeof(_Float16) * n_seq * DF);
		HK_ALLOC(d->esc, sizeof(float) * n_seq);
		HK_ALLOC(d->escb, sizeof(float) * n_seq * (F / kQK));
		HK_ALLOC(d->skpart, sizeof(float) * (skpart ? skpart : 1));
		d->skpart_floats = skpart;
	}
#undef HK_ALLOC
	if (rc) {
		hako_gpu_decoder_destroy(d);
		return rc;
	}
	// rope table with the reference's expression (src/nn.c:31-41)
	std::vector<float2> rope((size_t)max_seq * (HD / 2));
	for (int p = 0; p < max_seq; p++)
		for (int i = 0; i < HD / 2; i++) {
			const float freq = powf(m->rope_theta, -((float)(2 * i) / (float)HD));
			const float ang = (float)p * freq;
			rope[(size_t)p * (HD / 2) + i] = make_float2(cosf(ang), sinf(ang));
		}
	hipError_t e = hipMemcpy(d->rope, rope.data(), sizeof(float2) * rope.size(), hipMemcpyHostToDevice);
	if (e == hipSuccess) e = hipMemset(d->kc, 0, sizeof(float) * kvn);
	if (e == hipSuccess) e = hipMemset(d->vc, 0, sizeof(float) * kvn);
	if (e == hipSuccess) e = hipMemset(d->pos, 0, sizeof(int) * n_seq);
	if (e == hipSuccess) e = hipMemset(d->nout, 0, sizeof(int) * n_seq);
	if (e == hipSuccess) e = hipMemset(d->oacc, 0, sizeof(long long) * 4 * acc_row(D));
	if (e == hipSuccess) e = hipDeviceSynchronize();
	if (e != hipSuccess) {
		hako_gpu_decoder_destroy(d);
		return hip_fail(e, "decoder init", __FILE__, __LINE__);
	}
	*out = d;
	return ok();
}

int hako_gpu_decoder_destroy(hako_gpu_decoder *d) {
	if (!d) return ok();
	if (stream()) (void)hipStreamSynchronize(stream());
	if (d->exec) (void)hipGraphExecDestroy(d->exec);
	if (d->graph) (void)hipGraphDestroy(d->graph);
	for (void *p : d->allocs) (void)hipFree(p);
	if (d->on_destroy) d->on_destroy(d->on_destroy_arg);
	delete d;
	return ok();
}

int hako_gpu_decoder_on_destroy(hako_gpu_decoder *d, void (*fn)(void *), void *arg) {
	if (!d) return set_error(HAKO_GPU_EINVAL, "null decoder");
	d->on_destroy = fn;
	d->on_destroy_arg = fn ? arg : nullptr;
	return ok();
}

int hako_gpu_decoder_kv(hako_gpu_decoder *d, float **k_cache, float **v_cache) {
	if (!d) return set_error(HAKO_GPU_EINVAL, "null decoder");
	if (k_cache) *k_cache = d->kc;
	if (v_cache) *v_cache = d->vc;
	return ok();
}

int hako_gpu_decoder_set_pos(hako_gpu_decoder *d, const int *pos) {
	if (!d || !pos) return set_error(HAKO_GPU_EINVAL, "null decoder or positions");
	for (int s = 0; s < d->n_seq; s++)
		if (pos[s] < 0 || pos[s] >= d->max_seq)
			return set_error(HAKO_GPU_EINVAL, "position %d of sequence %d outside [0, %d)", pos[s], s, d->max_seq);
	HK_HIP(hipMemcpyAsync(d->pos, pos, sizeof(int) * d->n_seq, hipMemcpyHostToDevice, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	return ok();
}

int hako_gpu_decoder_step(hako_gpu_decoder *d, const int *tokens, float *logits, int *next) {
	if (!d || !tokens) return set_error(HAKO_GPU_EINVAL, "null decoder or tokens");
	if (int rc = check_room(d, 1)) return rc;
	if (int rc = set_tokens(d, tokens)) return rc;
	if (int rc = enqueue_step(d)) return rc;
	if (logits)
		HK_HIP(hipMemcpyAsync(logits, d->logits, sizeof(float) * d->n_seq * d->m.vocab, hipMemcpyDeviceToHost,
		                      stream()));
	if (next) HK_HIP(hipMemcpyAsync(next, d->tok, sizeof(int) * d->n_seq, hipMemcpyDeviceToHost, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	return ok();
}

int hako_gpu_decoder_generate(hako_gpu_decoder *d, const int *tokens, int n, int *out) {
	if (!d || !tokens || !out || n <= 0) return set_error(HAKO_GPU_EINVAL, "null argument or n <= 0");
	if (int rc = check_room(d, n)) return rc;
	if (int rc = set_tokens(d, tokens)) return rc;
	HK_HIP(hipMemsetAsync(d->nout, 0, sizeof(int) * d->n_seq, stream()));
	if (int rc = capture(d)) return rc;
	for (int i = 0; i < n; i++) HK_HIP(hipGraphLaunch(d->exec, stream()));
	std::vector<int> ring((size_t)d->n_seq * d->max_seq);
	HK_HIP(hipMemcpyAsync(ring.data(), d->ring, sizeof(int) * ring.size(), hipMemcpyDeviceToHost, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	for (int i = 0; i < n; i++)
		for (int s = 0; s < d->n_seq; s++) out[(size_t)i * d->n_seq + s] = ring[(size_t)s * d->max_seq + i];
	return ok();
}

int hako_gpu_decoder_prefill(hako_gpu_decoder *d, int seq, const int *tokens, int n, float *logits, int *next) {
	if (!d || !tokens || n <= 0) return set_error(HAKO_GPU_EINVAL, "null decoder or tokens, or n <= 0");
	if (seq < 0 || seq >= d->n_seq) return set_error(HAKO_GPU_EINVAL, "sequence %d of %d", seq, d->n_seq);
	const hako_gpu_model &m = d->m;
	for (int i = 0; i < n; i++)
		if (tokens[i] < 0 || tokens[i] >= m.vocab)
			return set_error(HAKO_GPU_EINVAL, "prompt token %d (%d) outside the vocabulary", i, tokens[i]);
	int pos0 = 0;
	HK_HIP(hipMemcpyAsync(&pos0, d->pos + seq, sizeof(int), hipMemcpyDeviceToHost, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	if (pos0 < 0 || pos0 + n > d->max_seq)
		return set_error(HAKO_GPU_EINVAL, "sequence %d at position %d has no room for %d prompt tokens (max_seq %d)",
		                 seq, pos0, n, d->max_seq);
	if (int rc = prefill_alloc(d)) return rc;
	const int D = m.d_model;
	int last = 0;
	for (int c0 = 0; c0 < n; c0 += last) {
		last = n - c0 < d->pf_chunk ? n - c0 : d->pf_chunk;
		// halved while the pass's records exceed the buffer
		while (last > 1 && prefill_rec_bytes(m, last, prefill_chunks(pos0 + c0 + last - 1)) > d->pf_part_bytes)
			last /= 2;
		if (prefill_rec_bytes(m, last, prefill_chunks(pos0 + c0 + last - 1)) > d->pf_part_bytes)
			return set_error(HAKO_GPU_EINVAL, "attention records of one prompt token at position %d exceed %zu bytes",
			                 pos0 + c0, d->pf_part_bytes);
		if (int rc = prefill_chunk(d, seq, tokens + c0, last, pos0 + c0)) return rc;
	}
	// logits of the last prompt token (what feed returns), into the
	// sequence's row of the step's logits
	float *lg = d->logits + (size_t)seq * m.vocab;
	if (int rc = rmsnorm(d->pf_x + (size_t)(last - 1) * D, m.out_norm, d->pf_xn, D, m.rms_eps, 1)) return rc;
	if (int rc = hako_gpu_matmul(lg, d->pf_xn, m.t_out, m.out_weight, nullptr, m.vocab, D)) return rc;
	const int pos1 = pos0 + n;
	HK_HIP(hipMemcpyAsync(d->pos + seq, &pos1, sizeof(int), hipMemcpyHostToDevice, stream()));
	std::vector<float> host;
	float *dst = logits;
	if (!dst && next) {
		host.resize(m.vocab);
		dst = host.data();
	}
	if (dst) HK_HIP(hipMemcpyAsync(dst, lg, sizeof(float) * m.vocab, hipMemcpyDeviceToHost, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	if (next) {
		// greedy pick as the device argmax: NaN never wins, ties take the lowest index
		int best = -1;
		for (int i = 0; i < m.vocab; i++)
			if (dst[i] == dst[i] && (best < 0 || dst[i] > dst[best])) best = i;
		*next = best < 0 ? 0 : best;
	}
	return ok();
}

int hako_gpu_decoder_replay(hako_gpu_decoder *d, int n) {
	if (!d || n < 0) return set_error(HAKO_GPU_EINVAL, "null decoder or n < 0");
	if (int rc = check_room(d, n)) return rc;
	if (int rc = capture(d)) return rc;
	for (int i = 0; i < n; i++) HK_HIP(hipGraphLaunch(d->exec, stream()));
	return ok();
}

}  // extern "C"
