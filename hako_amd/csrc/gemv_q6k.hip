// gemv_q6k.hip — Q6_K x fp32 GEMV for batch-1 decode (gfx950).
//
// Replaces the reference's generic row path for Q6_K weights: dequantize a row
// to fp32, then an fp32 dot with the unquantized activation (src/nn.c:84-95,
// src/quant.c:94-123). The activation stays fp32 here too: an int8
// activation would move results by ~1e-3 relative.
//
// A 210-byte super-block holds, per 128-weight half n, ql[64n..64n+64),
// qh[32n..32n+32) and scales[8n..8n+8); weight 128n + 32k + l (k < 4, l < 32)
// is nibble (k>>1) of ql[64n + 32(k&1) + l] with bits 2k..2k+1 of qh[32n + l]
// on top, minus 32, times d*scales[8n + 2k + l/16].
//
// Work split: 8 lanes per block. Lane sub-index s = c%8 takes half n = s/4
// and l in [l0, l0+8), l0 = 8*(s%4): 8-byte loads of ql at 64n+l0 and
// 64n+32+l0 and of qh at 32n+l0 give its 32 weights (k = 0..3, 8 each), all
// in four 16-wide scale groups. Blocks are only 2-byte aligned in the
// verbatim stream (210 = 2*105), so those loads are unaligned; gfx950 serves
// them in the HSA unaligned-access mode the compiler assumes for byte copies.
//
// The 6-bit values are assembled four at a time in a dword (nibbles | qh bits
// shifted to bits 4-5 of each byte), converted per byte (v_cvt_f32_ubyteN)
// and multiplied into the lane's fp32 activations; per scale group the sum is
// Σ q·x − 32·Σx with Σx precomputed once per lane.
//
// Workgroups of 4 waves; KS waves split a row group's 64-chunk tiles, R rows
// per wave, next tile's loads issued before the current tile is computed.
#include "hako_dev.h"
#include "hako_rt.h"

namespace hako {
namespace {

__device__ __forceinline__ uint2 ld_u2(const uint8_t *p) {
	uint2 v;
	__builtin_memcpy(&v, p, 8);
	return v;
}

struct Q6W {
	uint2 a, b, h, s;
	uint32_t d;
};

// The lane's activation columns for one chunk: xv[k][j] = x at weight
// 128n + 32k + l0 + j of block i, and -32·Σ_j xv[k][j].
struct Q6Col {
	float xv[4][8];
	float nsx[4];
};

__device__ __forceinline__ void q6_col(const float *__restrict__ x, int c, Q6Col &col) {
	const int i = c >> 3, s = c & 7, n = s >> 2, l0 = 8 * (s & 3);
	const float *xb = x + kQK * i + 128 * n + l0;
#pragma unroll
	for (int k = 0; k < 4; k++) {
		const float4 u = *(const float4 *)(xb + 32 * k);
		const float4 v = *(const float4 *)(xb + 32 * k + 4);
		col.xv[k][0] = u.x; col.xv[k][1] = u.y; col.xv[k][2] = u.z; col.xv[k][3] = u.w;
		col.xv[k][4] = v.x; col.xv[k][5] = v.y; col.xv[k][6] = v.z; col.xv[k][7] = v.w;
		float t = 0.0f;
#pragma unroll
		for (int j = 0; j < 8; j++) t += col.xv[k][j];
		col.nsx[k] = -32.0f * t;
	}
}

__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

// d · Σ_k sc_k · (Σ_j q_kj·x_kj − 32·Σ_j x_kj) over the lane's 32 weights.
__device__ __forceinline__ float q6_dot(const Q6W &W, const Q6Col &col, int sel) {
	float acc0 = col.nsx[0], acc1 = col.nsx[1], acc2 = col.nsx[2], acc3 = col.nsx[3];
	const uint32_t lo = 0x0F0F0F0Fu, hi = 0x30303030u;
#pragma unroll
	for (int u = 0; u < 2; u++) {
		const uint32_t l0 = u ? W.a.y : W.a.x, l1 = u ? W.b.y : W.b.x, hh = u ? W.h.y : W.h.x;
		const uint32_t w0 = (l0 & lo) | ((hh << 4) & hi);
		const uint32_t w1 = (l1 & lo) | ((hh << 2) & hi);
		const uint32_t w2 = ((l0 >> 4) & lo) | (hh & hi);
		const uint32_t w3 = ((l1 >> 4) & lo) | ((hh >> 2) & hi);
#pragma unroll
		for (int b = 0; b < 4; b++) {
			acc0 = __builtin_fmaf(byte_f(w0, b), col.xv[0][4 * u + b], acc0);
			acc1 = __builtin_fmaf(byte_f(w1, b), col.xv[1][4 * u + b], acc1);
			acc2 = __builtin_fmaf(byte_f(w2, b), col.xv[2][4 * u + b], acc2);
			acc3 = __builtin_fmaf(byte_f(w3, b), col.xv[3][4 * u + b], acc3);
		}
	}
	// scales[8n + sel + 2k]: k = 0,1 in the first dword, k = 2,3 in the second.
	const int sh0 = 8 * sel, sh1 = 8 * (sel + 2);
	const float s0 = (float)(int8_t)((W.s.x >> sh0) & 0xFFu);
	const float s1 = (float)(int8_t)((W.s.x >> sh1) & 0xFFu);
	const float s2 = (float)(int8_t)((W.s.y >> sh0) & 0xFFu);
	const float s3 = (float)(int8_t)((W.s.y >> sh1) & 0xFFu);
	const float part = s0 * acc0 + s1 * acc1 + s2 * acc2 + s3 * acc3;
	return f16_to_f32(W.d) * part;
}

template <int R, int KS, bool MULTI>
__global__ __launch_bounds__(256) void q6k_gemv_kernel(const uint8_t *__restrict__ w,
                                                       const float *__restrict__ x,
                                                       const float *__restrict__ bias,
                                                       float *__restrict__ out, int n_out, int n_in) {
	__shared__ float red_s[4 * R];
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int wk = wave % KS, wr = wave / KS;
	const int row0 = (blockIdx.x * (4 / KS) + wr) * R;
	const int NB = n_in >> 8, C = NB << 3, tiles = (C + 63) >> 6;
	const size_t rb = (size_t)NB * kQ6Bytes;

	auto load = [&](int T, Q6W *W) {
		const int c = (T << 6) + lane;
		const int i = c >> 3, s = c & 7, n = s >> 2, l0 = 8 * (s & 3);
#pragma unroll
		for (int r = 0; r < R; r++) {
			const int row = row0 + r;
			if (c < C && row < n_out) {
				const uint8_t *blk = w + (size_t)row * rb + (size_t)i * kQ6Bytes;
				W[r].a = ld_u2(blk + 64 * n + l0);
				W[r].b = ld_u2(blk + 64 * n + 32 + l0);
				W[r].h = ld_u2(blk + 128 + 32 * n + l0);
				W[r].s = ld_u2(blk + 192 + 8 * n);
				W[r].d = *(const uint16_t *)(blk + 208);
			} else {
				W[r].a = W[r].b = W[r].h = W[r].s = make_uint2(0, 0);
				W[r].d = 0;
			}
		}
	};

	Q6W Wn[R];
	if (wk < tiles) load(wk, Wn);

	float acc[R];
#pragma unroll
	for (int r = 0; r < R; r++) acc[r] = 0.0f;

	for (int T = wk; T < tiles; T += KS) {
		Q6W W[R];
#pragma unroll
		for (int r = 0; r < R; r++) W[r] = Wn[r];
		if (MULTI && T + KS < tiles) load(T + KS, Wn);
		const int c = (T << 6) + lane;
		if (c < C) {
			Q6Col col;
			q6_col(x, c, col);
			const int sel = (c & 3) >> 1;   // l0 / 16
#pragma unroll
			for (int r = 0; r < R; r++) acc[r] += q6_dot(W[r], col, sel);
		}
	}

	float tot[R];
#pragma unroll
	for (int r = 0; r < R; r++) tot[r] = wave_sum(acc[r]);
	if (KS == 1) {
		float v = tot[0];
#pragma unroll
		for (int r = 1; r < R; r++) v = (lane == r) ? tot[r] : v;
		const int row = row0 + lane;
		if (lane < R && row < n_out) out[row] = bias ? v + bias[row] : v;
	} else {
		if (lane == 0) {
#pragma unroll
			for (int r = 0; r < R; r++) red_s[wave * R + r] = tot[r];
		}
		__syncthreads();
		if (wk == 0 && lane < R) {
			float v = 0.0f;
#pragma unroll
			for (int k = 0; k < KS; k++) v += red_s[(wr * KS + k) * R + lane];
			const int row = row0 + lane;
			if (row < n_out) out[row] = bias ? v + bias[row] : v;
		}
	}
}

template <int R, int KS, bool MULTI>
int q6_launch3(int wgs, const uint8_t *w, const float *x, const float *bias, float *out, int n_out,
               int n_in) {
	hipLaunchKernelGGL((q6k_gemv_kernel<R, KS, MULTI>), dim3(wgs), dim3(256), 0, stream(), w, x, bias,
	                   out, n_out, n_in);
	HK_LAUNCHED("q6k_gemv");
	return ok();
}

template <int R, int KS>
int q6_launch2(bool multi, int wgs, const uint8_t *w, const float *x, const float *bias, float *out,
               int n_out, int n_in) {
	return multi ? q6_launch3<R, KS, true>(wgs, w, x, bias, out, n_out, n_in)
	             : q6_launch3<R, KS, false>(wgs, w, x, bias, out, n_out, n_in);
}

template <int R>
int q6_launch1(int KS, bool multi, int wgs, const uint8_t *w, const float *x, const float *bias,
               float *out, int n_out, int n_in) {
	switch (KS) {
	case 1: return q6_launch2<R, 1>(multi, wgs, w, x, bias, out, n_out, n_in);
	case 2: return q6_launch2<R, 2>(multi, wgs, w, x, bias, out, n_out, n_in);
	default: return q6_launch2<R, 4>(multi, wgs, w, x, bias, out, n_out, n_in);
	}
}

}  // namespace
}  // namespace hako

extern "C" int hako_gpu_q6k_gemv(float *out, const void *w, const float *x, const float *bias,
                                 int n_out, int n_in) {
	using namespace hako;
	if (int rc = require_device()) return rc;
	if (n_out <= 0 || n_in <= 0 || n_in % kQK != 0)
		return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV needs n_out > 0 and n_in %% 256 == 0 (got %d x %d)",
		                 n_out, n_in);
	if (((uintptr_t)w & 1) || ((uintptr_t)x & 15))
		return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV needs w 2-byte and x 16-byte aligned");
	const int tiles = (n_in / kQK * 8 + 63) / 64;
	const int KS = tiles >= 4 ? 4 : (tiles >= 2 ? 2 : 1);
	const bool multi = tiles > KS;
	int R = 1;
	for (int r : {4, 2}) {
		const int rows_per_wg = r * 4 / KS;
		if ((n_out + rows_per_wg - 1) / rows_per_wg >= 512) {
			R = r;
			break;
		}
	}
	const int rows_per_wg = R * 4 / KS;
	const int wgs = (n_out + rows_per_wg - 1) / rows_per_wg;
	const uint8_t *wb = (const uint8_t *)w;
	switch (R) {
	case 4: return q6_launch1<4>(KS, multi, wgs, wb, x, bias, out, n_out, n_in);
	case 2: return q6_launch1<2>(KS, multi, wgs, wb, x, bias, out, n_out, n_in);
	default: return q6_launch1<1>(KS, multi, wgs, wb, x, bias, out, n_out, n_in);
	}
}
