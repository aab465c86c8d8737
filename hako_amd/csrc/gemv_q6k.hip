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
// Lane work. Chunk c = 4i + s of a row is block i, half n = s/2 and l half
// lh = s%2: the 64 weights k = 0..3, l in [16lh, 16lh+16) of half n, four
// 16-wide scale groups. They come from two 16-byte loads of ql at
// 64n+16lh (low nibbles k = 0, high k = 2) and 64n+32+16lh (k = 1, 3), one
// of qh at 32n+16lh (bits 2k..2k+1), 8 bytes of scales and d: the four lanes
// of a block read each of its bytes once (232 bytes loaded per 210-byte
// block; a no-arithmetic probe of this pattern streams the 151936x2048
// vocab matrix at 5.9 TB/s against 4.7 for eight lanes of 32 weights, which
// load each qh byte twice and the scales four times). Blocks are only 2-byte
// aligned in the verbatim stream (210 = 2*105), so the loads are unaligned;
// gfx950 serves them in the HSA unaligned-access mode the compiler itself
// assumes for byte copies. The 6-bit values are assembled four to a dword
// (nibbles | qh bits moved to bits 4-5 of each byte), converted per byte
// (v_cvt_f32_ubyteN) and multiplied into the lane's fp32 activations; per
// scale group the sum is Σq·x − 32·Σx with −32·Σx precomputed.
//
// Grid. Persistent: about one workgroup per CU, each owning a contiguous row
// range. A row of C = 4*NB chunks is cut into ceil(C/64) parts; the
// workgroup has one wave group per part (W = parts x row-slices waves, at
// most 8), and wave (part p, slice r) visits rows r, r+RW, ... of the range
// with part p's activations hoisted in registers for all of them. Partial sums
// of a row meet in LDS. Each wave keeps four row loads in flight ahead of the
// row it computes.
#include "hako_dev.h"
#include "hako_rt.h"

namespace hako {
namespace {

constexpr int kQ6Depth = 4;
constexpr int kQ6MaxWaves = 8;
// waves of a flat wide workgroup: 8 parts of 64 chunks, 12 of 32 (rows up to
// 32768 / 24576 weights); the launch bound keeps 170+ registers per lane
template <int SEGW>
constexpr int q6_max_parts() { return SEGW == 64 ? 8 : 12; }

struct Q6Buf {
	uint4 qa, qb;    // ql 64n+16lh .. +16 (k = 0, 2) and 64n+32+16lh .. +16 (k = 1, 3)
	uint4 qh;        // qh 32n+16lh .. +16
	uint2 s;         // scales 8n .. 8n+8
	uint32_t d;
};

// The lane's activation columns for one chunk: xv[k][j] = x at weight
// 128n + 32k + 16lh + j of block i, and -32·Σ_j xv[k][j].
struct Q6Col {
	float xv[4][16];
	float nsx[4];
};

__device__ __forceinline__ void q6_col_load(const float *__restrict__ x, int c, Q6Col &col) {
	const int i = c >> 2, s = c & 3, n = s >> 1, lh = s & 1;
	const float *xb = x + kQK * i + 128 * n + 16 * lh;
#pragma unroll
	for (int k = 0; k < 4; k++) {
#pragma unroll
		for (int m = 0; m < 4; m++) {
			const float4 u = *(const float4 *)(xb + 32 * k + 4 * m);
			col.xv[k][4 * m] = u.x; col.xv[k][4 * m + 1] = u.y;
			col.xv[k][4 * m + 2] = u.z; col.xv[k][4 * m + 3] = u.w;
		}
	}
}

__device__ __forceinline__ void q6_col_sums(Q6Col &col) {
#pragma unroll
	for (int k = 0; k < 4; k++) {
		float t = 0.0f;
#pragma unroll
		for (int j = 0; j < 16; j++) t += col.xv[k][j];
		col.nsx[k] = -32.0f * t;
	}
}

__device__ __forceinline__ float byte_f(uint32_t w, int b) { return (float)((w >> (8 * b)) & 0xFFu); }

// d · Σ_k sc_k · (Σ_j q_k,j·x_k,j − 32·Σ_j x_k,j) over the lane's 64 weights
// (scale 8n + 2k + lh: byte 2k + lh of the lane's 8 scale bytes).
__device__ __forceinline__ float q6_dot(const Q6Buf &W, const Q6Col &col, int lh) {
	float acc[4] = {col.nsx[0], col.nsx[1], col.nsx[2], col.nsx[3]};
	const uint32_t lo = 0x0F0F0F0Fu, hb = 0x30303030u;
	const uint32_t qa[4] = {W.qa.x, W.qa.y, W.qa.z, W.qa.w}, qb[4] = {W.qb.x, W.qb.y, W.qb.z, W.qb.w};
	const uint32_t qh[4] = {W.qh.x, W.qh.y, W.qh.z, W.qh.w};
#pragma unroll
	for (int u = 0; u < 4; u++) {
		// qh bits 2k, 2k+1 of each byte to bits 4, 5 with at most one shift;
		// what the neighbouring bytes shift in lands outside bits 4-5
		uint32_t wk[4];
		wk[0] = (qa[u] & lo) | ((qh[u] << 4) & hb);
		wk[1] = (qb[u] & lo) | ((qh[u] << 2) & hb);
		wk[2] = ((qa[u] >> 4) & lo) | (qh[u] & hb);
		wk[3] = ((qb[u] >> 4) & lo) | ((qh[u] >> 2) & hb);
#pragma unroll
		for (int k = 0; k < 4; k++)
#pragma unroll
			for (int b = 0; b < 4; b++) acc[k] = __builtin_fmaf(byte_f(wk[k], b), col.xv[k][4 * u + b], acc[k]);
	}
	const int sh = 8 * lh;
	const float s0 = (float)(int8_t)((W.s.x >> sh) & 0xFFu), s1 = (float)(int8_t)((W.s.x >> (sh + 16)) & 0xFFu);
	const float s2 = (float)(int8_t)((W.s.y >> sh) & 0xFFu), s3 = (float)(int8_t)((W.s.y >> (sh + 16)) & 0xFFu);
	return f16_to_f32(W.d) * ((s0 * acc[0] + s1 * acc[1]) + (s2 * acc[2] + s3 * acc[3]));
}

// The lane's activation columns as integers, for grids whose lanes keep one
// chunk for many rows: group k (16 values, one scale group) scaled by its own
// power of two 2^s[k] so that its largest magnitude lies in [2^21, 2^22),
// rounded to integers D and split into three balanced signed bytes,
// D = d0 + 256 d1 + 65536 d2, packed four to a dword per byte plane. A group's
// sum over its 16 six-bit values is then three v_dot4_i32_i8 chains (exact in
// int32), recombined in fp32 and scaled back by 2^-s[k]: ~2 vector ops per
// weight against ~3 for the fp32 product per weight, the activation carried
// to 2^-22 of its group's maximum (well inside the 1e-5 output tolerance).
struct Q6Dig {
	uint32_t d[4][3][4];   // [group k][byte plane][positions 4u .. 4u+3]
	int s[4];
	float nsx[4];          // -32 * sum of the group's fp32 values
};

// false when a group holds an inf or NaN (its sum is not finite): the wave
// then keeps the fp32 path for all its lanes, which carries them as the
// reference does
__device__ __forceinline__ bool q6_digits(const Q6Col &col, Q6Dig &g) {
	bool ok = true;
#pragma unroll
	for (int k = 0; k < 4; k++) {
		float m = 0.0f;
#pragma unroll
		for (int j = 0; j < 16; j++) m = __builtin_fmaxf(m, __builtin_fabsf(col.xv[k][j]));
		ok = ok && __builtin_isfinite(col.nsx[k]);
		const int e = m > 0.0f ? __builtin_amdgcn_frexp_expf(m) : 0;
		const int sk = m > 0.0f ? 22 - e : 0;
		g.s[k] = sk;
		g.nsx[k] = col.nsx[k];
		uint32_t b[3][16];
#pragma unroll
		for (int j = 0; j < 16; j++) {
			const float v = __builtin_isfinite(col.xv[k][j]) ? col.xv[k][j] : 0.0f;
			const int D = (int)__builtin_rintf(__builtin_ldexpf(v, sk));
			const int d0 = (int)(int8_t)(D & 0xFF);
			const int D1 = (D - d0) >> 8;
			const int d1 = (int)(int8_t)(D1 & 0xFF);
			const int D2 = (D1 - d1) >> 8;
			b[0][j] = (uint32_t)D;
			b[1][j] = (uint32_t)D1;
			b[2][j] = (uint32_t)D2;
		}
#pragma unroll
		for (int p = 0; p < 3; p++)
#pragma unroll
			for (int u = 0; u < 4; u++) {
				const uint32_t lo = __builtin_amdgcn_perm(b[p][4 * u + 1], b[p][4 * u], 0x0c0c0400u);
				const uint32_t hi = __builtin_amdgcn_perm(b[p][4 * u + 3], b[p][4 * u + 2], 0x0c0c0400u);
				g.d[k][p][u] = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
			}
	}
	return ok;
}

// q6_dot on the integer columns: d · Σ_k sc_k · (2^-s_k Σ_j q_k,j·D_k,j − 32·Σ_j x_k,j)
__device__ __forceinline__ float q6_dot_dig(const Q6Buf &W, const Q6Dig &g, int lh) {
	const uint32_t lo = 0x0F0F0F0Fu, hb = 0x30303030u;
	const uint32_t qa[4] = {W.qa.x, W.qa.y, W.qa.z, W.qa.w}, qb[4] = {W.qb.x, W.qb.y, W.qb.z, W.qb.w};
	const uint32_t qh[4] = {W.qh.x, W.qh.y, W.qh.z, W.qh.w};
	int S[4][3] = {};
#pragma unroll
	for (int u = 0; u < 4; u++) {
		uint32_t wk[4];
		wk[0] = (qa[u] & lo) | ((qh[u] << 4) & hb);
		wk[1] = (qb[u] & lo) | ((qh[u] << 2) & hb);
		wk[2] = ((qa[u] >> 4) & lo) | (qh[u] & hb);
		wk[3] = ((qb[u] >> 4) & lo) | ((qh[u] >> 2) & hb);
#pragma unroll
		for (int k = 0; k < 4; k++)
#pragma unroll
			for (int p = 0; p < 3; p++) S[k][p] = sdot4((int)wk[k], (int)g.d[k][p][u], S[k][p]);
	}
	float acc[4];
#pragma unroll
	for (int k = 0; k < 4; k++) {
		const float t = ((float)S[k][0] + 256.0f * (float)S[k][1]) + 65536.0f * (float)S[k][2];
		acc[k] = __builtin_ldexpf(t, -g.s[k]) + g.nsx[k];
	}
	const int sh = 8 * lh;
	const float s0 = (float)(int8_t)((W.s.x >> sh) & 0xFFu), s1 = (float)(int8_t)((W.s.x >> (sh + 16)) & 0xFFu);
	const float s2 = (float)(int8_t)((W.s.y >> sh) & 0xFFu), s3 = (float)(int8_t)((W.s.y >> (sh + 16)) & 0xFFu);
	return f16_to_f32(W.d) * ((s0 * acc[0] + s1 * acc[1]) + (s2 * acc[2] + s3 * acc[3]));
}

struct Q6Geom {
	int C, seg, rt, tpr, rw, waves;
};

// `target` waves per workgroup (4 or 8): row slices = target / parts, >= 1.
__host__ __device__ inline Q6Geom q6_geom(int n_in, int target) {
	Q6Geom g;
	g.C = n_in / kQK * 4;
	if (g.C <= 64) {
		g.seg = 1;
		while (g.seg < g.C) g.seg <<= 1;
		g.rt = 64 / g.seg;
		g.tpr = 1;
		g.rw = target;
	} else {
		g.seg = 64;
		g.rt = 1;
		g.tpr = (g.C + 63) / 64;
		g.rw = target / g.tpr > 1 ? target / g.tpr : 1;
	}
	g.waves = g.tpr * g.rw;
	return g;
}

// One workgroup: waves = parts x row-slices (see q6_geom). DIG: the integer
// columns (q6_digits) when every lane of the wave has finite activations.
template <bool DIG>
__global__ __launch_bounds__(kQ6MaxWaves * kWave) void q6k_gemv_kernel(const uint8_t *__restrict__ w,
                                                                       const float *__restrict__ x,
                                                                       const float *__restrict__ bias,
                                                                       const float *res,
                                                                       float *out, int n_out,
                                                                       int n_in, int target) {
	extern __shared__ float red_s[];   // [rows of this workgroup][parts]: partial row sums
	const Q6Geom G = q6_geom(n_in, target);
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int part = wave % G.tpr, slice = wave / G.tpr;
	const int r0 = (int)((int64_t)blockIdx.x * n_out / gridDim.x);
	const int r1 = (int)((int64_t)(blockIdx.x + 1) * n_out / gridDim.x);
	const int nrows = r1 - r0;
	const size_t rb = (size_t)(n_in >> 8) * kQ6Bytes;
	const int sub = lane & (G.seg - 1), rsub = lane / G.seg;
	const int c = 64 * part + sub;              // this lane's chunk, fixed for every row
	const bool lane_on = c < G.C;
	const int ntiles = (nrows + G.rt - 1) / G.rt;
	const int nit = ntiles > slice ? (ntiles - slice + G.rw - 1) / G.rw : 0;
	auto item_row = [&](int it) -> int { return r0 + G.rt * (slice + G.rw * it) + rsub; };

	const int cc = min(c, G.C - 1);           // in-bounds chunk for idle lanes' loads
	const int i = cc >> 2, s = cc & 3, hn = s >> 1, lh = s & 1;
	const size_t in_row = (size_t)i * kQ6Bytes;
	// Weight loads are raw buffer loads, never predicated: slots with no work
	// use an offset past the stream (zeros, no memory traffic). A branch
	// around a load would make the compiler wait for all outstanding loads.
	const __amdgpu_buffer_rsrc_t wr = stream_rsrc(w, (uint32_t)(rb * n_out));
	auto issue = [&](Q6Buf &b, int it) {
		const int row = item_row(it);
		const bool on = it < nit && row < r1 && lane_on;
		const uint32_t blk = on ? (uint32_t)((size_t)row * rb + in_row) : kBufNone;
		b.qa = ld_b128(wr, blk + 64 * hn + 16 * lh);
		b.qb = ld_b128(wr, blk + 64 * hn + 32 + 16 * lh);
		b.qh = ld_b128(wr, blk + 128 + 32 * hn + 16 * lh);
		b.s = ld_b64(wr, blk + 192 + 8 * hn);
		b.d = ld_b16(wr, blk + 208);
	};

	Q6Col col;
	q6_col_load(x, cc, col);   // issued first: these loads return first
	// The residual and bias of the row this thread finishes, loaded now: at
	// the end they would add a round trip after the weight stream.
	float res0 = 0.0f, bias0 = 0.0f;
	if (threadIdx.x < nrows) {
		if (res) res0 = res[r0 + threadIdx.x];
		if (bias) bias0 = bias[r0 + threadIdx.x];
	}
	// Keep every weight load below the activation loads (completion is in
	// issue order).
	__builtin_amdgcn_sched_barrier(0);
	// Item loads go out in consumption order (the scheduler would otherwise
	// interleave them, and the first item would wait for all four).
	Q6Buf buf[kQ6Depth];
#pragma unroll
	for (int j = 0; j < kQ6Depth; j++) {
		issue(buf[j], j);
		__builtin_amdgcn_sched_barrier(0);
	}
	q6_col_sums(col);   // waits for x only: it was loaded first
	Q6Dig dg;
	bool dig = false;
	if (DIG) {
		const bool ok = q6_digits(col, dg);
		dig = __all(ok);
	}

	// Whole groups of kQ6Depth items (same load count every iteration; slots
	// past nit load nothing). Their arithmetic is skipped by a wave-uniform
	// branch that holds no loads; the group's four rows are reduced together.
	for (int base = 0; base < nit; base += kQ6Depth) {
		float rsum[kQ6Depth];
#pragma unroll
		for (int j = 0; j < kQ6Depth; j++) {
			const int it = base + j;
			const int row = item_row(it);
			float d = 0.0f;
			// Consume buf[j] in place, then reload it (no register rotation).
			if (it < nit) d = dig ? q6_dot_dig(buf[j], dg, lh) : q6_dot(buf[j], col, lh);
			issue(buf[j], it + kQ6Depth);
			__builtin_amdgcn_sched_barrier(0);
			rsum[j] = (lane_on && row < r1) ? d : 0.0f;
		}
		// Rows with a bias, and split rows, finish after the weight stream: a
		// bias load in the loop would wait for every weight load in flight.
		const float tot = seg_sum4(rsum, G.seg, lane);
		const int j = sub & 3;
		const int row = item_row(base + j);
		if (sub < kQ6Depth && base + j < nit && row < r1) {
			if (G.tpr > 1)
				red_s[(row - r0) * G.tpr + part] = tot;
			else if (bias || res)
				red_s[row - r0] = tot;
			else
				out[row] = tot;
		}
	}
	// Rows with a bias or a residual to add, and split rows, finish here: a
	// load of either inside the loop would wait for every weight load in flight.
	if (G.tpr > 1 || bias || res) {
		__syncthreads();
		for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
			float v = 0.0f;
			for (int p = 0; p < G.tpr; p++) v += red_s[r * G.tpr + p];
			const bool first = r == (int)threadIdx.x;
			if (bias) v += first ? bias0 : bias[r0 + r];
			out[r0 + r] = res ? (first ? res0 : res[r0 + r]) + v : v;
		}
	}
}

// Flat grid: every weight load of a wave issued at once, right after the
// activation (and bias / residual) loads, as the Q4_K flat GEMV does; latency
// is hidden by the many workgroups resident on each CU instead of a software
// pipeline. Rows of C <= 64 chunks: a workgroup of 4 waves, a wave owns ITEMS
// consecutive row tiles of rt = 64/seg rows. Wider rows: parts of SEGW
// chunks (64, or 32: two rows per wave instruction), a workgroup of P =
// ceil(C/SEGW) waves, wave p the chunks [SEGW p, SEGW p + SEGW) of ITEMS row
// tiles of rt = 64/SEGW rows; the P partial sums of a row meet in LDS. With
// 32-chunk parts a workgroup covers twice the rows for the same work per
// wave, so each row's activation part is read by half as many workgroups.
template <int ITEMS, int SEGW>
__global__ __launch_bounds__(q6_max_parts<SEGW>() * kWave) void q6k_gemv_flat_kernel(const uint8_t *__restrict__ w,
                                                                           const float *__restrict__ x,
                                                                           const float *__restrict__ bias,
                                                                           const float *res, float *out,
                                                                           int n_out, int n_in) {
	constexpr int NG = (ITEMS + 3) / 4;   // groups of four items reduced together
	constexpr int WRT = 64 / SEGW;        // rows per item of a wide workgroup
	__shared__ float red_s[q6_max_parts<SEGW>()][4 * NG * WRT];
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int NB = n_in >> 8, C = NB * 4;
	const bool wide = C > 64;
	const int seg = wide ? SEGW : next_pow2(C), rt = 64 / seg;
	const int sub = lane & (seg - 1), rsub = lane / seg;
	const int part = wide ? wave : 0;
	const int c = seg * part + sub;
	const bool lane_on = c < C;
	// first row of this wave's items; a wide workgroup's waves share rows
	const int wrow0 = wide ? blockIdx.x * ITEMS * rt : (blockIdx.x * 4 + wave) * ITEMS * rt;
	auto item_row = [&](int it) -> int { return wrow0 + rt * it + rsub; };
	const size_t rb = (size_t)NB * kQ6Bytes;

	const int cc = min(c, C - 1);
	const int i = cc >> 2, s = cc & 3, hn = s >> 1, lh = s & 1;

	// 1. activation, then bias / residual of the row this lane writes: in a
	//    narrow workgroup lane sub (< 4) of segment rsub writes item 4g + sub;
	//    in a wide one lane L of wave 0 writes row wrow0 + L
	Q6Col col;
	q6_col_load(x, cc, col);
	float rv[NG], bv[NG];
#pragma unroll
	for (int g = 0; g < NG; g++) {
		const int r = min(wide ? wrow0 + 64 * g + lane : item_row(4 * g + (sub & 3)), n_out - 1);
		rv[g] = res ? res[r] : 0.0f;
		bv[g] = bias ? bias[r] : 0.0f;
	}
	// out = res + (sum + bias), the persistent kernel's order of additions
	auto finish = [&](float v, int g) -> float {
		v = bias ? v + bv[g] : v;
		return res ? rv[g] + v : v;
	};
	__builtin_amdgcn_sched_barrier(0);
	// 2. every weight load of the wave, in consumption order
	const __amdgpu_buffer_rsrc_t wr = stream_rsrc(w, (uint32_t)(rb * n_out));
	Q6Buf buf[ITEMS];
#pragma unroll
	for (int j = 0; j < ITEMS; j++) {
		const int row = item_row(j);
		const bool on = row < n_out && lane_on;
		const uint32_t blk = on ? (uint32_t)((size_t)row * rb + (size_t)i * kQ6Bytes) : kBufNone;
		buf[j].qa = ld_b128(wr, blk + 64 * hn + 16 * lh);
		buf[j].qb = ld_b128(wr, blk + 64 * hn + 32 + 16 * lh);
		buf[j].qh = ld_b128(wr, blk + 128 + 32 * hn + 16 * lh);
		buf[j].s = ld_b64(wr, blk + 192 + 8 * hn);
		buf[j].d = ld_b16(wr, blk + 208);
		__builtin_amdgcn_sched_barrier(0);
	}
	q6_col_sums(col);   // waits for x only: it was loaded first

	// 3. the row sums
	float rsum[4 * NG];
#pragma unroll
	for (int j = 0; j < 4 * NG; j++) {
		rsum[j] = 0.0f;
		if (j >= ITEMS) continue;
		const float d = q6_dot(buf[j], col, lh);
		rsum[j] = (lane_on && item_row(j) < n_out) ? d : 0.0f;
	}
	// 4. lane sub = j (< 4) of each segment holds item 4g + j of its row rsub
	if (!wide) {
#pragma unroll
		for (int g = 0; g < NG; g++) {
			const float tot = seg_sum4(rsum + 4 * g, seg, lane);
			const int j = 4 * g + (sub & 3);
			const int row = item_row(j);
			if ((sub >> 2) == 0 && j < ITEMS && row < n_out) out[row] = finish(tot, g);
		}
		return;
	}
#pragma unroll
	for (int g = 0; g < NG; g++) {
		const float tot = seg_sum4(rsum + 4 * g, SEGW, lane);
		if (sub < 4) red_s[part][WRT * (4 * g + sub) + rsub] = tot;
	}
	__syncthreads();
	if (wave == 0) {
#pragma unroll
		for (int g = 0; g < NG; g++) {
			const int lr = 64 * g + lane;   // local row: item lr / WRT, segment lr % WRT
			const int row = wrow0 + lr;
			if (lr < ITEMS * WRT && row < n_out) {
				float v = 0.0f;
				for (int p = 0; p < (int)(blockDim.x >> 6); p++) v += red_s[p][lr];
				out[row] = finish(v, g);
			}
		}
	}
}

// Persistent rows grid: one workgroup per CU of W waves (a multiple of 4, so
// the four SIMDs carry equal work). A row tile is rt = 64/seg rows (seg =
// min(64, chunks) lanes per row), cut into P = ceil(C/seg) passes of seg
// chunks; each wave walks whole row tiles of the workgroup's row range pass
// by pass, so a row's sum never leaves its wave (lane sums over the passes,
// then the segment's lanes). D pass items are in flight per wave; an item's
// weight offsets are per-lane constants plus one wave-uniform row/pass
// offset. Rows of several passes take the activation from LDS, staged once
// per workgroup as [chunk][68] floats — the chunk's 64 values in the lane's
// order, then its four -32*sum(x) terms (the 68-float stride puts 8
// consecutive lanes' 16-byte reads on all 32 banks); one-pass rows keep it
// in registers.
constexpr uint32_t kRowsNone = 0x7FF00000u;   // a lane part or row part past every stream

template <int W, int D, bool XREG>
__global__ __launch_bounds__(W * kWave) void q6k_rows_kernel(const uint8_t *__restrict__ w,
                                                          const float *__restrict__ x,
                                                          const float *__restrict__ bias, const float *res,
                                                          float *out, int n_out, int n_in) {
	extern __shared__ __align__(16) float lds_f[];
	constexpr int T = W * kWave;
	constexpr int XS = 8192 / T;   // float4 loads per thread that stage up to 32768 inputs
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int NB = n_in >> 8, C = NB * 4;
	const int seg = C >= 64 ? 64 : next_pow2(C), rt = 64 / seg, P = (C + seg - 1) / seg;
	const int sub = lane & (seg - 1), rsub = lane / seg;
	const int r0 = (int)((int64_t)blockIdx.x * n_out / gridDim.x);
	const int r1 = (int)((int64_t)(blockIdx.x + 1) * n_out / gridDim.x);
	const int nrows = r1 - r0, ntiles = (nrows + rt - 1) / rt;
	const uint32_t rb = (uint32_t)NB * kQ6Bytes;
	float *xl = lds_f;                               // [C][68] floats (rows of several passes)
	float *red_s = lds_f + (XREG ? 0 : C * 68);      // [nrows] row sums
	const int s = sub & 3, hn = s >> 1, lh = s & 1;  // the lane's quarter of a block, every pass
	const bool last_on = seg * (P - 1) + sub < C;    // the lane has a chunk in the last pass
	// lane parts of the offsets (row rsub of the tile, block sub/4 of the pass)
	const uint32_t lb = (uint32_t)rsub * rb + (uint32_t)(sub >> 2) * kQ6Bytes;
	const uint32_t lbl = last_on ? lb : kRowsNone;
	const uint32_t oa = 64 * hn + 16 * lh, oh = 128 + 32 * hn + 16 * lh, os = 192 + 8 * hn;
	const __amdgpu_buffer_rsrc_t wr = stream_rsrc(w, rb * (uint32_t)n_out);
	// this wave's tiles: wave, wave + W, ...; its items: tile by tile, pass by pass
	const int nt_w = ntiles > wave ? (ntiles - wave + W - 1) / W : 0;
	const int NQ = nt_w * P;
	auto issue = [&](Q6Buf &b, int ti, int p) {
		const int tl = wave + W * ti;
		const uint32_t so = tl < ntiles ? (uint32_t)(r0 + rt * tl) * rb + (uint32_t)(p * (seg >> 2)) * kQ6Bytes
		                                : 0x80000000u;
		const uint32_t v = (p == P - 1 ? lbl : lb) + so;
		b.qa = ld_b128(wr, v + oa);
		b.qb = ld_b128(wr, v + oa + 32);
		b.qh = ld_b128(wr, v + oh);
		b.s = ld_b64(wr, v + os);
		b.d = ld_b16(wr, v + 208);
	};

	// 1. the activation, the first D items' weights, this thread's row's
	//    residual and bias. Staged rows load the activation first: after the
	//    first workgroups of an XCD it comes from L2, so its LDS copy is
	//    ready about when the first weights arrive (weights first left the
	//    waves waiting on the staging with their weights in hand: 7B down
	//    3584x18944 16.2 -> 15.3 us). One-pass rows keep it in registers
	//    and load it after the weights.
	Q6Buf buf[D];
	int ti_i = 0, p_i = 0;
	auto advance = [&](int &ti, int &p) {
		if (++p == P) {
			p = 0;
			ti++;
		}
	};
	Q6Col col;
	if (XREG) {
#pragma unroll
		for (int j = 0; j < D; j++) {
			issue(buf[j], ti_i, p_i);
			advance(ti_i, p_i);
			__builtin_amdgcn_sched_barrier(0);
		}
		q6_col_load(x, min(sub, C - 1), col);
	} else {
		// x as float4 f = t, t + T, ...: element 4f is j0..j0+3 of chunk c's run k
		const __amdgpu_buffer_rsrc_t xr = stream_rsrc(x, (uint32_t)n_in * 4u);
		// only the passes that hold inputs (a uniform bound: 10 of the 16 at
		// 18944 inputs; issuing the rest, out of range, cost 0.35 us at 7B down)
		const int nf4 = n_in >> 2;
		float4 xv4[XS];
#pragma unroll
		for (int u = 0; u < XS; u++) {
			xv4[u] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
			if (u * T < nf4) xv4[u] = __builtin_bit_cast(float4, ld_b128(xr, (uint32_t)(threadIdx.x + u * T) * 16u));
		}
		__builtin_amdgcn_sched_barrier(0);
#pragma unroll
		for (int j = 0; j < D; j++) {
			issue(buf[j], ti_i, p_i);
			advance(ti_i, p_i);
			__builtin_amdgcn_sched_barrier(0);
		}
#pragma unroll
		for (int u = 0; u < XS; u++) {
			const int f = threadIdx.x + u * T;
			const int e = 4 * f, i = e >> 8, n = (e >> 7) & 1, k = (e >> 5) & 3, l2 = (e >> 4) & 1, j0 = e & 15;
			const int c = 4 * i + 2 * n + l2;
			// sum of the run's 16 values: the four lanes of a quad hold it
			float t = ((xv4[u].x + xv4[u].y) + xv4[u].z) + xv4[u].w;
			t += dpp_f<kDppQuadSwap1>(t);
			t += dpp_f<kDppQuadSwap2>(t);
			if (f < nf4) {
				*(float4 *)(xl + c * 68 + 16 * k + j0) = xv4[u];
				if (j0 == 0) xl[c * 68 + 64 + k] = -32.0f * t;
			}
		}
	}
	float res0 = 0.0f, bias0 = 0.0f;
	if ((int)threadIdx.x < nrows) {
		if (res) res0 = res[r0 + threadIdx.x];
		if (bias) bias0 = bias[r0 + threadIdx.x];
	}
	if (!XREG) __syncthreads();
	else q6_col_sums(col);

	// 2. items in groups of D (the ring's slots are static): compute the
	//    item in slot j, then issue the item D later into it
	float racc = 0.0f;
	int ti_c = 0, p_c = 0;
	for (int q0 = 0; q0 < NQ; q0 += D) {
#pragma unroll
		for (int j = 0; j < D; j++) {
			if (q0 + j < NQ) {
				if (!XREG) {
					const float4 *xc = (const float4 *)(xl + min(seg * p_c + sub, C - 1) * 68);
#pragma unroll
					for (int k = 0; k < 4; k++)
#pragma unroll
						for (int m = 0; m < 4; m++) {
							const float4 u = xc[4 * k + m];
							col.xv[k][4 * m] = u.x; col.xv[k][4 * m + 1] = u.y;
							col.xv[k][4 * m + 2] = u.z; col.xv[k][4 * m + 3] = u.w;
						}
					const float4 ns = xc[16];
					col.nsx[0] = ns.x; col.nsx[1] = ns.y; col.nsx[2] = ns.z; col.nsx[3] = ns.w;
				}
				const float d = q6_dot(buf[j], col, lh);
				racc += (p_c < P - 1 || last_on) ? d : 0.0f;
				if (p_c == P - 1) {
					const float tot = seg_sum(racc, seg);
					const int lr = rt * (wave + W * ti_c) + rsub;
					if (sub == 0 && lr < nrows) red_s[lr] = tot;
					racc = 0.0f;
				}
			}
			issue(buf[j], ti_i, p_i);
			advance(ti_i, p_i);
			advance(ti_c, p_c);
			__builtin_amdgcn_sched_barrier(0);
		}
	}
	// 3. out = res + (sum + bias), each row by one thread
	__syncthreads();
	for (int r = threadIdx.x; r < nrows; r += T) {
		float v = red_s[r];
		const bool first = r == (int)threadIdx.x;
		if (bias) v += first ? bias0 : bias[r0 + r];
		out[r0 + r] = res ? (first ? res0 : res[r0 + r]) + v : v;
	}
}

int g_q6_wgs_per_cu = 1;
int g_q6_waves = 4;
// -1: by shape (below); 0: persistent grid; 1, 2, 4, 8: flat grid with that many items per wave
int g_q6_flat_items = -1;
// chunks per part of the flat grid's wide rows: 64, or 32 (0: by shape)
int g_q6_flat_seg = 0;
// rows grid: 0 by shape, -1 never, else 10 * waves + depth (44, 82, 84, 162)
int g_q6_rows = 0;
// persistent grid: integer activation columns (1) or the fp32 product per weight (0)
int g_q6_dig = 1;

// Measured on MI355X (us per launch, persistent / flat with 1, 2, 4, 8
// items): 2048x11008 (3 parts) 8.08 / 10.8 / 8.58 / 7.45 / 8.24; 1000x4608
// (2 parts) 5.29 / 4.75 / 4.66 / 4.45 / 6.40; 3584x18944 (5 parts) 18.1 /
// 28.5 / 25.0 / 22.7 / 22.5; 16384x3584 (4 parts) 13.0 / 20.7 / 16.8 / 13.6
// / 13.6; 151936x2048 48.4 / 88.7 / 65.3 / 54.5 / 53.3; 152064x3584 89.7 /
// 165 / 129 / 98.1 / 90.5; earlier, 256x2048 (one part) 3.75 / 2.99 / 3.38 /
// 3.92. Rows of 2..3 parts take the flat grid with 4 items; short matrices
// of one part the flat grid with one item; wider rows and tall matrices the
// persistent grid.
int q6_flat_items_for(int n_out, const Q6Geom &G) {
	if (g_q6_flat_items >= 0) return g_q6_flat_items;
	if (G.C > 64 && G.tpr <= 3 && n_out <= 8192) return 4;   // past ~8K rows the persistent grid streams faster
	if (G.C <= 64 && n_out <= 4096) return 1;
	return 0;
}

}  // namespace

void q6k_set_wgs_per_cu(int v) { g_q6_wgs_per_cu = v < 1 ? 1 : (v > 8 ? 8 : v); }
void q6k_set_waves(int v) { g_q6_waves = v >= 8 ? 8 : 4; }
void q6k_set_rows(int v) { g_q6_rows = v; }
void q6k_set_dig(int v) { g_q6_dig = v ? 1 : 0; }
void q6k_set_flat_seg(int v) { g_q6_flat_seg = v == 32 || v == 64 ? v : 0; }
void q6k_set_flat_items(int v) { g_q6_flat_items = v < 0 ? -1 : (v == 0 ? 0 : (v <= 1 ? 1 : (v <= 2 ? 2 : (v <= 4 ? 4 : 8)))); }

}  // namespace hako

namespace hako {

// out = W x (+ bias), or out = res + W x (+ bias) when res is not null (a
// residual add; res may equal out: each row is read before it is written, by
// the same thread).
int q6k_gemv(float *out, const void *w, const float *x, const float *bias, int n_out, int n_in, const float *res) {
	if (int rc = require_device()) return rc;
	if (n_out <= 0 || n_in <= 0 || n_in % kQK != 0)
		return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV needs n_out > 0 and n_in %% 256 == 0 (got %d x %d)",
		                 n_out, n_in);
	if (((uintptr_t)w & 1) || ((uintptr_t)x & 15))
		return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV needs w 2-byte and x 16-byte aligned");
	const Q6Geom G = q6_geom(n_in, g_q6_waves);
	if ((size_t)n_out * (n_in / kQK) * kQ6Bytes >= kBufNone)
		return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV weight of %d x %d exceeds 2 GiB", n_out, n_in);
	if (G.waves > kQ6MaxWaves || G.tpr > kQ6MaxWaves)
		return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV n_in %d exceeds %d", n_in, kQ6MaxWaves * 64 * 64);
	// rows of several passes that the flat grid does not take go to the rows
	// grid (8 waves, 2 items in flight: 7B down 3584x18944 17.9 -> 16.2 us;
	// 4 waves / 4 items 19.0, 8 / 4 17.7, 16 / 2 16.8)
	const int rows_cfg = g_q6_rows > 0 ? g_q6_rows
	                     : (g_q6_rows == 0 && G.C > 64 && q6_flat_items_for(n_out, G) == 0) ? 82 : 0;
	if (rows_cfg) {
		const int NB = n_in / kQK, C = 4 * NB;
		const int seg = C >= 64 ? 64 : next_pow2(C), rt = 64 / seg;
		const bool xreg = C <= 64;
		if ((size_t)n_out * NB * kQ6Bytes > kRowsNone)
			return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV rows grid: weight of %d x %d too large", n_out, n_in);
		if (n_in > 32768) return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV rows grid: n_in %d > 32768", n_in);
		int wgs = (n_out + rt - 1) / rt;
		const int max_wgs = g_q6_wgs_per_cu * cu_count();
		if (wgs > max_wgs) wgs = max_wgs;
		const int rows_per_wg = (n_out + wgs - 1) / wgs + 1;
		const size_t lds = (xreg ? 0 : (size_t)C * 68 * 4) + (size_t)rows_per_wg * 4;
		if (lds > 160 * 1024) return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV rows grid: %zu bytes of LDS", lds);
#define HK_Q6R(WV, DP) \
	hipLaunchKernelGGL((xreg ? q6k_rows_kernel<WV, DP, true> : q6k_rows_kernel<WV, DP, false>), dim3(wgs), \
	                   dim3(WV * kWave), lds, stream(), (const uint8_t *)w, x, bias, res, out, n_out, n_in)
		switch (rows_cfg) {
		case 44: HK_Q6R(4, 4); break;
		case 84: HK_Q6R(8, 4); break;
		case 162: HK_Q6R(16, 2); break;
		default: HK_Q6R(8, 2); break;
		}
#undef HK_Q6R
		HK_LAUNCHED("q6k_rows");
		return ok();
	}
	if (const int items = q6_flat_items_for(n_out, G)) {
		const bool wide = G.C > 64;
		const int segw = g_q6_flat_seg ? g_q6_flat_seg : 64;
		const int parts = (G.C + segw - 1) / segw;
		const int max_parts = segw == 32 ? q6_max_parts<32>() : q6_max_parts<64>();
		if (wide && parts > max_parts)
			return set_error(HAKO_GPU_EINVAL, "Q6_K GEMV flat grid: n_in %d needs more than %d parts", n_in, max_parts);
		const int rows_wg = wide ? items * (64 / segw) : 4 * items * G.rt;
		const int wgs = (n_out + rows_wg - 1) / rows_wg;
		const dim3 block(wide ? parts * kWave : 4 * kWave);
#define HK_Q6F(IT, SW) \
	hipLaunchKernelGGL((q6k_gemv_flat_kernel<IT, SW>), dim3(wgs), block, 0, stream(), (const uint8_t *)w, x, bias, res, \
	                   out, n_out, n_in)
		if (segw == 32) {
			if (items <= 1) HK_Q6F(1, 32);
			else if (items <= 2) HK_Q6F(2, 32);
			else if (items <= 4) HK_Q6F(4, 32);
			else HK_Q6F(8, 32);
		} else {
			if (items <= 1) HK_Q6F(1, 64);
			else if (items <= 2) HK_Q6F(2, 64);
			else if (items <= 4) HK_Q6F(4, 64);
			else HK_Q6F(8, 64);
		}
#undef HK_Q6F
		HK_LAUNCHED("q6k_gemv_flat");
		return ok();
	}
	const int min_rows = G.rt * G.rw;
	int wgs = (n_out + min_rows - 1) / min_rows;
	const int max_wgs = g_q6_wgs_per_cu * cu_count();
	if (wgs > max_wgs) wgs = max_wgs;
	// partial row sums in LDS: at most 8192 rows x parts per workgroup
	const int max_rows_per_wg = 8192 / G.tpr;
	if ((n_out + wgs - 1) / wgs > max_rows_per_wg) wgs = (n_out + max_rows_per_wg - 1) / max_rows_per_wg;
	const int rows_per_wg = (n_out + wgs - 1) / wgs;
	const size_t lds = (size_t)rows_per_wg * G.tpr * sizeof(float);
	if (g_q6_dig)
		hipLaunchKernelGGL(q6k_gemv_kernel<true>, dim3(wgs), dim3(G.waves * kWave), lds, stream(), (const uint8_t *)w,
		                   x, bias, res, out, n_out, n_in, g_q6_waves);
	else
		hipLaunchKernelGGL(q6k_gemv_kernel<false>, dim3(wgs), dim3(G.waves * kWave), lds, stream(), (const uint8_t *)w,
		                   x, bias, res, out, n_out, n_in, g_q6_waves);
	HK_LAUNCHED("q6k_gemv");
	return ok();
}

}  // namespace hako

extern "C" int hako_gpu_q6k_gemv(float *out, const void *w, const float *x, const float *bias,
                                 int n_out, int n_in) {
	return hako::q6k_gemv(out, w, x, bias, n_out, n_in, nullptr);
}
