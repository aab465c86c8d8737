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

// One workgroup: waves = parts x row-slices (see q6_geom).
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
			if (it < nit) d = q6_dot(buf[j], col, lh);
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
// consecutive row tiles of rt = 64/seg rows. Wider rows: a workgroup of P =
// ceil(C/64) waves, wave p the chunks [64p, 64p + 64) of ITEMS consecutive
// rows; the P partial sums of a row meet in LDS.
template <int ITEMS>
__global__ __launch_bounds__(kQ6MaxWaves * kWave) void q6k_gemv_flat_kernel(const uint8_t *__restrict__ w,
                                                                            const float *__restrict__ x,
                                                                            const float *__restrict__ bias,
                                                                            const float *res, float *out,
                                                                            int n_out, int n_in) {
	constexpr int NG = (ITEMS + 3) / 4;   // groups of four items reduced together
	__shared__ float red_s[kQ6MaxWaves][4 * NG];
	const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
	const int NB = n_in >> 8, C = NB * 4;
	const bool wide = C > 64;
	const int seg = wide ? 64 : next_pow2(C), rt = 64 / seg;
	const int sub = lane & (seg - 1), rsub = lane / seg;
	const int part = wide ? wave : 0;
	const int c = 64 * part + sub;
	const bool lane_on = c < C;
	// first row of this wave's items; a wide workgroup's waves share rows
	const int wrow0 = wide ? blockIdx.x * ITEMS : (blockIdx.x * 4 + wave) * ITEMS * rt;
	auto item_row = [&](int it) -> int { return wide ? wrow0 + it : wrow0 + rt * it + rsub; };
	const size_t rb = (size_t)NB * kQ6Bytes;

	const int cc = min(c, C - 1);
	const int i = cc >> 2, s = cc & 3, hn = s >> 1, lh = s & 1;

	// 1. activation, then bias / residual of the row this lane writes
	Q6Col col;
	q6_col_load(x, cc, col);
	float rv[NG], bv[NG];
#pragma unroll
	for (int g = 0; g < NG; g++) {
		const int r = min(item_row(4 * g + (sub & 3)), n_out - 1);
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
	// 4. lane sub = j (< 4) of each segment holds item 4g + j
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
		const float tot = seg_sum4(rsum + 4 * g, 64, lane);
		if (lane < 4) red_s[part][4 * g + lane] = tot;
	}
	__syncthreads();
	if (wave == 0 && lane < 4 * NG && lane < ITEMS) {
		const int row = wrow0 + lane;
		if (row < n_out) {
			float v = 0.0f;
			for (int p = 0; p < (int)(blockDim.x >> 6); p++) v += red_s[p][lane];
			out[row] = finish(v, lane >> 2);
		}
	}
}

int g_q6_wgs_per_cu = 1;
int g_q6_waves = 4;
// -1: by shape (below); 0: persistent grid; 1, 2, 4, 8: flat grid with that many items per wave
int g_q6_flat_items = -1;

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
	if (const int items = q6_flat_items_for(n_out, G)) {
		const bool wide = G.C > 64;
		const int rows_wg = wide ? items : 4 * items * G.rt;
		const int wgs = (n_out + rows_wg - 1) / rows_wg;
		const dim3 block(wide ? G.tpr * kWave : 4 * kWave);
#define HK_Q6F(IT) \
	hipLaunchKernelGGL(q6k_gemv_flat_kernel<IT>, dim3(wgs), block, 0, stream(), (const uint8_t *)w, x, bias, res, out, \
	                   n_out, n_in)
		if (items <= 1) HK_Q6F(1);
		else if (items <= 2) HK_Q6F(2);
		else if (items <= 4) HK_Q6F(4);
		else HK_Q6F(8);
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
	hipLaunchKernelGGL(q6k_gemv_kernel, dim3(wgs), dim3(G.waves * kWave), lds, stream(), (const uint8_t *)w, x,
	                   bias, res, out, n_out, n_in, g_q6_waves);
	HK_LAUNCHED("q6k_gemv");
	return ok();
}

}  // namespace hako

extern "C" int hako_gpu_q6k_gemv(float *out, const void *w, const float *x, const float *bias,
                                 int n_out, int n_in) {
	return hako::q6k_gemv(out, w, x, bias, n_out, n_in, nullptr);
}
