// gemv_q4k.hip — Q4_K x q8 GEMV for batch-1 decode (gfx950).
//
// Replaces the reference's row loop over q4k_vec_dot (src/nn.c:76-82,
// src/quant.c:150-232). The weight matrix is the verbatim stream of 144-byte
// super-blocks, n_in/256 per row.
//
// Lane work. A "chunk" is one 64-weight group of a block: 32 qs bytes whose
// low nibbles are sub-block 2g and high nibbles sub-block 2g+1 (g < 4), so a
// lane owns whole sub-blocks: its integer sums are the reference's iqx/ix
// exactly, and it decodes each (scale, min) pair once for 32 weights. Four
// lanes cover a block; a row of NB blocks has C = 4*NB chunks. When C <= 64
// a wave covers RT = 64/C' rows at once (C' = C rounded up to a power of two,
// lanes past C idle); wider rows take ceil(C/64) wave passes ("parts").
//
// Grid. Persistent: about one workgroup of 8 waves per CU, each owning a
// contiguous range of rows. A wave walks its items (row tiles, or row parts)
// with four item loads in flight ahead of the one it computes, so HBM sees
// the whole matrix requested within the first microsecond on small shapes and
// a steady stream on large ones.
//
// Activation. The workgroup's first memory operation loads x (fp32, fused
// path) or xq/xs (pre-quantized path); the weight loads follow, and the q8_32
// quantization into LDS (quantize_row_q8_32 once per workgroup) runs while
// they are in flight. Each lane then keeps its 64 activation bytes, their two
// scales and partial sums in registers across all the rows it visits.
//
// Arithmetic per chunk: 16 v_dot4_i32_i8 (exact int32: |Σ| <= 15*127*32),
// then the reference's fold xs*(d*s*iqx - dmin*m*ix) for the two sub-blocks,
// regrouped as d*(xsA*sA*iqxA + xsB*sB*iqxB) - dmin*(mA*xsA*ixA + mB*xsB*ixB).
#include "hako_dev.h"
#include "hako_rt.h"
#include "q4k_dev.h"

namespace hako {
namespace {

enum Q4Mode { kFused = 0, kPreq = 1, kIsums = 2 };

constexpr int kQ4Depth = 4;   // item loads in flight per wave

// WIDE: rows of more than 64 chunks (n_in > 4096), taken in 64-chunk parts.
// XP: activation quads per thread (x: 4 floats, xq: 16 bytes each), enough
// that the whole activation is fetched by straight-line loads.
template <int MODE, bool WIDE, int XP, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void q4k_gemv_kernel(
    const uint8_t *__restrict__ w, const float *__restrict__ x, const int8_t *__restrict__ xq_g,
    const float *__restrict__ xs_g, const float *__restrict__ bias, float *__restrict__ out,
    int32_t *__restrict__ iqx_o, int32_t *__restrict__ ix_o, int n_out, int n_in) {
	extern __shared__ __align__(16) uint8_t smem[];
	int8_t *xq_s = (int8_t *)smem;
	float *xs_s = (float *)(smem + n_in);
	float *sum_s = xs_s + (n_in >> 5);   // row sums awaiting their bias

	constexpr int T = WAVES * kWave;
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int NB = n_in >> 8, C = NB * 4;
	const int r0 = (int)((int64_t)blockIdx.x * n_out / gridDim.x);
	const int r1 = (int)((int64_t)(blockIdx.x + 1) * n_out / gridDim.x);
	const int nrows = r1 - r0;
	const size_t rb = (size_t)NB * kQ4Bytes;

	// lane geometry
	const int seg = WIDE ? 64 : next_pow2(C);
	const int rt = 64 / seg;                 // rows per item
	const int tpr = WIDE ? (C + 63) >> 6 : 1;   // parts per row
	const int sub = lane & (seg - 1), rsub = lane / seg;
	int nit;
	if (WIDE) {
		nit = nrows > wave ? ((nrows - wave + WAVES - 1) / WAVES) * tpr : 0;
	} else {
		const int ntiles = (nrows + rt - 1) / rt;
		nit = ntiles > wave ? (ntiles - wave + WAVES - 1) / WAVES : 0;
	}
	auto item_row = [&](int it) -> int {
		return WIDE ? r0 + wave + WAVES * (it / tpr) : r0 + rt * (wave + WAVES * it) + rsub;
	};
	auto item_chunk = [&](int it) -> int { return WIDE ? 64 * (it % tpr) + lane : sub; };

	// Weight loads are raw buffer loads, never predicated: pipeline slots with
	// no work (past the last item or row, idle lanes) use an offset past the
	// stream, which the hardware answers with zeros and no memory traffic. A
	// branch around a load would make the compiler wait for every outstanding
	// load (vmcnt(0)) before the activation prologue.
	const __amdgpu_buffer_rsrc_t wr = stream_rsrc(w, (uint32_t)(rb * n_out));
	auto issue = [&](Q4Buf &b, int it) {
		const int row = item_row(it), c = item_chunk(it);
		const bool on = it < nit && row < r1 && c < C;
		const uint32_t blk = on ? (uint32_t)((size_t)row * rb + (size_t)(c >> 2) * kQ4Bytes) : kBufNone;
		b.h = ld_b128(wr, blk);
		b.q0 = ld_b128(wr, blk + 16 + 32 * (c & 3));
		b.q1 = ld_b128(wr, blk + 32 + 32 * (c & 3));
	};

	// 1. activation loads first (they return first: loads complete in order).
	// Straight-line and unpredicated (clamped), so that the compiler counts
	// them exactly and waits only for them before quantizing.
	float4 xv[XP];
	int4 qv[XP];
	float sv[2];
	if (MODE == kFused) {
#pragma unroll
		for (int k = 0; k < XP; k++)
			xv[k] = *(const float4 *)(x + min((int)(threadIdx.x + k * T) * 4, n_in - 4));
	} else {
#pragma unroll
		for (int k = 0; k < XP; k++)
			qv[k] = *(const int4 *)(xq_g + min((int)(threadIdx.x + k * T) * 16, n_in - 16));
		if (MODE == kPreq) {
#pragma unroll
			for (int k = 0; k < 2; k++) sv[k] = xs_g[min((int)(threadIdx.x + k * T), (n_in >> 5) - 1)];
		}
	}
	// Keep the scheduler from moving the weight loads above the activation
	// loads: completion is in issue order, so x must be first in the queue.
	__builtin_amdgcn_sched_barrier(0);
	// 2. weight loads for the first items
	// Item loads go out in consumption order (the scheduler would otherwise
	// interleave them, and the first item would wait for all four).
	Q4Buf buf[kQ4Depth];
#pragma unroll
	for (int j = 0; j < kQ4Depth; j++) {
		issue(buf[j], j);
		__builtin_amdgcn_sched_barrier(0);
	}

	__builtin_amdgcn_sched_barrier(0);
	// 3. activation into LDS while the weights are in flight; quantized
	// unconditionally (clamped lanes repeat the last quad), stores predicated.
	if (MODE == kFused) {
#pragma unroll
		for (int k = 0; k < XP; k++) {
			const int e = (threadIdx.x + k * T) * 4;
			float sc;
			const uint32_t packed = q8_quant4(xv[k], sc);
			if (e < n_in) {
				*(uint32_t *)(xq_s + q8_lds_pos(e)) = packed;
				if ((threadIdx.x & 7) == 0) xs_s[e >> 5] = sc;
			}
		}
	} else {
#pragma unroll
		for (int k = 0; k < XP; k++) {
			const int e = (threadIdx.x + k * T) * 16;
			const int4 v = qv[k];
			if (e < n_in) *(int4 *)(xq_s + q8_lds_pos(e)) = v;
		}
#pragma unroll
		for (int k = 0; k < 2; k++) {
			const int e = threadIdx.x + k * T;
			const float v = MODE == kPreq ? sv[k] : 0.0f;
			if (e < (n_in >> 5)) xs_s[e] = v;
		}
	}
	__syncthreads();

	Q4Col col;
	if (!WIDE) q4_col(xq_s, xs_s, min(sub, C - 1), col);
	float acc = 0.0f;

	// Whole groups of kQ4Depth items, so every iteration issues the same
	// number of loads (slots past nit load nothing: out-of-range offsets).
	// Their arithmetic is skipped by a wave-uniform branch that holds no loads.
	for (int base = 0; base < nit; base += kQ4Depth) {
		float rsum[kQ4Depth];
#pragma unroll
		for (int j = 0; j < kQ4Depth; j++) {
			const int it = base + j;
			const int row = item_row(it), c = item_chunk(it);
			const bool valid = row < r1 && c < C;
			float f = 0.0f;
			int ia = 0, ib = 0;
			if (it < nit) {
				if (WIDE) q4_col(xq_s, xs_s, min(c, C - 1), col);
				// Consume buf[j] in place, then reload it: a copy would have to be
				// rotated back at the loop edge, waiting on the loads in flight.
				q4_isum(buf[j], col, ia, ib);
				if (MODE != kIsums) f = q4_fold(buf[j], 16u * (c & 1), (c & 3) >= 2 ? ~0u : 0u, ia, ib, col);
			}
			issue(buf[j], it + kQ4Depth);
			__builtin_amdgcn_sched_barrier(0);
			if (MODE == kIsums) {
				if (it < nit && valid) {
					const size_t o = (size_t)row * (n_in >> 5) + 2 * c;
					iqx_o[o] = ia;
					iqx_o[o + 1] = ib;
					ix_o[o] = col.ia_sum;
					ix_o[o + 1] = col.ib_sum;
				}
			} else if (WIDE) {
				// a row spans tpr items: accumulate, reduce at its last part
				acc += valid ? f : 0.0f;
				if (it < nit && (it % tpr) == tpr - 1) {
					const float tot = seg_sum(acc, 64);
					if (lane == 0 && row < r1) {
						if (bias)
							sum_s[row - r0] = tot;
						else
							out[row] = tot;
					}
					acc = 0.0f;
				}
			} else {
				rsum[j] = valid ? f : 0.0f;
			}
		}
		if (MODE != kIsums && !WIDE) {
			// lane with sub == j holds item j's row sum
			const float tot = seg_sum4(rsum, seg, lane);
			const int j = sub & 3;
			const int row = item_row(base + j);
			if (sub < kQ4Depth && base + j < nit && row < r1) {
				if (bias)
					sum_s[row - r0] = tot;
				else
					out[row] = tot;
			}
		}
	}
	// The bias is added after the weight stream: a bias load in the loop
	// would wait for every weight load in flight (loads complete in order).
	if (MODE != kIsums && bias) {
		__syncthreads();
		for (int r = threadIdx.x; r < nrows; r += T) out[r0 + r] = sum_s[r] + bias[r0 + r];
	}
}

// Flat grid for rows of at most 64 chunks (n_in <= 4096): a workgroup owns
// WAVES*ITEMS row items, a wave ITEMS consecutive ones, and every weight load
// of the wave is issued at once, right after the activation (and bias) loads.
// There is no loop: latency is hidden by the many workgroups resident on each
// CU rather than by a software pipeline.
template <int MODE, int XP, int WAVES, int ITEMS>
__global__ __launch_bounds__(WAVES * kWave) void q4k_gemv_flat_kernel(
    const uint8_t *__restrict__ w, const float *__restrict__ x, const int8_t *__restrict__ xq_g,
    const float *__restrict__ xs_g, const float *__restrict__ bias, float *__restrict__ out,
    int32_t *__restrict__ iqx_o, int32_t *__restrict__ ix_o, int n_out, int n_in) {
	extern __shared__ __align__(16) uint8_t smem[];
	int8_t *xq_s = (int8_t *)smem;
	float *xs_s = (float *)(smem + n_in);
	constexpr int T = WAVES * kWave;
	constexpr int NG = (ITEMS + 3) / 4;   // groups of four items reduced together
	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int NB = n_in >> 8, C = NB * 4;
	const int seg = next_pow2(C), rt = 64 / seg;
	const int sub = lane & (seg - 1), rsub = lane / seg;
	const size_t rb = (size_t)NB * kQ4Bytes;
	const int wrow0 = (blockIdx.x * WAVES + wave) * ITEMS * rt;
	auto item_row = [&](int it) -> int { return wrow0 + rt * it + rsub; };

	// 1. activation, then bias, loads (they complete first).
	float4 xv[XP];
	int4 qv[XP];
	float sv[2];
	if (MODE == kFused) {
#pragma unroll
		for (int k = 0; k < XP; k++)
			xv[k] = *(const float4 *)(x + min((int)(threadIdx.x + k * T) * 4, n_in - 4));
	} else {
#pragma unroll
		for (int k = 0; k < XP; k++)
			qv[k] = *(const int4 *)(xq_g + min((int)(threadIdx.x + k * T) * 16, n_in - 16));
		if (MODE == kPreq) {
#pragma unroll
			for (int k = 0; k < 2; k++) sv[k] = xs_g[min((int)(threadIdx.x + k * T), (n_in >> 5) - 1)];
		}
	}
	// The lane that writes item 4g + (sub & 3) loads that row's bias now; a
	// null bias reads out[] (in bounds, discarded).
	float bv[NG];
	if (MODE != kIsums) {
		const float *bsrc = bias ? bias : out;
#pragma unroll
		for (int g = 0; g < NG; g++) bv[g] = bsrc[min(item_row(4 * g + (sub & 3)), n_out - 1)];
	}
	__builtin_amdgcn_sched_barrier(0);
	// 2. every weight load of the wave, in consumption order
	const __amdgpu_buffer_rsrc_t wr = stream_rsrc(w, (uint32_t)(rb * n_out));
	Q4Buf buf[ITEMS];
#pragma unroll
	for (int j = 0; j < ITEMS; j++) {
		const int row = item_row(j);
		const bool on = row < n_out && sub < C;
		const uint32_t blk = on ? (uint32_t)((size_t)row * rb + (size_t)(sub >> 2) * kQ4Bytes) : kBufNone;
		buf[j].h = ld_b128(wr, blk);
		buf[j].q0 = ld_b128(wr, blk + 16 + 32 * (sub & 3));
		buf[j].q1 = ld_b128(wr, blk + 32 + 32 * (sub & 3));
		__builtin_amdgcn_sched_barrier(0);
	}
	// 3. activation into LDS while the weights are in flight
	if (MODE == kFused) {
#pragma unroll
		for (int k = 0; k < XP; k++) {
			const int e = (threadIdx.x + k * T) * 4;
			float sc;
			const uint32_t packed = q8_quant4(xv[k], sc);
			if (e < n_in) {
				*(uint32_t *)(xq_s + q8_lds_pos(e)) = packed;
				if ((threadIdx.x & 7) == 0) xs_s[e >> 5] = sc;
			}
		}
	} else {
#pragma unroll
		for (int k = 0; k < XP; k++) {
			const int e = (threadIdx.x + k * T) * 16;
			if (e < n_in) *(int4 *)(xq_s + q8_lds_pos(e)) = qv[k];
		}
#pragma unroll
		for (int k = 0; k < 2; k++) {
			const int e = threadIdx.x + k * T;
			if (e < (n_in >> 5)) xs_s[e] = MODE == kPreq ? sv[k] : 0.0f;
		}
	}
	__syncthreads();
	Q4Col col;
	q4_col(xq_s, xs_s, min(sub, C - 1), col);

	float rsum[4 * NG];
#pragma unroll
	for (int j = 0; j < 4 * NG; j++) {
		rsum[j] = 0.0f;
		if (j >= ITEMS) continue;
		const int row = item_row(j);
		const bool valid = row < n_out && sub < C;
		int ia, ib;
		q4_isum(buf[j], col, ia, ib);
		if (MODE == kIsums) {
			if (valid) {
				const size_t o = (size_t)row * (n_in >> 5) + 2 * sub;
				iqx_o[o] = ia;
				iqx_o[o + 1] = ib;
				ix_o[o] = col.ia_sum;
				ix_o[o + 1] = col.ib_sum;
			}
		} else {
			const float f = q4_fold(buf[j], 16u * (sub & 1), (sub & 3) >= 2 ? ~0u : 0u, ia, ib, col);
			rsum[j] = valid ? f : 0.0f;
		}
	}
	if (MODE != kIsums) {
#pragma unroll
		for (int g = 0; g < NG; g++) {
			const float tot = seg_sum4(rsum + 4 * g, seg, lane);
			const int j = 4 * g + (sub & 3);
			const int row = item_row(j);
			if ((sub >> 2) == 0 && j < ITEMS && row < n_out) out[row] = bias ? tot + bv[g] : tot;
		}
	}
}

constexpr int kMaxQ4Lds = 64 * 1024;
int g_q4_wgs_per_cu = 1;
int g_q4_waves = 4;
// -1: by shape (below); 0: persistent grid; 1, 2, 4, 8: flat grid with that many items per wave
int g_q4_flat_items = -1;

template <int MODE>
int q4_launch(const uint8_t *w, const float *x, const int8_t *xq, const float *xs, const float *bias,
              float *out, int32_t *iqx, int32_t *ix, int n_out, int n_in) {
	if (int rc = require_device()) return rc;
	if (n_out <= 0 || n_in <= 0 || n_in % kQK != 0)
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV needs n_out > 0 and n_in %% 256 == 0 (got %d x %d)",
		                 n_out, n_in);
	if (((uintptr_t)w & 15) || ((uintptr_t)x & 15) || ((uintptr_t)xq & 15) || ((uintptr_t)xs & 3))
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV needs w, x and xq 16-byte aligned");
	// 4-wave workgroups keep more of them in flight; very wide activations
	// need 8 waves to stage x in straight-line loads.
	const int waves = (g_q4_waves == 8 || n_in > 16 * 4 * 4 * kWave) ? 8 : 4, threads = waves * kWave;
	const size_t lds = (size_t)n_in + (size_t)(n_in / 32) * 4 + 2 * threads * sizeof(float);   // + row sums
	if (lds > (size_t)kMaxQ4Lds || n_in > 16 * 4 * threads)
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV n_in %d exceeds the LDS-resident limit", n_in);
	if ((size_t)n_out * (n_in / kQK) * kQ4Bytes >= kBufNone)
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV weight of %d x %d exceeds 2 GiB", n_out, n_in);
	const int C = n_in / kQK * 4;
	const bool wide = C > 64;
	int rows_per_item = 1;
	if (!wide) {
		int seg = 1;
		while (seg < C) seg <<= 1;
		rows_per_item = 64 / seg;
	}
	// By shape: the flat grid wins wherever the per-workgroup activation work
	// is small — always for a pre-quantized activation, and for the fused
	// quantization up to n_in = 2048; wider fused rows amortize the
	// quantization better over the persistent grid's longer row ranges.
	int items = g_q4_flat_items;
	if (items < 0) items = (MODE != kFused || n_in <= 2048) ? 2 : 0;
	if (!wide && items > 0) {
		const int per_wg = waves * items * rows_per_item;
		const int fwgs = (n_out + per_wg - 1) / per_wg;
		const size_t flds = (size_t)n_in + (size_t)(n_in / 32) * 4;
		const int per_round = MODE == kFused ? 4 * threads : 16 * threads;
		const int fxp = (n_in + per_round - 1) / per_round;
#define HK_Q4F(XP, WV, IT)                                                                                   \
	hipLaunchKernelGGL((q4k_gemv_flat_kernel<MODE, XP, WV, IT>), dim3(fwgs), dim3(WV * kWave), flds, stream(), \
	                   w, x, xq, xs, bias, out, iqx, ix, n_out, n_in)
#define HK_Q4F_IT(XP, WV)                         \
	do {                                          \
		if (items <= 1) HK_Q4F(XP, WV, 1);        \
		else if (items <= 2) HK_Q4F(XP, WV, 2);   \
		else if (items <= 4) HK_Q4F(XP, WV, 4);   \
		else HK_Q4F(XP, WV, 8);                   \
	} while (0)
#define HK_Q4F_XP(WV)                               \
	do {                                            \
		if (fxp <= 1) HK_Q4F_IT(1, WV);             \
		else if (fxp <= 2) HK_Q4F_IT(2, WV);        \
		else HK_Q4F_IT(4, WV);                      \
	} while (0)
		if (waves == 8)
			HK_Q4F_XP(8);
		else
			HK_Q4F_XP(4);
#undef HK_Q4F_XP
#undef HK_Q4F_IT
#undef HK_Q4F
		HK_LAUNCHED("q4k_gemv_flat");
		return ok();
	}
	// Persistent-style grid: a fixed number of workgroups per CU, each with a
	// contiguous row range, never more workgroups than give one item per wave.
	const int max_wgs = g_q4_wgs_per_cu * cu_count();
	const int min_rows = waves * rows_per_item;
	int wgs = (n_out + min_rows - 1) / min_rows;
	if (wgs > max_wgs) wgs = max_wgs;
	const int max_rows_per_wg = 2 * threads;   // row sums awaiting a bias, in LDS
	if ((n_out + wgs - 1) / wgs > max_rows_per_wg) wgs = (n_out + max_rows_per_wg - 1) / max_rows_per_wg;
	// activation quads per thread: 4 floats (fused) / 16 bytes per thread and round
	const int per_round = MODE == kFused ? 4 * threads : 16 * threads;
	const int xp = (n_in + per_round - 1) / per_round;
#define HK_Q4_LAUNCH(W, XP, WV)                                                                          \
	hipLaunchKernelGGL((q4k_gemv_kernel<MODE, W, XP, WV>), dim3(wgs), dim3(WV * kWave), lds, stream(), w, x, \
	                   xq, xs, bias, out, iqx, ix, n_out, n_in)
#define HK_Q4_LAUNCH_W(WV)                           \
	do {                                             \
		if (wide) {                                  \
			if (xp <= 4) HK_Q4_LAUNCH(true, 4, WV);  \
			else if (xp <= 8) HK_Q4_LAUNCH(true, 8, WV); \
			else HK_Q4_LAUNCH(true, 16, WV);         \
		} else {                                     \
			if (xp <= 1) HK_Q4_LAUNCH(false, 1, WV); \
			else if (xp <= 2) HK_Q4_LAUNCH(false, 2, WV); \
			else HK_Q4_LAUNCH(false, 4, WV);         \
		}                                            \
	} while (0)
	if (waves == 8)
		HK_Q4_LAUNCH_W(8);
	else
		HK_Q4_LAUNCH_W(4);
#undef HK_Q4_LAUNCH_W
#undef HK_Q4_LAUNCH
	HK_LAUNCHED("q4k_gemv");
	return ok();
}

}  // namespace

// Fused quantize + GEMV on device pointers (used by hako_gpu_matmul).
int q4k_matmul_fused(float *out, const float *x, const void *w, const float *bias, int n_out, int n_in) {
	return q4_launch<kFused>((const uint8_t *)w, x, nullptr, nullptr, bias, out, nullptr, nullptr, n_out,
	                         n_in);
}

void q4k_set_wgs_per_cu(int v) { g_q4_wgs_per_cu = v < 1 ? 1 : (v > 8 ? 8 : v); }
void q4k_set_waves(int v) { g_q4_waves = v >= 8 ? 8 : 4; }
void q4k_set_flat_items(int v) { g_q4_flat_items = v < 0 ? -1 : (v == 0 ? 0 : (v <= 1 ? 1 : (v <= 2 ? 2 : (v <= 4 ? 4 : 8)))); }

}  // namespace hako

extern "C" int hako_gpu_q4k_gemv(float *out, const void *w, const int8_t *xq, const float *xs,
                                 const float *bias, int n_out, int n_in) {
	return hako::q4_launch<hako::kPreq>((const uint8_t *)w, nullptr, xq, xs, bias, out, nullptr, nullptr,
	                                    n_out, n_in);
}

extern "C" int hako_gpu_q4k_isums(int32_t *iqx, int32_t *ix, const void *w, const int8_t *xq,
                                  int n_out, int n_in) {
	// The integer path reads no scales.
	return hako::q4_launch<hako::kIsums>((const uint8_t *)w, nullptr, xq, nullptr, nullptr, nullptr, iqx,
	                                     ix, n_out, n_in);
}
