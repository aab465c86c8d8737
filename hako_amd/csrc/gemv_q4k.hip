// gemv_q4k.hip — Q4_K x q8 GEMV for batch-1 decode (gfx950).
//
// Replaces the reference's row loop over q4k_vec_dot (src/nn.c:76-82,
// src/quant.c:150-232). The weight matrix is the verbatim stream of 144-byte
// super-blocks, n_in/256 per row.
//
// Work split. A row is cut into chunks of 16 qs bytes (8 per block, 32
// weights each): chunk c covers block i = c/8, qs bytes 16*(c%8)..+16, whose
// low nibbles belong to sub-block 2g (g = (c%8)/2) and high nibbles to
// sub-block 2g+1. Lane l of a wave takes chunks l, l+64, ... of a row, so a
// wave-wide load of a row's chunks is one contiguous 1 KiB run, and the
// activation columns a lane needs never change from row to row. Each lane
// also loads its block's 16-byte header (d, dmin, 12 scale bytes); the eight
// lanes of a block hit the same 16 bytes.
//
// A workgroup is 4 waves. KS waves share a row group and split its 64-chunk
// tiles between them (tile T goes to wave T % KS); each wave keeps R rows in
// flight, issuing the next tile's loads before it computes the current one.
//
// The activation lives in LDS as q8: either quantized there by the workgroup
// itself from the fp32 x (the fused path: quantize_row_q8_32 once per row, per
// workgroup, while the first weight loads are in flight), or copied from a
// pre-quantized xq/xs.
//
// Integer work per chunk: 8 v_dot4_i32_i8 over the nibbles, exact in int32
// (|sum| <= 15*127*32). The fp32 fold per sub-block is the reference's
// xs*(d*s*iqx - dmin*m*ix); the lane partial sums are added in a wave tree,
// so only the fold's association differs from the reference.
#include "hako_dev.h"
#include "hako_rt.h"

namespace hako {
namespace {

enum Q4Mode { kFused = 0, kPreq = 1, kIsums = 2 };

// The per-lane activation state of one chunk: the 16 xq values of each of its
// two sub-blocks that pair with its 16 qs bytes, their scales and partial Σxq.
struct Q4Col {
	int xa0, xa1, xa2, xa3, xb0, xb1, xb2, xb3;
	float xsa, xsb;
	int ixa, ixb;
};

__device__ __forceinline__ Q4Col q4_col(const int8_t *xq_s, const float *xs_s, int c) {
	const int i = c >> 3, p = c & 7, g = p >> 1, half = p & 1;
	const int base = kQK * i + 64 * g + 16 * half;
	const int4 a = *(const int4 *)(xq_s + base);
	const int4 b = *(const int4 *)(xq_s + base + 32);
	const float2 s = *(const float2 *)(xs_s + 8 * i + 2 * g);
	Q4Col col;
	col.xa0 = a.x; col.xa1 = a.y; col.xa2 = a.z; col.xa3 = a.w;
	col.xb0 = b.x; col.xb1 = b.y; col.xb2 = b.z; col.xb3 = b.w;
	col.xsa = s.x;
	col.xsb = s.y;
	const int ones = 0x01010101;
	col.ixa = sdot4(a.w, ones, sdot4(a.z, ones, sdot4(a.y, ones, sdot4(a.x, ones, 0))));
	col.ixb = sdot4(b.w, ones, sdot4(b.z, ones, sdot4(b.y, ones, sdot4(b.x, ones, 0))));
	return col;
}

// Σ q·xq over the chunk's 16 low nibbles (sub-block 2g) and 16 high nibbles
// (sub-block 2g+1).
__device__ __forceinline__ void q4_isum(uint4 q, const Q4Col &c, int &ia, int &ib) {
	const uint32_t m = 0x0F0F0F0Fu;
	ia = sdot4((int)(q.x & m), c.xa0, 0);
	ia = sdot4((int)(q.y & m), c.xa1, ia);
	ia = sdot4((int)(q.z & m), c.xa2, ia);
	ia = sdot4((int)(q.w & m), c.xa3, ia);
	ib = sdot4((int)((q.x >> 4) & m), c.xb0, 0);
	ib = sdot4((int)((q.y >> 4) & m), c.xb1, ib);
	ib = sdot4((int)((q.z >> 4) & m), c.xb2, ib);
	ib = sdot4((int)((q.w >> 4) & m), c.xb3, ib);
}

// xs·(d·s·iqx − dmin·m·ix) for both sub-blocks of the chunk (reference
// quant.c:222-225); h is the block header (d, dmin, scales as 4 dwords).
__device__ __forceinline__ float q4_fold(uint4 h, int g, int ia, int ib, const Q4Col &c) {
	const float d = f16_to_f32(h.x & 0xFFFFu), dmin = f16_to_f32(h.x >> 16);
	uint32_t sa, ma, sb, mb;
	scale_min_k4(2u * g, h.y, h.z, h.w, sa, ma);
	scale_min_k4(2u * g + 1u, h.y, h.z, h.w, sb, mb);
	const float ta = d * (float)sa * (float)ia - dmin * (float)ma * (float)c.ixa;
	const float tb = d * (float)sb * (float)ib - dmin * (float)mb * (float)c.ixb;
	return c.xsa * ta + c.xsb * tb;
}

template <int MODE, int R, int KS, bool MULTI>
__global__ __launch_bounds__(256) void q4k_gemv_kernel(
    const uint8_t *__restrict__ w, const float *__restrict__ x, const int8_t *__restrict__ xq_g,
    const float *__restrict__ xs_g, const float *__restrict__ bias, float *__restrict__ out,
    int32_t *__restrict__ iqx_o, int32_t *__restrict__ ix_o, int n_out, int n_in) {
	extern __shared__ __align__(16) uint8_t smem[];
	int8_t *xq_s = (int8_t *)smem;
	float *xs_s = (float *)(smem + n_in);
	float *red_s = xs_s + (n_in >> 5);   // [4 waves][R]

	const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
	const int wk = wave % KS, wr = wave / KS;
	const int row0 = (blockIdx.x * (4 / KS) + wr) * R;
	const int NB = n_in >> 8, C = NB << 3, tiles = (C + 63) >> 6;
	const size_t rb = (size_t)NB * kQ4Bytes;

	auto load = [&](int T, uint4 *q, uint4 *h) {
		const int c = (T << 6) + lane;
		const int i = c >> 3, p = c & 7;
#pragma unroll
		for (int r = 0; r < R; r++) {
			const int row = row0 + r;
			if (c < C && row < n_out) {
				const uint8_t *blk = w + (size_t)row * rb + (size_t)i * kQ4Bytes;
				h[r] = *(const uint4 *)blk;
				q[r] = *(const uint4 *)(blk + 16 + 16 * p);
			} else {
				h[r] = make_uint4(0, 0, 0, 0);
				q[r] = make_uint4(0, 0, 0, 0);
			}
		}
	};

	// Weight loads for the first tile go out before the activation prologue.
	uint4 qn[R], hn[R];
	if (wk < tiles) load(wk, qn, hn);

	if (MODE == kFused) {
		// 8 lanes per 32-block, 4 floats per lane.
		for (int e = threadIdx.x * 4; e < n_in; e += 1024) {
			const float4 v = *(const float4 *)(x + e);
			float sc;
			const uint32_t packed = q8_quant4(v, sc);
			*(uint32_t *)(xq_s + e) = packed;
			if ((threadIdx.x & 7) == 0) xs_s[e >> 5] = sc;
		}
	} else {
		for (int e = threadIdx.x * 16; e < n_in; e += 4096)
			*(int4 *)(xq_s + e) = *(const int4 *)(xq_g + e);
		for (int e = threadIdx.x; e < (n_in >> 5); e += 256) xs_s[e] = xs_g[e];
	}
	__syncthreads();

	float acc[R];
#pragma unroll
	for (int r = 0; r < R; r++) acc[r] = 0.0f;

	for (int T = wk; T < tiles; T += KS) {
		uint4 q[R], h[R];
#pragma unroll
		for (int r = 0; r < R; r++) {
			q[r] = qn[r];
			h[r] = hn[r];
		}
		if (MULTI && T + KS < tiles) load(T + KS, qn, hn);
		const int c = (T << 6) + lane;
		if (c < C) {
			const Q4Col col = q4_col(xq_s, xs_s, c);
			const int g = (c & 7) >> 1;
#pragma unroll
			for (int r = 0; r < R; r++) {
				int ia, ib;
				q4_isum(q[r], col, ia, ib);
				if (MODE == kIsums) {
					// Lanes c and c^1 hold the two halves of each sub-block.
					const int ia_t = ia + dpp_i<kDppQuadSwap1>(ia);
					const int ib_t = ib + dpp_i<kDppQuadSwap1>(ib);
					const int xa_t = col.ixa + dpp_i<kDppQuadSwap1>(col.ixa);
					const int xb_t = col.ixb + dpp_i<kDppQuadSwap1>(col.ixb);
					const int row = row0 + r;
					if ((c & 1) == 0 && row < n_out) {
						const size_t o = (size_t)row * (n_in >> 5) + 8 * (c >> 3) + 2 * g;
						iqx_o[o] = ia_t;
						iqx_o[o + 1] = ib_t;
						ix_o[o] = xa_t;
						ix_o[o + 1] = xb_t;
					}
				} else {
					acc[r] += q4_fold(h[r], g, ia, ib, col);
				}
			}
		}
	}

	if (MODE != kIsums) {
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
}

struct Q4Plan {
	int R, KS, wgs;
	bool multi;
	size_t lds;
};

constexpr int kMaxQ4Lds = 64 * 1024;

int q4_plan(int n_out, int n_in, Q4Plan &p) {
	if (n_out <= 0 || n_in <= 0 || n_in % kQK != 0)
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV needs n_out > 0 and n_in %% 256 == 0 (got %d x %d)",
		                 n_out, n_in);
	const int tiles = (n_in / kQK * 8 + 63) / 64;
	p.KS = tiles >= 4 ? 4 : (tiles >= 2 ? 2 : 1);
	p.multi = tiles > p.KS;
	p.R = 1;
	for (int R : {4, 2}) {
		const int rows_per_wg = R * 4 / p.KS;
		if ((n_out + rows_per_wg - 1) / rows_per_wg >= 512) {
			p.R = R;
			break;
		}
	}
	const int rows_per_wg = p.R * 4 / p.KS;
	p.wgs = (n_out + rows_per_wg - 1) / rows_per_wg;
	p.lds = (size_t)n_in + (size_t)(n_in / 32) * 4 + 16 * 4 * sizeof(float);
	if (p.lds > (size_t)kMaxQ4Lds)
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV n_in %d exceeds the LDS-resident limit", n_in);
	return HAKO_GPU_OK;
}

template <int MODE, int R, int KS, bool MULTI>
int q4_launch_rkm(const Q4Plan &p, const uint8_t *w, const float *x, const int8_t *xq,
                  const float *xs, const float *bias, float *out, int32_t *iqx, int32_t *ix,
                  int n_out, int n_in) {
	hipLaunchKernelGGL((q4k_gemv_kernel<MODE, R, KS, MULTI>), dim3(p.wgs), dim3(256), p.lds, stream(),
	                   w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	HK_LAUNCHED("q4k_gemv");
	return ok();
}

template <int MODE, int R, int KS>
int q4_launch_rk(const Q4Plan &p, const uint8_t *w, const float *x, const int8_t *xq, const float *xs,
                 const float *bias, float *out, int32_t *iqx, int32_t *ix, int n_out, int n_in) {
	return p.multi ? q4_launch_rkm<MODE, R, KS, true>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in)
	               : q4_launch_rkm<MODE, R, KS, false>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
}

template <int MODE, int R>
int q4_launch_r(const Q4Plan &p, const uint8_t *w, const float *x, const int8_t *xq, const float *xs,
                const float *bias, float *out, int32_t *iqx, int32_t *ix, int n_out, int n_in) {
	switch (p.KS) {
	case 1: return q4_launch_rk<MODE, R, 1>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	case 2: return q4_launch_rk<MODE, R, 2>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	default: return q4_launch_rk<MODE, R, 4>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	}
}

template <int MODE>
int q4_launch(const uint8_t *w, const float *x, const int8_t *xq, const float *xs, const float *bias,
              float *out, int32_t *iqx, int32_t *ix, int n_out, int n_in) {
	if (int rc = require_device()) return rc;
	if (((uintptr_t)w & 15) || ((uintptr_t)x & 15) || ((uintptr_t)xq & 15) || ((uintptr_t)xs & 3))
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMV needs w, x and xq 16-byte aligned");
	Q4Plan p;
	if (int rc = q4_plan(n_out, n_in, p)) return rc;
	switch (p.R) {
	case 4: return q4_launch_r<MODE, 4>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	case 2: return q4_launch_r<MODE, 2>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	default: return q4_launch_r<MODE, 1>(p, w, x, xq, xs, bias, out, iqx, ix, n_out, n_in);
	}
}

}  // namespace

// Fused quantize + GEMV on device pointers (used by hako_gpu_matmul).
int q4k_matmul_fused(float *out, const float *x, const void *w, const float *bias, int n_out, int n_in) {
	return q4_launch<kFused>((const uint8_t *)w, x, nullptr, nullptr, bias, out, nullptr, nullptr,
	                         n_out, n_in);
}

}  // namespace hako

extern "C" int hako_gpu_q4k_gemv(float *out, const void *w, const int8_t *xq, const float *xs,
                                 const float *bias, int n_out, int n_in) {
	return hako::q4_launch<hako::kPreq>((const uint8_t *)w, nullptr, xq, xs, bias, out, nullptr, nullptr,
	                                    n_out, n_in);
}

extern "C" int hako_gpu_q4k_isums(int32_t *iqx, int32_t *ix, const void *w, const int8_t *xq,
                                  int n_out, int n_in) {
	// The integer path never reads xs; any readable buffer of n_in/32 floats
	// serves, and xq itself is at least that long.
	return hako::q4_launch<hako::kIsums>((const uint8_t *)w, nullptr, xq, (const float *)xq, nullptr,
	                                     nullptr, iqx, ix, n_out, n_in);
}
