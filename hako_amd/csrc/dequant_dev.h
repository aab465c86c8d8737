// dequant_dev.h — k-quant dequantization of one 32-weight chunk per call.
// Dequantized values are exact products rounded once, so any evaluation
// order gives the reference's bits.
#pragma once
#include "hako_dev.h"

namespace hako {

// dequant_q4_K (reference quant.c:68-92), chunk c = 16 qs bytes (32 weights)
// of block c/8 of the stream w, into y (the whole stream's output).
__device__ __forceinline__ void dq4_chunk(const uint8_t *__restrict__ w, int64_t c, float *__restrict__ y) {
	{
		const int64_t i = c >> 3;
		const int p = (int)(c & 7), g = p >> 1, half = p & 1;
		const uint8_t *blk = w + i * kQ4Bytes;
		const uint4 h = *(const uint4 *)blk;
		const uint4 q = *(const uint4 *)(blk + 16 + 16 * p);
		const float d = f16_to_f32(h.x & 0xFFFFu), dmin = f16_to_f32(h.x >> 16);
		uint32_t sa, ma, sb, mb;
		scale_min_k4(2u * g, h.y, h.z, h.w, sa, ma);
		scale_min_k4(2u * g + 1u, h.y, h.z, h.w, sb, mb);
		const float da = d * (float)sa, mna = dmin * (float)ma;
		const float db = d * (float)sb, mnb = dmin * (float)mb;
		float *ya = y + i * kQK + 64 * g + 16 * half, *yb = ya + 32;
		const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
		for (int u = 0; u < 4; u++) {
			float4 va, vb;
			va.x = da * (float)((qw[u] >> 0) & 0xF) - mna;
			va.y = da * (float)((qw[u] >> 8) & 0xF) - mna;
			va.z = da * (float)((qw[u] >> 16) & 0xF) - mna;
			va.w = da * (float)((qw[u] >> 24) & 0xF) - mna;
			vb.x = db * (float)((qw[u] >> 4) & 0xF) - mnb;
			vb.y = db * (float)((qw[u] >> 12) & 0xF) - mnb;
			vb.z = db * (float)((qw[u] >> 20) & 0xF) - mnb;
			vb.w = db * (float)((qw[u] >> 28) & 0xF) - mnb;
			*(float4 *)(ya + 4 * u) = va;
			*(float4 *)(yb + 4 * u) = vb;
		}
	}
}

__device__ __forceinline__ uint2 ld_u2(const uint8_t *p) {
	uint2 v;
	__builtin_memcpy(&v, p, 8);
	return v;
}

// dequant_q6_K (reference quant.c:94-123), chunk c = 8 per block: the 32
// weights 128n + 32k + l0 + j (k < 4, j < 8) of half n = s/4, l0 = 8*(s%4).
__device__ __forceinline__ void dq6_chunk(const uint8_t *__restrict__ w, int64_t c, float *__restrict__ y) {
	{
		const int64_t i = c >> 3;
		const int s = (int)(c & 7), n = s >> 2, l0 = 8 * (s & 3), sel = l0 >> 4;
		const uint8_t *blk = w + i * kQ6Bytes;
		const uint2 a = ld_u2(blk + 64 * n + l0), b = ld_u2(blk + 64 * n + 32 + l0);
		const uint2 hq = ld_u2(blk + 128 + 32 * n + l0);
		const int8_t *sc = (const int8_t *)(blk + 192 + 8 * n);
		const float d = f16_to_f32(*(const uint16_t *)(blk + 208));
		float *yb = y + i * kQK + 128 * n + l0;
#pragma unroll
		for (int k = 0; k < 4; k++) {
			const float dk = d * (float)sc[sel + 2 * k];
			const uint2 lw = (k & 1) ? b : a;
			float o[8];
#pragma unroll
			for (int j = 0; j < 8; j++) {
				const uint32_t lb = ((j < 4 ? lw.x : lw.y) >> (8 * (j & 3))) & 0xFFu;
				const uint32_t hb = ((j < 4 ? hq.x : hq.y) >> (8 * (j & 3))) & 0xFFu;
				const int lo4 = (k & 2) ? (int)(lb >> 4) : (int)(lb & 0xF);
				const int q = (lo4 | (int)(((hb >> (2 * k)) & 3u) << 4)) - 32;
				o[j] = dk * (float)q;
			}
			*(float4 *)(yb + 32 * k) = make_float4(o[0], o[1], o[2], o[3]);
			*(float4 *)(yb + 32 * k + 4) = make_float4(o[4], o[5], o[6], o[7]);
		}
	}
}

}  // namespace hako
