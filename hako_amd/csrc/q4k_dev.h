// q4k_dev.h — lane-level Q4_K x q8 arithmetic shared by the GEMV kernels.
//
// A "chunk" is one 64-weight group g of a 144-byte block: 32 qs bytes whose
// low nibbles are sub-block 2g and high nibbles sub-block 2g+1 (reference
// src/quant.c:68-92), so a lane that owns a chunk owns whole sub-blocks and its
// integer sums are the reference's iqx / ix exactly (src/quant.c:214-220).
#pragma once
#include "hako_dev.h"

namespace hako {

struct Q4Buf {
	uint4 h, q0, q1;   // block header (d, dmin, scales), 32 qs bytes
};

// Activation state of one chunk for this lane.
struct Q4Col {
	int xa[8], xb[8];   // xq of sub-blocks 2g (paired with low nibbles) and 2g+1
	float xsa, xsb;     // their q8 scales
	float ixa, ixb;     // xs * Σxq of each sub-block
	int ia_sum, ib_sum; // Σxq of each sub-block (integer-sums mode)
};

// Place of byte e of a q8 activation row in LDS: the four 16-byte pieces of
// each 64-byte chunk c (one lane's two sub-blocks) are rotated by c/4, so
// that the 16-byte reads of sixteen neighbouring lanes' chunks (one piece
// each) fall in distinct banks (unrotated, chunks 64 bytes apart share four
// bank groups). Whole pieces stay contiguous.
__device__ __forceinline__ int q8_lds_pos(int e) {
	const int c = e >> 6, k = (e >> 4) & 3;
	return (e & ~63) | (((k + (c >> 2)) & 3) << 4) | (e & 15);
}

__device__ __forceinline__ void q4_col(const int8_t *xq_s, const float *xs_s, int c, Q4Col &col) {
	const int i = c >> 2, g = c & 3, rot = i & 3;
	const int8_t *p = xq_s + 64 * c;
	const int4 a0 = *(const int4 *)(p + 16 * (rot & 3)), a1 = *(const int4 *)(p + 16 * ((1 + rot) & 3));
	const int4 b0 = *(const int4 *)(p + 16 * ((2 + rot) & 3)), b1 = *(const int4 *)(p + 16 * ((3 + rot) & 3));
	col.xa[0] = a0.x; col.xa[1] = a0.y; col.xa[2] = a0.z; col.xa[3] = a0.w;
	col.xa[4] = a1.x; col.xa[5] = a1.y; col.xa[6] = a1.z; col.xa[7] = a1.w;
	col.xb[0] = b0.x; col.xb[1] = b0.y; col.xb[2] = b0.z; col.xb[3] = b0.w;
	col.xb[4] = b1.x; col.xb[5] = b1.y; col.xb[6] = b1.z; col.xb[7] = b1.w;
	const float2 s = *(const float2 *)(xs_s + 8 * i + 2 * g);
	col.xsa = s.x;
	col.xsb = s.y;
	int sa = 0, sb = 0;
#pragma unroll
	for (int k = 0; k < 8; k++) {
		sa = sdot4(col.xa[k], 0x01010101, sa);
		sb = sdot4(col.xb[k], 0x01010101, sb);
	}
	col.ia_sum = sa;
	col.ib_sum = sb;
	col.ixa = s.x * (float)sa;
	col.ixb = s.y * (float)sb;
}

// Σ q·xq over the 32 low nibbles (sub-block 2g) and 32 high nibbles (2g+1).
__device__ __forceinline__ void q4_isum(const Q4Buf &b, const Q4Col &c, int &ia, int &ib) {
	const uint32_t m = 0x0F0F0F0Fu;
	const uint32_t q[8] = {b.q0.x, b.q0.y, b.q0.z, b.q0.w, b.q1.x, b.q1.y, b.q1.z, b.q1.w};
	ia = 0;
	ib = 0;
#pragma unroll
	for (int k = 0; k < 8; k++) {
		ia = sdot4((int)(q[k] & m), c.xa[k], ia);
		ib = sdot4((int)((q[k] >> 4) & m), c.xb[k], ib);
	}
}

// d*(xsA*sA*ia + xsB*sB*ib) - dmin*(mA*xsA*ixA + mB*xsB*ixB). `sh` = 16*(g&1)
// brings scale bytes 2g&3, (2g+1)&3 to the bottom; `hi` = (g >= 2) selects the
// split 6-bit layout of sub-blocks 4-7 (reference quant.c:57-66).
// `hmask` is all ones for g >= 2, zero otherwise (a lane constant, blended
// without branches).
// The 6-bit (scale, min) pairs of sub-blocks 2g and 2g+1 from the three
// scale words of a block header: S holds s(2g) in bits 0-7 and s(2g+1) in
// bits 8-15, M the mins alike.
__device__ __forceinline__ void q4_scales2(uint32_t hy, uint32_t hz, uint32_t hw, uint32_t sh, uint32_t hmask,
                                           uint32_t &S, uint32_t &M) {
	const uint32_t a0 = hy >> sh, a1 = hz >> sh, a2 = hw >> sh;
	const uint32_t s_lo = a0 & 0x3F3Fu, m_lo = a1 & 0x3F3Fu;
	const uint32_t s_hi = (a2 & 0x0F0Fu) | ((a0 >> 2) & 0x3030u);
	const uint32_t m_hi = ((a2 >> 4) & 0x0F0Fu) | ((a1 >> 2) & 0x3030u);
	S = s_lo ^ ((s_lo ^ s_hi) & hmask);
	M = m_lo ^ ((m_lo ^ m_hi) & hmask);
}

__device__ __forceinline__ float q4_fold(const Q4Buf &b, uint32_t sh, uint32_t hmask, int ia, int ib,
                                         const Q4Col &c) {
	const float d = f16_to_f32(b.h.x & 0xFFFFu), dmin = f16_to_f32(b.h.x >> 16);
	uint32_t S, M;
	q4_scales2(b.h.y, b.h.z, b.h.w, sh, hmask, S, M);
	const float sA = (float)(S & 0xFFu), sB = (float)((S >> 8) & 0xFFu);
	const float mA = (float)(M & 0xFFu), mB = (float)((M >> 8) & 0xFFu);
	const float t1 = (c.xsa * sA) * (float)ia + (c.xsb * sB) * (float)ib;
	const float t2 = mA * c.ixa + mB * c.ixb;
	return d * t1 - dmin * t2;
}

}  // namespace hako
