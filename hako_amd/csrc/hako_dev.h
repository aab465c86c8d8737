// hako_dev.h — device helpers shared by the gfx950 kernels.
//
// Wave64 throughout: reductions use DPP inside 16-lane rows and two
// cross-row swaps, never 32-lane warp idioms.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hako {

constexpr int kWave = 64;
constexpr int kQK = 256;          // weights per super-block (reference quant.h:9)
constexpr int kQ4Bytes = 144;     // block_q4_K (reference quant.h:12-17)
constexpr int kQ6Bytes = 210;     // block_q6_K (reference quant.h:19-24)
constexpr float kFltMin = 1.17549435e-38f;

// Exact binary16 -> binary32 (v_cvt_f32_f16; fp16 denormals are kept in the
// default HIP float mode, so every input converts exactly).
__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
	return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// Binary32 subnormal -> 0: the reference runs with FTZ/DAZ (its -ffast-math
// build links gcc's crtfastmath), so its q8 quantizer never sees or makes a
// subnormal. Stated explicitly so the result does not depend on the GPU's
// denormal mode.
__device__ __forceinline__ float ftz(float v) { return __builtin_fabsf(v) < kFltMin ? 0.0f : v; }

// silu (reference src/nn.c:29)
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
	return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
	return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

// DPP controls (gfx9): quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror (lane i <-> 7-i within 8), row_mirror (i <-> 15-i within 16).
constexpr int kDppQuadSwap1 = 0xB1;
constexpr int kDppQuadSwap2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;
constexpr int kDppRowRor4 = 0x124;   // row_ror:4 (rotate within 16 lanes)
constexpr int kDppRowRor8 = 0x128;   // row_ror:8

// Sum over all 64 lanes; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
	v += dpp_f<kDppQuadSwap1>(v);
	v += dpp_f<kDppQuadSwap2>(v);
	v += dpp_f<kDppHalfMirror>(v);
	v += dpp_f<kDppMirror>(v);
	v += __shfl_xor(v, 16);
	v += __shfl_xor(v, 32);
	return v;
}

// Maximum over all 64 lanes; every lane receives it.
__device__ __forceinline__ float wave_max(float v) {
	v = __builtin_fmaxf(v, dpp_f<kDppQuadSwap1>(v));
	v = __builtin_fmaxf(v, dpp_f<kDppQuadSwap2>(v));
	v = __builtin_fmaxf(v, dpp_f<kDppHalfMirror>(v));
	v = __builtin_fmaxf(v, dpp_f<kDppMirror>(v));
	v = __builtin_fmaxf(v, __shfl_xor(v, 16));
	v = __builtin_fmaxf(v, __shfl_xor(v, 32));
	return v;
}

// Sum over aligned segments of `seg` lanes (a power of two, 4..64); every
// lane of a segment receives the segment's sum.
__device__ __forceinline__ float seg_sum(float v, int seg) {
	v += dpp_f<kDppQuadSwap1>(v);
	v += dpp_f<kDppQuadSwap2>(v);
	if (seg >= 8) v += dpp_f<kDppHalfMirror>(v);
	if (seg >= 16) v += dpp_f<kDppMirror>(v);
	if (seg >= 32) v += __shfl_xor(v, 16);
	if (seg >= 64) v += __shfl_xor(v, 32);
	return v;
}

// Four segment sums at once: v[j] is this lane's share of item j; lane L
// receives the sum of item (L & 3) over its segment of `seg` lanes (a power of
// two, 4..64). Two transposing swaps inside the quad halve the values each
// time, then one value per lane is summed over the lanes of equal L & 3 —
// one cross-row exchange per four items instead of one per item.
__device__ __forceinline__ float seg_sum4(const float v[4], int seg, int lane) {
	const bool odd = lane & 1, hi = lane & 2;
	const float ka = odd ? v[1] : v[0], kb = odd ? v[3] : v[2];
	const float sa = odd ? v[0] : v[1], sb = odd ? v[2] : v[3];
	const float wa = ka + dpp_f<kDppQuadSwap1>(sa), wb = kb + dpp_f<kDppQuadSwap1>(sb);
	float u = (hi ? wb : wa) + dpp_f<kDppQuadSwap2>(hi ? wa : wb);
	if (seg == 8) u += __shfl_xor(u, 4);
	if (seg >= 16) {
		u += dpp_f<kDppRowRor4>(u);
		u += dpp_f<kDppRowRor8>(u);
	}
	if (seg >= 32) u += __shfl_xor(u, 16);
	if (seg >= 64) u += __shfl_xor(u, 32);
	return u;
}

// Max over aligned groups of 8 lanes; every lane of the group receives it.
__device__ __forceinline__ float max8(float v) {
	v = __builtin_fmaxf(v, dpp_f<kDppQuadSwap1>(v));
	v = __builtin_fmaxf(v, dpp_f<kDppQuadSwap2>(v));
	v = __builtin_fmaxf(v, dpp_f<kDppHalfMirror>(v));
	return v;
}

// Raw buffer access to a weight stream. Buffer loads are range-checked by
// the hardware: an offset at or past `bytes` returns zeros without touching
// memory, so pipeline slots with no work (past the last row, idle lanes) can
// issue their loads unconditionally at no bandwidth cost.
constexpr int kBufFlags = 0x00020000;      // raw (stride 0) 32-bit-format descriptor word 3
constexpr uint32_t kBufNone = 0x80000000u; // an offset past every stream (streams < 2 GiB)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t stream_rsrc(const void *base, uint32_t bytes) {
	return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, kBufFlags);
}
// A pointer the compiler cannot prove wave-uniform (it is) in scalar
// registers, so that a descriptor built on it needs no per-lane loop.
template <class P>
__device__ __forceinline__ P *uniform_ptr(P *p) {
	const uint64_t v = (uint64_t)(uintptr_t)p;
	const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
	return (P *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float ld_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
	return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ __forceinline__ void st_f32(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
	__builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, (int)off, 0, 0);
}
__device__ __forceinline__ uint4 ld_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
	return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint2 ld_b64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
	return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}
__device__ __forceinline__ uint32_t ld_b16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
	return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, 0);
}

__host__ __device__ __forceinline__ int next_pow2(int v) {
	int p = 1;
	while (p < v) p <<= 1;
	return p;
}

// v_dot4_i32_i8: c + sum of the four signed byte products of a and b.
__device__ __forceinline__ int sdot4(int a, int b, int c) {
	return __builtin_amdgcn_sdot4(a, b, c, false);
}

// Q4_K 6-bit (scale, min) of sub-block j in [0,8) from the 12 scale bytes held
// as three little-endian dwords s0 = bytes 0-3, s1 = 4-7, s2 = 8-11
// (layout of reference quant.c:57-66: sub-blocks 0-3 use the low six bits of
// bytes j and j+4; sub-blocks 4-7 take a nibble of byte j+4 and the top two
// bits of bytes j-4 and j).
__device__ __forceinline__ void scale_min_k4(uint32_t j, uint32_t s0, uint32_t s1, uint32_t s2,
                                             uint32_t &s, uint32_t &m) {
	const uint32_t sh = 8u * (j & 3u);
	const uint32_t b0 = (s0 >> sh) & 0xFFu, b1 = (s1 >> sh) & 0xFFu, b2 = (s2 >> sh) & 0xFFu;
	if (j < 4u) {
		s = b0 & 63u;
		m = b1 & 63u;
	} else {
		s = (b2 & 0xFu) | ((b0 >> 6) << 4);
		m = (b2 >> 4) | ((b1 >> 6) << 4);
	}
}

// q8_32 of one block (reference quant.c:127-144 as compiled with
// -ffast-math): inputs flushed to zero below FLT_MIN, xs = amax*RN(1/127),
// inv = RN(127/amax) when xs > 0, codes round-half-even clamped to +-127.
// The reference's maximum starts at 0 and takes only larger values, so NaN
// inputs never enter it: a block of NaNs has amax 0 (here a NaN maximum,
// which only an all-NaN block yields under fmaxf, is taken as 0).
// A product that is not finite (only from inf/NaN inputs) converts to 0, as
// the reference's 64-bit conversion yields the "indefinite" value whose low
// 32 bits are 0. Clamping in float keeps the int conversion defined.
__device__ __forceinline__ float q8_xs(float amax) {   // RN(1/127) = 0x3C010204
	return ftz(__builtin_fmaxf(amax, 0.0f) * 0x1.020408p-7f);
}
__device__ __forceinline__ float q8_inv(float amax, float xs) { return xs > 0.0f ? 127.0f / amax : 0.0f; }
__device__ __forceinline__ uint32_t q8_code(float a, float inv) {
	float r = __builtin_rintf(a * inv);
	r = __builtin_isfinite(r) ? r : 0.0f;
	r = __builtin_fminf(__builtin_fmaxf(r, -127.0f), 127.0f);
	return (uint32_t)((int)r & 0xFF);
}

// q8_32 quantization of four consecutive floats held by one lane, eight lanes
// per 32-block (lanes 8k..8k+7 of the wave own block k of the call). Returns
// the four int8 results packed little-endian and the block scale in `scale`.
__device__ __forceinline__ uint32_t q8_quant4(float4 v, float &scale) {
	const float a0 = ftz(v.x), a1 = ftz(v.y), a2 = ftz(v.z), a3 = ftz(v.w);
	float amax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(a0), __builtin_fabsf(a1)),
	                             __builtin_fmaxf(__builtin_fabsf(a2), __builtin_fabsf(a3)));
	amax = max8(amax);
	const float xs = q8_xs(amax);
	const float inv = q8_inv(amax, xs);
	scale = xs;
	return q8_code(a0, inv) | (q8_code(a1, inv) << 8) | (q8_code(a2, inv) << 16) | (q8_code(a3, inv) << 24);
}

// Power-of-two scaling of a vector for the fp16 hi/lo representation: for
// max|x| = a, e with a in [2^e, 2^(e+1)) (0 when a is 0 or not finite;
// subnormal maxima clamp to -126, which keeps 2^-e finite and loses nothing
// that matters at that size). x * 2^-e is then below 2, hi = fp16(x*2^-e),
// lo = fp16(x*2^-e - hi); the scaling and the subtraction are exact.
__device__ __forceinline__ int f16_split_exp(float a) {
	int e = 0;
	if (a > 0.0f && __builtin_isfinite(a)) {
		e = (int)((__builtin_bit_cast(uint32_t, a) >> 23) & 0xFFu) - 127;
		e = e < -126 ? -126 : e;
	}
	return e;
}

}  // namespace hako
