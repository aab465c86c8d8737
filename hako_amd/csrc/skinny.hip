// skinny.hip — matmuls of up to 16 tokens at once (batched decode) on the
// gfx950 matrix cores, weights streamed from HBM once for all tokens.
//
// Y[t][r] for t < M <= 16: the M independent matmuls of M sequences stepping
// together (the reference steps each sequence on its own, one matmul call per
// token: src/nn.c:179-210). One wave owns 16 weight rows; one 16x16 MFMA tile
// covers the 16 tokens (A operand, padded with zeros past M) against the 16
// rows (B operand), so every lane owns one row (l % 16) and keeps that row's
// scales to itself, and holds four tokens (4*(l/16) + v) of the output.
//
// Q4_K runs a persistent grid whose workgroups share one 16-row group at a
// time (its waves split the group's K range) and reduce their sums in LDS;
// Q6_K runs a workgroup (4 waves, 64 rows) per tile and range of K. When K is
// split over several workgroups their partial results go to a buffer that
// skinny_reduce_kernel sums in split order, applying the epilogue (a kernel
// boundary, not a device-scope fence per workgroup, makes the partials
// visible).
//
// Q4_K x q8 (src/quant.c:150-232 per token and row): one
// v_mfma_i32_16x16x32_i8 per 32-wide sub-block gives the exact per-sub-block
// sums iqx; they are folded as iqx*(xs*d*s) on the VALU, and the min term
// sum over the block's sub-blocks of (dmin*m)*(-xs*sum xq) runs as two
// v_mfma_f32_16x16x4_f32.
//
// Q6_K x fp32 (src/nn.c:84-95): q-32 exact in fp16 against the activation as
// fp16 hi + lo after an exact per-token power-of-two scaling (the prefill
// GEMM's representation); two v_mfma_f32_16x16x16_f16 per 16-wide scale group,
// the group sums times sc, their block sum times d. Activations are staged through
// LDS one super-block at a time, double-buffered.
#include "hako_dev.h"
#include "hako_rt.h"
#include "skinny.h"

namespace hako {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

constexpr int kT = 256;      // threads per workgroup: 4 waves
constexpr int kRowsWave = 16;
constexpr int kRowsWg = 4 * kRowsWave;

__device__ __forceinline__ uint32_t ld_b32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
	return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// segment of a wave (segment starts are multiples of 16 rows)
struct SegView {
	const uint8_t *w;
	const float *bias;
	float *out;
	int row0, rows, ld;
};

// Fields picked with constant indices and masks: an indexed or selected
// access to the by-value argument makes the compiler copy it to scratch.
__device__ __forceinline__ SegView seg_of(const SkSegs s, int wrow0, bool swiglu) {
	const int si = swiglu ? 0 : (s.n > 2 && wrow0 >= s.s[2].row0) ? 2 : (s.n > 1 && wrow0 >= s.s[1].row0) ? 1 : 0;
	const uint64_t m0 = 0ull - (uint64_t)(si == 0), m1 = 0ull - (uint64_t)(si == 1), m2 = 0ull - (uint64_t)(si == 2);
	auto pick = [&](uint64_t a, uint64_t b, uint64_t c) { return (a & m0) | (b & m1) | (c & m2); };
	auto pp = [](const void *p) { return (uint64_t)(uintptr_t)p; };
	SegView v;
	v.w = (const uint8_t *)(uintptr_t)pick(pp(s.s[0].w), pp(s.s[1].w), pp(s.s[2].w));
	v.bias = (const float *)(uintptr_t)pick(pp(s.s[0].bias), pp(s.s[1].bias), pp(s.s[2].bias));
	v.out = (float *)(uintptr_t)pick(pp(s.s[0].out), pp(s.s[1].out), pp(s.s[2].out));
	v.row0 = (int)pick((uint32_t)s.s[0].row0, (uint32_t)s.s[1].row0, (uint32_t)s.s[2].row0);
	v.rows = (int)pick((uint32_t)s.s[0].rows, (uint32_t)s.s[1].rows, (uint32_t)s.s[2].rows);
	v.ld = (int)pick((uint32_t)s.s[0].ld, (uint32_t)s.s[1].ld, (uint32_t)s.s[2].ld);
	return v;
}

// ── Q4_K x q8 ──
//
// Persistent grid of G workgroups over the launch's 16-row groups: workgroup
// b takes groups b, b + G, b + 2G, ... Its threads load a group's weights
// (16 rows of consecutive bytes over the K range) as consecutive 16-byte
// pieces and park them in an LDS slot, from which each wave reads its
// super-block of the 16 rows in the matrix-core lane layout: the waves split
// the group's K range one super-block each. Whole-region loads stream at
// about 6 TB/s; loads in the lane layout (16 rows x 32 bytes per
// instruction) reach 4 TB/s at the same grid. Two groups are in flight in
// registers while a third is folded from LDS. A wave's super-block is the
// same for every group, so its activation operands (the 16 tokens' q8 bytes,
// scales and -xs*sum(xq) of that block) are read from LDS into registers
// once. The waves' sums of a group meet in LDS and are added in a fixed
// order, so the K range needs no partial sums in memory unless K is split
// over launches (more than kQ4SkMaxBlocks super-blocks).
constexpr int kQ4SkMaxBlocks = 16;   // super-blocks of K per launch split (K <= 4096: one split)
constexpr int kQ4SkWgs = 256;        // workgroups of the persistent grid: one per CU
constexpr int kQ4SkPieces = 3;       // 16-byte pieces per thread and group: 16 rows x 9 x nbk <= 2.25 T

// LDS of a workgroup over nbk super-blocks (W waves, nbk <= W). Region A
// holds first the staged q8 rows [16][nbk*256 + 16], then two slots of a
// group's weights [16][nbk*144 + 16]; then xs and -xs*sum(xq) per
// (sub-block, token) and two slots of the waves' sums of a group.
__host__ __device__ constexpr size_t q4sk_arow(int nbk) { return (size_t)nbk * kQK + 16; }
__host__ __device__ constexpr size_t q4sk_rstride(int nbk) { return (size_t)nbk * kQ4Bytes + 16; }
__host__ __device__ constexpr size_t q4sk_region(int nbk) {
	return 16 * q4sk_arow(nbk) > 2 * 16 * q4sk_rstride(nbk) ? 16 * q4sk_arow(nbk) : 2 * 16 * q4sk_rstride(nbk);
}
__host__ __device__ constexpr size_t q4sk_lds(int nbk, int W) {
	return q4sk_region(nbk) + 2 * (size_t)nbk * 8 * 16 * 4 + 2 * (size_t)W * 64 * 16;
}

// The segment of launch row r0 (uniform) with plain selects of its fields:
// scalar selects, no copy of the argument block.
__device__ __forceinline__ SegView seg_at(const SkSegs &s, int r0) {
	const bool in1 = s.n > 1 && r0 >= s.s[1].row0, in2 = s.n > 2 && r0 >= s.s[2].row0;
	SegView v;
	v.w = in2 ? s.s[2].w : in1 ? s.s[1].w : s.s[0].w;
	v.bias = in2 ? s.s[2].bias : in1 ? s.s[1].bias : s.s[0].bias;
	v.out = in2 ? s.s[2].out : in1 ? s.s[1].out : s.s[0].out;
	v.row0 = in2 ? s.s[2].row0 : in1 ? s.s[1].row0 : s.s[0].row0;
	v.rows = in2 ? s.s[2].rows : in1 ? s.s[1].rows : s.s[0].rows;
	v.ld = in2 ? s.s[2].ld : in1 ? s.s[1].ld : s.s[0].ld;
	return v;
}

// W waves, one super-block of the launch split's K range each (nbk <= W).
template <int EPI, int W>
__global__ __launch_bounds__(64 * W) void q4k_skinny_kernel(SkSegs segs, const int8_t *__restrict__ xq,
                                                            const float *__restrict__ xs, int M, int K, int vrows,
                                                            int nsplit, float *__restrict__ part) {
	constexpr int T = 64 * W;
	constexpr int PP = kQ4SkPieces;
	extern __shared__ __align__(16) uint8_t smem[];
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int j = lane & 15, kq = lane >> 4;
	const int NB = K >> 8, NS = K >> 5;
	const int split = blockIdx.y;
	const int kb_beg = (int)((int64_t)split * NB / nsplit), kb_end = (int)((int64_t)(split + 1) * NB / nsplit);
	const int nbk = kb_end - kb_beg;
	const int arow = (int)q4sk_arow(nbk), rstride = (int)q4sk_rstride(nbk);
	const size_t region = q4sk_region(nbk);
	int8_t *a_s = (int8_t *)smem;                         // staging: [16][arow]
	uint8_t *w_s = smem;                                  // then: [2][16][rstride]
	float *xs_s = (float *)(smem + region);               // [nbk*8][16]
	float *nu_s = xs_s + nbk * 8 * 16;                    // [nbk*8][16]
	float4 *red_s = (float4 *)(nu_s + nbk * 8 * 16);   // [2][W][64]
	const bool live = wave < nbk;   // this wave's super-block: kb_beg + wave
	const int ngroups = (vrows + 15) >> 4, G = gridDim.x;
	const uint32_t rb = (uint32_t)NB * kQ4Bytes;

	// the group's pieces of this thread: piece p = tid + T*i is bytes 16c..
	// of row r of the group's K range (PR pieces per row)
	const int PR = 9 * nbk, PG = 16 * PR;
	uint32_t goff[PP], loff[PP];
	int prow[PP];
#pragma unroll
	for (int i = 0; i < PP; i++) {
		const int p = tid + T * i, r = p / PR, c = p - r * PR;
		prow[i] = p < PG ? r : 1 << 20;   // pieces past the group: a row no group has
		goff[i] = (uint32_t)r * rb + (uint32_t)kb_beg * kQ4Bytes + 16u * c;
		loff[i] = (uint32_t)(r * rstride + 16 * c);
	}
	// A row outside the segment or the launch, a piece past the group and a
	// group past the last read nothing (zeros, no memory access).
	// the output this thread writes in the epilogue: token et of row er
	constexpr int Q = T / 256;   // threads per output: 2 (8 waves) or 4 (16 waves)
	const int eo = tid / Q, et = eo >> 4, er = eo & 15;
	const bool eq = tid % Q == 0 && et < M;
	auto gload = [&](uint4 (&v)[PP], float &ev, SegView &S, int g) {
		const int r0 = g * 16;
		S = seg_at(segs, r0);
		const int wr0 = r0 - S.row0;   // the group's first row in its segment
		const uint32_t wbytes = (uint32_t)S.rows * rb;
		const __amdgpu_buffer_rsrc_t r = stream_rsrc(S.w, g < ngroups ? wbytes : 0u);
		const int rmax = min(S.rows - wr0, vrows - r0);   // rows of the group in the segment and launch
#pragma unroll
		for (int i = 0; i < PP; i++)
			v[i] = ld_b128(r, prow[i] < rmax ? (uint32_t)wr0 * rb + goff[i] : wbytes);
		// the epilogue's operand, loaded with the weights so that the
		// epilogue waits on nothing: the bias (Store) or the output (Add)
		ev = 0.0f;
		if (EPI == kSkStore || EPI == kSkAdd) {
			const bool ok = eq && er < rmax;
			const float *src = uniform_ptr(EPI == kSkStore ? S.bias : (const float *)S.out);
			const uint32_t n = src ? (EPI == kSkStore ? (uint32_t)S.rows : (uint32_t)M * (uint32_t)S.ld) * 4u : 0u;
			const __amdgpu_buffer_rsrc_t er_rs = stream_rsrc(src ? (const void *)src : (const void *)xs, n);
			const uint32_t off = EPI == kSkStore ? 4u * (uint32_t)(wr0 + er) : 4u * ((uint32_t)et * S.ld + wr0 + er);
			ev = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(er_rs, ok ? (int)off : (int)kBufNone, 0, 0));
		}
	};
	// Parks a register set in a weight slot. Pieces past the group go to
	// this thread's own entry of reduction slot p, which the next finish
	// (slot p) overwrites before anyone reads it: no branch around the
	// stores (the wait-count pass turns one into waits on every load).
	const uint32_t red_off = (uint32_t)((uint8_t *)red_s - smem);
	auto gstore = [&](const uint4 (&v)[PP], int slot, int p) {
		const uint32_t ws = (uint32_t)slot * 16 * rstride, dummy = red_off + 16u * (p * W * 64 + tid);
#pragma unroll
		for (int i = 0; i < PP; i++) {
			const uint32_t a = prow[i] < 16 ? ws + loff[i] : dummy;   // a select, not a branch
			*(uint4 *)(smem + a) = v[i];
		}
	};

	// the wave's activation operands (registers, filled once): A operand
	// (token j, bytes 32sb + 8kq.. of the block), and xs and -xs*sum(xq) of
	// (token j, sub-blocks kq, kq+4)
	long av[8];
	float nu0 = 0.0f, nu1 = 0.0f;
	float xsw_t[2] = {0.0f, 0.0f};   // xs of (token j, sub-blocks kq, kq+4)
	const v16f zero16 = {};

	// per block: (s, m) of sub-blocks kq, kq+4 of the lane's row; d*s into
	// the scale-product MFMA, dmin*m into the min-term MFMA
	auto fold = [&](int slot, float (&y)[4]) {
		v4f acc = {0.0f, 0.0f, 0.0f, 0.0f}, accm = {0.0f, 0.0f, 0.0f, 0.0f};
		if (live) {
			const uint8_t *rowp = w_s + ((size_t)slot * 16 + j) * rstride + wave * kQ4Bytes;
			const uint4 hd = *(const uint4 *)rowp;
			uint2 qv[4];
#pragma unroll
			for (int g = 0; g < 4; g++) qv[g] = *(const uint2 *)(rowp + 16 + 32 * g + 8 * kq);
			const v4i zero = {0, 0, 0, 0};
			uint32_t s0, m0, s1, m1;
			scale_min_k4((uint32_t)kq, hd.y, hd.z, hd.w, s0, m0);
			scale_min_k4((uint32_t)kq + 4u, hd.y, hd.z, hd.w, s1, m1);
			const float dd = f16_to_f32(hd.x & 0xFFFFu), dmin = f16_to_f32(hd.x >> 16);
			accm = __builtin_amdgcn_mfma_f32_16x16x4f32(nu0, dmin * (float)m0, accm, 0, 0, 0);
			accm = __builtin_amdgcn_mfma_f32_16x16x4f32(nu1, dmin * (float)m1, accm, 0, 0, 0);
			// four integer products at a time, then their folds
#pragma unroll
			for (int half = 0; half < 2; half++) {
				// the fold's scale products P[token][row] = xs[token]*(d*s)[row] of
				// sub-blocks 4half..4half+3 as one four-block outer product on the
				// matrix cores: block b (lanes 16b..) is sub-block 4half + b, whose
				// d*s this lane computed above (b = kq), laid out like the int8
				// products: P[4i + v] pairs with di[i][v]
				const v16f P = __builtin_amdgcn_mfma_f32_16x16x1f32(xsw_t[half], dd * (float)(half ? s1 : s0), zero16,
				                                                   0, 0, 0);
				v4i di[4];
#pragma unroll
				for (int i = 0; i < 4; i++) {
					const int sb = 4 * half + i, g4 = sb >> 1, h = sb & 1;
					const uint2 q = qv[g4];
					const uint32_t w0 = h ? (q.x >> 4) & 0x0F0F0F0Fu : q.x & 0x0F0F0F0Fu;
					const uint32_t w1 = h ? (q.y >> 4) & 0x0F0F0F0Fu : q.y & 0x0F0F0F0Fu;
					di[i] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[sb], (long)(((uint64_t)w1 << 32) | w0), zero, 0,
					                                              0, 0);
				}
#pragma unroll
				for (int i = 0; i < 4; i++)
#pragma unroll
					for (int v = 0; v < 4; v++) acc[v] = __builtin_fmaf((float)di[i][v], P[4 * i + v], acc[v]);
			}
		}
#pragma unroll
		for (int v = 0; v < 4; v++) y[v] = acc[v] + accm[v];
	};

	// the waves' sums of group g (lane: tokens 4(l/16) + v of row l%16) to
	// LDS slot p; then every thread takes a quarter of the waves of output
	// (t, r) = tid/(T/256) (W/4 waves each, in order), the quarters meet in
	// neighbouring lanes, and the first applies the epilogue to token t of
	// row r of the group: the same order of additions at every call
	auto finish = [&](const float (&y)[4], const SegView &S, float ev, int g, int p) {
		red_s[(p * W + wave) * 64 + lane] = make_float4(y[0], y[1], y[2], y[3]);
		__syncthreads();
		constexpr int WQ = W / Q;     // waves per thread: 4
		const int qq = tid % Q, t = et, r = er;
		const float *src = (const float *)&red_s[(p * W + qq * WQ) * 64 + 16 * (t >> 2) + r] + (t & 3);
		float sum = 0.0f;
#pragma unroll
		for (int w = 0; w < WQ; w++) sum += src[w * 64 * 4];
		sum += dpp_f<kDppQuadSwap1>(sum);   // quarters 0+1, 2+3
		if (Q == 4) sum += dpp_f<kDppQuadSwap2>(sum);
		// through descriptors, with an offset past the stream for the lanes
		// that write nothing: no branch around memory operations
		const int vrow = g * 16 + r, wr = vrow - S.row0;
		const bool ok = qq == 0 && vrow < vrows && wr < S.rows;
		if (EPI == kSkPart) {   // tokens past M: zeros
			const __amdgpu_buffer_rsrc_t pr = stream_rsrc(part, (uint32_t)nsplit * 16u * (uint32_t)vrows * 4u);
			__builtin_amdgcn_raw_buffer_store_b32(
			    __builtin_bit_cast(uint32_t, sum), pr,
			    ok ? (int)(4u * (((uint32_t)split * 16u + t) * (uint32_t)vrows + vrow)) : (int)kBufNone, 0, 0);
		} else {
			const int ld = __builtin_amdgcn_readfirstlane(S.ld);
			const __amdgpu_buffer_rsrc_t orr = stream_rsrc(uniform_ptr(S.out), (uint32_t)M * (uint32_t)ld * 4u);
			const int off = ok && t < M ? (int)(4u * ((uint32_t)t * ld + wr)) : (int)kBufNone;
			const float v = EPI == kSkAdd ? ev + sum : sum + ev;
			__builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), orr, off, 0, 0);
		}
	};

	// groups in flight: two in registers (X, Y), one in an LDS slot
	uint4 X[PP], Y[PP];
	float eX, eY, e0, e1;         // the epilogue operands of the groups in X, Y and the two LDS slots
	SegView svX, svY, sv0, sv1;   // their segments
	const int g0 = blockIdx.x;
	gload(X, eX, svX, g0);
	gload(Y, eY, svY, g0 + G);

	// stage the q8 rows of the K range: piece c = (t, p) holds bytes 16p..
	// of token t's range and, for even p, the scale of its sub-block p/2
	// (zeros past M); a sub-block's two pieces sit in neighbouring lanes
	{
		const int PT = 16 * nbk;   // pieces per token
		const __amdgpu_buffer_rsrc_t qrs = stream_rsrc(xq, (uint32_t)M * (uint32_t)K);
		const __amdgpu_buffer_rsrc_t srs = stream_rsrc(xs, (uint32_t)M * (uint32_t)NS * 4u);
		constexpr int U = (16 * 16 * W + T - 1) / T;   // nbk <= W
		uint4 qv[U];
		float sv[U];
#pragma unroll
		for (int u = 0; u < U; u++) {
			const int c = tid + T * u, t = c / PT, p = c - t * PT;
			const bool in = c < 16 * PT && t < M;
			qv[u] = ld_b128(qrs, in ? (uint32_t)t * K + 256u * kb_beg + 16u * p : kBufNone);
			sv[u] = __builtin_bit_cast(float, ld_b32(srs, in && !(p & 1) ? 4u * ((uint32_t)t * NS + 8u * kb_beg + (p >> 1))
			                                                            : kBufNone));
		}
#pragma unroll
		for (int u = 0; u < U; u++) {
			const int c = tid + T * u, t = c / PT, p = c - t * PT;
			int ix = 0;
			ix = sdot4((int)qv[u].x, 0x01010101, ix);
			ix = sdot4((int)qv[u].y, 0x01010101, ix);
			ix = sdot4((int)qv[u].z, 0x01010101, ix);
			ix = sdot4((int)qv[u].w, 0x01010101, ix);
			ix += dpp_i<kDppQuadSwap1>(ix);   // the sub-block's other 16 bytes
			if (c < 16 * PT) {
				*(uint4 *)(a_s + t * arow + 16 * p) = qv[u];
				if (!(p & 1)) {
					xs_s[(p >> 1) * 16 + t] = sv[u];
					nu_s[(p >> 1) * 16 + t] = -sv[u] * (float)ix;
				}
			}
		}
	}
	// every load so far complete (the staging's waits sit on a branch that
	// the wait-count pass would otherwise carry into the loop as pending
	// loads, waiting out the whole prefetch at every use of their registers)
	__builtin_amdgcn_s_waitcnt(0);
	__syncthreads();
	if (live) {
		const int8_t *arow_p = a_s + j * arow + wave * kQK + 8 * kq;   // token j, K-slice 8kq of each sub-block
#pragma unroll
		for (int sb = 0; sb < 8; sb++) av[sb] = *(const long *)(arow_p + 32 * sb);
		nu0 = nu_s[(8 * wave + kq) * 16 + j];
		nu1 = nu_s[(8 * wave + kq + 4) * 16 + j];
		xsw_t[0] = xs_s[(8 * wave + kq) * 16 + j];
		xsw_t[1] = xs_s[(8 * wave + kq + 4) * 16 + j];
	}
	__syncthreads();   // the staging area becomes the weight slots
	gstore(X, 0, 0);
	sv0 = svX;
	e0 = eX;
	gload(X, eX, svX, g0 + 2 * G);
	__syncthreads();

	// iteration: fold the group in an LDS slot, park the older register set
	// in the other slot, reload that set with the group three ahead, reduce
	for (int g = g0; g < ngroups; g += 2 * G) {
		float y[4];
		fold(0, y);
		gstore(Y, 1, 0);
		sv1 = svY;
		e1 = eY;
		gload(Y, eY, svY, g + 3 * G);
		finish(y, sv0, e0, g, 0);
		if (g + G >= ngroups) break;
		fold(1, y);
		gstore(X, 0, 1);
		sv0 = svX;
		e0 = eX;
		gload(X, eX, svX, g + 4 * G);
		finish(y, sv1, e1, g + G, 1);
	}
}

// ── Q6_K x fp32 (fp16 hi/lo) ──

constexpr int kHPadSk = kQK + 8;     // fp16 per staged token row

struct Q6SkBuf {
	uint32_t ql[2][4];   // per half n: ql bytes 64n + 16q + 4kq .. +4, q = 0..3
	uint32_t qh[2][2];   // per half n: qh bytes 32n + 16p + 4kq .. +4, p = 0..1
	uint4 sc;            // the 16 scales
	uint32_t d;
};

// Weight staging of one wave: its 16 rows' super-block, fetched as 16-byte
// pieces (lane = piece p < 13 of row 4i + lane/16 in load i: bytes 0..207 of
// each row as one contiguous run; blocks are 2-byte aligned, so the pieces
// are unaligned loads) plus one 2-byte load of d per row (lane = row), written
// to a per-wave LDS tile and read back in the MFMA lane layout. Every byte
// read lies inside the block. A row of the tile is 240 bytes (60 dwords,
// -4 mod 64 banks: the dword reads of 16 rows x 4 lanes fall in 64 distinct
// banks).
constexpr int kQ6Pieces = 13;                 // 16-byte pieces of bytes 0..207 (d at 208 apart)
constexpr int kQ6TileRow = 240;               // bytes per staged row

// Workgroup (64-row tile, K split): the tile's rows over super-blocks
// [kb_beg, kb_end), the sums scaled by each token's power of two: esc[t] at
// the end, or (BLK) esc[t][kb] per super-block. EPI kSkStore / kSkAdd apply
// the epilogue directly (one split); kSkPart writes the partial sums to
// part[split][t][vrow].
template <int EPI, bool BLK>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(3))) void q6k_skinny_kernel(
    SkSegs segs, const _Float16 *__restrict__ xh, const _Float16 *__restrict__ xl, const float *__restrict__ esc,
    int M, int K, int vrows, int nsplit, float *__restrict__ part) {
	__shared__ __align__(16) _Float16 ah_s[2][16 * kHPadSk];
	__shared__ __align__(16) _Float16 al_s[2][16 * kHPadSk];
	__shared__ __align__(16) uint8_t w_s[4][16 * kQ6TileRow];
	__shared__ __align__(16) float es_s[2][16];   // BLK: esc[t][kb] of the staged block
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: segment and descriptors in SGPRs
	const int j = lane & 15, kq = lane >> 4;
	const int NB = K >> 8;
	const int tile = blockIdx.x / nsplit, split = blockIdx.x - tile * nsplit;
	const int kb_beg = (int)((int64_t)split * NB / nsplit), kb_end = (int)((int64_t)(split + 1) * NB / nsplit);
	const int wrow0 = (tile * 4 + wave) * kRowsWave;
	const SegView S = seg_of(segs, wrow0, false);
	const int vrow = wrow0 + j, wr = vrow - S.row0;
	const bool ok = vrow < vrows && wr < S.rows;
	const uint32_t rb = (uint32_t)NB * kQ6Bytes;
	// Every load and LDS store below is issued unconditionally: a lane with
	// nothing to load has an offset past its stream, a block past the range
	// loads through a descriptor of zero bytes (zeros, no memory access), and
	// a lane with nothing to store writes a pad. A branch around them makes
	// the wait-count pass wait for every load in flight.
	const __amdgpu_buffer_rsrc_t wrs = stream_rsrc(S.w, (uint32_t)S.rows * rb), wnone = stream_rsrc(S.w, 0);
	// staging loads: piece lp of row 4i + lr (i = 0..3), and d of row `lane`
	const int lp = lane & 15, lr = lane >> 4;
	uint32_t srow_off[4];
#pragma unroll
	for (int i = 0; i < 4; i++) {
		const int r = wrow0 + 4 * i + lr, rr = r - S.row0;
		srow_off[i] = (lp < kQ6Pieces && r < vrows && rr < S.rows) ? (uint32_t)rr * rb + 16u * lp : kBufNone;
	}
	uint32_t d_off;
	{
		const int r = wrow0 + lane, rr = r - S.row0;
		d_off = (lane < 16 && r < vrows && rr < S.rows) ? (uint32_t)rr * rb + 208u : kBufNone;
	}
	uint8_t *wt = w_s[wave];
	// LDS targets of the staged pieces (pieces 13..15: the row's pad at 224)
	// and of d (lanes 16..63: pad bytes 210..215 of row lane%16)
	const int pcol = lp < kQ6Pieces ? 16 * lp : 224;
	const int dpos = lane < 16 ? lane * kQ6TileRow + 208 : (lane & 15) * kQ6TileRow + 210 + 2 * ((lane >> 4) - 1);
	const uint32_t hbytes = (uint32_t)M * (uint32_t)K * 2u;
	const __amdgpu_buffer_rsrc_t hrs = stream_rsrc(xh, hbytes), lrs = stream_rsrc(xl, hbytes);
	const __amdgpu_buffer_rsrc_t hnone = stream_rsrc(xh, 0), lnone = stream_rsrc(xl, 0);
	const __amdgpu_buffer_rsrc_t ers = stream_rsrc(esc, BLK ? (uint32_t)M * (uint32_t)NB * 4u : 0u);
	const __amdgpu_buffer_rsrc_t enone = stream_rsrc(esc, 0);
	const int t0 = 4 * kq;
	// The epilogue's operands, loaded before the stream so that the end of the
	// workgroup waits on nothing (loaded there, each sat behind its own wait):
	// the per-token powers of two (not BLK), and the row's bias (Store) or the
	// lane's four outputs (Add).
	float ev[4], pv[4];
	{
		const __amdgpu_buffer_rsrc_t ets = stream_rsrc(esc, BLK ? 0u : (uint32_t)M * 4u);
		const float *bsrc = uniform_ptr(S.bias);
		const __amdgpu_buffer_rsrc_t brs = stream_rsrc(bsrc ? (const void *)bsrc : (const void *)esc,
		                                               EPI == kSkStore && bsrc ? (uint32_t)S.rows * 4u : 0u);
		const int ld = __builtin_amdgcn_readfirstlane(S.ld);
		const __amdgpu_buffer_rsrc_t ors = stream_rsrc(uniform_ptr(S.out), EPI == kSkAdd ? (uint32_t)M * (uint32_t)ld * 4u
		                                                                              : 0u);
		const float bv = ld_f32(brs, ok ? 4u * (uint32_t)wr : kBufNone);
#pragma unroll
		for (int v = 0; v < 4; v++) {
			const bool tv = t0 + v < M;
			ev[v] = ld_f32(ets, tv ? 4u * (uint32_t)(t0 + v) : kBufNone);
			pv[v] = EPI == kSkAdd ? ld_f32(ors, ok && tv ? 4u * ((uint32_t)(t0 + v) * ld + wr) : kBufNone) : bv;
		}
	}

	struct WBuf {
		uint4 v[4];
		uint32_t d;
	};
	auto issue = [&](WBuf &w, int kb) {
		const __amdgpu_buffer_rsrc_t r = kb < kb_end ? wrs : wnone;
		const int so = kb * kQ6Bytes;
#pragma unroll
		for (int i = 0; i < 4; i++)
			w.v[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)srow_off[i], so, 0));
		w.d = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)d_off, so, 0);
	};
	// the staged pieces to the wave's tile, then this lane's fields of row j
	auto unstage = [&](const WBuf &w, Q6SkBuf &b) {
#pragma unroll
		for (int i = 0; i < 4; i++) *(uint4 *)(wt + (4 * i + lr) * kQ6TileRow + pcol) = w.v[i];
		*(uint16_t *)(wt + dpos) = (uint16_t)w.d;
		__builtin_amdgcn_wave_barrier();
		const uint8_t *row = wt + j * kQ6TileRow;
#pragma unroll
		for (int n = 0; n < 2; n++) {
#pragma unroll
			for (int q = 0; q < 4; q++) b.ql[n][q] = *(const uint32_t *)(row + 64 * n + 16 * q + 4 * kq);
#pragma unroll
			for (int p = 0; p < 2; p++) b.qh[n][p] = *(const uint32_t *)(row + 128 + 32 * n + 16 * p + 4 * kq);
		}
		b.sc = *(const uint4 *)(row + 192);
		b.d = *(const uint16_t *)(row + 208);
		__builtin_amdgcn_wave_barrier();   // read before the next block's pieces land
	};
	// activation stage of block kb: 16 tokens x 256 K of hi and lo (zeros
	// past M) and, BLK, esc[t][kb] of token tid%16 (every thread: the same
	// value lands in es_s from sixteen threads)
	struct Stage {
		uint4 h[2], l[2];
		float e;
	};
	auto load_stage = [&](Stage &a, int kb) {
		const bool in = kb < kb_end;
#pragma unroll
		for (int u = 0; u < 2; u++) {
			const int c = tid + kT * u, t = c >> 5, p = c & 31;   // 16 tokens x 32 pieces of 8 fp16
			const int off = t < M ? (int)(2u * ((uint32_t)t * K + 8 * p)) : (int)kBufNone;
			a.h[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(in ? hrs : hnone, off, kb * 512, 0));
			a.l[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(in ? lrs : lnone, off, kb * 512, 0));
		}
		a.e = 0.0f;
		if (BLK) {
			const int t = tid & 15;
			a.e = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
			                                    in ? ers : enone, t < M ? (int)(4u * ((uint32_t)t * NB)) : (int)kBufNone,
			                                    kb * 4, 0));
		}
	};
	auto store_stage = [&](const Stage &a, int slot) {
#pragma unroll
		for (int u = 0; u < 2; u++) {
			const int c = tid + kT * u, t = c >> 5, p = c & 31;
			*(uint4 *)(ah_s[slot] + t * kHPadSk + 8 * p) = a.h[u];
			*(uint4 *)(al_s[slot] + t * kHPadSk + 8 * p) = a.l[u];
		}
		if (BLK) es_s[slot][tid & 15] = a.e;
	};

	// in flight: the weights of the next two blocks (W0, W1) and the stages
	// of the next two (S0, S1); weights of block kb + 2 and the stage of
	// kb + 3 are issued while block kb is folded
	WBuf W0, W1;
	Stage A0, A1;
	issue(W0, kb_beg);
	load_stage(A0, kb_beg);
	issue(W1, kb_beg + 1);
	load_stage(A1, kb_beg + 1);
	store_stage(A0, 0);
	load_stage(A0, kb_beg + 2);
	__syncthreads();
	v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
	const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
	for (int kb0 = kb_beg; kb0 < kb_end; kb0 += 2) {
#pragma unroll
		for (int half = 0; half < 2; half++) {
			const int kb = kb0 + half;
			WBuf &W = half ? W1 : W0;
			Stage &A = half ? A0 : A1;   // the stage of kb + 1
			Q6SkBuf b;
			unstage(W, b);
			issue(W, kb + 2);
			if (kb < kb_end) {
				const _Float16 *ah = ah_s[half] + j * kHPadSk + 4 * kq;
				const _Float16 *al = al_s[half] + j * kHPadSk + 4 * kq;
				const uint32_t scw[4] = {b.sc.x, b.sc.y, b.sc.z, b.sc.w};
				v4f accb = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
				for (int gg = 0; gg < 16; gg++) {
					// K = 16gg + 4kq + e: half n = gg/8, k = (gg/2)%4, l = 16(gg%2) + 4kq + e
					const int n = gg >> 3, k = (gg >> 1) & 3, p = gg & 1;
					const uint32_t qlw = b.ql[n][2 * (k & 1) + p], qhw = b.qh[n][p];
					const uint32_t nib = (k >> 1) ? (qlw >> 4) & 0x0F0F0F0Fu : qlw & 0x0F0F0F0Fu;
					// qh bits 2k, 2k+1 of each byte to bits 4, 5 with one shift (what
					// the neighbouring bytes shift in is masked off)
					const uint32_t hs = k < 2 ? qhw << (4 - 2 * k) : qhw >> (2 * k - 4);
					const uint32_t q6 = (hs & 0x30303030u) | nib;
					// 1024 + q as fp16: the exponent byte 0x64 picked beside each
					// 6-bit byte by the permute itself; minus 1056 gives q - 32 exactly
					const uint32_t lo2 = __builtin_amdgcn_perm(0x64646464u, q6, 0x04010400u);
					const uint32_t hi2 = __builtin_amdgcn_perm(0x64646464u, q6, 0x04030402u);
					const v2h bias2 = {(_Float16)1056.0f, (_Float16)1056.0f};
					const v2h w01 = __builtin_bit_cast(v2h, lo2) - bias2, w23 = __builtin_bit_cast(v2h, hi2) - bias2;
					const v4h wv = {w01[0], w01[1], w23[0], w23[1]};
					v4f pr = __builtin_amdgcn_mfma_f32_16x16x16f16(*(const v4h *)(ah + 16 * gg), wv, zero, 0, 0, 0);
					pr = __builtin_amdgcn_mfma_f32_16x16x16f16(*(const v4h *)(al + 16 * gg), wv, pr, 0, 0, 0);
					const float sg = (float)(int8_t)((scw[gg >> 2] >> (8 * (gg & 3))) & 0xFFu);
					accb[0] = __builtin_fmaf(pr[0], sg, accb[0]);
					accb[1] = __builtin_fmaf(pr[1], sg, accb[1]);
					accb[2] = __builtin_fmaf(pr[2], sg, accb[2]);
					accb[3] = __builtin_fmaf(pr[3], sg, accb[3]);
				}
				// the block's sums times d of the row (and, BLK, this block's
				// powers of two of the lane's tokens, staged with the activations)
				const float dd = f16_to_f32(b.d);
				if (BLK) {
					const float4 eb = *(const float4 *)&es_s[half][t0];
					acc[0] = __builtin_fmaf(accb[0], dd * eb.x, acc[0]);
					acc[1] = __builtin_fmaf(accb[1], dd * eb.y, acc[1]);
					acc[2] = __builtin_fmaf(accb[2], dd * eb.z, acc[2]);
					acc[3] = __builtin_fmaf(accb[3], dd * eb.w, acc[3]);
				} else {
					acc[0] = __builtin_fmaf(accb[0], dd, acc[0]);
					acc[1] = __builtin_fmaf(accb[1], dd, acc[1]);
					acc[2] = __builtin_fmaf(accb[2], dd, acc[2]);
					acc[3] = __builtin_fmaf(accb[3], dd, acc[3]);
				}
			}
			store_stage(A, half ^ 1);
			load_stage(A, kb + 3);
			__syncthreads();
		}
	}
	float y[4];
#pragma unroll
	for (int v = 0; v < 4; v++) y[v] = t0 + v < M ? (BLK ? acc[v] : acc[v] * ev[v]) : 0.0f;
	if (EPI == kSkPart) {
		if (ok)
#pragma unroll
			for (int v = 0; v < 4; v++) part[((size_t)split * 16 + t0 + v) * vrows + vrow] = y[v];
		return;
	}
	// Store: out[t][r] = y + bias[r] (+ 0 without a bias); Add: out[t][r] += y
	if (ok)
#pragma unroll
		for (int v = 0; v < 4; v++)
			if (t0 + v < M) S.out[(size_t)(t0 + v) * S.ld + wr] = EPI == kSkAdd ? pv[v] + y[v] : y[v] + pv[v];
}

// Grid (ceil(rows/256), M): the splits' sums, in split order, through the
// epilogue. Store / Add: row = vrow of the launch's row space; SwiGLU: row r
// of segment 0 combines gate row r and up row rows + r.
template <int EPI>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(SkSegs segs, const float *__restrict__ part, int nsplit,
                                                            int vrows) {
	const int vrow = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
	if (EPI == kSkSwiGLU) {
		const int F = segs.s[0].rows;
		if (vrow >= F) return;
		float g = 0.0f, u = 0.0f;
		for (int sp = 0; sp < nsplit; sp++) {
			g += part[((size_t)sp * 16 + t) * vrows + vrow];
			u += part[((size_t)sp * 16 + t) * vrows + F + vrow];
		}
		segs.s[0].out[(size_t)t * segs.s[0].ld + vrow] = g / (1.0f + expf(-g)) * u;
		return;
	}
	if (vrow >= vrows) return;
	float y = 0.0f;
	for (int sp = 0; sp < nsplit; sp++) y += part[((size_t)sp * 16 + t) * vrows + vrow];
	const SegView S = seg_of(segs, vrow, false);
	const int r = vrow - S.row0;
	float *o = S.out + (size_t)t * S.ld + r;
	if (EPI == kSkAdd)
		*o += y;
	else
		*o = y + (S.bias ? S.bias[r] : 0.0f);
}

// Grid (F/256, m): the gate/up partials of one 256-row block of segment 0
// (gate rows r, up rows F + r, splits summed in order as the SwiGLU reduce
// does), h = silu(g)*u, then h as fp16 hi + lo scaled by one power of two
// for the block: escb[t][block] = 2^e with e the exponent of the block's
// largest |h| (f16_split_exp), x = (hi + lo) * escb.
__global__ __launch_bounds__(256) void swiglu_split_kernel(const float *__restrict__ part, int nsplit, int F,
                                                           _Float16 *__restrict__ xh, _Float16 *__restrict__ xl,
                                                           float *__restrict__ escb) {
	__shared__ float red[4];
	const int r = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y, lane = threadIdx.x & 63;
	const int vrows = 2 * F;
	float g = 0.0f, u = 0.0f;
	for (int sp = 0; sp < nsplit; sp++) {
		g += part[((size_t)sp * 16 + t) * vrows + r];
		u += part[((size_t)sp * 16 + t) * vrows + F + r];
	}
	const float h = silu(g) * u;
	float a = __builtin_fabsf(h);
	a = __builtin_isfinite(a) ? a : 0.0f;
	a = wave_max(a);
	if (lane == 0) red[threadIdx.x >> 6] = a;
	__syncthreads();
	a = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
	const int e = f16_split_exp(a);
	const float f = h * __builtin_ldexpf(1.0f, -e);
	const _Float16 hi = (_Float16)f;
	xh[(size_t)t * F + r] = hi;
	xl[(size_t)t * F + r] = (_Float16)(f - (float)hi);
	if (threadIdx.x == 0) escb[(size_t)t * (F >> 8) + blockIdx.x] = __builtin_ldexpf(1.0f, e);
}

int reduce(const SkSegs &segs, int epi, const float *part, int nsplit, int m, int vrows) {
	const int rows = epi == kSkSwiGLU ? segs.s[0].rows : vrows;
	const dim3 rg((rows + 255) / 256, m);
	if (epi == kSkStore)
		hipLaunchKernelGGL(skinny_reduce_kernel<kSkStore>, rg, dim3(256), 0, stream(), segs, part, nsplit, vrows);
	else if (epi == kSkAdd)
		hipLaunchKernelGGL(skinny_reduce_kernel<kSkAdd>, rg, dim3(256), 0, stream(), segs, part, nsplit, vrows);
	else
		hipLaunchKernelGGL(skinny_reduce_kernel<kSkSwiGLU>, rg, dim3(256), 0, stream(), segs, part, nsplit, vrows);
	HK_LAUNCHED("skinny_reduce");
	return HAKO_GPU_OK;
}

}  // namespace

namespace {
int g_q4_target = kQ4SkWgs, g_q6_target = kSkTargetWgsQ6;
}

void q4k_skinny_set_target_wgs(int wgs) { g_q4_target = wgs > 0 ? wgs : kQ4SkWgs; }
void q6k_skinny_set_target_wgs(int wgs) { g_q6_target = wgs > 0 ? wgs : kSkTargetWgsQ6; }

int q4k_skinny_splits(int n_in, int vrows) {
	(void)vrows;
	const int nb = n_in / kQK;
	return (nb + kQ4SkMaxBlocks - 1) / kQ4SkMaxBlocks;
}

size_t q4k_skinny_part_floats(int n_in, int vrows, int epi) {
	const int ns = q4k_skinny_splits(n_in, vrows);
	return (ns > 1 || epi == kSkSwiGLU || epi == kSkPart) ? (size_t)ns * 16 * vrows : 0;
}

namespace {

template <int W>
int q4k_skinny_launch(const SkSegs &segs, bool direct, int epi, const int8_t *xq, const float *xs, int m, int n_in,
                      int vrows, int ns, float *part) {
	const int nb = n_in / kQK, ngroups = (vrows + 15) / 16;
	const dim3 grid(ngroups < g_q4_target ? ngroups : g_q4_target, ns);
	const size_t lds = q4sk_lds((nb + ns - 1) / ns, W);
	static bool attr_set[64];   // per device
	int dev = 0;
	HK_HIP(hipGetDevice(&dev));
	if (dev < 0 || dev >= 64) return set_error(HAKO_GPU_ENODEV, "device %d beyond the 64 the skinny launch tracks", dev);
	if (!attr_set[dev]) {   // more than 64 KB of dynamic LDS (gfx950 has 160 KB per CU)
		const int max_lds = (int)q4sk_lds(W, W);
		HK_HIP(hipFuncSetAttribute((const void *)q4k_skinny_kernel<kSkPart, W>,
		                           hipFuncAttributeMaxDynamicSharedMemorySize, max_lds));
		HK_HIP(hipFuncSetAttribute((const void *)q4k_skinny_kernel<kSkStore, W>,
		                           hipFuncAttributeMaxDynamicSharedMemorySize, max_lds));
		HK_HIP(hipFuncSetAttribute((const void *)q4k_skinny_kernel<kSkAdd, W>,
		                           hipFuncAttributeMaxDynamicSharedMemorySize, max_lds));
		attr_set[dev] = true;
	}
	const dim3 block(64 * W);
	if (!direct)
		hipLaunchKernelGGL((q4k_skinny_kernel<kSkPart, W>), grid, block, lds, stream(), segs, xq, xs, m, n_in, vrows,
		                   ns, part);
	else if (epi == kSkStore)
		hipLaunchKernelGGL((q4k_skinny_kernel<kSkStore, W>), grid, block, lds, stream(), segs, xq, xs, m, n_in, vrows,
		                   1, part);
	else
		hipLaunchKernelGGL((q4k_skinny_kernel<kSkAdd, W>), grid, block, lds, stream(), segs, xq, xs, m, n_in, vrows, 1,
		                   part);
	HK_LAUNCHED("q4k_skinny");
	return HAKO_GPU_OK;
}

}  // namespace

int q4k_skinny(const SkSegs &segs, int epi, const int8_t *xq, const float *xs, int m, int n_in, int vrows,
               float *part, size_t part_cap) {
	const int ns = q4k_skinny_splits(n_in, vrows), nb = n_in / kQK;
	const bool direct = ns == 1 && epi != kSkSwiGLU && epi != kSkPart;
	if (!direct && (!part || part_cap < q4k_skinny_part_floats(n_in, vrows, epi)))
		return set_error(HAKO_GPU_EINVAL, "Q4_K skinny split needs a workspace of %zu floats (has %zu)",
		                 q4k_skinny_part_floats(n_in, vrows, epi), part ? part_cap : (size_t)0);
	// a wave per super-block of the split: 8 waves up to 8 blocks, else 16
	const int nbk = (nb + ns - 1) / ns;
	const int rc = nbk <= 8 ? q4k_skinny_launch<8>(segs, direct, epi, xq, xs, m, n_in, vrows, ns, part)
	                        : q4k_skinny_launch<16>(segs, direct, epi, xq, xs, m, n_in, vrows, ns, part);
	if (rc) return rc;
	return (direct || epi == kSkPart) ? HAKO_GPU_OK : reduce(segs, epi, part, ns, m, vrows);
}

int swiglu_split(const float *part, int nsplit, int F, int m, _Float16 *xh, _Float16 *xl, float *escb) {
	if (F % kQK) return set_error(HAKO_GPU_EINVAL, "SwiGLU split needs whole 256-row blocks (F = %d)", F);
	hipLaunchKernelGGL(swiglu_split_kernel, dim3(F / kQK, m), dim3(256), 0, stream(), part, nsplit, F, xh, xl, escb);
	HK_LAUNCHED("swiglu_split");
	return HAKO_GPU_OK;
}

int q6k_skinny_splits(int n_in, int vrows) {
	const int tiles = (vrows + kRowsWg - 1) / kRowsWg, nb = n_in / kQK;
	int ns = g_q6_target / tiles;   // workgroups to fill the chip, all resident at once
	ns = ns > nb / 4 ? nb / 4 : ns;  // at least four super-blocks per split
	return ns < 1 ? 1 : ns;
}

size_t q6k_skinny_part_floats(int n_in, int vrows, int epi) {
	const int ns = q6k_skinny_splits(n_in, vrows);
	return (ns > 1 || epi == kSkPart) ? (size_t)ns * 16 * vrows : 0;
}

int q6k_skinny(const SkSegs &segs, int epi, const _Float16 *xh, const _Float16 *xl, const float *esc, int m,
               int n_in, int vrows, float *part, size_t part_cap, bool esc_per_block) {
	const int tiles = (vrows + kRowsWg - 1) / kRowsWg;
	const int ns = q6k_skinny_splits(n_in, vrows);
	const bool direct = ns == 1 && epi != kSkPart;
	if (!direct && (!part || part_cap < q6k_skinny_part_floats(n_in, vrows, epi)))
		return set_error(HAKO_GPU_EINVAL, "Q6_K skinny split needs a workspace of %zu floats (has %zu)",
		                 q6k_skinny_part_floats(n_in, vrows, epi), part ? part_cap : (size_t)0);
	const dim3 grid(tiles * ns);
#define HK_Q6SK(E, B, NS) \
	hipLaunchKernelGGL((q6k_skinny_kernel<E, B>), grid, dim3(kT), 0, stream(), segs, xh, xl, esc, m, n_in, vrows, NS, part)
	if (!direct) {
		if (esc_per_block) HK_Q6SK(kSkPart, true, ns);
		else HK_Q6SK(kSkPart, false, ns);
	} else if (epi == kSkStore) {
		if (esc_per_block) HK_Q6SK(kSkStore, true, 1);
		else HK_Q6SK(kSkStore, false, 1);
	} else {
		if (esc_per_block) HK_Q6SK(kSkAdd, true, 1);
		else HK_Q6SK(kSkAdd, false, 1);
	}
#undef HK_Q6SK
	HK_LAUNCHED("q6k_skinny");
	return (direct || epi == kSkPart) ? HAKO_GPU_OK : reduce(segs, epi, part, ns, m, vrows);
}

}  // namespace hako
