// gemm.hip — multi-token matmuls (prompt prefill) on the gfx950 matrix cores.
//
// The reference has no batched matmul: a prompt runs token by token, each
// token one matmul per weight (cli/main.c:56-60, src/nn.c:179-210). These
// kernels compute the same M independent products at once, Y[t][r] for
// tokens t < M and weight rows r < n_out, with the weight stream read once per
// 64-token tile instead of once per token.
//
// Q4_K x q8 (reference src/quant.c:150-232 per token and row). The activation
// rows are quantized with the q8_32 scheme first (one launch over all rows).
// One v_mfma_i32_32x32x32_i8 covers exactly one 32-wide sub-block, so its
// int32 results are the reference's own per-sub-block sums iqx = Σ q·xq
// (|iqx| <= 15*127*32, exact); they are folded per sub-block as
// xs*(d*s*iqx − dmin*m*ix), written iqx*(xs*ds) + (−xs*ix)*dm with
// ds = d*s and dm = dmin*m (exact fp32 products) precomputed per row. The
// first term takes three VALU ops per output and sub-block against 32 int8
// MACs of matrix-core work, so this kernel is bounded by the vector ALUs; the
// second term is a product over sub-blocks and runs on fp32 MFMA.
//
// Q6_K x fp32 (reference src/nn.c:84-95: dequantized rows, fp32 dot). The
// 6-bit values q−32 are exact in fp16 and so are the scales' products
// d*sc in fp32; the fp32 activation is carried as two fp16 halves
// hi + lo after scaling each token row by an exact power of two that brings
// its largest magnitude into [1, 2). One v_mfma_f32_32x32x16_f16 covers one
// 16-wide scale group: two of them (hi, lo) accumulate exact products in
// fp32, the group result is scaled by d*sc and added, and the power of two is
// applied at the end. The activation is thus represented to ~2^-22 relative,
// well inside the 1e-5 output tolerance.
//
// Tiles: 64 tokens x 64 rows per workgroup of 4 waves (2 x 2, one 32 x 32
// MFMA tile each); K advances one super-block (Q4_K) or half a super-block
// (Q6_K) per stage, staged through LDS with the next stage's global loads in
// flight during the current stage's arithmetic. Workgroup b runs on XCD
// b % 8, and each XCD is given a contiguous run of tiles in token-tile-major
// order: the workgroups resident on one XCD share one token tile, whose
// activations then stay in that XCD's L2.
#include "hako_dev.h"
#include "hako_rt.h"
#include "skinny.h"
#include "q4k_dev.h"

namespace hako {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kTM = 64, kTN = 64;   // tokens, weight rows per workgroup tile
constexpr int kGT = 256;            // threads per workgroup
constexpr int kXcds = 8;

__device__ __forceinline__ int xcd_tile(int b, int ntiles) {
	const int per = (ntiles + kXcds - 1) / kXcds;
	return (b % kXcds) * per + b / kXcds;
}

// Tile t of an XCD-contiguous order to its (token tile, row tile): groups of
// gm token tiles, row tiles major and token tiles minor within a group. An
// XCD's range of tiles then covers gm token tiles x (its share of) the row
// tiles, and the tiles that share a row tile's weights (or a token tile's
// activations) run on one XCD at the same time, sharing its L2.
__device__ __forceinline__ void tile_mn(int t, int ntiles, int gm, int &mt, int &nt) {
	const int span = gm * ntiles, g = t / span, r = t - g * span;
	nt = r / gm;
	mt = g * gm + (r - nt * gm);
}


// ── Q4_K x q8 ──

constexpr int kAPad = 272;   // bytes per staged token row: 256 + 16 (conflict-free 16-byte reads)
constexpr int kFPad = 72;    // entries per sub-block row of the fold factors (64 + 8)

// Rows of a launch come from up to three segments (SkSegs: weight rows
// [row0, row0 + rows) of the launch's N rows, each with its own output matrix
// out[t*ld + r] and bias); a 64-row tile lies in one segment (segment starts
// are multiples of 64). Epilogues: Store out = y (+ bias), Add out += y (a
// residual), SwiGLU: N = 2F rows, tile j holds gate rows 32j.. (segment 0) and
// the same up rows (segment 1); out (segment 0's) = silu(gate)*up.
template <int EPI>
__global__ __launch_bounds__(kGT, 3) void q4k_gemm_kernel(const SkSegs segs, const int8_t *__restrict__ xq,
                                                       const float *__restrict__ xs, int M, int N, int K, int gm) {
	__shared__ __align__(16) uint8_t w_s[kTN * kQ4Bytes];   // this stage's block of each row
	__shared__ __align__(16) int8_t a_s[kTM * kAPad];       // this stage's 256 xq of each token
	// [sub-block][row or token], rows padded to 72: the stores of a stage
	// (four sub-blocks of one row, eight of one token, from neighbouring
	// lanes) then fall in different banks
	__shared__ __align__(16) float ds_s[8][kFPad];          // d*s   [sub-block][row]
	__shared__ __align__(16) float dm_s[8][kFPad];          // dmin*m
	__shared__ __align__(16) float2 xn_s[8][kFPad];         // (xs, -xs*Σxq) [sub-block][token]

	const int mtiles = (M + kTM - 1) / kTM, ntiles = (N + kTN - 1) / kTN;
	const int tile = xcd_tile(blockIdx.x, mtiles * ntiles);
	if (tile >= mtiles * ntiles) return;
	int mt, nt;
	tile_mn(tile, ntiles, gm, mt, nt);
	const int m0 = mt * kTM, n0 = nt * kTN;
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int wr = wave & 1, wt = wave >> 1, li = lane & 31, kh = lane >> 5;
	const int NB = K >> 8, NS = K >> 5;
	const uint32_t rb = (uint32_t)NB * kQ4Bytes;
	// the tile's segment (Store / Add), or for SwiGLU the matrix this wave
	// stages (waves 0-1 gate rows, 2-3 up rows) and the tile's first output row
	const int si = EPI == kSkSwiGLU ? (wave >> 1)
	               : (segs.n > 2 && n0 >= segs.s[2].row0) ? 2 : (segs.n > 1 && n0 >= segs.s[1].row0) ? 1 : 0;
	const SkSeg S = si == 0 ? segs.s[0] : (si == 1 ? segs.s[1] : segs.s[2]);
	const int r0 = EPI == kSkSwiGLU ? 32 * (n0 / kTN) : n0 - S.row0;   // first row of the tile in S
	const __amdgpu_buffer_rsrc_t wrs = stream_rsrc(S.w, rb * (uint32_t)S.rows);
	const __amdgpu_buffer_rsrc_t ars = stream_rsrc(xq, (uint32_t)M * (uint32_t)K);
	const __amdgpu_buffer_rsrc_t srs = stream_rsrc(xs, (uint32_t)M * (uint32_t)NS * 4u);

	// Stage map (one super-block of K per stage). Weights: the tile's 64 rows
	// x 8 pieces of 16 qs bytes, 2 per thread; a thread's rows come from the
	// matrix of its half of the workgroup (SwiGLU: threads 0-127 gate rows,
	// 128-255 the same up rows), so each wave's descriptor is uniform. Each
	// thread also loads the 16-byte header (d, dmin, scales) of row tid/4 and
	// derives (d*s, dmin*m) of its sub-blocks 2(tid%4), 2(tid%4)+1.
	// Activations: 64 tokens x 16 pieces of 16 xq bytes (half a sub-block),
	// 4 per thread, all of piece tid%16: the two halves of a sub-block sit in
	// neighbouring lanes, which add their sums of xq; and the q8 scale of each
	// of the thread's four (token, sub-block) pairs.
	const int half = tid >> 7;                       // matrix half of the tile
	auto srow_of = [&](int row) { return r0 + (EPI == kSkSwiGLU ? row - 32 * half : row); };
	const int wpc = tid & 7;                         // qs piece
	const int hrow = tid >> 2;                       // header row
	const int apc = tid & 15, asb = apc >> 1;        // activation piece, its sub-block
	uint4 wreg[2], hreg, areg[4];
	float sreg[4];
	auto load_stage = [&](int kb) {
		const uint32_t kbo = (uint32_t)kb * kQ4Bytes;
#pragma unroll
		for (int u = 0; u < 2; u++) {
			const int row = 32 * half + (((tid & 127) + 128 * u) >> 3), srow = srow_of(row);
			wreg[u] = ld_b128(wrs, srow < S.rows ? (uint32_t)srow * rb + kbo + 16u + 16u * wpc : kBufNone);
		}
		{
			const int srow = srow_of(hrow);
			hreg = ld_b128(wrs, srow < S.rows ? (uint32_t)srow * rb + kbo : kBufNone);
		}
#pragma unroll
		for (int u = 0; u < 4; u++) {
			const int tok = (tid >> 4) + 16 * u;
			const bool on = m0 + tok < M;
			areg[u] = ld_b128(ars, on ? (uint32_t)(m0 + tok) * K + 256u * kb + 16u * apc : kBufNone);
			sreg[u] = ld_f32(srs, on ? 4u * ((uint32_t)(m0 + tok) * NS + 8u * kb + asb) : kBufNone);
		}
	};
	// the loaded stage into LDS, with the per-row and per-token factors of the fold
	auto store_stage = [&]() {
		// LDS addresses recomputed per stage from an opaque copy of the thread
		// index: kept live across the loop they would be spilled (and reloaded
		// from scratch every stage)
		int t = threadIdx.x;
		asm volatile("" : "+v"(t));
		const int hrow = t >> 2, hg = t & 3, asb = (t & 15) >> 1;
#pragma unroll
		for (int u = 0; u < 2; u++) {
			const int row = 32 * (t >> 7) + (((t & 127) + 128 * u) >> 3);
			*(uint4 *)(w_s + row * kQ4Bytes + 16 + 16 * (t & 7)) = wreg[u];
		}
		{
			uint32_t S2, M2;
			q4_scales2(hreg.y, hreg.z, hreg.w, 16u * (hg & 1), hg >= 2 ? ~0u : 0u, S2, M2);
			const float d = f16_to_f32(hreg.x & 0xFFFFu), dmin = f16_to_f32(hreg.x >> 16);
			ds_s[2 * hg][hrow] = d * (float)(S2 & 0xFFu);
			ds_s[2 * hg + 1][hrow] = d * (float)((S2 >> 8) & 0xFFu);
			dm_s[2 * hg][hrow] = dmin * (float)(M2 & 0xFFu);
			dm_s[2 * hg + 1][hrow] = dmin * (float)((M2 >> 8) & 0xFFu);
		}
#pragma unroll
		for (int u = 0; u < 4; u++) {
			const int tok = (t >> 4) + 16 * u;
			*(uint4 *)(a_s + tok * kAPad + 16 * (t & 15)) = areg[u];
			int ix = sdot4((int)areg[u].x, 0x01010101, 0);
			ix = sdot4((int)areg[u].y, 0x01010101, ix);
			ix = sdot4((int)areg[u].z, 0x01010101, ix);
			ix = sdot4((int)areg[u].w, 0x01010101, ix);
			ix += dpp_i<kDppQuadSwap1>(ix);   // + the other half of the sub-block
			// both lanes of the pair write the same value
			xn_s[asb][tok] = make_float2(sreg[u], -sreg[u] * (float)ix);
		}
	};

	v16f acc = {}, accm = {};
	const v16i zero = {};
	const v32f zero32 = {};
	const uint32_t lo4 = 0x0F0F0F0Fu;
	load_stage(0);
	for (int kb = 0; kb < NB; kb++) {
		store_stage();
		__syncthreads();
		if (kb + 1 < NB) load_stage(kb + 1);   // in flight during this stage's arithmetic
		// The min term Σ_sb dm[row][sb] * (−xs*Σxq)[token][sb] is a small fp32
		// product over the block's 8 sub-blocks: four v_mfma_f32_32x32x2_f32
		// into their own accumulator (K index = sub-block, one per lane half).
#pragma unroll
		for (int p = 0; p < 4; p++) {
			const int sb = 2 * p + kh;
			accm = __builtin_amdgcn_mfma_f32_32x32x2f32(dm_s[sb][32 * wr + li], xn_s[sb][32 * wt + li].y, accm, 0,
			                                           0, 0);
		}
#pragma unroll
		for (int g = 0; g < 4; g++) {
			// The fold's scale products P[row][token] = (d*s)[row] * xs[token] of
			// sub-blocks 2g and 2g+1 as one two-block outer product on the matrix
			// cores (block h: lane half h supplies sub-block 2g+h), laid out like
			// the int8 products: P[16h + v] pairs with d[v] of sub-block 2g+h.
			const v32f P = __builtin_amdgcn_mfma_f32_32x32x1f32(ds_s[2 * g + kh][32 * wr + li],
			                                                    xn_s[2 * g + kh][32 * wt + li].x, zero32, 0, 0, 0);
			// weight row 32wr+li: qs bytes 32g+16kh.. hold K 16kh.. of sub-blocks 2g (low
			// nibbles) and 2g+1 (high nibbles)
			const uint4 q = *(const uint4 *)(w_s + (32 * wr + li) * kQ4Bytes + 16 + 32 * g + 16 * kh);
			const v4i qlo = {(int)(q.x & lo4), (int)(q.y & lo4), (int)(q.z & lo4), (int)(q.w & lo4)};
			const v4i qhi = {(int)((q.x >> 4) & lo4), (int)((q.y >> 4) & lo4), (int)((q.z >> 4) & lo4),
			                 (int)((q.w >> 4) & lo4)};
#pragma unroll
			for (int h = 0; h < 2; h++) {
				const int sb = 2 * g + h;
				const v4i b = *(const v4i *)(a_s + (32 * wt + li) * kAPad + 32 * sb + 16 * kh);
				const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(h ? qhi : qlo, b, zero, 0, 0, 0);
#pragma unroll
				for (int v = 0; v < 16; v++) acc[v] = __builtin_fmaf((float)d[v], P[16 * h + v], acc[v]);
			}
		}
		__syncthreads();   // before the next stage overwrites LDS
	}
	// lane: token m0+32wt+li, tile rows 32wr+8q4+4kh+r
	const int tok = m0 + 32 * wt + li;
	if (EPI == kSkSwiGLU) {
		// the up half (wr = 1) hands its sums to the gate half through LDS
		// (the loop ended with a barrier: a_s is free)
		float *up_s = (float *)a_s + (wt * 64 + lane) * 16;
		if (wr == 1)
#pragma unroll
			for (int v = 0; v < 16; v++) up_s[v] = acc[v] + accm[v];
		__syncthreads();
		if (wr == 1 || tok >= M) return;
		float *hr = segs.s[0].out + (size_t)tok * segs.s[0].ld;
#pragma unroll
		for (int q4 = 0; q4 < 4; q4++) {
			const int f = r0 + 8 * q4 + 4 * kh;
#pragma unroll
			for (int r = 0; r < 4; r++)
				if (f + r < segs.s[0].rows) hr[f + r] = silu(acc[4 * q4 + r] + accm[4 * q4 + r]) * up_s[4 * q4 + r];
		}
		return;
	}
	// Store / Add: every operand load (the bias, or the output the sums are
	// added to) first, then the stores; lanes past the rows or tokens use an
	// offset past the stream (no access), so no branch separates the loads
	// and each does not wait for the one before
	const int ld = __builtin_amdgcn_readfirstlane(S.ld), srows = __builtin_amdgcn_readfirstlane(S.rows);
	float *out = uniform_ptr(S.out);
	const float *bias = uniform_ptr(S.bias);
	const __amdgpu_buffer_rsrc_t ors = stream_rsrc(out, (uint32_t)M * (uint32_t)ld * 4u);
	const __amdgpu_buffer_rsrc_t brs =
	    stream_rsrc(bias ? (const void *)bias : (const void *)out, (EPI == kSkStore && bias) ? (uint32_t)srows * 4u : 0u);
	uint32_t off[16];
	float ev[16];
#pragma unroll
	for (int q4 = 0; q4 < 4; q4++) {
		const int row = r0 + 32 * wr + 8 * q4 + 4 * kh;
#pragma unroll
		for (int r = 0; r < 4; r++) {
			const bool ok = tok < M && row + r < srows;
			off[4 * q4 + r] = ok ? 4u * ((uint32_t)tok * ld + row + r) : kBufNone;
			ev[4 * q4 + r] = EPI == kSkAdd ? ld_f32(ors, off[4 * q4 + r]) : ld_f32(brs, ok ? 4u * (row + r) : kBufNone);
		}
	}
#pragma unroll
	for (int v = 0; v < 16; v++) st_f32(ors, off[v], EPI == kSkAdd ? ev[v] + (acc[v] + accm[v]) : (acc[v] + accm[v]) + ev[v]);
}

// ── Q4_K x q8, resident token tile ──
//
// The tiled kernel above stages a 64-token activation block from L2 for
// every 64-row weight tile and waits out one memory round trip per stage.
// Here a workgroup keeps all K of 32 tokens in LDS (32·(K+16) bytes of q8 plus
// the per-(sub-block, token) factors (xs, −xs·Σxq), 40·K + 512 bytes in
// all: K up to 3840) and its twelve waves stream weight rows past it, each
// wave a 32-row unit through the whole K with the next super-block's loads in
// flight, weights straight from memory into the MFMA operand registers. The
// arithmetic is the tiled kernel's: per sub-block one
// v_mfma_i32_32x32x32_i8 (the reference's iqx), the fold
// acc += iqx·(d·s·xs) with the products d·s·xs from a v_mfma_f32_32x32x1f32
// outer product, and the min term on v_mfma_f32_32x32x2f32.
// Units: Store / Add rows 32u .. 32u+31 of the launch (a unit lies in one
// segment: segment starts are multiples of 64); SwiGLU features
// 16u .. 16u+15, MFMA rows 0-15 their gate rows and 16-31 their up rows, so a
// lane holds each feature's gate and up sums side by side.
// Grid: token tiles x R row ranges, in XCD-contiguous order with the token
// tiles minor: the workgroups of one XCD share a row range, whose weights
// then come from that XCD's L2 after the first read.
constexpr int kRT = 32;          // tokens per workgroup
constexpr int kRWaves = 12;      // waves per workgroup (one workgroup per CU: LDS), three per SIMD
constexpr int kRMaxK = 3840;     // largest K whose token tile fits 160 KB of LDS

__host__ __device__ inline size_t q4k_res_lds(int K) { return (size_t)kRT * (K + 16) + (size_t)(K / 32) * kRT * 8; }

template <int EPI>
__global__ __launch_bounds__(kRWaves * kWave, 1) void q4k_gemm_res_kernel(const SkSegs segs,
                                                                       const int8_t *__restrict__ xq,
                                                                       const float *__restrict__ xs, int M, int K,
                                                                       int R, int units) {
	extern __shared__ __align__(16) uint8_t res_lds[];
	const int AP = K + 16;                              // bytes per staged token row
	int8_t *a_s = (int8_t *)res_lds;
	float2 *xn_s = (float2 *)(res_lds + kRT * AP);      // [sub-block][token]
	const int mt = (M + kRT - 1) / kRT, G = mt * R;
	const int p = xcd_tile(blockIdx.x, G);
	if (p >= G) return;
	const int rr = p / mt, m0 = (p - rr * mt) * kRT;
	const int NB = K >> 8, NS = K >> 5;
	const int tid = threadIdx.x, lane = tid & 63;
	const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
	const int li = lane & 31, kh = lane >> 5;

	// 1. the token tile: 16-byte pieces, all loads of a thread issued before
	//    its stores (rows past M read as zero)
	{
		const __amdgpu_buffer_rsrc_t ars = stream_rsrc(xq, (uint32_t)M * (uint32_t)K);
		const int ppr = K >> 4, total = kRT * ppr;
		constexpr int kPer = (kRT * (kRMaxK / 16) + kRWaves * kWave - 1) / (kRWaves * kWave);
		uint4 v[kPer];
#pragma unroll
		for (int u = 0; u < kPer; u++) {
			const int c = tid + kRWaves * kWave * u, tok = c / ppr, pc = c - tok * ppr;
			const bool on = c < total && m0 + tok < M;
			v[u] = ld_b128(ars, on ? (uint32_t)(m0 + tok) * K + 16u * pc : kBufNone);
		}
#pragma unroll
		for (int u = 0; u < kPer; u++) {
			const int c = tid + kRWaves * kWave * u, tok = c / ppr, pc = c - tok * ppr;
			if (c < total) *(uint4 *)(a_s + tok * AP + 16 * pc) = v[u];
		}
	}
	__syncthreads();
	{
		const __amdgpu_buffer_rsrc_t srs = stream_rsrc(xs, (uint32_t)M * (uint32_t)NS * 4u);
		for (int c = tid; c < kRT * NS; c += kRWaves * kWave) {
			const int sb = c / kRT, tok = c - sb * kRT;
			const float f = ld_f32(srs, m0 + tok < M ? 4u * ((uint32_t)(m0 + tok) * NS + sb) : kBufNone);
			const int4 a = *(const int4 *)(a_s + tok * AP + 32 * sb), b = *(const int4 *)(a_s + tok * AP + 32 * sb + 16);
			int ix = sdot4(a.x, 0x01010101, 0);
			ix = sdot4(a.y, 0x01010101, ix);
			ix = sdot4(a.z, 0x01010101, ix);
			ix = sdot4(a.w, 0x01010101, ix);
			ix = sdot4(b.x, 0x01010101, ix);
			ix = sdot4(b.y, 0x01010101, ix);
			ix = sdot4(b.z, 0x01010101, ix);
			ix = sdot4(b.w, 0x01010101, ix);
			xn_s[sb * kRT + tok] = make_float2(f, -f * (float)ix);
		}
	}
	__syncthreads();

	// 2. the units of this row range, one per wave at a time
	const int u0 = (int)((long long)rr * units / R), u1 = (int)((long long)(rr + 1) * units / R);
	const uint32_t rb = (uint32_t)NB * kQ4Bytes;
	const int8_t *a_row = a_s + li * AP + 16 * kh;      // B operand: token li, K 16kh.. of each sub-block
	const float2 *xn_row = xn_s + li;
	const uint32_t lo4 = 0x0F0F0F0Fu;
	const v16i zero = {};
	const v32f zero32 = {};
	struct Wt {
		uint4 q[4];   // qs bytes 32g + 16kh .. +16 of the lane's row
		uint4 h;      // d, dmin, 12 scale bytes
	};
	for (int u = u0 + wave; u < u1; u += kRWaves) {
		// the lane's weight row (clamped into its matrix; rows past the end are
		// computed and not stored)
		const int r32 = 32 * u;
		const int si = EPI == kSkSwiGLU ? 0
		               : (segs.n > 2 && r32 >= segs.s[2].row0) ? 2 : (segs.n > 1 && r32 >= segs.s[1].row0) ? 1 : 0;
		const SkSeg S = si == 0 ? segs.s[0] : (si == 1 ? segs.s[1] : segs.s[2]);
		const int srows = S.rows;
		// first output row of the unit in its segment (SwiGLU: first feature),
		// the lane's weight row and matrix
		const int out_row0 = EPI == kSkSwiGLU ? 16 * u : r32 - S.row0;
		const int srow = EPI == kSkSwiGLU ? out_row0 + (li & 15) : out_row0 + li;
		const uint8_t *wmat = (EPI == kSkSwiGLU && li >= 16) ? segs.s[1].w : S.w;
		const uint8_t *wrow = wmat + (size_t)min(srow, srows - 1) * rb;
		auto load = [&](Wt &w, int kb) {
			const uint8_t *b = wrow + (size_t)kb * kQ4Bytes;
			w.h = *(const uint4 *)b;
#pragma unroll
			for (int g = 0; g < 4; g++) w.q[g] = *(const uint4 *)(b + 16 + 32 * g + 16 * kh);
		};
		v16f acc = {}, accm = {};
		auto compute = [&](const Wt &w, int kb) {
			// (d·s, dmin·m) of sub-blocks 2g + kh, g = 0..3: bytes kh and 2 + kh
			// of the scale words (reference quant.c:57-66 packing)
			const float d = f16_to_f32(w.h.x & 0xFFFFu), dmin = f16_to_f32(w.h.x >> 16);
			const uint32_t sh = 8u * kh;
			const uint32_t a0 = w.h.y >> sh, a1 = w.h.z >> sh, a2 = w.h.w >> sh;
			const uint32_t s_lo = a0 & 0x003F003Fu, m_lo = a1 & 0x003F003Fu;
			const uint32_t s_hi = (a2 & 0x000F000Fu) | ((a0 >> 2) & 0x00300030u);
			const uint32_t m_hi = ((a2 >> 4) & 0x000F000Fu) | ((a1 >> 2) & 0x00300030u);
			const float ds[4] = {d * (float)(s_lo & 0xFFu), d * (float)(s_lo >> 16), d * (float)(s_hi & 0xFFu),
			                     d * (float)(s_hi >> 16)};
			const float dm[4] = {dmin * (float)(m_lo & 0xFFu), dmin * (float)(m_lo >> 16),
			                     dmin * (float)(m_hi & 0xFFu), dmin * (float)(m_hi >> 16)};
			const float2 *xn = xn_row + 8 * kb * kRT;
#pragma unroll
			for (int g = 0; g < 4; g++)
				accm = __builtin_amdgcn_mfma_f32_32x32x2f32(dm[g], xn[(2 * g + kh) * kRT].y, accm, 0, 0, 0);
			// the block's eight activation operands, all LDS reads issued at once
			v4i bb[8];
#pragma unroll
			for (int j = 0; j < 8; j++) bb[j] = *(const v4i *)(a_row + 256 * kb + 32 * j);
#pragma unroll
			for (int g = 0; g < 4; g++) {
				const v32f P = __builtin_amdgcn_mfma_f32_32x32x1f32(ds[g], xn[(2 * g + kh) * kRT].x, zero32, 0, 0, 0);
				const uint4 q = w.q[g];
				const v4i qlo = {(int)(q.x & lo4), (int)(q.y & lo4), (int)(q.z & lo4), (int)(q.w & lo4)};
				const v4i qhi = {(int)((q.x >> 4) & lo4), (int)((q.y >> 4) & lo4), (int)((q.z >> 4) & lo4),
				                 (int)((q.w >> 4) & lo4)};
#pragma unroll
				for (int h = 0; h < 2; h++) {
					const v4i b = bb[2 * g + h];
					const v16i iq = __builtin_amdgcn_mfma_i32_32x32x32_i8(h ? qhi : qlo, b, zero, 0, 0, 0);
#pragma unroll
					for (int v = 0; v < 16; v++) acc[v] = __builtin_fmaf((float)iq[v], P[16 * h + v], acc[v]);
				}
			}
		};
		// super-blocks in pairs, so each register set is named statically; the
		// loads in the loop are unconditional (past the last block they repeat
		// it), so the wait before each block's arithmetic counts only the older
		// set
		Wt wa, wb;
		load(wa, 0);
		int kb = 0;
		for (; kb + 1 < NB; kb += 2) {
			load(wb, kb + 1);
			__builtin_amdgcn_sched_barrier(0);   // issued here, not next to their use
			compute(wa, kb);
			load(wa, min(kb + 2, NB - 1));
			__builtin_amdgcn_sched_barrier(0);
			compute(wb, kb + 1);
		}
		if (kb < NB) compute(wa, kb);   // odd NB: the last block, loaded into wa

		// 3. epilogue; lane: token m0 + li, MFMA rows 8q4 + 4kh + r
		const int tok = m0 + li;
		if (EPI == kSkSwiGLU) {
			if (tok < M) {
				float *hr = S.out + (size_t)tok * S.ld;
#pragma unroll
				for (int q4 = 0; q4 < 2; q4++) {
					const int f = out_row0 + 8 * q4 + 4 * kh;
#pragma unroll
					for (int r = 0; r < 4; r++)
						if (f + r < srows)
							hr[f + r] = silu(acc[4 * q4 + r] + accm[4 * q4 + r]) *
							            (acc[4 * q4 + 8 + r] + accm[4 * q4 + 8 + r]);
				}
			}
			continue;
		}
		const int ld = __builtin_amdgcn_readfirstlane(S.ld);
		float *out = uniform_ptr(S.out);
		const float *bias = uniform_ptr(S.bias);
		const __amdgpu_buffer_rsrc_t ors = stream_rsrc(out, (uint32_t)M * (uint32_t)ld * 4u);
		const __amdgpu_buffer_rsrc_t brs =
		    stream_rsrc(bias ? (const void *)bias : (const void *)out, (EPI == kSkStore && bias) ? (uint32_t)srows * 4u : 0u);
		uint32_t off[16];
		float ev[16];
#pragma unroll
		for (int q4 = 0; q4 < 4; q4++) {
			const int row = out_row0 + 8 * q4 + 4 * kh;
#pragma unroll
			for (int r = 0; r < 4; r++) {
				const bool ok = tok < M && row + r < srows;
				off[4 * q4 + r] = ok ? 4u * ((uint32_t)tok * ld + row + r) : kBufNone;
				ev[4 * q4 + r] = EPI == kSkAdd ? ld_f32(ors, off[4 * q4 + r]) : ld_f32(brs, ok ? 4u * (row + r) : kBufNone);
			}
		}
#pragma unroll
		for (int v = 0; v < 16; v++)
			st_f32(ors, off[v], EPI == kSkAdd ? ev[v] + (acc[v] + accm[v]) : (acc[v] + accm[v]) + ev[v]);
	}
}

// ── Q6_K x fp32 ──

// Token row t of x (K floats): s = 2^-e with max|x_t| in [2^e, 2^(e+1)),
// hi = fp16(x*s), lo = fp16(x*s - hi), esc[t] = 2^e. The scaling is exact,
// and x*s - hi is exact in fp32. 1024 threads per row; up to kSplitPer float4 per thread are
// loaded once, all at the start, and kept in registers for both passes
// (rows longer than that run the tail from memory).
constexpr int kSplitT = 1024, kSplitPer = 8;
__global__ __launch_bounds__(kSplitT) void f16_split_kernel(const float *__restrict__ x, _Float16 *__restrict__ xh,
                                                            _Float16 *__restrict__ xl, float *__restrict__ esc,
                                                            int K) {
	__shared__ float red[kSplitT / kWave];
	const size_t base = (size_t)blockIdx.x * K;
	const float *xr = x + base;
	float4 v[kSplitPer];
#pragma unroll
	for (int u = 0; u < kSplitPer; u++) {
		const int i = (threadIdx.x + kSplitT * u) * 4;
		v[u] = *(const float4 *)(xr + min(i, K - 4));
	}
	auto amax4 = [](float4 q) {
		return __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(q.x), __builtin_fabsf(q.y)),
		                       __builtin_fmaxf(__builtin_fabsf(q.z), __builtin_fabsf(q.w)));
	};
	float a = 0.0f;
#pragma unroll
	for (int u = 0; u < kSplitPer; u++) a = __builtin_fmaxf(a, amax4(v[u]));   // clamped repeats are harmless
	for (int i = (threadIdx.x + kSplitT * kSplitPer) * 4; i < K; i += kSplitT * 4)
		a = __builtin_fmaxf(a, amax4(*(const float4 *)(xr + i)));
	a = __builtin_fmaxf(a, dpp_f<kDppQuadSwap1>(a));
	a = __builtin_fmaxf(a, dpp_f<kDppQuadSwap2>(a));
	a = __builtin_fmaxf(a, dpp_f<kDppHalfMirror>(a));
	a = __builtin_fmaxf(a, dpp_f<kDppMirror>(a));
	a = __builtin_fmaxf(a, __shfl_xor(a, 16));
	a = __builtin_fmaxf(a, __shfl_xor(a, 32));
	if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = a;
	__syncthreads();
	a = 0.0f;
#pragma unroll
	for (int w = 0; w < kSplitT / kWave; w++) a = __builtin_fmaxf(a, red[w]);
	const int e = f16_split_exp(a);
	const float s = __builtin_ldexpf(1.0f, -e);
	if (threadIdx.x == 0) esc[blockIdx.x] = __builtin_ldexpf(1.0f, e);
	auto put = [&](int i, float4 q) {
		const float f[4] = {q.x * s, q.y * s, q.z * s, q.w * s};
		typedef _Float16 v4h_t __attribute__((ext_vector_type(4)));
		v4h_t h, l;
#pragma unroll
		for (int k = 0; k < 4; k++) {
			h[k] = (_Float16)f[k];
			l[k] = (_Float16)(f[k] - (float)h[k]);
		}
		*(v4h_t *)(xh + base + i) = h;
		*(v4h_t *)(xl + base + i) = l;
	};
#pragma unroll
	for (int u = 0; u < kSplitPer; u++) {
		const int i = (threadIdx.x + kSplitT * u) * 4;
		if (i < K) put(i, v[u]);
	}
	for (int i = (threadIdx.x + kSplitT * kSplitPer) * 4; i < K; i += kSplitT * 4) put(i, *(const float4 *)(xr + i));
}

// Two of the 6-bit values in `v` (bytes picked by the v_perm selector `sel`
// into the low byte of each half, selector byte 4 placing the exponent byte
// 0x64 above each) as the fp16 pair (q0 - 32, q1 - 32): 0x6400 | q is
// 1024 + q exactly, and 1024 + q - 1056 is exact.
__device__ __forceinline__ uint32_t q6_pair(uint32_t v, uint32_t sel) {
	typedef _Float16 v2h __attribute__((ext_vector_type(2)));
	const uint32_t t = __builtin_amdgcn_perm(0x64646464u, v, sel);
	const v2h r = __builtin_bit_cast(v2h, t) - (v2h){(_Float16)1056.0f, (_Float16)1056.0f};
	return __builtin_bit_cast(uint32_t, r);
}

constexpr int kQ6Stage = 128;        // K per stage: half a super-block
constexpr int kHPad = kQ6Stage + 8;  // fp16 per staged row (272 B: conflict-free 16-byte reads)

// LDS of one stage buffer of a TN-row tile: activation hi and lo
// [64][kHPad], q - 32 [TN][kHPad] (fp16), d*sc [8 groups][TN] (fp32).
__host__ __device__ constexpr size_t q6g_buf_bytes(int tn) {
	return (size_t)(2 * kTM + tn) * kHPad * 2 + (size_t)8 * tn * 4;
}

// Tile: 64 tokens x TN rows (64 or 128), one thread per (weight row,
// quarter of a stage's bytes), waves of one 32 x 32 MFMA tile each (2 token
// halves x TN/32 row quarters), so every output's arithmetic is the same at
// both widths. TN = 64: two workgroups per CU, one LDS buffer, two barriers
// per stage. TN = 128 (DB): one workgroup per CU with the stage buffers
// double-buffered in LDS, one barrier per stage; a stage's activation then serves twice
// the rows, so each output needs ~40% fewer staged bytes.
//
// Epilogue of a 32 x 32 MFMA tile: lane (li, kh) of wave (wr, wt) holds
// row n0+32wr+li, tokens m0+32wt+8q4+4kh+r. Every operand load (token
// scales, bias, the output added to) first, then the stores; lanes past the
// rows or tokens use an offset past the stream.
__device__ __forceinline__ void q6g_epilogue(const v16f &acc, int m0, int n0, int wr, int wt, int li, int kh, int M,
                                             int N, float *y, const float *esc, const float *bias, int add) {
	const int row = n0 + 32 * wr + li;
	const bool rok = row < N;
	const __amdgpu_buffer_rsrc_t yrs = stream_rsrc(y, (uint32_t)M * (uint32_t)N * 4u);
	const __amdgpu_buffer_rsrc_t ars = stream_rsrc(y, add ? (uint32_t)M * (uint32_t)N * 4u : 0u);
	const __amdgpu_buffer_rsrc_t ers = stream_rsrc(esc, (uint32_t)M * 4u);
	const __amdgpu_buffer_rsrc_t brs = stream_rsrc(bias ? (const void *)bias : (const void *)esc, bias ? (uint32_t)N * 4u : 0u);
	const float bv = ld_f32(brs, rok ? 4u * row : kBufNone);
	uint32_t off[16];
	float ev[16], ov[16];
#pragma unroll
	for (int u = 0; u < 16; u++) {
		const int tok = m0 + 32 * wt + 8 * (u >> 2) + 4 * kh + (u & 3);
		const bool ok = rok && tok < M;
		off[u] = ok ? 4u * ((uint32_t)tok * N + row) : kBufNone;
		ev[u] = ld_f32(ers, ok ? 4u * tok : kBufNone);
		ov[u] = ld_f32(ars, off[u]);
	}
#pragma unroll
	for (int u = 0; u < 16; u++) {
		const float r = acc[u] * ev[u] + bv;
		st_f32(yrs, off[u], add ? ov[u] + r : r);
	}
}

//
// SK (stream-K, with DB): the grid's G workgroups split the launch's
// tiles x super-blocks evenly, workgroup v (its place in the XCD-contiguous
// order) taking units [v·U/G, (v+1)·U/G) of the U = tiles·NB in tile order.
// (Used when tiles < G, so a range is no longer than a tile and meets at
// most two tiles.) The workgroup leaves
// each tile's sums, unscaled, in its slot v·2 + (first tile ? 0 : 1) of
// `skp` (the thread's 16 sums side by side), and q6k_gemm_sk_fixup_kernel
// adds a tile's slots in workgroup order and applies the epilogue. With 224
// tiles of 128 rows on 256 CUs (7B down over 512 tokens) every CU works
// instead of 7 in 8.
template <int TN, bool DB, bool SK = false>
__global__ __launch_bounds__(4 * TN, DB ? 1 : 2) void q6k_gemm_kernel(const uint8_t *__restrict__ w,
                                                                     const _Float16 *__restrict__ xh,
                                                                     const _Float16 *__restrict__ xl,
                                                                     const float *__restrict__ esc,
                                                                     const float *__restrict__ bias,
                                                                     float *__restrict__ y, int M, int N, int K,
                                                                     int add, int gm, float *__restrict__ skp) {
	static_assert(!SK || DB, "stream-K runs the double-buffered tiles");
	constexpr int T = 4 * TN;           // threads
	constexpr int PA = kTM * 16 / T;    // activation pieces (16 B) per thread, hi and lo each
	constexpr int RQ = TN / 32;         // row quarters (waves per token half)
	extern __shared__ __align__(16) uint8_t q6g_lds[];
	struct View {
		_Float16 *ah, *al, *wq;
		float *dsc;   // [8][TN]
	};
	auto view = [&](int b) -> View {
		uint8_t *p = q6g_lds + (size_t)b * q6g_buf_bytes(TN);
		View v;
		v.ah = (_Float16 *)p;
		v.al = v.ah + kTM * kHPad;
		v.wq = v.al + kTM * kHPad;
		v.dsc = (float *)(v.wq + TN * kHPad);
		return v;
	};

	const int mtiles = (M + kTM - 1) / kTM, ntiles = (N + TN - 1) / TN;
	const int NB = K >> 8;
	// SK: this workgroup's units (super-blocks of tiles in tile order)
	int64_t u_beg = 0, u_end = 0;
	int tile, vpos = 0;
	if constexpr (SK) {
		vpos = xcd_tile(blockIdx.x, gridDim.x);
		const int64_t U = (int64_t)mtiles * ntiles * NB;
		u_beg = (int64_t)vpos * U / gridDim.x;
		u_end = (int64_t)(vpos + 1) * U / gridDim.x;
		if (u_end <= u_beg) return;
		tile = (int)(u_beg / NB);
	} else {
		tile = xcd_tile(blockIdx.x, mtiles * ntiles);
		if (tile >= mtiles * ntiles) return;
	}
	int mt, nt;
	tile_mn(tile, ntiles, gm, mt, nt);
	int m0 = mt * kTM, n0 = nt * TN;
	const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
	const int wr = wave % RQ, wt = wave / RQ, li = lane & 31, kh = lane >> 5;
	const uint32_t rb = (uint32_t)NB * kQ6Bytes;
	const __amdgpu_buffer_rsrc_t wrs = stream_rsrc(w, rb * (uint32_t)N);
	const __amdgpu_buffer_rsrc_t hrs = stream_rsrc(xh, (uint32_t)M * (uint32_t)K * 2u);
	const __amdgpu_buffer_rsrc_t lrs = stream_rsrc(xl, (uint32_t)M * (uint32_t)K * 2u);

	// Stage st = half n of block st/2. Activations: 64 tokens x 16 pieces of
	// 16 B (8 fp16) for hi and lo, PA + PA per thread. Weights: thread (row
	// tid/4, part p = tid%4) takes ql[64n+16p, +16) — K 32(p/2)+16(p%2)+b
	// (low nibbles) and that + 64 (high nibbles) of the half — with qh
	// [32n+16(p%2), +16), and the scales 8n+2p, 8n+2p+1 and d.
	const int wrow = tid >> 2, part = tid & 3;
	// The activation loads of two stages are in flight while a third is
	// computed: one stage's arithmetic is too short to cover a load's latency
	// by itself. The weight pieces (a sixth of the bytes) go one stage ahead.
	struct Acts {
		uint4 h[PA], l[PA];
	};
	struct Wts {
		uint2 ql[2], qh[2];
		uint32_t sc, d;
	};
	const int NSt = NB * 2;
	int s_end = NSt;   // stages past it load nothing
	// unconditional: a stage past the last loads nothing (out-of-range offsets)
	auto load_acts = [&](Acts &r, int st) {
		const uint32_t k0 = (uint32_t)kQ6Stage * st;
#pragma unroll
		for (int u = 0; u < PA; u++) {
			const int c = tid + T * u, tok = c >> 4, piece = c & 15;
			const bool on = st < s_end && m0 + tok < M;
			const uint32_t off = on ? 2u * ((uint32_t)(m0 + tok) * K + k0 + 8u * piece) : kBufNone;
			r.h[u] = ld_b128(hrs, off);
			r.l[u] = ld_b128(lrs, off);
		}
	};
	auto load_wts = [&](Wts &r, int st) {
		const int kb = st >> 1, n = st & 1;
		const bool on = st < s_end && n0 + wrow < N;
		const uint32_t blk = on ? (uint32_t)(n0 + wrow) * rb + (uint32_t)kb * kQ6Bytes : kBufNone;
		const uint32_t oql = 64u * n + 16u * part, oqh = 128u + 32u * n + 16u * (part & 1);
		r.ql[0] = ld_b64(wrs, blk + oql);
		r.ql[1] = ld_b64(wrs, blk + oql + 8);
		r.qh[0] = ld_b64(wrs, blk + oqh);
		r.qh[1] = ld_b64(wrs, blk + oqh + 8);
		r.sc = ld_b16(wrs, blk + 192u + 8u * n + 2u * part);
		r.d = ld_b16(wrs, blk + 208u);
	};
	auto store_acts = [&](const Acts &r, const View &v) {
#pragma unroll
		for (int u = 0; u < PA; u++) {
			const int c = tid + T * u, tok = c >> 4, piece = c & 15;
			*(uint4 *)(v.ah + tok * kHPad + 8 * piece) = r.h[u];
			*(uint4 *)(v.al + tok * kHPad + 8 * piece) = r.l[u];
		}
	};
	auto store_wts = [&](const Wts &r, const View &v) {
		// 6-bit values: low nibble | qh bits 2k1 (k1 = part/2) -> K 32k1 + l,
		// high nibble | qh bits 2k1+4 -> K 32(k1+2) + l, with l = 16(part%2) + b.
		const int k1 = part >> 1, l0 = 16 * (part & 1);
		const uint32_t ql[4] = {r.ql[0].x, r.ql[0].y, r.ql[1].x, r.ql[1].y};
		const uint32_t qh[4] = {r.qh[0].x, r.qh[0].y, r.qh[1].x, r.qh[1].y};
		uint32_t lo[8], hi[8];   // fp16 pairs
#pragma unroll
		for (int j = 0; j < 4; j++) {
			// qh bits 2k1, 2k1+1 (and 2k1+4, 2k1+5) of each byte to bits 4, 5
			const uint32_t vlo = ((qh[j] << (4 - 2 * k1)) & 0x30303030u) | (ql[j] & 0x0F0F0F0Fu);
			const uint32_t vhi = ((qh[j] >> (2 * k1)) & 0x30303030u) | ((ql[j] >> 4) & 0x0F0F0F0Fu);
			lo[2 * j] = q6_pair(vlo, 0x04010400u);
			lo[2 * j + 1] = q6_pair(vlo, 0x04030402u);
			hi[2 * j] = q6_pair(vhi, 0x04010400u);
			hi[2 * j + 1] = q6_pair(vhi, 0x04030402u);
		}
		uint8_t *wrow_s = (uint8_t *)(v.wq + wrow * kHPad);
		*(uint4 *)(wrow_s + 2 * (32 * k1 + l0)) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
		*(uint4 *)(wrow_s + 2 * (32 * k1 + l0 + 8)) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
		*(uint4 *)(wrow_s + 2 * (32 * (k1 + 2) + l0)) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
		*(uint4 *)(wrow_s + 2 * (32 * (k1 + 2) + l0 + 8)) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
		// group gg = 2*part + i covers K [16gg, 16gg+16): scale 8n + gg
		const float d = f16_to_f32(r.d);
		v.dsc[(2 * part) * TN + wrow] = d * (float)(int8_t)(r.sc & 0xFFu);
		v.dsc[(2 * part + 1) * TN + wrow] = d * (float)(int8_t)(r.sc >> 8);
	};

	v16f acc = {};
	const v16f zero = {};
	auto compute = [&](const View &v) {
		const _Float16 *ah = v.ah + (32 * wt + li) * kHPad + 8 * kh;
		const _Float16 *al = v.al + (32 * wt + li) * kHPad + 8 * kh;
		const _Float16 *wq = v.wq + (32 * wr + li) * kHPad + 8 * kh;
#pragma unroll
		for (int gg = 0; gg < 8; gg++) {
			const v8h b = *(const v8h *)(wq + 16 * gg);
			v16f p = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const v8h *)(ah + 16 * gg), b, zero, 0, 0, 0);
			p = __builtin_amdgcn_mfma_f32_32x32x16_f16(*(const v8h *)(al + 16 * gg), b, p, 0, 0, 0);
			const float s = v.dsc[gg * TN + 32 * wr + li];
#pragma unroll
			for (int u = 0; u < 16; u++) acc[u] = __builtin_fmaf(p[u], s, acc[u]);
			// DB: the operand reads of four groups at a time (all eight hoisted
			// spill beside the second stage buffer's addresses)
			if (DB && (gg & 3) == 3) __builtin_amdgcn_sched_barrier(0);
		}
	};
	const View v0 = view(0);
	if constexpr (!DB) {
		Acts aa, ab;
		Wts wts;
		load_acts(aa, 0);
		load_wts(wts, 0);
		load_acts(ab, 1);
		// NSt is even: the loop takes the stages in pairs, so each activation
		// register set is named statically
		for (int st = 0; st < NSt; st += 2) {
			store_acts(aa, v0);
			store_wts(wts, v0);
			__syncthreads();
			load_wts(wts, st + 1);
			load_acts(aa, st + 2);
			compute(v0);
			__syncthreads();
			store_acts(ab, v0);
			store_wts(wts, v0);
			__syncthreads();
			load_wts(wts, st + 2);
			load_acts(ab, st + 3);
			compute(v0);
			__syncthreads();
		}
	} else {
		// Stage st lives in LDS buffer st % 2. A wave stores stage st only
		// after the barrier that followed the stores of stage st - 1, which
		// every wave passes after computing stage st - 2, the buffer's last
		// reader: one barrier per stage.
		const View v1 = view(1);
		Acts aa, ab;
		Wts wts;
		// stages [sa, sb) of the current tile
		auto pipeline = [&](int sa, int sb) {
			s_end = sb;
			load_acts(aa, sa);
			load_wts(wts, sa);
			load_acts(ab, sa + 1);
			for (int st = sa; st < sb; st += 2) {
				store_acts(aa, v0);
				store_wts(wts, v0);
				__syncthreads();
				load_wts(wts, st + 1);
				load_acts(aa, st + 2);
				compute(v0);
				store_acts(ab, v1);
				store_wts(wts, v1);
				__syncthreads();
				load_wts(wts, st + 2);
				load_acts(ab, st + 3);
				compute(v1);
			}
		};
		if constexpr (SK) {
			// one or two tiles: each piece's sums to its slot, then the next
			// tile (the buffers' last readers passed a barrier since: v0 was
			// read before the barrier that followed the stores of v1, and v1
			// is next written after the barrier that follows those of v0)
			const int first = tile;
			for (;;) {
				const int64_t t0u = (int64_t)tile * NB;
				const int ka = (int)(u_beg > t0u ? u_beg - t0u : 0);
				const int kb = (int)(u_end < t0u + NB ? u_end - t0u : NB);
				pipeline(2 * ka, 2 * kb);
				float4 *dst = (float4 *)(skp + ((size_t)(2 * vpos + (tile == first ? 0 : 1)) * T + tid) * 16);
#pragma unroll
				for (int q = 0; q < 4; q++) dst[q] = make_float4(acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]);
				if (t0u + NB >= u_end) return;
				acc = zero;
				tile++;
				tile_mn(tile, ntiles, gm, mt, nt);
				m0 = mt * kTM;
				n0 = nt * TN;
			}
		} else {
			pipeline(0, NSt);
		}
	}
	q6g_epilogue(acc, m0, n0, wr, wt, li, kh, M, N, y, esc, bias, add);
}

// Sums of the stream-K pieces of tile blockIdx.x (q6k_gemm_kernel<128, true,
// true>: same threads, same slots), added in workgroup order, that is in
// order of K, and the GEMM's epilogue.
__global__ __launch_bounds__(512) void q6k_gemm_sk_fixup_kernel(const float *__restrict__ skp,
                                                                const float *__restrict__ esc,
                                                                const float *__restrict__ bias, float *__restrict__ y,
                                                                int M, int N, int NB, int G, int gm, int add) {
	constexpr int TN = 128, T = 4 * TN, RQ = TN / 32;
	const int mtiles = (M + kTM - 1) / kTM, ntiles = (N + TN - 1) / TN;
	const int tile = blockIdx.x;
	const int64_t U = (int64_t)mtiles * ntiles * NB;
	auto start = [&](int v) -> int64_t { return (int64_t)v * U / G; };
	const int64_t a = (int64_t)tile * NB, b = a + NB;
	int v = (int)(a * G / U);   // the workgroup holding unit a
	while (start(v + 1) <= a) v++;
	while (v > 0 && start(v) > a) v--;
	const int tid = threadIdx.x;
	v16f acc = {};
	for (; v < G && start(v) < b; v++) {
		const int64_t s0 = start(v), s1 = start(v + 1);
		if (s1 <= s0 || s1 <= a) continue;
		const int which = s0 / NB == tile ? 0 : 1;   // the tile is the workgroup's first or second
		const float4 *src = (const float4 *)(skp + ((size_t)(2 * v + which) * T + tid) * 16);
#pragma unroll
		for (int q = 0; q < 4; q++) {
			const float4 t = src[q];
			acc[4 * q] += t.x;
			acc[4 * q + 1] += t.y;
			acc[4 * q + 2] += t.z;
			acc[4 * q + 3] += t.w;
		}
	}
	int mt, nt;
	tile_mn(tile, ntiles, gm, mt, nt);
	const int lane = tid & 63, wave = tid >> 6;
	q6g_epilogue(acc, mt * kTM, nt * TN, wave % RQ, wave / RQ, lane & 31, lane >> 5, M, N, y, esc, bias, add);
}

// Split-K partials of the skinny matmuls (workspace slot 5).
int skinny_split_workspace(size_t floats, float **part) {
	*part = nullptr;
	if (!floats) return HAKO_GPU_OK;
	void *ws = nullptr;
	if (int rc = workspace(5, floats * 4, &ws)) return rc;
	*part = (float *)ws;
	return HAKO_GPU_OK;
}

// Token tiles per XCD group (tile_mn): the divisor of the token tiles that
// minimizes what one XCD reads, gm token tiles of act_tile bytes each plus
// its share of the row tiles of w_tile bytes each.
int gemm_gm(int M, int N, double act_tile, double w_tile, int tn = kTN) {
	const int mtiles = (M + kTM - 1) / kTM, ntiles = (N + tn - 1) / tn;
	const double per = (double)mtiles * ntiles / kXcds;
	int best = 1;
	double best_bytes = 1e300;
	for (int gm = 1; gm <= mtiles; gm++) {
		if (mtiles % gm) continue;
		const double rows = per / gm < 1.0 ? 1.0 : per / gm;
		const double bytes = gm * act_tile + rows * w_tile;
		if (bytes < best_bytes) {
			best_bytes = bytes;
			best = gm;
		}
	}
	return best;
}

int gemm_grid(int M, int N, int tn = kTN) {
	const int tiles = ((M + kTM - 1) / kTM) * ((N + tn - 1) / tn);
	return kXcds * ((tiles + kXcds - 1) / kXcds);
}

// Q4_K GEMM with K <= 3840: the resident-token-tile kernel (1) or the tiled
// one (0); a launch-shape knob
int g_q4_gemm_res = 1;
// Q6_K GEMM tile width: -1 by shape, else 64 or 128 rows (a launch-shape knob;
// the outputs do not depend on it)
int g_q6_gemm_tn = -1;
// Stream-K for 128-row tile counts below the workgroups of one round: in the
// decoder's prompt pass (1), there and in the standalone matmul entry points
// (2), or never (0). Measured on 512x3584x18944: inside the 7B prompt pass
// the stream-K kernel and its fixup took 243.8 + 7.0 us against 263.7 us for
// whole tiles (the pass 18.45 -> 18.12 ms); the same launch repeated back to
// back, the chip's power limit holding its clocks, 270 against 258 us (with
// a 3 ms pause before each launch 288 against 300 us).
int g_q6_gemm_sk = 1;

int check_gemm(const char *what, int m, int n_out, int n_in, size_t row_bytes, const void *w) {
	if (int rc = require_device()) return rc;
	if (m <= 0 || n_out <= 0 || n_in <= 0 || n_in % kQK != 0)
		return set_error(HAKO_GPU_EINVAL, "%s needs m, n_out > 0 and n_in %% 256 == 0 (got %d x %d x %d)", what,
		                 m, n_out, n_in);
	if (row_bytes * (size_t)n_out >= kBufNone || (size_t)m * n_in * 2 >= kBufNone)
		return set_error(HAKO_GPU_EINVAL, "%s operands exceed 2 GiB (%d x %d x %d)", what, m, n_out, n_in);
	if ((uintptr_t)w & 1) return set_error(HAKO_GPU_EINVAL, "%s needs a 2-byte aligned weight", what);
	return HAKO_GPU_OK;
}

}  // namespace

void q4k_gemm_set_res(int v) { g_q4_gemm_res = v ? 1 : 0; }
void q6k_gemm_set_tn(int v) { g_q6_gemm_tn = (v == 64 || v == 128) ? v : -1; }
void q6k_gemm_set_sk(int v) { g_q6_gemm_sk = v < 0 ? 0 : (v > 2 ? 2 : v); }

int q4k_gemm(float *y, const void *w, const int8_t *xq, const float *xs, const float *bias, int m, int n_out,
             int n_in) {
	if (int rc = check_gemm("Q4_K GEMM", m, n_out, n_in, (size_t)n_in / kQK * kQ4Bytes, w)) return rc;
	if (((uintptr_t)w & 15) || ((uintptr_t)xq & 15) || ((uintptr_t)xs & 3))
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMM needs w and xq 16-byte aligned");
	SkSegs segs{};
	segs.n = 1;
	segs.s[0] = {(const uint8_t *)w, bias, y, 0, n_out, n_out};
	if (m <= kSkMaxTokens) {   // a few tokens: the skinny kernel
		float *part = nullptr;
		const size_t pf = q4k_skinny_part_floats(n_in, n_out, kSkStore);
		if (int rc = skinny_split_workspace(pf, &part)) return rc;
		if (int rc = q4k_skinny(segs, kSkStore, xq, xs, m, n_in, n_out, part, pf)) return rc;
		return ok();
	}
	return q4k_gemm_segs(segs, kSkStore, xq, xs, m, n_in, n_out);
}

int q4k_gemm_segs(const SkSegs &segs, int epi, const int8_t *xq, const float *xs, int m, int n_in, int vrows) {
	if (m <= kSkMaxTokens || n_in % kQK || segs.n < 1 || segs.n > 3 || (epi == kSkSwiGLU && segs.n != 2))
		return set_error(HAKO_GPU_EINVAL, "Q4_K GEMM segments: m %d > %d, n_in %% 256 == 0, 1-3 segments", m,
		                 kSkMaxTokens);
	for (int i = 0; i < segs.n; i++) {
		const SkSeg &g = segs.s[i];
		if (int rc = check_gemm("Q4_K GEMM", m, g.rows, n_in, (size_t)n_in / kQK * kQ4Bytes, g.w)) return rc;
		if (((uintptr_t)g.w & 15) || ((uintptr_t)xq & 15) || ((uintptr_t)xs & 3))
			return set_error(HAKO_GPU_EINVAL, "Q4_K GEMM needs w and xq 16-byte aligned");
		const bool tiled = epi == kSkSwiGLU ? g.row0 == 0 && g.rows == segs.s[0].rows && g.rows % 32 == 0
		                                    : g.row0 % kTN == 0 && (i + 1 == segs.n || g.row0 + g.rows == segs.s[i + 1].row0);
		if (!tiled) return set_error(HAKO_GPU_EINVAL, "Q4_K GEMM segment %d does not fit the 64-row tiles", i);
	}
	const int N = epi == kSkSwiGLU ? 2 * segs.s[0].rows : vrows;
	if (g_q4_gemm_res && n_in <= kRMaxK) {
		const int mt = (m + kRT - 1) / kRT;
		const int R = cu_count() / mt > 1 ? cu_count() / mt : 1;
		const int units = epi == kSkSwiGLU ? (segs.s[0].rows + 15) / 16 : (vrows + 31) / 32;
		const int G = mt * R;
		const dim3 rgrid(kXcds * ((G + kXcds - 1) / kXcds)), rblock(kRWaves * kWave);
		const size_t lds = q4k_res_lds(n_in);
		switch (epi) {
		case kSkStore: hipLaunchKernelGGL(q4k_gemm_res_kernel<kSkStore>, rgrid, rblock, lds, stream(), segs, xq, xs, m, n_in, R, units); break;
		case kSkAdd: hipLaunchKernelGGL(q4k_gemm_res_kernel<kSkAdd>, rgrid, rblock, lds, stream(), segs, xq, xs, m, n_in, R, units); break;
		case kSkSwiGLU: hipLaunchKernelGGL(q4k_gemm_res_kernel<kSkSwiGLU>, rgrid, rblock, lds, stream(), segs, xq, xs, m, n_in, R, units); break;
		default: return set_error(HAKO_GPU_EINVAL, "Q4_K GEMM epilogue %d", epi);
		}
		HK_LAUNCHED("q4k_gemm_res");
		return ok();
	}
	const dim3 grid(gemm_grid(m, N));
	const int gm = gemm_gm(m, N, (double)kTM * (n_in + n_in / 32 * 4), (double)kTN * (n_in / kQK) * kQ4Bytes);
	switch (epi) {
	case kSkStore: hipLaunchKernelGGL(q4k_gemm_kernel<kSkStore>, grid, dim3(kGT), 0, stream(), segs, xq, xs, m, N, n_in, gm); break;
	case kSkAdd: hipLaunchKernelGGL(q4k_gemm_kernel<kSkAdd>, grid, dim3(kGT), 0, stream(), segs, xq, xs, m, N, n_in, gm); break;
	case kSkSwiGLU: hipLaunchKernelGGL(q4k_gemm_kernel<kSkSwiGLU>, grid, dim3(kGT), 0, stream(), segs, xq, xs, m, N, n_in, gm); break;
	default: return set_error(HAKO_GPU_EINVAL, "Q4_K GEMM epilogue %d", epi);
	}
	HK_LAUNCHED("q4k_gemm");
	return ok();
}

int f16_split(const float *x, _Float16 *xh, _Float16 *xl, float *esc, int m, int n) {
	hipLaunchKernelGGL(f16_split_kernel, dim3(m), dim3(kSplitT), 0, stream(), x, xh, xl, esc, n);
	HK_LAUNCHED("f16_split");
	return HAKO_GPU_OK;
}

int q6k_gemm(float *y, const void *w, const float *x, const float *bias, int m, int n_out, int n_in) {
	if (int rc = check_gemm("Q6_K GEMM", m, n_out, n_in, (size_t)n_in / kQK * kQ6Bytes, w)) return rc;
	if ((uintptr_t)x & 15) return set_error(HAKO_GPU_EINVAL, "Q6_K GEMM needs x 16-byte aligned");
	// workspace: fp16 hi and lo of x, one power of two per token
	const size_t half_bytes = (size_t)m * n_in * 2, esc_off = 2 * ((half_bytes + 255) & ~(size_t)255);
	void *ws = nullptr;
	if (int rc = workspace(3, esc_off + (size_t)m * 4, &ws)) return rc;
	_Float16 *xh = (_Float16 *)ws;
	_Float16 *xl = (_Float16 *)((uint8_t *)ws + esc_off / 2);
	float *esc = (float *)((uint8_t *)ws + esc_off);
	if (int rc = f16_split(x, xh, xl, esc, m, n_in)) return rc;
	if (m <= kSkMaxTokens) {   // a few tokens: the skinny kernel
		SkSegs segs{};
		segs.n = 1;
		segs.s[0] = {(const uint8_t *)w, bias, y, 0, n_out, n_out};
		float *part = nullptr;
		const size_t pf = q6k_skinny_part_floats(n_in, n_out, kSkStore);
		if (int rc = skinny_split_workspace(pf, &part)) return rc;
		if (int rc = q6k_skinny(segs, kSkStore, xh, xl, esc, m, n_in, n_out, part, pf)) return rc;
		return ok();
	}
	float *skp = nullptr;
	size_t skf = 0;
	if (g_q6_gemm_sk == 2) {   // stream-K slots (workspace slot 6)
		skf = q6k_gemm_sk_floats(q6k_gemm_sk_grid());
		void *p = nullptr;
		if (int rc = workspace(6, skf * 4, &p)) return rc;
		skp = (float *)p;
	}
	return q6k_gemm_split(y, w, xh, xl, esc, bias, m, n_out, n_in, false, skp, skf);
}

// The stream-K slots of a launch on G workgroups (floats).
size_t q6k_gemm_sk_floats(int G) { return (size_t)G * 2 * 512 * 16; }
int q6k_gemm_sk_grid() { return cu_count() / kXcds * kXcds; }

int q6k_gemm_split(float *y, const void *w, const _Float16 *xh, const _Float16 *xl, const float *esc,
                   const float *bias, int m, int n_out, int n_in, bool add, float *skp, size_t skp_floats) {
	if (int rc = check_gemm("Q6_K GEMM", m, n_out, n_in, (size_t)n_in / kQK * kQ6Bytes, w)) return rc;
	if (m <= kSkMaxTokens) return set_error(HAKO_GPU_EINVAL, "Q6_K GEMM on split rows needs m > %d", kSkMaxTokens);
	// 128-row tiles when they still give about one workgroup per CU
	const int wide_tiles = ((m + kTM - 1) / kTM) * ((n_out + 127) / 128);
	const bool wide = g_q6_gemm_tn == 128 || (g_q6_gemm_tn < 0 && 4 * wide_tiles >= 3 * cu_count());
	const int tn = wide ? 128 : kTN;
	const int gm = gemm_gm(m, n_out, (double)kTM * n_in * 4, (double)tn * (n_in / kQK) * kQ6Bytes, tn);
	// stream-K when the 128-row tiles leave CUs idle and the caller holds the slots
	const int G = q6k_gemm_sk_grid();
	const bool sk = wide && g_q6_gemm_sk && skp && skp_floats >= q6k_gemm_sk_floats(G) && wide_tiles < G &&
	                n_in / kQK >= 2;
	if (sk) {
		hipLaunchKernelGGL((q6k_gemm_kernel<128, true, true>), dim3(G), dim3(4 * 128), 2 * q6g_buf_bytes(128), stream(),
		                   (const uint8_t *)w, xh, xl, esc, bias, y, m, n_out, n_in, add ? 1 : 0, gm, skp);
		HK_LAUNCHED("q6k_gemm");
		hipLaunchKernelGGL(q6k_gemm_sk_fixup_kernel, dim3(wide_tiles), dim3(512), 0, stream(), skp, esc, bias, y, m,
		                   n_out, n_in / kQK, G, gm, add ? 1 : 0);
		HK_LAUNCHED("q6k_gemm_sk_fixup");
		return ok();
	}
	if (wide)
		hipLaunchKernelGGL((q6k_gemm_kernel<128, true>), dim3(gemm_grid(m, n_out, 128)), dim3(4 * 128),
		                   2 * q6g_buf_bytes(128), stream(), (const uint8_t *)w, xh, xl, esc, bias, y, m, n_out, n_in,
		                   add ? 1 : 0, gm, nullptr);
	else
		hipLaunchKernelGGL((q6k_gemm_kernel<kTN, false>), dim3(gemm_grid(m, n_out)), dim3(4 * kTN), q6g_buf_bytes(kTN),
		                   stream(), (const uint8_t *)w, xh, xl, esc, bias, y, m, n_out, n_in, add ? 1 : 0, gm, nullptr);
	HK_LAUNCHED("q6k_gemm");
	return ok();
}

}  // namespace hako

extern "C" int hako_gpu_q4k_gemm(float *y, const void *w, const int8_t *xq, const float *xs, const float *bias,
                                 int m, int n_out, int n_in) {
	return hako::q4k_gemm(y, w, xq, xs, bias, m, n_out, n_in);
}

extern "C" int hako_gpu_q6k_gemm(float *y, const void *w, const float *x, const float *bias, int m, int n_out,
                                 int n_in) {
	return hako::q6k_gemm(y, w, x, bias, m, n_out, n_in);
}

extern "C" int hako_gpu_matmul_batch(float *y, const float *x, int type, const void *w, const float *bias, int m,
                                     int n_out, int n_in) {
	using namespace hako;
	if (int rc = require_device()) return rc;
	if (m <= 0) return set_error(HAKO_GPU_EINVAL, "matmul_batch needs m > 0 (got %d)", m);
	if (m == 1) return hako_gpu_matmul(y, x, type, w, bias, n_out, n_in);
	switch (type) {
	case HAKO_TYPE_Q4_K: {
		if (int rc = check_gemm("Q4_K GEMM", m, n_out, n_in, (size_t)n_in / kQK * kQ4Bytes, w)) return rc;
		const size_t qbytes = ((size_t)m * n_in + 255) & ~(size_t)255;
		void *ws = nullptr;
		if (int rc = workspace(4, qbytes + (size_t)m * (n_in / 32) * 4, &ws)) return rc;
		int8_t *xq = (int8_t *)ws;
		float *xs = (float *)((uint8_t *)ws + qbytes);
		if (int rc = hako_gpu_quantize_q8_32(x, m, n_in, xq, xs)) return rc;
		return q4k_gemm(y, w, xq, xs, bias, m, n_out, n_in);
	}
	case HAKO_TYPE_Q6_K:
		return q6k_gemm(y, w, x, bias, m, n_out, n_in);
	case HAKO_TYPE_F32:
	case HAKO_TYPE_F16:
		for (int t = 0; t < m; t++)
			if (int rc = hako_gpu_dense_gemv(y + (size_t)t * n_out, type, w, x + (size_t)t * n_in, bias, n_out, n_in))
				return rc;
		return ok();
	default:
		return set_error(HAKO_GPU_ETYPE, "unsupported tensor type %d", type);
	}
}
