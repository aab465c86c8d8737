// noalloc.hip — hako_gpu_matmul_batch_noalloc: the multi-token matmul of
// hako_gpu_matmul_batch with no device allocation, for callers that cannot
// allocate (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).
//
// Its scratch (the q8_32 rows and scales of a Q4_K activation, the fp16 hi/lo
// rows of a Q6_K activation, the split-K partial sums of a skinny launch)
// lives in one file-scope device array of kScratchBytes. Each device the
// library runs on holds its own copy of the array at its own address until
// the process ends; hako_gpu_init looks that address up once per device
// (noalloc_setup) and every call passes it, never the array's name, to the
// kernels. Nothing here needs zeroed scratch: every byte a call reads was
// written earlier in the same call.
//
// Calls on one device share the array and keep the last call's contents:
// calls that overlap in time on one device (several streams, or graphs
// replayed concurrently) race on it. The library stream serializes the calls
// it makes itself.
#include <mutex>

#include "hako_dev.h"
#include "hako_rt.h"
#include "skinny.h"

namespace hako {
namespace {

// 7B-prompt shapes fit: 512 tokens x 18944 inputs as fp16 hi + lo (38.8 MB),
// or as q8_32 rows (10.9 MB), plus the partials of a 16-token split.
constexpr size_t kScratchBytes = (size_t)48 << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
void *g_scratch[kMaxDevices];   // device address of `scratch`, per device

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

// Device address of this device's copy of the scratch array, looked up once
// (hako_gpu_init calls it with the device current).
int noalloc_setup(int device) {
	if (device < 0 || device >= kMaxDevices)
		return set_error(HAKO_GPU_ENODEV, "device %d beyond the %d the scratch table holds", device, kMaxDevices);
	std::lock_guard<std::mutex> lk(g_mu);
	if (g_scratch[device]) return HAKO_GPU_OK;
	void *p = nullptr;
	const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
	if (e != hipSuccess || !p) {
		(void)hipGetLastError();
		return set_error(HAKO_GPU_EHIP, "hipGetSymbolAddress of the no-allocation scratch: %s",
		                 hipGetErrorString(e));
	}
	g_scratch[device] = p;
	return HAKO_GPU_OK;
}

}  // namespace hako

extern "C" int hako_gpu_matmul_batch_noalloc(float *y, const float *x, int type, const void *w, const float *bias,
                                             int m, int n_out, int n_in) {
	using namespace hako;
	if (int rc = require_device()) return rc;
	int dev = -1;
	HK_HIP(hipGetDevice(&dev));
	uint8_t *base = nullptr;
	{
		std::lock_guard<std::mutex> lk(g_mu);
		if (dev >= 0 && dev < kMaxDevices) base = (uint8_t *)g_scratch[dev];
	}
	if (!base) return set_error(HAKO_GPU_ENODEV, "no-allocation scratch of device %d is not set up", dev);
	if (m <= 0 || n_out <= 0 || n_in <= 0)
		return set_error(HAKO_GPU_EINVAL, "matmul_batch_noalloc needs m, n_out, n_in > 0 (got %d x %d x %d)", m,
		                 n_out, n_in);
	if (m == 1) return hako_gpu_matmul(y, x, type, w, bias, n_out, n_in);   // one launch, no scratch
	if (type == HAKO_TYPE_F32 || type == HAKO_TYPE_F16) {
		for (int t = 0; t < m; t++)
			if (int rc = hako_gpu_dense_gemv(y + (size_t)t * n_out, type, w, x + (size_t)t * n_in, bias, n_out, n_in))
				return rc;
		return ok();
	}
	if (type != HAKO_TYPE_Q4_K && type != HAKO_TYPE_Q6_K) return set_error(HAKO_GPU_ETYPE, "unsupported tensor type %d", type);
	if (n_in % kQK) return set_error(HAKO_GPU_EINVAL, "matmul_batch_noalloc needs n_in %% 256 == 0 (got %d)", n_in);
	const size_t rb = (size_t)n_in / kQK * (type == HAKO_TYPE_Q4_K ? kQ4Bytes : kQ6Bytes);
	if (rb * (size_t)n_out >= kBufNone || (size_t)m * n_in * 2 >= kBufNone)
		return set_error(HAKO_GPU_EINVAL, "matmul_batch_noalloc operands exceed 2 GiB (%d x %d x %d)", m, n_out, n_in);
	if (((uintptr_t)x & 15) || ((uintptr_t)w & (type == HAKO_TYPE_Q4_K ? 15 : 1)))
		return set_error(HAKO_GPU_EINVAL, "matmul_batch_noalloc needs x 16-byte and w %d-byte aligned",
		                 type == HAKO_TYPE_Q4_K ? 16 : 2);
	const bool skinny = m <= kSkMaxTokens;
	// scratch layout: the activation section, then the split partials
	const size_t act = type == HAKO_TYPE_Q4_K
	                       ? align256((size_t)m * n_in) + align256((size_t)m * (n_in / 32) * 4)
	                       : 2 * align256((size_t)m * n_in * 2) + align256((size_t)m * 4);
	const size_t pf = !skinny ? 0
	                  : type == HAKO_TYPE_Q4_K ? q4k_skinny_part_floats(n_in, n_out, kSkStore)
	                                           : q6k_skinny_part_floats(n_in, n_out, kSkStore);
	const size_t need = act + pf * 4;
	if (need > kScratchBytes)
		return set_error(HAKO_GPU_EINVAL,
		                 "matmul_batch_noalloc of %d x %d x %d needs %zu bytes of scratch; it has %zu (use "
		                 "hako_gpu_matmul_batch, or fewer tokens per call)",
		                 m, n_out, n_in, need, kScratchBytes);
	float *part = pf ? (float *)(base + act) : nullptr;
	SkSegs segs{};
	segs.n = 1;
	segs.s[0] = {(const uint8_t *)w, bias, y, 0, n_out, n_out};
	if (type == HAKO_TYPE_Q4_K) {
		int8_t *xq = (int8_t *)base;
		float *xs = (float *)(base + align256((size_t)m * n_in));
		if (int rc = hako_gpu_quantize_q8_32(x, m, n_in, xq, xs)) return rc;
		if (skinny) {
			if (int rc = q4k_skinny(segs, kSkStore, xq, xs, m, n_in, n_out, part, pf)) return rc;
		} else if (int rc = q4k_gemm_segs(segs, kSkStore, xq, xs, m, n_in, n_out)) {
			return rc;
		}
		return ok();
	}
	const size_t half = align256((size_t)m * n_in * 2);
	_Float16 *xh = (_Float16 *)base;
	_Float16 *xl = (_Float16 *)(base + half);
	float *esc = (float *)(base + 2 * half);
	if (int rc = f16_split(x, xh, xl, esc, m, n_in)) return rc;
	if (skinny) {
		if (int rc = q6k_skinny(segs, kSkStore, xh, xl, esc, m, n_in, n_out, part, pf)) return rc;
	} else if (int rc = q6k_gemm_split(y, w, xh, xl, esc, bias, m, n_out, n_in, false)) {
		return rc;
	}
	return ok();
}
