// runtime.hip — device selection, the library stream, memory, events, the
// verbatim-upload mirrors and error reporting of the hako_gpu C ABI.
#include <hip/hip_runtime.h>

#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <vector>

#include "hako_rt.h"

namespace hako {
namespace {

thread_local char g_err[512] = "";

// Plain streaming copy, 16 bytes per lane per step (also the known-size
// kernel that calibrates the HBM byte counters).
__global__ __launch_bounds__(256) void copy16_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                     int64_t n16) {
	for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
	     i += (int64_t)gridDim.x * blockDim.x)
		dst[i] = src[i];
}

// The device's constant-rate wall clock (s_memrealtime) at the moment the
// kernel runs, stored through a vector store by one lane: a timing mark that
// can sit inside a captured graph, where events cannot be timed.
__global__ __launch_bounds__(64) void stamp_kernel(unsigned long long *dst) {
	const unsigned long long t = wall_clock64();
	if (threadIdx.x == 0) dst[threadIdx.x] = t;
}

struct Mirror {
	const uint8_t *host;
	size_t bytes;
	uint8_t *dev;
};

struct State {
	std::mutex mu;
	int device = -1;
	hipStream_t stream = nullptr;
	hipDeviceProp_t prop{};
	std::vector<Mirror> mirrors;
	void *ws[8] = {};
	size_t ws_bytes[8] = {};
	// workspaces outgrown by a later call: a graph captured earlier may still
	// address them, so they live until hako_gpu_shutdown
	std::vector<void *> ws_retired;
};

State &st() {
	static State s;
	return s;
}

}  // namespace

int set_error(int code, const char *fmt, ...) {
	va_list ap;
	va_start(ap, fmt);
	vsnprintf(g_err, sizeof g_err, fmt, ap);
	va_end(ap);
	return code;
}

int ok() {
	g_err[0] = '\0';
	return HAKO_GPU_OK;
}

int hip_fail(hipError_t e, const char *what, const char *file, int line) {
	return set_error(HAKO_GPU_EHIP, "%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
}

hipStream_t stream() { return st().stream; }

int cu_count() {
	const int n = st().prop.multiProcessorCount;
	return n > 0 ? n : 256;
}

int require_device() {
	if (st().device < 0) return set_error(HAKO_GPU_ENODEV, "hako_gpu_init has not been called");
	return HAKO_GPU_OK;
}

int workspace(int slot, size_t bytes, void **ptr) {
	State &s = st();
	if (slot < 0 || slot >= 8) return set_error(HAKO_GPU_EINVAL, "workspace slot %d", slot);
	if (s.ws_bytes[slot] < bytes) {
		// Grow by at least half again, so the retired buffers of a slot stay
		// below twice its size.
		size_t want = bytes < 4096 ? 4096 : bytes;
		if (want < s.ws_bytes[slot] + s.ws_bytes[slot] / 2) want = s.ws_bytes[slot] + s.ws_bytes[slot] / 2;
		void *p = nullptr;
		if (hipMalloc(&p, want) != hipSuccess) {
			(void)hipGetLastError();
			return set_error(HAKO_GPU_ENOMEM, "workspace of %zu bytes", want);
		}
		// The old buffer is retired, not freed: the stream, or a graph
		// captured around an earlier call, may still address it.
		if (s.ws[slot]) s.ws_retired.push_back(s.ws[slot]);
		s.ws[slot] = p;
		s.ws_bytes[slot] = want;
	}
	*ptr = s.ws[slot];
	return HAKO_GPU_OK;
}

}  // namespace hako

using namespace hako;

extern "C" {

int hako_gpu_init(int device) {
	State &s = st();
	std::lock_guard<std::mutex> lk(s.mu);
	if (s.device == device) return ok();
	if (s.device >= 0) return set_error(HAKO_GPU_EINVAL, "already initialised on device %d", s.device);
	int n = 0;
	if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
		(void)hipGetLastError();
		return set_error(HAKO_GPU_ENODEV, "no HIP device visible");
	}
	if (device < 0 || device >= n) return set_error(HAKO_GPU_ENODEV, "device %d of %d", device, n);
	HK_HIP(hipSetDevice(device));
	HK_HIP(hipGetDeviceProperties(&s.prop, device));
	if (strncmp(s.prop.gcnArchName, "gfx950", 6) != 0)
		return set_error(HAKO_GPU_ENODEV, "device %d is %s; this library is built for gfx950",
		                 device, s.prop.gcnArchName);
	if (int rc = noalloc_setup(device)) return rc;
	HK_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
	s.device = device;
	return ok();
}

int hako_gpu_shutdown(void) {
	State &s = st();
	std::lock_guard<std::mutex> lk(s.mu);
	if (s.device < 0) return ok();
	HK_HIP(hipStreamSynchronize(s.stream));
	for (auto &m : s.mirrors) HK_HIP(hipFree(m.dev));
	s.mirrors.clear();
	for (int i = 0; i < 8; i++) {
		if (s.ws[i]) HK_HIP(hipFree(s.ws[i]));
		s.ws[i] = nullptr;
		s.ws_bytes[i] = 0;
	}
	for (void *p : s.ws_retired) HK_HIP(hipFree(p));
	s.ws_retired.clear();
	HK_HIP(hipStreamDestroy(s.stream));
	s.stream = nullptr;
	s.device = -1;
	return ok();
}

const char *hako_gpu_last_error(void) { return g_err; }

int hako_gpu_tune(int knob, int value) {
	switch (knob) {
	case HAKO_TUNE_Q4K_WGS_PER_CU: q4k_set_wgs_per_cu(value); return ok();
	case HAKO_TUNE_Q6K_WGS_PER_CU: q6k_set_wgs_per_cu(value); return ok();
	case HAKO_TUNE_Q4K_WAVES: q4k_set_waves(value); return ok();
	case HAKO_TUNE_Q6K_WAVES: q6k_set_waves(value); return ok();
	case HAKO_TUNE_Q6K_FLAT_ITEMS: q6k_set_flat_items(value); return ok();
	case HAKO_TUNE_Q6K_FLAT_SEG: q6k_set_flat_seg(value); return ok();
	case HAKO_TUNE_Q6K_ROWS: q6k_set_rows(value); return ok();
	case HAKO_TUNE_Q4K_FLAT_ITEMS: q4k_set_flat_items(value); return ok();
	case HAKO_TUNE_Q4K_GEMM_RES: q4k_gemm_set_res(value); return ok();
	case HAKO_TUNE_Q6K_GEMM_TN: q6k_gemm_set_tn(value); return ok();
	case HAKO_TUNE_Q6K_DIGITS: q6k_set_dig(value); return ok();
	case HAKO_TUNE_Q6K_GEMM_SK: q6k_gemm_set_sk(value); return ok();
	case HAKO_TUNE_SKINNY_Q4K_WGS: q4k_skinny_set_target_wgs(value); return ok();
	case HAKO_TUNE_SKINNY_Q6K_WGS: q6k_skinny_set_target_wgs(value); return ok();
	case HAKO_TUNE_DEC_GU_ITEMS: dec_set_gu_items(value); return ok();
	case HAKO_TUNE_DEC_GU_GRID: dec_set_gu_grid(value); return ok();
	case HAKO_TUNE_DEC_MERGE_ROWS: dec_set_merge_rows(value); return ok();
	case HAKO_TUNE_DEC_QKV_ITEMS: dec_set_qkv_items(value); return ok();
	case HAKO_TUNE_DEC_ATTN_PARTS: dec_set_attn_parts(value); return ok();
	default: return set_error(HAKO_GPU_EINVAL, "unknown tuning knob %d", knob);
	}
}

int hako_gpu_device_info(hako_gpu_info *out) {
	if (int rc = require_device()) return rc;
	const hipDeviceProp_t &p = st().prop;
	memset(out, 0, sizeof *out);
	snprintf(out->name, sizeof out->name, "%s", p.gcnArchName);
	out->compute_units = p.multiProcessorCount;
	out->clock_khz = p.clockRate;
	out->hbm_bytes = p.totalGlobalMem;
	out->l2_bytes = p.l2CacheSize;
	out->lds_bytes_per_cu = (int)p.maxSharedMemoryPerMultiProcessor;
	return ok();
}

int hako_gpu_malloc(void **dptr, size_t bytes) {
	if (int rc = require_device()) return rc;
	if (!dptr) return set_error(HAKO_GPU_EINVAL, "null output pointer");
	if (hipMalloc(dptr, bytes ? bytes : 1) != hipSuccess) {
		(void)hipGetLastError();
		*dptr = nullptr;
		return set_error(HAKO_GPU_ENOMEM, "hipMalloc of %zu bytes", bytes);
	}
	return ok();
}

int hako_gpu_free(void *dptr) {
	if (int rc = require_device()) return rc;
	if (dptr) HK_HIP(hipFree(dptr));
	return ok();
}

int hako_gpu_memcpy_h2d(void *dst, const void *src, size_t bytes) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st().stream));
	HK_HIP(hipStreamSynchronize(st().stream));
	return ok();
}

int hako_gpu_memcpy_d2h(void *dst, const void *src, size_t bytes) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st().stream));
	HK_HIP(hipStreamSynchronize(st().stream));
	return ok();
}

int hako_gpu_memcpy_d2d(void *dst, const void *src, size_t bytes) {
	if (int rc = require_device()) return rc;
	if (bytes == 0) return ok();
	if ((((uintptr_t)dst | (uintptr_t)src | bytes) & 15) == 0) {
		const int64_t n16 = (int64_t)(bytes / 16);
		int64_t grid = (n16 + 255) / 256;
		if (grid > 8192) grid = 8192;
		hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)grid), dim3(256), 0, st().stream,
		                   (const uint4 *)src, (uint4 *)dst, n16);
		HK_LAUNCHED("copy16");
		return ok();
	}
	HK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st().stream));
	return ok();
}

int hako_gpu_sync(void) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipStreamSynchronize(st().stream));
	return ok();
}

void *hako_gpu_stream(void) { return (void *)st().stream; }

int hako_gpu_event_create(void **ev) {
	if (int rc = require_device()) return rc;
	hipEvent_t e;
	HK_HIP(hipEventCreate(&e));
	*ev = (void *)e;
	return ok();
}

int hako_gpu_event_record(void *ev) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipEventRecord((hipEvent_t)ev, st().stream));
	return ok();
}

int hako_gpu_event_elapsed_ms(void *start, void *stop, float *ms) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipEventSynchronize((hipEvent_t)stop));
	HK_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
	return ok();
}

int hako_gpu_event_destroy(void *ev) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipEventDestroy((hipEvent_t)ev));
	return ok();
}

int hako_gpu_timestamp(void *dst) {
	if (int rc = require_device()) return rc;
	if (!dst || ((uintptr_t)dst & 7)) return set_error(HAKO_GPU_EINVAL, "timestamp needs an 8-byte aligned address");
	hipLaunchKernelGGL(stamp_kernel, dim3(1), dim3(64), 0, st().stream, (unsigned long long *)dst);
	HK_LAUNCHED("stamp");
	return ok();
}

int hako_gpu_timestamp_hz(double *hz) {
	if (int rc = require_device()) return rc;
	int khz = 0;
	HK_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, st().device));
	if (khz <= 0) return set_error(HAKO_GPU_EINVAL, "device reports no wall-clock rate");
	*hz = 1e3 * khz;
	return ok();
}

int hako_gpu_capture_begin(void) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipStreamBeginCapture(st().stream, hipStreamCaptureModeThreadLocal));
	return ok();
}

int hako_gpu_capture_end(void **graph) {
	if (int rc = require_device()) return rc;
	hipGraph_t g = nullptr;
	HK_HIP(hipStreamEndCapture(st().stream, &g));
	hipGraphExec_t ge = nullptr;
	hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
	(void)hipGraphDestroy(g);
	if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
	*graph = (void *)ge;
	return ok();
}

int hako_gpu_graph_launch(void *graph) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipGraphLaunch((hipGraphExec_t)graph, st().stream));
	return ok();
}

int hako_gpu_graph_destroy(void *graph) {
	if (int rc = require_device()) return rc;
	HK_HIP(hipGraphExecDestroy((hipGraphExec_t)graph));
	return ok();
}

int hako_gpu_mirror_upload(const void *host, size_t bytes, void **dev) {
	if (int rc = require_device()) return rc;
	State &s = st();
	std::lock_guard<std::mutex> lk(s.mu);
	const uint8_t *h = (const uint8_t *)host;
	// An overlap is refused, never reused: the older mirror may hold memory
	// that was freed or unmapped since, now holding other bytes.
	for (auto &m : s.mirrors)
		if (h < m.host + m.bytes && m.host < h + bytes)
			return set_error(HAKO_GPU_EINVAL,
			                 "host range [%p, +%zu) overlaps the mirror of [%p, +%zu): release that mirror first "
			                 "(host memory freed or unmapped while mirrored leaves its mirror in place)",
			                 (const void *)h, bytes, (const void *)m.host, m.bytes);
	Mirror m{h, bytes, nullptr};
	if (hipMalloc((void **)&m.dev, bytes ? bytes : 1) != hipSuccess) {
		(void)hipGetLastError();
		return set_error(HAKO_GPU_ENOMEM, "mirror of %zu bytes", bytes);
	}
	hipError_t e = hipMemcpyAsync(m.dev, host, bytes, hipMemcpyHostToDevice, s.stream);
	if (e == hipSuccess) e = hipStreamSynchronize(s.stream);
	if (e != hipSuccess) {
		(void)hipFree(m.dev);
		return hip_fail(e, "mirror upload", __FILE__, __LINE__);
	}
	s.mirrors.push_back(m);
	if (dev) *dev = m.dev;
	return ok();
}

int hako_gpu_mirror_release(const void *host) {
	if (int rc = require_device()) return rc;
	State &s = st();
	std::lock_guard<std::mutex> lk(s.mu);
	for (size_t i = 0; i < s.mirrors.size(); i++) {
		if (s.mirrors[i].host == (const uint8_t *)host) {
			HK_HIP(hipStreamSynchronize(s.stream));
			HK_HIP(hipFree(s.mirrors[i].dev));
			s.mirrors.erase(s.mirrors.begin() + (long)i);
			return ok();
		}
	}
	return set_error(HAKO_GPU_ENOTFOUND, "no mirror starts at %p", host);
}

void *hako_gpu_mirror_lookup(const void *p) {
	State &s = st();
	std::lock_guard<std::mutex> lk(s.mu);
	const uint8_t *h = (const uint8_t *)p;
	for (auto &m : s.mirrors)
		if (h >= m.host && h < m.host + m.bytes) return m.dev + (h - m.host);
	return nullptr;
}

}  // extern "C"
