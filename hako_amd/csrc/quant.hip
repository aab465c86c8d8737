// quant.hip — q8_32 activation quantizer, k-quant dequantizers, the dense
// F32/F16 GEMV and the matmul dispatch of the hako_gpu C ABI.
#include "hako_dev.h"
#include "hako_rt.h"
#include "dequant_dev.h"

namespace hako {

int q4k_matmul_fused(float *out, const float *x, const void *w, const float *bias, int n_out, int n_in);

namespace {

// quantize_row_q8_32 over rows*n floats: thread t owns elements 4t..4t+3,
// 8 consecutive lanes one 32-block (blocks never straddle rows: n % 32 == 0).
__global__ __launch_bounds__(256) void q8_kernel(const float *__restrict__ x, int8_t *__restrict__ xq,
                                                 float *__restrict__ xs, int64_t quads) {
	for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < quads;
	     t += (int64_t)gridDim.x * blockDim.x) {
		const float4 v = *(const float4 *)(x + 4 * t);
		float sc;
		const uint32_t packed = q8_quant4(v, sc);
		*(uint32_t *)(xq + 4 * t) = packed;
		if ((t & 7) == 0) xs[t >> 3] = sc;
	}
}

// dequant_q4_K / dequant_q6_K over `chunks` chunks of 32 weights.
__global__ __launch_bounds__(256) void dq4_kernel(const uint8_t *__restrict__ w, float *__restrict__ y,
                                                  int64_t chunks) {
	for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks;
	     c += (int64_t)gridDim.x * blockDim.x)
		dq4_chunk(w, c, y);
}

__global__ __launch_bounds__(256) void dq6_kernel(const uint8_t *__restrict__ w, float *__restrict__ y,
                                                  int64_t chunks) {
	for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < chunks;
	     c += (int64_t)gridDim.x * blockDim.x)
		dq6_chunk(w, c, y);
}

__global__ __launch_bounds__(256) void dqf16_kernel(const uint16_t *__restrict__ h, float *__restrict__ y,
                                                    int64_t n) {
	for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n;
	     t += (int64_t)gridDim.x * blockDim.x)
		y[t] = f16_to_f32(h[t]);
}

// F32 / F16 weight rows (the reference's generic path, nn.c:84-95, for the
// non-k-quant types): one wave per row, lanes strided over the columns.
template <bool F16>
__global__ __launch_bounds__(256) void dense_gemv_kernel(const void *__restrict__ w,
                                                         const float *__restrict__ x,
                                                         const float *__restrict__ bias,
                                                         float *__restrict__ out, int n_out, int n_in) {
	const int lane = threadIdx.x & 63;
	const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
	if (row >= n_out) return;
	float acc = 0.0f;
	if (F16) {
		const uint16_t *wr = (const uint16_t *)w + (size_t)row * n_in;
		for (int c = lane; c < n_in; c += 64) acc = __builtin_fmaf(f16_to_f32(wr[c]), x[c], acc);
	} else {
		const float *wr = (const float *)w + (size_t)row * n_in;
		for (int c = lane; c < n_in; c += 64) acc = __builtin_fmaf(wr[c], x[c], acc);
	}
	acc = wave_sum(acc);
	if (lane == 0) out[row] = bias ? acc + bias[row] : acc;
}

int grid_for(int64_t items) {
	int64_t g = (items + 255) / 256;
	if (g > 65536) g = 65536;
	return (int)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace hako

using namespace hako;

extern "C" {

int hako_gpu_quantize_q8_32(const float *x, int64_t rows, int n, int8_t *xq, float *xs) {
	if (int rc = require_device()) return rc;
	if (rows < 0 || n < 0 || n % 32 != 0)
		return set_error(HAKO_GPU_EINVAL, "quantize_q8_32 needs n %% 32 == 0 (got %d)", n);
	if (((uintptr_t)x & 15) || ((uintptr_t)xq & 3) || ((uintptr_t)xs & 3))
		return set_error(HAKO_GPU_EINVAL, "quantize_q8_32 needs x 16-byte and xq/xs 4-byte aligned");
	const int64_t quads = rows * (int64_t)n / 4;
	if (quads == 0) return ok();
	hipLaunchKernelGGL(q8_kernel, dim3(grid_for(quads)), dim3(256), 0, stream(), x, xq, xs, quads);
	HK_LAUNCHED("q8");
	return ok();
}

int hako_gpu_dequant(int type, const void *src, float *out, int64_t nelem) {
	if (int rc = require_device()) return rc;
	if (nelem < 0) return set_error(HAKO_GPU_EINVAL, "nelem %lld", (long long)nelem);
	if (nelem == 0) return ok();
	switch (type) {
	case HAKO_TYPE_F32:
		HK_HIP(hipMemcpyAsync(out, src, (size_t)nelem * 4, hipMemcpyDeviceToDevice, stream()));
		return ok();
	case HAKO_TYPE_F16:
		if ((uintptr_t)src & 1) return set_error(HAKO_GPU_EINVAL, "F16 source must be 2-byte aligned");
		hipLaunchKernelGGL(dqf16_kernel, dim3(grid_for(nelem)), dim3(256), 0, stream(),
		                   (const uint16_t *)src, out, nelem);
		HK_LAUNCHED("dqf16");
		return ok();
	case HAKO_TYPE_Q4_K:
		if (nelem % kQK) return set_error(HAKO_GPU_EINVAL, "Q4_K nelem %% 256 != 0");
		if (((uintptr_t)src & 15) || ((uintptr_t)out & 15))
			return set_error(HAKO_GPU_EINVAL, "Q4_K dequant needs 16-byte aligned src and out");
		hipLaunchKernelGGL(dq4_kernel, dim3(grid_for(nelem / 32)), dim3(256), 0, stream(),
		                   (const uint8_t *)src, out, nelem / 32);
		HK_LAUNCHED("dq4");
		return ok();
	case HAKO_TYPE_Q6_K:
		if (nelem % kQK) return set_error(HAKO_GPU_EINVAL, "Q6_K nelem %% 256 != 0");
		if (((uintptr_t)src & 1) || ((uintptr_t)out & 15))
			return set_error(HAKO_GPU_EINVAL, "Q6_K dequant needs 2-byte aligned src, 16-byte aligned out");
		hipLaunchKernelGGL(dq6_kernel, dim3(grid_for(nelem / 32)), dim3(256), 0, stream(),
		                   (const uint8_t *)src, out, nelem / 32);
		HK_LAUNCHED("dq6");
		return ok();
	default:
		return set_error(HAKO_GPU_ETYPE, "unsupported tensor type %d", type);
	}
}

int hako_gpu_dense_gemv(float *out, int type, const void *w, const float *x, const float *bias,
                        int n_out, int n_in) {
	if (int rc = require_device()) return rc;
	if (n_out <= 0 || n_in <= 0) return set_error(HAKO_GPU_EINVAL, "dense GEMV %d x %d", n_out, n_in);
	const int wgs = (n_out + 3) / 4;
	if (type == HAKO_TYPE_F32) {
		hipLaunchKernelGGL((dense_gemv_kernel<false>), dim3(wgs), dim3(256), 0, stream(), w, x, bias, out,
		                   n_out, n_in);
	} else if (type == HAKO_TYPE_F16) {
		hipLaunchKernelGGL((dense_gemv_kernel<true>), dim3(wgs), dim3(256), 0, stream(), w, x, bias, out,
		                   n_out, n_in);
	} else {
		return set_error(HAKO_GPU_ETYPE, "dense GEMV type %d", type);
	}
	HK_LAUNCHED("dense_gemv");
	return ok();
}

int hako_gpu_matmul(float *out, const float *x, int type, const void *w, const float *bias, int n_out,
                    int n_in) {
	if (int rc = require_device()) return rc;
	switch (type) {
	case HAKO_TYPE_Q4_K:
		if (((uintptr_t)w & 15) || ((uintptr_t)x & 15))
			return set_error(HAKO_GPU_EINVAL, "Q4_K matmul needs 16-byte aligned w and x");
		return q4k_matmul_fused(out, x, w, bias, n_out, n_in);
	case HAKO_TYPE_Q6_K:
		return hako_gpu_q6k_gemv(out, w, x, bias, n_out, n_in);
	case HAKO_TYPE_F32:
	case HAKO_TYPE_F16:
		return hako_gpu_dense_gemv(out, type, w, x, bias, n_out, n_in);
	default:
		return set_error(HAKO_GPU_ETYPE, "unsupported tensor type %d", type);
	}
}

int hako_gpu_matmul_host(float *out, const float *x, int type, const void *w_host, const float *bias_host,
                         int n_out, int n_in) {
	if (int rc = require_device()) return rc;
	if (n_out <= 0 || n_in <= 0) return set_error(HAKO_GPU_EINVAL, "matmul %d x %d", n_out, n_in);
	const void *w = hako_gpu_mirror_lookup(w_host);
	if (!w) return set_error(HAKO_GPU_ENOTFOUND, "weight %p is not inside an uploaded mirror", w_host);
	void *xd, *od, *bd = nullptr;
	if (int rc = workspace(0, (size_t)n_in * 4, &xd)) return rc;
	if (int rc = workspace(1, (size_t)n_out * 4, &od)) return rc;
	const float *bias = nullptr;
	if (bias_host) {
		bias = (const float *)hako_gpu_mirror_lookup(bias_host);
		if (!bias) {
			if (int rc = workspace(2, (size_t)n_out * 4, &bd)) return rc;
			HK_HIP(hipMemcpyAsync(bd, bias_host, (size_t)n_out * 4, hipMemcpyHostToDevice, stream()));
			bias = (const float *)bd;
		}
	}
	HK_HIP(hipMemcpyAsync(xd, x, (size_t)n_in * 4, hipMemcpyHostToDevice, stream()));
	if (int rc = hako_gpu_matmul((float *)od, (const float *)xd, type, w, bias, n_out, n_in)) return rc;
	HK_HIP(hipMemcpyAsync(out, od, (size_t)n_out * 4, hipMemcpyDeviceToHost, stream()));
	HK_HIP(hipStreamSynchronize(stream()));
	return ok();
}

}  // extern "C"
