// hako_rt.h — host-side internals shared by the library's translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/hako_gpu.h"

namespace hako {

// Record `msg` (printf-style) as this thread's last error; returns `code`.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
// Clear the thread's last error; returns HAKO_GPU_OK.
int ok();
// Map a failed HIP call to HAKO_GPU_EHIP with its text.
int hip_fail(hipError_t e, const char *what, const char *file, int line);

// The library stream, or nullptr before hako_gpu_init.
hipStream_t stream();
// HAKO_GPU_OK when a device is initialised, otherwise an ENODEV error.
int require_device();
// Compute units of the initialised device.
int cu_count();
// Workgroups per CU of the persistent GEMV grids (tuning; default 1).
void q4k_set_wgs_per_cu(int v);
void q6k_set_wgs_per_cu(int v);
void q4k_set_waves(int v);
void q6k_set_waves(int v);
void q6k_set_flat_items(int v);
void q6k_set_flat_seg(int v);
void q6k_set_rows(int v);
void q4k_set_flat_items(int v);
void q4k_gemm_set_res(int v);
void q6k_set_dig(int v);
void q6k_gemm_set_tn(int v);
void q6k_gemm_set_sk(int v);
// Target workgroups of the skinny (<= 16 token) launches (0: default).
void q4k_skinny_set_target_wgs(int wgs);
void q6k_skinny_set_target_wgs(int wgs);
void dec_set_gu_items(int v);
void dec_set_gu_grid(int v);
void dec_set_merge_rows(int v);
void dec_set_qkv_items(int v);
void dec_set_attn_parts(int v);
// Grow-only device workspace slot `slot` (0..7) of at least `bytes`.
int workspace(int slot, size_t bytes, void **ptr);
// Look up this device's address of the no-allocation scratch array (with
// the device current; once per device).
int noalloc_setup(int device);

}  // namespace hako

#define HK_HIP(call)                                                        \
	do {                                                                    \
		hipError_t hk_e_ = (call);                                          \
		if (hk_e_ != hipSuccess) return hako::hip_fail(hk_e_, #call, __FILE__, __LINE__); \
	} while (0)

// After a kernel launch: report a launch failure as EHIP.
#define HK_LAUNCHED(name) HK_HIP(hipGetLastError())
