"""ctypes view of the hako_gpu C ABI (include/hako_gpu.h) for tests and the bench.

Python never computes here: every call below is a C-ABI call into
``lib/libhako_gpu.so``. Loading fails loudly if the library has not been
built; there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
GPU_LIB = os.path.join(LIB_DIR, "libhako_gpu.so")
HOST_LIB = os.path.join(LIB_DIR, "libhako.so")

TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 12, 14

_vp, _i, _i64, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_size_t

# name -> (restype, argtypes); mirrors include/hako_gpu.h one to one.
SIGNATURES = {
    "hako_gpu_init": (_i, [_i]),
    "hako_gpu_shutdown": (_i, []),
    "hako_gpu_last_error": (C.c_char_p, []),
    "hako_gpu_tune": (_i, [_i, _i]),
    "hako_gpu_device_info": (_i, [_vp]),
    "hako_gpu_malloc": (_i, [C.POINTER(_vp), _sz]),
    "hako_gpu_free": (_i, [_vp]),
    "hako_gpu_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "hako_gpu_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "hako_gpu_memcpy_d2d": (_i, [_vp, _vp, _sz]),
    "hako_gpu_sync": (_i, []),
    "hako_gpu_stream": (_vp, []),
    "hako_gpu_event_create": (_i, [C.POINTER(_vp)]),
    "hako_gpu_event_record": (_i, [_vp]),
    "hako_gpu_event_elapsed_ms": (_i, [_vp, _vp, C.POINTER(C.c_float)]),
    "hako_gpu_event_destroy": (_i, [_vp]),
    "hako_gpu_timestamp": (_i, [_vp]),
    "hako_gpu_timestamp_hz": (_i, [C.POINTER(C.c_double)]),
    "hako_gpu_capture_begin": (_i, []),
    "hako_gpu_capture_end": (_i, [C.POINTER(_vp)]),
    "hako_gpu_graph_launch": (_i, [_vp]),
    "hako_gpu_graph_destroy": (_i, [_vp]),
    "hako_gpu_mirror_upload": (_i, [_vp, _sz, C.POINTER(_vp)]),
    "hako_gpu_mirror_release": (_i, [_vp]),
    "hako_gpu_mirror_lookup": (_vp, [_vp]),
    "hako_gpu_quantize_q8_32": (_i, [_vp, _i64, _i, _vp, _vp]),
    "hako_gpu_dequant": (_i, [_i, _vp, _vp, _i64]),
    "hako_gpu_q4k_gemv": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "hako_gpu_q4k_isums": (_i, [_vp, _vp, _vp, _vp, _i, _i]),
    "hako_gpu_q6k_gemv": (_i, [_vp, _vp, _vp, _vp, _i, _i]),
    "hako_gpu_dense_gemv": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i]),
    "hako_gpu_matmul": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i]),
    "hako_gpu_matmul_host": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i]),
    "hako_gpu_q4k_gemm": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i]),
    "hako_gpu_q6k_gemm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i]),
    "hako_gpu_matmul_batch": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i, _i]),
    "hako_gpu_matmul_batch_noalloc": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i, _i]),
    "hako_gpu_decoder_create": (_i, [_vp, _i, _i, C.POINTER(_vp)]),
    "hako_gpu_decoder_destroy": (_i, [_vp]),
    "hako_gpu_decoder_kv": (_i, [_vp, C.POINTER(_vp), C.POINTER(_vp)]),
    "hako_gpu_decoder_set_pos": (_i, [_vp, _vp]),
    "hako_gpu_decoder_step": (_i, [_vp, _vp, _vp, _vp]),
    "hako_gpu_decoder_generate": (_i, [_vp, _vp, _i, _vp]),
    "hako_gpu_decoder_replay": (_i, [_vp, _i]),
    "hako_gpu_decoder_prefill": (_i, [_vp, _i, _vp, _i, _vp, _vp]),
    "hako_gpu_decoder_on_destroy": (_i, [_vp, _vp, _vp]),
}


class HakoGpuError(RuntimeError):
    pass


class DeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("compute_units", C.c_int), ("clock_khz", C.c_int),
                ("hbm_bytes", C.c_size_t), ("l2_bytes", C.c_int), ("lds_bytes_per_cu", C.c_int)]


_lib = None


def load_library() -> C.CDLL:
    """Load libhako_gpu.so with every C-ABI signature declared."""
    global _lib
    if _lib is None:
        if not os.path.exists(GPU_LIB):
            raise HakoGpuError(f"{GPU_LIB} is not built; run __graft_entry__.build() (make -C hako_amd)")
        lib = C.CDLL(GPU_LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _lib = lib
    return _lib


def _ptr(a) -> int | None:
    if a is None:
        return None
    if isinstance(a, DevBuf):
        return a.ptr
    if isinstance(a, np.ndarray):
        assert a.flags["C_CONTIGUOUS"]
        return a.ctypes.data
    return int(a)


class DevBuf:
    """A device allocation made through hako_gpu_malloc."""

    def __init__(self, gpu: "Gpu", nbytes: int):
        self.gpu, self.nbytes = gpu, int(nbytes)
        p = C.c_void_p()
        gpu.check(gpu.lib.hako_gpu_malloc(C.byref(p), self.nbytes), "malloc")
        self.ptr = p.value

    def free(self):
        if self.ptr:
            self.gpu.check(self.gpu.lib.hako_gpu_free(self.ptr), "free")
            self.ptr = None

    def offset(self, nbytes: int) -> int:
        return self.ptr + int(nbytes)


class Gpu:
    """One initialised device; all work goes to the library stream."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        self.check(self.lib.hako_gpu_init(device), "init")

    def check(self, rc: int, what: str):
        if rc != 0:
            msg = self.lib.hako_gpu_last_error().decode(errors="replace")
            raise HakoGpuError(f"hako_gpu {what}: rc={rc}: {msg}")

    def tune(self, knob: int, value: int):
        self.check(self.lib.hako_gpu_tune(knob, value), "tune")

    def info(self) -> DeviceInfo:
        d = DeviceInfo()
        self.check(self.lib.hako_gpu_device_info(C.byref(d)), "device_info")
        return d

    # memory
    def alloc(self, nbytes: int) -> DevBuf:
        return DevBuf(self, nbytes)

    def upload(self, arr: np.ndarray) -> DevBuf:
        arr = np.ascontiguousarray(arr)
        b = DevBuf(self, max(arr.nbytes, 1))
        self.check(self.lib.hako_gpu_memcpy_h2d(b.ptr, arr.ctypes.data, arr.nbytes), "h2d")
        return b

    def h2d(self, dst, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        self.check(self.lib.hako_gpu_memcpy_h2d(_ptr(dst), arr.ctypes.data, arr.nbytes), "h2d")

    def download(self, src, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        self.check(self.lib.hako_gpu_memcpy_d2h(out.ctypes.data, _ptr(src), out.nbytes), "d2h")
        return out

    def sync(self):
        self.check(self.lib.hako_gpu_sync(), "sync")

    # events
    def event(self) -> int:
        e = C.c_void_p()
        self.check(self.lib.hako_gpu_event_create(C.byref(e)), "event_create")
        return e.value

    def record(self, ev: int):
        self.check(self.lib.hako_gpu_event_record(ev), "event_record")

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = C.c_float()
        self.check(self.lib.hako_gpu_event_elapsed_ms(a, b, C.byref(ms)), "event_elapsed")
        return ms.value

    def timestamp(self, dst):
        """The device wall clock written to dst (8 bytes) when this mark runs."""
        self.check(self.lib.hako_gpu_timestamp(_ptr(dst)), "timestamp")

    def timestamp_hz(self) -> float:
        hz = C.c_double()
        self.check(self.lib.hako_gpu_timestamp_hz(C.byref(hz)), "timestamp_hz")
        return hz.value

    # graphs
    def capture_begin(self):
        self.check(self.lib.hako_gpu_capture_begin(), "capture_begin")

    def capture_end(self) -> int:
        gr = C.c_void_p()
        self.check(self.lib.hako_gpu_capture_end(C.byref(gr)), "capture_end")
        return gr.value

    def graph_launch(self, graph: int):
        self.check(self.lib.hako_gpu_graph_launch(graph), "graph_launch")

    def graph_destroy(self, graph: int):
        self.check(self.lib.hako_gpu_graph_destroy(graph), "graph_destroy")

    # kernels (device pointers or DevBuf)
    def quantize_q8_32(self, x, rows: int, n: int, xq, xs):
        self.check(self.lib.hako_gpu_quantize_q8_32(_ptr(x), rows, n, _ptr(xq), _ptr(xs)), "quantize_q8_32")

    def dequant(self, qtype: int, src, out, nelem: int):
        self.check(self.lib.hako_gpu_dequant(qtype, _ptr(src), _ptr(out), nelem), "dequant")

    def q4k_gemv(self, out, w, xq, xs, bias, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_q4k_gemv(_ptr(out), _ptr(w), _ptr(xq), _ptr(xs), _ptr(bias),
                                              n_out, n_in), "q4k_gemv")

    def q4k_isums(self, iqx, ix, w, xq, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_q4k_isums(_ptr(iqx), _ptr(ix), _ptr(w), _ptr(xq), n_out, n_in),
                   "q4k_isums")

    def q6k_gemv(self, out, w, x, bias, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_q6k_gemv(_ptr(out), _ptr(w), _ptr(x), _ptr(bias), n_out, n_in),
                   "q6k_gemv")

    def matmul(self, out, x, qtype: int, w, bias, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_matmul(_ptr(out), _ptr(x), qtype, _ptr(w), _ptr(bias), n_out, n_in),
                   "matmul")

    def q4k_gemm(self, y, w, xq, xs, bias, m: int, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_q4k_gemm(_ptr(y), _ptr(w), _ptr(xq), _ptr(xs), _ptr(bias), m, n_out, n_in),
                   "q4k_gemm")

    def q6k_gemm(self, y, w, x, bias, m: int, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_q6k_gemm(_ptr(y), _ptr(w), _ptr(x), _ptr(bias), m, n_out, n_in), "q6k_gemm")

    def matmul_batch(self, y, x, qtype: int, w, bias, m: int, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_matmul_batch(_ptr(y), _ptr(x), qtype, _ptr(w), _ptr(bias), m, n_out, n_in),
                   "matmul_batch")

    def matmul_host(self, out: np.ndarray, x: np.ndarray, qtype: int, w_host: np.ndarray,
                    bias: np.ndarray | None, n_out: int, n_in: int):
        self.check(self.lib.hako_gpu_matmul_host(_ptr(out), _ptr(x), qtype, _ptr(w_host), _ptr(bias),
                                                 n_out, n_in), "matmul_host")

    def mirror_upload(self, host: np.ndarray) -> int:
        d = C.c_void_p()
        self.check(self.lib.hako_gpu_mirror_upload(host.ctypes.data, host.nbytes, C.byref(d)), "mirror_upload")
        return d.value

    def mirror_release(self, host: np.ndarray):
        self.check(self.lib.hako_gpu_mirror_release(host.ctypes.data), "mirror_release")
