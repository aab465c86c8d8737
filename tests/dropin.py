"""Loading helpers for the drop-in tests: libhako.so (the product's quant.h /
nn.h surface) and the reference's model.c bound to it."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from hako_amd.gpu import HOST_LIB

_vp, _i = C.c_void_p, C.c_int

HOST_SIGS = {
    "f16_to_f32": (C.c_float, [C.c_uint16]),
    "dequant_q4_K": (None, [_vp, _vp, _i]),
    "dequant_q6_K": (None, [_vp, _vp, _i]),
    "dequantize_row_q4_K": (None, [_vp, _vp, C.c_int64]),
    "dequantize_row_q6_K": (None, [_vp, _vp, C.c_int64]),
    "dequant_tensor": (_i, [_i, _vp, _vp, _i]),
    "quantize_row_q8_32": (None, [_vp, _i, _vp, _vp]),
    "q4k_vec_dot": (C.c_float, [_vp, _i, _vp, _vp]),
    "matmul": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
    "deq_row": (None, [_vp, _vp, _i, _i, _vp]),
    "rmsnorm": (None, [_vp, _vp, _vp, _i, C.c_float]),
    "softmax": (None, [_vp, _i]),
    "silu_f": (C.c_float, [C.c_float]),
    "rope_neox": (None, [_vp, _i, _i, C.c_float]),
    "hako_model_upload": (_i, [_vp]),
    "hako_model_release": (_i, [_vp]),
}

_host = None


def host_lib() -> C.CDLL:
    """libhako.so, loaded RTLD_GLOBAL so that a caller library loaded after it
    (the reference's model.c) binds matmul, deq_row, rmsnorm, ... to it."""
    global _host
    if _host is None:
        if not os.path.exists(HOST_LIB):
            raise FileNotFoundError(f"{HOST_LIB} not built")
        lib = C.CDLL(HOST_LIB, mode=C.RTLD_GLOBAL)
        for n, (r, a) in HOST_SIGS.items():
            f = getattr(lib, n)
            f.restype, f.argtypes = r, a
        _host = lib
    return _host


CTX_SIGS = {
    "hakm_ctx_new": (_vp, [C.c_char_p, _i]),
    "hakm_ctx_free": (None, [_vp]),
    "hakm_forward": (_vp, [_vp, _i]),
    "hakm_reset": (None, [_vp]),
}


def bind_ctx(lib: C.CDLL) -> C.CDLL:
    for n, (r, a) in CTX_SIGS.items():
        f = getattr(lib, n)
        f.restype, f.argtypes = r, a
    return lib


def greedy(lib: C.CDLL, path: str, start: int, steps: int, vocab: int, max_seq: int = 64, release=None):
    """Greedy decode through a library exporting the reference's model.h API:
    returns the token ids and the logits of every step. `release(ctx)`, when
    given, runs before hakm_ctx_free unmaps the model (the drop-in's
    hako_model_release: the model's HBM mirror goes with its mapping)."""
    ctx = lib.hakm_ctx_new(path.encode(), max_seq)
    assert ctx, f"hakm_ctx_new({path}) failed"
    toks, logits = [start], []
    try:
        for _ in range(steps):
            p = lib.hakm_forward(ctx, toks[-1])
            lg = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(vocab,)).copy()
            logits.append(lg)
            toks.append(ref_greedy_pick(lg))   # the reference's own pick, src/sample.c:28-32
    finally:
        if release is not None:
            release(ctx)
        lib.hakm_ctx_free(ctx)
    return toks[1:], np.stack(logits)


from oracle.hako_oracle import HakmCtx, prefilled_greedy, ref_greedy_pick  # noqa: E402,F401
