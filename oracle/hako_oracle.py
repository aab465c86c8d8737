"""ctypes bindings of the CPU checker.

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and bench.py's
CPU-baseline leg, never by product code.

* ``Oracle`` — this repository's C restatement (oracle/hako_oracle.c, built
  into oracle/_build/libhako_oracle.so).
* ``RefLib`` — the reference's own quant.c/nn.c/loader.c/model.c/sample.c
  compiled by oracle/ref.mk into oracle/_ref/libhakm_ref.so. Loading it sets
  FTZ/DAZ on the loading thread (its -ffast-math build carries gcc's
  crtfastmath constructor), exactly as the reference executable runs.
"""
from __future__ import annotations

import ctypes as C
import time
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(ORACLE_DIR, "_build", "libhako_oracle.so")
REF_LIB = os.path.join(ORACLE_DIR, "_ref", "libhakm_ref.so")
REF_MODEL_LIB = os.path.join(ORACLE_DIR, "_ref", "libhakm_ref_model.so")
# the same reference sources built without -ffast-math (oracle/ref.mk)
REF_NOFAST_LIB = os.path.join(ORACLE_DIR, "_ref", "libhakm_ref_nofast.so")

_vp, _i, _i64 = C.c_void_p, C.c_int, C.c_int64


def _p(a):
    if a is None:
        return None
    assert isinstance(a, np.ndarray) and a.flags["C_CONTIGUOUS"], type(a)
    return a.ctypes.data


class Oracle:
    """The C restatement of the reference's arithmetic."""

    _sigs = {
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_dequant_tensor": (_i, [_i, _vp, _vp, _i64]),
        "orc_quantize_row_q8_32": (None, [_vp, _i, _vp, _vp]),
        "orc_q4k_isums": (None, [_vp, _i, _vp, _vp, _vp]),
        "orc_q4k_vec_dot": (C.c_float, [_vp, _i, _vp, _vp]),
        "orc_q4k_vec_dot_f64": (C.c_double, [_vp, _i, _vp, _vp]),
        "orc_matmul": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i, _i, _i]),
        "orc_matmul_batch": (_i, [_vp, _vp, _i, _i, _vp, _vp, _i, _i, _i, _i]),
        "orc_argmax": (_i, [_vp, _i]),
    }

    def __init__(self, path: str = ORACLE_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle)")
        self.lib = C.CDLL(path)
        for n, (r, a) in self._sigs.items():
            f = getattr(self.lib, n)
            f.restype, f.argtypes = r, a

    def f16_to_f32(self, h: int) -> float:
        return self.lib.orc_f16_to_f32(h)

    def dequant(self, qtype: int, src: np.ndarray, nelem: int) -> np.ndarray:
        out = np.empty(nelem, np.float32)
        rc = self.lib.orc_dequant_tensor(qtype, _p(np.ascontiguousarray(src)), _p(out), nelem)
        if rc:
            raise ValueError(f"type {qtype}")
        return out

    def quantize_q8_32(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        xq = np.empty(x.size, np.int8)
        xs = np.empty(x.size // 32, np.float32)
        self.lib.orc_quantize_row_q8_32(_p(x), x.size, _p(xq), _p(xs))
        return xq, xs

    def q4k_isums(self, w: np.ndarray, xq: np.ndarray, n_out: int, n_in: int):
        """Per (row, sub-block) Σq·xq and Σxq, [n_out, n_in/32] each."""
        w = np.ascontiguousarray(w).reshape(n_out, -1)
        iqx = np.empty((n_out, n_in // 32), np.int32)
        ix = np.empty((n_out, n_in // 32), np.int32)
        for r in range(n_out):
            self.lib.orc_q4k_isums(_p(w[r]), n_in, _p(xq), _p(iqx[r]), _p(ix[r]))
        return iqx, ix

    def q4k_vec_dot(self, w_row: np.ndarray, n_in: int, xq, xs, f64: bool = False) -> float:
        fn = self.lib.orc_q4k_vec_dot_f64 if f64 else self.lib.orc_q4k_vec_dot
        return fn(_p(np.ascontiguousarray(w_row)), n_in, _p(xq), _p(xs))

    def matmul(self, qtype: int, w: np.ndarray, x: np.ndarray, n_out: int, n_in: int,
               bias: np.ndarray | None = None, f64: bool = True, threads: int = 8) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        if x.ndim == 2:
            M = x.shape[0]
            out = np.empty((M, n_out), np.float32)
            rc = self.lib.orc_matmul_batch(_p(out), _p(x), M, qtype, _p(np.ascontiguousarray(w)),
                                           _p(bias), n_out, n_in, int(f64), threads)
        else:
            out = np.empty(n_out, np.float32)
            rc = self.lib.orc_matmul(_p(out), _p(x), qtype, _p(np.ascontiguousarray(w)), _p(bias),
                                     n_out, n_in, int(f64), threads)
        if rc:
            raise ValueError(f"type {qtype}")
        return out

    def argmax(self, logits: np.ndarray) -> int:
        logits = np.ascontiguousarray(logits, np.float32)
        return self.lib.orc_argmax(_p(logits), logits.size)


class MlfTensor(C.Structure):
    """reference include/mlf2.h:80-87 (packed, 104 bytes)."""
    _pack_ = 1
    _fields_ = [("name", C.c_char * 48), ("type", C.c_uint32), ("n_dims", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("data_off", C.c_uint64), ("nbytes", C.c_uint64)]


class HakmModel(C.Structure):
    """reference src/loader.h:6-13 (header bytes, then five pointers/sizes)."""
    _fields_ = [("h", C.c_uint8 * 128), ("tensors", _vp), ("data", _vp), ("tok", _vp),
                ("map", _vp), ("map_size", C.c_size_t)]


assert C.sizeof(MlfTensor) == 104 and C.sizeof(HakmModel) == 168


def fake_model(w: np.ndarray, qtype: int, n_in: int, n_out: int):
    """A loaded-model view over one weight buffer (no file, no mapping)."""
    t = MlfTensor()
    t.name = b"w"
    t.type = qtype
    t.n_dims = 2
    t.dims[0], t.dims[1] = n_in, n_out
    t.data_off = 0
    t.nbytes = w.nbytes
    m = HakmModel()
    m.tensors = C.addressof(t)
    m.data = w.ctypes.data
    return m, t


class RefLib:
    """The reference's own C path, compiled unmodified (oracle/ref.mk)."""

    _sigs = {
        "f16_to_f32": (C.c_float, [C.c_uint16]),
        "dequant_q4_K": (None, [_vp, _vp, _i]),
        "dequant_q6_K": (None, [_vp, _vp, _i]),
        "dequant_tensor": (_i, [_i, _vp, _vp, _i]),
        "quantize_row_q8_32": (None, [_vp, _i, _vp, _vp]),
        "q4k_vec_dot": (C.c_float, [_vp, _i, _vp, _vp]),
        "matmul": (None, [_vp, _vp, _vp, _vp, _vp, _i, _i]),
        "deq_row": (None, [_vp, _vp, _i, _i, _vp]),
        "hakm_ctx_new": (_vp, [C.c_char_p, _i]),
        "hakm_ctx_free": (None, [_vp]),
        "hakm_forward": (_vp, [_vp, _i]),
        "hakm_reset": (None, [_vp]),
    }

    def __init__(self, path: str = REF_LIB, threads: int | None = None):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -f oracle/ref.mk)")
        if threads is not None:
            # read once, at the reference's first matmul (src/nn.c:99-107)
            os.environ["HAKM_THREADS"] = str(threads)
        self.lib = C.CDLL(path)
        for n, (r, a) in self._sigs.items():
            f = getattr(self.lib, n)
            f.restype, f.argtypes = r, a

    def dequant(self, qtype: int, src: np.ndarray, nelem: int) -> np.ndarray:
        out = np.empty(nelem, np.float32)
        rc = self.lib.dequant_tensor(qtype, _p(np.ascontiguousarray(src)), _p(out), nelem)
        if rc:
            raise ValueError(f"type {qtype}")
        return out

    def quantize_q8_32(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        xq = np.empty(x.size, np.int8)
        xs = np.empty(x.size // 32, np.float32)
        self.lib.quantize_row_q8_32(_p(x), x.size, _p(xq), _p(xs))
        return xq, xs

    def q4k_vec_dot(self, w_row: np.ndarray, n_in: int, xq: np.ndarray, xs: np.ndarray) -> float:
        return self.lib.q4k_vec_dot(_p(np.ascontiguousarray(w_row)), n_in, _p(xq), _p(xs))

    def matmul(self, qtype: int, w: np.ndarray, x: np.ndarray, n_out: int, n_in: int,
               bias: np.ndarray | None = None) -> np.ndarray:
        """reference matmul (src/nn.c:179-210) over a fake one-tensor model.
        Its thread pool starts at the first call: that call must have
        n_out >= the thread count (src/nn.c:182-184)."""
        w = np.ascontiguousarray(w)
        m, t = fake_model(w, qtype, n_in, n_out)
        out = np.empty(n_out, np.float32)
        self.lib.matmul(_p(out), _p(np.ascontiguousarray(x, np.float32)), C.byref(m), C.byref(t),
                        _p(bias), n_out, n_in)
        return out


class HakmCtx(C.Structure):
    """The reference's hakm_ctx (src/model.h:12-26), for tests that fill its
    KV cache and position directly (a prefilled context)."""
    _fields_ = [("model", C.c_uint8 * 168), ("layers", _vp), ("tok_embd", _vp), ("out_norm", _vp),
                ("out_weight", _vp), ("d_model", _i), ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i),
                ("kv_dim", _i), ("ffn_dim", _i), ("n_layers", _i), ("vocab", _i), ("rope_theta", C.c_float),
                ("rms_eps", C.c_float), ("max_seq", _i), ("pos", _i), ("k_cache", _vp), ("v_cache", _vp),
                ("xb", _vp), ("xn", _vp), ("q", _vp), ("k", _vp), ("v", _vp), ("att_out", _vp),
                ("gate_buf", _vp), ("up_buf", _vp), ("deq", _vp), ("logits", _vp)]


assert C.sizeof(HakmCtx) == 344


class Sampler(C.Structure):
    """The reference's sampler (src/sample.h:6-11); temp <= 0 is greedy."""
    _fields_ = [("temp", C.c_float), ("top_p", C.c_float), ("top_k", C.c_int), ("rng", C.c_uint64)]


_PICK = None


def ref_greedy_pick(logits: np.ndarray) -> int:
    """The reference's greedy pick (sample_token with temp 0,
    src/sample.c:27-32, from the compiled reference): the scan starts from
    logits[0] and only a strictly larger value replaces the best, so the
    first maximum wins, a NaN never does, and a NaN at index 0 is kept."""
    global _PICK
    if _PICK is None:
        lib = C.CDLL(REF_LIB)
        lib.sample_token.restype = C.c_int
        lib.sample_token.argtypes = [C.POINTER(Sampler), _vp, _i]
        _PICK = lib
    lg = np.ascontiguousarray(logits, np.float32).copy()
    s = Sampler(0.0, 0.0, 0, 1)
    return int(_PICK.sample_token(C.byref(s), _p(lg), lg.size))


def prefilled_greedy(lib: C.CDLL, path: str, kv: np.ndarray, pos: int, start: int, steps: int, vocab: int,
                     max_seq: int, times: list | None = None, release=None):
    """Greedy decode through the reference's model.h API after writing the
    caches directly: kv[0] / kv[1] are [n_layers][pos][kv_dim] keys / values
    placed at positions 0..pos-1, and ctx.pos = pos. `times`, when given,
    receives the wall time of each hakm_forward call (src/model.c:93);
    `release(ctx)`, when given, runs before hakm_ctx_free unmaps the model."""
    ctx = lib.hakm_ctx_new(path.encode(), max_seq)
    assert ctx, f"hakm_ctx_new({path}) failed"
    toks, logits = [start], []
    try:
        c = HakmCtx.from_address(ctx)
        n_layers, kvd = kv.shape[1], kv.shape[3]
        for which, ptr in ((0, c.k_cache), (1, c.v_cache)):
            cache = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=(n_layers, max_seq, kvd))
            cache[:, :pos, :] = kv[which]
        c.pos = pos
        for _ in range(steps):
            t0 = time.perf_counter()
            p = lib.hakm_forward(ctx, toks[-1])
            if times is not None:
                times.append(time.perf_counter() - t0)
            lg = np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(vocab,)).copy()
            logits.append(lg)
            toks.append(ref_greedy_pick(lg))
    finally:
        if release is not None:
            release(ctx)
        lib.hakm_ctx_free(ctx)
    return toks[1:], np.stack(logits)


def prefilled_forced(lib: C.CDLL, path: str, kv: np.ndarray, pos: int, tokens, vocab: int, max_seq: int):
    """As prefilled_greedy, but each step is fed the given token (teacher
    forcing): the logits of hakm_forward for tokens[0], tokens[1], ... from
    the prefilled caches."""
    ctx = lib.hakm_ctx_new(path.encode(), max_seq)
    assert ctx, f"hakm_ctx_new({path}) failed"
    logits = []
    try:
        c = HakmCtx.from_address(ctx)
        n_layers, kvd = kv.shape[1], kv.shape[3]
        for which, ptr in ((0, c.k_cache), (1, c.v_cache)):
            cache = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=(n_layers, max_seq, kvd))
            cache[:, :pos, :] = kv[which]
        c.pos = pos
        for t in tokens:
            p = lib.hakm_forward(ctx, int(t))
            logits.append(np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(vocab,)).copy())
    finally:
        lib.hakm_ctx_free(ctx)
    return np.stack(logits)
