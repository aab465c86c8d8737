"""CPU-only checks of the product's host side: the C ABI libraries load and
export every function the headers declare, errors surface without a device,
the MLF2 writer produces files the reference's own loader and forward
accept, and the drop-in's host elementwise helpers agree with the reference."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from hako_amd import mlf2, synth
from hako_amd.gpu import GPU_LIB, HOST_LIB, SIGNATURES, load_library
from helpers import maxabs_rel

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HAS_GPU = os.path.exists("/dev/kfd")


def declared_functions(header: str):
    src = open(os.path.join(REPO, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    names = re.findall(r"^[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\([^;{]*\)\s*(?:__attribute__\(\(.*?\)\))?\s*;",
                       src, flags=re.M)
    return sorted(set(names))


def test_gpu_abi_exports_every_declared_function():
    names = sorted(declared_functions("hako_gpu.h") + declared_functions("hako_decode.h"))
    assert len(names) >= 35
    lib = C.CDLL(GPU_LIB)
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(SIGNATURES) == names


def test_dropin_exports_quant_and_nn_surface():
    lib = C.CDLL(HOST_LIB)
    names = declared_functions("hako_quant.h") + declared_functions("hako_nn.h")
    for n in ("f16_to_f32", "dequant_q4_K", "dequant_q6_K", "dequant_tensor", "quantize_row_q8_32",
              "q4k_vec_dot", "matmul", "deq_row", "rmsnorm", "softmax", "silu_f", "rope_neox"):
        assert n in names
    for n in names:
        assert hasattr(lib, n), n


@pytest.mark.skipif(HAS_GPU, reason="checks the no-device error path")
def test_no_device_is_reported():
    lib = load_library()
    p = C.c_void_p()
    assert lib.hako_gpu_malloc(C.byref(p), 16) == -2          # not initialised
    assert b"hako_gpu_init" in lib.hako_gpu_last_error()
    assert lib.hako_gpu_init(0) == -2                          # no device here
    assert lib.hako_gpu_last_error() != b""


def test_mlf2_writer_layout(tmp_path):
    cfg = mlf2.Qwen2Config(n_layers=1, d_model=256, n_heads=2, n_kv_heads=1, head_dim=128,
                           ffn_dim=512, vocab=512)
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed=3)
    f = mlf2.Mlf2File(path)
    assert f.header["data_off"] % 32 == 0
    assert all(t["data_off"] % 32 == 0 for t in f.tensors.values())
    assert f.tensors["blk.0.ffn_down.weight"]["type"] == synth.TYPE_Q6_K
    assert f.tensors["blk.0.attn_q.weight"]["nbytes"] == 256 * 144
    assert "output.weight" not in f.tensors
    emb = f.data("token_embd.weight")
    assert emb.size == 512 * 210


def test_reference_loads_and_runs_written_model(tmp_path):
    """The reference's own mlf2_open / hakm_ctx_new / hakm_forward (CPU)
    accept the synthetic file and produce finite logits."""
    from oracle.hako_oracle import REF_LIB
    import sys
    sys.path.insert(0, os.path.dirname(__file__))
    from dropin import bind_ctx, greedy
    cfg = mlf2.Qwen2Config(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64,
                           ffn_dim=512, vocab=1024, ctx=64)
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed=5)
    toks, logits = greedy(bind_ctx(C.CDLL(REF_LIB)), path, start=1, steps=3, vocab=1024)
    assert len(toks) == 3 and np.all(np.isfinite(logits))


def test_host_elementwise_helpers_match_reference():
    """rmsnorm / softmax / silu_f / rope_neox of libhako.so (host code) against
    the reference's compiled nn.c."""
    from oracle.hako_oracle import REF_LIB
    ours, ref = C.CDLL(HOST_LIB), C.CDLL(REF_LIB)
    for lib in (ours, ref):
        lib.rmsnorm.argtypes = [C.c_void_p] * 3 + [C.c_int, C.c_float]
        lib.softmax.argtypes = [C.c_void_p, C.c_int]
        lib.silu_f.argtypes = [C.c_float]
        lib.silu_f.restype = C.c_float
        lib.rope_neox.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_float]
    rng = np.random.default_rng(9)
    x = rng.standard_normal(2048).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    ya, yb = np.empty_like(x), np.empty_like(x)
    ours.rmsnorm(ya.ctypes.data, x.ctypes.data, w.ctypes.data, 2048, C.c_float(1e-6))
    ref.rmsnorm(yb.ctypes.data, x.ctypes.data, w.ctypes.data, 2048, C.c_float(1e-6))
    assert maxabs_rel(ya, yb) < 1e-6
    sa, sb = x.copy(), x.copy()
    ours.softmax(sa.ctypes.data, 2048)
    ref.softmax(sb.ctypes.data, 2048)
    assert maxabs_rel(sa, sb) < 1e-5
    for v in (-20.0, -1.5, 0.0, 0.3, 7.0):
        assert abs(ours.silu_f(v) - ref.silu_f(v)) <= 1e-6 * max(1.0, abs(v))
    for pos in (0, 1, 1023, 4095):
        ra, rb = x[:128].copy(), x[:128].copy()
        ours.rope_neox(ra.ctypes.data, 128, pos, C.c_float(1e6))
        ref.rope_neox(rb.ctypes.data, 128, pos, C.c_float(1e6))
        assert maxabs_rel(ra, rb) < 1e-4, pos
