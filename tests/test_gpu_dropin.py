"""The C11 drop-in (libhako.so) under the reference's own API and callers.

* quant.h surface: dequant_q4_K / dequant_q6_K / dequant_tensor,
  quantize_row_q8_32, q4k_vec_dot, against the reference's golden outputs.
* nn.h surface: matmul / deq_row on a model view, against the golden matmul.
* The reference's model.c (compiled from its sources into
  oracle/_ref/libhakm_ref_model.so) linked against libhako.so in place of
  nn.c: greedy tokens of a synthetic Qwen2 MLF2 must equal those of the
  reference's all-CPU build.
"""
import ctypes as C
import os

import numpy as np
import pytest

from hako_amd import mlf2, synth
from helpers import maxabs_rel, within

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def host(gpu):
    from dropin import host_lib
    return host_lib()


def P(a):
    return a.ctypes.data


def test_f16_to_f32(host):
    for v in (0x0000, 0x0001, 0x03FF, 0x3C00, 0x7BFF, 0x8001, 0xFC00):
        want = np.array([v], np.uint16).view(np.float16).astype(np.float32)[0]
        assert host.f16_to_f32(v) == want


def test_dequant_golden(host, golden):
    for qt, name, fn in ((12, "q4k_dequant.npz", host.dequant_q4_K), (14, "q6k_dequant.npz", host.dequant_q6_K)):
        g = golden(name)
        n = g["blocks"].shape[0] * 256
        for f in (fn, lambda b, o, n_, qt=qt: host.dequant_tensor(qt, b, o, n_)):
            out = np.empty(n, np.float32)
            f(P(g["blocks"]), P(out), n)
            assert np.array_equal(out.view(np.uint32), g["out"].view(np.uint32)), name
    assert host.dequant_tensor(7, None, None, 256) == -1


def test_quantize_and_dot_golden(host, golden):
    g = golden("q8.npz")
    for r in range(g["x"].shape[0]):
        xq = np.empty(2048, np.int8)
        xs = np.empty(64, np.float32)
        host.quantize_row_q8_32(P(g["x"][r]), 2048, P(xq), P(xs))
        assert np.array_equal(xq, g["xq"][r])
        assert np.array_equal(xs.view(np.uint32), g["xs"][r].view(np.uint32))
    d = golden("q4k_dot.npz")
    xq = np.empty(2048, np.int8)
    xs = np.empty(64, np.float32)
    host.quantize_row_q8_32(P(d["x"]), 2048, P(xq), P(xs))
    got = np.array([host.q4k_vec_dot(P(d["w"][r]), 2048, P(xq), P(xs)) for r in range(16)])
    assert maxabs_rel(got, d["out"]) < 1e-5


@pytest.mark.parametrize("name", ["q4k", "q6k", "q6k_long", "f16", "f32"])
def test_nn_matmul_golden(host, golden, name):
    from oracle.hako_oracle import fake_model
    g = golden("matmul.npz")
    qt, n_out, n_in = (int(v) for v in g[f"{name}_shape"])
    w = np.ascontiguousarray(g[f"{name}_w"])
    m, t = fake_model(w, qt, n_in, n_out)
    bias = g.get(f"{name}_bias")
    out = np.empty(n_out, np.float32)
    host.matmul(P(out), P(g[f"{name}_x"]), C.byref(m), C.byref(t), None if bias is None else P(bias),
                n_out, n_in)
    assert maxabs_rel(out, g[f"{name}_out"]) < 1e-5
    row = np.empty(n_in, np.float32)
    host.deq_row(C.byref(m), C.byref(t), n_out - 1, n_in, P(row))
    from oracle.hako_oracle import Oracle
    want = Oracle().dequant(qt, w.reshape(n_out, -1)[n_out - 1], n_in)
    assert np.array_equal(row.view(np.uint32), want.view(np.uint32))


TINY = mlf2.Qwen2Config(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512,
                        vocab=1024, ctx=64)
TINY_UNTIED = mlf2.Qwen2Config(n_layers=2, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768,
                               vocab=768, ctx=64, tied=False, embd_type=synth.TYPE_Q4_K)


@pytest.mark.parametrize("cfg,seed", [(TINY, 1), (TINY_UNTIED, 2)])
def test_reference_model_c_on_dropin(host, tmp_path, cfg, seed):
    """The reference's hakm_forward, unchanged, calling this library's matmul."""
    from dropin import bind_ctx, greedy
    from oracle.hako_oracle import REF_LIB, REF_MODEL_LIB
    path = str(tmp_path / "tiny.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    ref = bind_ctx(C.CDLL(REF_LIB))                 # all-CPU reference build
    dropin = bind_ctx(C.CDLL(REF_MODEL_LIB))        # model.c + loader.c -> libhako.so
    assert os.path.exists(REF_MODEL_LIB)
    t_ref, l_ref = greedy(ref, path, start=1, steps=8, vocab=cfg.vocab)
    t_gpu, l_gpu = greedy(dropin, path, start=1, steps=8, vocab=cfg.vocab, release=host.hako_model_release)
    assert t_gpu == t_ref
    # measured 6.6e-7 and 6.8e-7
    within(f"model.c on drop-in logits {cfg.d_model}", l_gpu, l_ref, 3.3e-6)


@pytest.mark.timeout(600)
def test_reference_model_c_on_dropin_qwen2_3b(host, tmp_path):
    """The reference's hakm_forward, unchanged (src/model.c:93-165), on the
    full Qwen2.5-3B shape from a cache prefilled to 1024 positions, its 253
    matmuls per token through this library: two greedy steps give the
    all-CPU reference's tokens and logits."""
    from dropin import bind_ctx, prefilled_greedy
    from oracle.hako_oracle import REF_LIB, REF_MODEL_LIB
    cfg = mlf2.QWEN2_3B
    path = str(tmp_path / "qwen2_3b.mlf2")
    mlf2.write_qwen2(path, cfg, 33)
    pos, max_seq = 1024, 1032
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = np.random.default_rng(34).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    ref = bind_ctx(C.CDLL(REF_LIB))
    dropin = bind_ctx(C.CDLL(REF_MODEL_LIB))
    t_ref, l_ref = prefilled_greedy(ref, path, kv, pos, start=21, steps=2, vocab=cfg.vocab, max_seq=max_seq)
    t_gpu, l_gpu = prefilled_greedy(dropin, path, kv, pos, start=21, steps=2, vocab=cfg.vocab, max_seq=max_seq,
                                    release=host.hako_model_release)
    assert t_gpu == t_ref
    within("model.c on drop-in, 3B at 1024", l_gpu, l_ref, 8e-5)   # measured 1.7e-5
