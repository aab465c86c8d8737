"""The device decode step (include/hako_decode.h) against the reference's own
forward (src/model.c:93-165, compiled from its sources, all-CPU) and greedy
pick (src/sample.c:28-32), on seeded synthetic Qwen2 MLF2 files.

Bar: identical greedy token sequences. Logits are compared loosely: the q8
re-quantization of activations that differ in the last bit (rmsnorm's sum
order) flips single int8 values, which moves logits by ~1e-3 of their range.
"""
import ctypes as C

import numpy as np
import pytest

from hako_amd import mlf2, synth
from helpers import maxabs_rel

pytestmark = pytest.mark.gpu

TINY = mlf2.Qwen2Config(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512,
                        vocab=1024, ctx=256)
TINY_UNTIED = mlf2.Qwen2Config(n_layers=2, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768,
                               vocab=768, ctx=256, tied=False, embd_type=synth.TYPE_Q4_K)
SMALL_128 = mlf2.Qwen2Config(n_layers=3, d_model=1024, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=2816,
                             vocab=4096, ctx=512)
# 7 query heads per KV head (the 7B grouping): one sequence's attention
# splits a group's heads 2 + 2 + 2 + 1 over four workgroups
GQA7 = mlf2.Qwen2Config(n_layers=2, d_model=1792, n_heads=14, n_kv_heads=2, head_dim=128, ffn_dim=1536,
                        vocab=2000, ctx=256)
# the 7-head grouping with ffn_dim 2304: the reference scores positions in its
# ffn_dim-long gate buffer (src/model.c:125), so positions up to 2300 stay in it
GQA7_LONG = mlf2.Qwen2Config(n_layers=2, d_model=1792, n_heads=14, n_kv_heads=2, head_dim=128, ffn_dim=2304,
                             vocab=2000, ctx=4096)
# one KV head per query head pair with head_dim 64 (two head parts of one head)
GQA2 = mlf2.Qwen2Config(n_layers=2, d_model=512, n_heads=8, n_kv_heads=4, head_dim=64, ffn_dim=768,
                        vocab=1024, ctx=256)


@pytest.fixture(scope="module")
def ref():
    from dropin import bind_ctx
    from oracle.hako_oracle import REF_LIB
    return bind_ctx(C.CDLL(REF_LIB))


def make_decoder(gpu, path, max_seq):
    from hako_amd.decoder import Decoder
    return Decoder(gpu, path, n_seq=1, max_seq=max_seq)


@pytest.mark.parametrize("cfg,seed", [(TINY, 1), (TINY_UNTIED, 2), (SMALL_128, 3), (GQA7, 4), (GQA2, 5)])
def test_greedy_tokens_match_reference(gpu, ref, tmp_path, cfg, seed):
    from dropin import greedy
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    steps = 24
    want, want_logits = greedy(ref, path, start=3, steps=steps, vocab=cfg.vocab, max_seq=128)
    assert np.all(np.isfinite(want_logits))
    dec = make_decoder(gpu, path, max_seq=128)
    try:
        dec.set_pos(0)
        got, logits, tok = [], [], 3
        for _ in range(steps):
            nxt, lg = dec.step(tok, logits=True)
            tok = int(nxt[0])
            got.append(tok)
            logits.append(lg[0])
            assert tok == int(np.argmax(lg[0]))      # device argmax == first maximum
    finally:
        dec.close()
    assert got == want
    assert maxabs_rel(np.stack(logits), want_logits) < 2e-2


# position 2200: 35 chunks, more than the merge loads in its first round trip
@pytest.mark.parametrize("cfg,seed,pos", [(TINY, 4, 100), (SMALL_128, 5, 300), (GQA7, 6, 250),
                                          (GQA7_LONG, 7, 2200)])
def test_prefilled_cache_matches_reference(gpu, ref, tmp_path, cfg, seed, pos):
    """KV cache filled with seeded N(0,1) keys and values at 0..pos-1, as the
    decode benchmarks start: the attention spans several 64-position chunks."""
    from dropin import prefilled_greedy
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    max_seq = max(512, pos + 64)
    kvd = cfg.n_kv_heads * cfg.head_dim
    rng = np.random.default_rng(seed)
    kv = rng.standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    steps = 12
    want, want_logits = prefilled_greedy(ref, path, kv, pos, start=7, steps=steps, vocab=cfg.vocab,
                                         max_seq=max_seq)
    assert np.all(np.isfinite(want_logits))
    dec = make_decoder(gpu, path, max_seq=max_seq)
    try:
        k, v = dec.kv()
        for l in range(cfg.n_layers):
            gpu.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
            gpu.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
        dec.set_pos(pos)
        got = dec.generate(7, steps)[:, 0].tolist()
    finally:
        dec.close()
    assert got == want


def test_graph_replays_equal_eager_steps(gpu, tmp_path):
    """generate() replays one captured step; every replay must equal the
    eager launch sequence, also across two generate calls."""
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, SMALL_128, 6)
    dec = make_decoder(gpu, path, max_seq=256)
    try:
        dec.set_pos(0)
        eager, tok = [], 11
        for _ in range(20):
            tok = int(dec.step(tok)[0])
            eager.append(tok)
        dec.set_pos(0)
        first = dec.generate(11, 10)[:, 0].tolist()
        second = dec.generate(first[-1], 10)[:, 0].tolist()
    finally:
        dec.close()
    assert first + second == eager


def test_decoder_from_mapped_model_in_c(gpu, ref, tmp_path):
    """The C11 drop-in builds the same decoder from the reference's own mapped
    model (hakm_ctx.model), as hako's engine would."""
    from dropin import greedy, host_lib
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, TINY_UNTIED, 8)
    want, _ = greedy(ref, path, start=5, steps=10, vocab=TINY_UNTIED.vocab, max_seq=64)
    host = host_lib()
    host.hako_decoder_from_model.restype = C.c_int
    host.hako_decoder_from_model.argtypes = [C.c_void_p, C.c_int, C.c_int, C.POINTER(C.c_void_p)]
    ctx = ref.hakm_ctx_new(path.encode(), 64)
    assert ctx
    d = C.c_void_p()
    try:
        assert host.hako_decoder_from_model(ctx, 1, 64, C.byref(d)) == 0
        lib = gpu.lib
        pos = np.zeros(1, np.int32)
        assert lib.hako_gpu_decoder_set_pos(d, pos.ctypes.data) == 0
        tok = np.array([5], np.int32)
        out = np.empty(10, np.int32)
        assert lib.hako_gpu_decoder_generate(d, tok.ctypes.data, 10, out.ctypes.data) == 0
        assert lib.hako_gpu_decoder_destroy(d) == 0
    finally:
        host.hako_model_release(ctx)
        ref.hakm_ctx_free(ctx)
    assert out.tolist() == want


def test_decoder_rejects_bad_use(gpu, tmp_path):
    from hako_amd.gpu import HakoGpuError
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, TINY, 9)
    dec = make_decoder(gpu, path, max_seq=16)
    try:
        with pytest.raises(HakoGpuError, match="position"):
            dec.set_pos(16)
        dec.set_pos(10)
        with pytest.raises(HakoGpuError, match="no room"):
            dec.generate(1, 7)
        with pytest.raises(HakoGpuError, match="vocabulary"):
            dec.step(TINY.vocab)
    finally:
        dec.close()


def test_qwen2_3b_decode_at_position_1024(gpu, ref, tmp_path):
    """The full Qwen2.5-3B shape (36 layers, Q4_K_M mix, tied Q6_K
    embedding) with the KV cache prefilled to 1024 positions: greedy tokens
    equal the reference's."""
    from dropin import prefilled_greedy
    cfg = mlf2.QWEN2_3B
    path = str(tmp_path / "qwen2_3b.mlf2")
    mlf2.write_qwen2(path, cfg, 30)
    pos, max_seq, steps = 1024, 1040, 6
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = np.random.default_rng(31).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    want, want_logits = prefilled_greedy(ref, path, kv, pos, start=9, steps=steps, vocab=cfg.vocab,
                                         max_seq=max_seq)
    assert np.all(np.isfinite(want_logits))
    dec = make_decoder(gpu, path, max_seq=max_seq)
    try:
        k, v = dec.kv()
        for l in range(cfg.n_layers):
            gpu.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
            gpu.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
        dec.set_pos(pos)
        first, lg = dec.step(9, logits=True)
        got = [int(first[0])] + dec.generate(int(first[0]), steps - 1)[:, 0].tolist()
    finally:
        dec.close()
    assert got == want
    # this random 3B model repeats one token, so the logits carry the check
    assert maxabs_rel(lg[0], want_logits[0]) < 1e-3
