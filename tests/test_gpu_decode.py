"""The device decode step (include/hako_decode.h) against the reference's own
forward (src/model.c:93-165, compiled from its sources, all-CPU) and greedy
pick (src/sample.c:28-32), on seeded synthetic Qwen2 MLF2 files.

Bars: identical greedy token sequences, and logits within a max-abs-normalised
bar set per case at most 5x the value measured on MI355X (1e-7 .. 2e-5 here):
the reference and the device add in different orders, and where the q8
re-quantization of an activation that differs in its last bit flips one int8
value the logits move by up to ~5e-4 of their range. The device step is
bit-reproducible, so each case's value is fixed.
"""
import ctypes as C

import numpy as np
import pytest

from hako_amd import mlf2, synth
from helpers import maxabs_rel, near_max_steps, within

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


# (cfg, seed, logits bar: measured 6.3e-7, 2.6e-6, 3.9e-6, 5.5e-7, 6.0e-7)
@pytest.mark.parametrize("cfg,seed,bar", [(TINY, 1, 3e-6), (TINY_UNTIED, 2, 1.3e-5), (SMALL_128, 3, 2e-5),
                                          (GQA7, 4, 2.8e-6), (GQA2, 5, 3e-6)])
def test_greedy_tokens_match_reference(gpu, ref, tmp_path, cfg, seed, bar):
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
    within(f"decode logits {cfg.d_model}/{seed}", np.stack(logits), want_logits, bar)


# position 2200: 35 chunks, more than the merge loads in its first round trip
# (logits bars: measured 3.9e-7, 2.1e-6, 7.1e-7, 5.8e-7)
@pytest.mark.parametrize("cfg,seed,pos,bar", [(TINY, 4, 100, 2e-6), (SMALL_128, 5, 300, 1e-5),
                                              (GQA7, 6, 250, 3.5e-6), (GQA7_LONG, 7, 2200, 2.9e-6)])
def test_prefilled_cache_matches_reference(gpu, ref, tmp_path, cfg, seed, pos, bar):
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
        # two eager steps with their logits, then the captured step
        got, logits, tok = [], [], 7
        for _ in range(2):
            nxt, lg = dec.step(tok, logits=True)
            tok = int(nxt[0])
            got.append(tok)
            logits.append(lg[0])
        got += dec.generate(tok, steps - 2)[:, 0].tolist()
    finally:
        dec.close()
    assert got == want
    # the random model's greedy tokens repeat: the logits carry the check of
    # every chunk's softmax weight and value sum
    within(f"prefilled logits {cfg.d_model}/{pos}", np.stack(logits), want_logits[:2], bar)


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
        # the decoder reads the model's mirror: releasing it is refused while it lives
        assert host.hako_model_release(ctx) != 0
        assert lib.hako_gpu_decoder_generate(d, tok.ctypes.data, 10, out.ctypes.data) == 0
        assert lib.hako_gpu_decoder_destroy(d) == 0
        assert host.hako_model_release(ctx) == 0
    finally:
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
    equal the reference's over six steps; then 16 distinct start tokens, one
    step each from the same cache, give the reference's argmax and logits
    (this random model repeats one token from any start, so the per-start
    logits are what tells a wrong attention weight apart); and a repeated
    step is bit-identical."""
    from dropin import prefilled_greedy
    from oracle.hako_oracle import HakmCtx
    cfg = mlf2.QWEN2_3B
    path = str(tmp_path / "qwen2_3b.mlf2")
    mlf2.write_qwen2(path, cfg, 30)
    pos, max_seq, steps = 1024, 1040, 6
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = np.random.default_rng(31).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    want, want_logits = prefilled_greedy(ref, path, kv, pos, start=9, steps=steps, vocab=cfg.vocab,
                                         max_seq=max_seq)
    assert np.all(np.isfinite(want_logits))
    starts = [int(t) for t in np.random.default_rng(32).choice(cfg.vocab, 16, replace=False)]
    # the reference: one context, its cache filled once, position reset per start
    ctx = ref.hakm_ctx_new(path.encode(), max_seq)
    assert ctx
    want_one = []
    try:
        c = HakmCtx.from_address(ctx)
        for which, ptr in ((0, c.k_cache), (1, c.v_cache)):
            cache = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=(cfg.n_layers, max_seq, kvd))
            cache[:, :pos, :] = kv[which]
        for t in starts:
            c.pos = pos
            p = ref.hakm_forward(ctx, t)
            want_one.append(np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(cfg.vocab,)).copy())
    finally:
        ref.hakm_ctx_free(ctx)
    dec = make_decoder(gpu, path, max_seq=max_seq)
    try:
        k, v = dec.kv()
        for l in range(cfg.n_layers):
            gpu.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
            gpu.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
        dec.set_pos(pos)
        first, lg = dec.step(9, logits=True)
        got = [int(first[0])] + dec.generate(int(first[0]), steps - 1)[:, 0].tolist()
        got_one = []
        for t in starts:
            dec.set_pos(pos)
            nxt, l1 = dec.step(t, logits=True)
            assert int(nxt[0]) == int(np.argmax(l1[0]))
            got_one.append(l1[0])
        dec.set_pos(pos)
        _, again = dec.step(starts[-1], logits=True)
    finally:
        dec.close()
    assert got == want
    # measured: 1.6e-5 (start 9), 6.2e-7 .. 1.7e-5 over the 16 starts
    within("3B logits, start 9", lg[0], want_logits[0], 8e-5)
    want_one, got_one = np.stack(want_one), np.stack(got_one)
    assert [int(np.argmax(r)) for r in got_one] == [int(np.argmax(r)) for r in want_one]
    for t, g, w in zip(starts, got_one, want_one):
        within(f"3B logits, start {t}", g, w, 8e-5)
    assert np.array_equal(again[0].view(np.uint32), got_one[-1].view(np.uint32))


@pytest.mark.parametrize("cfg,seed,pos", [(SMALL_128, 11, 300), (GQA7, 12, 250)])
def test_steps_are_bit_reproducible(gpu, tmp_path, cfg, seed, pos):
    """Two steps from the same state give bit-identical logits, eager and
    through the captured graph: every sum has a fixed order (the output
    projection's block sums meet in an integer accumulator)."""
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = np.random.default_rng(seed).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    dec = make_decoder(gpu, path, max_seq=pos + 64)
    try:
        k, v = dec.kv()
        for l in range(cfg.n_layers):
            gpu.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
            gpu.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
        runs = []
        for _ in range(3):
            dec.set_pos(pos)
            _, a = dec.step(5, logits=True)
            _, b = dec.step(6, logits=True)
            runs.append(np.stack([a[0], b[0]]))
        toks = []
        for _ in range(2):
            dec.set_pos(pos)
            toks.append(dec.generate(5, 8)[:, 0].tolist())
    finally:
        dec.close()
    for r in runs[1:]:
        assert np.array_equal(r.view(np.uint32), runs[0].view(np.uint32))
    assert toks[0] == toks[1]


@pytest.mark.timeout(600)
def test_qwen2_7b_decode_at_position_1024(gpu, ref, tmp_path):
    """The full Qwen2-7B shape (28 layers, d_model 3584, 28/4 heads, ffn
    18944, Q4_K attn/gate/up, Q6_K down and untied Q6_K output 152064 x 3584)
    through the one-sequence step, KV cache prefilled to 1024 positions:
    greedy tokens equal the reference's forward (src/model.c:93-165) over four
    steps, and four distinct start tokens, one step each from the same cache,
    give its argmax and logits."""
    from dropin import prefilled_greedy
    cfg = mlf2.QWEN2_7B
    path = str(tmp_path / "qwen2_7b.mlf2")
    mlf2.write_qwen2(path, cfg, 60)
    pos, max_seq, steps = 1024, 1040, 4
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = np.random.default_rng(61).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    starts = [int(t) for t in np.random.default_rng(62).choice(cfg.vocab, 4, replace=False)]
    want, want_logits = prefilled_greedy(ref, path, kv, pos, start=starts[0], steps=steps, vocab=cfg.vocab,
                                         max_seq=max_seq)
    want_one = [prefilled_greedy(ref, path, kv, pos, start=t, steps=1, vocab=cfg.vocab, max_seq=max_seq)[1][0]
                for t in starts[1:]]
    assert np.all(np.isfinite(want_logits))
    dec = make_decoder(gpu, path, max_seq=max_seq)
    try:
        k, v = dec.kv()
        for l in range(cfg.n_layers):
            gpu.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
            gpu.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
        dec.set_pos(pos)
        first, lg = dec.step(starts[0], logits=True)
        got = [int(first[0])] + dec.generate(int(first[0]), steps - 1)[:, 0].tolist()
        got_one = []
        for t in starts[1:]:
            dec.set_pos(pos)
            nxt, l1 = dec.step(t, logits=True)
            assert int(nxt[0]) == int(np.argmax(l1[0]))
            got_one.append(l1[0])
    finally:
        dec.close()
    assert got == want
    # measured: 8.5e-6 (first start), 9.9e-6 .. 1.1e-5 over the other three
    within(f"7B logits, start {starts[0]}", lg[0], want_logits[0], 6e-5)
    assert [int(np.argmax(r)) for r in got_one] == [int(np.argmax(r)) for r in want_one]
    for t, g, w in zip(starts[1:], got_one, want_one):
        within(f"7B logits, start {t}", g, w, 6e-5)


# lane geometries: two rows per wave instruction (d_model 1792), four (1024,
# head_dim 128) and eight (512, head_dim 64, untied output)
@pytest.mark.parametrize("cfg", [GQA7, SMALL_128, TINY_UNTIED], ids=["gqa7", "small128", "tiny_untied"])
def test_gate_up_items_knob_gives_identical_steps(gpu, tmp_path, cfg):
    """The gate/up launch's grid (flat with 4 or 8 row items per wave, or the
    persistent grid with its prologue once per workgroup), the merge+o
    launch's rows per workgroup (64 or 128), the q/k/v launch's row items
    per wave (2, 4 or 8) and the attention's workgroups per query-head group
    (1, 2, 4 or 7; all by shape by default) change
    only which workgroup computes a row, never the order of a row's additions
    (the merge+o sums meet in an integer accumulator): three greedy steps give
    bit-identical logits either way."""
    path = str(tmp_path / "model.mlf2")
    mlf2.write_qwen2(path, cfg, 21)
    HAKO_TUNE_DEC_GU_ITEMS, HAKO_TUNE_DEC_GU_GRID, HAKO_TUNE_DEC_MERGE_ROWS, HAKO_TUNE_DEC_QKV_ITEMS = 9, 16, 17, 18
    HAKO_TUNE_DEC_ATTN_PARTS = 19
    runs = []
    try:
        for items, grid, mrows, qi, parts in ((4, 1, 64, 2, 4), (8, 1, 64, 4, 2), (0, 2, 64, 8, 7), (0, 2, 128, 2, 1)):
            gpu.tune(HAKO_TUNE_DEC_GU_ITEMS, items)
            gpu.tune(HAKO_TUNE_DEC_GU_GRID, grid)
            gpu.tune(HAKO_TUNE_DEC_MERGE_ROWS, mrows)
            gpu.tune(HAKO_TUNE_DEC_QKV_ITEMS, qi)
            gpu.tune(HAKO_TUNE_DEC_ATTN_PARTS, parts)
            dec = make_decoder(gpu, path, max_seq=64)
            try:
                tok, lg = 7, []
                for _ in range(3):
                    nxt, l1 = dec.step(tok, logits=True)
                    lg.append(l1[0].copy())
                    tok = int(nxt[0])
            finally:
                dec.close()
            runs.append(np.stack(lg))
    finally:
        gpu.tune(HAKO_TUNE_DEC_GU_ITEMS, 0)
        gpu.tune(HAKO_TUNE_DEC_GU_GRID, 0)
        gpu.tune(HAKO_TUNE_DEC_MERGE_ROWS, 0)
        gpu.tune(HAKO_TUNE_DEC_QKV_ITEMS, 0)
        gpu.tune(HAKO_TUNE_DEC_ATTN_PARTS, 0)
    assert np.all(np.isfinite(runs[0]))
    for r in runs[1:]:
        assert np.array_equal(runs[0].view(np.uint32), r.view(np.uint32))


# Per-layer mixes of weight types (the reference's matmul takes any type per
# tensor, src/nn.c:179-210): an output projection that is not Q4_K in some
# layers, the last layer's among them, and FFN matrices of other types.
MIXED_O = mlf2.Qwen2Config(n_layers=4, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768,
                           vocab=1024, ctx=256,
                           layer_types=(((1, "attn_output"), synth.TYPE_Q6_K), ((3, "attn_output"), synth.TYPE_F16)))
MIXED_FFN = mlf2.Qwen2Config(n_layers=3, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768,
                             vocab=1024, ctx=256, tied=False, embd_type=synth.TYPE_Q4_K,
                             layer_types=(((0, "attn_output"), synth.TYPE_F16), ((1, "ffn_gate"), synth.TYPE_Q6_K),
                                          ((1, "ffn_up"), synth.TYPE_Q6_K), ((2, "ffn_down"), synth.TYPE_Q4_K),
                                          ((2, "attn_v"), synth.TYPE_Q6_K)))


@pytest.mark.parametrize("cfg,seed,bar", [(MIXED_O, 25, 2e-5), (MIXED_FFN, 14, 2e-5)])
def test_mixed_layer_types_match_reference(gpu, ref, tmp_path, cfg, seed, bar):
    """Greedy tokens and logits of models whose layers differ in their
    matrices' types, eager steps and the captured graph, against the
    reference's forward."""
    from dropin import greedy
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    steps = 16
    want, want_logits = greedy(ref, path, start=3, steps=steps, vocab=cfg.vocab, max_seq=128)
    assert np.all(np.isfinite(want_logits))
    dec = make_decoder(gpu, path, max_seq=128)
    try:
        dec.set_pos(0)
        got, logits, tok = [], [], 3
        for _ in range(4):
            nxt, lg = dec.step(tok, logits=True)
            tok = int(nxt[0])
            got.append(tok)
            logits.append(lg[0])
        got += dec.generate(tok, steps - 4)[:, 0].tolist()
    finally:
        dec.close()
    assert got == want
    within(f"mixed-type logits {seed}", np.stack(logits), want_logits[:4], bar)


def plant(path: str, info: dict, name: str, where, value: float):
    """Overwrite one value of tensor `name` in an MLF2 file: element `where`
    of an F32 tensor, or the fp16 scale d of block (row, block) `where` of a
    Q4_K (bytes 0-1) or Q6_K (bytes 208-209) matrix."""
    qt, n_in, _, off, _ = info[name]
    f = mlf2.Mlf2File(path)
    base = f.header["data_off"] + off
    del f
    if qt == synth.TYPE_F32:
        at, data = base + 4 * where, np.float32(value).tobytes()
    else:
        r, b = where
        bsz = synth.Q4K_BYTES if qt == synth.TYPE_Q4_K else synth.Q6K_BYTES
        at = base + r * synth.row_nbytes(qt, n_in) + b * bsz + (0 if qt == synth.TYPE_Q4_K else 208)
        data = np.float16(value).tobytes()
    with open(path, "r+b") as fh:
        fh.seek(at)
        fh.write(data)


# (tensor, element or (row, block), value): NaN in norm weights and a bias
# (the q8 quantizer of the next Q4_K matmul maps NaN to code 0, so the
# reference's logits stay finite, or all turn NaN through the fp32 lm_head);
# a non-finite scale in an output projection block (NaN or +inf in the
# residual: every later logit NaN, token 0); NaN in one lm_head row (row 0:
# the reference's pick keeps index 0; row 7: NaN never wins).
NON_FINITE = [("blk.0.attn_norm.weight", 5, np.nan), ("blk.1.ffn_norm.weight", 100, np.nan),
              ("output_norm.weight", 7, np.nan), ("blk.1.attn_q.bias", 3, np.nan),
              ("blk.0.attn_output.weight", (5, 1), np.nan), ("blk.0.attn_output.weight", (9, 0), np.inf),
              ("blk.1.ffn_down.weight", (3, 1), np.inf),
              ("output.weight", (0, 0), np.nan), ("output.weight", (7, 1), np.nan)]


@pytest.mark.parametrize("name,where,value", NON_FINITE)
def test_non_finite_values_follow_reference(gpu, ref, tmp_path, name, where, value):
    """A non-finite weight value: the device step gives the reference's
    greedy tokens (src/sample.c:28-31), the same NaN and infinite logits,
    and the finite logits within the usual bar."""
    from dropin import greedy
    cfg = TINY_UNTIED
    path = str(tmp_path / "m.mlf2")
    info = mlf2.write_qwen2(path, cfg, 2)
    plant(path, info, name, where, value)
    want, want_logits = greedy(ref, path, start=3, steps=3, vocab=cfg.vocab, max_seq=64)
    dec = make_decoder(gpu, path, max_seq=64)
    try:
        dec.set_pos(0)
        got, logits, tok = [], [], 3
        for _ in range(3):
            nxt, lg = dec.step(tok, logits=True)
            tok = int(nxt[0])
            got.append(tok)
            logits.append(lg[0])
        dec.set_pos(0)
        replayed = dec.generate(3, 3)[:, 0].tolist()
    finally:
        dec.close()
    got_logits = np.stack(logits)
    print(f"[non-finite] {name} {where}: tokens {want}, NaN logits per step "
          f"{[int(n) for n in np.isnan(want_logits).sum(1)]}", flush=True)
    assert got == want and replayed == want
    assert np.array_equal(np.isnan(got_logits), np.isnan(want_logits))
    assert np.array_equal(np.isposinf(got_logits), np.isposinf(want_logits))
    assert np.array_equal(np.isneginf(got_logits), np.isneginf(want_logits))
    fin = np.isfinite(want_logits)
    if fin.any():
        within(f"finite logits, {name}", got_logits[fin], want_logits[fin], 3e-5)


@pytest.fixture(scope="module")
def ref_nofast():
    """The reference's sources built without -ffast-math (oracle/ref.mk): a
    second correct build, whose drift from the first measures how much a
    model amplifies differences in rounding order."""
    from dropin import bind_ctx
    from oracle.hako_oracle import REF_NOFAST_LIB
    return bind_ctx(C.CDLL(REF_NOFAST_LIB))


@pytest.mark.timeout(900)
@pytest.mark.parametrize("shape,seed", [("3b", 70), ("7b", 71)])
def test_full_shape_varied_tokens_teacher_forced(gpu, ref, ref_nofast, tmp_path, shape, seed):
    """The full Qwen2.5-3B / Qwen2-7B shapes with zero-mean Q4_K matrices
    (mlf2.Qwen2Config.centered; with uniform scale/min bytes a random model
    repeats one greedy token), KV cache prefilled to 1024 positions. Such a
    model amplifies every difference in rounding order: the reference's own
    build without -ffast-math drifts from it by ~1e-2 of the logit range
    within a few layers, more than many top-2 gaps, so no build need pick the
    same tokens. Each step is fed the reference's previous greedy token (16
    steps, tokens that change from step to step): the device's logits drift
    from the reference's no more than 4x the reference builds' drift from
    each other, and at every step the reference's pick is within that drift
    of the device's maximum."""
    import dataclasses
    from dropin import prefilled_greedy
    from oracle.hako_oracle import prefilled_forced, ref_greedy_pick
    cfg = dataclasses.replace(mlf2.QWEN2_3B if shape == "3b" else mlf2.QWEN2_7B, centered=True)
    path = str(tmp_path / f"qwen2_{shape}_centered.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    pos, max_seq, steps = 1024, 1048, 16
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = np.random.default_rng(seed + 1).standard_normal((2, cfg.n_layers, pos, kvd)).astype(np.float32)
    want, want_logits = prefilled_greedy(ref, path, kv, pos, start=11, steps=steps, vocab=cfg.vocab,
                                         max_seq=max_seq)
    assert len(set(want)) >= steps // 2, want     # not one repeated token
    fed = [11] + want[:-1]
    nf_logits = prefilled_forced(ref_nofast, path, kv, pos, fed, cfg.vocab, max_seq)
    dec = make_decoder(gpu, path, max_seq=max_seq)
    try:
        k, v = dec.kv()
        for l in range(cfg.n_layers):
            gpu.h2d(k + dec.kv_offset(0, l, 0), kv[0, l])
            gpu.h2d(v + dec.kv_offset(0, l, 0), kv[1, l])
        dec.set_pos(pos)
        got, logits = [], []
        for t in fed:
            nxt, lg = dec.step(t, logits=True)
            got.append(int(nxt[0]))
            logits.append(lg[0])
    finally:
        dec.close()
    err_dev = max(maxabs_rel(g, w) for g, w in zip(logits, want_logits))
    err_nf = max(maxabs_rel(g, w) for g, w in zip(nf_logits, want_logits))
    nf_picks = [ref_greedy_pick(l) for l in nf_logits]
    print(f"[drift] {shape} centered: device {err_dev:.3e}, reference without fast-math {err_nf:.3e}; "
          f"picks equal to the reference's: device {sum(a == b for a, b in zip(got, want))}/{steps}, "
          f"reference without fast-math {sum(a == b for a, b in zip(nf_picks, want))}/{steps}", flush=True)
    assert err_dev <= 4 * max(err_nf, 1e-5)
    assert near_max_steps(logits, want, want_logits, 2 * max(err_nf, err_dev)) == []
