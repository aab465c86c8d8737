"""Prompt prefill through the model (hako_gpu_decoder_prefill) against the
reference's feed (src/hakm_api.c:105-111: one hakm_forward per prompt token,
src/model.c:93-165, compiled from its sources) followed by greedy decoding.

Bars: the greedy tokens after the prompt identical; the KV cache rows the
prompt writes and the last prompt token's logits within a max-abs-normalised
bar set per case at most 5x the value measured on MI355X (logits 2e-7 ..
4e-6; cache rows of the deeper layer up to 1e-3, where the q8
re-quantization of an activation that differs in its last bit flips one int8
value of a row). Cache rows that differ by more than 1e-5 are held to twice
the drift of the reference's own build without -ffast-math on the same feed.
"""
import ctypes as C

import numpy as np
import pytest

from hako_amd import mlf2, synth
from helpers import within

pytestmark = pytest.mark.gpu

TINY = mlf2.Qwen2Config(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512,
                        vocab=1024, ctx=40000)
TINY_UNTIED = mlf2.Qwen2Config(n_layers=2, d_model=512, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=768,
                               vocab=768, ctx=256, tied=False, embd_type=synth.TYPE_Q4_K)
SMALL_128 = mlf2.Qwen2Config(n_layers=3, d_model=1024, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=2816,
                             vocab=4096, ctx=512)
# dense weight types: the generic multi-token matmuls
DENSE = mlf2.Qwen2Config(n_layers=1, d_model=256, n_heads=2, n_kv_heads=1, head_dim=128, ffn_dim=512, vocab=640,
                         ctx=256, attn_type=synth.TYPE_F16, gate_up_type=synth.TYPE_F32, down_type=synth.TYPE_Q4_K,
                         embd_type=synth.TYPE_F16)


@pytest.fixture(scope="module")
def ref():
    from dropin import bind_ctx
    from oracle.hako_oracle import REF_LIB
    return bind_ctx(C.CDLL(REF_LIB))


class RefSeq:
    """One reference context fed token by token."""

    def __init__(self, lib, path, max_seq, cfg):
        from oracle.hako_oracle import HakmCtx
        self.lib, self.cfg, self.max_seq = lib, cfg, max_seq
        self.ctx = lib.hakm_ctx_new(path.encode(), max_seq)
        assert self.ctx
        self.c = HakmCtx.from_address(self.ctx)

    def forward(self, tok):
        p = self.lib.hakm_forward(self.ctx, int(tok))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), shape=(self.cfg.vocab,)).copy()

    def feed(self, toks):
        lg = None
        for t in toks:
            lg = self.forward(t)
        return lg

    def greedy(self, lg, steps):
        out = []
        for _ in range(steps):
            out.append(int(np.argmax(lg)))
            lg = self.forward(out[-1])
        return out

    def fill(self, kv, pos):
        """Write kv[0] / kv[1] ([n_layers][pos][kv_dim]) at positions 0..pos-1 and set the position."""
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        shape = (self.cfg.n_layers, self.max_seq, kvd)
        for which, ptr in ((0, self.c.k_cache), (1, self.c.v_cache)):
            np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=shape)[:, :pos] = kv[which]
        self.c.pos = pos

    def kv(self, upto, start=0):
        kvd = self.cfg.n_kv_heads * self.cfg.head_dim
        shape = (self.cfg.n_layers, self.max_seq, kvd)
        k = np.ctypeslib.as_array(C.cast(self.c.k_cache, C.POINTER(C.c_float)), shape=shape)[:, start:upto].copy()
        v = np.ctypeslib.as_array(C.cast(self.c.v_cache, C.POINTER(C.c_float)), shape=shape)[:, start:upto].copy()
        return k, v

    def close(self):
        self.lib.hakm_ctx_free(self.ctx)


def device_kv(gpu, dec, seq, upto, start=0):
    k, v = dec.kv()
    kvd = dec.kv_dim
    out = []
    for base in (k, v):
        out.append(np.stack([gpu.download(base + dec.kv_offset(seq, l, start), np.float32, (upto - start, kvd))
                             for l in range(dec.cfg["n_layers"])]))
    return out


def fill_device_kv(gpu, dec, seq, kv, pos):
    k, v = dec.kv()
    for l in range(dec.cfg["n_layers"]):
        gpu.h2d(k + dec.kv_offset(seq, l, 0), np.ascontiguousarray(kv[0, l, :pos]))
        gpu.h2d(v + dec.kv_offset(seq, l, 0), np.ascontiguousarray(kv[1, l, :pos]))


def make(gpu, path, n_seq, max_seq):
    from hako_amd.decoder import Decoder
    return Decoder(gpu, path, n_seq=n_seq, max_seq=max_seq)


# The reference's forward keeps the attention scores of a head in its
# ffn_dim-float gate buffer (src/model.c:123-124, "needs pos+1 <= F"): a
# context longer than ffn_dim overruns its heap, so long prompts run on a
# model whose ffn_dim covers them.
TINY_LONG = mlf2.Qwen2Config(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=1024,
                             vocab=1024, ctx=40000)


# a prompt fed at position 9000 of a 10000-position context: four KV heads of
# head_dim 128 make a 512-token pass's attention records 1.3 GB there (more
# than the 1 GiB record buffer); ffn_dim 9728 covers the positions (the
# reference scores in its gate buffer)
LONG_CTX = mlf2.Qwen2Config(n_layers=1, d_model=512, n_heads=4, n_kv_heads=4, head_dim=128, ffn_dim=9728,
                            vocab=512, ctx=10000)


# (cfg, seed, prompt length, max_seq, start position, K/V bar, logits bar):
# 600 tokens cross a 512-token pass. The pass's attention records are sized
# by the positions it reaches: from position 0 with max_seq 40000, 300 tokens
# are one pass; from position 9000 of LONG_CTX a 512-token pass would need
# 1.3 GB of records (more than the 1 GiB buffer), so the 600 tokens go as
# 256 + 256 + 88. Measured K/V: 2.7e-7, 3.0e-7, 1.4e-4, 2.4e-7, 1.1e-3, 4.4e-4,
# 3.2e-7; logits 4.6e-7, 5.1e-7, 6.0e-7, 3.5e-7, 2.6e-7, 4.2e-7, 5.8e-7.
@pytest.mark.parametrize("cfg,seed,n_prompt,max_seq,pos0,kv_bar,lg_bar", [
    (TINY, 1, 37, 384, 0, 1.4e-6, 2.3e-6), (TINY_UNTIED, 2, 50, 384, 0, 1.5e-6, 2.6e-6),
    (SMALL_128, 3, 140, 384, 0, 3.8e-4, 3e-6), (DENSE, 4, 21, 384, 0, 1.2e-6, 1.8e-6),
    (TINY_LONG, 5, 600, 640, 0, 5.3e-3, 1.3e-6), (TINY, 6, 300, 40000, 0, 2.2e-3, 2.1e-6),
    (LONG_CTX, 12, 600, 10000, 9000, 1.6e-6, 2.9e-6)])
def test_prefill_matches_reference_feed(gpu, ref, tmp_path, cfg, seed, n_prompt, max_seq, pos0, kv_bar, lg_bar):
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    steps = 8
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, cfg.vocab, n_prompt).astype(np.int32)
    kvd = cfg.n_kv_heads * cfg.head_dim
    kv = rng.standard_normal((2, cfg.n_layers, pos0, kvd), dtype=np.float32)
    end = pos0 + n_prompt
    r = RefSeq(ref, path, max_seq, cfg)
    try:
        r.fill(kv, pos0)
        want_lg = r.feed(prompt)
        want_k, want_v = r.kv(end, pos0)
        want = r.greedy(want_lg, steps)
    finally:
        r.close()
    dec = make(gpu, path, 1, max_seq)
    try:
        fill_device_kv(gpu, dec, 0, kv, pos0)
        dec.set_pos(pos0)
        first, lg = dec.prefill(prompt, logits=True)
        got_k, got_v = device_kv(gpu, dec, 0, end, pos0)
        got = [first] + dec.generate(first, steps - 1)[:, 0].tolist()
    finally:
        dec.close()
    assert first == int(np.argmax(lg))
    err_k = within(f"prefill K {cfg.d_model}/{n_prompt}/{max_seq}/{pos0}", got_k, want_k, kv_bar)
    err_v = within(f"prefill V {cfg.d_model}/{n_prompt}/{max_seq}/{pos0}", got_v, want_v, kv_bar)
    within(f"prefill logits {cfg.d_model}/{n_prompt}/{max_seq}/{pos0}", lg, want_lg, lg_bar)
    assert got == want
    if max(err_k, err_v) > 1e-5:
        # cache rows beyond float noise: the reference's own build without
        # -ffast-math (the same arithmetic in another rounding order) drifts
        # as far on the same feed, i.e. the size is the model's sensitivity
        # to one int8 of a q8 row rounded the other way
        from dropin import bind_ctx
        from helpers import maxabs_rel
        from oracle.hako_oracle import REF_NOFAST_LIB
        rn = RefSeq(bind_ctx(C.CDLL(REF_NOFAST_LIB)), path, max_seq, cfg)
        try:
            rn.fill(kv, pos0)
            rn.feed(prompt)
            nf_k, nf_v = rn.kv(end, pos0)
        finally:
            rn.close()
        err_nf = max(maxabs_rel(nf_k, want_k), maxabs_rel(nf_v, want_v))
        print(f"[drift] prefill cache rows: device {max(err_k, err_v):.2e}, reference without fast-math "
              f"{err_nf:.2e}", flush=True)
        assert max(err_k, err_v) <= 2 * err_nf


HAKO_TUNE_Q6K_GEMM_TN, HAKO_TUNE_Q6K_GEMM_SK = 13, 15


def test_prefill_stream_k_down_matches_reference_feed(gpu, ref, tmp_path):
    """The down projection's Q6_K GEMM in its stream-K form inside the prompt
    pass (128-row tiles forced: 3 x 8 tiles of 11 super-blocks over the
    grid, so every tile's K is split over many workgroups and the fixup adds
    the pieces into the residual) against whole tiles and the reference's
    feed: the same greedy tokens, K/V rows and logits within the bars of the
    SMALL_128 case above."""
    cfg, seed, n_prompt, max_seq = SMALL_128, 21, 140, 384
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, seed)
    steps = 6
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, n_prompt).astype(np.int32)
    r = RefSeq(ref, path, max_seq, cfg)
    try:
        want_lg = r.feed(prompt)
        want_k, want_v = r.kv(n_prompt)
        want = r.greedy(want_lg, steps)
    finally:
        r.close()
    got = {}
    gpu.tune(HAKO_TUNE_Q6K_GEMM_TN, 128)
    try:
        for sk in (0, 1):
            gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, sk)
            dec = make(gpu, path, 1, max_seq)
            try:
                dec.set_pos(0)
                first, lg = dec.prefill(prompt, logits=True)
                k, v = device_kv(gpu, dec, 0, n_prompt)
                toks = [first] + dec.generate(first, steps - 1)[:, 0].tolist()
            finally:
                dec.close()
            got[sk] = (lg, k, v, toks)
    finally:
        gpu.tune(HAKO_TUNE_Q6K_GEMM_TN, 0)
        gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, 1)
    for sk, (lg, k, v, toks) in got.items():
        within(f"stream-K {sk} K", k, want_k, 3.8e-4)
        within(f"stream-K {sk} V", v, want_v, 3.8e-4)
        within(f"stream-K {sk} logits", lg, want_lg, 3e-6)
        assert toks == want, sk


# head_dim 64 takes the chunk-record attention, head_dim 128 (SMALL_128) the
# matrix-core prompt attention, here for a pass that starts past position 0
# (measured K/V 2.4e-7, 1.1e-4; logits 3.1e-7, 4.6e-7)
@pytest.mark.parametrize("cfg,kv_bar,lg_bar", [(TINY, 2.6e-3, 2e-6), (SMALL_128, 6e-4, 3e-6)])
def test_prefill_after_decode_steps(gpu, ref, tmp_path, cfg, kv_bar, lg_bar):
    """Prompt, three decode steps, a second prompt at the new position, then
    greedy decoding: as the reference fed the same tokens one by one; the
    second prompt's K/V rows and last logits against the reference's."""
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, 7)
    rng = np.random.default_rng(7)
    p1, p2 = rng.integers(0, cfg.vocab, 20), rng.integers(0, cfg.vocab, 45)
    at = len(p1) + 3
    r = RefSeq(ref, path, 128, cfg)
    try:
        lg = r.feed(p1)
        fed = r.greedy(lg, 3)                 # tokens fed by the three steps
        want_lg = r.feed(p2)
        want_k, want_v = r.kv(at + len(p2), at)
        want = r.greedy(want_lg, 5)
    finally:
        r.close()
    dec = make(gpu, path, 1, 128)
    try:
        dec.set_pos(0)
        t = dec.prefill(p1)
        steps = []
        for _ in range(3):
            steps.append(t)
            t = int(dec.step(t)[0])
        nxt, lg = dec.prefill(p2, logits=True)
        got_k, got_v = device_kv(gpu, dec, 0, at + len(p2), at)
        got = [nxt] + dec.generate(nxt, 4)[:, 0].tolist()
    finally:
        dec.close()
    assert steps == fed
    within(f"continued prompt K {cfg.head_dim}", got_k, want_k, kv_bar)
    within(f"continued prompt V {cfg.head_dim}", got_v, want_v, kv_bar)
    within(f"continued prompt logits {cfg.head_dim}", lg, want_lg, lg_bar)
    assert got == want


# measured K/V 2.9e-7, 1.2e-4 (worst sequence)
@pytest.mark.parametrize("cfg,kv_bar", [(TINY, 2e-6), (SMALL_128, 6e-4)])
def test_prefill_sequences_of_a_batched_decoder(gpu, ref, tmp_path, cfg, kv_bar):
    """Four sequences, each prefilled with its own prompt length, then decoded
    together: every sequence as the reference's own context, and every
    sequence's K/V rows (each in its own slice of the caches) as the
    reference's."""
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, 8)
    rng = np.random.default_rng(8)
    prompts = [rng.integers(0, cfg.vocab, n) for n in (10, 25, 3, 140)]
    steps = 6
    dec = make(gpu, path, 4, 256)
    try:
        dec.set_pos([0, 0, 0, 0])
        firsts = [dec.prefill(p, seq=s) for s, p in enumerate(prompts)]
        kvs = [device_kv(gpu, dec, s, len(p)) for s, p in enumerate(prompts)]
        got = np.concatenate([np.array(firsts)[None], dec.generate(np.array(firsts), steps - 1)])
    finally:
        dec.close()
    for s, p in enumerate(prompts):
        r = RefSeq(ref, path, 256, cfg)
        try:
            want = r.greedy(r.feed(p), steps)
            want_k, want_v = r.kv(len(p))
        finally:
            r.close()
        within(f"sequence {s} prompt K {cfg.head_dim}", kvs[s][0], want_k, kv_bar)
        within(f"sequence {s} prompt V {cfg.head_dim}", kvs[s][1], want_v, kv_bar)
        assert got[:, s].tolist() == want, f"sequence {s}"


def test_prefill_qwen2_3b_prompt(gpu, ref, tmp_path):
    """The full Qwen2.5-3B shape: a 150-token prompt, last logits and three
    greedy tokens against the reference's feed."""
    cfg = mlf2.QWEN2_3B
    path = str(tmp_path / "qwen2_3b.mlf2")
    mlf2.write_qwen2(path, cfg, 32)
    prompt = np.random.default_rng(32).integers(0, cfg.vocab, 150)
    r = RefSeq(ref, path, 160, cfg)
    try:
        want_lg = r.feed(prompt)
        want = r.greedy(want_lg, 3)
    finally:
        r.close()
    dec = make(gpu, path, 1, 160)
    try:
        dec.set_pos(0)
        first, lg = dec.prefill(prompt, logits=True)
        got = [first] + dec.generate(first, 2)[:, 0].tolist()
    finally:
        dec.close()
    within("prefill 3B logits", lg, want_lg, 1.7e-5)   # measured 3.5e-6
    assert got == want


def test_prefill_qwen2_3b_prompt_varied_tokens(gpu, ref, tmp_path):
    """The full Qwen2.5-3B shape with zero-mean Q4_K matrices (a random model
    whose greedy tokens change from step to step and which amplifies every
    difference in rounding order): a 150-token prompt in one pass, then 8
    steps each fed the reference's previous greedy token. The device's logits
    drift from the reference's no more than 4x the reference's own build
    without -ffast-math does, and at every step the reference's pick is
    within that drift of the device's maximum."""
    import dataclasses
    from dropin import bind_ctx
    from helpers import maxabs_rel
    from oracle.hako_oracle import REF_NOFAST_LIB
    ref_nofast = bind_ctx(C.CDLL(REF_NOFAST_LIB))
    cfg = dataclasses.replace(mlf2.QWEN2_3B, centered=True)
    path = str(tmp_path / "qwen2_3b_centered.mlf2")
    mlf2.write_qwen2(path, cfg, 33)
    prompt = np.random.default_rng(33).integers(0, cfg.vocab, 150)
    r, rn = RefSeq(ref, path, 168, cfg), RefSeq(ref_nofast, path, 168, cfg)
    try:
        lg = r.feed(prompt)
        nlg = rn.feed(prompt)
        want, want_lg, nf_lg = [], [lg], [nlg]
        for _ in range(8):
            want.append(int(np.argmax(lg)))
            lg = r.forward(want[-1])
            nf_lg.append(rn.forward(want[-1]))
            want_lg.append(lg)
    finally:
        r.close()
        rn.close()
    assert len(set(want)) >= 4, want
    dec = make(gpu, path, 1, 168)
    try:
        dec.set_pos(0)
        first, lg = dec.prefill(prompt, logits=True)
        got, logits = [first], [lg]
        for t in want:
            nxt, l1 = dec.step(t, logits=True)
            got.append(int(nxt[0]))
            logits.append(l1[0])
    finally:
        dec.close()
    from helpers import near_max_steps
    err_dev = max(maxabs_rel(g, w) for g, w in zip(logits, want_lg))
    err_nf = max(maxabs_rel(g, w) for g, w in zip(nf_lg, want_lg))
    print(f"[drift] 3B prompt centered: device {err_dev:.3e}, reference without fast-math {err_nf:.3e}; "
          f"picks equal to the reference's {sum(a == b for a, b in zip(got, want))}/8", flush=True)
    assert err_dev <= 4 * max(err_nf, 1e-5)
    assert near_max_steps(logits[:8], want, want_lg[:8], 2 * max(err_nf, err_dev)) == []


@pytest.mark.timeout(900)
def test_prefill_qwen2_7b_512_token_prompt(gpu, ref, tmp_path):
    """The benchmarked prompt workload: the full Qwen2-7B shape (28 layers,
    28/4 heads, ffn 18944, Q4_K attn/gate/up, Q6_K down and untied output), a
    512-token prompt from position 0 in one pass (the q/k/v, gate/up and
    residual GEMM epilogues at 3584 + 512 + 512 and 2 x 18944 rows, the prompt
    attention at 7 query heads per KV head). Against the reference's feed,
    one hakm_forward per token: the last logits, the K/V rows of layers 0
    and 27, and three greedy tokens."""
    cfg = mlf2.QWEN2_7B
    path = str(tmp_path / "qwen2_7b.mlf2")
    mlf2.write_qwen2(path, cfg, 50)
    n = 512
    prompt = np.random.default_rng(50).integers(0, cfg.vocab, n)
    r = RefSeq(ref, path, n + 8, cfg)
    try:
        want_lg = r.feed(prompt)
        want_k, want_v = r.kv(n)
        want = r.greedy(want_lg, 3)
    finally:
        r.close()
    dec = make(gpu, path, 1, n + 8)
    try:
        dec.set_pos(0)
        first, lg = dec.prefill(prompt, logits=True)
        got_k, got_v = device_kv(gpu, dec, 0, n)
        got = [first] + dec.generate(first, 2)[:, 0].tolist()
    finally:
        dec.close()
    for l in (0, cfg.n_layers - 1):
        within(f"7B prompt K layer {l}", got_k[l], want_k[l], 5e-3)
        within(f"7B prompt V layer {l}", got_v[l], want_v[l], 5e-3)
    within("7B prompt logits", lg, want_lg, 1e-4)
    assert got == want


def test_prefill_rejects_bad_use(gpu, tmp_path):
    from hako_amd.gpu import HakoGpuError
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, TINY, 9)
    dec = make(gpu, path, 2, 32)
    try:
        dec.set_pos([0, 30])
        with pytest.raises(HakoGpuError, match="no room"):
            dec.prefill([1, 2, 3], seq=1)
        with pytest.raises(HakoGpuError, match="sequence 2"):
            dec.prefill([1], seq=2)
        with pytest.raises(HakoGpuError, match="vocabulary"):
            dec.prefill([1, TINY.vocab], seq=0)
        assert isinstance(dec.prefill([1, 2, 3], seq=0), int)
    finally:
        dec.close()


def test_prefill_of_one_token_equals_a_step(gpu, tmp_path):
    """A one-token prompt is one forward: the same logits as a decode step
    from the same state (the pass's matmuls are the single-token GEMVs)."""
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, SMALL_128, 10)
    dec = make(gpu, path, 1, 64)
    try:
        dec.set_pos(0)
        t = dec.prefill([5, 6, 7])
        _, a = dec.prefill([t], logits=True)
        dec.set_pos(0)
        dec.prefill([5, 6, 7])
        _, b = dec.step(t, logits=True)
    finally:
        dec.close()
    # the pass's single-token matmuls against the step's fused kernels: measured 4.2e-7
    within("one-token prefill vs step logits", a, b[0], 2e-6)


def test_prefill_fills_the_cache_to_max_seq(gpu, ref, tmp_path):
    """A prompt that ends exactly at max_seq: the last position is written,
    the logits are the reference's, and no further step fits."""
    from hako_amd.gpu import HakoGpuError
    cfg = TINY
    path = str(tmp_path / "m.mlf2")
    mlf2.write_qwen2(path, cfg, 11)
    max_seq = 96
    prompt = np.random.default_rng(11).integers(0, cfg.vocab, max_seq)
    r = RefSeq(ref, path, max_seq, cfg)
    try:
        want_lg = r.feed(prompt)
    finally:
        r.close()
    dec = make(gpu, path, 1, max_seq)
    try:
        dec.set_pos(0)
        _, lg = dec.prefill(prompt, logits=True)
        with pytest.raises(HakoGpuError, match="no room"):
            dec.step(1)
    finally:
        dec.close()
    within("prefill to max_seq logits", lg, want_lg, 1.6e-6)   # measured 3.2e-7
