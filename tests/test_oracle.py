"""Pins the CPU oracle (oracle/hako_oracle.c) before anything is checked against it.

Each reference function the oracle restates is pinned by at least one check
that a plausible slip (wrong nibble, wrong index, transposed operand, the
source-text rounding of the q8 scale) would fail:

* golden vectors written by the reference's own compiled C (tests/golden/);
* closed forms and one-hot structure checks derived from the block layouts;
* exhaustive enumeration where the domain is small (fp16, 6-bit scales).
"""
import numpy as np
import pytest

from hako_amd import synth
from helpers import maxabs_rel


# ── f16_to_f32 (reference quant.c:31-54) ──

def test_f16_exhaustive_matches_ieee(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ── get_scale_min_k4 (reference quant.c:57-66) ──

def pack_scale_min(s, m):
    """Inverse of the 12-byte 6-bit packing: sub-blocks 0-3 in the low six
    bits of bytes j (scale) and j+4 (min); sub-blocks 4-7 as nibbles of byte
    j+4 (scale low, min high) plus their top two bits in bytes j-4 / j."""
    b = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            b[j] |= s[j] & 63
            b[j + 4] |= m[j] & 63
        else:
            b[j + 4] |= (s[j] & 15) | ((m[j] & 15) << 4)
            b[j - 4] |= (s[j] >> 4) << 6
            b[j] |= (m[j] >> 4) << 6
    return b


def test_scale_min_exhaustive_per_field(oracle):
    """Every 6-bit value in every one of the 16 (scale, min) fields decodes to
    itself: d=1, dmin=0, all nibbles 1 gives y = s of the sub-block; d=0,
    dmin=1 gives y = -m."""
    rng = np.random.default_rng(1)
    for v in range(64):
        for field in range(16):
            s = rng.integers(0, 64, 8)
            m = rng.integers(0, 64, 8)
            (s if field < 8 else m)[field % 8] = v
            blk = np.zeros(144, np.uint8)
            blk[4:16] = pack_scale_min(s, m)
            blk[16:] = 0x11
            blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
            y = oracle.dequant(synth.TYPE_Q4_K, blk, 256).reshape(8, 32)
            assert np.array_equal(y, np.repeat(s.astype(np.float32)[:, None], 32, 1))
            blk[0:2] = 0
            blk[2:4] = np.array([1.0], np.float16).view(np.uint8)
            y = oracle.dequant(synth.TYPE_Q4_K, blk, 256).reshape(8, 32)
            assert np.array_equal(y, np.repeat(-m.astype(np.float32)[:, None], 32, 1))


# ── dequant_q4_K / dequant_q6_K (reference quant.c:68-123) ──

def test_q4k_dequant_golden(oracle, golden):
    g = golden("q4k_dequant.npz")
    got = oracle.dequant(synth.TYPE_Q4_K, g["blocks"], g["blocks"].shape[0] * 256)
    assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))


def test_q6k_dequant_golden(oracle, golden):
    g = golden("q6k_dequant.npz")
    got = oracle.dequant(synth.TYPE_Q6_K, g["blocks"], g["blocks"].shape[0] * 256)
    assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))


def test_q4k_one_hot_positions(oracle):
    """Nibble k of qs lands at weight 64*(k//32) + k%32 (low) or +32 (high)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[4:16] = pack_scale_min(np.ones(8, int), np.zeros(8, int))
    for k in range(128):
        for shift, off in ((0, 0), (4, 32)):
            b = blk.copy()
            b[16 + k] = 1 << shift
            y = oracle.dequant(synth.TYPE_Q4_K, b, 256)
            want = np.zeros(256, np.float32)
            want[64 * (k // 32) + off + k % 32] = 1.0
            assert np.array_equal(y, want), (k, shift)


def test_q6k_one_hot_positions(oracle):
    """A single ql nibble or qh bit pair moves exactly one weight, at
    128n + 32k + l, with scale index 8n + 2k + l//16."""
    blk = np.zeros(210, np.uint8)
    blk[208:210] = np.array([1.0], np.float16).view(np.uint8)
    blk[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    base = oracle.dequant(synth.TYPE_Q6_K, blk, 256)
    sc = np.arange(1, 17)
    for n in range(2):
        for k in range(4):
            for l in range(32):
                e = 128 * n + 32 * k + l
                assert base[e] == -32 * sc[8 * n + 2 * k + l // 16]
                b = blk.copy()
                b[64 * n + 32 * (k & 1) + l] = 1 << (4 if k >= 2 else 0)
                d = oracle.dequant(synth.TYPE_Q6_K, b, 256) - base
                assert np.count_nonzero(d) == 1 and d[e] == sc[8 * n + 2 * k + l // 16]
                b = blk.copy()
                b[128 + 32 * n + l] = 1 << (2 * k)
                d = oracle.dequant(synth.TYPE_Q6_K, b, 256) - base
                assert np.count_nonzero(d) == 1 and d[e] == 16 * sc[8 * n + 2 * k + l // 16]


def test_dequant_closed_form_exact(oracle):
    """Q4_K y = d*s*q - dmin*m and Q6_K y = d*sc*(q-32) with exact products:
    the fp64 evaluation rounded once equals the oracle bit for bit."""
    rng = np.random.default_rng(7)
    b4 = synth.q4k_blocks(rng, 64)
    y = oracle.dequant(synth.TYPE_Q4_K, b4, 64 * 256).reshape(64, 256)
    for i in range(64):
        d = float(b4[i, 0:2].view(np.float16)[0]); dm = float(b4[i, 2:4].view(np.float16)[0])
        for e in range(0, 256, 37):
            g, h, l = e // 64, (e // 32) % 2, e % 32
            j = 2 * g + h
            sc = b4[i, 4:16]
            if j < 4:
                s, m = sc[j] & 63, sc[j + 4] & 63
            else:
                s = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4)
                m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
            q = (b4[i, 16 + 32 * g + l] >> (4 * h)) & 15
            assert y[i, e] == np.float32(d * s * q - dm * m)


# ── quantize_row_q8_32 (reference quant.c:127-144, compiled form) ──

def test_q8_golden_bit_exact(oracle, golden):
    g = golden("q8.npz")
    for r in range(g["x"].shape[0]):
        xq, xs = oracle.quantize_q8_32(g["x"][r])
        assert np.array_equal(xq, g["xq"][r]), r
        assert np.array_equal(xs.view(np.uint32), g["xs"][r].view(np.uint32)), r


def q8_non_finite_rows() -> np.ndarray:
    """32-blocks holding NaN and infinities in the places that matter to the
    quantizer's maximum and codes: one NaN (first, middle, last), a block of
    NaNs, +inf, -inf, both, NaN with inf, and a block of infinities."""
    rng = np.random.default_rng(77)
    rows = rng.standard_normal((10, 64)).astype(np.float32)
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows[0, 0] = nan
    rows[1, 17] = nan
    rows[2, 31] = nan
    rows[3, :32] = nan
    rows[4, 5] = inf
    rows[5, 40] = -inf
    rows[6, 3], rows[6, 9] = inf, -inf
    rows[7, 3], rows[7, 9] = nan, inf
    rows[8, 32:] = inf
    rows[9, :] = nan
    return rows


def test_q8_non_finite_matches_compiled_reference(oracle):
    """NaN and infinite inputs: the oracle's codes and scales against the
    reference's compiled quantize_row_q8_32 (a NaN never enters the block
    maximum; a non-finite product converts to code 0; an infinite maximum
    gives an infinite scale)."""
    from oracle.hako_oracle import RefLib
    ref = RefLib()
    for r, x in enumerate(q8_non_finite_rows()):
        wq, ws = ref.quantize_q8_32(x)
        oq, os_ = oracle.quantize_q8_32(x)
        assert np.array_equal(oq, wq), r
        assert np.array_equal(os_.view(np.uint32), ws.view(np.uint32)), r


def test_q8_known_answer():
    """amax 0x400861D9: the compiled form gives xs 0x3C8974C2."""
    from oracle.hako_oracle import Oracle
    x = np.zeros(32, np.float32)
    x[3] = np.array([0x400861D9], np.uint32).view(np.float32)[0]
    _, xs = Oracle().quantize_q8_32(x)
    assert xs.view(np.uint32)[0] == 0x3C8974C2


def test_q8_golden_rejects_source_text_rounding(golden):
    """The literal reading (scale = amax/127, inv = 1/scale) is a plausible
    slip; the golden vectors must tell it apart from the compiled rounding."""
    g = golden("q8.npz")
    x = g["x"][:6].reshape(-1, 32).astype(np.float32)
    amax = np.abs(x).max(axis=1)
    scale = (amax / np.float32(127)).astype(np.float32)
    assert np.count_nonzero(scale.view(np.uint32) != g["xs"][:6].reshape(-1).view(np.uint32)) > 0


# ── q4k_vec_dot integer sums and fold (reference quant.c:150-232) ──

def test_q4k_isums_golden(oracle, golden):
    g = golden("q4k_isums.npz")
    for n_in in (2048, 3584):
        w, xq = g[f"w_{n_in}"], g[f"xq_{n_in}"]
        iqx, ix = oracle.q4k_isums(w, xq, w.shape[0], n_in)
        assert np.array_equal(iqx, g[f"iqx_{n_in}"])
        assert np.array_equal(ix, g[f"ix_{n_in}"])


def test_q4k_isums_brute_force(oracle):
    """Σq·xq by dequantizing with d=1, s=1, dmin=0 and dotting in int64."""
    rng = np.random.default_rng(3)
    w = synth.q4k_weight(rng, 3, 1024)
    xq = rng.integers(-127, 128, 1024).astype(np.int8)
    iqx, ix = oracle.q4k_isums(w, xq, 3, 1024)
    for r in range(3):
        b = w[r].reshape(4, 144).copy()
        b[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
        b[:, 2:4] = 0
        b[:, 4:16] = pack_scale_min(np.ones(8, int), np.zeros(8, int))
        q = oracle.dequant(synth.TYPE_Q4_K, b, 1024).astype(np.int64)
        want = (q * xq).reshape(-1, 32).sum(1)
        assert np.array_equal(iqx[r], want)
        assert np.array_equal(ix[r], xq.astype(np.int64).reshape(-1, 32).sum(1))


def test_q4k_dot_golden(oracle, golden):
    g = golden("q4k_dot.npz")
    xq, xs = oracle.quantize_q8_32(g["x"])
    got = np.array([oracle.q4k_vec_dot(g["w"][r], 2048, xq, xs) for r in range(16)])
    assert maxabs_rel(got, g["out"]) < 1e-6
    got64 = np.array([oracle.q4k_vec_dot(g["w"][r], 2048, xq, xs, f64=True) for r in range(16)])
    assert maxabs_rel(got64, g["out"]) < 1e-6


# ── matmul (reference nn.c:179-210) ──

@pytest.mark.parametrize("name", ["q4k", "q6k", "q6k_long", "f16", "f32"])
def test_matmul_golden(oracle, golden, name):
    g = golden("matmul.npz")
    qt, n_out, n_in = (int(v) for v in g[f"{name}_shape"])
    bias = g.get(f"{name}_bias")
    # The fp64 fold sits within the reference's own fp32 rounding of the
    # truth; the oracle's sequential fp32 order drifts further on long rows
    # (11008 terms) but stays inside the 1e-5 parity bound.
    for f64, tol in ((True, 2e-6), (False, 1e-5)):
        got = oracle.matmul(qt, g[f"{name}_w"], g[f"{name}_x"], n_out, n_in, bias=bias, f64=f64)
        assert maxabs_rel(got, g[f"{name}_out"]) < tol, (name, f64)


def test_matmul_batch_equals_rows(oracle):
    rng = np.random.default_rng(5)
    w = synth.q4k_weight(rng, 40, 512)
    x = synth.activation(rng, 512, rows=3)
    out = oracle.matmul(synth.TYPE_Q4_K, w, x, 40, 512)
    for t in range(3):
        assert np.array_equal(out[t], oracle.matmul(synth.TYPE_Q4_K, w, x[t], 40, 512))


def test_argmax_lowest_index_wins(oracle):
    v = np.array([0.5, 2.0, -1.0, 2.0, 2.0], np.float32)
    assert oracle.argmax(v) == 1


def test_greedy_pick_non_finite_rules(oracle):
    """The reference's compiled greedy pick (src/sample.c:28-31) and the
    oracle's agree on the non-finite rules the device argmax follows: a NaN
    at index 0 is kept, a NaN elsewhere never wins, ties go to the lowest
    index, +inf wins, all -inf keeps index 0."""
    from oracle.hako_oracle import ref_greedy_pick
    nan, inf = np.nan, np.inf
    cases = [([nan, 1.0, 2.0], 0), ([0.0, nan, 2.0, 2.0], 2), ([1.0, nan, nan], 0), ([nan, nan], 0),
             ([-1.0, inf, 3.0, inf], 1), ([-inf, -inf, nan], 0), ([0.5, 2.0, -1.0, 2.0], 1)]
    for v, want in cases:
        v = np.array(v, np.float32)
        assert ref_greedy_pick(v) == want, v
        assert oracle.argmax(v) == want, v
