"""GPU parity of the multi-token matmuls (prompt prefill) against the oracle.

The reference computes a prompt token by token; the oracle's matmul_batch is
the same M independent matmuls. Bars: fp32 outputs max|Δ|/max|ref| <= 1e-5;
crafted inputs whose outputs are exact integers pin the int8 matrix-core sums
(Q4_K) and the fp16 hi/lo path (Q6_K) bit for bit.
"""
import numpy as np
import pytest

from hako_amd import synth
from helpers import maxabs_rel

pytestmark = pytest.mark.gpu

TOL = 1e-5
Q4, Q6 = synth.TYPE_Q4_K, synth.TYPE_Q6_K
HAKO_TUNE_Q6K_GEMM_TN = 13   # include/hako_gpu.h
HAKO_TUNE_Q6K_GEMM_SK = 15


def run_batch(gpu, qtype, w, x, n_out, n_in, bias=None):
    m = x.shape[0]
    dw, dx, dy = gpu.upload(w), gpu.upload(x), gpu.alloc(m * n_out * 4)
    db = gpu.upload(bias) if bias is not None else None
    gpu.matmul_batch(dy, dx, qtype, dw, db, m, n_out, n_in)
    y = gpu.download(dy, np.float32, (m, n_out))
    for b in (dw, dx, dy, db):
        if b is not None:
            b.free()
    return y


def run_q4k_gemm(gpu, w, xq, xs, n_out, n_in):
    m = xq.shape[0]
    dw, dq, ds, dy = gpu.upload(w), gpu.upload(xq), gpu.upload(xs), gpu.alloc(m * n_out * 4)
    gpu.q4k_gemm(dy, dw, dq, ds, None, m, n_out, n_in)
    y = gpu.download(dy, np.float32, (m, n_out))
    for b in (dw, dq, ds, dy):
        b.free()
    return y


GEMM_SHAPES = [(64, 64, 256), (130, 200, 2048), (17, 100, 3584), (64, 512, 3584), (200, 37, 1280),
               (96, 300, 11008),
               # up to 16 tokens: the skinny kernels (batched decode)
               (2, 64, 256), (5, 100, 2048), (16, 512, 3584), (16, 1000, 1280), (1 + 15, 37, 2048), (3, 18944, 3584),
               # one split per 64-row tile, two passes of the weight prefetch ring
               (16, 32832, 2048)]


@pytest.mark.parametrize("m,n_out,n_in", GEMM_SHAPES)
def test_q4k_batch_vs_oracle(gpu, oracle, m, n_out, n_in):
    rng = np.random.default_rng(m * 1000 + n_out + n_in)
    w = synth.q4k_weight(rng, n_out, n_in)
    x = rng.standard_normal((m, n_in)).astype(np.float32)
    bias = 0.1 * rng.standard_normal(n_out).astype(np.float32)
    got = run_batch(gpu, Q4, w, x, n_out, n_in, bias)
    want = oracle.matmul(Q4, w, x, n_out, n_in, bias=bias, f64=True)
    assert maxabs_rel(got, want) < TOL


@pytest.mark.parametrize("m,n_out,n_in", GEMM_SHAPES + [(70, 100, 18944), (16, 100, 18944), (7, 3584, 11008)])
def test_q6k_batch_vs_oracle(gpu, oracle, m, n_out, n_in):
    rng = np.random.default_rng(m * 1001 + n_out + n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = rng.standard_normal((m, n_in)).astype(np.float32)
    bias = 0.1 * rng.standard_normal(n_out).astype(np.float32)
    got = run_batch(gpu, Q6, w, x, n_out, n_in, bias)
    want = oracle.matmul(Q6, w, x, n_out, n_in, bias=bias, f64=True)
    assert maxabs_rel(got, want) < TOL


def test_q6k_batch_token_rows_of_any_magnitude(gpu, oracle):
    """Each token row is scaled by its own power of two: rows of 1e-30, 1e4
    and subnormal-only values stay within tolerance of their own outputs."""
    rng = np.random.default_rng(5)
    n_out, n_in = 128, 2048
    w = synth.q6k_weight(rng, n_out, n_in)
    x = rng.standard_normal((6, n_in)).astype(np.float32)
    x[1] *= 1e-30
    x[2] *= 1e4
    x[3] = np.float32(1e-42) * np.sign(x[3])   # subnormal
    x[4] = 0.0
    x[5, ::7] *= 1e3                           # wide range within a row
    got = run_batch(gpu, Q6, w, x, n_out, n_in)
    want = oracle.matmul(Q6, w, x, n_out, n_in, f64=True)
    for t in range(6):
        ref = np.max(np.abs(want[t]))
        if ref == 0:
            assert np.all(got[t] == 0)
        else:
            assert np.max(np.abs(got[t] - want[t])) / ref < TOL, t


def _one_hot_scales(n_blocks, sb, which):
    """12 scale bytes giving (s, m) = (1, 0) (which='s') or (0, 1) (which='m')
    for sub-block sb and (0, 0) elsewhere (packing of reference quant.c:57-66)."""
    sc = np.zeros(12, np.uint8)
    if sb < 4:
        sc[sb if which == "s" else sb + 4] = 1
    else:
        sc[sb + 4] = 1 if which == "s" else 0x10
    return np.tile(sc, (n_blocks, 1))


@pytest.mark.parametrize("m", [80, 16, 5])
@pytest.mark.parametrize("sb", [0, 3, 4, 7])
@pytest.mark.parametrize("which", ["s", "m"])
def test_q4k_gemm_integer_sums_exact(gpu, oracle, m, sb, which):
    """d = 1, dmin = 1, one (s, m) = (1, 0) or (0, 1) per block and xs = 1:
    each output is Σ over blocks of the sub-block's iqx (or −ix), an integer
    the fp32 fold represents exactly — bit-exact against the oracle's sums."""
    rng = np.random.default_rng(sb * 3 + (which == "m") + m)
    n_out, n_in = 96, 3584
    nb = n_in // 256
    w = synth.q4k_weight(rng, n_out, n_in).reshape(n_out * nb, 144).copy()
    w[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w[:, 2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w[:, 4:16] = _one_hot_scales(n_out * nb, sb, which)
    w = w.reshape(n_out, nb * 144)
    xq = rng.integers(-127, 128, (m, n_in)).astype(np.int8)
    xs = np.ones((m, n_in // 32), np.float32)
    got = run_q4k_gemm(gpu, w, xq, xs, n_out, n_in)
    want = np.empty((m, n_out), np.float64)
    for t in range(m):
        iqx, ix = oracle.q4k_isums(w, xq[t], n_out, n_in)
        sel = iqx if which == "s" else -ix
        want[t] = sel[:, sb::8].sum(axis=1)
    assert np.array_equal(got, want.astype(np.float32))


@pytest.mark.parametrize("m", [70, 16, 3])
def test_q6k_gemm_exact_integers(gpu, oracle, m):
    """Small-integer activations (exact in fp16, lo = 0) and d = 1: outputs are
    integers the fp32 accumulation holds exactly — bit-exact against the
    oracle's double-precision result."""
    rng = np.random.default_rng(9 + m)
    n_out, n_in = 90, 2048
    nb = n_in // 256
    w = synth.q6k_weight(rng, n_out, n_in).reshape(n_out * nb, 210).copy()
    w[:, 208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    w = w.reshape(n_out, nb * 210)
    x = rng.integers(-8, 9, (m, n_in)).astype(np.float32)
    got = run_batch(gpu, Q6, w, x, n_out, n_in)
    want = oracle.matmul(Q6, w, x, n_out, n_in, f64=True)
    assert np.array_equal(got, want)


def test_q4k_gemm_full_7b_shape_sampled_rows(gpu, oracle):
    """The 7B ffn_up prefill shape (512 tokens x 18944 x 3584); rows sampled
    for the oracle, plus batch == per-token GEMV consistency on all of it."""
    rng = np.random.default_rng(77)
    m, n_out, n_in = 512, 18944, 3584
    w = synth.q4k_weight(rng, n_out, n_in)
    x = rng.standard_normal((m, n_in)).astype(np.float32)
    got = run_batch(gpu, Q4, w, x, n_out, n_in)
    rows = np.unique(np.concatenate([np.arange(64), rng.integers(0, n_out, 128), [n_out - 1]]))
    want = oracle.matmul(Q4, w[rows], x, rows.size, n_in, f64=True)
    assert maxabs_rel(got[:, rows], want) < TOL
    # every token against the single-token GEMV of the same weights
    dw, dx, do = gpu.upload(w), gpu.upload(x[[0, 255, 511]]), gpu.alloc(n_out * 4)
    for i, t in enumerate((0, 255, 511)):
        gpu.matmul(do, dx.offset(i * n_in * 4), Q4, dw, None, n_out, n_in)
        assert maxabs_rel(got[t], gpu.download(do, np.float32, (n_out,))) < TOL
    for b in (dw, dx, do):
        b.free()


@pytest.mark.parametrize("m,n_out,n_in", [(64, 128, 256), (130, 200, 2048), (77, 3648, 1024), (512, 384, 4608)])
def test_q6k_gemm_tile_widths_agree_bit_exact(gpu, oracle, m, n_out, n_in):
    """The 64-row and the 128-row (double-buffered) tiles do the same
    arithmetic per output in the same order, so their outputs are
    bit-identical, ragged token and row edges included; both within the bar
    of the oracle. (Stream-K, which adds a tile's K pieces after the fact,
    is off here and tested below.)"""
    rng = np.random.default_rng(m + n_out + n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = rng.standard_normal((m, n_in)).astype(np.float32)
    bias = 0.1 * rng.standard_normal(n_out).astype(np.float32)
    got = {}
    gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, 0)   # (the standalone call's default leaves it off too)
    try:
        for tn in (64, 128):
            gpu.tune(HAKO_TUNE_Q6K_GEMM_TN, tn)
            got[tn] = run_batch(gpu, Q6, w, x, n_out, n_in, bias)
    finally:
        gpu.tune(HAKO_TUNE_Q6K_GEMM_TN, 0)
        gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, 1)
    assert np.array_equal(got[64].view(np.uint32), got[128].view(np.uint32))
    want = oracle.matmul(Q6, w, x, n_out, n_in, bias=bias, f64=True)
    assert maxabs_rel(got[128], want) < TOL


@pytest.mark.parametrize("m,n_out,n_in", [(130, 200, 2048), (77, 3648, 1024), (512, 384, 4608), (64, 128, 512),
                                         (512, 3584, 4608)])
def test_q6k_gemm_stream_k(gpu, oracle, m, n_out, n_in):
    """128-row tiles in stream-K form (every CU takes an equal share of the
    tiles' super-blocks; a tile's pieces meet in a second launch, in order of
    K) against the same tiles whole: within 1e-6, and the GEMM bar of the
    oracle. The shapes give tiles held by one to several workgroups, pieces
    of one super-block, ragged token and row edges; twice in a row, the
    second call on other inputs, so no stale slot passes."""
    rng = np.random.default_rng(3 * m + n_out + n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    bias = 0.1 * rng.standard_normal(n_out).astype(np.float32)
    gpu.tune(HAKO_TUNE_Q6K_GEMM_TN, 128)
    try:
        for call in range(2):
            x = rng.standard_normal((m, n_in)).astype(np.float32) * (1.0 + 9.0 * call)
            gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, 0)
            whole = run_batch(gpu, Q6, w, x, n_out, n_in, bias)
            gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, 2)
            got = run_batch(gpu, Q6, w, x, n_out, n_in, bias)
            assert maxabs_rel(got, whole) < 1e-6
            want = oracle.matmul(Q6, w, x, n_out, n_in, bias=bias, f64=True)
            assert maxabs_rel(got, want) < TOL
    finally:
        gpu.tune(HAKO_TUNE_Q6K_GEMM_TN, 0)
        gpu.tune(HAKO_TUNE_Q6K_GEMM_SK, 1)


def test_q6k_gemm_full_7b_shape_sampled_rows(gpu, oracle):
    rng = np.random.default_rng(78)
    m, n_out, n_in = 512, 3584, 18944
    w = synth.q6k_weight(rng, n_out, n_in)
    x = rng.standard_normal((m, n_in)).astype(np.float32)
    got = run_batch(gpu, Q6, w, x, n_out, n_in)
    rows = np.unique(np.concatenate([np.arange(32), rng.integers(0, n_out, 64), [n_out - 1]]))
    want = oracle.matmul(Q6, w[rows], x, rows.size, n_in, f64=True)
    assert maxabs_rel(got[:, rows], want) < TOL


def test_gemm_bad_shapes_are_rejected(gpu):
    from hako_amd.gpu import HakoGpuError
    dw, dx, dy = gpu.alloc(1 << 16), gpu.alloc(1 << 16), gpu.alloc(1 << 16)
    with pytest.raises(HakoGpuError, match="256"):
        gpu.matmul_batch(dy, dx, Q4, dw, None, 4, 4, 100)
    with pytest.raises(HakoGpuError, match="256"):
        gpu.matmul_batch(dy, dx, Q6, dw, None, 4, 4, 300)
    with pytest.raises(HakoGpuError, match="m > 0"):
        gpu.matmul_batch(dy, dx, Q6, dw, None, 0, 4, 256)
    for b in (dw, dx, dy):
        b.free()
