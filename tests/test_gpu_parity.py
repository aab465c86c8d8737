"""GPU parity: the gfx950 kernels behind the C ABI against the pinned oracle
and the reference's own golden outputs.

Bars: bit-exact for the q8 quantizer, the dequantizers and the per-sub-block
int32 sums; max|Δ|/max|ref| <= 1e-5 for fp32 GEMV outputs.
"""
import numpy as np
import pytest

from hako_amd import synth
from helpers import maxabs_rel

pytestmark = pytest.mark.gpu

TOL = 1e-5
Q4, Q6 = synth.TYPE_Q4_K, synth.TYPE_Q6_K


def gpu_q8(gpu, x: np.ndarray):
    x = np.ascontiguousarray(x, np.float32)
    rows = 1 if x.ndim == 1 else x.shape[0]
    n = x.shape[-1]
    dx = gpu.upload(x)
    dq, ds = gpu.alloc(rows * n), gpu.alloc(rows * n // 32 * 4)
    gpu.quantize_q8_32(dx, rows, n, dq, ds)
    xq = gpu.download(dq, np.int8, x.shape)
    xs = gpu.download(ds, np.float32, x.shape[:-1] + (n // 32,))
    for b in (dx, dq, ds):
        b.free()
    return xq, xs


def gpu_dequant(gpu, qtype, blocks, nelem):
    db, do = gpu.upload(blocks), gpu.alloc(nelem * 4)
    gpu.dequant(qtype, db, do, nelem)
    y = gpu.download(do, np.float32, (nelem,))
    db.free(); do.free()
    return y


def gpu_matmul(gpu, qtype, w, x, n_out, n_in, bias=None):
    dw, dx, do = gpu.upload(w), gpu.upload(x), gpu.alloc(n_out * 4)
    db = gpu.upload(bias) if bias is not None else None
    gpu.matmul(do, dx, qtype, dw, db, n_out, n_in)
    y = gpu.download(do, np.float32, (n_out,))
    for b in (dw, dx, do, db):
        if b is not None:
            b.free()
    return y


# ── q8 activation quantizer ──

def test_q8_golden(gpu, golden):
    g = golden("q8.npz")
    xq, xs = gpu_q8(gpu, g["x"])
    assert np.array_equal(xq, g["xq"])
    assert np.array_equal(xs.view(np.uint32), g["xs"].view(np.uint32))


@pytest.mark.parametrize("rows,n", [(1, 2048), (1, 3584), (1, 32), (512, 3584), (7, 18944)])
def test_q8_random_vs_oracle(gpu, oracle, rows, n):
    rng = np.random.default_rng(rows * 100003 + n)
    x = synth.activation(rng, n, rows=rows) * np.float32(rng.uniform(1e-3, 1e3))
    xq, xs = gpu_q8(gpu, x)
    for r in range(rows):
        oq, os_ = oracle.quantize_q8_32(x[r])
        assert np.array_equal(xq[r], oq), r
        assert np.array_equal(xs[r].view(np.uint32), os_.view(np.uint32)), r


def test_q8_non_finite_vs_oracle(gpu, oracle):
    """NaN and infinite inputs (a block of NaNs has scale 0, as the
    reference's maximum starts at 0 and takes only larger values)."""
    from test_oracle import q8_non_finite_rows
    x = q8_non_finite_rows()
    xq, xs = gpu_q8(gpu, x)
    for r in range(x.shape[0]):
        oq, os_ = oracle.quantize_q8_32(x[r])
        assert np.array_equal(xq[r], oq), r
        assert np.array_equal(xs[r].view(np.uint32), os_.view(np.uint32)), r


# ── dequantizers ──

@pytest.mark.parametrize("qtype,name", [(Q4, "q4k_dequant.npz"), (Q6, "q6k_dequant.npz")])
def test_dequant_golden(gpu, golden, qtype, name):
    g = golden(name)
    n = g["blocks"].shape[0] * 256
    y = gpu_dequant(gpu, qtype, g["blocks"], n)
    assert np.array_equal(y.view(np.uint32), g["out"].view(np.uint32))


@pytest.mark.parametrize("qtype,n_blocks", [(Q4, 88064), (Q6, 88064), (Q6, 1)])
def test_dequant_large_vs_oracle(gpu, oracle, qtype, n_blocks):
    rng = np.random.default_rng(n_blocks + qtype)
    b = synth.q4k_blocks(rng, n_blocks) if qtype == Q4 else synth.q6k_blocks(rng, n_blocks, scale_range=(-128, 127))
    y = gpu_dequant(gpu, qtype, b, n_blocks * 256)
    assert np.array_equal(y.view(np.uint32), oracle.dequant(qtype, b, n_blocks * 256).view(np.uint32))


def test_dequant_f16(gpu):
    h = np.arange(0, 65536, 1, dtype=np.uint32).astype(np.uint16)
    y = gpu_dequant(gpu, synth.TYPE_F16, h, h.size)
    want = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(want)
    assert np.array_equal(y[ok].view(np.uint32), want[ok].view(np.uint32))
    assert np.all(np.isnan(y[~ok]))


# ── Q4_K x q8: integer sums bit-exact ──

def gpu_isums(gpu, w, xq, n_out, n_in):
    dw, dq = gpu.upload(w), gpu.upload(xq)
    di, dx = gpu.alloc(n_out * n_in // 32 * 4), gpu.alloc(n_out * n_in // 32 * 4)
    gpu.q4k_isums(di, dx, dw, dq, n_out, n_in)
    iqx = gpu.download(di, np.int32, (n_out, n_in // 32))
    ix = gpu.download(dx, np.int32, (n_out, n_in // 32))
    for b in (dw, dq, di, dx):
        b.free()
    return iqx, ix


def test_isums_golden(gpu, golden):
    g = golden("q4k_isums.npz")
    for n_in in (2048, 3584):
        w, xq = g[f"w_{n_in}"], g[f"xq_{n_in}"]
        iqx, ix = gpu_isums(gpu, w, xq, w.shape[0], n_in)
        assert np.array_equal(iqx, g[f"iqx_{n_in}"])
        assert np.array_equal(ix, g[f"ix_{n_in}"])


@pytest.mark.parametrize("n_out,n_in", [(11008, 2048), (18944, 3584), (37, 11008), (5, 256), (3, 18944)])
def test_isums_vs_oracle(gpu, oracle, n_out, n_in):
    rng = np.random.default_rng(n_out * 7 + n_in)
    w = synth.q4k_weight(rng, n_out, n_in)
    xq = rng.integers(-127, 128, n_in).astype(np.int8)
    iqx, ix = gpu_isums(gpu, w, xq, n_out, n_in)
    rows = np.unique(np.concatenate([np.arange(min(n_out, 64)), rng.integers(0, n_out, 64)]))
    oi, ox = oracle.q4k_isums(w[rows], xq, rows.size, n_in)
    assert np.array_equal(iqx[rows], oi)
    assert np.array_equal(ix[rows], ox)


# ── GEMV fp32 outputs ──

Q4_SHAPES = [(11008, 2048), (2048, 2048), (256, 2048), (18944, 3584), (3584, 3584), (512, 3584),
             (1, 256), (3, 512), (17, 11008), (5, 18944)]


@pytest.mark.parametrize("n_out,n_in", Q4_SHAPES)
def test_q4k_matmul_fused_vs_oracle(gpu, oracle, n_out, n_in):
    rng = np.random.default_rng(n_out * 31 + n_in)
    w = synth.q4k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    bias = 0.1 * synth.activation(rng, n_out)
    got = gpu_matmul(gpu, Q4, w, x, n_out, n_in, bias)
    want = oracle.matmul(Q4, w, x, n_out, n_in, bias=bias, f64=True)
    assert maxabs_rel(got, want) < TOL


@pytest.mark.parametrize("n_out,n_in", [(11008, 2048), (18944, 3584), (7, 11008)])
def test_q4k_gemv_prequantized_vs_oracle(gpu, oracle, n_out, n_in):
    rng = np.random.default_rng(n_out + n_in)
    w = synth.q4k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    xq, xs = oracle.quantize_q8_32(x)
    dw, dq, ds, do = gpu.upload(w), gpu.upload(xq), gpu.upload(xs), gpu.alloc(n_out * 4)
    gpu.q4k_gemv(do, dw, dq, ds, None, n_out, n_in)
    got = gpu.download(do, np.float32, (n_out,))
    for b in (dw, dq, ds, do):
        b.free()
    want = np.array([oracle.q4k_vec_dot(w[r], n_in, xq, xs, f64=True) for r in range(n_out)])
    assert maxabs_rel(got, want) < TOL


HAKO_TUNE_Q4K_WAVES, HAKO_TUNE_Q4K_FLAT_ITEMS = 3, 5


@pytest.mark.parametrize("n_out,n_in", [(11008, 2048), (1000, 3584), (37, 256), (300, 1280)])
def test_q4k_launch_shapes_agree_bit_exact(gpu, oracle, n_out, n_in):
    """Persistent and flat grids, 4 or 8 waves, 1..8 row items per wave: the
    lane work and reduction order are the same, so outputs are identical."""
    rng = np.random.default_rng(n_out + 3 * n_in)
    w = synth.q4k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    bias = synth.activation(rng, n_out)
    xq, xs = oracle.quantize_q8_32(x)
    dw, dx, db, do = gpu.upload(w), gpu.upload(x), gpu.upload(bias), gpu.alloc(n_out * 4)
    dq, ds = gpu.upload(xq), gpu.upload(xs)
    di, dix = gpu.alloc(n_out * n_in // 32 * 4), gpu.alloc(n_out * n_in // 32 * 4)
    seen = {}
    try:
        for items in (-1, 0, 1, 2, 4, 8):
            for waves in (4, 8):
                gpu.tune(HAKO_TUNE_Q4K_FLAT_ITEMS, items)
                gpu.tune(HAKO_TUNE_Q4K_WAVES, waves)
                gpu.matmul(do, dx, Q4, dw, db, n_out, n_in)
                fused = gpu.download(do, np.float32, (n_out,))
                gpu.q4k_gemv(do, dw, dq, ds, None, n_out, n_in)
                preq = gpu.download(do, np.float32, (n_out,))
                gpu.q4k_isums(di, dix, dw, dq, n_out, n_in)
                sums = gpu.download(di, np.int32, (n_out, n_in // 32))
                for k, v in (("fused", fused), ("preq", preq), ("isums", sums)):
                    if k in seen:
                        assert np.array_equal(seen[k].view(np.uint32), v.view(np.uint32)), (k, items, waves)
                    else:
                        seen[k] = v
    finally:
        gpu.tune(HAKO_TUNE_Q4K_FLAT_ITEMS, -1)
        gpu.tune(HAKO_TUNE_Q4K_WAVES, 4)
        for b in (dw, dx, db, do, dq, ds, di, dix):
            b.free()
    want = oracle.matmul(Q4, w, x, n_out, n_in, bias=bias, f64=True)
    assert maxabs_rel(seen["fused"], want) < TOL


Q6_SHAPES = [(2048, 11008), (151936, 2048), (3584, 18944), (256, 2048), (1, 256), (9, 768), (33, 11008),
             (40000, 512), (5, 20480), (5, 32000)]


@pytest.mark.parametrize("n_out,n_in", Q6_SHAPES)
def test_q6k_gemv_vs_oracle(gpu, oracle, n_out, n_in):
    rng = np.random.default_rng(n_out * 17 + n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    got = gpu_matmul(gpu, Q6, w, x, n_out, n_in)
    want = oracle.matmul(Q6, w, x, n_out, n_in, f64=True, threads=16)
    assert maxabs_rel(got, want) < TOL


@pytest.mark.parametrize("n_out,n_in", [(300, 2048), (40000, 768), (33, 11008)])
def test_q6k_block_magnitudes(gpu, oracle, n_out, n_in):
    """Activation blocks 1e-30 .. 1e30 apart, an all-zero block and a block of
    subnormals, with a bias; then single blocks alone, each against the
    oracle's float64 sums (not the subnormal one: the reference's fast-math
    build flushes it to zero)."""
    rng = np.random.default_rng(n_out + 3 * n_in)
    nb = n_in // 256
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    mags = np.float32(10.0) ** rng.integers(-30, 31, nb).astype(np.float32)
    x = (x.reshape(nb, 256) * mags[:, None]).astype(np.float32)
    x[0] = 0.0
    if nb > 2:
        x[2] = (rng.standard_normal(256) * 1e-39).astype(np.float32)   # subnormal
    x = x.reshape(-1)
    bias = synth.activation(rng, n_out)
    got = gpu_matmul(gpu, Q6, w, x, n_out, n_in, bias=bias)
    want = oracle.matmul(Q6, w, x, n_out, n_in, bias=bias, f64=True, threads=16)
    assert maxabs_rel(got, want) < TOL
    alone = [b for b in range(nb) if not (nb > 2 and b == 2)]
    for b in rng.choice(alone, size=min(len(alone), 3), replace=False):
        xb = np.zeros_like(x)
        xb[256 * b:256 * b + 256] = x[256 * b:256 * b + 256]
        got = gpu_matmul(gpu, Q6, w, xb, n_out, n_in)
        want = oracle.matmul(Q6, w, xb, n_out, n_in, f64=True, threads=16)
        assert maxabs_rel(got, want) < TOL, b


@pytest.mark.parametrize("n_out,n_in", [(300, 2048), (40000, 512), (2048, 11008)])
def test_q6k_nan_propagates(gpu, n_out, n_in):
    """A NaN anywhere in the activation makes every output NaN, as the
    reference's fp32 dot does (every weight multiplies it)."""
    rng = np.random.default_rng(7)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    x[n_in - 3] = np.nan
    got = gpu_matmul(gpu, Q6, w, x, n_out, n_in)
    assert np.all(np.isnan(got))


HAKO_TUNE_Q6K_WGS_PER_CU, HAKO_TUNE_Q6K_WAVES, HAKO_TUNE_Q6K_FLAT_ITEMS = 2, 4, 8
HAKO_TUNE_Q6K_FLAT_SEG, HAKO_TUNE_Q6K_ROWS, HAKO_TUNE_Q6K_DIGITS = 10, 11, 14


@pytest.mark.parametrize("n_out,n_in", [(2048, 11008), (300, 2048), (77, 18944), (100, 1792), (64, 512)])
def test_q6k_launch_shapes_agree_bit_exact(gpu, oracle, n_out, n_in):
    """Persistent grid (4 or 8 waves, 1 or 2 workgroups per CU) and flat grid
    (1..8 row items per wave), with and without a bias: the lane work and the
    order of every addition are the same, so outputs are identical. (The rows
    grid, which wide rows take by default, adds in its own order: off here,
    its own test below; so do the persistent grid's integer columns, off here
    and tested below.)"""
    rng = np.random.default_rng(n_out + 5 * n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    bias = synth.activation(rng, n_out)
    dw, dx, db, do = gpu.upload(w), gpu.upload(x), gpu.upload(bias), gpu.alloc(n_out * 4)
    seen = {}
    gpu.tune(HAKO_TUNE_Q6K_ROWS, -1)
    gpu.tune(HAKO_TUNE_Q6K_DIGITS, 0)
    try:
        for items, waves, wgs in ((-1, 4, 1), (0, 4, 1), (0, 8, 1), (0, 4, 2), (1, 4, 1), (2, 4, 1), (4, 4, 1),
                                  (8, 4, 1)):
            gpu.tune(HAKO_TUNE_Q6K_FLAT_ITEMS, items)
            gpu.tune(HAKO_TUNE_Q6K_WAVES, waves)
            gpu.tune(HAKO_TUNE_Q6K_WGS_PER_CU, wgs)
            for b in (None, db):
                gpu.q6k_gemv(do, dw, dx, b, n_out, n_in)
                v = gpu.download(do, np.float32, (n_out,))
                key = b is None
                if key in seen:
                    assert np.array_equal(seen[key].view(np.uint32), v.view(np.uint32)), (items, waves, wgs, key)
                else:
                    seen[key] = v
    finally:
        gpu.tune(HAKO_TUNE_Q6K_FLAT_ITEMS, -1)
        gpu.tune(HAKO_TUNE_Q6K_WAVES, 4)
        gpu.tune(HAKO_TUNE_Q6K_WGS_PER_CU, 1)
        gpu.tune(HAKO_TUNE_Q6K_ROWS, 0)
        gpu.tune(HAKO_TUNE_Q6K_DIGITS, 1)
        for b in (dw, dx, db, do):
            b.free()
    want = oracle.matmul(Q6, w, x, n_out, n_in, bias=bias, f64=True, threads=16)
    assert maxabs_rel(seen[False], want) < TOL


@pytest.mark.parametrize("n_out,n_in", [(151936, 2048), (4000, 3584), (300, 2048), (40000, 768), (64, 512)])
def test_q6k_integer_columns(gpu, oracle, n_out, n_in):
    """The persistent grid's integer activation columns (each 16-value group
    scaled by its own power of two and carried as three signed bytes) against
    its fp32 product per weight and the oracle: within 2e-6 of the first, the
    GEMV bar of the second; on activation blocks 1e-30 .. 1e30 apart with an
    all-zero block; and with an inf in one group, which sends every wave
    whose lanes hold it to the fp32 path: the same outputs (NaN, as the
    reference gives them) either way."""
    rng = np.random.default_rng(n_out + 7 * n_in)
    nb = n_in // 256
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    xm = (x.reshape(nb, 256) * (np.float32(10.0) ** rng.integers(-30, 31, nb).astype(np.float32))[:, None])
    xm = xm.astype(np.float32)
    xm[0] = 0.0
    xi = x.copy()
    xi[n_in // 2 + 5] = np.inf
    gpu.tune(HAKO_TUNE_Q6K_ROWS, -1)
    gpu.tune(HAKO_TUNE_Q6K_FLAT_ITEMS, 0)
    try:
        for xv in (x, xm.reshape(-1)):
            gpu.tune(HAKO_TUNE_Q6K_DIGITS, 0)
            base = gpu_matmul(gpu, Q6, w, xv, n_out, n_in)
            gpu.tune(HAKO_TUNE_Q6K_DIGITS, 1)
            got = gpu_matmul(gpu, Q6, w, xv, n_out, n_in)
            assert maxabs_rel(got, base) < 2e-6
            if n_out <= 40000:
                want = oracle.matmul(Q6, w, xv, n_out, n_in, f64=True, threads=16)
                assert maxabs_rel(got, want) < TOL
        gpu.tune(HAKO_TUNE_Q6K_DIGITS, 0)
        base = gpu_matmul(gpu, Q6, w, xi, n_out, n_in)
        gpu.tune(HAKO_TUNE_Q6K_DIGITS, 1)
        got = gpu_matmul(gpu, Q6, w, xi, n_out, n_in)
        assert np.array_equal(np.isnan(got), np.isnan(base)) and np.array_equal(np.isinf(got), np.isinf(base))
        fin = np.isfinite(base)
        assert np.array_equal(got[fin].view(np.uint32), base[fin].view(np.uint32))
    finally:
        gpu.tune(HAKO_TUNE_Q6K_ROWS, 0)
        gpu.tune(HAKO_TUNE_Q6K_FLAT_ITEMS, -1)
        gpu.tune(HAKO_TUNE_Q6K_DIGITS, 1)


@pytest.mark.parametrize("n_out,n_in", [(77, 18944), (3584, 18944), (5, 32000), (300, 2048), (9, 4608)])
def test_q6k_rows_grid(gpu, oracle, n_out, n_in):
    """The rows grid (each wave sums whole rows: its lanes over the passes,
    then the lanes; activation staged in LDS for rows of several passes) at
    4, 8 and 16 waves and 2 or 4 items in flight, with and without a bias:
    identical outputs (the order of additions does not depend on the grid),
    within 1e-5 of the oracle; a NaN in the activation reaches every row."""
    rng = np.random.default_rng(n_out + 7 * n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    bias = synth.activation(rng, n_out)
    dw, dx, db, do = gpu.upload(w), gpu.upload(x), gpu.upload(bias), gpu.alloc(n_out * 4)
    seen = {}
    try:
        for cfg in (44, 82, 84, 162):
            gpu.tune(HAKO_TUNE_Q6K_ROWS, cfg)
            for b in (None, db):
                gpu.q6k_gemv(do, dw, dx, b, n_out, n_in)
                v = gpu.download(do, np.float32, (n_out,))
                key = b is None
                if key in seen:
                    assert np.array_equal(seen[key].view(np.uint32), v.view(np.uint32)), (cfg, key)
                else:
                    seen[key] = v
        xn = x.copy()
        xn[n_in // 2 + 5] = np.nan
        dxn = gpu.upload(xn)
        gpu.q6k_gemv(do, dw, dxn, None, n_out, n_in)
        nan_out = gpu.download(do, np.float32, (n_out,))
        dxn.free()
    finally:
        gpu.tune(HAKO_TUNE_Q6K_ROWS, 0)
        for b in (dw, dx, db, do):
            b.free()
    assert np.all(np.isnan(nan_out))
    want = oracle.matmul(Q6, w, x, n_out, n_in, bias=bias, f64=True, threads=16)
    assert maxabs_rel(seen[False], want) < TOL
    want = oracle.matmul(Q6, w, x, n_out, n_in, f64=True, threads=16)
    assert maxabs_rel(seen[True], want) < TOL


@pytest.mark.parametrize("n_out,n_in", [(2048, 11008), (33, 11008), (500, 18944)])
def test_q6k_flat_part_widths(gpu, oracle, n_out, n_in):
    """The flat grid's wide rows cut into 32- or 64-chunk parts (2 and 4 row
    items per wave): within 1e-5 of the oracle."""
    rng = np.random.default_rng(n_out + 11 * n_in)
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    want = oracle.matmul(Q6, w, x, n_out, n_in, f64=True, threads=16)
    try:
        for seg in (32, 64):
            for items in (2, 4):
                gpu.tune(HAKO_TUNE_Q6K_FLAT_SEG, seg)
                gpu.tune(HAKO_TUNE_Q6K_FLAT_ITEMS, items)
                got = gpu_matmul(gpu, Q6, w, x, n_out, n_in)
                assert maxabs_rel(got, want) < TOL, (seg, items)
    finally:
        gpu.tune(HAKO_TUNE_Q6K_FLAT_SEG, 0)
        gpu.tune(HAKO_TUNE_Q6K_FLAT_ITEMS, -1)


def test_q6k_full_int8_scales(gpu, oracle):
    rng = np.random.default_rng(11)
    w = synth.q6k_blocks(rng, 300 * 8, scale_range=(-128, 127)).reshape(300, -1)
    x = synth.activation(rng, 2048)
    got = gpu_matmul(gpu, Q6, w, x, 300, 2048)
    assert maxabs_rel(got, oracle.matmul(Q6, w, x, 300, 2048)) < TOL


@pytest.mark.parametrize("name", ["q4k", "q6k", "q6k_long", "f16", "f32"])
def test_matmul_vs_reference_golden(gpu, golden, name):
    g = golden("matmul.npz")
    qt, n_out, n_in = (int(v) for v in g[f"{name}_shape"])
    got = gpu_matmul(gpu, qt, g[f"{name}_w"], g[f"{name}_x"], n_out, n_in, g.get(f"{name}_bias"))
    assert maxabs_rel(got, g[f"{name}_out"]) < TOL


def test_matmul_host_uses_mirror(gpu, oracle):
    rng = np.random.default_rng(21)
    w = synth.q4k_weight(rng, 600, 2048)
    x = synth.activation(rng, 2048)
    gpu.mirror_upload(w)
    out = np.empty(600, np.float32)
    gpu.matmul_host(out, x, Q4, w, None, 600, 2048)
    gpu.mirror_release(w)
    assert maxabs_rel(out, oracle.matmul(Q4, w, x, 600, 2048)) < TOL


def test_mirror_overlaps_are_refused(gpu):
    """A range overlapping a live mirror (inside it, or across its end) is
    refused rather than served from the older copy; after the release the
    same bytes upload again."""
    from hako_amd.gpu import HakoGpuError
    buf = np.arange(4096, dtype=np.uint8)
    gpu.mirror_upload(buf[1024:3072])
    try:
        for view in (buf[1024:3072], buf[2048:2560], buf[0:1500], buf[3000:]):
            with pytest.raises(HakoGpuError, match="overlaps"):
                gpu.mirror_upload(view)
        gpu.mirror_upload(buf[:1024])        # adjacent, disjoint
        gpu.mirror_release(buf[:1024])
    finally:
        gpu.mirror_release(buf[1024:3072])
    d = gpu.mirror_upload(buf[0:1500])
    gpu.mirror_release(buf[0:1500])
    assert d


def test_q6k_widest_row(gpu, oracle):
    """n_in = 32768 fills the widest workgroup (8 parts of 64 chunks of 64
    weights) and matches the reference's generic row path; one super-block
    more is refused before anything is launched."""
    from hako_amd.gpu import HakoGpuError
    rng = np.random.default_rng(32768)
    n_out, n_in = 7, 32768
    w = synth.q6k_weight(rng, n_out, n_in)
    x = synth.activation(rng, n_in)
    got = gpu_matmul(gpu, Q6, w, x, n_out, n_in)
    assert maxabs_rel(got, oracle.matmul(Q6, w, x, n_out, n_in, f64=True, threads=16)) < TOL
    wide = n_in + 256
    dw, dx, do = gpu.alloc(wide // 256 * 210 * 2), gpu.alloc(wide * 4), gpu.alloc(64)
    try:
        with pytest.raises(HakoGpuError, match="exceeds"):
            gpu.q6k_gemv(do, dw, dx, None, 2, wide)
    finally:
        for b in (dw, dx, do):
            b.free()


def test_bad_shapes_are_rejected(gpu):
    from hako_amd.gpu import HakoGpuError
    dw, dx, do = gpu.alloc(4096), gpu.alloc(4096), gpu.alloc(4096)
    with pytest.raises(HakoGpuError, match="256"):
        gpu.matmul(do, dx, Q4, dw, None, 4, 100)
    with pytest.raises(HakoGpuError, match="256"):
        gpu.matmul(do, dx, Q6, dw, None, 4, 300)
    with pytest.raises(HakoGpuError, match="type"):
        gpu.matmul(do, dx, 7, dw, None, 4, 256)
    for b in (dw, dx, do):
        b.free()
