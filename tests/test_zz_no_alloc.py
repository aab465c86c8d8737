"""hako_gpu_matmul_batch_noalloc (include/hako_gpu.h): the multi-token matmul
with its scratch in a device array instead of library workspaces. It runs the
same kernels in the same order as hako_gpu_matmul_batch, so its outputs are
bit-identical to that entry point's. Each case makes two calls in a row
through the C ABI, the second with a smaller input (the scratch keeps the
first call's contents), and compares both with hako_gpu_matmul_batch.
"""
import numpy as np
import pytest

from hako_amd import synth

pytestmark = pytest.mark.gpu


def run(gpu, fn, qt, dw, x, m, n_out, n_in, bias=None):
    dx = gpu.upload(np.ascontiguousarray(x[:m]))
    dy = gpu.alloc(4 * m * n_out)
    db = None if bias is None else gpu.upload(bias)
    try:
        gpu.check(fn(dy.ptr, dx.ptr, qt, dw.ptr, None if db is None else db.ptr, m, n_out, n_in), fn.__name__)
        gpu.sync()
        return gpu.download(dy, np.float32, (m, n_out))
    finally:
        for b in (dx, dy, db):
            if b is not None:
                b.free()


# (type, n_in, [(m, n_out) of the two calls]): a GEMM-sized call, then a
# skinny one with fewer rows. The skinny Q4_K matmul splits K only past 4096
# inputs and the Q6_K one by its own rule: the 18944-wide Q4_K case and the
# Q6_K case keep split-K partials in the scratch, the other Q4_K cases
# reduce in LDS.
CASES = [
    (synth.TYPE_Q4_K, 3584, [(40, 4096), (9, 1024)]),
    (synth.TYPE_Q6_K, 4608, [(33, 1536), (6, 512)]),
    (synth.TYPE_Q4_K, 2048, [(16, 2560), (2, 256)]),
    (synth.TYPE_Q4_K, 18944, [(24, 512), (8, 256)]),
]


@pytest.mark.parametrize("qt,n_in,calls", CASES)
def test_noalloc_equals_matmul_batch(gpu, qt, n_in, calls):
    rng = np.random.default_rng(n_in + qt)
    n_max = max(n for _, n in calls)
    w = synth.weight(rng, qt, n_max, n_in)
    x = rng.standard_normal((max(m for m, _ in calls), n_in)).astype(np.float32)
    bias = rng.standard_normal(n_max).astype(np.float32)
    dw = gpu.upload(w)
    try:
        for m, n_out in calls:
            b = bias[:n_out]
            got = run(gpu, gpu.lib.hako_gpu_matmul_batch_noalloc, qt, dw, x, m, n_out, n_in, b)
            want = run(gpu, gpu.lib.hako_gpu_matmul_batch, qt, dw, x, m, n_out, n_in, b)
            assert np.all(np.isfinite(want))
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (qt, m, n_out)
    finally:
        dw.free()


def test_noalloc_refuses_more_than_its_scratch(gpu):
    """512 tokens of 32768 Q6_K inputs need 64 MiB of fp16 rows: refused before
    any launch, with the reason."""
    from hako_amd.gpu import HakoGpuError
    m, n_out, n_in = 512, 256, 32768
    dw = gpu.alloc(n_out * (n_in // 256) * 210)
    dx, dy = gpu.alloc(4 * m * n_in), gpu.alloc(4 * m * n_out)
    try:
        with pytest.raises(HakoGpuError, match="scratch"):
            gpu.check(gpu.lib.hako_gpu_matmul_batch_noalloc(dy.ptr, dx.ptr, synth.TYPE_Q6_K, dw.ptr, None, m,
                                                            n_out, n_in), "matmul_batch_noalloc")
    finally:
        for b in (dw, dx, dy):
            b.free()
