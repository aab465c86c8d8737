"""hako_amd — MI355X (gfx950) implementation of hako's quantized-matmul hot path.

The product is two in-tree shared libraries built by ``make -C hako_amd``:

* ``lib/libhako_gpu.so`` — hand-written gfx950 HIP kernels behind the plain C
  ABI of ``include/hako_gpu.h``;
* ``lib/libhako.so`` — a C11 drop-in for the reference's ``quant.h`` /
  ``nn.h`` surface, reaching the GPU only through that ABI.

This Python package is plumbing for tests and the bench: ``gpu`` is a ctypes
view of the C ABI, ``synth`` draws seeded workloads, ``mlf2`` writes and reads
the weight container.
"""
import os

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PACKAGE_DIR)
