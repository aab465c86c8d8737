#!/usr/bin/env python3
"""Write the golden fixtures in tests/golden/ from the reference's own C path.

Runs in the build container only: it loads oracle/_ref/libhakm_ref.so, the
reference's quant.c/nn.c compiled unmodified by oracle/ref.mk with its
Makefile flags (-O3 -ffast-math; FTZ/DAZ come with that build). The fixtures
hold inputs and the reference's outputs, nothing else.

    make -f oracle/ref.mk && python3 tests/golden/make_golden.py

Fixtures:
  q4k_dequant.npz   Q4_K blocks -> dequant_q4_K (reference quant.c:68-92)
  q6k_dequant.npz   Q6_K blocks -> dequant_q6_K (reference quant.c:94-123)
  q8.npz            fp32 rows   -> quantize_row_q8_32 xq, xs (quant.c:127-144)
  q4k_isums.npz     Q4_K rows, xq -> per-sub-block Σq·xq and Σxq, recovered
                    exactly from q4k_vec_dot (quant.c:150-232) by crafted
                    headers and one-hot xs
  q4k_dot.npz       Q4_K rows, x -> q4k_vec_dot fp32 results
  matmul.npz        matmul (nn.c:179-210) on Q4_K (+bias), Q6_K, F16, F32
"""
from __future__ import annotations

import json
import os
import platform
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from hako_amd import synth  # noqa: E402
from oracle.hako_oracle import RefLib  # noqa: E402

SEED = 20261201


def f16bits(v: float) -> np.ndarray:
    return np.array([v], np.float16).view(np.uint8)


def q4k_special(rng) -> np.ndarray:
    """Edge-case Q4_K blocks: zero scales, saturated 6-bit fields, fp16
    subnormal / negative / largest d and dmin, every high-bit pattern."""
    out = []
    base = synth.q4k_blocks(rng, 12)
    b = base.copy()
    b[0, 0:4] = 0                                   # d = dmin = 0
    b[1, 4:16] = 0xFF                               # s = m = 63 everywhere
    b[2, 0:2] = [0x01, 0x00]                        # d = smallest subnormal
    b[2, 2:4] = [0xFF, 0x03]                        # dmin = largest subnormal
    b[3, 0:2] = f16bits(1.0); b[3, 2:4] = f16bits(1.0)
    b[4, 0:2] = f16bits(-1.0); b[4, 2:4] = f16bits(-0.5)
    b[5, 0:2] = [0xFF, 0x7B]; b[5, 2:4] = [0xFF, 0x7B]   # 65504
    b[6, 4:12] = 0xC0                               # only the spare top bits set
    b[6, 12:16] = 0x00
    b[7, 4:12] = 0x3F; b[7, 12:16] = 0xFF           # low six bits + nibbles set
    b[8, 16:144] = 0xFF                             # all nibbles 15
    b[9, 16:144] = 0x00                             # all nibbles 0
    b[10, 4:16] = np.arange(12, dtype=np.uint8) * 21
    out.append(b)
    return np.concatenate(out)


def q6k_special(rng) -> np.ndarray:
    b = synth.q6k_blocks(rng, 10, scale_range=(-128, 127))
    b[0, 208:210] = 0                               # d = 0
    b[1, 208:210] = [0x01, 0x00]                    # subnormal d
    b[2, 208:210] = f16bits(-1.0)
    b[3, 208:210] = [0xFF, 0x7B]                    # 65504
    b[3, 192:208] = np.array([-128, 127] * 8, np.int8).view(np.uint8)
    b[4, 0:192] = 0xFF                              # q = 63 everywhere
    b[5, 0:192] = 0x00                              # q = 0 everywhere (-32)
    b[6, 128:192] = 0xAA                            # qh pattern 10 10 10 10
    b[7, 128:192] = 0x55
    return b


def q8_rows(rng) -> np.ndarray:
    rows = [synth.activation(rng, 2048) for _ in range(6)]
    # amax known-answer block: amax bits 0x400861D9, xs = 0x3C8974C2 under the
    # compiled rounding (the literal reading gives 0x3C8974C3).
    kat = rng.standard_normal(32).astype(np.float32)
    kat = kat / np.abs(kat).max() * np.float32(1.5)
    kat[5] = np.array([0x400861D9], np.uint32).view(np.float32)[0]
    # ties: amax 127 -> inv exactly 1, x*inv = k + 1/2
    ties = (np.arange(32, dtype=np.float32) - 16.0) + np.float32(0.5)
    ties[0] = 127.0
    ties[1] = -126.5
    zeros = np.zeros(32, np.float32)
    one = np.zeros(32, np.float32); one[7] = -3.25
    neg0 = np.full(32, -0.0, np.float32); neg0[31] = 1e-3
    tiny = rng.standard_normal(32).astype(np.float32) * np.float32(1e-37)    # xs flushes to 0
    small = rng.standard_normal(32).astype(np.float32) * np.float32(2e-36)   # xs normal, inv huge
    sub = rng.standard_normal(32).astype(np.float32) * np.float32(1e-3)
    sub[::3] = np.array([0x00000001, 0x007FFFFF, 0x80400000], np.uint32).view(np.float32)[np.arange(11) % 3]
    big = rng.standard_normal(32).astype(np.float32) * np.float32(1e30)
    huge = np.full(32, 3.0e38, np.float32); huge[::2] *= -1
    edge = np.linspace(-1.0, 1.0, 32).astype(np.float32)
    special = np.concatenate([kat, ties, zeros, one, neg0, tiny, small, sub, big, huge, edge])
    special = np.concatenate([special, synth.activation(rng, 2048 - special.size)])
    rows.append(special)
    return np.stack(rows)


def crafted_isums(ref: RefLib, row: np.ndarray, n_in: int, xq: np.ndarray):
    """Recover Σq·xq and Σxq of every sub-block of `row` from q4k_vec_dot:
    d = 1, dmin = 0, every (s, m) = 1 and xs one-hot at sub-block j returns
    Σq·xq of j; d = 0, dmin = 1 returns -Σxq of j (both exact, |.| < 2^24)."""
    nb = n_in // 256
    blocks = row.reshape(nb, 144).copy()
    blocks[:, 4:8] = 1
    blocks[:, 8:12] = 1
    blocks[:, 12:16] = 0x11
    wa, wb = blocks.copy(), blocks.copy()
    wa[:, 0:2] = f16bits(1.0); wa[:, 2:4] = 0
    wb[:, 0:2] = 0; wb[:, 2:4] = f16bits(1.0)
    nsb = n_in // 32
    iqx = np.empty(nsb, np.int32)
    ix = np.empty(nsb, np.int32)
    for j in range(nsb):
        xs = np.zeros(nsb, np.float32)
        xs[j] = 1.0
        a = ref.q4k_vec_dot(wa, n_in, xq, xs)
        b = ref.q4k_vec_dot(wb, n_in, xq, xs)
        assert a == int(a) and b == int(b), (a, b)
        iqx[j], ix[j] = int(a), -int(b)
    return iqx, ix


def main():
    ref = RefLib(threads=4)
    rng = np.random.default_rng(SEED)
    meta = {"seed": SEED, "generator": "numpy PCG64 (default_rng)", "numpy": np.__version__,
            "reference_build": "oracle/ref.mk: gcc -O3 -std=c11 -ffast-math -pthread -march=x86-64-v3",
            "gcc": subprocess.run(["gcc", "--version"], capture_output=True, text=True).stdout.splitlines()[0],
            "host": platform.processor() or platform.machine()}

    # dequant
    q4 = np.concatenate([synth.q4k_blocks(rng, 40), q4k_special(rng)])
    np.savez(os.path.join(HERE, "q4k_dequant.npz"), blocks=q4,
             out=ref.dequant(synth.TYPE_Q4_K, q4, q4.shape[0] * 256))
    q6 = np.concatenate([synth.q6k_blocks(rng, 40), synth.q6k_blocks(rng, 8, scale_range=(-128, 127)),
                         q6k_special(rng)])
    np.savez(os.path.join(HERE, "q6k_dequant.npz"), blocks=q6,
             out=ref.dequant(synth.TYPE_Q6_K, q6, q6.shape[0] * 256))

    # q8 quantizer
    x = q8_rows(rng)
    xq = np.empty(x.shape, np.int8)
    xs = np.empty((x.shape[0], x.shape[1] // 32), np.float32)
    for r in range(x.shape[0]):
        xq[r], xs[r] = ref.quantize_q8_32(x[r])
    assert xs[6, 0].view(np.uint32) == 0x3C8974C2, hex(xs[6, 0].view(np.uint32))
    np.savez(os.path.join(HERE, "q8.npz"), x=x, xq=xq, xs=xs)

    # integer sums
    fx = {}
    for n_out, n_in in ((4, 2048), (2, 3584)):
        w = synth.q4k_weight(rng, n_out, n_in)
        xqv = rng.integers(-127, 128, size=n_in).astype(np.int8)
        xqv[:32] = 127
        xqv[32:64] = -127
        res = [crafted_isums(ref, w[r], n_in, xqv) for r in range(n_out)]
        fx[f"w_{n_in}"] = w
        fx[f"xq_{n_in}"] = xqv
        fx[f"iqx_{n_in}"] = np.stack([a for a, _ in res])
        fx[f"ix_{n_in}"] = np.stack([b for _, b in res])
    np.savez(os.path.join(HERE, "q4k_isums.npz"), **fx)

    # fp32 dot
    w = synth.q4k_weight(rng, 16, 2048)
    xd = synth.activation(rng, 2048)
    dq, ds = ref.quantize_q8_32(xd)
    dots = np.array([ref.q4k_vec_dot(w[r], 2048, dq, ds) for r in range(16)], np.float32)
    np.savez(os.path.join(HERE, "q4k_dot.npz"), w=w, x=xd, out=dots)

    # matmul, every weight type (first call has n_out >= threads: nn.c:182-184)
    mm = {}
    cases = [("q4k", synth.TYPE_Q4_K, 64, 2048, True), ("q6k", synth.TYPE_Q6_K, 64, 1024, False),
             ("q6k_long", synth.TYPE_Q6_K, 32, 11008, False), ("f16", synth.TYPE_F16, 32, 256, False),
             ("f32", synth.TYPE_F32, 32, 96, True)]
    for name, qt, n_out, n_in, with_bias in cases:
        w = synth.weight(rng, qt, n_out, n_in)
        xm = synth.activation(rng, n_in)
        bias = (0.1 * synth.activation(rng, n_out)) if with_bias else None
        mm[f"{name}_w"] = w
        mm[f"{name}_x"] = xm
        if bias is not None:
            mm[f"{name}_bias"] = bias
        mm[f"{name}_out"] = ref.matmul(qt, w, xm, n_out, n_in, bias)
        mm[f"{name}_shape"] = np.array([qt, n_out, n_in], np.int64)
    np.savez(os.path.join(HERE, "matmul.npz"), **mm)

    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump(meta, f, indent=1)
        f.write("\n")
    for fn in sorted(os.listdir(HERE)):
        if fn.endswith(".npz"):
            print(f"{fn}: {os.path.getsize(os.path.join(HERE, fn))} bytes")


if __name__ == "__main__":
    main()
