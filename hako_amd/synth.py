"""Seeded synthetic weights and activations in hako's verbatim block layouts.

No real checkpoints are available offline, so every workload is drawn here,
from numpy's PCG64 generator, with the distributions the benchmark
configurations specify:

* Q4_K super-block (144 B, reference src/quant.h:12-17): fp16 ``d`` and
  ``dmin`` uniform in [1e-3, 2e-2] (rounded to fp16 nearest-even), the 12
  packed scale/min bytes and the 128 nibble bytes uniform over 0..255.
* Q6_K super-block (210 B, reference src/quant.h:19-24): ``ql`` and ``qh``
  bytes uniform, the 16 int8 scales uniform in [-32, 31], fp16 ``d`` uniform
  in [1e-3, 1e-2].
* Activations: fp32 N(0, 1).
"""
from __future__ import annotations

import numpy as np

QK_K = 256
Q4K_BYTES = 144
Q6K_BYTES = 210
TYPE_F32, TYPE_F16, TYPE_Q4_K, TYPE_Q6_K = 0, 1, 12, 14


def row_nbytes(qtype: int, n_in: int) -> int:
    """Bytes in one row of ``n_in`` weights (reference src/nn.c:45-53)."""
    if qtype == TYPE_Q4_K:
        return n_in // QK_K * Q4K_BYTES
    if qtype == TYPE_Q6_K:
        return n_in // QK_K * Q6K_BYTES
    if qtype == TYPE_F16:
        return n_in * 2
    if qtype == TYPE_F32:
        return n_in * 4
    raise ValueError(f"unsupported type {qtype}")


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return v.astype(np.float16).view(np.uint8).reshape(-1, 2)


def q4k_blocks(rng: np.random.Generator, n_blocks: int,
               d_range=(1e-3, 2e-2)) -> np.ndarray:
    """``n_blocks`` Q4_K super-blocks as a uint8 array [n_blocks, 144]."""
    b = rng.integers(0, 256, size=(n_blocks, Q4K_BYTES), dtype=np.uint8)
    b[:, 0:2] = _f16_bytes(rng.uniform(*d_range, n_blocks))
    b[:, 2:4] = _f16_bytes(rng.uniform(*d_range, n_blocks))
    return b


def pack_scale_min(s: np.ndarray, m: np.ndarray) -> np.ndarray:
    """The 12-byte field of 6-bit (scale, min) pairs of Q4_K blocks, from
    s, m [n_blocks, 8] (values 0..63): sub-blocks 0-3 in the low six bits of
    bytes j (scale) and j+4 (min); sub-blocks 4-7 as the nibbles of byte j+4
    (scale low, min high) with their top two bits in bytes j-4 and j
    (the layout reference src/quant.c:57-66 decodes)."""
    s = np.asarray(s, np.uint8)
    m = np.asarray(m, np.uint8)
    b = np.zeros((s.shape[0], 12), np.uint8)
    b[:, 0:4] = (s[:, 0:4] & 63) | ((s[:, 4:8] >> 4) << 6)
    b[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    b[:, 8:12] = (s[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    return b


def q4k_blocks_centered(rng: np.random.Generator, n_blocks: int, d_range=(1e-3, 2e-2)) -> np.ndarray:
    """Q4_K super-blocks whose weights average about zero: dmin = d, scales
    s uniform in 1..8 and mins m = round(7.5 s), so a weight d*(s*q - m)
    with q uniform over 0..15 has mean d*(7.5 s - m), at most d/2. (Uniform
    scale and min bytes give every matrix a large mean, which a random model
    turns into one repeated greedy token.)"""
    b = rng.integers(0, 256, size=(n_blocks, Q4K_BYTES), dtype=np.uint8)
    d = _f16_bytes(rng.uniform(*d_range, n_blocks))
    b[:, 0:2] = d
    b[:, 2:4] = d
    s = rng.integers(1, 9, size=(n_blocks, 8))
    b[:, 4:16] = pack_scale_min(s, np.rint(7.5 * s).astype(np.int64))
    return b


def q6k_blocks(rng: np.random.Generator, n_blocks: int,
               d_range=(1e-3, 1e-2), scale_range=(-32, 31)) -> np.ndarray:
    """``n_blocks`` Q6_K super-blocks as a uint8 array [n_blocks, 210]."""
    b = rng.integers(0, 256, size=(n_blocks, Q6K_BYTES), dtype=np.uint8)
    lo, hi = scale_range
    b[:, 192:208] = rng.integers(lo, hi + 1, size=(n_blocks, 16)).astype(np.int8).view(np.uint8)
    b[:, 208:210] = _f16_bytes(rng.uniform(*d_range, n_blocks))
    return b


def q4k_weight(rng: np.random.Generator, n_out: int, n_in: int) -> np.ndarray:
    """Q4_K weight matrix [n_out, n_in/256*144] bytes, rows back to back."""
    assert n_in % QK_K == 0
    return q4k_blocks(rng, n_out * (n_in // QK_K)).reshape(n_out, -1)


def q6k_weight(rng: np.random.Generator, n_out: int, n_in: int) -> np.ndarray:
    """Q6_K weight matrix [n_out, n_in/256*210] bytes, rows back to back."""
    assert n_in % QK_K == 0
    return q6k_blocks(rng, n_out * (n_in // QK_K)).reshape(n_out, -1)


def weight(rng: np.random.Generator, qtype: int, n_out: int, n_in: int, centered: bool = False,
           scale: float = 1.0) -> np.ndarray:
    """A weight matrix of `qtype`; `centered` draws zero-mean Q4_K blocks,
    `scale` multiplies the d (and dmin) ranges of k-quant blocks."""
    nb = n_out * (n_in // QK_K)
    if qtype == TYPE_Q4_K:
        rq = (1e-3 * scale, 2e-2 * scale)
        if centered:
            return q4k_blocks_centered(rng, nb, rq).reshape(n_out, -1)
        return q4k_blocks(rng, nb, rq).reshape(n_out, -1) if scale != 1.0 else q4k_weight(rng, n_out, n_in)
    if qtype == TYPE_Q6_K:
        if scale != 1.0:
            return q6k_blocks(rng, nb, (1e-3 * scale, 1e-2 * scale)).reshape(n_out, -1)
        return q6k_weight(rng, n_out, n_in)
    if qtype == TYPE_F16:
        return rng.standard_normal((n_out, n_in)).astype(np.float16).view(np.uint8).reshape(n_out, -1)
    if qtype == TYPE_F32:
        return rng.standard_normal((n_out, n_in)).astype(np.float32).view(np.uint8).reshape(n_out, -1)
    raise ValueError(f"unsupported type {qtype}")


def activation(rng: np.random.Generator, n: int, rows: int | None = None) -> np.ndarray:
    """fp32 N(0,1) activation of length n (or [rows, n])."""
    shape = (n,) if rows is None else (rows, n)
    return rng.standard_normal(shape).astype(np.float32)
