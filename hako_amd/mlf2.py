"""MLF2 container: writer for seeded synthetic Qwen2 models, and a reader.

Layout (reference include/mlf2.h:18-102; the converter's placement rules,
tools/gguf2mlf.py:138-150):

* a packed 128-byte header at offset 0;
* the tensor directory (104-byte packed entries) right after it;
* the tokenizer blob (here the empty one: two zero uint32 counts);
* the data section, 32-byte aligned, each tensor at a 32-byte aligned offset
  within it, its blocks copied verbatim.

Weights are random, not trained: norms 1 + 0.1*N(0,1), q/k/v biases
0.1*N(0,1), k-quant blocks as in ``synth``; every draw comes from one seeded
PCG64 stream, tensor by tensor in directory order.
"""
from __future__ import annotations

import dataclasses
import os
import struct

import numpy as np

from . import synth

HEADER_FMT = "<4sIIIIIIIIIIffIIQQQII36s"
HEADER_SIZE = 128
ENTRY_SIZE = 104
ALIGN = 32
FLAG_QKV_BIAS = 1
FLAG_TIED_EMBED = 2
assert struct.calcsize(HEADER_FMT) == HEADER_SIZE


@dataclasses.dataclass
class Qwen2Config:
    n_layers: int
    d_model: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn_dim: int
    vocab: int
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    ctx: int = 32768
    qkv_bias: bool = True
    tied: bool = True
    # weight types (Q4_K_M mix)
    attn_type: int = synth.TYPE_Q4_K
    gate_up_type: int = synth.TYPE_Q4_K
    down_type: int = synth.TYPE_Q6_K
    embd_type: int = synth.TYPE_Q6_K
    out_type: int = synth.TYPE_Q6_K
    # per-layer exceptions: ((layer, role), type) pairs, role one of attn_q,
    # attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down
    layer_types: tuple = ()
    # Q4_K matrices drawn with zero-mean weights (synth.q4k_blocks_centered):
    # the greedy tokens of such a random model change from step to step
    centered: bool = False
    # scale of the d (and dmin) ranges of the attn_output and ffn_down blocks:
    # below 1 each layer adds a smaller update to the residual stream
    resid_scale: float = 1.0


# The two model shapes the benchmarks use (Qwen2.5-3B and Qwen2-7B).
QWEN2_3B = Qwen2Config(n_layers=36, d_model=2048, n_heads=16, n_kv_heads=2, head_dim=128,
                       ffn_dim=11008, vocab=151936, tied=True, embd_type=synth.TYPE_Q6_K)
QWEN2_7B = Qwen2Config(n_layers=28, d_model=3584, n_heads=28, n_kv_heads=4, head_dim=128,
                       ffn_dim=18944, vocab=152064, tied=False, embd_type=synth.TYPE_Q4_K,
                       out_type=synth.TYPE_Q6_K)


def tensor_plan(cfg: Qwen2Config):
    """(name, type, n_in, n_out) of every tensor model.c resolves
    (reference src/model.c:30-57), in directory order. 1-D tensors have
    n_out = 1."""
    D, F, KV = cfg.d_model, cfg.ffn_dim, cfg.n_kv_heads * cfg.head_dim
    over = dict(cfg.layer_types)
    plan = [("token_embd.weight", cfg.embd_type, D, cfg.vocab)]
    for l in range(cfg.n_layers):
        p = f"blk.{l}."

        def t(role, default):
            return over.get((l, role), default)
        plan += [(p + "attn_norm.weight", synth.TYPE_F32, D, 1),
                 (p + "attn_q.weight", t("attn_q", cfg.attn_type), D, D),
                 (p + "attn_k.weight", t("attn_k", cfg.attn_type), D, KV),
                 (p + "attn_v.weight", t("attn_v", cfg.attn_type), D, KV)]
        if cfg.qkv_bias:
            plan += [(p + "attn_q.bias", synth.TYPE_F32, D, 1),
                     (p + "attn_k.bias", synth.TYPE_F32, KV, 1),
                     (p + "attn_v.bias", synth.TYPE_F32, KV, 1)]
        plan += [(p + "attn_output.weight", t("attn_output", cfg.attn_type), D, D),
                 (p + "ffn_norm.weight", synth.TYPE_F32, D, 1),
                 (p + "ffn_gate.weight", t("ffn_gate", cfg.gate_up_type), D, F),
                 (p + "ffn_up.weight", t("ffn_up", cfg.gate_up_type), D, F),
                 (p + "ffn_down.weight", t("ffn_down", cfg.down_type), F, D)]
    plan.append(("output_norm.weight", synth.TYPE_F32, D, 1))
    if not cfg.tied:
        plan.append(("output.weight", cfg.out_type, D, cfg.vocab))
    return plan


def _tensor_bytes(rng, name: str, qtype: int, n_in: int, n_out: int, centered: bool = False,
                  scale: float = 1.0) -> np.ndarray:
    if name.endswith("norm.weight"):
        v = (1.0 + 0.1 * rng.standard_normal(n_in)).astype(np.float32)
        return v.view(np.uint8)
    if name.endswith(".bias"):
        return (0.1 * rng.standard_normal(n_in)).astype(np.float32).view(np.uint8)
    return synth.weight(rng, qtype, n_out, n_in, centered, scale).reshape(-1)


def write_qwen2(path: str, cfg: Qwen2Config, seed: int) -> dict:
    """Write a synthetic Qwen2 MLF2 file; returns {name: (type, n_in, n_out,
    data_off, nbytes)}."""
    plan = tensor_plan(cfg)
    rng = np.random.default_rng(seed)
    tok_blob = struct.pack("<II", 0, 0)
    tensors_off = HEADER_SIZE
    tokenizer_off = tensors_off + ENTRY_SIZE * len(plan)
    data_off = (tokenizer_off + len(tok_blob) + ALIGN - 1) // ALIGN * ALIGN
    entries, cur = [], 0
    for name, qt, n_in, n_out in plan:
        nbytes = synth.row_nbytes(qt, n_in) * n_out
        entries.append((name, qt, n_in, n_out, cur, nbytes))
        cur += (nbytes + ALIGN - 1) // ALIGN * ALIGN
    flags = (FLAG_QKV_BIAS if cfg.qkv_bias else 0) | (FLAG_TIED_EMBED if cfg.tied else 0)
    hdr = struct.pack(HEADER_FMT, b"MLF2", 2, 0, cfg.n_layers, cfg.d_model, cfg.n_heads,
                      cfg.n_kv_heads, cfg.head_dim, cfg.ffn_dim, cfg.ctx, cfg.vocab,
                      cfg.rope_theta, cfg.rms_eps, flags, len(plan), tensors_off, tokenizer_off,
                      data_off, 0, 0, b"\0" * 36)
    with open(path, "wb") as f:
        f.write(hdr)
        for name, qt, n_in, n_out, off, nbytes in entries:
            one_d = n_out == 1 and qt == synth.TYPE_F32
            dims = (n_in, 0, 0, 0) if one_d else (n_in, n_out, 0, 0)
            f.write(name.encode().ljust(48, b"\0"))
            f.write(struct.pack("<II4QQQ", qt, 1 if one_d else 2, *dims, off, nbytes))
        f.write(tok_blob)
        f.write(b"\0" * (data_off - f.tell()))
        for name, qt, n_in, n_out, off, nbytes in entries:
            f.seek(data_off + off)
            scale = cfg.resid_scale if name.endswith(("attn_output.weight", "ffn_down.weight")) else 1.0
            f.write(_tensor_bytes(rng, name, qt, n_in, n_out, cfg.centered, scale).tobytes())
        f.truncate(data_off + cur)
    return {e[0]: e[1:] for e in entries}


class Mlf2File:
    """Read-only view of an MLF2 file (memory-mapped)."""

    def __init__(self, path: str):
        self.path = path
        self.buf = np.memmap(path, dtype=np.uint8, mode="r")
        h = struct.unpack_from(HEADER_FMT, self.buf[:HEADER_SIZE].tobytes())
        if h[0] != b"MLF2" or h[1] != 2:
            raise ValueError(f"{path}: not an MLF2 v2 file")
        keys = ["magic", "version", "arch", "n_layers", "d_model", "n_heads", "n_kv_heads", "head_dim",
                "ffn_dim", "ctx", "vocab", "rope_theta", "rms_eps", "flags", "n_tensors", "tensors_off",
                "tokenizer_off", "data_off", "bos_id", "eos_id"]
        self.header = dict(zip(keys, h[:-1]))
        self.tensors = {}
        off = self.header["tensors_off"]
        for i in range(self.header["n_tensors"]):
            e = self.buf[off + i * ENTRY_SIZE: off + (i + 1) * ENTRY_SIZE].tobytes()
            name = e[:48].rstrip(b"\0").decode()
            qt, nd, d0, d1, d2, d3, doff, nbytes = struct.unpack_from("<II4QQQ", e, 48)
            self.tensors[name] = dict(type=qt, dims=(d0, d1, d2, d3)[:nd], data_off=doff, nbytes=nbytes)

    def data(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        start = self.header["data_off"] + t["data_off"]
        return self.buf[start:start + t["nbytes"]]


def check_bytes(buf) -> str:
    """The library's structural check (hako_mlf2_check, include/hako_mlf2.h)
    of an MLF2 image held in `buf` (bytes, bytearray or a uint8 array): ''
    when it passes, else the reason."""
    import ctypes as C
    from hako_amd.gpu import HOST_LIB
    lib = C.CDLL(HOST_LIB)
    lib.hako_mlf2_check.restype = C.c_int
    lib.hako_mlf2_check.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]
    arr = np.frombuffer(buf, dtype=np.uint8) if not isinstance(buf, np.ndarray) else buf
    msg = C.create_string_buffer(256)
    rc = lib.hako_mlf2_check(arr.ctypes.data if arr.size else None, arr.size, msg, len(msg))
    return "" if rc == 0 else (msg.value.decode() or "rejected")


def check(path: str) -> str:
    """hako_mlf2_check of the file at `path` (memory-mapped)."""
    return check_bytes(np.memmap(path, dtype=np.uint8, mode="r"))
