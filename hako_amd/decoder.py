"""ctypes view of the device decoder (include/hako_decode.h) over an MLF2 file.

The file's data section is mirrored into HBM verbatim (hako_gpu_mirror_upload)
and every tensor the reference's hakm_ctx_new resolves (src/model.c:30-57) is
handed to hako_gpu_decoder_create at its mirror address. Python only plumbs
pointers here; each step runs in the library.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import mlf2
from .gpu import Gpu

_vp, _i, _f = C.c_void_p, C.c_int, C.c_float


class Block(C.Structure):
    """hako_gpu_block (include/hako_decode.h)."""
    _fields_ = [("attn_norm", _vp), ("ffn_norm", _vp), ("wq", _vp), ("wk", _vp), ("wv", _vp), ("wo", _vp),
                ("bq", _vp), ("bk", _vp), ("bv", _vp), ("gate", _vp), ("up", _vp), ("down", _vp),
                ("t_q", _i), ("t_k", _i), ("t_v", _i), ("t_o", _i), ("t_gate", _i), ("t_up", _i), ("t_down", _i)]


class Model(C.Structure):
    """hako_gpu_model (include/hako_decode.h)."""
    _fields_ = [("n_layers", _i), ("d_model", _i), ("n_heads", _i), ("n_kv_heads", _i), ("head_dim", _i),
                ("ffn_dim", _i), ("vocab", _i), ("rope_theta", _f), ("rms_eps", _f), ("tok_embd", _vp),
                ("t_embd", _i), ("out_norm", _vp), ("out_weight", _vp), ("t_out", _i),
                ("blocks", C.POINTER(Block))]


class Decoder:
    """A device decoder for the MLF2 file at `path` (n_seq sequences of up to
    max_seq positions)."""

    def __init__(self, gpu: Gpu, path: str, n_seq: int = 1, max_seq: int = 2048):
        self.gpu, self.lib = gpu, gpu.lib
        why = mlf2.check(path)
        if why:
            raise ValueError(f"{path}: {why}")
        self.f = mlf2.Mlf2File(path)
        h = self.f.header
        start = h["data_off"]
        self.data = self.f.buf[start:]
        self.base = gpu.mirror_upload(self.data)
        self.n_seq, self.max_seq = n_seq, max_seq
        self.cfg = dict(n_layers=h["n_layers"], d_model=h["d_model"], n_heads=h["n_heads"],
                        n_kv_heads=h["n_kv_heads"], head_dim=h["head_dim"], ffn_dim=h["ffn_dim"], vocab=h["vocab"])
        self.kv_dim = h["n_kv_heads"] * h["head_dim"]

        def dev(name, required=True):
            t = self.f.tensors.get(name)
            if t is None:
                if required:
                    raise KeyError(name)
                return None, 0
            return self.base + int(t["data_off"]), int(t["type"])

        blocks = (Block * h["n_layers"])()
        for l in range(h["n_layers"]):
            b, p = blocks[l], f"blk.{l}."
            b.attn_norm = dev(p + "attn_norm.weight")[0]
            b.ffn_norm = dev(p + "ffn_norm.weight")[0]
            b.wq, b.t_q = dev(p + "attn_q.weight")
            b.wk, b.t_k = dev(p + "attn_k.weight")
            b.wv, b.t_v = dev(p + "attn_v.weight")
            b.wo, b.t_o = dev(p + "attn_output.weight")
            b.bq = dev(p + "attn_q.bias", False)[0]
            b.bk = dev(p + "attn_k.bias", False)[0]
            b.bv = dev(p + "attn_v.bias", False)[0]
            b.gate, b.t_gate = dev(p + "ffn_gate.weight")
            b.up, b.t_up = dev(p + "ffn_up.weight")
            b.down, b.t_down = dev(p + "ffn_down.weight")
        m = Model(n_layers=h["n_layers"], d_model=h["d_model"], n_heads=h["n_heads"], n_kv_heads=h["n_kv_heads"],
                  head_dim=h["head_dim"], ffn_dim=h["ffn_dim"], vocab=h["vocab"], rope_theta=h["rope_theta"],
                  rms_eps=h["rms_eps"])
        m.tok_embd, m.t_embd = dev("token_embd.weight")
        m.out_norm = dev("output_norm.weight")[0]
        if h["flags"] & mlf2.FLAG_TIED_EMBED:
            m.out_weight, m.t_out = m.tok_embd, m.t_embd
        else:
            m.out_weight, m.t_out = dev("output.weight")
        m.blocks = blocks
        d = _vp()
        try:
            gpu.check(self.lib.hako_gpu_decoder_create(C.byref(m), n_seq, max_seq, C.byref(d)), "decoder_create")
        except Exception:
            gpu.mirror_release(self.data)
            raise
        self.d = d.value

    def close(self):
        if self.d:
            self.gpu.check(self.lib.hako_gpu_decoder_destroy(self.d), "decoder_destroy")
            self.d = None
            self.gpu.mirror_release(self.data)

    def kv(self):
        """Device addresses of the K and V caches, [n_seq][n_layers][max_seq][kv_dim] fp32."""
        k, v = _vp(), _vp()
        self.gpu.check(self.lib.hako_gpu_decoder_kv(self.d, C.byref(k), C.byref(v)), "decoder_kv")
        return k.value, v.value

    def kv_offset(self, seq: int, layer: int, pos: int) -> int:
        """Byte offset of (seq, layer, pos) in either cache."""
        return 4 * ((seq * self.cfg["n_layers"] + layer) * self.max_seq + pos) * self.kv_dim

    def set_pos(self, pos):
        p = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (self.n_seq,)))
        self.gpu.check(self.lib.hako_gpu_decoder_set_pos(self.d, p.ctypes.data), "decoder_set_pos")

    def step(self, tokens, logits: bool = False):
        t = np.ascontiguousarray(np.broadcast_to(np.asarray(tokens, np.int32), (self.n_seq,)))
        nxt = np.empty(self.n_seq, np.int32)
        lg = np.empty((self.n_seq, self.cfg["vocab"]), np.float32) if logits else None
        self.gpu.check(self.lib.hako_gpu_decoder_step(self.d, t.ctypes.data, None if lg is None else lg.ctypes.data,
                                                      nxt.ctypes.data), "decoder_step")
        return (nxt, lg) if logits else nxt

    def generate(self, tokens, n: int) -> np.ndarray:
        t = np.ascontiguousarray(np.broadcast_to(np.asarray(tokens, np.int32), (self.n_seq,)))
        out = np.empty((n, self.n_seq), np.int32)
        self.gpu.check(self.lib.hako_gpu_decoder_generate(self.d, t.ctypes.data, n, out.ctypes.data),
                       "decoder_generate")
        return out

    def prefill(self, tokens, seq: int = 0, logits: bool = False):
        """Feed a prompt to sequence `seq` from its position; returns the
        greedy id after it (and the last prompt token's logits)."""
        t = np.ascontiguousarray(np.asarray(tokens, np.int32).reshape(-1))
        nxt = np.zeros(1, np.int32)
        lg = np.empty(self.cfg["vocab"], np.float32) if logits else None
        self.gpu.check(self.lib.hako_gpu_decoder_prefill(self.d, seq, t.ctypes.data, t.size,
                                                         None if lg is None else lg.ctypes.data, nxt.ctypes.data),
                       "decoder_prefill")
        return (int(nxt[0]), lg) if logits else int(nxt[0])

    def replay(self, n: int):
        self.gpu.check(self.lib.hako_gpu_decoder_replay(self.d, n), "decoder_replay")
