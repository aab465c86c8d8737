"""The MLF2 container: the writer of the synthetic Qwen2 files and the
library's structural check (hako_mlf2_check).

Pins: files the writer produces pass the check and load in the reference's
own loader and model lookup (src/loader.c:12-52, src/model.c:30-57, compiled
from its sources); every corruption the reference loader refuses (size,
magic, version, section offsets) the check refuses too; and each rule the
check adds (types, nbytes, alignment, bounds, names, model tensors, the
tokenizer records) refuses a file broken in exactly that way.
"""
import ctypes as C
import os
import struct

import numpy as np
import pytest

from hako_amd import mlf2, synth

CONFIGS = {
    "tied_bias": mlf2.Qwen2Config(n_layers=2, d_model=256, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512,
                                  vocab=512, ctx=64),
    "untied_q4_embd": mlf2.Qwen2Config(n_layers=1, d_model=512, n_heads=4, n_kv_heads=1, head_dim=128,
                                       ffn_dim=768, vocab=300, ctx=64, tied=False, embd_type=synth.TYPE_Q4_K),
    "no_bias_f16": mlf2.Qwen2Config(n_layers=1, d_model=256, n_heads=2, n_kv_heads=2, head_dim=128, ffn_dim=256,
                                    vocab=256, ctx=64, qkv_bias=False, attn_type=synth.TYPE_F16,
                                    gate_up_type=synth.TYPE_F32, down_type=synth.TYPE_Q4_K),
}


# header field offsets (packed, include/mlf2.h:55-77)
HDR_FLAGS, HDR_N_TENSORS, HDR_TENSORS_OFF, HDR_TOKENIZER_OFF, HDR_DATA_OFF = 52, 56, 60, 68, 76


def ref_lib():
    from oracle.hako_oracle import REF_LIB
    if not os.path.exists(REF_LIB):
        pytest.skip("reference library not built")
    lib = C.CDLL(REF_LIB)
    lib.hakm_ctx_new.restype = C.c_void_p
    lib.hakm_ctx_new.argtypes = [C.c_char_p, C.c_int]
    lib.hakm_ctx_free.argtypes = [C.c_void_p]
    return lib


def ref_accepts(lib, path) -> bool:
    ctx = lib.hakm_ctx_new(str(path).encode(), 16)
    if ctx:
        lib.hakm_ctx_free(ctx)
    return bool(ctx)


@pytest.fixture(scope="module")
def image(tmp_path_factory):
    path = tmp_path_factory.mktemp("mlf2") / "m.mlf2"
    mlf2.write_qwen2(str(path), CONFIGS["tied_bias"], 3)
    return path, bytes(open(path, "rb").read())


def entry_off(buf, name):
    tensors_off, n = struct.unpack_from("<Q", buf, HDR_TENSORS_OFF)[0], struct.unpack_from("<I", buf, HDR_N_TENSORS)[0]
    for i in range(n):
        off = tensors_off + i * mlf2.ENTRY_SIZE
        if buf[off:off + 48].rstrip(b"\0").decode() == name:
            return off
    raise KeyError(name)


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_written_files_pass_and_load_in_the_reference(tmp_path, name):
    path = tmp_path / "m.mlf2"
    mlf2.write_qwen2(str(path), CONFIGS[name], 1)
    assert mlf2.check(str(path)) == ""
    assert ref_accepts(ref_lib(), path)


# corruptions the reference loader itself refuses (src/loader.c:26-43)
def _truncate_header(b):
    return b[:100]


def _magic(b):
    b[0:4] = b"MLF3"
    return b


def _version(b):
    struct.pack_into("<I", b, 4, 3)
    return b


def _tensors_off(b):
    struct.pack_into("<Q", b, HDR_TENSORS_OFF, len(b) + 8)
    return b


def _data_off(b):
    struct.pack_into("<Q", b, HDR_DATA_OFF, len(b) + 64)
    return b


REF_REFUSED = {"file too small": _truncate_header, "bad magic": _magic, "version": _version,
               "directory": _tensors_off, "data offset": _data_off}


@pytest.mark.parametrize("what", sorted(REF_REFUSED))
def test_check_refuses_what_the_reference_refuses(image, tmp_path, what):
    path, img = image
    bad = REF_REFUSED[what](bytearray(img))
    p = tmp_path / "bad.mlf2"
    p.write_bytes(bytes(bad))
    assert not ref_accepts(ref_lib(), p)
    assert what in mlf2.check_bytes(bytes(bad))


def _entry(b, name, fmt, rel, value):
    struct.pack_into(fmt, b, entry_off(b, name) + rel, value)
    return b


# entry fields: name @0, type @48, n_dims @52, dims @56.., data_off @88, nbytes @96
ADDED_RULES = {
    "arch": (lambda b: struct.pack_into("<I", b, 8, 1) or b, "architecture"),
    "head_shape": (lambda b: struct.pack_into("<I", b, 28, 32) or b, "head_dim"),
    "flags": (lambda b: struct.pack_into("<I", b, HDR_FLAGS, 0x10) or b, "flags"),
    "data_misaligned": (lambda b: struct.pack_into("<Q", b, HDR_DATA_OFF,
                                                   struct.unpack_from("<Q", b, HDR_DATA_OFF)[0] - 8) or b,
                        "aligned"),
    "type": (lambda b: _entry(b, "blk.0.attn_q.weight", "<I", 48, 7), "unknown type"),
    "nbytes": (lambda b: _entry(b, "blk.0.ffn_up.weight", "<Q", 96, 1000), "nbytes"),
    "q4_row": (lambda b: _entry(b, "blk.1.attn_k.weight", "<Q", 56, 200), "blocks"),
    "n_dims": (lambda b: _entry(b, "blk.0.attn_norm.weight", "<I", 52, 5), "n_dims"),
    "dims_past_n_dims": (lambda b: _entry(b, "output_norm.weight", "<Q", 64, 3), "past n_dims"),
    "tensor_misaligned": (lambda b: _entry(b, "blk.0.ffn_gate.weight", "<Q", 88,
                                           struct.unpack_from("<Q", b, entry_off(b, "blk.0.ffn_gate.weight") + 88)[0]
                                           + 4), "aligned"),
    "past_end": (lambda b: b[:len(b) - 64], "past the data section"),
    "name": (lambda b: b.__setitem__(slice(entry_off(b, "blk.0.attn_v.weight"),
                                           entry_off(b, "blk.0.attn_v.weight") + 48), b"x" * 48) or b,
             "not terminated"),
    "duplicate": (lambda b: b.__setitem__(slice(entry_off(b, "blk.1.ffn_up.weight"),
                                                entry_off(b, "blk.1.ffn_up.weight") + 48),
                                          b"blk.1.ffn_gate.weight".ljust(48, b"\0")) or b, "twice"),
    "missing": (lambda b: b.__setitem__(slice(entry_off(b, "blk.1.ffn_down.weight"),
                                              entry_off(b, "blk.1.ffn_down.weight") + 48),
                                        b"blk.1.ffn_dawn.weight".ljust(48, b"\0")) or b,
                "missing tensor blk.1.ffn_down.weight"),
    # self-consistent entries (nbytes matching) that break the model's shape
    "model_dims": (lambda b: _entry(_entry(b, "blk.0.attn_k.weight", "<Q", 64, 64), "blk.0.attn_k.weight", "<Q", 96,
                                    64 * 144), "blk.0.attn_k.weight: dims"),
    "norm_type": (lambda b: _entry(_entry(b, "blk.1.ffn_norm.weight", "<I", 48, 1), "blk.1.ffn_norm.weight", "<Q",
                                   96, 512), "expected F32"),
    "tokenizer": (lambda b: struct.pack_into("<I", b, struct.unpack_from("<Q", b, HDR_TOKENIZER_OFF)[0], 1000) or b,
                  "tokenizer"),
}


@pytest.mark.parametrize("what", sorted(ADDED_RULES))
def test_check_refuses_each_broken_rule(image, what):
    _, img = image
    fn, expect = ADDED_RULES[what]
    bad = fn(bytearray(img))
    msg = mlf2.check_bytes(bytes(bad))
    assert expect in msg, msg


def test_bias_flag_requires_the_biases(tmp_path):
    path = tmp_path / "m.mlf2"
    mlf2.write_qwen2(str(path), CONFIGS["no_bias_f16"], 2)
    b = bytearray(path.read_bytes())
    assert mlf2.check_bytes(bytes(b)) == ""
    struct.pack_into("<I", b, HDR_FLAGS, struct.unpack_from("<I", b, HDR_FLAGS)[0] | mlf2.FLAG_QKV_BIAS)
    assert "missing tensor blk.0.attn_q.bias" in mlf2.check_bytes(bytes(b))


def test_tokenizer_records_are_walked(image):
    """A blob of real records (type, length, bytes; then merges) passes; a
    last record one byte longer than its section fails."""
    _, img = image
    toks, merges = [b"a", b"bc", b"\xc4\xa0the"], [b"a b"]
    blob = struct.pack("<II", len(toks), len(merges))
    for t in toks:
        blob += struct.pack("<BI", 1, len(t)) + t
    for m in merges:
        blob += struct.pack("<I", len(m)) + m
    b = bytearray(img)
    tok_off = struct.unpack_from("<Q", b, HDR_TOKENIZER_OFF)[0]
    data_off = struct.unpack_from("<Q", b, HDR_DATA_OFF)[0]
    shift = (len(blob) + 31) // 32 * 32     # keeps the data section 32-byte aligned
    nb = b[:tok_off] + blob + b"\0" * (data_off - tok_off + shift - len(blob)) + b[data_off:]
    struct.pack_into("<Q", nb, HDR_DATA_OFF, data_off + shift)
    assert mlf2.check_bytes(bytes(nb)) == ""
    room = data_off + shift - tok_off
    # the merge record's length reaching one byte past the section
    merge_len_at = tok_off + len(blob) - len(merges[0]) - 4
    struct.pack_into("<I", nb, merge_len_at, room - (merge_len_at + 4 - tok_off) + 1)
    assert "tokenizer record 3 truncated" in mlf2.check_bytes(bytes(nb))
