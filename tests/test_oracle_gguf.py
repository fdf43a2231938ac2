"""Pins the GGUF oracle (oracle/gguf_ref.py): bytes assembled by hand from the
format description, round trips through the writer (tests/gguf_writer.py) over
every metadata type, header versions and alignments, the reader's rejection
rules, and the model-metadata rules. CPU only."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import gguf_writer as W
from oracle import gguf_ref as R

# A v3 file spelled out field by field: 1 tensor, 3 metadata entries.
KAT = bytes.fromhex(
    "47475546" "03000000"                                   # 'GGUF', version 3
    "0100000000000000" "0300000000000000"                   # 1 tensor, 3 kv
    "1400000000000000" + b"general.architecture".hex() +    # key
    "08000000" "0500000000000000" + b"qwen3".hex() +        # string "qwen3"
    "1100000000000000" + b"general.alignment".hex() +
    "04000000" "40000000" +                                 # u32 64
    "0400000000000000" + b"pi64".hex() +
    "0c000000" + struct.pack("<d", 3.25).hex() +            # f64 3.25
    "0100000000000000" + b"w".hex() +                       # tensor "w"
    "02000000" "0400000000000000" "0200000000000000"        # dims [4, 2]
    "00000000" "0000000000000000")                          # F32, offset 0


def test_hand_assembled_file():
    head = KAT
    pad = (-len(head)) % 64
    data = np.arange(8, dtype=np.float32).tobytes()
    g = R.read(head + b"\0" * pad + data)
    assert g["version"] == 3 and g["arch"] == "qwen3" and g["alignment"] == 64
    assert g["meta"]["general.alignment"] == 64.0 and g["meta"]["pi64"] == 3.25
    (t,) = g["tensors"]
    assert t["name"] == "w" and t["dims"] == [4, 2] and t["type"] == 0 and t["n_bytes"] == 32
    assert t["file_offset"] == len(head) + pad == g["data_start"] and g["data_start"] % 64 == 0
    # the writer produces the same bytes for the same content
    built = W.build([("general.architecture", W.STR, "qwen3"), ("general.alignment", W.U32, 64),
                     ("pi64", W.F64, 3.25)], [("w", [4, 2], 0, data)], alignment=64)
    assert built == head + b"\0" * pad + data


def test_round_trip_every_value_type():
    rng = np.random.default_rng(0)
    kv = [("general.architecture", W.STR, "qwen3"), ("u8", W.U8, 200), ("i8", W.I8, -100), ("u16", W.U16, 60000),
          ("i16", W.I16, -30000), ("u32", W.U32, 4000000000), ("i32", W.I32, -2000000000), ("f32", W.F32, 0.1),
          ("b0", W.BOOL, False), ("b1", W.BOOL, True), ("s", W.STR, "héllo"), ("u64", W.U64, 2 ** 60 + 1),
          ("i64", W.I64, -(2 ** 40)), ("f64", W.F64, 1e-300),
          ("arr", W.ARR, (W.I32, [1, -2, 3])), ("arrs", W.ARR, (W.STR, ["a", "", "ccc"])),
          ("nested", W.ARR, (W.ARR, [(W.U8, [1, 2]), (W.U8, [])]))]
    tensors = [(f"t{i}", dims, t, W.random_tensor(rng, t, dims)) for i, (dims, t) in
               enumerate([([256, 3], 12), ([512], 14), ([7], 0), ([32, 2], 8), ([4, 4, 2, 2], 1)])]
    for version in (1, 2, 3):
        for align in (8, 32, 256):
            extra = [] if align == 32 else [("general.alignment", W.U32, align)]
            g = R.read(W.build(kv + extra, tensors, version=version, alignment=align))
            m = g["meta"]
            assert m["u8"] == 200 and m["i8"] == -100 and m["u16"] == 60000 and m["i16"] == -30000
            assert m["u32"] == 4e9 and m["i32"] == -2e9 and m["f32"] == float(np.float32(0.1))
            assert m["b0"] is False and m["b1"] is True and m["s"] == "héllo"
            assert m["u64"] == float(2 ** 60 + 1) and m["i64"] == -(2.0 ** 40) and m["f64"] == 1e-300
            assert m["arr"] == [1.0, -2.0, 3.0] and m["arrs"] == ["a", "", "ccc"] and m["nested"] == [[1.0, 2.0], []]
            assert [t["name"] for t in g["tensors"]] == [t[0] for t in tensors]
            blob = W.build(kv + extra, tensors, version=version, alignment=align)
            for t, (name, dims, gt, raw) in zip(g["tensors"], tensors):
                assert t["dims"] == dims and t["type"] == gt and t["n_bytes"] == len(raw)
                assert t["file_offset"] % align == 0
                assert blob[t["file_offset"]:t["file_offset"] + t["n_bytes"]] == raw


def bad_files():
    """(label, bytes) of files the reference reader rejects."""
    arch = [("general.architecture", W.STR, "qwen3")]
    ok_t = [("w", [4], 0, bytes(16))]
    good = W.build(arch, ok_t)
    out = [("too small", good[:20]), ("bad magic", b"GGUX" + good[4:]),
           ("version 0", good[:4] + struct.pack("<I", 0) + good[8:]),
           ("version 4", good[:4] + struct.pack("<I", 4) + good[8:]),
           ("no architecture", W.build([("x", W.U8, 1)], ok_t)),
           ("alignment 12", W.build(arch + [("general.alignment", W.U32, 12)], ok_t, alignment=12)),
           ("alignment 0", W.build(arch + [("general.alignment", W.U32, 0)], ok_t)),
           ("bool 2", W.build(arch + [("b", W.BOOL, 2)], ok_t)),
           ("unknown value type", W.build(arch, ok_t)[:24] + b""),
           ("0 dims", W.build(arch, [("w", [], 0, b"")])),
           ("5 dims", W.build(arch, [("w", [1, 1, 1, 1, 4], 0, bytes(16))])),
           ("zero dim", W.build(arch, [("w", [0], 0, b"")])),
           ("dim 2^40", W.build(arch, [("w", [1 << 40], 0, b"")], offsets=[0])),
           ("unknown ggml type", W.build(arch, [("w", [4], 4, bytes(16))])),
           ("not a block multiple", W.build(arch, [("w", [100], 12, bytes(144))])),
           ("duplicate names", W.build(arch, [("w", [4], 0, bytes(16)), ("w", [4], 0, bytes(16))])),
           ("tensor past the end", W.build(arch, ok_t, offsets=[1 << 20])),
           ("truncated data", good[:-8]),
           ("truncated metadata", good[:30])]
    # an unknown metadata value type (13) spelled by hand
    blob = bytearray(W.build(arch, ok_t))
    raw = bytearray(b"GGUF" + struct.pack("<IQQ", 3, 0, 2) + W.gstr("general.architecture") +
                    struct.pack("<I", W.STR) + W.gstr("qwen3") + W.gstr("x") + struct.pack("<I", 13) + bytes(16))
    out = [o for o in out if o[0] != "unknown value type"] + [("unknown value type", bytes(raw))]
    del blob
    return out


@pytest.mark.parametrize("label,blob", bad_files(), ids=[b[0] for b in bad_files()])
def test_rejections(label, blob):
    with pytest.raises(R.GgufError):
        R.read(blob)


def test_model_meta_rules():
    rng = np.random.default_rng(1)
    blob, tensors, kv = W.qwen3_model(rng)
    m = R.model_meta(R.read(blob))
    assert (m["n_layers"], m["hidden"], m["n_heads"], m["n_kv_heads"], m["head_dim"], m["intermediate"],
            m["vocab"]) == (2, 256, 2, 1, 128, 512, 1000)
    assert m["rope_theta"] == 1e6 and m["rms_eps"] == float(np.float32(1e-6)) and m["context_length"] == 40960
    assert m["bos_id"] == 151643 and m["eos_id"] == 151645 and m["add_bos"] is False and not m["tied_embeddings"]
    assert m["weight_bytes"] == sum(len(t[3]) for t in tensors) and m["name"] == "synthetic-qwen3"
    # tied when neither output.weight nor lm_head.weight exists
    blob, _, _ = W.qwen3_model(rng, tied=True)
    assert R.model_meta(R.read(blob))["tied_embeddings"]
    # head_dim falls back to hidden / heads without key_length (here 256 / 2)
    blob, _, _ = W.qwen3_model(rng, key_length=False)
    m = R.model_meta(R.read(blob))
    assert m["head_dim"] == 128 and m["value_dim"] == 128
    # defaults: context 4096, theta 10000, eps 1e-6 when the keys are absent
    g = R.read(W.build([("general.architecture", W.STR, "qwen3"), ("qwen3.block_count", W.U32, 1),
                        ("qwen3.embedding_length", W.U32, 256), ("qwen3.attention.head_count", W.U32, 2),
                        ("qwen3.feed_forward_length", W.U32, 512)],
                       [("token_embd.weight", [256, 10], 0, bytes(256 * 10 * 4))]))
    m = R.model_meta(g)
    assert m["context_length"] == 4096 and m["rope_theta"] == 10000.0 and m["n_kv_heads"] == 2
    assert m["bos_id"] == -1 and m["name"] == "(unnamed)"
    # rejections
    for bad in ([("general.architecture", W.STR, "llama")],):
        with pytest.raises(R.GgufError):
            R.model_meta(R.read(W.build(bad, [("token_embd.weight", [4, 1], 0, bytes(16))])))
    blob, _, _ = W.qwen3_model(rng, extra_kv=[("qwen3.attention.head_count_kv", W.U32, 3)])
    with pytest.raises(R.GgufError):
        R.model_meta(R.read(blob))  # 2 heads are not a multiple of 3 kv heads (the later key wins)
