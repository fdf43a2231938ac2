"""The native GGUF reader and ReadModelMeta (rpg_gguf_* in librpg_ops.so) against
the oracle (oracle/gguf_ref.py, pinned in test_oracle_gguf.py). Host code only:
runs without a GPU."""
from __future__ import annotations

import ctypes
import struct

import numpy as np
import pytest

import gguf_writer as W
from oracle import gguf_ref as R
from test_oracle_gguf import bad_files


@pytest.fixture(scope="module")
def ops():
    from rpgbarenginecuda_amd import ops as o

    o.load_library()
    return o


def write(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


def same_value(g, key, want, item=-1):
    got = g.meta(key, item)
    if isinstance(want, list):
        assert got == ("array", len(want)), key
        if item < 0:  # first-level items
            for i, w in enumerate(want):
                if isinstance(w, list):
                    assert g.meta(key, i) == ("array", len(w))
                else:
                    assert g.meta(key, i) == w, (key, i)
        return
    assert type(got) is type(want) and got == want, (key, got, want)


def check_against_oracle(ops, path, blob):
    want = R.read(blob)
    with ops.GgufFile(path) as g:
        tensors = g.tensors()
        assert [t["name"] for t in tensors] == [t["name"] for t in want["tensors"]]
        for t, w in zip(tensors, want["tensors"]):
            assert t["dims"] == w["dims"] and t["type"] == w["type"] and t["n_bytes"] == w["n_bytes"]
            assert t["n_elements"] == w["n_elements"] and t["file_offset"] == w["file_offset"]
            assert ctypes.string_at(t["data"], t["n_bytes"]) == blob[w["file_offset"]:w["file_offset"] + w["n_bytes"]]
        for key, val in want["meta"].items():
            same_value(g, key, val)
        assert g.meta("no.such.key") is None
        assert "GGUF v%d" % want["version"] in g.describe()
        if want["arch"] == "qwen3":
            try:
                m = R.model_meta(want)
            except R.GgufError:
                with pytest.raises(ops.RpgError):
                    g.model_meta()
            else:
                got = g.model_meta()
                for k, v in m.items():
                    assert got[k] == v, (k, got[k], v)


def test_files_match_oracle(ops, tmp_path):
    rng = np.random.default_rng(11)
    cases = []
    for version in (1, 2, 3):
        for align in (32, 64):
            cases.append(W.qwen3_model(rng, version=version, alignment=align)[0])
    cases.append(W.qwen3_model(rng, tied=True)[0])
    cases.append(W.qwen3_model(rng, key_length=False)[0])
    cases.append(W.qwen3_model(rng, extra_kv=[("qwen3.attention.head_count_kv", W.U32, 3)])[0])  # meta rejects
    kv = [("general.architecture", W.STR, "qwen3"), ("u64", W.U64, 2 ** 60 + 1), ("i8", W.I8, -5),
          ("f64", W.F64, -0.5), ("b", W.BOOL, True), ("s", W.STR, "x" * 1000),
          ("nested", W.ARR, (W.ARR, [(W.U8, [1, 2]), (W.STR, ["q"])])), ("dup", W.U8, 1), ("dup", W.STR, "second")]
    cases.append(W.build(kv, [("a", [32, 3], 8, W.random_tensor(rng, 8, [32, 3])),
                              ("b", [2, 2, 2, 2], 1, W.random_tensor(rng, 1, [2, 2, 2, 2]))]))
    for i, blob in enumerate(cases):
        check_against_oracle(ops, write(tmp_path, f"c{i}.gguf", blob), blob)


@pytest.mark.parametrize("label,blob", bad_files(), ids=[b[0] for b in bad_files()])
def test_native_rejects_what_the_reference_rejects(ops, tmp_path, label, blob):
    path = write(tmp_path, "bad.gguf", blob)
    with pytest.raises(ops.RpgError):
        ops.GgufFile(path)


def test_open_errors(ops, tmp_path):
    with pytest.raises(ops.RpgError, match="cannot open"):
        ops.GgufFile(str(tmp_path / "missing.gguf"))
    with pytest.raises(ops.RpgError, match="empty"):
        ops.GgufFile(write(tmp_path, "empty.gguf", b""))
    rng = np.random.default_rng(2)
    blob, _, _ = W.qwen3_model(rng)
    with ops.GgufFile(write(tmp_path, "m.gguf", blob)) as g:
        with pytest.raises(ops.RpgError, match="not an array"):
            g.meta("general.name", 0)
        with pytest.raises(ops.RpgError, match="out of range"):
            g.meta("tokenizer.ggml.tokens", 8)
    llama = W.build([("general.architecture", W.STR, "llama")], [("token_embd.weight", [4, 1], 0, bytes(16))])
    with ops.GgufFile(write(tmp_path, "l.gguf", llama)) as g:
        with pytest.raises(ops.RpgError, match="qwen3"):
            g.model_meta()


def _raw_kv_file(key: str, value_bytes: bytes) -> bytes:
    """A v3 GGUF with general.architecture, one extra key whose type + value bytes
    are given raw (so counts can lie), no tensors, and 64 bytes of padding."""
    body = W.gstr("general.architecture") + struct.pack("<I", W.STR) + W.gstr("qwen3")
    body += W.gstr(key) + value_bytes
    return b"GGUF" + struct.pack("<IQQ", 3, 0, 2) + body + bytes(64)  # + room for the aligned data start


def test_forged_array_count_fails_as_truncation(ops, tmp_path):
    """An array claiming 2^32 - 1 u32 items with 72 bytes left: rejected as
    truncated before anything is allocated for it (both readers)."""
    blob = _raw_kv_file("big", struct.pack("<IIQ", W.ARR, W.U32, (1 << 32) - 1) + bytes(8))
    with pytest.raises(ops.RpgError, match="truncated"):
        ops.GgufFile(write(tmp_path, "big.gguf", blob))
    with pytest.raises(R.GgufError):
        R.read(blob)


def _nested(depth: int) -> bytes:
    """Type + value bytes of `depth` arrays nested one in another around one u8."""
    inner = struct.pack("<IQ", W.U8, 1) + b"\x07"
    for _ in range(depth - 1):
        inner = struct.pack("<IQ", W.ARR, 1) + inner
    return struct.pack("<I", W.ARR) + inner


def test_array_nesting_is_bounded(ops, tmp_path):
    ok = _raw_kv_file("deep", _nested(64))
    g = ops.GgufFile(write(tmp_path, "ok.gguf", ok))
    g.close()
    assert R.read(ok)["meta"]["deep"] is not None
    deep = _raw_kv_file("deep", _nested(65))
    with pytest.raises(ops.RpgError, match="levels deep"):
        ops.GgufFile(write(tmp_path, "deep.gguf", deep))
    with pytest.raises(R.GgufError):
        R.read(deep)
    huge = _raw_kv_file("deep", _nested(100000))  # would exhaust the stack without the bound
    with pytest.raises(ops.RpgError, match="levels deep"):
        ops.GgufFile(write(tmp_path, "huge.gguf", huge))
