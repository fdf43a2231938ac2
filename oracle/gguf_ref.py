"""Python restatement of the reference's GGUF reader and model-metadata rules.

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the native GGUF
reader and model upload, never by the product. Follows src/gguf.cc:74-167
(GgufFile::Open: header, metadata, tensor table, alignment, bounds),
src/gguf.cc:170-205 (MetaInt / MetaFloat / MetaBool / MetaStr over numbers kept
as doubles) and src/model_meta.cc:11-78 (ReadModelMeta). Parity pinned in
tests/test_oracle_gguf.py against bytes assembled by hand from the format
description, writer round trips and the rejection cases.
"""
from __future__ import annotations

import struct

# ggml type id -> (block elements, block bytes): the file-format table (reference src/quant.h:22-38)
BLOCKS = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
          9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
          15: (256, 292)}


class GgufError(ValueError):
    pass


class _Reader:
    def __init__(self, data: bytes):
        self.d = data
        self.p = 0

    def take(self, n: int) -> bytes:
        if n > len(self.d) - self.p:
            raise GgufError(f"truncated at {self.p}: need {n}")
        b = self.d[self.p:self.p + n]
        self.p += n
        return b

    def get(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.get("<Q")
        return self.take(n).decode("utf-8", "surrogateescape")


MAX_ARRAY_DEPTH = 64  # nesting bound of this build's reader (the reference recurses without one)


def _value(r: _Reader, t: int, depth: int = 0):
    """Numbers become float (as the reference's JSON doubles), then bool, str, list."""
    fmts = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}
    if t in fmts:
        return float(r.get(fmts[t]))
    if t == 7:
        b = r.get("<B")
        if b > 1:
            raise GgufError(f"bool {b}")
        return bool(b)
    if t == 8:
        return r.string()
    if t == 9:
        if depth >= MAX_ARRAY_DEPTH:
            raise GgufError("arrays nested too deep")
        et = r.get("<I")
        n = r.get("<Q")
        if n >= 1 << 32:
            raise GgufError("array too long")
        return [_value(r, et, depth + 1) for _ in range(n)]
    raise GgufError(f"unknown metadata type {t}")


def read(data: bytes) -> dict:
    """{version, meta (dict, insertion order, last duplicate wins), arch, alignment,
    data_start, tensors [{name, dims, type, offset, n_elements, n_bytes, file_offset}]}."""
    if len(data) < 24:
        raise GgufError("too small")
    r = _Reader(data)
    if r.get("<I") != 0x46554747:
        raise GgufError("bad magic")
    version = r.get("<I")
    if not 1 <= version <= 3:
        raise GgufError(f"version {version}")
    if version == 1:
        n_t, n_kv = r.get("<I"), r.get("<I")
    else:
        n_t, n_kv = r.get("<Q"), r.get("<Q")
    meta = {}
    for _ in range(n_kv):
        key = r.string()
        t = r.get("<I")
        meta[key] = _value(r, t)
    g = {"version": version, "meta": meta}
    arch = meta.get("general.architecture")
    if not isinstance(arch, str) or not arch:
        raise GgufError("no general.architecture")
    g["arch"] = arch
    align = meta_int(g, "general.alignment", 32)
    if not (0 < align <= 0xFFFFFFFF and align % 8 == 0):
        raise GgufError(f"alignment {align}")
    g["alignment"] = align
    tensors, names = [], set()
    for _ in range(n_t):
        name = r.string()
        nd = r.get("<I")
        if not 1 <= nd <= 4:
            raise GgufError(f"{nd} dims")
        dims = []
        for _ in range(nd):
            d = r.get("<Q")
            if not 0 < d < 1 << 40:
                raise GgufError(f"dim {d}")
            dims.append(d)
        t = r.get("<I")
        off = r.get("<Q")
        if t not in BLOCKS:
            raise GgufError(f"type {t}")
        n = 1
        for d in dims:
            n *= d
        if n > 1 << 62:
            raise GgufError("element count overflows")
        be, bb = BLOCKS[t]
        if n % be:
            raise GgufError("not a block multiple")
        if name in names:
            raise GgufError(f"duplicate {name}")
        names.add(name)
        tensors.append({"name": name, "dims": dims, "type": t, "offset": off, "n_elements": n,
                        "n_bytes": n // be * bb})
    start = (r.p + align - 1) // align * align
    if start > len(data):
        raise GgufError("data start past the end")
    for t in tensors:
        if start + t["offset"] + t["n_bytes"] > len(data):
            raise GgufError(f"tensor {t['name']} out of bounds")
        t["file_offset"] = start + t["offset"]
    g["data_start"] = start
    g["tensors"] = tensors
    return g


def meta_int(g: dict, key: str, default: int) -> int:
    v = g["meta"].get(key)
    if isinstance(v, bool):
        return int(v)
    if isinstance(v, float):
        return int(v)  # C++ float -> int64 conversion truncates toward zero
    return default


def meta_float(g: dict, key: str, default: float) -> float:
    v = g["meta"].get(key)
    return float(struct.unpack("<f", struct.pack("<f", v))[0]) if isinstance(v, float) and not isinstance(v, bool) \
        else default


def meta_bool(g: dict, key: str, default: bool) -> bool:
    v = g["meta"].get(key)
    if isinstance(v, bool):
        return v
    if isinstance(v, float):
        return int(v) != 0
    return default


def meta_str(g: dict, key: str, default: str = "") -> str:
    v = g["meta"].get(key)
    return v if isinstance(v, str) else default


def _i32(x: int) -> int:
    return (int(x) + 2 ** 31) % 2 ** 32 - 2 ** 31


def model_meta(g: dict) -> dict:
    """ReadModelMeta (src/model_meta.cc:11-78)."""
    if g["arch"] != "qwen3":
        raise GgufError("not qwen3")
    a = "qwen3."
    m = {"arch": g["arch"], "name": meta_str(g, "general.name", meta_str(g, "general.basename", "(unnamed)"))}
    m["n_layers"] = _i32(meta_int(g, a + "block_count", 0))
    m["hidden"] = _i32(meta_int(g, a + "embedding_length", 0))
    m["n_heads"] = _i32(meta_int(g, a + "attention.head_count", 0))
    m["n_kv_heads"] = _i32(meta_int(g, a + "attention.head_count_kv", m["n_heads"]))
    m["intermediate"] = _i32(meta_int(g, a + "feed_forward_length", 0))
    m["context_length"] = _i32(meta_int(g, a + "context_length", 4096))
    kl = meta_int(g, a + "attention.key_length", 0)
    if kl > 0:
        m["head_dim"] = _i32(kl)
    else:
        if not (m["n_heads"] > 0 and m["hidden"] % m["n_heads"] == 0):
            raise GgufError("no key_length and hidden not divisible")
        m["head_dim"] = m["hidden"] // m["n_heads"]
    m["value_dim"] = _i32(meta_int(g, a + "attention.value_length", m["head_dim"]))
    m["rope_theta"] = meta_float(g, a + "rope.freq_base", 10000.0)
    m["rms_eps"] = meta_float(g, a + "attention.layer_norm_rms_epsilon", float(struct.unpack("<f", struct.pack("<f", 1e-6))[0]))
    m["bos_id"] = _i32(meta_int(g, "tokenizer.ggml.bos_token_id", -1))
    m["eos_id"] = _i32(meta_int(g, "tokenizer.ggml.eos_token_id", -1))
    m["pad_id"] = _i32(meta_int(g, "tokenizer.ggml.padding_token_id", -1))
    m["add_bos"] = meta_bool(g, "tokenizer.ggml.add_bos_token", False)
    names = {t["name"]: t for t in g["tensors"]}
    if "token_embd.weight" not in names:
        raise GgufError("no token_embd.weight")
    emb = names["token_embd.weight"]
    m["vocab"] = _i32(emb["dims"][1] if len(emb["dims"]) >= 2 else 1)
    for k in ("n_layers", "hidden", "n_heads", "n_kv_heads", "head_dim", "intermediate", "vocab"):
        if m[k] <= 0:
            raise GgufError(f"incomplete metadata: {k}")
    if m["n_heads"] % m["n_kv_heads"]:
        raise GgufError("heads not a multiple of kv heads")
    if m["value_dim"] != m["head_dim"]:
        raise GgufError("value_length != key_length")
    m["tied_embeddings"] = "output.weight" not in names and "lm_head.weight" not in names
    m["weight_bytes"] = sum(t["n_bytes"] for t in g["tensors"])
    return m
