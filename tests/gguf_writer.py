"""GGUF writer built from the published format description (ggml docs/gguf.md,
versions 1-3) -- test infrastructure for the GGUF reader and the model upload.

Layout written: magic 'GGUF' | version u32 | tensor_count, kv_count (u32 in v1,
u64 later) | kv entries (u64-length key, u32 value type, value) | tensor infos
(name, u32 n_dims, u64 dims (fastest first), u32 ggml type, u64 offset) |
padding to the alignment | tensor data, each tensor at an aligned offset from the
start of the data section.
"""
from __future__ import annotations

import struct

import numpy as np

import synth

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}

# ggml type ids and block shapes (elements, bytes)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 8, 12, 14
BLOCKS = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
          9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
          15: (256, 292)}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STR:
        return gstr(v)
    if t == ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(value(et, x) for x in items)
    if t == BOOL:
        return struct.pack("<B", int(v))
    return struct.pack(_FMT[t], v)


def tensor_bytes(ggml_type: int, dims) -> int:
    e, b = BLOCKS[ggml_type]
    n = int(np.prod(dims))
    assert n % e == 0
    return n // e * b


def build(kv, tensors, version: int = 3, alignment: int = 32, offsets=None, pad_data: int = 0) -> bytes:
    """kv: [(key, type, value)]; tensors: [(name, dims, ggml_type, raw bytes)].
    `alignment` places the data (the caller adds general.alignment to kv when it
    is not 32); `offsets` overrides the tensor offsets and leaves the data
    section empty (for malformed files)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<I", version)
    out += struct.pack("<II", len(tensors), len(kv)) if version == 1 else struct.pack("<QQ", len(tensors), len(kv))
    for key, t, v in kv:
        out += gstr(key) + struct.pack("<I", t) + value(t, v)
    offs = []
    cur = 0
    for name, dims, gt, raw in tensors:
        cur = (cur + alignment - 1) // alignment * alignment
        offs.append(cur)
        cur += len(raw)
    if offsets is not None:
        offs = list(offsets)
    for (name, dims, gt, raw), off in zip(tensors, offs):
        out += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", gt, off)
    out += b"\0" * ((-len(out)) % alignment)
    data = bytearray()
    for (name, dims, gt, raw), off in zip(tensors, offs):
        if offsets is None:
            data += b"\0" * (off - len(data))
            data += raw
    # with explicit offsets (malformed files) no tensor data is written, only `pad_data` zero bytes
    return bytes(out + data + b"\0" * pad_data)


def random_tensor(rng: np.random.Generator, ggml_type: int, dims, model_like: bool = False) -> bytes:
    """Random tensor bytes. model_like: matrices with zero-mean, trained-weight-like
    values (synth.model_table) instead of the benchmark's uniform blocks."""
    rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
    cols = int(dims[0])
    if model_like and len(dims) > 1 and ggml_type in (GGML_F32, GGML_Q4_K, GGML_Q6_K):
        return synth.model_table(rng, ggml_type, rows, cols).tobytes()
    if ggml_type == GGML_F32:
        return rng.normal(1.0, 0.1, size=rows * cols).astype(np.float32).tobytes()
    if ggml_type == GGML_F16:
        return rng.normal(1.0, 0.1, size=rows * cols).astype(np.float16).tobytes()
    if ggml_type in (GGML_Q4_K, GGML_Q6_K):
        return synth.quant_table(rng, ggml_type, rows, cols).tobytes()
    return rng.integers(0, 256, size=tensor_bytes(ggml_type, dims), dtype=np.uint8).tobytes()


def byte_to_unicode() -> dict:
    """The byte -> character map of byte-level BPE vocabularies (GPT-2's, used by
    Qwen): printable Latin-1 bytes stand for themselves, every other byte b is
    the character 256 + (its rank among those bytes)."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAD)) + list(range(0xAE, 0x100))
    out, extra = {}, 0
    for b in range(256):
        if b in keep:
            out[b] = chr(b)
        else:
            out[b] = chr(256 + extra)
            extra += 1
    return out


CHATML_SPECIALS = ("<|endoftext|>", "<|im_start|>", "<|im_end|>")


def ascii_bpe_vocab(n_vocab: int):
    """A byte-level BPE vocabulary whose every token decodes to ASCII: one token
    per printable byte and newline, the ChatML control tokens (type 3), then
    filler tokens "x<i>" up to n_vocab, and one merge ("z q") that no test text
    contains. Returns (tokens, types, merges)."""
    b2u = byte_to_unicode()
    tokens = [b2u[b] for b in [10] + list(range(0x20, 0x7F))]
    types = [1] * len(tokens)
    tokens += list(CHATML_SPECIALS)
    types += [3] * len(CHATML_SPECIALS)
    tokens.append("zq")
    types.append(1)
    i = len(tokens)
    while len(tokens) < n_vocab:
        tokens.append(f"x{i}")
        types.append(1)
        i += 1
    return tokens, types, ["z q"]


def tokenizer_kv(n_vocab: int):
    """GGUF tokenizer metadata for ascii_bpe_vocab: tokens, token types, merges,
    eos = <|im_end|>, bos = <|endoftext|> (not prepended)."""
    tokens, types, merges = ascii_bpe_vocab(n_vocab)
    return [("tokenizer.ggml.model", STR, "gpt2"), ("tokenizer.ggml.tokens", ARR, (STR, tokens)),
            ("tokenizer.ggml.token_type", ARR, (I32, types)), ("tokenizer.ggml.merges", ARR, (STR, merges)),
            ("tokenizer.ggml.bos_token_id", U32, tokens.index("<|endoftext|>")),
            ("tokenizer.ggml.eos_token_id", U32, tokens.index("<|im_end|>")),
            ("tokenizer.ggml.padding_token_id", U32, tokens.index("<|endoftext|>"))]


def qwen3_model(rng: np.random.Generator, n_layers=2, hidden=256, n_heads=2, n_kv_heads=1, head_dim=128,
                inter=512, vocab=1000, tied=False, version=3, alignment=32, mat_type=None, norm_type=GGML_F32,
                key_length=True, extra_kv=(), drop=(), override=None, model_like=False, tokenizer=False):
    """(bytes, tensors, kv) of a synthetic qwen3 GGUF with Q4_K / Q6_K matrices
    (Q4_K_M-like: attn_v, ffn_down and the embeddings Q6_K, the rest Q4_K).
    model_like: zero-mean weights of trained-model size, for forward tests.
    tokenizer: replace the placeholder token list with tokenizer_kv(vocab)."""
    kv = [("general.architecture", STR, "qwen3"), ("general.name", STR, "synthetic-qwen3"),
          ("qwen3.block_count", U32, n_layers), ("qwen3.embedding_length", U32, hidden),
          ("qwen3.attention.head_count", U32, n_heads), ("qwen3.attention.head_count_kv", U32, n_kv_heads),
          ("qwen3.feed_forward_length", U32, inter), ("qwen3.context_length", U32, 40960),
          ("qwen3.rope.freq_base", F32, 1000000.0), ("qwen3.attention.layer_norm_rms_epsilon", F32, 1e-6),
          ("tokenizer.ggml.bos_token_id", U32, 151643), ("tokenizer.ggml.eos_token_id", U32, 151645),
          ("tokenizer.ggml.padding_token_id", U32, 151643), ("tokenizer.ggml.add_bos_token", BOOL, False),
          ("tokenizer.ggml.tokens", ARR, (STR, [f"t{i}" for i in range(8)]))]
    if tokenizer:
        tok = tokenizer_kv(vocab)
        names = {k for k, _, _ in tok}
        kv = [e for e in kv if e[0] not in names] + tok
    if key_length:
        kv += [("qwen3.attention.key_length", U32, head_dim), ("qwen3.attention.value_length", U32, head_dim)]
    if alignment != 32:
        kv.append(("general.alignment", U32, alignment))
    kv += list(extra_kv)
    q, kvd = n_heads * head_dim, n_kv_heads * head_dim

    def mt(name, default):
        if override and name in override:
            return override[name]
        return mat_type if mat_type is not None else default

    specs = [("token_embd.weight", [hidden, vocab], mt("token_embd.weight", GGML_Q6_K))]
    if not tied:
        specs.append(("output.weight", [hidden, vocab], mt("output.weight", GGML_Q6_K)))
    specs.append(("output_norm.weight", [hidden], norm_type))
    for layer in range(n_layers):
        p = f"blk.{layer}."
        specs += [(p + "attn_norm.weight", [hidden], norm_type), (p + "ffn_norm.weight", [hidden], norm_type),
                  (p + "attn_q_norm.weight", [head_dim], GGML_F32), (p + "attn_k_norm.weight", [head_dim], GGML_F32),
                  (p + "attn_q.weight", [hidden, q], mt(p + "attn_q.weight", GGML_Q4_K)),
                  (p + "attn_k.weight", [hidden, kvd], mt(p + "attn_k.weight", GGML_Q4_K)),
                  (p + "attn_v.weight", [hidden, kvd], mt(p + "attn_v.weight", GGML_Q6_K)),
                  (p + "attn_output.weight", [q, hidden], mt(p + "attn_output.weight", GGML_Q4_K)),
                  (p + "ffn_gate.weight", [hidden, inter], mt(p + "ffn_gate.weight", GGML_Q4_K)),
                  (p + "ffn_up.weight", [hidden, inter], mt(p + "ffn_up.weight", GGML_Q4_K)),
                  (p + "ffn_down.weight", [inter, hidden], mt(p + "ffn_down.weight", GGML_Q6_K))]
    tensors = [(n, d, t, random_tensor(rng, t, d, model_like)) for n, d, t in specs if n not in drop]
    return build(kv, tensors, version=version, alignment=alignment), tensors, kv


def write_file(path: str, kv, specs, fill, version: int = 3, alignment: int = 32, chunk: int = 64 << 20) -> int:
    """Streams a GGUF to `path` without holding the tensor data in memory:
    specs = [(name, dims, ggml_type)], fill(name, nbytes) -> bytes. Returns the file size."""
    sizes = [tensor_bytes(t, d) for _, d, t in specs]
    head = bytearray(b"GGUF") + struct.pack("<I", version)
    head += struct.pack("<II", len(specs), len(kv)) if version == 1 else struct.pack("<QQ", len(specs), len(kv))
    for key, t, v in kv:
        head += gstr(key) + struct.pack("<I", t) + value(t, v)
    offs, cur = [], 0
    for n in sizes:
        cur = (cur + alignment - 1) // alignment * alignment
        offs.append(cur)
        cur += n
    for (name, dims, t), off in zip(specs, offs):
        head += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", t, off)
    head += b"\0" * ((-len(head)) % alignment)
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for (name, dims, t), off, n in zip(specs, offs, sizes):
            f.write(b"\0" * (off - pos))
            left = n
            while left > 0:
                k = min(chunk, left)
                f.write(fill(name, k))
                left -= k
            pos = off + n
        return f.tell()


def qwen3_1_7b_specs(tied: bool = True):
    """Tensor table of Qwen3-1.7B in a Q4_K_M layout (Q6_K embeddings, attn_v and
    ffn_down; Q4_K elsewhere; f32 norms) with its metadata."""
    h, nh, nkv, d, inter, vocab, layers = 2048, 16, 8, 128, 6144, 151936, 28
    kv = [("general.architecture", STR, "qwen3"), ("general.name", STR, "Qwen3-1.7B (synthetic weights)"),
          ("qwen3.block_count", U32, layers), ("qwen3.embedding_length", U32, h),
          ("qwen3.attention.head_count", U32, nh), ("qwen3.attention.head_count_kv", U32, nkv),
          ("qwen3.attention.key_length", U32, d), ("qwen3.attention.value_length", U32, d),
          ("qwen3.feed_forward_length", U32, inter), ("qwen3.context_length", U32, 40960),
          ("qwen3.rope.freq_base", F32, 1000000.0), ("qwen3.attention.layer_norm_rms_epsilon", F32, 1e-6)]
    specs = [("token_embd.weight", [h, vocab], GGML_Q6_K)]
    if not tied:
        specs.append(("output.weight", [h, vocab], GGML_Q6_K))
    specs.append(("output_norm.weight", [h], GGML_F32))
    for layer in range(layers):
        p = f"blk.{layer}."
        specs += [(p + "attn_norm.weight", [h], GGML_F32), (p + "ffn_norm.weight", [h], GGML_F32),
                  (p + "attn_q_norm.weight", [d], GGML_F32), (p + "attn_k_norm.weight", [d], GGML_F32),
                  (p + "attn_q.weight", [h, nh * d], GGML_Q4_K), (p + "attn_k.weight", [h, nkv * d], GGML_Q4_K),
                  (p + "attn_v.weight", [h, nkv * d], GGML_Q6_K), (p + "attn_output.weight", [nh * d, h], GGML_Q4_K),
                  (p + "ffn_gate.weight", [h, inter], GGML_Q4_K), (p + "ffn_up.weight", [h, inter], GGML_Q4_K),
                  (p + "ffn_down.weight", [inter, h], GGML_Q6_K)]
    return kv, specs
