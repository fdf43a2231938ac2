"""Binding and helpers for the reference engine's 10-function C ABI
(include/rpg_engine.h:52-117) built over this library (oracle/_ref/librpg_engine.so,
`make -C oracle engine`).

The ctypes signatures are the ones the reference's own host binding declares
(tests/abi_smoke.py:41-76): generate / model_info return char* received as
c_void_p so the engine's buffer can be handed back to rpg_engine_free.

The prompt helpers restate, for the ascii_bpe_vocab test vocabulary only, what
the engine does before its forward: ChatML for one user turn with a generation
prompt (src/chat_template.cc:85-204), special tokens matched first and every
other byte as its own token (src/tokenizer.cc:237-342 with no applicable
merge), and what it does after: byte-level decoding, then the control-marker
strip and ASCII trim of the output parser (src/tool_parser.cc:97-176).
"""
from __future__ import annotations

import ctypes
import json
import os

import gguf_writer as gw

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENGINE_LIB = os.path.join(REPO, "oracle", "_ref", "librpg_engine.so")

ABI = ("rpg_engine_version", "rpg_engine_last_error", "rpg_engine_load_model", "rpg_engine_unload_model",
       "rpg_engine_session_create", "rpg_engine_session_destroy", "rpg_engine_session_reset",
       "rpg_engine_generate", "rpg_engine_free", "rpg_engine_model_info")


def bind(path: str = ENGINE_LIB):
    import torch  # noqa: F401  (the process's HIP runtime first, as for librpg_ops)

    lib = ctypes.CDLL(path)
    c = ctypes
    lib.rpg_engine_version.restype = c.c_char_p
    lib.rpg_engine_last_error.restype = c.c_char_p
    lib.rpg_engine_load_model.argtypes = [c.c_char_p, c.c_char_p]
    lib.rpg_engine_load_model.restype = c.c_int32
    lib.rpg_engine_unload_model.argtypes = [c.c_int32]
    lib.rpg_engine_unload_model.restype = None
    lib.rpg_engine_session_create.argtypes = [c.c_int32, c.c_char_p]
    lib.rpg_engine_session_create.restype = c.c_int32
    lib.rpg_engine_session_destroy.argtypes = [c.c_int32]
    lib.rpg_engine_session_destroy.restype = None
    lib.rpg_engine_session_reset.argtypes = [c.c_int32]
    lib.rpg_engine_session_reset.restype = c.c_int32
    lib.rpg_engine_generate.argtypes = [c.c_int32, c.c_char_p]
    lib.rpg_engine_generate.restype = c.c_void_p
    lib.rpg_engine_model_info.argtypes = [c.c_int32]
    lib.rpg_engine_model_info.restype = c.c_void_p
    lib.rpg_engine_free.argtypes = [c.c_void_p]
    lib.rpg_engine_free.restype = None
    return lib


def take_json(lib, ptr):
    """Reads an engine-allocated JSON string, frees it, returns the parsed object
    (None for a NULL pointer)."""
    if not ptr:
        return None
    text = ctypes.cast(ptr, ctypes.c_char_p).value.decode("utf-8")
    lib.rpg_engine_free(ptr)
    return json.loads(text)


def last_error(lib) -> str:
    return (lib.rpg_engine_last_error() or b"").decode("utf-8", "replace")


def chatml_one_turn(user_text: str) -> str:
    return f"<|im_start|>user\n{user_text}<|im_end|>\n<|im_start|>assistant\n"


def encode(text: str, n_vocab: int) -> list:
    tokens, _, _ = gw.ascii_bpe_vocab(n_vocab)
    ids = {t: i for i, t in enumerate(tokens)}
    b2u = gw.byte_to_unicode()
    out, i = [], 0
    specials = sorted(gw.CHATML_SPECIALS, key=len, reverse=True)
    while i < len(text):
        hit = next((s for s in specials if text.startswith(s, i)), None)
        if hit is not None:
            out.append(ids[hit])
            i += len(hit)
            continue
        out.extend(ids[b2u[b]] for b in text[i].encode())
        i += 1
    return out


def decode(ids, n_vocab: int) -> str:
    tokens, _, _ = gw.ascii_bpe_vocab(n_vocab)
    u2b = {u: b for b, u in gw.byte_to_unicode().items()}
    out = bytearray()
    for i in ids:
        t = tokens[i]
        if t in gw.CHATML_SPECIALS:
            out += t.encode()
        else:
            out += bytes(u2b[ch] for ch in t)
    return out.decode("ascii")


def parsed_text(raw: str) -> str:
    """Control markers removed (<|im_start|> with a following role line,
    <|im_end|>, <|endoftext|>), then ASCII whitespace trimmed."""
    start = "<|im_start|>"
    while start in raw:
        p = raw.index(start)
        end = p + len(start)
        for role in ("system", "user", "assistant", "tool"):
            if raw.startswith(role + "\n", end):
                end += len(role) + 1
                break
        raw = raw[:p] + raw[end:]
    for marker in ("<|im_end|>", "<|endoftext|>"):
        raw = raw.replace(marker, "")
    return raw.strip(" \t\n\r\f\v")
