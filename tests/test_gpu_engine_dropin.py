"""The reference engine (src/engine.cc, compiled unchanged over this library:
oracle/_ref/librpg_engine.so) generating on the GPU through its C ABI.

A synthetic qwen3 GGUF carries the ascii_bpe_vocab tokenizer, so the prompt ids
the engine derives (ChatML, then byte-level BPE) are known exactly, and every
generated token decodes to ASCII. The engine's answer is checked against the
same prompt run straight through librpg_ops (GpuForwardFull + GpuGenerate with
the engine's sampling defaults: top_k off, top_p 0.95, stop at <|im_end|>):
the response text must be the decoded, marker-stripped, trimmed ids, and the
usage counts the prompt and generated lengths. Greedy and sampled (seeded)
generation, a repeated request served from the session's cached prefix, and a
session reset (after which the answer repeats bit for bit) are covered.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import engine_abi as E
import gguf_writer as gw

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not os.path.exists(E.ENGINE_LIB),
                                 reason="oracle/_ref/librpg_engine.so not built (make -C oracle engine)")]

VOCAB = 1000


def _case(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def _generate(lib, session: int, req: dict) -> dict:
    out = E.take_json(lib, lib.rpg_engine_generate(session, json.dumps(req).encode()))
    assert out is not None, E.last_error(lib)
    return out


def _library_answer(gpu, path, prompt_ids, max_tokens, temperature, seed):
    """(generated ids, stop ids) for the prompt through librpg_ops directly."""
    m = gpu.GpuModel(str(path), 256)
    kv = gpu.GpuKvCache(m, 256)
    s = gpu.GpuScratch()
    try:
        gpu.GpuForwardFull(m, np.asarray(prompt_ids, np.int32), s, want_logits=False, kv=kv)
        tokens, _, _ = gw.ascii_bpe_vocab(VOCAB)
        stops = [tokens.index("<|im_end|>")]
        first = s.logits_dev() + 4 * VOCAB * (len(prompt_ids) - 1)
        opt = gpu.GpuGenerateOptions(max_tokens=max_tokens, stop_ids=stops,
                                     sample=gpu.SampleOptions(temperature, 0, 0.95), seed=seed)
        ids, _ = gpu.GpuGenerate(m, kv, s, first, opt)
        return ids, stops
    finally:
        s.free()
        kv.free()
        m.free()


def _expect(response, prompt_ids, ids, stops, max_tokens):
    assert response["usage"] == {"prompt_tokens": len(prompt_ids), "completion_tokens": len(ids)}
    assert response["text"] == E.parsed_text(E.decode(ids, VOCAB))
    assert response["tool_calls"] == []
    stopped = len(ids) > 0 and ids[-1] in stops
    assert response["finish_reason"] == ("stop" if stopped or len(ids) < max_tokens else "length")


def test_engine_generate_equals_library_path(gpu, tmp_path):
    lib = E.bind()
    raw, _, _ = gw.qwen3_model(np.random.default_rng(11), n_layers=2, hidden=256, n_heads=4, n_kv_heads=2,
                               inter=512, vocab=VOCAB, tokenizer=True, model_like=True)
    path = tmp_path / "engine.gguf"
    path.write_bytes(raw)

    _case("engine load_model / model_info on the GPU")
    h = lib.rpg_engine_load_model(str(path).encode(), b'{"context": 256}')
    assert h >= 0, E.last_error(lib)
    try:
        info = E.take_json(lib, lib.rpg_engine_model_info(h))
        assert info["device_available"] is True and info["device_bytes"] > 0
        assert info["vocab"] == VOCAB and info["max_pos"] == 256
        s = lib.rpg_engine_session_create(h, b'{"max_seq": 256, "max_tokens": 16}')
        assert s >= 0, E.last_error(lib)
        try:
            user = "Hello from MI355X, tell me a story."
            prompt_ids = E.encode(E.chatml_one_turn(user), VOCAB)
            for temperature, seed in ((0.0, 0), (0.7, 1234)):
                _case(f"engine generate vs library, temperature {temperature}, seed {seed}")
                req = {"messages": [{"role": "user", "content": user}], "max_tokens": 12,
                       "temperature": temperature, "seed": seed}
                ids, stops = _library_answer(gpu, path, prompt_ids, 12, temperature, seed)
                assert lib.rpg_engine_session_reset(s) == 0  # a fresh cache: the engine runs the whole prefill
                first = _generate(lib, s, req)
                print(f"  engine: {json.dumps(first)}\n  library ids: {ids}", flush=True)
                _expect(first, prompt_ids, ids, stops, 12)
                # The same request again: the session's cache already holds the prompt
                # (and the previous answer), so the engine keeps the cached prefix and
                # re-runs only the last prompt position, a one-token forward whose
                # logits come from the decode kernels rather than the prefill ones
                # (equal to rounding, not bit for bit): the answer is well formed and
                # counts the same prompt.
                again = _generate(lib, s, req)
                assert again["usage"]["prompt_tokens"] == len(prompt_ids)
                assert 1 <= again["usage"]["completion_tokens"] <= 12
                assert again["finish_reason"] in ("stop", "length")
                # After a reset the session runs the full prefill again: bit for bit
                # the first answer.
                assert lib.rpg_engine_session_reset(s) == 0
                assert _generate(lib, s, req) == first
        finally:
            lib.rpg_engine_session_destroy(s)
    finally:
        lib.rpg_engine_unload_model(h)
    assert E.take_json(lib, lib.rpg_engine_model_info(h)) is None
