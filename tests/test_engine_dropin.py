"""The reference engine's C ABI (include/rpg_engine.h:52-117) running on this
library: src/engine.cc and its host layer compiled unchanged, the GPU layer
replaced by rpgbarenginecuda_amd/engine_compat over librpg_ops.so
(`make -C oracle engine` -> oracle/_ref/librpg_engine.so).

CPU side (no device): the library exports exactly the 10 functions, and the
checks of the reference's own ABI smoke test (tests/abi_smoke.py) hold --
version, readable last_error on a bad handle, error returns for a null path, a
missing file and malformed JSON, no-op unload / destroy / free of bad handles --
plus the engine's metadata-only mode (src/engine.cc:280-288): load_model reads
the GGUF, model_info reports its shapes, and a session is refused.
"""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

import engine_abi as E
import gguf_writer as gw

pytestmark = pytest.mark.skipif(not os.path.exists(E.ENGINE_LIB),
                                reason="oracle/_ref/librpg_engine.so not built (needs the reference sources: "
                                       "make -C oracle engine)")


@pytest.fixture(scope="module")
def lib():
    return E.bind()


def device_available() -> bool:
    from rpgbarenginecuda_amd import ops

    return ops.device_info()[0]


def test_exports_exactly_the_reference_abi():
    out = subprocess.run(["nm", "-D", "--defined-only", E.ENGINE_LIB], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert exported == set(E.ABI)


def test_reference_abi_smoke_error_paths(lib):
    assert lib.rpg_engine_version().decode() == "0.1.0"
    assert lib.rpg_engine_session_create(-999, None) < 0
    assert "-999" in E.last_error(lib)
    assert lib.rpg_engine_load_model(None, None) < 0
    assert E.last_error(lib)
    assert lib.rpg_engine_load_model(b"/nonexistent/nope.gguf", None) < 0
    assert E.last_error(lib)
    assert lib.rpg_engine_load_model(b"/nonexistent/nope.gguf", b"{not json}") < 0
    lib.rpg_engine_unload_model(-999)
    lib.rpg_engine_session_destroy(-999)
    lib.rpg_engine_free(None)
    assert lib.rpg_engine_session_reset(-999) < 0
    assert E.take_json(lib, lib.rpg_engine_model_info(-999)) is None
    assert lib.rpg_engine_generate(-999, b"{}") is None


def test_load_model_metadata_and_model_info(lib, tmp_path):
    raw, tensors, kv = gw.qwen3_model(np.random.default_rng(5), n_layers=3, hidden=256, n_heads=4, n_kv_heads=2,
                                      inter=512, vocab=1000, tokenizer=True)
    path = tmp_path / "model.gguf"
    path.write_bytes(raw)
    h = lib.rpg_engine_load_model(str(path).encode(), b'{"context": 2048}')
    assert h >= 0, E.last_error(lib)
    try:
        info = E.take_json(lib, lib.rpg_engine_model_info(h))
        want = {"arch": "qwen3", "name": "synthetic-qwen3", "n_layers": 3, "hidden": 256, "n_heads": 4,
                "n_kv_heads": 2, "head_dim": 128, "intermediate": 512, "vocab": 1000, "context_length": 40960,
                "tied_embeddings": False, "max_pos": 2048, "default_max_seq": 2048, "sessions": 0,
                "path": str(path), "weight_bytes": sum(len(t[3]) for t in tensors)}
        for key, value in want.items():
            assert info[key] == value, (key, info[key], value)
        assert info["rope_theta"] == pytest.approx(1e6)
        if device_available():
            pytest.skip("a GPU is present: the metadata-only mode does not apply (see the GPU test)")
        assert info["device_available"] is False and "device_bytes" not in info
        # metadata-only load: sessions are refused, with a reason
        assert lib.rpg_engine_session_create(h, None) < 0
        assert E.last_error(lib)
    finally:
        lib.rpg_engine_unload_model(h)
    assert E.take_json(lib, lib.rpg_engine_model_info(h)) is None
