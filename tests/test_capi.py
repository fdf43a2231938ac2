"""The C-ABI library: it loads, exports exactly what include/rpg_ops.h declares,
and its host-side logic (argument checks, row sizes, RoPE table) behaves as the
reference's operator layer does. No GPU work is launched here: every call that
reaches a kernel is either a documented no-op or rejected before the launch."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "rpg_ops.h")


def header_symbols() -> set[str]:
    text = open(HEADER).read()
    return set(re.findall(r"RPG_OPS_API\s+[\w\s\*]+?\b(rpg_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def ops():
    from rpgbarenginecuda_amd import ops as o

    o.load_library()
    return o


def test_library_exports_exactly_the_header(ops):
    declared = header_symbols()
    assert len(declared) == 74
    out = subprocess.run(["nm", "-D", "--defined-only", ops.LIB_PATH], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert exported == declared
    assert set(ops.SIGNATURES) == declared
    lib = ops.load_library()
    for name in declared:
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_version_and_device_info(ops):
    assert ops.version() == "0.1.0"
    avail, desc = ops.device_info()
    assert isinstance(avail, bool) and desc


def test_type_row_bytes(ops):
    assert ops.type_row_bytes(12, 2048) == 1152
    assert ops.type_row_bytes(14, 2048) == 1680
    assert ops.type_row_bytes(0, 2048) == 8192
    assert ops.type_row_bytes(12, 2560) == 1440
    with pytest.raises(ops.RpgError, match="not supported"):
        ops.type_row_bytes(13, 256)            # Q5_K never reaches the device
    with pytest.raises(ops.RpgError, match="multiple"):
        ops.type_row_bytes(12, 100)


def test_rope_table_matches_oracle(ops, ora):
    # 40960 rows: a table whose inverse frequencies differ from the reference's in the
    # last double bit agrees on the first few thousand positions and then drifts
    for theta in (1e6, 5e5, 1e4):
        got = ops.build_rope_table(128, theta, 40960)
        want = ora.build_rope_table(128, theta, 40960)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), theta
    got4 = ops.build_rope_table(64, 1e4, 17)
    assert np.array_equal(got4, ora.build_rope_table(64, 1e4, 17))


def _lib(ops):
    return ops.load_library()


FAKE = ctypes.c_void_p(0x1000)  # never dereferenced: every call below fails its host check first


def test_kv_write_range_checks(ops):
    lib = _lib(ops)
    rc = lib.rpg_op_kv_write(FAKE, FAKE, 8, 128, 4090, 10, FAKE, FAKE, 4096)
    assert rc < 0 and "run past the 4096 cache slots" in lib.rpg_ops_last_error().decode()
    rc = lib.rpg_op_kv_write(FAKE, FAKE, 8, 128, -1, 1, FAKE, FAKE, 4096)
    assert rc < 0 and "start position -1 is negative" in lib.rpg_ops_last_error().decode()
    rc = lib.rpg_op_kv_write(FAKE, FAKE, 8, 128, 0, 0, FAKE, FAKE, 4096)
    assert rc < 0 and "have to be positive" in lib.rpg_ops_last_error().decode()


def test_rms_norm_and_rope_argument_checks(ops):
    lib = _lib(ops)
    assert lib.rpg_op_rms_norm(FAKE, FAKE, 4, 0, 0, 1e-6, FAKE) < 0
    assert lib.rpg_op_rms_norm(FAKE, FAKE, 4, 128, 64, 1e-6, FAKE) < 0      # stride < n
    assert "stride at least n" in lib.rpg_ops_last_error().decode()
    assert lib.rpg_op_rope(FAKE, 16, 127, FAKE, 0, 3) < 0                   # odd head_dim
    assert "head_dim has to be even" in lib.rpg_ops_last_error().decode()
    assert lib.rpg_op_add_rms_norm(FAKE, FAKE, FAKE, 2, 2048, 1e-6, FAKE) < 0  # out aliases x
    assert "alias" in lib.rpg_ops_last_error().decode()


def test_qk_fused_argument_checks(ops):
    lib = _lib(ops)
    rc = lib.rpg_op_qk_norm_rope_kv(FAKE, FAKE, FAKE, FAKE, FAKE, 16, 8, 128, FAKE, 100, 95, 10, 1e-6, FAKE,
                                    FAKE, 4096, 0)
    assert rc < 0 and "RoPE table" in lib.rpg_ops_last_error().decode()
    rc = lib.rpg_op_qk_norm_rope_kv(FAKE, FAKE, FAKE, FAKE, FAKE, 16, 8, 128, FAKE, 8192, 4095, 2, 1e-6, FAKE,
                                    FAKE, 4096, 0)
    assert rc < 0 and "cache slots" in lib.rpg_ops_last_error().decode()


def test_dequant_and_gather_type_checks(ops):
    lib = _lib(ops)
    assert lib.rpg_op_dequant_row(2, FAKE, 256, FAKE) < 0                   # Q4_0
    assert "not supported" in lib.rpg_ops_last_error().decode()
    assert lib.rpg_op_dequant_row(12, FAKE, 300, FAKE) < 0
    assert "whole blocks" in lib.rpg_ops_last_error().decode()
    assert lib.rpg_op_embedding_lookup(14, FAKE, 10, 1000, FAKE, 3, FAKE) < 0
    assert lib.rpg_op_embedding_lookup(12, FAKE, 0, 2048, FAKE, 3, FAKE) < 0


def test_empty_inputs_are_no_ops(ops):
    lib = _lib(ops)
    # n <= 0 returns before any launch (src/kernels_gpu.cu:1114, :1120).
    assert lib.rpg_op_silu_mul_inplace(FAKE, FAKE, 0) == 0
    assert lib.rpg_op_vec_add_inplace(FAKE, FAKE, -5) == 0
    assert lib.rpg_op_embedding_lookup(12, FAKE, 10, 2048, FAKE, 0, FAKE) == 0
    assert lib.rpg_op_rope(FAKE, 16, 128, FAKE, 0, 0) == 0


def test_error_text_is_thread_local(ops):
    import threading

    lib = _lib(ops)
    assert lib.rpg_op_dequant_row(2, FAKE, 256, FAKE) < 0
    seen = {}

    def worker():
        seen["msg"] = lib.rpg_ops_last_error().decode()

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "not supported" in lib.rpg_ops_last_error().decode()


def test_python_mirror_rejects_undersized_tensors(ops):
    """The host mirror refuses a tensor smaller than what the operator would touch."""
    import torch

    x = torch.zeros(10)
    with pytest.raises(ops.RpgError, match="not on the GPU"):
        ops.GpuVecAddInPlace(x, x, 10)


def test_host_random_source_matches_oracle(ops, ora):
    """DevSplitMix64 / DevCounterRng / DevCounterUniform are host code: bit-exact
    with the oracle (itself pinned to SplitMix64's published outputs)."""
    for x in (0, 1, 0x9E3779B97F4A7C15, 2 ** 63 + 12345, 2 ** 64 - 1):
        assert ops.DevSplitMix64(x) == ora.split_mix64(x)
    for seed in (0, 11, 2 ** 40 + 7):
        for c in (0, 1, 2, 4095, 2 ** 33):
            assert ops.DevCounterRng(seed, c) == ora.counter_rng(seed, c)
            assert ops.DevCounterUniform(seed, c) == ora.counter_uniform(seed, c)


def test_sampler_host_argument_errors(ops):
    lib = ops.load_library()
    assert lib.rpg_op_argmax(None, 10, FAKE) < 0
    assert "null" in ops.load_library().rpg_ops_last_error().decode()
    assert lib.rpg_op_argmax(FAKE, 0, FAKE) < 0                               # empty vocabulary
    assert lib.rpg_op_argmax(FAKE, (1 << 22) + 1, FAKE) < 0                   # beyond the sampler limit
    assert "limit" in ops.load_library().rpg_ops_last_error().decode()
    assert lib.rpg_op_inverse_sample(FAKE, 10, 1.0, FAKE) < 0                 # u outside [0, 1)
    assert "[0, 1)" in ops.load_library().rpg_ops_last_error().decode()
    assert lib.rpg_op_inverse_sample(FAKE, 10, -0.5, FAKE) < 0
    assert lib.rpg_op_filter_to_probs(FAKE, 10, 1.0, 0, 1.0, None) < 0
    assert lib.rpg_op_sample_token_dev(FAKE, 10, 0.7, 0, 0.9, 1, None, FAKE, FAKE) < 0  # no device counter
    assert "counter" in ops.load_library().rpg_ops_last_error().decode()
