"""The C++ operator layer linked directly, as the engine's own forward code would
link it: tests/native/op_check calls the reference-signature functions (namespace
rpg, reference src/kernels_gpu.h:39-154) and checks them against the C oracle."""
from __future__ import annotations

import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BINARY = os.path.join(HERE, "native", "bin", "op_check")


def test_native_binary_is_built():
    assert os.path.isfile(BINARY) and os.access(BINARY, os.X_OK), "run __graft_entry__.build() first"


@pytest.mark.gpu
def test_native_cpp_operator_layer(gpu):
    print("case: native op_check", flush=True)
    proc = subprocess.run([BINARY], capture_output=True, text=True, timeout=100)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "FAIL" not in proc.stdout
