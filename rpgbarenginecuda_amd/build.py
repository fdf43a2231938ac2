"""Build recipe for librpg_ops.so (hipcc, gfx950, in-tree).

Every HIP source is compiled for gfx950 only, with
  * -ffp-contract=off: the dequant and residual-add paths are bit-exact with
    the CPU reference only if no multiply-add is fused;
  * -Xclang -target-feature -Xclang -packed-fp32-ops: no packed fp32 math;
  * -mcode-object-version=5: loadable by the ROCm runtime bundled with torch.
Symbols are hidden except the extern "C" entry points of include/rpg_ops.h.
The same objects are also archived into librpg_ops_objs.a for C++ callers that
link the operator layer (namespace rpg) directly.

Usage: python -m rpgbarenginecuda_amd.build   (or __graft_entry__.build())
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "librpg_ops.so")
ARCHIVE_PATH = os.path.join(PKG_DIR, "librpg_ops_objs.a")

HIP_SOURCES = ["k_norm.hip", "k_rope_kv.hip", "k_elementwise.hip", "k_dequant.hip", "k_matmul.hip", "k_matmul_mfma.hip", "k_attention.hip", "k_sample.hip"]
HOST_SOURCES = ["common.cc", "hip_common.cc", "quant_types.cc", "kv_cache.cc", "gguf.cc", "gpu_model.cc", "qwen3_gpu.cc", "capi.cc"]

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
    f"-I{CSRC}",
    f"-I{os.path.join(REPO_DIR, 'include')}",
]
DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True) -> str:
    """Compile every source and link librpg_ops.so; returns the library path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    jobs = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        jobs.append([hipcc, *COMMON_FLAGS, *DEVICE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD_DIR, src.replace(".cc", ".o"))
        jobs.append([hipcc, *COMMON_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    workers = min(len(jobs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(_run, jobs))
    objs = [j[-1] for j in jobs]
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, "-shared", "-fPIC", "--offload-arch=gfx950", "-Wl,-soname,librpg_ops.so", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    if os.path.exists(ARCHIVE_PATH):
        os.remove(ARCHIVE_PATH)
    _run(["ar", "rcs", ARCHIVE_PATH, *objs])
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
