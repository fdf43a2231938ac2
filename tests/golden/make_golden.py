"""Writes tests/golden/dequant_ref.npz from the reference's own CPU dequant.

Run in the build container, where /root/reference exists:
    make -C oracle ref && python tests/golden/make_golden.py

The reference's src/quant.cc + src/common.cc are compiled where they lie into
oracle/_ref/libref_quant.so (oracle/Makefile); this script feeds them seeded
synthetic Q4_K / Q6_K blocks (plus hand-made edge-case blocks) and stores inputs
and outputs. The fixture is data only: raw block bytes in, fp32 bit patterns out.
It lets tests on the GPU box, where the reference does not exist, check the
oracle and the device path against the reference's own answers.

Also stored: the reference F16ToF32 over all 65536 halves (as a SHA-256 of the
fp32 bytes), and its F32ToF16 (src/dtypes.h:50-76) on a few exact ties, which
shows that helper rounds ties away from zero and is not the KV write's rounding.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)
sys.path.insert(0, os.path.dirname(HERE))

from oracle import pyoracle  # noqa: E402
import synth  # noqa: E402

SEED = 0x5EED2026


def main() -> None:
    ref = pyoracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_quant.so missing: run `make -C oracle ref` where /root/reference exists")
    rng = np.random.default_rng(SEED)
    q4 = np.concatenate([synth.q4k_blocks(rng, 48), synth.special_q4k_blocks()])
    q6 = np.concatenate([synth.q6k_blocks(rng, 48, bench_scales=True), synth.special_q6k_blocks()])
    q4_out = pyoracle.ref_dequantize_row(12, q4.reshape(-1), q4.shape[0] * 256)
    q6_out = pyoracle.ref_dequantize_row(14, q6.reshape(-1), q6.shape[0] * 256)

    f16_all = pyoracle.ref_f16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    f16_sha = hashlib.sha256(f16_all.tobytes()).hexdigest()

    # Exact fp32 ties between two halves: 1 + k*2^-11 for odd k (mantissa bit 12 set, lower bits clear).
    ties = np.array([1.0 + k * 2.0 ** -11 for k in (1, 3, 5, 7)] + [-(1.0 + 2.0 ** -11), 2049.0, 65520.0],
                    dtype=np.float32)
    ties_dtypes = np.array([ref.ref_f32_to_f16_dtypes(float(t)) for t in ties], dtype=np.uint16)

    out = os.path.join(HERE, "dequant_ref.npz")
    np.savez_compressed(
        out,
        seed=np.uint64(SEED),
        q4k_blocks=q4,
        q4k_out_bits=q4_out.view(np.uint32),
        q6k_blocks=q6,
        q6k_out_bits=q6_out.view(np.uint32),
        f16_to_f32_sha256=np.array(f16_sha),
        ties=ties,
        ties_dtypes_f32_to_f16=ties_dtypes,
    )
    print(f"wrote {out}: {q4.shape[0]} Q4_K + {q6.shape[0]} Q6_K blocks")


if __name__ == "__main__":
    main()
