"""Path equivalence of the quantised matmul (GpuSetForceGenericMatMul,
src/kernels_gpu.h:51-58; the reference's bitwise generic-vs-specialised check,
tools/matmul_bench.cu:149-219): every specialised kernel -- the one-token decode
matvecs (2 and 4 rows per wave, and the split-columns form), the tiled
small-batch kernel and the matrix-core prefill GEMM with and without split K,
decoding per tile or from decoded weight planes --
against the generic per-element kernel on the same weights and inputs.

The kernels sum in different orders (that is where their speed comes from), so
bit equality is asked on inputs where every order gives the exact sum: fp16
scales that are powers of two (Q4_K d = dmin = 2^-4, Q6_K d = 2^-6, Q6_K scales
over the whole int8 range, one -128 per block) and activations in {-1, 0, 1}.
Every product is then a multiple of the scale below 2^12 of it, and every partial
sum an exact multiple of it below 2^24 of it (checked per row: sum |w| stays
below that) -- including the matrix cores' fp16-split operands, which are exact
integers here -- so any misplaced block, scale, nibble or column shows as a bit
difference, and both must equal the oracle's exact float64 result. On general
inputs (random scales and activations) the generic kernel is held to the same
fp32 summation bound as the specialised ones.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14


def _case(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def exact_table(rng, qtype, rows, cols):
    """Raw blocks whose dequantised weights are small multiples of a power of two."""
    bb = 144 if qtype == Q4_K else 210
    blocks = rows * cols // 256
    raw = rng.integers(0, 256, size=(blocks, bb), dtype=np.uint8)
    if qtype == Q4_K:
        raw[:, 0:2] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)  # d
        raw[:, 2:4] = np.frombuffer(np.float16(2.0 ** -4).tobytes(), np.uint8)  # dmin
    else:
        sc = rng.integers(-128, 128, size=(blocks, 16)).astype(np.int8)  # scales, the whole int8 range
        sc[np.arange(blocks), rng.integers(0, 16, size=blocks)] = -128
        raw[:, 192:208] = sc.view(np.uint8)
        raw[:, 208:210] = np.frombuffer(np.float16(2.0 ** -6).tobytes(), np.uint8)  # d
    return raw.reshape(-1)


CASES = [
    # (name, type, rows, cols, n_tokens, specialised kernel the call must take: a name prefix, the
    # matrix-core kernels having a ping-pong form for small grids)
    ("decode Q4_K, 2 rows per wave", Q4_K, 2048, 2048, 1, "MatVecQ4KKernel"),
    ("decode Q4_K, 4 rows per wave", Q4_K, 32768, 2048, 1, "MatVecQ4KKernel"),
    ("decode Q6_K", Q6_K, 1024, 2048, 1, "MatVecQ6KKernel"),
    ("decode Q6_K, split columns", Q6_K, 2048, 6144, 1, "MatVecSplitQ6KKernel"),
    ("decode Q6_K, tall matrix", Q6_K, 16400, 2048, 1, "MatVecQ6KKernel"),
    ("decode Q6_K, tall, 10 blocks per row", Q6_K, 16384, 2560, 1, "MatVecSplitQ6KKernel"),
    ("decode Q4_K, split columns", Q4_K, 1024, 4096, 1, "MatVecSplitQ4KKernel"),
    ("small batch Q4_K", Q4_K, 2048, 2048, 8, "MatMulQ4KKernel"),
    ("small batch Q6_K", Q6_K, 1024, 2048, 5, "MatMulQ6KKernel"),
    ("matrix cores Q4_K", Q4_K, 6144, 2048, 300, "MatMulMfmaQ4K"),
    ("matrix cores Q6_K", Q6_K, 2048, 6144, 300, "MatMulMfmaQ6K"),
    ("matrix cores Q4_K, split K", Q4_K, 1024, 2048, 48, "MatMulSplitReduceKernel"),
    ("decoded weight planes Q4_K", Q4_K, 6144, 2048, 700, "MatMulMfmaQ4KPlanes"),
    ("decoded weight planes Q6_K", Q6_K, 2048, 2048, 600, "MatMulMfmaQ6KPlanes"),
    ("decoded weight planes Q4_K, split K, ragged", Q4_K, 1152, 2048, 513, "MatMulMfmaQ4KPlanes"),
    ("decoded weight planes Q4_K, whole rounds + split tail", Q4_K, 4352, 512, 2048, "MatMulPlanesReduceKernel"),
    ("decoded weight planes Q6_K, whole rounds + split tail", Q6_K, 2176, 512, 2000, "MatMulPlanesReduceKernel"),
    ("decoded weight planes Q6_K above 64 MB: two row slices, the last ragged", Q6_K, 8300, 2048, 512,
     "MatMulMfmaQ6KPlanes"),
    ("decoded weight planes Q4_K, 10 blocks per row (4B shape)", Q4_K, 1024, 2560, 520, "MatMulMfmaQ4KPlanes"),
]


def _dequant(ora, qtype, raw, rows, cols):
    return ora.dequantize_row(qtype, raw, rows * cols).reshape(rows, cols).astype(np.float64)


def _run(gpu, qtype, w, rows, cols, x, n_tokens, force_generic):
    import torch

    out = torch.full((n_tokens, rows), float("nan"), dtype=torch.float32, device="cuda")
    gpu.GpuSetForceGenericMatMul(force_generic)
    try:
        gpu.profile_start(64)
        gpu.GpuMatMulQuant(gpu.GpuTensor(w, qtype, rows, cols), x, n_tokens, out)
        gpu.profile_stop()
        kernels = set(gpu.profile_report())
    finally:
        gpu.GpuSetForceGenericMatMul(False)
    torch.cuda.synchronize()
    return out.cpu().numpy(), kernels


@pytest.mark.parametrize("name,qtype,rows,cols,n_tokens,kernel", CASES, ids=[c[0] for c in CASES])
def test_specialised_equals_generic_bit_for_bit(gpu, ora, name, qtype, rows, cols, n_tokens, kernel):
    import torch

    _case(f"generic vs specialised: {name} [{rows} x {cols}] x {n_tokens} tokens")
    rng = np.random.default_rng(rows * 7 + cols + n_tokens)
    raw = exact_table(rng, qtype, rows, cols)
    unit = 2.0 ** -6 if qtype == Q6_K else 2.0 ** -4  # every weight is an integer multiple of d
    wabs = np.abs(_dequant(ora, qtype, raw, rows, cols)).sum(axis=1, dtype=np.float64)
    assert np.all(wabs / unit < 2.0 ** 24), "premise: every partial sum exact in fp32"
    x = rng.integers(-1, 2, size=(n_tokens, cols)).astype(np.float32)
    w = torch.from_numpy(raw).cuda()
    xd = torch.from_numpy(x).cuda()
    spec, k_spec = _run(gpu, qtype, w, rows, cols, xd, n_tokens, False)
    gen, k_gen = _run(gpu, qtype, w, rows, cols, xd, n_tokens, True)
    assert any(k.startswith(kernel) for k in k_spec), k_spec
    assert k_gen == {"MatMulGenericKernel"}, k_gen
    assert not gpu.GpuForceGenericMatMul()
    assert np.array_equal(spec.view(np.uint32), gen.view(np.uint32)), \
        f"{int(np.sum(spec.view(np.uint32) != gen.view(np.uint32)))} outputs differ"
    exact = ora.matmul_quant_f64(qtype, raw, rows, cols, x)[0]
    assert np.array_equal(gen.astype(np.float64), exact)


def test_generic_kernel_within_the_summation_bound(gpu, ora):
    """General inputs: the generic path obeys the fp32 summation bound of the
    specialised kernels (|out - exact| <= (cols / 8 + 7) 2^-24 sum|w x|)."""
    import torch

    import synth

    rng = np.random.default_rng(9)
    for qtype, rows, cols, n_tokens in ((Q4_K, 512, 2048, 3), (Q6_K, 256, 6144, 1)):
        _case(f"generic kernel, random inputs: type {qtype} [{rows} x {cols}] x {n_tokens}")
        raw = (synth.q4k_blocks(rng, rows * cols // 256) if qtype == Q4_K
               else synth.q6k_blocks(rng, rows * cols // 256)).reshape(-1)
        x = rng.normal(0, 1, (n_tokens, cols)).astype(np.float32)
        got, kernels = _run(gpu, qtype, torch.from_numpy(raw).cuda(), rows, cols, torch.from_numpy(x).cuda(),
                            n_tokens, True)
        assert kernels == {"MatMulGenericKernel"}
        exact, absdot = ora.matmul_quant_f64(qtype, raw, rows, cols, x)
        bound = (cols // 8 + 7) * 2.0 ** -24 * absdot + 1e-37
        assert np.all(np.abs(got.astype(np.float64) - exact) <= bound)
