"""Quantised matmul (GpuMatMulQuant, src/kernels_gpu.h:42-49) on the GPU against the
float64 oracle.

Bar: the GPU sums fp32 products of bit-exact dequantised weights, so its error
against the exact dot product is bounded by fp32 summation error:
    |gpu - exact| <= D * 2^-24 * sum_e |w_e * x_e|
with D the longest chain of roundings from one product to the result. Any
kernel that keeps at least 8 independent partial sums of cols / 8 terms each and
combines them by a tree of depth <= 7 has D <= cols / 8 + 7; the kernels here
(at most 32 * ceil(cols / 2048) sequential fused multiply-adds per lane and a
64-lane butterfly) stay well inside it. For Q4_K the decode kernels evaluate
d1 * sum(q x) - m1 * sum(x) per run, whose two terms can partly cancel, so the
bound there also counts sum_e (|d1 q_e| + |m1|) |x_e|. A dropped, doubled or
misplaced term breaks the bound by many orders of magnitude.
"""
from __future__ import annotations

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def case(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def last_error(gpu) -> str:
    msg = gpu.load_library().rpg_ops_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def factored_magnitude(ora, t, w, rows, cols, x):
    """Q4_K only: sum_e (|d1 q_e| + |m1|) |x_e|, the scale of the error of the
    factored form d1 * sum(q x) - m1 * sum(x) that the decode kernels use. A copy
    of the matrix with every quant zeroed dequantises to -m1 exactly, and
    w - (-m1) = d1 q."""
    if t != 12:
        return 0.0
    z = np.array(w, copy=True).reshape(-1, 144)
    z[:, 16:] = 0
    n = rows * cols
    wd = ora.dequantize_row(t, np.ascontiguousarray(w), n).reshape(rows, cols).astype(np.float64)
    w0 = ora.dequantize_row(t, z.reshape(-1), n).reshape(rows, cols).astype(np.float64)
    mag = np.abs(wd - w0) + np.abs(w0)
    return np.abs(np.asarray(x, np.float64).reshape(-1, cols)) @ mag.T


def check(got, exact, absdot, cols, extra=0.0):
    bound = (cols // 8 + 7) * U * (absdot + extra) + 1e-37
    err = np.abs(got.astype(np.float64) - exact)
    worst = float(np.max(err / np.maximum(bound, 1e-300)))
    assert np.all(err <= bound), f"max error / bound = {worst:.3g}"
    return worst


SHAPES = [
    # (type, rows, cols, n_tokens): Qwen3-1.7B / 4B decode matrices, small batches, ragged tiles
    (12, 2048, 2048, 1),     # attn_q / attn_o
    (12, 1024, 2048, 1),     # attn_k
    (14, 1024, 2048, 1),     # attn_v (Q6_K in Q4_K_M files)
    (12, 6144, 2048, 1),     # ffn_gate / ffn_up
    (14, 2048, 6144, 1),     # ffn_down (Q6_K)
    (12, 2048, 6144, 1),     # ffn_down (Q4_K)
    (12, 9728, 2560, 1),     # 4B ffn_gate: 10 blocks per row (not a multiple of 8), 2 rows per wave
    (14, 2560, 9728, 1),     # 4B ffn_down: 38 blocks per row (activations staged in LDS)
    (12, 2048, 6144, 1),     # 24 blocks per row, Q4_K run sums from LDS
    (12, 300, 16384, 1),     # 64 blocks per row: the widest LDS-staged decode
    (14, 100, 20480, 1),     # 80 blocks per row: the tiled kernel
    (12, 40000, 2048, 1),    # 4 rows per wave
    (14, 40001, 2048, 1),    # tall Q6_K (output-projection width), odd row count
    (14, 16384, 2048, 1),
    (14, 16393, 2560, 1),    # ... 10 blocks per row (4B width)
    (12, 2048, 2048, 2),
    (14, 2048, 2048, 3),
    (12, 1000, 2048, 4),
    (14, 1000, 2560, 5),
    (12, 777, 2048, 8),
    (14, 513, 2048, 13),     # two tiles of 8, the second ragged
    (12, 256, 256, 21),      # the CPU-runnable n = 21
    (12, 2048, 2048, 64),    # matrix-core GEMM: one token tile, 16 row tiles
    (14, 1024, 2048, 130),   # ragged token tiles
    (12, 300, 2560, 200),    # ragged row tile, 10 blocks per row
    (14, 777, 6144, 129),    # 24 blocks per row, ragged both ways
    (14, 128, 256, 32),      # the smallest matrix-core case
    (12, 64, 512, 31),       # just below it: the tiled kernel
    (12, 6144, 2048, 17),    # wide matrix: matrix cores from 16 tokens, K split 8 ways
    (14, 4096, 2560, 16),    # ... Q6_K, 10 blocks per row split one each
    (12, 4095, 2048, 16),    # one row short of wide: the tiled kernel
    (12, 2048, 2048, 600),   # decoded weight planes (from 512 tokens): 8 x 5 tiles, K split
    (14, 1024, 2048, 700),   # ... Q6_K, ragged token tile, K split
    (12, 1100, 2560, 513),   # ... ragged row tile (1100 = 4.3 x 256), 10 blocks per row
    (14, 2048, 6144, 1030),  # ... ffn_down shape, 24 blocks per row
    (12, 6144, 2048, 700),   # ... ffn_gate shape, 24 x 6 tiles: one slice, no split
    (12, 4352, 512, 2048),   # ... 17 x 16 = 272 tiles: one whole round unsplit, the 16 left split along K
    (14, 2176, 512, 2000),   # ... Q6_K likewise, ragged token tile
    (14, 2560, 9728, 520),   # ... 4B ffn_down: 38 blocks per row, K slices of unequal length
]


@pytest.mark.parametrize("t,rows,cols,n", SHAPES)
def test_matmul_quant_vs_f64(gpu, ora, t, rows, cols, n):
    import torch

    case(f"matmul type={t} rows={rows} cols={cols} n={n}")
    rng = np.random.default_rng(700 + rows + cols + n + t)
    w = synth.quant_table(rng, t, rows, cols)
    x = rng.normal(0, 1, (n, cols)).astype(np.float32)
    out = torch.full((n, rows), np.nan, dtype=torch.float32, device="cuda")
    gpu.GpuMatMulQuant(gpu.GpuTensor(dev(w), t, rows, cols), dev(x), n, out)
    exact, absdot = ora.matmul_quant_f64(t, w, rows, cols, x)
    check(host(out), exact, absdot, cols, factored_magnitude(ora, t, w, rows, cols, x))


@pytest.mark.parametrize("bench_scales", [False, True], ids=["int8 scales", "bench scales"])
def test_matmul_quant_lm_head_shape(gpu, ora, bench_scales):
    """The 1.7B output projection: [151936, 2048] Q6_K at n = 1, with the scales
    a quantised model carries (the whole int8 range, -128 in every block) and
    with the benchmark's table (scales in -32..31)."""
    import torch

    t, rows, cols = 14, 151936, 2048
    case(f"matmul lm_head rows={rows} bench_scales={bench_scales}")
    rng = np.random.default_rng(790)
    w = synth.quant_table(rng, t, rows, cols, bench_scales=bench_scales)
    x = rng.normal(0, 1, (1, cols)).astype(np.float32)
    out = torch.empty((1, rows), dtype=torch.float32, device="cuda")
    wd = dev(w)
    gpu.GpuMatMulQuant(gpu.GpuTensor(wd, t, rows, cols), dev(x), 1, out)
    exact, absdot = ora.matmul_quant_f64(t, w, rows, cols, x)
    got = host(out)
    check(got, exact, absdot, cols)
    # deterministic: a second call gives the same bits
    out2 = torch.empty_like(out)
    gpu.GpuMatMulQuant(gpu.GpuTensor(wd, t, rows, cols), dev(x), 1, out2)
    assert np.array_equal(host(out2).view(np.uint32), got.view(np.uint32))


@pytest.mark.parametrize("scale", [0.0, 1e-30, 1e30, "outlier"])
def test_matmul_q6k_decode_activation_range(gpu, ora, scale):
    """Tall Q6_K one-token matvec (the output projection's kernel): all-zero rows,
    tiny and huge activations and one outlier 2^20 times the rest all stay within
    the summation bound, with scales over the whole int8 range."""
    import torch

    t, rows, cols = 14, 16400, 2048
    case(f"matmul Q6_K tall decode, activations x {scale}")
    rng = np.random.default_rng(791)
    w = synth.quant_table(rng, t, rows, cols)
    x = rng.normal(0, 1, (1, cols)).astype(np.float32)
    if scale == "outlier":
        x[0, 77] = 2.0 ** 20
    else:
        x = (x * np.float32(scale)).astype(np.float32)
    out = torch.full((1, rows), np.nan, dtype=torch.float32, device="cuda")
    gpu.GpuMatMulQuant(gpu.GpuTensor(dev(w), t, rows, cols), dev(x), 1, out)
    exact, absdot = ora.matmul_quant_f64(t, w, rows, cols, x)
    got = host(out)
    if scale == 0.0:
        assert np.all(got == 0.0)
    check(got, exact, absdot, cols)


def test_matmul_q6k_extreme_scales(gpu, ora):
    """Q6_K blocks at the ends of the format: scales -128 and 127 with quants 0
    and 63, so |sc (q - 32)| reaches 4096 (12 significant bits, more than fp16
    holds) in every decode and prefill kernel; the results must stay within the
    summation bound, and -128 * -32 * d exact."""
    import torch

    cols = 2048
    for rows, n in ((16400, 1), (1024, 1), (300, 5), (2048, 64)):
        case(f"matmul Q6_K extreme scales [{rows} x {cols}] x {n}")
        rng = np.random.default_rng(792 + n)
        w = synth.quant_table(rng, 14, rows, cols).reshape(-1, 210)
        w[:, 0:128] = np.where(rng.random((w.shape[0], 128)) < 0.5, 0x00, 0xFF)  # q low nibbles 0 / 15
        w[:, 128:192] = np.where(rng.random((w.shape[0], 64)) < 0.5, 0x00, 0xFF)  # high bits 0 / 3 -> q 0 / 63
        sc = np.where(rng.random((w.shape[0], 16)) < 0.5, -128, 127).astype(np.int8)
        w[:, 192:208] = sc.view(np.uint8)
        w = w.reshape(-1)
        x = rng.normal(0, 1, (n, cols)).astype(np.float32)
        out = torch.full((n, rows), np.nan, dtype=torch.float32, device="cuda")
        gpu.GpuMatMulQuant(gpu.GpuTensor(dev(w), 14, rows, cols), dev(x), n, out)
        exact, absdot = ora.matmul_quant_f64(14, w, rows, cols, x)
        check(host(out), exact, absdot, cols)


@pytest.mark.parametrize("t,w_off,x_off", [(12, 4, 0), (14, 1, 0), (14, 2, 0), (12, 0, 1), (0, 0, 0), (0, 4, 3)])
def test_matmul_quant_generic_paths(gpu, ora, t, w_off, x_off):
    """F32 matrices, weights that are not 16- (Q4_K) / 2-byte (Q6_K) aligned and
    unaligned activations take the per-element kernel; same bar."""
    import torch

    rows, cols, n = 300, 512, 3
    case(f"matmul generic type={t} w_off={w_off} x_off={x_off}")
    rng = np.random.default_rng(800 + t + w_off + x_off)
    w = synth.quant_table(rng, t, rows, cols)
    wbuf = np.zeros(w.size + 16, np.uint8)
    wbuf[w_off:w_off + w.size] = w
    x = rng.normal(0, 1, (n, cols)).astype(np.float32)
    xbuf = np.zeros(x.size + 4, np.float32)
    xbuf[x_off:x_off + x.size] = x.reshape(-1)
    wd, xd = dev(wbuf), dev(xbuf)
    out = torch.empty((n, rows), dtype=torch.float32, device="cuda")
    rc = gpu.load_library().rpg_op_matmul_quant(t, wd.data_ptr() + w_off, rows, cols, xd.data_ptr() + 4 * x_off, n,
                                                 out.data_ptr())
    assert rc == 0, last_error(gpu)
    exact, absdot = ora.matmul_quant_f64(t, w, rows, cols, x)
    check(host(out), exact, absdot, cols, factored_magnitude(ora, t, w, rows, cols, x))


def test_matmul_quant_one_hot_selects_columns(gpu, ora):
    """One-hot activations: every output is a single product w * 1.0, so the GPU
    result equals the dequantised weight bit for bit (no summation error exists)."""
    import torch

    rows, cols = 1000, 2048
    for t in (12, 14):
        case(f"matmul one-hot type={t}")
        rng = np.random.default_rng(810 + t)
        w = synth.quant_table(rng, t, rows, cols)
        picks = [0, 31, 32, 255, 256, 1000, 2047]
        x = np.zeros((len(picks), cols), np.float32)
        x[np.arange(len(picks)), picks] = 1.0
        out = torch.empty((len(picks), rows), dtype=torch.float32, device="cuda")
        gpu.GpuMatMulQuant(gpu.GpuTensor(dev(w), t, rows, cols), dev(x), len(picks), out)
        rb = ora.row_bytes(t, cols)
        wd = np.stack([ora.dequantize_row(t, w[r * rb:(r + 1) * rb], cols) for r in range(rows)])
        want = wd[:, picks].T
        got = host(out)
        # +0 and -0 products sum to +0 in fp32 FMA chains; compare values, not bits, for zeros
        assert np.array_equal(got == 0, want == 0)
        nz = want != 0
        assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))


def test_matmul_quant_rejects_bad_shapes(gpu):
    import torch

    case("matmul host errors")
    w = torch.zeros(144 * 4, dtype=torch.uint8, device="cuda")
    x = torch.zeros(512, dtype=torch.float32, device="cuda")
    out = torch.zeros(8, dtype=torch.float32, device="cuda")
    L = gpu.load_library()
    assert L.rpg_op_matmul_quant(12, w.data_ptr(), 2, 300, x.data_ptr(), 1, out.data_ptr()) != 0
    assert "do not fill whole blocks of 256" in last_error(gpu)
    assert L.rpg_op_matmul_quant(12, w.data_ptr(), 2, 512, x.data_ptr(), 0, out.data_ptr()) != 0
    assert L.rpg_op_matmul_quant(99, w.data_ptr(), 2, 512, x.data_ptr(), 1, out.data_ptr()) != 0


GROUPS = [
    # (label, [(type, rows)], cols, n_tokens)
    ("q/k/v of a 1.7B layer", [(12, 2048), (12, 1024), (14, 1024)], 2048, 1),
    ("gate/up", [(12, 6144), (12, 6144)], 2048, 1),
    ("four Q6_K", [(14, 256), (14, 512), (14, 130), (14, 1000)], 1024, 1),
    ("mixed runs", [(14, 300), (12, 200), (12, 128), (14, 64), (14, 64)], 512, 1),
    ("Q6_K first, mixed launch", [(14, 300), (12, 200), (12, 128), (14, 64)], 512, 1),
    ("mixed, one Q6_K of odd rows (not fused)", [(12, 256), (14, 7)], 256, 1),
    ("odd rows (not fused)", [(12, 1001), (12, 7)], 256, 1),
    ("Q4_K of 32768+ rows (own shape)", [(12, 20000), (12, 16000)], 256, 1),
    # mixed types with several row steps per wave (the mixed kernel's two row buffers in turn)
    ("mixed, ~3 row steps per wave, buffer loads", [(12, 12000), (14, 12000)], 512, 1),
    ("mixed, ~3 row steps per wave, unaligned Q6_K rows", [(12, 20000), (14, 4000)], 256, 1),
    ("prefill (one call per matrix)", [(12, 256), (14, 128)], 512, 40),
    ("prefill, decoded planes", [(12, 2048), (12, 1024), (14, 1024)], 2048, 600),
    ("small batch", [(12, 256), (12, 256)], 512, 3),
]


@pytest.mark.parametrize("label,mats,cols,n", GROUPS, ids=[g[0] for g in GROUPS])
def test_matmul_group_equals_separate_calls(gpu, ora, label, mats, cols, n):
    """GpuMatMulQuantGroup: every output bit-identical to its own GpuMatMulQuant,
    and within the matmul bound of the float64 oracle."""
    import torch

    case(f"matmul group {label}")
    rng = np.random.default_rng(900 + cols + n + len(mats))
    ws, outs, want = [], [], []
    x = rng.normal(0, 1, (n, cols)).astype(np.float32)
    xd = dev(x)
    for t, rows in mats:
        w = synth.quant_table(rng, t, rows, cols)
        g = gpu.GpuTensor(dev(w), t, rows, cols)
        ws.append((g, w))
        outs.append(torch.full((n, rows), np.nan, dtype=torch.float32, device="cuda"))
        ref = torch.full((n, rows), np.nan, dtype=torch.float32, device="cuda")
        gpu.GpuMatMulQuant(g, xd, n, ref)
        want.append(ref)
    gpu.GpuMatMulQuantGroup([g for g, _ in ws], xd, n, outs)
    for (g, w), o, r, (t, rows) in zip(ws, outs, want, mats):
        assert torch.equal(o, r), (label, t, rows)
        exact, absdot = ora.matmul_quant_f64(t, w, rows, cols, x)
        check(host(o), exact, absdot, cols, factored_magnitude(ora, t, w, rows, cols, x))


SWIGLU = [
    (12, 6144, 2048, 1),   # Qwen3-1.7B gate / up (Q4_K): one paired launch
    (14, 6144, 2048, 1),   # the same in Q6_K
    (12, 9728, 2560, 1),   # Qwen3-4B: 10 blocks per row, not a paired shape
    (12, 300, 512, 1),     # small paired shape, ragged last wave
    (12, 6144, 2048, 3),   # several tokens: group matmul, then SwiGLU
    (12, 6144, 2048, 40),  # the matrix-core path
]


@pytest.mark.parametrize("t,rows,cols,n", SWIGLU)
def test_matmul_swiglu_equals_group_then_silu(gpu, t, rows, cols, n):
    """GpuMatMulQuantSwiGLU: gate bit-identical to GpuMatMulQuantGroup({gate, up})
    followed by GpuSiluMulInPlace (the paired kernel forms each row pair's totals
    exactly as the unpaired kernel does, and the same SwiGLU expression)."""
    import torch

    case(f"matmul swiglu type={t} rows={rows} cols={cols} n={n}")
    rng = np.random.default_rng(1300 + rows + cols + n + t)
    wg = gpu.GpuTensor(dev(synth.quant_table(rng, t, rows, cols)), t, rows, cols)
    wu = gpu.GpuTensor(dev(synth.quant_table(rng, t, rows, cols)), t, rows, cols)
    x = dev(rng.normal(0, 1, (n, cols)).astype(np.float32))
    g1 = torch.full((n, rows), np.nan, dtype=torch.float32, device="cuda")
    u1 = torch.full_like(g1, np.nan)
    gpu.GpuMatMulQuantGroup([wg, wu], x, n, [g1, u1])
    gpu.GpuSiluMulInPlace(g1, u1, n * rows)
    g2 = torch.full_like(g1, np.nan)
    u2 = torch.full_like(g1, np.nan)
    gpu.GpuMatMulQuantSwiGLU(wg, wu, x, n, g2, u2)
    assert torch.equal(g2, g1)


def test_matmul_group_rejects_mixed_widths(gpu):
    import torch

    case("matmul group host errors")
    a = gpu.GpuTensor(torch.zeros(256 * 144 // 256 * 4, dtype=torch.uint8, device="cuda"), 12, 4, 256)
    b = gpu.GpuTensor(torch.zeros(512 * 144 // 256 * 4, dtype=torch.uint8, device="cuda"), 12, 4, 512)
    x = torch.zeros(512, device="cuda")
    with pytest.raises(gpu.RpgError, match="width"):
        gpu.GpuMatMulQuantGroup([a, b], x, 1, [torch.zeros(4, device="cuda"), torch.zeros(4, device="cuda")])


# The sub-layer norm inside the one-token matmul (GpuNormMatMulQuantGroup /
# GpuNormMatMulQuantSwiGLU). Reference path: GpuAddRmsNorm (or GpuRmsNorm with no
# delta) into h, then the plain call on h. The fused kernels take the double sum
# of squares in another order, so h could differ in the last fp32 bit only if
# the double sum fell within ~2^-29 (relative) of an fp32 rounding boundary of
# the scale; for these seeded inputs it does not, so the outputs must be
# bit-identical to the two-step path (and both within the matmul bound of the
# float64 oracle on h).
NORM_GROUPS = [
    # (label, [(type, rows)], cols, with_d, with_x_out)
    ("q/k/v of a 1.7B layer, pending residual", [(12, 2048), (12, 1024), (14, 1024)], 2048, True, True),
    ("first layer: no residual delta", [(12, 2048), (12, 1024), (14, 1024)], 2048, False, False),
    ("output norm + Q6_K head, residual not kept", [(14, 5000)], 2048, True, False),
    ("Q4_K of 32768+ rows (4 rows per wave)", [(12, 33000)], 256, True, True),
    ("runs, odd rows", [(14, 300), (12, 200), (12, 7), (14, 64), (14, 64)], 512, True, True),
    ("three blocks per row", [(12, 128), (14, 96)], 768, True, True),
    ("mixed, ~3 row steps per wave", [(12, 12000), (14, 12000)], 512, True, True),
]


def _norm_inputs(gpu, rng, cols, with_d, eps=1e-6):
    import torch

    x = dev(rng.normal(0, 1, cols).astype(np.float32))
    d = dev(rng.normal(0, 1, cols).astype(np.float32)) if with_d else None
    w = dev(rng.normal(1, 0.1, cols).astype(np.float32))
    xr = x.clone()
    h = torch.full_like(x, np.nan)
    if with_d:
        gpu.GpuAddRmsNorm(xr, d, w, 1, cols, eps, h)
    else:
        gpu.GpuRmsNorm(xr, w, 1, cols, cols, eps, h)
    return x, d, w, xr, h


@pytest.mark.parametrize("label,mats,cols,with_d,with_x_out", NORM_GROUPS, ids=[g[0] for g in NORM_GROUPS])
def test_norm_matmul_group_equals_two_step(gpu, ora, label, mats, cols, with_d, with_x_out):
    import torch

    case(f"norm matmul group {label}")
    rng = np.random.default_rng(1700 + cols + len(mats))
    eps = 1e-6
    x, d, w, xr, h = _norm_inputs(gpu, rng, cols, with_d, eps)
    ws, want, outs = [], [], []
    for t, rows in mats:
        wq = synth.quant_table(rng, t, rows, cols)
        ws.append((gpu.GpuTensor(dev(wq), t, rows, cols), wq))
        want.append(torch.full((1, rows), np.nan, dtype=torch.float32, device="cuda"))
        outs.append(torch.full((1, rows), np.nan, dtype=torch.float32, device="cuda"))
    gpu.GpuMatMulQuantGroup([g for g, _ in ws], h, 1, want)
    x_out = torch.full_like(x, np.nan) if with_x_out else None
    x0 = x.clone()
    assert gpu.GpuNormMatMulQuantGroup(x, d, w, eps, x_out, [g for g, _ in ws], outs)
    assert torch.equal(x, x0)
    if with_x_out:
        assert torch.equal(x_out, xr)  # x + d, one IEEE add
    hh = host(h)[None, :]
    for (g, wq), o, r, (t, rows) in zip(ws, outs, want, mats):
        assert torch.equal(o, r), (label, t, rows)
        exact, absdot = ora.matmul_quant_f64(t, wq, rows, cols, hh)
        check(host(o), exact, absdot, cols, factored_magnitude(ora, t, wq, rows, cols, hh))


@pytest.mark.parametrize("t,rows,cols", [(12, 6144, 2048), (14, 6144, 2048), (12, 130, 1024)])
def test_norm_matmul_swiglu_equals_two_step(gpu, t, rows, cols):
    import torch

    case(f"norm matmul swiglu type={t} rows={rows} cols={cols}")
    rng = np.random.default_rng(1800 + rows + cols + t)
    eps = 1e-6
    x, d, w, xr, h = _norm_inputs(gpu, rng, cols, True, eps)
    wg = gpu.GpuTensor(dev(synth.quant_table(rng, t, rows, cols)), t, rows, cols)
    wu = gpu.GpuTensor(dev(synth.quant_table(rng, t, rows, cols)), t, rows, cols)
    g1 = torch.full((1, rows), np.nan, dtype=torch.float32, device="cuda")
    u1 = torch.full_like(g1, np.nan)
    gpu.GpuMatMulQuantSwiGLU(wg, wu, h, 1, g1, u1)
    g2 = torch.full_like(g1, np.nan)
    u2 = torch.full_like(g1, np.nan)
    x_out = torch.full_like(x, np.nan)
    assert gpu.GpuNormMatMulQuantSwiGLU(x, d, w, eps, x_out, wg, wu, g2, u2)
    assert torch.equal(g2, g1)
    assert torch.equal(x_out, xr)


def test_norm_matmul_without_fused_form(gpu):
    """Rows wider than 2048 columns (the 4B hidden size) have no fused form: the
    call launches nothing and says so; an x_out aliasing x is refused."""
    import torch

    case("norm matmul group: no fused form, aliasing")
    rng = np.random.default_rng(1900)
    cols = 2560
    x, d, w, _, _ = _norm_inputs(gpu, rng, cols, True)
    g = gpu.GpuTensor(dev(synth.quant_table(rng, 12, 64, cols)), 12, 64, cols)
    out = torch.full((1, 64), np.nan, dtype=torch.float32, device="cuda")
    x_out = torch.full_like(x, np.nan)
    assert not gpu.GpuNormMatMulQuantGroup(x, d, w, 1e-6, x_out, [g], [out])
    torch.cuda.synchronize()
    assert torch.isnan(out).all() and torch.isnan(x_out).all()
    g2 = gpu.GpuTensor(dev(synth.quant_table(rng, 12, 64, 2048)), 12, 64, 2048)
    x2 = torch.zeros(2048, device="cuda")
    with pytest.raises(gpu.RpgError, match="alias"):
        gpu.GpuNormMatMulQuantGroup(x2, x2.clone(), x2.clone(), 1e-6, x2, [g2], [out])
