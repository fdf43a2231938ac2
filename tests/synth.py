"""Seeded synthetic inputs shaped like the benchmark configurations (test infrastructure).

All generators take a numpy Generator so a test's seed fixes its inputs.
Q4_K / Q6_K tables follow the benchmark's description of the synthetic token_embd:
  Q4_K: d, dmin = fp16_rne(|N(0, 0.01)|); the 12 packed scale bytes uniform
        (every unpacked 6-bit scale/min uniform over 0..63); qs uniform bytes.
  Q6_K: d = fp16_rne(|N(0, 0.01)|); ql / qh uniform bytes (6-bit quants uniform);
        scales int8 over the format's whole range by default: uniform over
        -128..127 with one scale of each block set to -128, which is what the
        llama.cpp quantiser writes (the block's largest-magnitude scale maps to
        -128). bench_scales=True gives the benchmark's table instead, scales
        uniform over -32..31, where every sc * (q - 32) fits in 11 bits.
"""
from __future__ import annotations

import numpy as np

Q4K_BYTES = 144
Q6K_BYTES = 210

QWEN3_1_7B = dict(hidden=2048, n_heads=16, n_kv_heads=8, head_dim=128, inter=6144, n_layers=28)
QWEN3_4B = dict(hidden=2560, n_heads=32, n_kv_heads=8, head_dim=128, inter=9728, n_layers=36)
EPS = 1e-6
THETA = 1e6


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def q4k_blocks(rng: np.random.Generator, n_blocks: int) -> np.ndarray:
    """n_blocks raw Q4_K super-blocks, shape [n_blocks, 144] uint8."""
    b = rng.integers(0, 256, size=(n_blocks, Q4K_BYTES), dtype=np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, 0.01, n_blocks)))
    dmin = f16_bits(np.abs(rng.normal(0.0, 0.01, n_blocks)))
    b[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    b[:, 2:4] = dmin.view(np.uint8).reshape(n_blocks, 2)
    return b


def q6k_blocks(rng: np.random.Generator, n_blocks: int, bench_scales: bool = False) -> np.ndarray:
    """n_blocks raw Q6_K super-blocks, shape [n_blocks, 210] uint8."""
    b = rng.integers(0, 256, size=(n_blocks, Q6K_BYTES), dtype=np.uint8)
    if bench_scales:
        sc = rng.integers(-32, 32, size=(n_blocks, 16)).astype(np.int8)
    else:
        sc = rng.integers(-128, 128, size=(n_blocks, 16)).astype(np.int8)
        sc[np.arange(n_blocks), rng.integers(0, 16, size=n_blocks)] = -128
    b[:, 192:208] = sc.view(np.uint8)
    d = f16_bits(np.abs(rng.normal(0.0, 0.01, n_blocks)))
    b[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return b


def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """[n, 8] 6-bit scales and mins -> the 12 packed bytes of a Q4_K block (the
    inverse of the format's get_scale_min_k4: entries 0-3 in the low 6 bits of
    bytes 0-3 / 4-7, entries 4-7 split over bytes 8-11 and the top 2 bits)."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.zeros((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return out


def model_q4k_blocks(rng: np.random.Generator, n_blocks: int, d: float = 0.002) -> np.ndarray:
    """Q4_K blocks whose values look like trained weights: zero mean, std ~ 10 d.
    Scales uniform over 1..8 with the min m = round(7.5 sc), so d (sc q - m)
    centres q = 0..15 on zero."""
    b = rng.integers(0, 256, size=(n_blocks, Q4K_BYTES), dtype=np.uint8)
    dd = f16_bits(np.full(n_blocks, d) * rng.uniform(0.5, 1.5, n_blocks))
    b[:, 0:2] = dd.view(np.uint8).reshape(n_blocks, 2)
    b[:, 2:4] = dd.view(np.uint8).reshape(n_blocks, 2)  # dmin = d
    sc = rng.integers(1, 9, size=(n_blocks, 8))
    m = np.rint(7.5 * sc).astype(np.int64)
    b[:, 4:16] = pack_q4k_scales(sc, m)
    return b


def model_q6k_blocks(rng: np.random.Generator, n_blocks: int, d: float = 2.5e-5) -> np.ndarray:
    """Q6_K blocks with trained-weight-like values: d sc (q - 32), zero mean, the
    scales over the whole int8 range with one -128 per block (as quantised)."""
    b = rng.integers(0, 256, size=(n_blocks, Q6K_BYTES), dtype=np.uint8)
    sc = rng.integers(-128, 128, size=(n_blocks, 16)).astype(np.int8)
    sc[np.arange(n_blocks), rng.integers(0, 16, size=n_blocks)] = -128
    b[:, 192:208] = sc.view(np.uint8)
    dd = f16_bits(np.full(n_blocks, d) * rng.uniform(0.5, 1.5, n_blocks))
    b[:, 208:210] = dd.view(np.uint8).reshape(n_blocks, 2)
    return b


def model_table(rng: np.random.Generator, ggml_type: int, rows: int, cols: int) -> np.ndarray:
    """quant_table with model_q4k_blocks / model_q6k_blocks (F32: N(0, 0.02))."""
    nb = cols // 256
    if ggml_type == 12:
        return model_q4k_blocks(rng, rows * nb).reshape(-1)
    if ggml_type == 14:
        return model_q6k_blocks(rng, rows * nb).reshape(-1)
    if ggml_type == 0:
        return rng.normal(0.0, 0.02, rows * cols).astype(np.float32).view(np.uint8)
    raise ValueError(ggml_type)


def quant_table(rng: np.random.Generator, ggml_type: int, rows: int, cols: int,
                bench_scales: bool = False) -> np.ndarray:
    """A [rows, cols] table as raw bytes, shape [rows * row_bytes] uint8."""
    nb = cols // 256
    if ggml_type == 12:
        return q4k_blocks(rng, rows * nb).reshape(-1)
    if ggml_type == 14:
        return q6k_blocks(rng, rows * nb, bench_scales).reshape(-1)
    if ggml_type == 0:
        return rng.normal(0.0, 1.0, rows * cols).astype(np.float32).view(np.uint8)
    raise ValueError(ggml_type)


def special_q4k_blocks() -> np.ndarray:
    """Hand-made Q4_K blocks that reach the edge cases of the formula."""
    out = []
    z = np.zeros(Q4K_BYTES, np.uint8)
    out.append(z.copy())                                   # all zero
    b = np.full(Q4K_BYTES, 0xFF, np.uint8)                 # d = dmin = NaN pattern 0xFFFF avoided below
    b[0:4] = np.array([0x00, 0x3C, 0x00, 0x3C], np.uint8)  # d = dmin = 1.0, every scale/min 63, q = 15
    out.append(b)
    b = z.copy()
    b[0:2] = [0x01, 0x00]                                  # d = smallest f16 subnormal 2^-24
    b[2:4] = [0xFF, 0x03]                                  # dmin = largest subnormal
    b[4:16] = np.arange(12, dtype=np.uint8) * 21           # mixed 6-bit scales / high bits
    b[16:] = np.arange(128, dtype=np.uint8)
    out.append(b)
    b = z.copy()
    b[0:2] = [0x00, 0x3C]                                  # d = 1, dmin = 0 -> y = sc*q exactly
    b[4:16] = 0x3F
    b[16:] = 0xA5
    out.append(b)
    b = z.copy()
    b[0:2] = [0x00, 0x00]                                  # d = 0 -> y = -(dmin*m) (negative or -0)
    b[2:4] = [0x00, 0x40]                                  # dmin = 2
    b[4:16] = np.array([0, 1, 2, 63, 0, 5, 6, 63, 0xC1, 0x72, 0x0F, 0xF0], np.uint8)
    b[16:] = 0x3C
    out.append(b)
    return np.stack(out)


def special_q6k_blocks() -> np.ndarray:
    """Hand-made Q6_K blocks: zero, q = 32 with negative scales (-0.0), extremes, subnormal d."""
    out = []
    z = np.zeros(Q6K_BYTES, np.uint8)
    out.append(z.copy())                                   # all zero: q = -32, sc = 0
    b = z.copy()
    b[0:128] = 0x00                                        # low nibbles 0
    b[128:192] = 0xAA                                      # every 2-bit high part = 2 -> q = 32 - 32 = 0
    b[192:208] = np.array([-1, -32, 5, -7] * 4, np.int8).view(np.uint8)
    b[208:210] = [0x00, 0x3C]                              # d = 1: y = (1*sc)*0 = -0.0 for sc < 0
    out.append(b)
    b = np.full(Q6K_BYTES, 0xFF, np.uint8)                 # q = 31 everywhere
    b[192:208] = np.array([-32, 31] * 8, np.int8).view(np.uint8)
    b[208:210] = [0xFF, 0x7B]                              # d = 65504 (largest finite half)
    out.append(b)
    b = z.copy()
    b[0:192] = np.arange(192, dtype=np.uint8)
    b[192:208] = np.arange(-8, 8, dtype=np.int8).view(np.uint8)
    b[208:210] = [0x01, 0x00]                              # d = 2^-24 (subnormal)
    out.append(b)
    return np.stack(out)


def normal(rng: np.random.Generator, shape, mean=0.0, std=1.0) -> np.ndarray:
    return rng.normal(mean, std, size=shape).astype(np.float32)


# ----------------------------------------------------------------------------- sampling

# The reference's sampler case matrix (tools/sample_check.cu:48-61):
# (temperature, top_k, top_p, seed, tie, description).
SAMPLE_CASES = [
    (0.0, 0, 1.0, 11, False, "greedy"),
    (0.0, 8, 0.9, 12, False, "greedy, filters ignored"),
    (1.0, 0, 1.0, 13, False, "plain distribution"),
    (0.7, 40, 1.0, 14, False, "temperature + top_k 40"),
    (1.3, 0, 0.9, 15, False, "temperature + top_p 0.9"),
    (0.5, 20, 0.95, 16, False, "all three"),
    (1.0, 2, 1.0, 17, False, "top_k 2"),
    (1.0, 0, 0.05, 18, False, "top_p 0.05"),
    (0.001, 0, 1.0, 19, False, "tiny temperature"),
    (5.0, 0, 1.0, 20, False, "large temperature"),
    (1.0, 8, 1.0, 21, True, "exact ties + top_k 8"),
    (0.0, 0, 1.0, 22, True, "exact ties + greedy"),
]
SAMPLE_U_COUNT = 16  # u values drawn per case (tools/sample_check.cu:63)

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def split_mix64_np(x: np.ndarray) -> np.ndarray:
    """SplitMix64 over a uint64 array (wrapping arithmetic)."""
    with np.errstate(over="ignore"):
        z = x.astype(np.uint64) + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def sample_logits(seed: int, tie: bool, n: int) -> np.ndarray:
    """The reference's synthetic logits (tools/sample_check.cu:65-76): x in [0, 1)
    from SplitMix64(seed * 1000003 + i) >> 40, v = (x - 0.5) * 16, with `tie`
    rounded to multiples of 1/8 (exact ties)."""
    with np.errstate(over="ignore"):
        base = np.uint64(seed) * np.uint64(1000003)
        h = split_mix64_np(base + np.arange(n, dtype=np.uint64))
    x = (h >> np.uint64(40)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    v = (x - np.float32(0.5)) * np.float32(16.0)
    if tie:  # std::round: halves away from zero (exact in float64 for float32 input)
        y = (v * np.float32(8.0)).astype(np.float64)
        r = (np.sign(y) * np.floor(np.abs(y) + 0.5)).astype(np.float32)
        v = (r / np.float32(8.0)).astype(np.float32)
    return v.astype(np.float32)


def order_key_np(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return np.where(u & np.uint32(0x80000000), ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def from_order_key_np(k) -> np.ndarray:
    k = np.asarray(k, dtype=np.uint32)
    u = np.where(k & np.uint32(0x80000000), k & np.uint32(0x7FFFFFFF), ~k).astype(np.uint32)
    return u.view(np.float32)
