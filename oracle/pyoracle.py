"""numpy/ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker, never as the measured or
shipped path. Also binds oracle/_ref/libref_quant.so (the reference's own
quant.cc, built by `make -C oracle ref`) when that library exists.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_quant.so")

F32, Q4_K, Q6_K = 0, 12, 14

_vp, _i32, _i64, _u32, _f32, _f64 = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32,
                                     ctypes.c_float, ctypes.c_double)
_SIGS = {
    "ora_f16_to_f32": (_f32, [ctypes.c_uint16]),
    "ora_f32_to_f16_rne": (ctypes.c_uint16, [_f32]),
    "ora_f32_to_f16_rne_array": (None, [_vp, _i64, _vp]),
    "ora_f16_to_f32_array": (None, [_vp, _i64, _vp]),
    "ora_type_row_bytes": (_i64, [_u32, _i64]),
    "ora_dequantize_row": (ctypes.c_int, [_u32, _vp, _i64, _vp]),
    "ora_embedding_lookup": (ctypes.c_int, [_u32, _vp, _i64, _i64, _vp, _i64, _vp]),
    "ora_matmul_quant_f64": (ctypes.c_int, [_u32, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "ora_attention_f64": (ctypes.c_int, [_vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _i64, _vp, _vp, _vp]),
    "ora_split_mix64": (ctypes.c_uint64, [ctypes.c_uint64]),
    "ora_counter_rng": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
    "ora_counter_uniform": (_f32, [ctypes.c_uint64, ctypes.c_uint64]),
    "ora_argmax": (_i32, [_vp, _i64, _f32]),
    "ora_filter_to_probs": (ctypes.c_int, [_vp, _i64, _f32, _i32, _f32, _vp, _vp]),
    "ora_inverse_sample": (_i32, [_vp, _i64, _f32]),
    "ora_top_p_cut_key": (ctypes.c_uint32, [_vp, _i64, _f32, ctypes.c_int, _vp]),
    "ora_sample_token": (_i32, [_vp, _i64, _f32, _i32, _f32, ctypes.c_uint64, ctypes.c_uint64, _vp]),
    "ora_rms_norm": (None, [_vp, _vp, _i64, _i64, _i64, _f32, _vp]),
    "ora_build_rope_table": (None, [_i32, _f64, _i64, _vp]),
    "ora_rope": (None, [_vp, _i32, _i32, _vp, _i64, _i64]),
    "ora_kv_write": (ctypes.c_int, [_vp, _vp, _i32, _i32, _i64, _i64, _vp, _vp, _i64]),
    "ora_silu_mul": (None, [_vp, _vp, _i64]),
    "ora_vec_add": (None, [_vp, _vp, _i64]),
    "ora_add_rms_norm": (None, [_vp, _vp, _vp, _i64, _i64, _f32, _vp]),
    "ora_qk_norm_rope_kv": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i64, _i64, _f32, _vp,
                                           _vp, _i64]),
    "ora_rms_norm_f64": (None, [_vp, _vp, _i64, _i64, _i64, _f64, _vp]),
    "ora_rope_f64": (None, [_vp, _i32, _i32, _vp, _i64, _i64, _vp]),
    "ora_silu_mul_f64": (None, [_vp, _vp, _i64, _vp]),
    "ora_norm_rope_f64": (None, [_vp, _vp, _i32, _i32, _vp, _i64, _i64, _f64, _vp]),
    "ora_bench_layer_chain": (_f64, [ctypes.c_int, _i64, _i64, _i32, _i32, _i64, ctypes.c_int]),
    "ora_bench_layer_op": (_f64, [ctypes.c_int, ctypes.c_int, _i64, _i64, _i32, _i32, _i64, ctypes.c_int]),
    "ora_bench_gather": (_f64, [ctypes.c_int, _u32, _i64, _i64, _i64, ctypes.c_int]),
    "ora_bench_matmul": (_f64, [_u32, _i64, _i64, ctypes.c_int]),
}

_lib = None
_ref = None


def build() -> None:
    """Compiles liboracle.so (gcc) in place."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ref_lib():
    """The reference's own quant.cc compiled into oracle/_ref, or None if absent."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        R = ctypes.CDLL(REF_LIB_PATH)
        R.ref_dequantize_row.restype = ctypes.c_int
        R.ref_dequantize_row.argtypes = [_u32, _vp, _i64, _vp]
        R.ref_type_row_bytes.restype = _i64
        R.ref_type_row_bytes.argtypes = [_u32, _i64]
        R.ref_f16_to_f32_array.restype = None
        R.ref_f16_to_f32_array.argtypes = [_vp, _i64, _vp]
        R.ref_f32_to_f16_dtypes.restype = ctypes.c_uint16
        R.ref_f32_to_f16_dtypes.argtypes = [_f32]
        if hasattr(R, "ref_bench_gather"):
            R.ref_bench_gather.restype = ctypes.c_double
            R.ref_bench_gather.argtypes = [_u32, _vp, _i64, _vp, _i64, _i64, _vp, ctypes.c_int]
        _ref = R
    return _ref


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------------- fp16


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.empty(bits.size, dtype=np.float32)
    lib().ora_f16_to_f32_array(_p(bits), bits.size, _p(out))
    return out


def ref_f16_to_f32(bits: np.ndarray):
    R = ref_lib()
    if R is None:
        return None
    bits = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.empty(bits.size, dtype=np.float32)
    R.ref_f16_to_f32_array(_p(bits), bits.size, _p(out))
    return out


def f32_to_f16_rne(x: np.ndarray) -> np.ndarray:
    x = _f(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().ora_f32_to_f16_rne_array(_p(x), x.size, _p(out))
    return out


# ------------------------------------------------------------------------- dequant


def row_bytes(ggml_type: int, n: int) -> int:
    return int(lib().ora_type_row_bytes(ggml_type, n))


def dequantize_row(ggml_type: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    assert raw.size >= row_bytes(ggml_type, n)
    out = np.empty(n, dtype=np.float32)
    assert lib().ora_dequantize_row(ggml_type, _p(raw), n, _p(out)) == 0
    return out


def embedding_lookup(ggml_type: int, table: np.ndarray, rows: int, cols: int, toks: np.ndarray) -> np.ndarray:
    table = np.ascontiguousarray(table, dtype=np.uint8)
    toks = np.ascontiguousarray(toks, dtype=np.int32)
    out = np.empty((toks.size, cols), dtype=np.float32)
    assert lib().ora_embedding_lookup(ggml_type, _p(table), rows, cols, _p(toks), toks.size, _p(out)) == 0
    return out


def matmul_quant_f64(ggml_type: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray):
    """(out, absdot), both float64 [n_tokens, rows]: OUT = X . W^T to double accuracy and
    sum |w * x| per output (the scale of fp32 summation error)."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    assert w.size >= rows * row_bytes(ggml_type, cols)
    out = np.empty((x.shape[0], rows), dtype=np.float64)
    absdot = np.empty_like(out)
    assert lib().ora_matmul_quant_f64(ggml_type, _p(w), rows, cols, _p(x), x.shape[0], _p(out), _p(absdot)) == 0
    return out, absdot


def attention_f64(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, max_seq: int, n_heads: int, n_kv_heads: int,
                  d: int, pos0: int, seq: int):
    """(out, smag, vmax) in float64: out [seq, n_heads, d]; smag / vmax [seq, n_heads]."""
    q = np.ascontiguousarray(q, dtype=np.float32).reshape(-1)
    kc = np.ascontiguousarray(kc, dtype=np.uint16).reshape(-1)
    vc = np.ascontiguousarray(vc, dtype=np.uint16).reshape(-1)
    out = np.empty((seq, n_heads, d), dtype=np.float64)
    smag = np.empty((seq, n_heads), dtype=np.float64)
    vmax = np.empty((seq, n_heads), dtype=np.float64)
    assert lib().ora_attention_f64(_p(q), _p(kc), _p(vc), max_seq, n_heads, n_kv_heads, d, pos0, seq, _p(out),
                                   _p(smag), _p(vmax)) == 0
    return out, smag, vmax


def ref_bench_gather(ggml_type: int, rows: int, cols: int, seq: int, reps: int):
    """Seconds for the reference's own CPU gather (one DequantizeRow per token
    row, one thread) of `seq` random rows of a [rows, cols] table with uniform
    block bytes and fp16 scales |N(0, 0.01)|, or None without oracle/_ref."""
    R = ref_lib()
    if R is None or not hasattr(R, "ref_bench_gather"):
        return None
    rb = int(R.ref_type_row_bytes(ggml_type, cols))
    rng = np.random.default_rng(7)
    table = rng.integers(0, 256, size=rows * rb, dtype=np.uint8)
    blk = table.reshape(-1, 144 if ggml_type == Q4_K else 210)
    # the benchmark configuration's fp16 scales: d (and dmin) = |N(0, 0.01)|
    scales = [0, 2] if ggml_type == Q4_K else [208]
    for off in scales:
        half = np.abs(rng.normal(0.0, 0.01, blk.shape[0])).astype(np.float16)
        blk[:, off:off + 2] = half.view(np.uint8).reshape(-1, 2)
    ids = rng.integers(0, rows, size=seq).astype(np.int32)
    out = np.empty(seq * cols, dtype=np.float32)
    s = float(R.ref_bench_gather(ggml_type, _p(table), rb, _p(ids), seq, cols, _p(out), reps))
    return s if s > 0 else None


def ref_dequantize_row(ggml_type: int, raw: np.ndarray, n: int):
    R = ref_lib()
    if R is None:
        return None
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    assert R.ref_dequantize_row(ggml_type, _p(raw), n, _p(out)) == 0
    return out


# ------------------------------------------------------------------------- layer ops (fp32)


def split_mix64(x: int) -> int:
    return int(lib().ora_split_mix64(x))


def counter_rng(seed: int, counter: int) -> int:
    return int(lib().ora_counter_rng(seed, counter))


def counter_uniform(seed: int, counter: int) -> float:
    return float(lib().ora_counter_uniform(seed, counter))


def argmax(x: np.ndarray, init: float) -> int:
    x = _f(x)
    return int(lib().ora_argmax(_p(x), x.size, init))


def filter_to_probs(logits: np.ndarray, temperature: float, top_k: int, top_p: float):
    """(probs, margin): the filtered distribution and top_p's decision margin."""
    logits = _f(logits)
    probs = np.empty_like(logits)
    margin = ctypes.c_double(0.0)
    rc = lib().ora_filter_to_probs(_p(logits), logits.size, temperature, top_k, top_p, _p(probs),
                                   ctypes.byref(margin))
    if rc != 0:
        raise ValueError("ora_filter_to_probs failed")
    return probs, float(margin.value)


TOPP_EXACT, TOPP_GRID62, TOPP_DOUBLE = 0, 1, 2


def top_p_cut(probs: np.ndarray, top_p: float, rule: int) -> float:
    """The top_p cut value (every p <= it is dropped) under `rule`: TOPP_EXACT (the
    oracle's exact mass), TOPP_GRID62 (the device kernel's 2^-62 grid) or
    TOPP_DOUBLE (the reference's double sums)."""
    probs = _f(probs)
    key = int(lib().ora_top_p_cut_key(_p(probs), probs.size, top_p, rule, None))
    assert key != 0, "allocation failed"
    u = key & 0x7FFFFFFF if key & 0x80000000 else ~key & 0xFFFFFFFF
    return float(np.array([u], np.uint32).view(np.float32)[0])


def inverse_sample(probs: np.ndarray, u: float) -> int:
    probs = _f(probs)
    return int(lib().ora_inverse_sample(_p(probs), probs.size, u))


def sample_token(logits: np.ndarray, temperature: float, top_k: int, top_p: float, seed: int, counter: int) -> int:
    logits = _f(logits)
    scratch = np.empty_like(logits)
    return int(lib().ora_sample_token(_p(logits), logits.size, temperature, top_k, top_p, seed, counter,
                                      _p(scratch)))


def rms_norm(x: np.ndarray, w: np.ndarray, n_rows: int, n: int, stride: int, eps: float) -> np.ndarray:
    x = _f(x)
    out = x.copy()
    lib().ora_rms_norm(_p(x), _p(_f(w)), n_rows, n, stride, eps, _p(out))
    return out


def build_rope_table(head_dim: int, theta: float, n_pos: int) -> np.ndarray:
    out = np.empty((n_pos, head_dim), dtype=np.float32)
    lib().ora_build_rope_table(head_dim, theta, n_pos, _p(out))
    return out


def rope(x: np.ndarray, n_heads: int, head_dim: int, tab: np.ndarray, pos0: int, n_rows: int) -> np.ndarray:
    out = _f(x).copy()
    lib().ora_rope(_p(out), n_heads, head_dim, _p(_f(tab)), pos0, n_rows)
    return out


def kv_write(k, v, n_kv_heads, head_dim, pos0, seq, k_layer: np.ndarray, v_layer: np.ndarray, max_seq) -> int:
    assert k_layer.dtype == np.uint16 and v_layer.dtype == np.uint16
    return lib().ora_kv_write(_p(_f(k)), _p(_f(v)), n_kv_heads, head_dim, pos0, seq, _p(k_layer), _p(v_layer),
                              max_seq)


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    out = _f(gate).copy()
    lib().ora_silu_mul(_p(out), _p(_f(up)), out.size)
    return out


def vec_add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    out = _f(a).copy()
    lib().ora_vec_add(_p(out), _p(_f(b)), out.size)
    return out


def add_rms_norm(x, d, w, n_rows, n, eps):
    """Returns (x + d, RMSNorm(x + d) * w)."""
    xs = _f(x).copy()
    out = np.empty_like(xs)
    lib().ora_add_rms_norm(_p(xs), _p(_f(d)), _p(_f(w)), n_rows, n, eps, _p(out))
    return xs, out


def qk_norm_rope_kv(q, k, v, q_norm, k_norm, n_heads, n_kv_heads, head_dim, tab, pos0, seq, eps,
                    k_layer: np.ndarray, v_layer: np.ndarray, max_seq):
    """Returns (q', k') after the composition; writes the caches in place."""
    qo = _f(q).copy()
    ko = _f(k).copy()
    rc = lib().ora_qk_norm_rope_kv(_p(qo), _p(ko), _p(_f(v)), _p(_f(q_norm)), _p(_f(k_norm)), n_heads, n_kv_heads,
                                   head_dim, _p(_f(tab)), pos0, seq, eps, _p(k_layer), _p(v_layer), max_seq)
    assert rc == 0
    return qo, ko


# ------------------------------------------------------------------------- float64 restatements


def rms_norm_f64(x, w, n_rows, n, stride, eps) -> np.ndarray:
    out = np.empty((n_rows, n), dtype=np.float64)
    lib().ora_rms_norm_f64(_p(_f(x)), _p(_f(w)), n_rows, n, stride, eps, _p(out))
    return out


def rope_f64(x, n_heads, head_dim, tab, pos0, n_rows) -> np.ndarray:
    out = np.empty(n_rows * n_heads * head_dim, dtype=np.float64)
    lib().ora_rope_f64(_p(_f(x)), n_heads, head_dim, _p(_f(tab)), pos0, n_rows, _p(out))
    return out


def silu_mul_f64(gate, up) -> np.ndarray:
    g = _f(gate)
    out = np.empty(g.size, dtype=np.float64)
    lib().ora_silu_mul_f64(_p(g), _p(_f(up)), g.size, _p(out))
    return out


def norm_rope_f64(x, w, n_heads, head_dim, tab, pos0, n_rows, eps) -> np.ndarray:
    out = np.empty(n_rows * n_heads * head_dim, dtype=np.float64)
    lib().ora_norm_rope_f64(_p(_f(x)), _p(_f(w)), n_heads, head_dim, _p(_f(tab)), pos0, n_rows, eps, _p(out))
    return out


# ------------------------------------------------------------------------- CPU baseline timing


def bench_layer_chain(threads, n, hidden, n_heads, n_kv_heads, inter, reps) -> float:
    return float(lib().ora_bench_layer_chain(threads, n, hidden, n_heads, n_kv_heads, inter, reps))


def bench_layer_op(op, threads, n, hidden, n_heads, n_kv_heads, inter, reps) -> float:
    return float(lib().ora_bench_layer_op(op, threads, n, hidden, n_heads, n_kv_heads, inter, reps))


def bench_gather(threads, ggml_type, rows, cols, seq, reps) -> float:
    return float(lib().ora_bench_gather(threads, ggml_type, rows, cols, seq, reps))


def bench_matmul(ggml_type, rows, cols, reps) -> float:
    return float(lib().ora_bench_matmul(ggml_type, rows, cols, reps))
