"""Host-side mirror of the reference operator layer, over librpg_ops.so (ctypes).

Names, argument order and meaning follow the reference's operators
(src/kernels_gpu.h:39-154) so callers and tests read like the reference's own
tools (tools/kv_map_check.cu, tools/dequant_check.cu). Arguments that are
device buffers may be torch tensors on the GPU (their size and dtype are checked
against what the operator will touch before anything is launched) or raw
integer device addresses (then the caller vouches for the sizes).

Failures raise RpgError carrying rpg_ops_last_error(); nothing falls back to a
CPU path: if the library is missing, loading it raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "librpg_ops.so")

GGML_F32 = 0
GGML_Q4_K = 12
GGML_Q6_K = 14
QK_K = 256
BLOCK_BYTES = {GGML_F32: 4, GGML_Q4_K: 144, GGML_Q6_K: 210}
BLOCK_ELEMS = {GGML_F32: 1, GGML_Q4_K: 256, GGML_Q6_K: 256}

# Every symbol include/rpg_ops.h declares, with its ctypes signature.
_i32, _i64, _u32, _f32, _f64, _vp = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_float,
                                     ctypes.c_double, ctypes.c_void_p)
SIGNATURES = {
    "rpg_ops_version": (ctypes.c_char_p, []),
    "rpg_ops_last_error": (ctypes.c_char_p, []),
    "rpg_ops_init": (_i32, []),
    "rpg_ops_set_stream": (_i32, [_vp]),
    "rpg_ops_get_stream": (_vp, []),
    "rpg_ops_stage_pos0": (_i32, [_i64]),
    "rpg_ops_pos_staging_ptr": (_vp, []),
    "rpg_gguf_open": (_i32, [ctypes.c_char_p, _vp]),
    "rpg_gguf_close": (_i32, [_vp]),
    "rpg_gguf_tensor_count": (_i64, [_vp]),
    "rpg_gguf_tensor_info": (_i32, [_vp, _i64, ctypes.c_char_p, _i32, _vp]),
    "rpg_gguf_meta": (_i32, [_vp, ctypes.c_char_p, _i64, _vp, _vp, ctypes.c_char_p, _i32, _vp]),
    "rpg_gguf_model_meta": (_i32, [_vp, _vp]),
    "rpg_gguf_describe": (_i32, [_vp, ctypes.c_char_p, _i32]),
    "rpg_model_load": (_i32, [ctypes.c_char_p, _i32, _vp]),
    "rpg_model_free": (_i32, [_vp]),
    "rpg_model_meta": (_i32, [_vp, _vp]),
    "rpg_model_tensor": (_i32, [_vp, ctypes.c_char_p, _vp]),
    "rpg_model_rope": (_i32, [_vp, _vp, _vp]),
    "rpg_model_describe": (_i32, [_vp, ctypes.c_char_p, _i32]),
    "rpg_model_upload_stats": (_i32, [_vp, _vp, _vp, _vp]),
    "rpg_model_device_bytes": (_i32, [_vp, _vp]),
    "rpg_kv_create": (_i32, [_vp, _i64, _vp]),
    "rpg_kv_create_shape": (_i32, [_i32, _i32, _i32, _i64, _vp]),
    "rpg_kv_free": (_i32, [_vp]),
    "rpg_kv_info": (_i32, [_vp, _vp, _vp, _vp]),
    "rpg_kv_set_len": (_i32, [_vp, _i64]),
    "rpg_kv_layer": (_i32, [_vp, _i32, _vp, _vp]),
    "rpg_scratch_create": (_i32, [_vp]),
    "rpg_scratch_free": (_i32, [_vp]),
    "rpg_scratch_logits": (_i32, [_vp, _vp, _vp]),
    "rpg_forward_full": (_i32, [_vp, _vp, _i64, _vp, _vp, _i32, _vp, _vp]),
    "rpg_forward_step": (_i32, [_vp, _i32, _i64, _vp, _vp, _vp]),
    "rpg_forward_step_dev": (_i32, [_vp, _vp, _i64, _vp, _vp]),
    "rpg_generate": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _vp]),
    "rpg_op_matmul_quant_group": (_i32, [_i32, _vp, _vp, _vp, _i64, _vp, _i64, _vp]),
    "rpg_op_matmul_quant_swiglu": (_i32, [_u32, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "rpg_op_norm_matmul_quant_group": (_i32, [_i32, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _f32, _vp, _vp, _vp]),
    "rpg_op_norm_matmul_quant_swiglu": (_i32, [_u32, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _f32, _vp, _vp, _vp,
                                               _vp]),
    "rpg_op_argmax": (_i32, [_vp, _i64, _vp]),
    "rpg_sample_split_mix64": (ctypes.c_uint64, [ctypes.c_uint64]),
    "rpg_sample_counter_rng": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
    "rpg_sample_counter_uniform": (_f32, [ctypes.c_uint64, ctypes.c_uint64]),
    "rpg_op_filter_to_probs": (_i32, [_vp, _i64, _f32, _i32, _f32, _vp]),
    "rpg_op_inverse_sample": (_i32, [_vp, _i64, _f32, _vp]),
    "rpg_op_sample_token": (_i32, [_vp, _i64, _f32, _i32, _f32, ctypes.c_uint64, ctypes.c_uint64, _vp, _vp]),
    "rpg_op_sample_token_dev": (_i32, [_vp, _i64, _f32, _i32, _f32, ctypes.c_uint64, _vp, _vp, _vp]),
    "rpg_op_sampler_warmup": (_i32, []),
    "rpg_ops_device_info": (_i32, [ctypes.c_char_p, _i32]),
    "rpg_ops_type_row_bytes": (_i64, [_u32, _i64]),
    "rpg_ops_build_rope_table": (_i32, [_i32, _f64, _i64, _vp]),
    "rpg_op_dequant_row": (_i32, [_u32, _vp, _i64, _vp]),
    "rpg_op_rms_norm": (_i32, [_vp, _vp, _i64, _i64, _i64, _f32, _vp]),
    "rpg_op_rope": (_i32, [_vp, _i32, _i32, _vp, _i64, _i64]),
    "rpg_op_kv_write": (_i32, [_vp, _vp, _i32, _i32, _i64, _i64, _vp, _vp, _i64]),
    "rpg_op_silu_mul_inplace": (_i32, [_vp, _vp, _i64]),
    "rpg_op_vec_add_inplace": (_i32, [_vp, _vp, _i64]),
    "rpg_op_embedding_lookup": (_i32, [_u32, _vp, _i64, _i64, _vp, _i64, _vp]),
    "rpg_op_matmul_quant": (_i32, [_u32, _vp, _i64, _i64, _vp, _i64, _vp]),
    "rpg_op_set_force_generic_matmul": (_i32, [_i32]),
    "rpg_op_force_generic_matmul": (_i32, []),
    "rpg_op_attention_from_cache": (_i32, [_vp, _i32, _i32, _i32, _i64, _i64, _vp, _vp, _i64, _vp, _i64]),
    "rpg_op_qk_norm_rope_kv_attention": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i64, _i64, _f32,
                                                _vp, _vp, _i64, _vp, _i64, _vp]),
    "rpg_op_attention_from_cache_noalloc": (_i32, [_vp, _i32, _i32, _i32, _i64, _i64, _vp, _vp, _i64, _vp, _i64]),
    "rpg_op_attention_warmup": (_i32, [_i64]),
    "rpg_op_add_rms_norm": (_i32, [_vp, _vp, _vp, _i64, _i64, _f32, _vp]),
    "rpg_op_qk_norm_rope_kv": (_i32, [_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32, _vp, _i64, _i64, _i64, _f32,
                                      _vp, _vp, _i64, _i32]),
    "rpg_op_stream_copy": (_i32, [_vp, _vp, _i64]),
    "rpg_op_stream_fill": (_i32, [_vp, _i64, _u32]),
    "rpg_op_stream_read": (_i32, [_vp, _i64, _u32, _vp]),
    "rpg_op_f16_sweep": (_i32, [_vp]),
    "rpg_ops_profile_start": (_i32, [_i32]),
    "rpg_ops_profile_stop": (_i32, []),
    "rpg_ops_profile_report": (_i32, [ctypes.c_char_p, _i32]),
}


class RpgError(RuntimeError):
    """An operator rejected its arguments or a HIP call failed."""


_lib: Optional[ctypes.CDLL] = None


def load_library() -> ctypes.CDLL:
    """Loads librpg_ops.so once. torch is imported first so the library binds to
    the HIP runtime torch already loaded (both carry SONAME libamdhip64.so.7)
    and device pointers from torch allocations are valid in it."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  (load order matters, see above)

    if not os.path.exists(LIB_PATH):
        raise RpgError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                       "(python -m rpgbarenginecuda_amd.build)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc: int) -> int:
    if rc < 0:
        msg = load_library().rpg_ops_last_error()
        raise RpgError(msg.decode("utf-8", "replace") if msg else f"error {rc}")
    return rc


def _addr(buf, nbytes: int = 0, dtype=None, name: str = "buffer"):
    """Device address of `buf` (torch tensor or int), checking that a tensor is
    on the GPU, contiguous, of `dtype` and at least `nbytes` long."""
    if buf is None:
        return None
    if isinstance(buf, int):
        return buf
    import torch

    if not isinstance(buf, torch.Tensor):
        raise TypeError(f"{name}: expected a torch tensor or a device address, got {type(buf)}")
    if not buf.is_cuda:
        raise RpgError(f"{name}: tensor is not on the GPU")
    if not buf.is_contiguous():
        raise RpgError(f"{name}: tensor must be contiguous")
    if dtype is not None and buf.dtype != dtype:
        raise RpgError(f"{name}: expected dtype {dtype}, got {buf.dtype}")
    have = buf.numel() * buf.element_size()
    if have < nbytes:
        raise RpgError(f"{name}: operator touches {nbytes} bytes but the tensor holds {have}")
    return buf.data_ptr()


def _t():
    import torch

    return torch


# ----------------------------------------------------------------------------- runtime


def version() -> str:
    return load_library().rpg_ops_version().decode()


def init() -> None:
    """Allocates the pos0 staging scalar (required before any graph capture)."""
    _check(load_library().rpg_ops_init())


def set_stream(stream) -> None:
    """Routes launches to `stream` (torch.cuda.Stream, raw hipStream_t int, or None)."""
    handle = getattr(stream, "cuda_stream", stream)
    _check(load_library().rpg_ops_set_stream(handle or None))


def get_stream() -> int:
    return load_library().rpg_ops_get_stream() or 0


class ScopedEngineStream:
    """Context manager mirroring ScopedEngineStream (src/cuda_common.h:128-137)."""

    def __init__(self, stream):
        self._stream = stream
        self._prev = None

    def __enter__(self):
        self._prev = get_stream()
        set_stream(self._stream)
        return self

    def __exit__(self, *exc):
        set_stream(self._prev)
        return False


def stage_pos0(pos: int) -> None:
    _check(load_library().rpg_ops_stage_pos0(int(pos)))


def pos_staging_ptr() -> int:
    """Device address of the pos0 staging scalar (reference PosStagingPtr, src/cuda_common.h:153)."""
    p = load_library().rpg_ops_pos_staging_ptr()
    if not p:
        _check(-1)
    return p


def device_info() -> tuple[bool, str]:
    buf = ctypes.create_string_buffer(512)
    rc = _check(load_library().rpg_ops_device_info(buf, 512))
    return rc == 1, buf.value.decode()


def type_row_bytes(ggml_type: int, n_elems: int) -> int:
    return _check(load_library().rpg_ops_type_row_bytes(ggml_type, n_elems))


def build_rope_table(head_dim: int, theta: float, n_pos: int):
    """Host RoPE table as a numpy float32 array [n_pos, head_dim]."""
    import numpy as np

    out = np.empty((n_pos, head_dim), dtype=np.float32)
    _check(load_library().rpg_ops_build_rope_table(head_dim, float(theta), n_pos,
                                                   out.ctypes.data_as(ctypes.c_void_p)))
    return out


class GpuTensor:
    """Raw GGUF bytes of a weight tensor resident on the GPU (src/gpu_model.h:42-55)."""

    def __init__(self, data, ggml_type: int, rows: int, cols: int):
        self.buf = data
        self.type = int(ggml_type)
        self.rows = int(rows)
        self.cols = int(cols)
        self.matrix = True
        self.n_elements = self.rows * self.cols

    def row_bytes(self) -> int:
        return (self.cols // BLOCK_ELEMS[self.type]) * BLOCK_BYTES[self.type]


# ----------------------------------------------------------------------------- reference operators


def GpuDequantRow(ggml_type: int, src, n_elems: int, dst) -> None:
    torch = _t()
    nbytes = type_row_bytes(ggml_type, n_elems) if ggml_type in BLOCK_BYTES else 0
    _check(load_library().rpg_op_dequant_row(ggml_type, _addr(src, nbytes, name="src"), n_elems,
                                             _addr(dst, 4 * n_elems, torch.float32, "dst")))


def GpuRmsNorm(x, w, n_rows: int, n: int, stride: int, eps: float, out) -> None:
    torch = _t()
    span = 4 * ((n_rows - 1) * stride + n) if n_rows > 0 else 0
    _check(load_library().rpg_op_rms_norm(_addr(x, span, torch.float32, "x"), _addr(w, 4 * n, torch.float32, "w"),
                                          n_rows, n, stride, eps, _addr(out, span, torch.float32, "out")))


def GpuRope(x, n_heads: int, head_dim: int, rope_tab, pos0: int, n_rows: int) -> None:
    torch = _t()
    _check(load_library().rpg_op_rope(
        _addr(x, 4 * n_rows * n_heads * head_dim, torch.float32, "x"), n_heads, head_dim,
        _addr(rope_tab, 4 * (pos0 + n_rows) * head_dim, torch.float32, "rope_tab"), pos0, n_rows))


def GpuKvWrite(k, v, n_kv_heads: int, head_dim: int, pos0: int, seq: int, k_layer, v_layer, max_seq: int) -> None:
    torch = _t()
    src = 4 * seq * n_kv_heads * head_dim
    dst = 2 * n_kv_heads * max_seq * head_dim
    _check(load_library().rpg_op_kv_write(
        _addr(k, src, torch.float32, "k"), _addr(v, src, torch.float32, "v"), n_kv_heads, head_dim, pos0, seq,
        _addr(k_layer, dst, None, "k_layer"), _addr(v_layer, dst, None, "v_layer"), max_seq))


def GpuSiluMulInPlace(gate, up, n: int) -> None:
    torch = _t()
    nb = 4 * max(n, 0)
    _check(load_library().rpg_op_silu_mul_inplace(_addr(gate, nb, torch.float32, "gate"),
                                                  _addr(up, nb, torch.float32, "up"), n))


def GpuVecAddInPlace(a, b, n: int) -> None:
    torch = _t()
    nb = 4 * max(n, 0)
    _check(load_library().rpg_op_vec_add_inplace(_addr(a, nb, torch.float32, "a"), _addr(b, nb, torch.float32, "b"),
                                                 n))


def GpuEmbeddingLookup(emb: GpuTensor, toks, seq: int, x) -> None:
    torch = _t()
    _check(load_library().rpg_op_embedding_lookup(
        emb.type, _addr(emb.buf, emb.rows * emb.row_bytes(), name="emb"), emb.rows, emb.cols,
        _addr(toks, 4 * seq, torch.int32, "toks"), seq, _addr(x, 4 * seq * emb.cols, torch.float32, "x")))


def GpuSetForceGenericMatMul(force: bool) -> None:
    """Routes every matmul to the generic kernel (reference GpuSetForceGenericMatMul,
    src/kernels_gpu.h:57); verification only."""
    _check(load_library().rpg_op_set_force_generic_matmul(1 if force else 0))


def GpuForceGenericMatMul() -> bool:
    return load_library().rpg_op_force_generic_matmul() == 1


def GpuMatMulQuant(w: GpuTensor, x, n_tokens: int, out) -> None:
    """OUT[n_tokens, rows] = X[n_tokens, cols] . W^T (reference GpuMatMulQuant, src/kernels_gpu.h:42-49)."""
    torch = _t()
    _check(load_library().rpg_op_matmul_quant(
        w.type, _addr(w.buf, w.rows * w.row_bytes(), name="w"), w.rows, w.cols,
        _addr(x, 4 * n_tokens * w.cols, torch.float32, "x"), n_tokens,
        _addr(out, 4 * n_tokens * w.rows, torch.float32, "out")))


def GpuMatMulQuantSwiGLU(w_gate: GpuTensor, w_up: GpuTensor, x, n_tokens: int, gate, up) -> None:
    """gate <- silu(x . W_gate^T) * (x . W_up^T), up is scratch (the layer's gate / up + SwiGLU; no reference
    counterpart). Bit-identical to GpuMatMulQuantGroup + GpuSiluMulInPlace."""
    torch = _t()
    if (w_gate.type, w_gate.rows, w_gate.cols) != (w_up.type, w_up.rows, w_up.cols):
        raise RpgError("GpuMatMulQuantSwiGLU: gate and up must have the same type and shape")
    nbytes = w_gate.rows * w_gate.row_bytes()
    no = 4 * n_tokens * w_gate.rows
    _check(load_library().rpg_op_matmul_quant_swiglu(
        w_gate.type, _addr(w_gate.buf, nbytes, name="w_gate"), _addr(w_up.buf, nbytes, name="w_up"), w_gate.rows,
        w_gate.cols, _addr(x, 4 * n_tokens * w_gate.cols, torch.float32, "x"), n_tokens,
        _addr(gate, no, torch.float32, "gate"), _addr(up, no, torch.float32, "up")))


def GpuMatMulQuantGroup(ws: list, x, n_tokens: int, outs: list) -> None:
    """OUT_i = X . W_i^T for matrices sharing X (no reference counterpart): same-type runs fused at n = 1, one
    activation split for all matrices on the matrix-core path; outputs bit-identical to GpuMatMulQuant calls."""
    torch = _t()
    n = len(ws)
    if n == 0 or n != len(outs):
        raise RpgError("GpuMatMulQuantGroup needs one output per matrix and at least one matrix")
    cols = ws[0].cols
    if any(w.cols != cols for w in ws):
        raise RpgError(f"GpuMatMulQuantGroup matrices must share their width ({[w.cols for w in ws]})")
    types = (ctypes.c_uint32 * n)(*[w.type for w in ws])
    ptrs = (ctypes.c_void_p * n)(*[_addr(w.buf, w.rows * w.row_bytes(), name="w") for w in ws])
    rows = (ctypes.c_int64 * n)(*[w.rows for w in ws])
    optrs = (ctypes.c_void_p * n)(*[_addr(o, 4 * n_tokens * w.rows, torch.float32, "out") for o, w in zip(outs, ws)])
    _check(load_library().rpg_op_matmul_quant_group(n, types, ptrs, rows, cols,
                                                    _addr(x, 4 * n_tokens * cols, torch.float32, "x"), n_tokens,
                                                    optrs))


def GpuNormMatMulQuantGroup(x, d, norm_w, eps: float, x_out, ws: list, outs: list) -> bool:
    """One token: OUT_i = (RMSNorm(x + d) * norm_w) . W_i^T with the norm formed inside the matmul launches, and
    x_out <- x + d (no reference counterpart). Returns False, having launched nothing, when the group has no fused
    form (the caller then runs GpuAddRmsNorm + GpuMatMulQuantGroup)."""
    torch = _t()
    n = len(ws)
    if n == 0 or n != len(outs):
        raise RpgError("GpuNormMatMulQuantGroup needs one output per matrix and at least one matrix")
    cols = ws[0].cols
    if any(w.cols != cols for w in ws):
        raise RpgError(f"GpuNormMatMulQuantGroup matrices must share their width ({[w.cols for w in ws]})")
    types = (ctypes.c_uint32 * n)(*[w.type for w in ws])
    ptrs = (ctypes.c_void_p * n)(*[_addr(w.buf, w.rows * w.row_bytes(), name="w") for w in ws])
    rows = (ctypes.c_int64 * n)(*[w.rows for w in ws])
    optrs = (ctypes.c_void_p * n)(*[_addr(o, 4 * w.rows, torch.float32, "out") for o, w in zip(outs, ws)])
    fused = ctypes.c_int32(0)
    row = 4 * cols
    _check(load_library().rpg_op_norm_matmul_quant_group(
        n, types, ptrs, rows, cols, _addr(x, row, torch.float32, "x"), _addr(d, row, torch.float32, "d"),
        _addr(norm_w, row, torch.float32, "norm_w"), eps, _addr(x_out, row, torch.float32, "x_out"), optrs,
        ctypes.byref(fused)))
    return bool(fused.value)


def GpuNormMatMulQuantSwiGLU(x, d, norm_w, eps: float, x_out, w_gate: GpuTensor, w_up: GpuTensor, gate, up) -> bool:
    """GpuNormMatMulQuantGroup in front of GpuMatMulQuantSwiGLU (one token; no reference counterpart)."""
    torch = _t()
    if (w_gate.type, w_gate.rows, w_gate.cols) != (w_up.type, w_up.rows, w_up.cols):
        raise RpgError("GpuNormMatMulQuantSwiGLU: gate and up must have the same type and shape")
    nbytes = w_gate.rows * w_gate.row_bytes()
    row = 4 * w_gate.cols
    fused = ctypes.c_int32(0)
    _check(load_library().rpg_op_norm_matmul_quant_swiglu(
        w_gate.type, _addr(w_gate.buf, nbytes, name="w_gate"), _addr(w_up.buf, nbytes, name="w_up"), w_gate.rows,
        w_gate.cols, _addr(x, row, torch.float32, "x"), _addr(d, row, torch.float32, "d"),
        _addr(norm_w, row, torch.float32, "norm_w"), eps, _addr(x_out, row, torch.float32, "x_out"),
        _addr(gate, 4 * w_gate.rows, torch.float32, "gate"), _addr(up, 4 * w_gate.rows, torch.float32, "up"),
        ctypes.byref(fused)))
    return bool(fused.value)


def GpuAttentionFromCache(n_heads: int, n_kv_heads: int, head_dim: int, pos0: int, q, seq: int, k_layer, v_layer,
                          max_seq: int, out, sh_positions: int = -1) -> None:
    """Causal attention over one fp16 cache layer (reference GpuAttentionFromCache,
    src/kernels_gpu.h:113-116, with ModelMeta flattened to the head counts)."""
    torch = _t()
    span = 4 * seq * n_heads * head_dim
    cache = 2 * n_kv_heads * max_seq * head_dim
    _check(load_library().rpg_op_attention_from_cache(
        _addr(q, span, torch.float32, "q"), n_heads, n_kv_heads, head_dim, pos0, seq,
        _addr(k_layer, cache, name="k_layer"), _addr(v_layer, cache, name="v_layer"), max_seq,
        _addr(out, span, torch.float32, "out"), sh_positions))


def GpuQkNormRopeKvAttention(n_heads: int, n_kv_heads: int, head_dim: int, pos0: int, q, k, v, q_norm, k_norm,
                             rope_tab, rope_rows: int, eps: float, k_layer, v_layer, max_seq: int, out,
                             sh_positions: int = -1) -> bool:
    """One token: GpuQkNormRopeKv + GpuAttentionFromCache in one decode launch (no reference counterpart); q, k, v
    are the raw projections and stay unchanged. Returns False, having launched nothing, when the shape has no
    fused kernel."""
    torch = _t()
    cache = 2 * n_kv_heads * max_seq * head_dim
    fused = ctypes.c_int32(0)
    _check(load_library().rpg_op_qk_norm_rope_kv_attention(
        _addr(q, 4 * n_heads * head_dim, torch.float32, "q"), _addr(k, 4 * n_kv_heads * head_dim, torch.float32, "k"),
        _addr(v, 4 * n_kv_heads * head_dim, torch.float32, "v"), _addr(q_norm, 4 * head_dim, torch.float32, "q_norm"),
        _addr(k_norm, 4 * head_dim, torch.float32, "k_norm"), n_heads, n_kv_heads, head_dim,
        _addr(rope_tab, 4 * rope_rows * head_dim, torch.float32, "rope_tab"), rope_rows, pos0, eps,
        _addr(k_layer, cache, name="k_layer"), _addr(v_layer, cache, name="v_layer"), max_seq,
        _addr(out, 4 * n_heads * head_dim, torch.float32, "out"), sh_positions, ctypes.byref(fused)))
    return bool(fused.value)


def GpuAttentionWarmupShmem(sh_positions: int) -> None:
    _check(load_library().rpg_op_attention_warmup(sh_positions))


# ----------------------------------------------------------------------------- GGUF and the device model


class ModelMetaC(ctypes.Structure):
    """rpg_model_meta_t (ModelMeta, reference src/model_meta.h:27-65)."""
    _fields_ = [("arch", ctypes.c_char * 32), ("name", ctypes.c_char * 128), ("n_layers", _i32), ("hidden", _i32),
                ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32), ("value_dim", _i32),
                ("intermediate", _i32), ("vocab", _i32), ("context_length", _i32), ("rope_theta", _f32),
                ("rms_eps", _f32), ("tied_embeddings", _i32), ("bos_id", _i32), ("eos_id", _i32), ("pad_id", _i32),
                ("add_bos", _i32), ("weight_bytes", _i64)]

    def as_dict(self) -> dict:
        d = {k: getattr(self, k) for k, _ in self._fields_}
        d["arch"] = self.arch.decode()
        d["name"] = self.name.decode()
        d["tied_embeddings"] = bool(self.tied_embeddings)
        d["add_bos"] = bool(self.add_bos)
        return d


class TensorInfoC(ctypes.Structure):
    """rpg_tensor_info_t."""
    _fields_ = [("data", _vp), ("type", _u32), ("n_dims", _i32), ("dims", _i64 * 4), ("n_elements", _i64),
                ("n_bytes", _i64), ("file_offset", _i64)]

    def as_dict(self) -> dict:
        return {"data": self.data or 0, "type": int(self.type), "dims": [int(self.dims[i]) for i in range(self.n_dims)],
                "n_elements": int(self.n_elements), "n_bytes": int(self.n_bytes), "file_offset": int(self.file_offset)}


class GgufFile:
    """A parsed GGUF file (reference GgufFile, src/gguf.h:43-97); host only."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        _check(load_library().rpg_gguf_open(os.fsencode(path), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if self._h:
            load_library().rpg_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self) -> list:
        lib = load_library()
        n = lib.rpg_gguf_tensor_count(self._h)
        if n < 0:
            _check(-1)
        out = []
        name = ctypes.create_string_buffer(512)
        info = TensorInfoC()
        for i in range(n):
            _check(lib.rpg_gguf_tensor_info(self._h, i, name, 512, ctypes.byref(info)))
            d = info.as_dict()
            d["name"] = name.value.decode()
            out.append(d)
        return out

    def meta(self, key: str, item: int = -1):
        """None (absent), float, bool, str, or ("array", n_items)."""
        lib = load_library()
        kind, num, n_items = ctypes.c_int32(), ctypes.c_double(), ctypes.c_int64()
        buf = ctypes.create_string_buffer(256)
        n = _check(lib.rpg_gguf_meta(self._h, key.encode(), item, ctypes.byref(kind), ctypes.byref(num), buf, 256,
                                     ctypes.byref(n_items)))
        if kind.value == 3 and n >= 256:
            buf = ctypes.create_string_buffer(n + 1)
            _check(lib.rpg_gguf_meta(self._h, key.encode(), item, ctypes.byref(kind), ctypes.byref(num), buf, n + 1,
                                     ctypes.byref(n_items)))
        return {0: lambda: None, 1: lambda: num.value, 2: lambda: bool(num.value),
                3: lambda: buf.raw[:n].decode("utf-8", "replace"), 4: lambda: ("array", n_items.value)}[kind.value]()

    def model_meta(self) -> dict:
        m = ModelMetaC()
        _check(load_library().rpg_gguf_model_meta(self._h, ctypes.byref(m)))
        return m.as_dict()

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(1024)
        _check(load_library().rpg_gguf_describe(self._h, buf, 1024))
        return buf.value.decode()


class GpuModel:
    """A qwen3 GGUF on the device (reference GpuModel::Load, src/gpu_model.cu:148-246)."""

    def __init__(self, path: str, max_pos: int = 4096):
        h = ctypes.c_void_p()
        _check(load_library().rpg_model_load(os.fsencode(path), max_pos, ctypes.byref(h)))
        self._h = h

    def free(self) -> None:
        if self._h:
            load_library().rpg_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def meta(self) -> dict:
        m = ModelMetaC()
        _check(load_library().rpg_model_meta(self._h, ctypes.byref(m)))
        return m.as_dict()

    def tensor(self, name: str) -> dict:
        info = TensorInfoC()
        _check(load_library().rpg_model_tensor(self._h, name.encode(), ctypes.byref(info)))
        return info.as_dict()

    def gpu_tensor(self, name: str) -> "GpuTensor":
        """A GpuTensor view (for GpuMatMulQuant / GpuEmbeddingLookup) of a loaded matrix."""
        t = self.tensor(name)
        return GpuTensor(t["data"], t["type"], t["dims"][1], t["dims"][0])

    def rope(self):
        tab, n = ctypes.c_void_p(), ctypes.c_int64()
        _check(load_library().rpg_model_rope(self._h, ctypes.byref(tab), ctypes.byref(n)))
        return tab.value, n.value

    def describe(self) -> str:
        buf = ctypes.create_string_buffer(2048)
        _check(load_library().rpg_model_describe(self._h, buf, 2048))
        return buf.value.decode()

    def upload_stats(self) -> dict:
        b, p, u = ctypes.c_int64(), ctypes.c_double(), ctypes.c_double()
        _check(load_library().rpg_model_upload_stats(self._h, ctypes.byref(b), ctypes.byref(p), ctypes.byref(u)))
        return {"bytes": b.value, "parse_seconds": p.value, "upload_seconds": u.value}


# ----------------------------------------------------------------------------- forward and generation


class _Handle:
    _free_fn = ""

    def free(self) -> None:
        if getattr(self, "_h", None):
            getattr(load_library(), self._free_fn)(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GpuKvCache(_Handle):
    """fp16 KV cache of a model, allocated in full (reference GpuKvCache, src/kv_cache_gpu.h:50-100)."""
    _free_fn = "rpg_kv_free"

    def __init__(self, model: GpuModel, max_seq: int):
        h = ctypes.c_void_p()
        _check(load_library().rpg_kv_create(model._h, max_seq, ctypes.byref(h)))
        self._h = h

    def _info(self):
        n, cap, b = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        _check(load_library().rpg_kv_info(self._h, ctypes.byref(n), ctypes.byref(cap), ctypes.byref(b)))
        return n.value, cap.value, b.value

    def len(self) -> int:
        return self._info()[0]

    def max_seq(self) -> int:
        return self._info()[1]

    def bytes(self) -> int:
        return self._info()[2]

    def set_len(self, n: int) -> None:
        _check(load_library().rpg_kv_set_len(self._h, n))

    def reset(self) -> None:
        self.set_len(0)

    def layer(self, layer: int):
        """(k, v) device addresses of one layer ([n_kv_heads][max_seq][head_dim] fp16)."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        _check(load_library().rpg_kv_layer(self._h, layer, ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value


class GpuScratch(_Handle):
    """Grow-only forward activations and the decode graph (reference GpuScratch, src/qwen3_gpu.h:47-113)."""
    _free_fn = "rpg_scratch_free"

    def __init__(self):
        h = ctypes.c_void_p()
        _check(load_library().rpg_scratch_create(ctypes.byref(h)))
        self._h = h

    def logits_dev(self) -> int:
        """Device address of the logits [seq, vocab] of the last forward."""
        p = ctypes.c_void_p()
        _check(load_library().rpg_scratch_logits(self._h, ctypes.byref(p), None))
        return p.value

    def token_dev(self) -> int:
        """Device address of the sampled-token slot (int32)."""
        p = ctypes.c_void_p()
        _check(load_library().rpg_scratch_logits(self._h, None, ctypes.byref(p)))
        return p.value


def GpuForwardFull(m: GpuModel, tokens, s: GpuScratch, want_logits: bool = True, layer_limit: int = 0,
                   capture_hidden: bool = False, kv: Optional[GpuKvCache] = None):
    """Forward of host token ids (reference GpuForwardFull, src/qwen3_gpu.h:136-139).
    Returns (logits [seq, vocab] or None, hidden [n_use + 1, seq, hidden] or None) as numpy float32."""
    import numpy as np

    toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
    seq = int(toks.size)
    meta = m.meta()
    n_use = layer_limit if 0 < layer_limit < meta["n_layers"] else meta["n_layers"]
    logits = np.empty((seq, meta["vocab"]), np.float32) if want_logits and seq > 0 else None
    hidden = np.empty((n_use + 1, seq, meta["hidden"]), np.float32) if capture_hidden and seq > 0 else None
    _check(load_library().rpg_forward_full(
        m._h, toks.ctypes.data_as(ctypes.c_void_p), seq, s._h,
        logits.ctypes.data_as(ctypes.c_void_p) if logits is not None else None, layer_limit,
        hidden.ctypes.data_as(ctypes.c_void_p) if hidden is not None else None, kv._h if kv is not None else None))
    return logits, hidden


def GpuForwardStep(m: GpuModel, token: int, pos: int, kv: GpuKvCache, s: GpuScratch, want_logits: bool = True):
    """One token at pos == kv.len() (reference GpuForwardStep, src/qwen3_gpu.h:145-146)."""
    import numpy as np

    logits = np.empty(m.meta()["vocab"], np.float32) if want_logits else None
    _check(load_library().rpg_forward_step(m._h, int(token), pos, kv._h, s._h,
                                           logits.ctypes.data_as(ctypes.c_void_p) if logits is not None else None))
    return logits


def GpuForwardStepDev(m: GpuModel, token_dev, pos: int, kv: GpuKvCache, s: GpuScratch) -> None:
    """One token whose id is on the device (reference GpuForwardStepDev, src/qwen3_gpu.h:151-152)."""
    torch = _t()
    _check(load_library().rpg_forward_step_dev(m._h, _addr(token_dev, 4, torch.int32, "token_dev"), pos, kv._h,
                                               s._h))


class GenerateOptsC(ctypes.Structure):
    _fields_ = [("max_tokens", ctypes.c_int32), ("stop_ids", ctypes.c_void_p), ("n_stop", ctypes.c_int32),
                ("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("top_p", ctypes.c_float),
                ("seed", ctypes.c_uint64), ("use_graph", ctypes.c_int32), ("step_logits", ctypes.c_void_p),
                ("step_logits_cap", ctypes.c_int64)]


class GpuGenerateOptions:
    """Reference GpuGenerateOptions (src/qwen3_gpu.h:156-181): temperature 0 is greedy."""

    def __init__(self, max_tokens: int = 64, stop_ids=(), sample: Optional["SampleOptions"] = None, seed: int = 0,
                 step_logits: bool = False, use_graph: bool = False):
        self.max_tokens = int(max_tokens)
        self.stop_ids = [int(x) for x in stop_ids]
        self.sample = sample if sample is not None else SampleOptions(temperature=0.0)
        self.seed = int(seed)
        self.step_logits = bool(step_logits)
        self.use_graph = bool(use_graph)


def GpuGenerate(m: GpuModel, kv: GpuKvCache, s: GpuScratch, first_logits_dev, opt: GpuGenerateOptions):
    """Generates from the distribution at first_logits_dev (reference GpuGenerate,
    src/qwen3_gpu.h:197-199). Returns (ids, step_logits [n, vocab] or None)."""
    import numpy as np

    torch = _t()
    vocab = m.meta()["vocab"]
    stops = np.asarray(opt.stop_ids, dtype=np.int32)
    out = np.empty(max(opt.max_tokens, 1), np.int32)
    steps = np.empty((max(opt.max_tokens, 1), vocab), np.float32) if opt.step_logits else None
    c = GenerateOptsC(opt.max_tokens, stops.ctypes.data if stops.size else None, int(stops.size),
                       opt.sample.temperature, opt.sample.top_k, opt.sample.top_p, opt.seed & (2 ** 64 - 1),
                       int(opt.use_graph), steps.ctypes.data if steps is not None else None,
                       steps.size if steps is not None else 0)
    n = ctypes.c_int32()
    _check(load_library().rpg_generate(m._h, kv._h, s._h, _addr(first_logits_dev, 4 * vocab, torch.float32,
                                                                 "first_logits"),
                                       ctypes.byref(c), out.ctypes.data_as(ctypes.c_void_p), out.size,
                                       ctypes.byref(n)))
    ids = out[:n.value].tolist()
    return ids, (steps[:n.value].copy() if steps is not None else None)


def GpuGenerateGreedy(m: GpuModel, kv: GpuKvCache, s: GpuScratch, first_logits_dev, opt: GpuGenerateOptions):
    """GpuGenerate with temperature 0 (reference src/qwen3_gpu.h:207-210)."""
    g = GpuGenerateOptions(opt.max_tokens, opt.stop_ids, SampleOptions(0.0, opt.sample.top_k, opt.sample.top_p),
                           opt.seed, opt.step_logits, opt.use_graph)
    return GpuGenerate(m, kv, s, first_logits_dev, g)


# ----------------------------------------------------------------------------- argmax and sampling


class SampleOptions:
    """Sampling parameters (reference SampleOptions, src/sampler.h:35-46)."""

    def __init__(self, temperature: float = 1.0, top_k: int = 0, top_p: float = 1.0):
        self.temperature = float(temperature)
        self.top_k = int(top_k)
        self.top_p = float(top_p)


def GpuArgMax(x, n: int, out_idx) -> None:
    """out_idx[0] = first index of the largest x[i] above -FLT_MAX (reference GpuArgMax, src/kernels_gpu.h:131-143)."""
    torch = _t()
    _check(load_library().rpg_op_argmax(_addr(x, 4 * n, torch.float32, "x"), n,
                                        _addr(out_idx, 4, torch.int32, "out_idx")))


def DevSplitMix64(x: int) -> int:
    return int(load_library().rpg_sample_split_mix64(x))


def DevCounterRng(seed: int, counter: int) -> int:
    return int(load_library().rpg_sample_counter_rng(seed, counter))


def DevCounterUniform(seed: int, counter: int) -> float:
    return float(load_library().rpg_sample_counter_uniform(seed, counter))


def GpuFilterToProbs(logits, n: int, opt: SampleOptions, probs) -> None:
    """Filtered, normalised distribution (reference GpuFilterToProbs, src/sampler_gpu.h:86-87)."""
    torch = _t()
    _check(load_library().rpg_op_filter_to_probs(
        _addr(logits, 4 * n, torch.float32, "logits"), n, opt.temperature, opt.top_k, opt.top_p,
        _addr(probs, 4 * n, torch.float32, "probs")))


def GpuInverseSample(probs, n: int, u: float, out_idx) -> None:
    """Inverse transform at a host u (reference GpuInverseSample, src/sampler_gpu.h:95-96)."""
    torch = _t()
    _check(load_library().rpg_op_inverse_sample(_addr(probs, 4 * n, torch.float32, "probs"), n, u,
                                                _addr(out_idx, 4, torch.int32, "out_idx")))


def GpuSampleToken(logits, n: int, opt: SampleOptions, seed: int, counter: int, probs, out_idx) -> None:
    """One token (reference GpuSampleToken, src/sampler_gpu.h:108-110)."""
    torch = _t()
    _check(load_library().rpg_op_sample_token(
        _addr(logits, 4 * n, torch.float32, "logits"), n, opt.temperature, opt.top_k, opt.top_p, seed, counter,
        _addr(probs, 4 * n, torch.float32, "probs"), _addr(out_idx, 4, torch.int32, "out_idx")))


def GpuSampleTokenDev(logits, n: int, opt: SampleOptions, seed: int, counter_dev, probs, out_idx) -> None:
    """One token with the counter read on the device (reference GpuSampleTokenDev, src/sampler_gpu.h:124-126)."""
    torch = _t()
    _check(load_library().rpg_op_sample_token_dev(
        _addr(logits, 4 * n, torch.float32, "logits"), n, opt.temperature, opt.top_k, opt.top_p, seed,
        _addr(counter_dev, 8, name="counter_dev"), _addr(probs, 4 * n, torch.float32, "probs"),
        _addr(out_idx, 4, torch.int32, "out_idx")))


def GpuSamplerWarmup() -> None:
    _check(load_library().rpg_op_sampler_warmup())


# ----------------------------------------------------------------------------- fused operators


def GpuAddRmsNorm(x, d, w, n_rows: int, n: int, eps: float, out) -> None:
    torch = _t()
    span = 4 * n_rows * n
    _check(load_library().rpg_op_add_rms_norm(
        _addr(x, span, torch.float32, "x"), _addr(d, span, torch.float32, "d"), _addr(w, 4 * n, torch.float32, "w"),
        n_rows, n, eps, _addr(out, span, torch.float32, "out")))


def GpuQkNormRopeKv(q, k, v, q_norm, k_norm, n_heads: int, n_kv_heads: int, head_dim: int, rope_tab,
                    rope_rows: int, pos0: int, seq: int, eps: float, k_layer, v_layer, max_seq: int,
                    write_k_f32: bool = False) -> None:
    torch = _t()
    kvb = 4 * seq * n_kv_heads * head_dim
    cache = 2 * n_kv_heads * max_seq * head_dim
    _check(load_library().rpg_op_qk_norm_rope_kv(
        _addr(q, 4 * seq * n_heads * head_dim, torch.float32, "q"), _addr(k, kvb, torch.float32, "k"),
        _addr(v, kvb, torch.float32, "v"), _addr(q_norm, 4 * head_dim, torch.float32, "q_norm"),
        _addr(k_norm, 4 * head_dim, torch.float32, "k_norm"), n_heads, n_kv_heads, head_dim,
        _addr(rope_tab, 4 * rope_rows * head_dim, torch.float32, "rope_tab"), rope_rows, pos0, seq, eps,
        _addr(k_layer, cache, None, "k_layer"), _addr(v_layer, cache, None, "v_layer"), max_seq,
        1 if write_k_f32 else 0))


# ----------------------------------------------------------------------------- measurement


def GpuStreamCopy(src, dst, nbytes: int) -> None:
    _check(load_library().rpg_op_stream_copy(_addr(src, nbytes, name="src"), _addr(dst, nbytes, name="dst"), nbytes))


def GpuStreamFill(dst, nbytes: int, pattern: int) -> None:
    _check(load_library().rpg_op_stream_fill(_addr(dst, nbytes, name="dst"), nbytes, pattern & 0xFFFFFFFF))


def GpuStreamRead(src, nbytes: int, sink, key: int = 0x9E3779B9) -> None:
    """Reads nbytes of src and writes nothing (unless a thread's XOR fold equals key;
    then one word goes to sink, an int32 device tensor)."""
    torch = _t()
    _check(load_library().rpg_op_stream_read(_addr(src, nbytes, name="src"), nbytes, key & 0xFFFFFFFF,
                                             _addr(sink, 4, torch.int32, "sink")))


def profile_start(max_launches: int) -> None:
    """Times the next `max_launches` kernel launches with dispatch-attached HIP events."""
    _check(load_library().rpg_ops_profile_start(int(max_launches)))


def profile_stop() -> None:
    _check(load_library().rpg_ops_profile_stop())


def profile_report() -> dict:
    """Per-kernel {count, avg_us, min_us, max_us, total_us} of the profiled launches."""
    import json

    cap = 1 << 16
    while True:
        buf = ctypes.create_string_buffer(cap)
        n = _check(load_library().rpg_ops_profile_report(buf, cap))
        if n < cap:
            return json.loads(buf.value.decode())
        cap = n + 1


def GpuF16Sweep(out) -> None:
    torch = _t()
    _check(load_library().rpg_op_f16_sweep(_addr(out, 4 * 65536, torch.float32, "out")))
