"""GGUF -> device upload (rpg_model_*): every loaded tensor equals the file's bytes
(norms: fp32, quantized norms dequantized bit-exactly), the RoPE table equals
the oracle's, tied embeddings resolve to token_embd, the loaded tensors drive the
operators exactly as the same bytes uploaded by other means, and the loader
rejects what the reference rejects. Synthetic qwen3 GGUFs from
tests/gguf_writer.py."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import gguf_writer as W
from oracle import gguf_ref as R

pytestmark = pytest.mark.gpu


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


_HIP = None


def d2h(ptr: int, nbytes: int) -> bytes:
    """Device bytes at ptr (hipMemcpy device -> host)."""
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
        _HIP.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _HIP.hipDeviceSynchronize.restype = ctypes.c_int
    import torch

    torch.cuda.synchronize()
    buf = ctypes.create_string_buffer(nbytes)
    assert _HIP.hipMemcpy(buf, ctypes.c_void_p(ptr), nbytes, 2) == 0  # hipMemcpyDeviceToHost
    return buf.raw


def write(tmp_path, name, blob):
    p = tmp_path / name
    p.write_bytes(blob)
    return str(p)


@pytest.mark.parametrize("version,alignment,tied", [(3, 32, False), (2, 64, True), (1, 32, False)])
def test_loaded_tensors_equal_file_bytes(gpu, ora, tmp_path, version, alignment, tied):
    case(f"model upload v{version} align {alignment} tied={tied}")
    rng = np.random.default_rng(version * 10 + alignment)
    blob, tensors, _ = W.qwen3_model(rng, version=version, alignment=alignment, tied=tied)
    m = gpu.GpuModel(write(tmp_path, "m.gguf", blob), max_pos=512)
    meta = m.meta()
    want_meta = R.model_meta(R.read(blob))
    for k, v in want_meta.items():
        assert meta[k] == v, k
    for name, dims, t, raw in tensors:
        info = m.tensor(name)
        assert info["type"] == (t if len(dims) == 2 else 0)
        assert info["data"] % 256 == 0  # arena slices are 256-byte aligned
        got = d2h(info["data"], info["n_bytes"])
        if len(dims) == 2:
            assert info["dims"] == dims and got == raw, name
        else:
            assert np.array_equal(np.frombuffer(got, np.float32), np.frombuffer(raw, np.float32)), name
    if tied:
        assert m.tensor("output.weight")["data"] == m.tensor("token_embd.weight")["data"]
    tab, n_pos = m.rope()
    assert n_pos == 512
    want = ora.build_rope_table(128, float(np.float32(1e6)), n_pos)
    got = np.frombuffer(d2h(tab, n_pos * 128 * 4), np.float32).reshape(n_pos, 128)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    st = m.upload_stats()
    assert st["bytes"] == sum(len(r) for _, _, _, r in tensors) and st["upload_seconds"] > 0
    assert "device arena" in m.describe()
    m.free()


def test_quantized_norms_dequantized_on_device(gpu, ora, tmp_path):
    case("model upload with Q4_K / Q6_K norms")
    rng = np.random.default_rng(5)
    for nt in (W.GGML_Q4_K, W.GGML_Q6_K):
        blob, tensors, _ = W.qwen3_model(rng, norm_type=nt)
        m = gpu.GpuModel(write(tmp_path, f"n{nt}.gguf", blob))
        for name, dims, t, raw in tensors:
            if len(dims) == 1 and t == nt:
                want = ora.dequantize_row(nt, np.frombuffer(raw, np.uint8), dims[0])
                info = m.tensor(name)
                assert info["type"] == 0 and info["n_bytes"] == 4 * dims[0]
                got = np.frombuffer(d2h(info["data"], info["n_bytes"]), np.float32)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name
        m.free()


def test_rope_positions_capped_by_context(gpu, tmp_path):
    case("model rope cap")
    rng = np.random.default_rng(6)
    blob, _, _ = W.qwen3_model(rng, extra_kv=[("qwen3.context_length", W.U32, 100)])
    m = gpu.GpuModel(write(tmp_path, "c.gguf", blob), max_pos=4096)
    assert m.rope()[1] == 100 and m.meta()["context_length"] == 100
    m.free()


def test_loaded_tensors_drive_the_operators(gpu, ora, tmp_path):
    """The loaded embeddings and matrices through GpuEmbeddingLookup and
    GpuMatMulQuant: the gather is bit-exact against the oracle's dequant of the
    file bytes, the matmul bit-identical to the same bytes uploaded by torch."""
    import torch

    case("model tensors through the operators")
    rng = np.random.default_rng(7)
    blob, tensors, _ = W.qwen3_model(rng, vocab=3000)
    m = gpu.GpuModel(write(tmp_path, "e.gguf", blob))
    raw = {n: r for n, _, _, r in tensors}
    emb = m.gpu_tensor("token_embd.weight")
    ids = rng.integers(0, 3000, size=37).astype(np.int32)
    out = torch.empty((37, 256), dtype=torch.float32, device="cuda")
    gpu.GpuEmbeddingLookup(emb, torch.from_numpy(ids).cuda(), 37, out)
    want = ora.embedding_lookup(W.GGML_Q6_K, np.frombuffer(raw["token_embd.weight"], np.uint8), 3000, 256, ids)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    for name in ("blk.1.attn_q.weight", "blk.0.ffn_down.weight", "output.weight"):
        w = m.gpu_tensor(name)
        for n_tok in (1, 5, 40):
            x = torch.randn((n_tok, w.cols), device="cuda")
            a = torch.empty((n_tok, w.rows), device="cuda")
            b = torch.empty_like(a)
            gpu.GpuMatMulQuant(w, x, n_tok, a)
            same = torch.from_numpy(np.frombuffer(raw[name], np.uint8).copy()).cuda()
            gpu.GpuMatMulQuant(gpu.GpuTensor(same, w.type, w.rows, w.cols), x, n_tok, b)
            assert torch.equal(a, b), (name, n_tok)
    m.free()


def test_loader_rejections(gpu, tmp_path):
    case("model upload rejections")
    rng = np.random.default_rng(8)
    bad = {
        "implements only": W.qwen3_model(rng, override={"blk.1.attn_q.weight": W.GGML_Q8_0})[0],
        "wrong shape": W.qwen3_model(rng, extra_kv=[("qwen3.attention.head_count", W.U32, 4)])[0],
        "not found": W.qwen3_model(rng, drop=("blk.1.ffn_up.weight",))[0],
        "qwen3": W.build([("general.architecture", W.STR, "llama")], [("token_embd.weight", [4, 1], 0, bytes(16))]),
    }
    for i, (msg, blob) in enumerate(bad.items()):
        with pytest.raises(gpu.RpgError, match=msg):
            gpu.GpuModel(write(tmp_path, f"b{i}.gguf", blob))
    with pytest.raises(gpu.RpgError, match="no tensor"):
        blob, _, _ = W.qwen3_model(rng)
        m = gpu.GpuModel(write(tmp_path, "ok.gguf", blob))
        try:
            m.tensor("blk.9.attn_q.weight")
        finally:
            m.free()
