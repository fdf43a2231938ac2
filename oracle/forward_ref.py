"""float64 restatement of the reference's Qwen3 forward (the caller of the hot path).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the device
forward (rpg_forward_* / rpg_generate), never by the product.

Follows the reference's op order:
  * GpuForwardLayer, src/qwen3_gpu.cu:47-109: pre-norm (RMSNorm of x into h),
    q / k / v = h W^T; per-head RMSNorm of q and k BEFORE RoPE; NeoX RoPE on q
    and k (not v); with a cache, K/V stored as fp16 first and attention reading
    the whole cache (positions <= pos0 + t); x += attn W_o^T; h = RMSNorm(x);
    x += (silu(h W_gate^T) * (h W_up^T)) W_down^T;
  * ForwardCore, src/qwen3_gpu.cu:120-180: embedding without sqrt(hidden)
    scaling, the layers, output RMSNorm, lm_head (token_embd when tied);
  * attention maths, src/kernels_gpu.cu:737-823: s = q.k / sqrt(head_dim),
    softmax, sum p v, kv head = h / (n_heads / n_kv_heads).
Every number is float64 except what the device stores: the weights are the
exact fp32 values of the oracle's dequantisation (pinned against the golden
vectors), the RoPE table is the fp32 table of the oracle (src/gpu_model.cu:90-120),
and on the cache path K and V are rounded to fp16 (round to nearest even) as
they are written.

Pinned by tests/test_oracle_forward.py against an independent published
implementation of the architecture (transformers' Qwen3ForCausalLM in float64)
and by invariants: causality (a prefix's outputs do not depend on later
tokens), one-token attention (output = v), and cached decoding equal to the
cached prefill of the same tokens.
"""
from __future__ import annotations

import numpy as np

from oracle import pyoracle as ora


def _rms(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x [..., n] -> x / sqrt(mean(x^2) + eps) * w (src/kernels_gpu.cu:564-591)."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _rope(x: np.ndarray, tab: np.ndarray, pos: np.ndarray) -> np.ndarray:
    """NeoX rotation of x [seq, heads, d] at positions pos [seq] (src/kernels_gpu.cu:593-621):
    pairs (i, i + d/2), a' = a c - b s, b' = b c + a s."""
    half = x.shape[-1] // 2
    c = tab[pos, :half][:, None, :]
    s = tab[pos, half:][:, None, :]
    a, b = x[..., :half], x[..., half:]
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)


def _fp16(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float32).astype(np.float16).astype(np.float64)


class Qwen3Ref:
    """A qwen3 model from GGUF tensors [(name, dims, ggml_type, raw bytes)] and
    its metadata (oracle.gguf_ref.model_meta)."""

    def __init__(self, tensors, meta: dict, max_pos: int = 4096):
        self.c = meta
        self.w = {}
        for name, dims, t, raw in tensors:
            n = int(np.prod(dims))
            vals = ora.dequantize_row(t, np.frombuffer(raw, np.uint8), n).astype(np.float64)
            self.w[name] = vals.reshape(dims[::-1]) if len(dims) > 1 else vals
        if "output.weight" not in self.w:
            self.w["output.weight"] = self.w["token_embd.weight"]
        n_pos = max(1, min(max_pos, meta["context_length"] or max_pos))
        self.tab = ora.build_rope_table(meta["head_dim"], float(np.float32(meta["rope_theta"])),
                                        n_pos).astype(np.float64)
        self.eps = float(np.float32(meta["rms_eps"]))

    def new_cache(self, max_seq: int) -> dict:
        c = self.c
        shape = (c["n_layers"], c["n_kv_heads"], max_seq, c["head_dim"])
        return {"k": np.zeros(shape), "v": np.zeros(shape), "len": 0, "max_seq": max_seq}

    def _attention(self, q, keys, values, pos):
        """q [seq, Hq, d]; keys / values [Hkv, P, d]; token t sees keys 0..pos[t]."""
        c = self.c
        group = c["n_heads"] // c["n_kv_heads"]
        seq, hq, d = q.shape
        out = np.zeros_like(q)
        kh = np.arange(hq) // group
        for t in range(seq):
            k = keys[kh, : pos[t] + 1]            # [Hq, n, d]
            v = values[kh, : pos[t] + 1]
            s = np.einsum("hd,hnd->hn", q[t], k) / np.sqrt(d)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=1, keepdims=True)
            out[t] = np.einsum("hn,hnd->hd", p, v)
        return out

    def _qk(self, x, w, pos):
        """Per-head RMSNorm, then RoPE (src/qwen3_gpu.cu:77-83)."""
        return _rope(_rms(x, w, self.eps), self.tab, pos)

    def _mlp(self, h, p):
        """SwiGLU feed-forward (src/qwen3_gpu.cu:103-107; silu(v) = v / (1 + e^-v), src/kernels_gpu.cu:868)."""
        g = h @ self.w[p + "ffn_gate.weight"].T
        u = h @ self.w[p + "ffn_up.weight"].T
        return (g / (1.0 + np.exp(-g)) * u) @ self.w[p + "ffn_down.weight"].T

    def forward(self, tokens, cache: dict | None = None, layer_limit: int = 0):
        """(logits [seq, vocab] or None, hidden [n_use + 1, seq, hidden]) in float64;
        with a cache the segment is appended at cache['len']."""
        c, w = self.c, self.w
        tokens = np.asarray(tokens, dtype=np.int64)
        seq = tokens.size
        pos0 = cache["len"] if cache is not None else 0
        pos = pos0 + np.arange(seq)
        assert pos0 + seq <= self.tab.shape[0]
        hq, hkv, d = c["n_heads"], c["n_kv_heads"], c["head_dim"]
        n_use = layer_limit if 0 < layer_limit < c["n_layers"] else c["n_layers"]
        x = w["token_embd.weight"][tokens].copy()
        hidden = [x.copy()]
        for layer in range(n_use):
            p = f"blk.{layer}."
            h = _rms(x, w[p + "attn_norm.weight"], self.eps)
            q = (h @ w[p + "attn_q.weight"].T).reshape(seq, hq, d)
            k = (h @ w[p + "attn_k.weight"].T).reshape(seq, hkv, d)
            v = (h @ w[p + "attn_v.weight"].T).reshape(seq, hkv, d)
            q = self._qk(q, w[p + "attn_q_norm.weight"], pos)
            k = self._qk(k, w[p + "attn_k_norm.weight"], pos)
            if cache is not None:
                assert pos0 + seq <= cache["max_seq"]
                cache["k"][layer][:, pos0:pos0 + seq] = _fp16(k).transpose(1, 0, 2)
                cache["v"][layer][:, pos0:pos0 + seq] = _fp16(v).transpose(1, 0, 2)
                a = self._attention(q, cache["k"][layer], cache["v"][layer], pos)
            else:
                a = self._attention(q, k.transpose(1, 0, 2), v.transpose(1, 0, 2), pos)
            x = x + a.reshape(seq, hq * d) @ w[p + "attn_output.weight"].T
            x = x + self._mlp(_rms(x, w[p + "ffn_norm.weight"], self.eps), p)
            hidden.append(x.copy())
        if cache is not None:
            cache["len"] = pos0 + seq
        if n_use < c["n_layers"]:
            return None, np.stack(hidden)
        logits = _rms(x, w["output_norm.weight"], self.eps) @ w["output.weight"].T
        return logits, np.stack(hidden)


# Relative-error statistic of the reference's whole-layer comparison
# (tests/cmp_layers.py:35-46): elements with |ref| > REL_FLOOR, quantiles of |d| / |ref|.
REL_FLOOR = 1e-3


def rel_stats(ours: np.ndarray, ref: np.ndarray):
    """(median, p99, max) relative error and max |difference|."""
    d = np.abs(np.asarray(ours, np.float64) - np.asarray(ref, np.float64))
    a = np.abs(np.asarray(ref, np.float64))
    m = a > REL_FLOOR
    if not m.any():
        return 0.0, 0.0, 0.0, float(d.max())
    rel = d[m] / a[m]
    return float(np.median(rel)), float(np.percentile(rel, 99)), float(rel.max()), float(d.max())


def full_scale_rel(ours: np.ndarray, ref: np.ndarray) -> float:
    """max |ours - ref| / max |ref|: the criterion of the reference's KV self-check
    (cache vs no-cache logits, bar 1e-3; tools/gen_check.cu:224-246), where fp16
    K/V make per-element relative errors meaningless for small logits."""
    d = np.abs(np.asarray(ours, np.float64) - np.asarray(ref, np.float64))
    return float(d.max() / np.abs(np.asarray(ref, np.float64)).max())
