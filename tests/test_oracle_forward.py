"""Pins the float64 forward oracle (oracle/forward_ref.py) that the device forward
is checked against.

  * against an independent published implementation of the architecture:
    transformers' Qwen3ForCausalLM in float64, loaded with the same dequantised
    weights (its RMSNorm and RoPE angles run in fp32, hence the 1e-4 bar);
  * mistakes planted in the oracle (GQA head mapping, RoPE pairing, q/k norm
    after RoPE, no 1/sqrt(d) score scale, ReLU for SiLU) must fail that comparison;
  * invariants: causality, cached prefill in pieces == cached prefill whole,
    and the cache path differs from the no-cache path only by fp16 rounding
    (the reference's self-check bar: max |d| <= 1e-3 max |logits|, same argmax).
CPU only.
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_writer as W
from oracle import forward_ref as F
from oracle import gguf_ref as R

SHAPES = [dict(n_heads=2, n_kv_heads=1), dict(n_heads=4, n_kv_heads=2), dict(n_heads=2, n_kv_heads=2)]


def tiny(seed, tied=False, n_layers=2, **shape):
    rng = np.random.default_rng(seed)
    kw = dict(n_layers=n_layers, hidden=256, inter=512, vocab=1000, tied=tied, model_like=True)
    kw.update(shape)
    blob, tensors, _ = W.qwen3_model(rng, **kw)
    meta = R.model_meta(R.read(blob))
    return F.Qwen3Ref(tensors, meta, max_pos=128), rng


def hf_forward(ref: F.Qwen3Ref, toks):
    """transformers Qwen3ForCausalLM (float64, eager attention) with the oracle's weights."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    c, w = ref.c, ref.w
    cfg = tr.Qwen3Config(vocab_size=c["vocab"], hidden_size=c["hidden"], intermediate_size=c["intermediate"],
                         num_hidden_layers=c["n_layers"], num_attention_heads=c["n_heads"],
                         num_key_value_heads=c["n_kv_heads"], head_dim=c["head_dim"], rms_norm_eps=ref.eps,
                         tie_word_embeddings=bool(c["tied_embeddings"]),
                         rope_parameters={"rope_type": "default", "rope_theta": float(c["rope_theta"])},
                         max_position_embeddings=128, attention_bias=False)
    cfg._attn_implementation = "eager"
    m = tr.Qwen3ForCausalLM(cfg).to(torch.float64).eval()

    def t(a):
        return torch.from_numpy(np.ascontiguousarray(a))

    sd = {"model.embed_tokens.weight": t(w["token_embd.weight"]), "model.norm.weight": t(w["output_norm.weight"]),
          "lm_head.weight": t(w["output.weight"])}
    names = {"input_layernorm": "attn_norm", "post_attention_layernorm": "ffn_norm", "self_attn.q_proj": "attn_q",
             "self_attn.k_proj": "attn_k", "self_attn.v_proj": "attn_v", "self_attn.o_proj": "attn_output",
             "self_attn.q_norm": "attn_q_norm", "self_attn.k_norm": "attn_k_norm", "mlp.gate_proj": "ffn_gate",
             "mlp.up_proj": "ffn_up", "mlp.down_proj": "ffn_down"}
    for layer in range(c["n_layers"]):
        for hf, gg in names.items():
            sd[f"model.layers.{layer}.{hf}.weight"] = t(w[f"blk.{layer}.{gg}.weight"])
    m.load_state_dict(sd, strict=True)
    with torch.no_grad():
        out = m(input_ids=torch.from_numpy(np.asarray(toks, np.int64))[None], output_hidden_states=True)
    # hidden_states: the embedding, the output of every layer but the last, then norm(x_L)
    return out.logits[0].numpy(), [h[0].numpy() for h in out.hidden_states]


def compare_with_hf(ref, toks):
    logits, hidden = ref.forward(toks)
    hl, hh = hf_forward(ref, toks)
    stats = [F.rel_stats(hh[i], hidden[i])[1] for i in range(ref.c["n_layers"])]
    last = F._rms(hidden[-1], ref.w["output_norm.weight"], ref.eps)
    stats.append(F.rel_stats(hh[-1], last)[1])
    stats.append(F.rel_stats(hl, logits)[1])
    return max(stats)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"h{s['n_heads']}kv{s['n_kv_heads']}")
@pytest.mark.parametrize("tied", [False, True])
def test_oracle_matches_transformers_qwen3(shape, tied):
    ref, rng = tiny(3 + shape["n_heads"] + 7 * tied, tied=tied, **shape)
    toks = rng.integers(0, 1000, size=23)
    assert compare_with_hf(ref, toks) < 1e-4


def _interleaved_rope(x, tab, pos):
    # planted: pairs (2i, 2i + 1) instead of (i, i + d/2)
    half = x.shape[-1] // 2
    c = tab[pos, :half][:, None, :]
    s = tab[pos, half:][:, None, :]
    a, b = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = a * c - b * s
    out[..., 1::2] = b * c + a * s
    return out


@pytest.mark.parametrize("mistake", ["gqa", "rope_pairs", "norm_after_rope", "no_scale", "relu"])
def test_planted_mistakes_fail_the_transformers_pin(monkeypatch, mistake):
    ref, rng = tiny(41, n_heads=4, n_kv_heads=2)
    toks = rng.integers(0, 1000, size=23)
    attn, mlp = F.Qwen3Ref._attention, F.Qwen3Ref._mlp
    if mistake == "gqa":
        # query head h reads kv head h % 2 instead of h / 2 (heads 1 and 2 swap kv heads)
        monkeypatch.setattr(F.Qwen3Ref, "_attention",
                            lambda self, q, k, v, p: attn(self, q[:, [0, 2, 1, 3]], k, v, p)[:, [0, 2, 1, 3]])
    elif mistake == "rope_pairs":
        monkeypatch.setattr(F, "_rope", _interleaved_rope)
    elif mistake == "norm_after_rope":
        monkeypatch.setattr(F.Qwen3Ref, "_qk", lambda self, x, w, pos: F._rms(F._rope(x, self.tab, pos), w, self.eps))
    elif mistake == "no_scale":
        monkeypatch.setattr(F.Qwen3Ref, "_attention",
                            lambda self, q, k, v, p: attn(self, q * np.sqrt(q.shape[-1]), k, v, p))
    elif mistake == "relu":
        def relu_mlp(self, h, p):
            g = h @ self.w[p + "ffn_gate.weight"].T
            u = h @ self.w[p + "ffn_up.weight"].T
            return (np.maximum(g, 0.0) * u) @ self.w[p + "ffn_down.weight"].T
        monkeypatch.setattr(F.Qwen3Ref, "_mlp", relu_mlp)
    del mlp
    assert compare_with_hf(ref, toks) > 1e-2


def test_oracle_is_causal():
    ref, rng = tiny(5, n_heads=4, n_kv_heads=2)
    toks = rng.integers(0, 1000, size=20)
    lg, hid = ref.forward(toks)
    lg7, hid7 = ref.forward(toks[:7])
    np.testing.assert_allclose(lg7, lg[:7], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(hid7, hid[:, :7], rtol=1e-12, atol=1e-12)


def test_oracle_cache_pieces_equal_whole_and_differ_from_no_cache_by_fp16_only():
    ref, rng = tiny(6, n_heads=4, n_kv_heads=2)
    toks = rng.integers(0, 1000, size=24)
    whole = ref.new_cache(64)
    lg_w, hid_w = ref.forward(toks, cache=whole)
    parts = ref.new_cache(64)
    a, _ = ref.forward(toks[:10], cache=parts)
    b, _ = ref.forward(toks[10:17], cache=parts)
    rows = [a, b] + [ref.forward(toks[t:t + 1], cache=parts)[0] for t in range(17, 24)]
    np.testing.assert_allclose(np.concatenate(rows), lg_w, rtol=1e-10, atol=1e-10)
    assert whole["len"] == parts["len"] == 24
    np.testing.assert_array_equal(whole["k"][:, :, :24], parts["k"][:, :, :24])
    # the cache holds fp16 values, which the no-cache path does not round
    lg_n, hid_n = ref.forward(toks)
    fs = F.full_scale_rel(lg_w, lg_n)
    assert 0 < fs < 1e-3
    assert (lg_w.argmax(axis=1) == lg_n.argmax(axis=1)).all()
    k16 = whole["k"][:, :, :24]
    assert np.array_equal(k16, k16.astype(np.float16).astype(np.float64))


def test_rel_stats_matches_the_reference_statistic():
    # elements with |ref| <= 1e-3 are ignored; quantiles over |d| / |ref|
    ref = np.array([1.0, -2.0, 1e-4, 4.0])
    assert F.full_scale_rel(np.array([1.0, -2.0, 1e-4, 4.2]), ref) == pytest.approx(0.05)
    ours = np.array([1.1, -2.0, 5.0, 4.4])
    med, p99, mx, dmax = F.rel_stats(ours, ref)
    assert mx == pytest.approx(0.1) and med == pytest.approx(0.1) and dmax == pytest.approx(4.9999)
    assert p99 == pytest.approx(np.percentile([0.1, 0.0, 0.1], 99))
