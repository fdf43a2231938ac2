"""The device Qwen3 forward and generation (rpg_forward_* / rpg_generate) against
the float64 forward oracle (oracle/forward_ref.py, pinned against transformers'
Qwen3ForCausalLM in test_oracle_forward.py), with the reference's own criteria:

  * whole-layer parity on the no-cache path: the residual stream after the
    embedding and after every layer, and the logits, p99 relative error <= 1e-3
    over |ref| > 1e-3 (tests/cmp_layers.py:35-46);
  * on the cache path K and V are fp16, and a value within an fp32 ulp of an fp16
    rounding boundary lands on either side depending on the last bits of the
    computation (the oracle's own cache and no-cache paths differ by p99 ~2e-2
    per element), so there the reference's fp16-KV criterion applies: max |d|
    <= 1e-3 max |ref| per layer and for the logits, and the same argmax;
  * KV self-check: cache path vs no-cache path on the same tokens, max |d| <=
    1e-3 max |logits| and the same argmax at every position
    (tools/gen_check.cu:216-278);
  * decoding: each step equals the cached prefill of the same tokens; greedy
    tokens are the oracle's argmax (teacher-forced), sampled tokens are the
    oracle sampler's draw from the step's distribution with counter = position;
    the HIP-graph decode loop returns the same tokens as the per-step loop,
    replay after replay, also after eager work and after the scratch grew.
Synthetic qwen3 GGUFs with zero-mean, trained-weight-sized Q4_K / Q6_K matrices.
"""
from __future__ import annotations

import numpy as np
import pytest

import gguf_writer as W
from oracle import forward_ref as F
from oracle import gguf_ref as R
from test_gpu_model import d2h

pytestmark = pytest.mark.gpu

CONFIGS = {
    # name: tests/gguf_writer.qwen3_model arguments
    "h256_g2": dict(n_layers=2, hidden=256, n_heads=2, n_kv_heads=1, inter=512, vocab=1000),
    "h512_g4_tied": dict(n_layers=2, hidden=512, n_heads=4, n_kv_heads=1, inter=1024, vocab=3000, tied=True),
    "h256_g3": dict(n_layers=2, hidden=256, n_heads=6, n_kv_heads=2, inter=512, vocab=1000),
    "qwen3_1_7b_2layers": dict(n_layers=2, hidden=2048, n_heads=16, n_kv_heads=8, inter=6144, vocab=4096),
    # rows of 10 blocks (the 4B hidden size): one-token steps take the unfused norm + matmul path
    "h2560_g4_1layer": dict(n_layers=1, hidden=2560, n_heads=16, n_kv_heads=4, inter=1024, vocab=1500),
}


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def models(gpu, tmp_path_factory):
    """name -> (device model, oracle model); built on first use."""
    cache = {}
    tmp = tmp_path_factory.mktemp("fwd")

    def get(name):
        if name not in cache:
            rng = np.random.default_rng(sum(map(ord, name)))
            blob, tensors, _ = W.qwen3_model(rng, model_like=True, **CONFIGS[name])
            path = tmp / f"{name}.gguf"
            path.write_bytes(blob)
            meta = R.model_meta(R.read(blob))
            cache[name] = (gpu.GpuModel(str(path), max_pos=512), F.Qwen3Ref(tensors, meta, max_pos=512))
        return cache[name]

    yield get
    for m, _ in cache.values():
        m.free()


def tokens(name, n, seed=0):
    return np.random.default_rng(seed + n).integers(0, CONFIGS[name]["vocab"], size=n).astype(np.int32)


def assert_layers(name, hid_gpu, hid_ref, lg_gpu=None, lg_ref=None, bar=1e-3):
    worst = 0.0
    for i in range(hid_ref.shape[0]):
        med, p99, mx, _ = F.rel_stats(hid_gpu[i], hid_ref[i])
        worst = max(worst, p99)
        assert p99 <= bar, (name, "layer", i, med, p99, mx)
    if lg_ref is not None:
        med, p99, mx, _ = F.rel_stats(lg_gpu, lg_ref)
        worst = max(worst, p99)
        assert p99 <= bar, (name, "logits", med, p99, mx)
    print(f"  worst p99 {worst:.3g}", flush=True)


def assert_full_scale(name, hid_gpu, hid_ref, lg_gpu=None, lg_ref=None, bar=1e-3):
    """fp16-KV criterion (tools/gen_check.cu:224-246), per layer and for the logits."""
    worst = 0.0
    for i in range(hid_ref.shape[0]):
        fs = F.full_scale_rel(hid_gpu[i], hid_ref[i])
        worst = max(worst, fs)
        assert fs <= bar, (name, "layer", i, fs)
    if lg_ref is not None:
        fs = F.full_scale_rel(lg_gpu, lg_ref)
        worst = max(worst, fs)
        assert fs <= bar, (name, "logits", fs)
    print(f"  worst full-scale {worst:.3g}", flush=True)


def assert_argmax_or_tie(logits_gpu, logits_ref, tol=1e-3):
    """Same argmax per row, except where the oracle's top two are within tol * max|row|."""
    for r in range(logits_ref.shape[0]):
        g, o = int(np.argmax(logits_gpu[r])), int(np.argmax(logits_ref[r]))
        if g != o:
            row = logits_ref[r]
            assert row[o] - row[g] <= tol * np.abs(row).max(), (r, g, o, row[o] - row[g])


@pytest.mark.parametrize("name,seq", [("h256_g2", 1), ("h256_g2", 19), ("h256_g2", 80), ("h512_g4_tied", 37),
                                      ("h256_g3", 70), ("qwen3_1_7b_2layers", 80)])
@pytest.mark.parametrize("cached", [False, True])
def test_forward_matches_oracle(gpu, models, name, seq, cached):
    case(f"forward {name} seq {seq} cached={cached}")
    m, ref = models(name)
    toks = tokens(name, seq)
    s = gpu.GpuScratch()
    kv = gpu.GpuKvCache(m, 256) if cached else None
    lg, hid = gpu.GpuForwardFull(m, toks, s, capture_hidden=True, kv=kv)
    rc = ref.new_cache(256) if cached else None
    lg_r, hid_r = ref.forward(toks, cache=rc)
    if cached:
        assert_full_scale(name, hid, hid_r, lg, lg_r)
    else:
        assert_layers(name, hid, hid_r, lg, lg_r)
    assert_argmax_or_tie(lg, lg_r)
    if cached:
        assert kv.len() == seq
        kv.free()
    s.free()


@pytest.mark.parametrize("name,seq", [("h256_g2", 33), ("h512_g4_tied", 90), ("h256_g3", 21),
                                      ("qwen3_1_7b_2layers", 70)])
def test_kv_self_check(gpu, models, name, seq):
    """The reference's self-check: cached forward vs no-cache forward of the same tokens."""
    case(f"kv self-check {name} seq {seq}")
    m, _ = models(name)
    toks = tokens(name, seq, seed=3)
    s = gpu.GpuScratch()
    plain, _ = gpu.GpuForwardFull(m, toks, s)
    kv = gpu.GpuKvCache(m, 128)
    cached, _ = gpu.GpuForwardFull(m, toks, s, kv=kv)
    fs = F.full_scale_rel(cached, plain)
    print(f"  full-scale {fs:.3g}", flush=True)
    assert 0 < fs <= 1e-3
    assert (cached.argmax(axis=1) == plain.argmax(axis=1)).all()
    kv.free()
    s.free()


@pytest.mark.parametrize("name", ["h256_g2", "h512_g4_tied", "h256_g3", "h2560_g4_1layer"])
def test_prefill_pieces_and_decode_steps_match_oracle(gpu, models, name):
    """Segments at pos0 > 0 (one of them >= 64 tokens, the matrix-core attention)
    and single-token steps, each against the oracle's cached forward."""
    import torch

    case(f"pieces + steps {name}")
    m, ref = models(name)
    toks = tokens(name, 190, seed=5)
    s = gpu.GpuScratch()
    kv = gpu.GpuKvCache(m, 256)
    rc = ref.new_cache(256)
    rows_gpu, rows_ref = [], []
    for a, b in ((0, 11), (11, 100), (100, 187)):
        lg, _ = gpu.GpuForwardFull(m, toks[a:b], s, kv=kv)
        lr, _ = ref.forward(toks[a:b], cache=rc)
        rows_gpu.append(lg)
        rows_ref.append(lr)
    assert kv.len() == 187
    lg = gpu.GpuForwardStep(m, int(toks[187]), 187, kv, s)
    rows_gpu.append(lg[None])
    rows_ref.append(ref.forward(toks[187:188], cache=rc)[0])
    # the token id on the device (GpuForwardStepDev): logits stay in the scratch
    tok_dev = torch.tensor([int(toks[188])], dtype=torch.int32, device="cuda")
    gpu.GpuForwardStepDev(m, tok_dev, 188, kv, s)
    vocab = CONFIGS[name]["vocab"]
    rows_gpu.append(np.frombuffer(d2h(s.logits_dev(), 4 * vocab), np.float32)[None])
    rows_ref.append(ref.forward(toks[188:189], cache=rc)[0])
    assert kv.len() == 189
    lg_gpu, lg_ref = np.concatenate(rows_gpu), np.concatenate(rows_ref)
    fs = F.full_scale_rel(lg_gpu, lg_ref)
    print(f"  logits full-scale {fs:.3g}", flush=True)
    assert fs <= 1e-3
    assert_argmax_or_tie(lg_gpu, lg_ref)
    with pytest.raises(gpu.RpgError, match="end of the cache"):
        gpu.GpuForwardStep(m, 1, 200, kv, s)
    kv.free()
    s.free()


def test_layer_limit_and_errors(gpu, models):
    case("layer_limit / argument errors")
    m, ref = models("h256_g2")
    toks = tokens("h256_g2", 9)
    s = gpu.GpuScratch()
    lg, hid = gpu.GpuForwardFull(m, toks, s, want_logits=False, layer_limit=1, capture_hidden=True)
    assert lg is None and hid.shape == (2, 9, 256)
    _, hid_r = ref.forward(toks, layer_limit=1)
    assert_layers("h256_g2/limit1", hid, hid_r)
    with pytest.raises(gpu.RpgError, match="truncated"):
        gpu.GpuForwardFull(m, toks, s, layer_limit=1)
    with pytest.raises(gpu.RpgError, match="out of range"):
        gpu.GpuForwardFull(m, np.array([1, 1000], np.int32), s)
    with pytest.raises(gpu.RpgError, match="empty"):
        gpu.GpuForwardFull(m, np.array([], np.int32), s, want_logits=False)
    kv = gpu.GpuKvCache(m, 8)
    with pytest.raises(gpu.RpgError, match="capacity"):
        gpu.GpuForwardFull(m, tokens("h256_g2", 9), s, kv=kv)
    assert kv.len() == 0
    kv.free()
    s.free()


def prefill(gpu, m, toks, max_seq):
    s = gpu.GpuScratch()
    kv = gpu.GpuKvCache(m, max_seq)
    gpu.GpuForwardFull(m, toks, s, want_logits=False, kv=kv)
    vocab = m.meta()["vocab"]
    return s, kv, s.logits_dev() + 4 * vocab * (len(toks) - 1)


@pytest.mark.parametrize("name", ["h256_g2", "h256_g3"])
def test_greedy_generation(gpu, models, name):
    case(f"greedy generate {name}")
    m, ref = models(name)
    prompt = tokens(name, 15, seed=7)
    n_new = 12
    results = {}
    for use_graph in (False, True):
        s, kv, first = prefill(gpu, m, prompt, 64)
        ids, _ = gpu.GpuGenerate(m, kv, s, first, gpu.GpuGenerateOptions(max_tokens=n_new, use_graph=use_graph))
        assert len(ids) == n_new and kv.len() == 15 + n_new  # every returned token is in the cache
        results[use_graph] = ids
        kv.free()
        s.free()
    assert results[True] == results[False]
    # teacher-forced oracle: token i is the argmax of the row that produced it
    seq = np.concatenate([prompt, np.array(results[False][:-1], np.int32)])
    lg_r, _ = ref.forward(seq, cache=ref.new_cache(64))
    rows = lg_r[14:]
    for i, t in enumerate(results[False]):
        o = int(np.argmax(rows[i]))
        assert t == o or rows[i][o] - rows[i][t] <= 1e-3 * np.abs(rows[i]).max(), (i, t, o)


def test_sampled_generation_matches_oracle_sampler(gpu, models, ora):
    case("sampled generate h512_g4_tied")
    m, _ = models("h512_g4_tied")
    prompt = tokens("h512_g4_tied", 20, seed=9)
    opt = dict(max_tokens=10, sample=gpu.SampleOptions(0.8, 40, 0.9), seed=0x5EED2026)
    s, kv, first = prefill(gpu, m, prompt, 64)
    ids, steps = gpu.GpuGenerate(m, kv, s, first, gpu.GpuGenerateOptions(step_logits=True, **opt))
    assert steps.shape == (10, 3000)
    for i, t in enumerate(ids):  # counter = the absolute position the token is written at
        assert ora.sample_token(steps[i], 0.8, 40, 0.9, 0x5EED2026, 20 + i) == t, i
    kv.free()
    s.free()
    s, kv, first = prefill(gpu, m, prompt, 64)
    ids_g, _ = gpu.GpuGenerate(m, kv, s, first, gpu.GpuGenerateOptions(use_graph=True, **opt))
    assert ids_g == ids
    kv.free()
    s.free()


def test_stop_ids_and_full_context(gpu, models):
    case("generate stop ids / context full")
    m, _ = models("h256_g2")
    prompt = tokens("h256_g2", 10, seed=11)
    s, kv, first = prefill(gpu, m, prompt, 64)
    ids, _ = gpu.GpuGenerate(m, kv, s, first, gpu.GpuGenerateOptions(max_tokens=8))
    kv.free()
    s.free()
    for use_graph in (False, True):
        s, kv, first = prefill(gpu, m, prompt, 64)
        got, _ = gpu.GpuGenerate(m, kv, s, first,
                                 gpu.GpuGenerateOptions(max_tokens=8, stop_ids=[ids[3]], use_graph=use_graph))
        stop_at = ids.index(ids[3])
        assert got == ids[:stop_at + 1] and kv.len() == 10 + stop_at + 1
        kv.free()
        s.free()
        s, kv, first = prefill(gpu, m, prompt, 13)
        with pytest.raises(gpu.RpgError, match="KV cache has no free slot"):
            gpu.GpuGenerate(m, kv, s, first, gpu.GpuGenerateOptions(max_tokens=8, use_graph=use_graph))
        assert kv.len() == 13
        kv.free()
        s.free()


def test_graph_replays_after_eager_work_and_scratch_growth(gpu, models):
    """Two sessions run the same calls, one with the graph loop and one without:
    every token matches, across replays of one captured graph separated by eager
    steps, and after a longer prefill reallocated the scratch (the graph must be
    captured again, not replayed onto freed buffers)."""
    case("graph replays vs per-step loop")
    m, _ = models("h256_g2")
    prompt = tokens("h256_g2", 12, seed=13)
    longer = tokens("h256_g2", 150, seed=14)
    out = {}
    for use_graph in (False, True):
        s, kv, first = prefill(gpu, m, prompt, 256)
        seq = []
        ids, _ = gpu.GpuGenerate(m, kv, s, first, gpu.GpuGenerateOptions(max_tokens=5, use_graph=use_graph))
        seq += ids
        gpu.GpuForwardStep(m, 7, kv.len(), kv, s, want_logits=False)  # eager work between replays
        ids, _ = gpu.GpuGenerate(m, kv, s, s.logits_dev(), gpu.GpuGenerateOptions(max_tokens=5, use_graph=use_graph))
        seq += ids
        kv.reset()
        gpu.GpuForwardFull(m, longer, s, want_logits=False, kv=kv)  # grows the scratch
        vocab = 1000
        ids, _ = gpu.GpuGenerate(m, kv, s, s.logits_dev() + 4 * vocab * 149,
                                 gpu.GpuGenerateOptions(max_tokens=5, use_graph=use_graph))
        seq += ids
        out[use_graph] = seq
        kv.free()
        s.free()
    assert out[True] == out[False]
