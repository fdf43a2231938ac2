"""Attention over the fp16 KV cache (GpuAttentionFromCache, src/kernels_gpu.h:113-116)
on the GPU against the float64 oracle.

Bar: the GPU computes each score as an fp32 dot product of 128 terms (plus the
scale), so |s_gpu - s| <= delta = (d + 2) 2^-24 smag, with smag = max_j scale
sum_d |q_d k_jd|. A perturbation of every score by at most delta changes each
softmax weight by a factor within e^(+-2 delta), so the weighted sum of the v
rows moves by at most (e^(2 delta) - 1) vmax. The exponentials, the running sums
and the weighted sums add fp32 rounding over at most pos + 1 terms and one merge:
(pos + 64) 2^-24 vmax more. A wrong row, head, scale or causal limit breaks the
bound by orders of magnitude.
"""
from __future__ import annotations

import numpy as np
import pytest

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


def check(got, ref, smag, vmax, pos0, d=128):
    """got / ref [seq, heads, d]; smag / vmax [seq, heads]; token t sees pos0 + t + 1 keys."""
    seq = ref.shape[0]
    keys = (pos0 + 1 + np.arange(seq, dtype=np.float64))[:, None]
    delta = (d + 2) * U * smag
    bound = (np.expm1(2 * delta) + (keys + 64) * U) * vmax + 1e-30
    err = np.max(np.abs(got.reshape(ref.shape).astype(np.float64) - ref), axis=-1)
    assert err.shape == bound.shape
    assert np.all(err <= bound), f"max error / bound = {float(np.max(err / bound)):.3g}"


def make(rng, nh, nkv, max_seq, seq, d=128, qscale=1.0):
    q = rng.normal(0, qscale, (seq, nh, d)).astype(np.float32)
    kc = rng.normal(0, 1, (nkv, max_seq, d)).astype(np.float16).view(np.uint16)
    vc = rng.normal(0, 1, (nkv, max_seq, d)).astype(np.float16).view(np.uint16)
    return q, kc, vc


CASES = [
    # (name, n_heads, n_kv_heads, max_seq, pos0, seq)
    ("1.7B decode at 2731", 16, 8, 4096, 2731, 1),
    ("1.7B decode at 0", 16, 8, 4096, 0, 1),
    ("1.7B decode at 4095 (full cache)", 16, 8, 4096, 4095, 1),
    ("4B decode at 1000", 32, 8, 4096, 1000, 1),
    # several 32-key slabs per chunk: the rescale between slabs and the two alternating slab buffers
    ("1.7B decode at 100 (one chunk, 4 slabs)", 16, 8, 4096, 100, 1),
    ("4B decode at 90 (one chunk, 3 slabs, group 4)", 32, 8, 4096, 90, 1),
    ("1.7B decode at 6000 of 8192 (64-key chunks, 2 slabs each, merged)", 16, 8, 8192, 6000, 1),
    ("1.7B prefill n=21", 16, 8, 4096, 0, 21),
    ("1.7B small batch continuation", 16, 8, 4096, 300, 3),
    ("1.7B prefill n=512 after 100", 16, 8, 1024, 100, 512),
    ("MHA, odd sizes", 4, 4, 200, 37, 70),
    # group sizes the grouped decode kernel does not take (one wave per query head)
    ("GQA group 8 decode", 64, 8, 1024, 700, 1),
    ("GQA group 3, two tokens", 12, 4, 512, 300, 2),
    ("MHA decode (group 1)", 8, 8, 2048, 1999, 1),
    # matrix-core prefill (>= 64 tokens): tile edges, GQA groups, a long cached prefix
    ("prefill n=64 (threshold)", 4, 2, 256, 0, 64),
    ("prefill n=129 (tile edge)", 8, 2, 512, 5, 129),
    ("1.7B prefill n=1024", 16, 8, 1024, 0, 1024),
    ("4B prefill n=300 after 1000", 32, 8, 4096, 1000, 300),
    # key chunks of the matrix-core prefill: up to 4 merged by the last workgroup of each
    # (token tile, head), more by a separate merge launch
    ("1.7B prefill n=128 after 1920 (4 key chunks, merged in the launch)", 16, 8, 4096, 1920, 128),
    ("1.7B prefill n=300 after 3000 (7 key chunks, merge launch)", 16, 8, 4096, 3000, 300),
]


@pytest.mark.parametrize("name,nh,nkv,max_seq,pos0,seq", CASES)
def test_attention_from_cache(gpu, ora, name, nh, nkv, max_seq, pos0, seq):
    import torch

    case(f"attention {name}")
    rng = np.random.default_rng(1300 + pos0 + seq + nh)
    q, kc, vc = make(rng, nh, nkv, max_seq, seq, qscale=0.5)
    out = torch.full((seq, nh, 128), np.nan, dtype=torch.float32, device="cuda")
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc), dev(vc), max_seq, out)
    ref, smag, vmax = ora.attention_f64(q, kc, vc, max_seq, nh, nkv, 128, pos0, seq)
    check(host(out), ref, smag, vmax, pos0)


def test_attention_prefill_ignores_rows_past_the_limit(gpu, ora):
    """Matrix-core prefill: cache rows past pos0 + seq - 1 (inf / NaN garbage) do
    not change a bit of the result."""
    import torch

    case("attention prefill causal limit")
    nh, nkv, max_seq, pos0, seq = 16, 8, 1024, 40, 200
    rng = np.random.default_rng(1450)
    q, kc, vc = make(rng, nh, nkv, max_seq, seq)
    out1 = torch.empty((seq, nh, 128), dtype=torch.float32, device="cuda")
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc), dev(vc), max_seq, out1)
    kc2, vc2 = kc.copy().reshape(nkv, max_seq, 128), vc.copy().reshape(nkv, max_seq, 128)
    kc2[:, pos0 + seq:] = np.float16(np.inf).view(np.uint16)
    vc2[:, pos0 + seq:] = np.float16(np.nan).view(np.uint16)
    out2 = torch.empty_like(out1)
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc2.reshape(-1)), dev(vc2.reshape(-1)), max_seq,
                              out2)
    assert torch.equal(out1, out2)
    ref, smag, vmax = ora.attention_f64(q, kc, vc, max_seq, nh, nkv, 128, pos0, seq)
    check(host(out1), ref, smag, vmax, pos0)


def test_attention_prefill_long_one_head(gpu, ora):
    """Matrix-core prefill of 16512 tokens on one head: 129 token tiles x 8 key
    chunks, more (tile, chunk) pairs than the launch's ordered list holds, so the
    workgroups run last tile first. Rows from the first tile, a chunk boundary
    and the last tile are held to the bound (token t's result depends only on
    q_t and keys <= pos0 + t, so a slice of the oracle covers them)."""
    import torch

    case("attention prefill n=16512, one head")
    nh, nkv, max_seq, pos0, seq = 1, 1, 16512, 0, 16512
    rng = np.random.default_rng(1460)
    q, kc, vc = make(rng, nh, nkv, max_seq, seq, qscale=0.5)
    out = torch.full((seq, nh, 128), np.nan, dtype=torch.float32, device="cuda")
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc), dev(vc), max_seq, out)
    got = host(out)
    for t0, n in ((0, 64), (2080, 64), (seq - 48, 48)):
        ref, smag, vmax = ora.attention_f64(q[t0:t0 + n], kc, vc, max_seq, nh, nkv, 128, pos0 + t0, n)
        check(got[t0:t0 + n], ref, smag, vmax, pos0 + t0)


def test_attention_causal_limit_and_budget(gpu, ora):
    """Cache rows past pos0 + t are never read into the result (garbage there
    changes nothing, bit for bit); a larger position budget (the graph-capture
    layout) gives the same bits as the default one."""
    import torch

    case("attention causal limit / budget")
    nh, nkv, max_seq, pos0, seq = 16, 8, 4096, 1500, 1
    rng = np.random.default_rng(1400)
    q, kc, vc = make(rng, nh, nkv, max_seq, seq)
    out1 = torch.empty((seq, nh, 128), dtype=torch.float32, device="cuda")
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc), dev(vc), max_seq, out1)
    kc2, vc2 = kc.copy().reshape(nkv, max_seq, 128), vc.copy().reshape(nkv, max_seq, 128)
    kc2[:, pos0 + seq:] = np.float16(np.inf).view(np.uint16)
    vc2[:, pos0 + seq:] = np.float16(np.nan).view(np.uint16)
    out2 = torch.empty_like(out1)
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc2), dev(vc2), max_seq, out2)
    a = host(out1)
    assert np.array_equal(a.view(np.uint32), host(out2).view(np.uint32))
    # the graph layout: chunks planned for the whole cache, same positions used
    gpu.GpuAttentionWarmupShmem(max_seq)
    out3 = torch.empty_like(out1)
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, dev(q), seq, dev(kc), dev(vc), max_seq, out3, max_seq)
    ref, smag, vmax = ora.attention_f64(q, kc, vc, max_seq, nh, nkv, 128, pos0, seq)
    check(host(out3), ref, smag, vmax, pos0)


def test_attention_graph_replay_reads_staged_pos0(gpu, ora):
    """Decode attention captured in a HIP graph with the position budget of the
    whole cache; each replay reads pos0 from the staging scalar."""
    import torch

    case("attention graph replay")
    nh, nkv, max_seq = 16, 8, 1024
    rng = np.random.default_rng(1500)
    q, kc, vc = make(rng, nh, nkv, max_seq, 1)
    qd, kd, vd = dev(q), dev(kc), dev(vc)
    out = torch.empty((1, nh, 128), dtype=torch.float32, device="cuda")
    gpu.init()
    gpu.GpuAttentionWarmupShmem(max_seq)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with gpu.ScopedEngineStream(s):
            g.capture_begin()
            gpu.GpuAttentionFromCache(nh, nkv, 128, 5, qd, 1, kd, vd, max_seq, out, max_seq)
            g.capture_end()
    torch.cuda.synchronize()
    for pos in (5, 17, 640, 1023, 64):
        gpu.stage_pos0(pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref, smag, vmax = ora.attention_f64(q, kc, vc, max_seq, nh, nkv, 128, pos, 1)
        check(host(out), ref, smag, vmax, pos)


def test_attention_rejects_bad_arguments(gpu):
    import torch

    case("attention host errors")
    q = torch.zeros(128 * 16, dtype=torch.float32, device="cuda")
    kc = torch.zeros(8 * 64 * 128, dtype=torch.int16, device="cuda")
    out = torch.zeros_like(q)
    with pytest.raises(gpu.RpgError, match="cache capacity"):
        gpu.GpuAttentionFromCache(16, 8, 128, 64, q, 1, kc, kc, 64, out)
    with pytest.raises(gpu.RpgError, match="multiple"):
        gpu.GpuAttentionFromCache(16, 6, 128, 0, q, 1, kc, kc, 64, out)
    with pytest.raises(gpu.RpgError, match="head_dim"):
        gpu.GpuAttentionFromCache(16, 8, 64, 0, q, 1, kc, kc, 64, out)


# GpuQkNormRopeKvAttention: at one token the q/k norm, RoPE and the K/V store run
# inside the decode attention launch with the same routines as GpuQkNormRopeKv,
# so the output and the whole cache must be bit-identical to the two calls.
FUSED = [
    # (name, n_heads, n_kv_heads, max_seq, pos0)
    ("1.7B at 0", 16, 8, 4096, 0),
    ("1.7B at 21", 16, 8, 4096, 21),
    ("1.7B at 127 (last single-chunk position)", 16, 8, 4096, 127),
    ("1.7B at 128 (first split)", 16, 8, 4096, 128),
    ("1.7B at 2731", 16, 8, 4096, 2731),
    ("1.7B at 4095 (full cache)", 16, 8, 4096, 4095),
    ("4B at 1000", 32, 8, 4096, 1000),
    ("MHA at 1999", 8, 8, 2048, 1999),
]


def _fused_inputs(gpu, rng, nh, nkv, max_seq):
    q = dev(rng.normal(0, 2, (1, nh, 128)).astype(np.float32))
    k = dev(rng.normal(0, 2, (1, nkv, 128)).astype(np.float32))
    v = dev(rng.normal(0, 1, (1, nkv, 128)).astype(np.float32))
    qn = dev(rng.normal(1, 0.1, 128).astype(np.float32))
    kn = dev(rng.normal(1, 0.1, 128).astype(np.float32))
    tab = dev(gpu.build_rope_table(128, 1e6, max_seq))
    _, kc, vc = make(rng, nh, nkv, max_seq, 1)
    return q, k, v, qn, kn, tab, dev(kc), dev(vc)


def _two_calls(gpu, nh, nkv, max_seq, pos0, q, k, v, qn, kn, tab, kc, vc, sh=-1):
    import torch

    qa, ka = q.clone(), k.clone()
    out = torch.full((1, nh, 128), np.nan, dtype=torch.float32, device="cuda")
    gpu.GpuQkNormRopeKv(qa, ka, v, qn, kn, nh, nkv, 128, tab, max_seq, pos0, 1, 1e-6, kc, vc, max_seq)
    gpu.GpuAttentionFromCache(nh, nkv, 128, pos0, qa, 1, kc, vc, max_seq, out, sh)
    return out


@pytest.mark.parametrize("name,nh,nkv,max_seq,pos0", FUSED, ids=[f[0] for f in FUSED])
def test_qk_norm_rope_kv_attention_equals_two_calls(gpu, ora, name, nh, nkv, max_seq, pos0):
    import torch

    case(f"fused q/k prep + attention {name}")
    rng = np.random.default_rng(2100 + pos0 + nh)
    q, k, v, qn, kn, tab, kc, vc = _fused_inputs(gpu, rng, nh, nkv, max_seq)
    kc2, vc2 = kc.clone(), vc.clone()
    want = _two_calls(gpu, nh, nkv, max_seq, pos0, q, k, v, qn, kn, tab, kc, vc)
    q0, k0, v0 = q.clone(), k.clone(), v.clone()
    out = torch.full((1, nh, 128), np.nan, dtype=torch.float32, device="cuda")
    assert gpu.GpuQkNormRopeKvAttention(nh, nkv, 128, pos0, q, k, v, qn, kn, tab, max_seq, 1e-6, kc2, vc2, max_seq,
                                        out)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)  # the new row at pos0, nothing else touched
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)
    # and the attention itself against the float64 oracle on the stored operands
    qa = q.clone()
    gpu.GpuQkNormRopeKv(qa, k.clone(), v, qn, kn, nh, nkv, 128, tab, max_seq, pos0, 1, 1e-6, kc.clone(), vc.clone(),
                        max_seq)
    ref, smag, vmax = ora.attention_f64(host(qa), host(kc), host(vc), max_seq, nh, nkv, 128, pos0, 1)
    check(host(out), ref, smag, vmax, pos0)


def test_qk_norm_rope_kv_attention_without_fused_form(gpu):
    """A GQA group of 8 has no fused kernel: nothing runs and the caller is told."""
    import torch

    case("fused q/k prep + attention: group 8")
    rng = np.random.default_rng(2200)
    nh, nkv, max_seq = 64, 8, 512
    q, k, v, qn, kn, tab, kc, vc = _fused_inputs(gpu, rng, nh, nkv, max_seq)
    kc0 = kc.clone()
    out = torch.full((1, nh, 128), np.nan, dtype=torch.float32, device="cuda")
    assert not gpu.GpuQkNormRopeKvAttention(nh, nkv, 128, 7, q, k, v, qn, kn, tab, max_seq, 1e-6, kc, vc, max_seq,
                                            out)
    torch.cuda.synchronize()
    assert torch.isnan(out).all() and torch.equal(kc, kc0)


def test_qk_norm_rope_kv_attention_graph_replay(gpu):
    """Captured once with the whole cache as the position budget; each replay
    reads pos0 from the staging scalar, writes that row and attends up to it,
    bit-identical to the two eager calls at the same position."""
    import torch

    case("fused q/k prep + attention graph replay")
    nh, nkv, max_seq = 16, 8, 1024
    rng = np.random.default_rng(2300)
    q, k, v, qn, kn, tab, kc, vc = _fused_inputs(gpu, rng, nh, nkv, max_seq)
    kc2, vc2 = kc.clone(), vc.clone()
    out = torch.empty((1, nh, 128), dtype=torch.float32, device="cuda")
    gpu.init()
    gpu.GpuAttentionWarmupShmem(max_seq)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with gpu.ScopedEngineStream(s):
            g.capture_begin()
            assert gpu.GpuQkNormRopeKvAttention(nh, nkv, 128, 5, q, k, v, qn, kn, tab, max_seq, 1e-6, kc2, vc2,
                                                max_seq, out, max_seq)
            g.capture_end()
    torch.cuda.synchronize()
    for pos in (5, 17, 127, 128, 640, 1023, 64):
        want = _two_calls(gpu, nh, nkv, max_seq, pos, q, k, v, qn, kn, tab, kc, vc, sh=max_seq)  # same chunk plan
        gpu.stage_pos0(pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), pos
        assert torch.equal(kc2, kc) and torch.equal(vc2, vc), pos
