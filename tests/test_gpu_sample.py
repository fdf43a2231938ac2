"""GPU parity of device argmax and sampling (rpg_op_argmax, rpg_op_filter_to_probs,
rpg_op_inverse_sample, rpg_op_sample_token[_dev]) against the CPU oracle
(oracle/cpu_sample.c, pinned in test_oracle_sample.py).

Bars: argmax, one-hot filters, kept sets and tokens are exact; probabilities
agree to 2^-20 relative per element (the device expf and glibc's expf differ by
an ulp or so); the inverse transform on the device's own probabilities equals the
serial double loop exactly, including u on exact boundaries. The case matrix and
synthetic logits are the reference's (tools/sample_check.cu:48-76).
"""
from __future__ import annotations

import numpy as np
import pytest

from synth import SAMPLE_CASES, SAMPLE_U_COUNT, sample_logits

pytestmark = pytest.mark.gpu

F32_MAX = float(np.finfo(np.float32).max)
PROB_RTOL = 2.0 ** -20


def case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def idx_buf():
    import torch

    return torch.full((1,), -1, dtype=torch.int32, device="cuda")


def gpu_argmax(gpu, x: np.ndarray) -> int:
    out = idx_buf()
    gpu.GpuArgMax(dev(x), x.size, out)
    return int(host(out)[0])


def gpu_filter(gpu, logits_dev, n, t, k, p) -> np.ndarray:
    import torch

    probs = torch.full((n,), np.nan, dtype=torch.float32, device="cuda")
    gpu.GpuFilterToProbs(logits_dev, n, gpu.SampleOptions(t, k, p), probs)
    return host(probs)


def gpu_inverse(gpu, probs_dev, n, u) -> int:
    out = idx_buf()
    gpu.GpuInverseSample(probs_dev, n, u, out)
    return int(host(out)[0])


@pytest.mark.parametrize("n", [1, 7, 1023, 1024, 1025, 4096, 151936, 1 << 22])
def test_argmax_matches_oracle(gpu, ora, n):
    case(f"argmax n={n}")
    rng = np.random.default_rng(n)
    x = rng.normal(size=n).astype(np.float32)
    assert gpu_argmax(gpu, x) == ora.argmax(x, -F32_MAX) == int(np.argmax(x))
    ties = np.round(x * 2).astype(np.float32)  # many equal maxima: the smallest index wins
    assert gpu_argmax(gpu, ties) == ora.argmax(ties, -F32_MAX) == int(np.argmax(ties))
    if n > 1:
        last = x.copy()
        last[-1] = 100.0
        assert gpu_argmax(gpu, last) == n - 1


def test_argmax_floors_and_specials(gpu, ora):
    case("argmax specials")
    x = np.full(5000, -np.inf, np.float32)
    assert gpu_argmax(gpu, x) == 0
    x[4321] = -F32_MAX  # not above GpuArgMax's -FLT_MAX floor
    assert gpu_argmax(gpu, x) == ora.argmax(x, -F32_MAX) == 0
    x[17] = np.nan  # NaN never wins
    x[3000] = -1e30
    assert gpu_argmax(gpu, x) == ora.argmax(x, -F32_MAX) == 3000
    c = np.full(3000, 2.5, np.float32)
    assert gpu_argmax(gpu, c) == 0


@pytest.mark.parametrize("n", [4096, 151936])
@pytest.mark.parametrize("cfg", SAMPLE_CASES, ids=[c[5] for c in SAMPLE_CASES])
def test_filter_matches_oracle(gpu, ora, cfg, n):
    t, k, p, seed, tie, what = cfg
    case(f"filter {what} n={n}")
    logits = sample_logits(seed, tie, n)
    got = gpu_filter(gpu, dev(logits), n, t, k, p)
    want, margin = ora.filter_to_probs(logits, t, k, p)
    assert margin > 1e-9, "top_p decision too close to call for two implementations"
    assert np.array_equal(got > 0, want > 0), "kept sets differ"
    if not t > 0:
        assert np.array_equal(got, want)  # one-hot
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= PROB_RTOL * np.abs(want)), float(np.max(err / np.maximum(np.abs(want), 1e-38)))


def _tied_block_logits(n, block, seed):
    """`block` values exactly 1.0 among n (the rest uniform in [-8, 0.5)): the
    tied block holds ~90% of the softmax mass and one level-1 key bin."""
    rng = np.random.default_rng(seed)
    v = rng.uniform(-8.0, 0.5, n).astype(np.float32)
    v[rng.choice(n, block, replace=False)] = np.float32(1.0)
    return v


@pytest.mark.parametrize("top_k,top_p", [(0, 0.5), (60000, 0.5), (0, 0.97)])
def test_sample_many_candidates(gpu, ora, top_k, top_p):
    """Radix selects whose level-1 digit holds tens of thousands of values (a
    tied block of 60000): the candidates overflow the last workgroup's LDS copy
    and every level reads them from their slices' regions. Kept set exact,
    probabilities to 2^-20, tokens as the oracle's."""
    import torch

    n = 151936
    case(f"many candidates: top_k {top_k}, top_p {top_p}")
    logits = _tied_block_logits(n, 60000, 31)
    logits_dev = dev(logits)
    got = gpu_filter(gpu, logits_dev, n, 1.0, top_k, top_p)
    want, margin = ora.filter_to_probs(logits, 1.0, top_k, top_p)
    assert margin > 1e-9
    assert np.array_equal(got > 0, want > 0), "kept sets differ"
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= PROB_RTOL * np.abs(want))
    probs = torch.empty(n, dtype=torch.float32, device="cuda")
    for c in range(4):
        out = idx_buf()
        gpu.GpuSampleToken(logits_dev, n, gpu.SampleOptions(1.0, top_k, top_p), 7, c, probs, out)
        assert int(host(out)[0]) == ora.sample_token(logits, 1.0, top_k, top_p, 7, c)


@pytest.mark.parametrize("cfg", [c for c in SAMPLE_CASES if c[0] > 0], ids=[c[5] for c in SAMPLE_CASES if c[0] > 0])
def test_inverse_sample_exact_on_device_probs(gpu, ora, cfg):
    """The transform is a pure function of (probs, u): on the device's own
    probabilities it must equal the serial double loop for every u."""
    t, k, p, seed, tie, what = cfg
    n = 151936
    case(f"inverse sample {what}")
    logits_dev = dev(sample_logits(seed, tie, n))
    probs = gpu_filter(gpu, logits_dev, n, t, k, p)
    probs_dev = dev(probs)
    us = [ora.counter_uniform(seed, c) for c in range(48)] + [0.0, 0.5, float(np.float32(0.99999994))]
    cum = np.cumsum(probs.astype(np.float64))
    us += [float(np.float32(cum[i])) for i in (0, 1, n // 2, n - 2) if np.float32(cum[i]) < 1.0]  # near boundaries
    for u in us:
        assert gpu_inverse(gpu, probs_dev, n, u) == ora.inverse_sample(probs, u), u


def test_inverse_sample_boundaries_and_fallbacks(gpu, ora):
    case("inverse sample boundaries")
    # dyadic probabilities: exact running sums, u exactly on each boundary
    rng = np.random.default_rng(7)
    n = 151936
    w = rng.integers(0, 4, size=n).astype(np.float64)
    w[rng.integers(0, n, size=n // 2)] = 0.0
    probs = (w / 2.0 ** 20).astype(np.float32)  # sum < 1, every prefix exact
    pd = dev(probs)
    cum = np.cumsum(probs.astype(np.float64))
    for i in list(rng.integers(0, n, size=24)) + [0, n - 1]:
        u = float(cum[i])
        assert np.float32(u) == u and u < 1.0
        assert gpu_inverse(gpu, pd, n, u) == ora.inverse_sample(probs, u), u
    # the whole sum is below u: the first maximum
    assert gpu_inverse(gpu, pd, n, 0.9999) == ora.inverse_sample(probs, 0.9999) == int(np.argmax(probs))
    small = np.array([0.1, 0.2, 0.2, 0.0], np.float32)
    assert gpu_inverse(gpu, dev(small), 4, 0.75) == 1
    # values the fixed-point path does not take (>= 2): the serial loop decides
    odd = np.array([0.0, 3.0, 0.5, 1e-3], np.float32)
    for u in (0.0, 0.3, 0.9):
        assert gpu_inverse(gpu, dev(odd), 4, u) == ora.inverse_sample(odd, u)


@pytest.mark.parametrize("n", [4096, 151936])
@pytest.mark.parametrize("cfg", SAMPLE_CASES, ids=[c[5] for c in SAMPLE_CASES])
def test_sample_token_matches_oracle(gpu, ora, cfg, n):
    import torch

    t, k, p, seed, tie, what = cfg
    case(f"sample token {what} n={n}")
    logits = sample_logits(seed, tie, n)
    logits_dev = dev(logits)
    probs = torch.empty(n, dtype=torch.float32, device="cuda")
    ref_probs, _ = ora.filter_to_probs(logits, t, k, p)
    ref_cum = np.cumsum(ref_probs.astype(np.float64))
    toks = []
    for c in range(SAMPLE_U_COUNT):
        out = idx_buf()
        gpu.GpuSampleToken(logits_dev, n, gpu.SampleOptions(t, k, p), seed, c, probs, out)
        tok = int(host(out)[0])
        toks.append(tok)
        want = ora.sample_token(logits, t, k, p, seed, c)
        if tok != want:  # allowed only where an ulp of expf can move u across a boundary
            u = ora.counter_uniform(seed, c)
            assert abs(u - ref_cum[want]) < 1e-6 or abs(u - ref_cum[tok]) < 1e-6, (c, tok, want, u)
        if t > 0:  # on the device's own probabilities the transform is exact
            assert tok == ora.inverse_sample(host(probs), ora.counter_uniform(seed, c))
    if not t > 0:
        assert set(toks) == {int(np.argmax(logits))}
    if t == 1.0 and k == 0 and p == 1.0 and not tie:
        assert len(set(toks)) > 1  # u is used


def test_sample_token_dev_counter_and_graph_replay(gpu, ora):
    """GpuSampleTokenDev reads the counter from the pos0 staging scalar: eager and
    graph-replayed draws equal GpuSampleToken with the host counter."""
    import torch

    case("sample token dev + graph")
    n = 151936
    seed = 99
    logits_dev = dev(sample_logits(5, False, n))
    gpu.init()
    gpu.GpuSamplerWarmup()
    counter_dev = gpu.pos_staging_ptr()
    configs = [(0.7, 0, 0.95), (1.0, 20, 0.9), (0.0, 0, 1.0)]
    probs = torch.empty(n, dtype=torch.float32, device="cuda")
    want = {}
    for cfg in configs:
        for c in (0, 1, 2, 1000):
            out = idx_buf()
            gpu.GpuSampleToken(logits_dev, n, gpu.SampleOptions(*cfg), seed, c, probs, out)
            want[cfg, c] = int(host(out)[0])
            gpu.stage_pos0(c)
            out2 = idx_buf()
            gpu.GpuSampleTokenDev(logits_dev, n, gpu.SampleOptions(*cfg), seed, counter_dev, probs, out2)
            assert int(host(out2)[0]) == want[cfg, c], (cfg, c)
    for cfg in configs:
        out = idx_buf()
        gprobs = torch.empty(n, dtype=torch.float32, device="cuda")
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with gpu.ScopedEngineStream(s):
                g.capture_begin()
                gpu.GpuSampleTokenDev(logits_dev, n, gpu.SampleOptions(*cfg), seed, counter_dev, gprobs, out)
                g.capture_end()
        torch.cuda.synchronize()
        for c in (2, 0, 1000, 1):
            gpu.stage_pos0(c)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert int(host(out)[0]) == want[cfg, c], (cfg, c)


def test_inverse_sample_refuses_graph_capture(gpu):
    import torch

    case("inverse sample capture check")
    n = 4096
    probs = torch.full((n,), 1.0 / n, dtype=torch.float32, device="cuda")
    out = idx_buf()
    gpu.GpuSamplerWarmup()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with gpu.ScopedEngineStream(s):
            g.capture_begin()
            try:
                with pytest.raises(gpu.RpgError, match="not capturable"):
                    gpu.GpuInverseSample(probs, n, 0.5, out)
            finally:
                g.capture_end()
    torch.cuda.synchronize()
