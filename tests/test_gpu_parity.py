"""Parity of the HIP operators (through the C ABI) with the CPU oracle.

Bars (written into each test):
  * dequant, gather, fp16 KV write, residual add: bit-exact;
  * RMSNorm, RoPE, SwiGLU: |gpu - ref| <= 1e-6 + 1e-5 * |ref| against the float64
    restatement, and (where the op order is the same) near-identical to the fp32
    oracle.
Sizes are the benchmark's configurations (Qwen3-1.7B / 4B shapes, n = 1, 21, 2811, 4096)
plus ragged / unaligned / edge cases. Every case prints its name before launching.
"""
from __future__ import annotations

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

RTOL = 1e-5
ATOL = 1e-6
EPS = 1e-6


def case(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def within(got, ref, rtol=RTOL, atol=ATOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref) - (atol + rtol * np.abs(ref))
    return bool(np.all(err <= 0)), float(np.max(np.abs(got - ref)))


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


# ----------------------------------------------------------------------------- dequant / gather


def test_f16_sweep_exhaustive(gpu, ora):
    import torch

    case("f16 sweep 65536")
    out = torch.empty(65536, dtype=torch.float32, device="cuda")
    gpu.GpuF16Sweep(out)
    want = ora.f16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    assert np.array_equal(bits(host(out)), bits(want))


@pytest.mark.parametrize("t,key", [(12, "q4k"), (14, "q6k")])
def test_dequant_row_reference_golden(gpu, golden, t, key):
    import torch

    case(f"dequant golden {key}")
    blocks = golden[f"{key}_blocks"]
    n = blocks.shape[0] * 256
    dst = torch.empty(n, dtype=torch.float32, device="cuda")
    gpu.GpuDequantRow(t, dev(blocks.reshape(-1)), n, dst)
    assert np.array_equal(bits(host(dst)), golden[f"{key}_out_bits"])


@pytest.mark.parametrize("t", [0, 12, 14])
@pytest.mark.parametrize("offset", [0, 2, 4, 1])
def test_dequant_row_random_and_unaligned(gpu, ora, t, offset):
    import torch

    case(f"dequant random type={t} offset={offset}")
    rng = np.random.default_rng(100 + t + offset)
    n = 64 * 256
    raw = synth.quant_table(rng, t, 1, n)
    buf = np.zeros(raw.size + 16, np.uint8)
    buf[offset:offset + raw.size] = raw
    d_buf = dev(buf)
    dst = torch.empty(n, dtype=torch.float32, device="cuda")
    gpu.GpuDequantRow(t, d_buf.data_ptr() + offset, n, dst)
    want = ora.dequantize_row(t, raw, n)
    assert np.array_equal(bits(host(dst)), bits(want))


@pytest.mark.parametrize("t", [12, 14])
def test_embedding_gather_full_table(gpu, ora, t):
    """The gather configuration: token_embd [151936, 2048], 2811 uniform ids, bit-exact."""
    import torch

    rows, cols, seq = 151936, 2048, 2811
    case(f"gather full table type={t} rows={rows} seq={seq}")
    rng = np.random.default_rng(200 + t)
    table = synth.quant_table(rng, t, rows, cols)
    toks = rng.integers(0, rows, seq, dtype=np.int64).astype(np.int32)
    toks[:3] = [0, rows - 1, 7]
    emb = gpu.GpuTensor(dev(table), t, rows, cols)
    x = torch.empty((seq, cols), dtype=torch.float32, device="cuda")
    gpu.GpuEmbeddingLookup(emb, dev(toks), seq, x)
    want = ora.embedding_lookup(t, table, rows, cols, toks)
    assert np.array_equal(bits(host(x)), bits(want))


@pytest.mark.parametrize("t", [12, 14])
def test_embedding_gather_vocab_shards(gpu, ora, t):
    """The vocabulary-parallel form of the gather over 8 GPUs: shard s holds rows
    [s R, (s + 1) R) of token_embd and looks up ids - s R, so ids outside its rows
    give zero rows. Each shard's rows for its own ids equal the full gather's bit
    for bit, every other row is +0.0, and the sum over shards (the all-reduce)
    equals the full gather."""
    import torch

    rows, cols, seq, shards = 151936, 2048, 2811, 8
    shard_rows = rows // shards
    case(f"gather vocab shards type={t} rows={rows} shards={shards}")
    rng = np.random.default_rng(260 + t)
    table = synth.quant_table(rng, t, rows, cols)
    row_bytes = table.size // rows
    toks = rng.integers(0, rows, seq, dtype=np.int64).astype(np.int32)
    toks[:4] = [0, rows - 1, shard_rows - 1, shard_rows]
    full = torch.empty((seq, cols), dtype=torch.float32, device="cuda")
    gpu.GpuEmbeddingLookup(gpu.GpuTensor(dev(table), t, rows, cols), dev(toks), seq, full)
    want = host(full)
    total = np.zeros((seq, cols), np.float32)
    for sh in range(shards):
        part = table.reshape(rows, row_bytes)[sh * shard_rows:(sh + 1) * shard_rows].reshape(-1)
        x = torch.full((seq, cols), np.nan, dtype=torch.float32, device="cuda")
        gpu.GpuEmbeddingLookup(gpu.GpuTensor(dev(part), t, shard_rows, cols), dev(toks - sh * shard_rows), seq, x)
        got = host(x)
        mine = (toks >= sh * shard_rows) & (toks < (sh + 1) * shard_rows)
        assert np.array_equal(bits(got[mine]), bits(want[mine])), sh
        assert np.all(bits(got[~mine]) == 0), sh
        total += got
    assert np.array_equal(total, want)  # -0.0 values come back as +0.0 from the sum, as from the all-reduce


@pytest.mark.parametrize("t", [0, 12, 14])
@pytest.mark.parametrize("cols", [2560, 8448])
def test_embedding_gather_edges(gpu, ora, t, cols):
    """4B width (2560) and a width past one workgroup per token (33 blocks), duplicates,
    out-of-range ids -> zero rows, n = 1."""
    import torch

    rows = 300
    case(f"gather edges type={t} cols={cols}")
    rng = np.random.default_rng(300 + t)
    table = synth.quant_table(rng, t, rows, cols)
    toks = np.array([5, 5, 299, 0, -1, 300, 2 ** 31 - 1, 17], np.int32)
    emb = gpu.GpuTensor(dev(table), t, rows, cols)
    x = torch.full((toks.size, cols), 7.0, dtype=torch.float32, device="cuda")
    gpu.GpuEmbeddingLookup(emb, dev(toks), toks.size, x)
    assert np.array_equal(bits(host(x)), bits(ora.embedding_lookup(t, table, rows, cols, toks)))
    x1 = torch.empty((1, cols), dtype=torch.float32, device="cuda")
    gpu.GpuEmbeddingLookup(emb, dev(toks[2:3]), 1, x1)
    assert np.array_equal(bits(host(x1)), bits(ora.embedding_lookup(t, table, rows, cols, toks[2:3])))


# ----------------------------------------------------------------------------- KV write


def test_kv_write_reference_kat(gpu):
    """tools/kv_map_check.cu:51-186 verbatim: 3 heads x dim 8, capacity 12, positions [4, 9)."""
    import torch

    case("kv map KAT")
    heads, dim, max_seq, pos0, seq = 3, 8, 12, 4, 5
    t, h, d = np.meshgrid(np.arange(seq), np.arange(heads), np.arange(dim), indexing="ij")
    k = (h * 100 + t * 10 + d).astype(np.float32)
    v = k + np.float32(1000)
    kc = torch.zeros(heads * max_seq * dim, dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    gpu.GpuKvWrite(dev(k), dev(v), heads, dim, pos0, seq, kc, vc, max_seq)
    kh = host(kc).view(np.float16).reshape(heads, max_seq, dim).astype(np.float32)
    vh = host(vc).view(np.float16).reshape(heads, max_seq, dim).astype(np.float32)
    for hh in range(heads):
        for tt in range(seq):
            assert np.array_equal(kh[hh, pos0 + tt], hh * 100 + tt * 10 + np.arange(dim))
            assert np.array_equal(vh[hh, pos0 + tt], hh * 100 + tt * 10 + np.arange(dim) + 1000)
    untouched = np.ones(max_seq, bool)
    untouched[pos0:pos0 + seq] = False
    assert np.all(host(kc).reshape(heads, max_seq, dim)[:, untouched] == 0)
    assert np.all(host(vc).reshape(heads, max_seq, dim)[:, untouched] == 0)
    with pytest.raises(gpu.RpgError, match="run past the .* cache slots"):
        gpu.GpuKvWrite(dev(k), dev(v), heads, dim, 8, seq, kc, vc, max_seq)


@pytest.mark.parametrize("head_dim,pos0,seq", [(128, 0, 2811), (128, 4095, 1), (128, 1285, 2811), (6, 2, 9)])
def test_kv_write_rne_bitexact(gpu, ora, head_dim, pos0, seq):
    import torch

    heads, max_seq = 8, 4096
    case(f"kv write d={head_dim} pos0={pos0} seq={seq}")
    rng = np.random.default_rng(400 + pos0)
    k = synth.normal(rng, (seq, heads, head_dim))
    v = synth.normal(rng, (seq, heads, head_dim))
    # exact half-way values, subnormal halves, overflow, infinities
    specials = np.array([1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, -2049.0, 65519.0, 65520.0, -70000.0, 3e-8,
                         -6.0e-8, 2.0 ** -25, np.inf], np.float32)
    k.reshape(-1)[: specials.size] = specials
    v.reshape(-1)[-specials.size:] = specials
    kc = torch.full((heads * max_seq * head_dim,), 0x1234, dtype=torch.int16, device="cuda")
    vc = torch.full_like(kc, 0x1234)
    gpu.GpuKvWrite(dev(k), dev(v), heads, head_dim, pos0, seq, kc, vc, max_seq)
    want_k = np.full(heads * max_seq * head_dim, 0x1234, np.uint16)
    want_v = want_k.copy()
    assert ora.kv_write(k, v, heads, head_dim, pos0, seq, want_k, want_v, max_seq) == 0
    assert np.array_equal(host(kc).view(np.uint16), want_k)
    assert np.array_equal(host(vc).view(np.uint16), want_v)


# ----------------------------------------------------------------------------- RMSNorm


@pytest.mark.parametrize("rows,n", [(21, 2048), (2811, 2048), (1, 2048), (4096, 2560), (7, 4096)])
def test_rms_norm_hidden(gpu, ora, rows, n):
    import torch

    case(f"rms_norm hidden rows={rows} n={n}")
    rng = np.random.default_rng(500 + rows)
    x = synth.normal(rng, (rows, n))
    w = synth.normal(rng, n, 1.0, 0.1)
    out = torch.empty((rows, n), dtype=torch.float32, device="cuda")
    gpu.GpuRmsNorm(dev(x), dev(w), rows, n, n, EPS, out)
    got = host(out)
    ok, err = within(got, ora.rms_norm_f64(x, w, rows, n, n, EPS))
    assert ok, err
    ref32 = ora.rms_norm(x, w, rows, n, n, EPS)
    assert np.mean(bits(got) == bits(ref32)) > 0.999  # only the double-summation order differs


@pytest.mark.parametrize("rows", [21 * 16, 2811 * 8, 1])
def test_rms_norm_head_inplace(gpu, ora, rows):
    case(f"rms_norm head rows={rows} in place")
    rng = np.random.default_rng(600 + rows)
    x = synth.normal(rng, (rows, 128))
    w = synth.normal(rng, 128, 1.0, 0.1)
    xd = dev(x)
    gpu.GpuRmsNorm(xd, dev(w), rows, 128, 128, EPS, xd)
    ok, err = within(host(xd), ora.rms_norm_f64(x, w, rows, 128, 128, EPS))
    assert ok, err


@pytest.mark.parametrize("rows,n,stride,off", [(5, 100, 130, 0), (3, 2048, 2048, 1), (9, 128, 129, 0),
                                               (4, 300, 300, 0)])
def test_rms_norm_generic_paths(gpu, ora, rows, n, stride, off):
    import torch

    case(f"rms_norm generic rows={rows} n={n} stride={stride} off={off}")
    rng = np.random.default_rng(700 + n)
    x = synth.normal(rng, rows * stride + off)
    w = synth.normal(rng, n, 1.0, 0.1)
    xd = dev(x)
    outd = torch.zeros_like(xd)
    gpu.GpuRmsNorm(xd.data_ptr() + 4 * off, dev(w), rows, n, stride, EPS, outd.data_ptr() + 4 * off)
    got = host(outd)[off:]
    want = ora.rms_norm_f64(x[off:], w, rows, n, stride, EPS)
    for r in range(rows):
        ok, err = within(got[r * stride:r * stride + n], want[r])
        assert ok, (r, err)


@pytest.mark.parametrize("rows,n", [(21, 2048), (2811, 2048), (1, 2048), (4096, 2560), (5, 1000), (3, 768)])
def test_add_rms_norm(gpu, ora, rows, n):
    import torch

    case(f"add_rms_norm rows={rows} n={n}")
    rng = np.random.default_rng(800 + rows)
    x = synth.normal(rng, (rows, n))
    d = synth.normal(rng, (rows, n))
    w = synth.normal(rng, n, 1.0, 0.1)
    xd = dev(x)
    h = torch.empty_like(xd)
    gpu.GpuAddRmsNorm(xd, dev(d), dev(w), rows, n, EPS, h)
    assert np.array_equal(bits(host(xd)), bits(x + d))       # the residual add is bit-exact
    ok, err = within(host(h), ora.rms_norm_f64(x + d, w, rows, n, n, EPS))
    assert ok, err


@pytest.mark.parametrize("rows,n", [(2811, 2048), (4096, 2560), (2049, 4096), (2048, 2048), (2100, 512), (2300, 3072)])
def test_add_rms_norm_persistent_equals_row_blocks(gpu, ora, rows, n):
    """Launches of at least two rows per workgroup of a four-per-CU grid run the
    persistent kernel (the next row's loads in flight); smaller launches run one
    workgroup per row. The same rows in one launch and in slices of 1000 and of 50
    rows must give the same bits (2049 rows: one workgroup of a 1024 grid takes three
    rows, the others two)."""
    import torch

    case(f"add_rms_norm persistent rows={rows} n={n}")
    rng = np.random.default_rng(850 + rows)
    x = synth.normal(rng, (rows, n))
    d = synth.normal(rng, (rows, n))
    w = synth.normal(rng, n, 1.0, 0.1)
    dd, wd = dev(d), dev(w)
    xa = dev(x)
    ha = torch.empty_like(xa)
    gpu.profile_start(4)
    gpu.GpuAddRmsNorm(xa, dd, wd, rows, n, EPS, ha)
    gpu.profile_stop()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if rows >= 2 * 4 * cus:
        assert "AddRmsNormRowsKernel" in gpu.profile_report()
    assert np.array_equal(bits(host(xa)), bits(x + d))
    for step in (1000, 50):  # one workgroup per row
        xb = dev(x)
        hb = torch.empty_like(xb)
        for r0 in range(0, rows, step):
            r1 = min(rows, r0 + step)
            gpu.GpuAddRmsNorm(xb[r0:r1], dd[r0:r1], wd, r1 - r0, n, EPS, hb[r0:r1])
        assert np.array_equal(bits(host(xa)), bits(host(xb))), step
        assert np.array_equal(bits(host(ha)), bits(host(hb))), step
    ok, err = within(host(ha), ora.rms_norm_f64(x + d, w, rows, n, n, EPS))
    assert ok, err


# ----------------------------------------------------------------------------- RoPE


@pytest.mark.parametrize("rows,heads,head_dim,pos0", [(21, 16, 128, 0), (2811, 8, 128, 0), (1, 16, 128, 3999),
                                                      (13, 4, 64, 5)])
def test_rope(gpu, ora, rows, heads, head_dim, pos0):
    case(f"rope rows={rows} heads={heads} d={head_dim} pos0={pos0}")
    rng = np.random.default_rng(900 + rows)
    tab = ora.build_rope_table(head_dim, 1e6, 4096)
    x = synth.normal(rng, (rows, heads, head_dim))
    xd = dev(x)
    gpu.GpuRope(xd, heads, head_dim, dev(tab), pos0, rows)
    got = host(xd)
    ok, err = within(got.reshape(-1), ora.rope_f64(x, heads, head_dim, tab, pos0, rows))
    assert ok, err
    # same op order as the fp32 oracle (a*c - b*s with separate roundings): identical bits
    assert np.array_equal(bits(got.reshape(-1)), bits(ora.rope(x, heads, head_dim, tab, pos0, rows).reshape(-1)))
    if pos0 == 0:
        assert np.array_equal(got[0], x[0])                    # position 0 is the identity


# ----------------------------------------------------------------------------- fused q/k norm + RoPE + KV


QK_CASES = [
    # (name, Hq, Hkv, seq, pos0): the n = 21, decode, n = 2811 and 4B n = 4096 configurations
    ("1.7B n=21", 16, 8, 21, 0),
    ("1.7B decode n=1", 16, 8, 1, 2731),
    ("1.7B prefill n=2811", 16, 8, 2811, 0),
    ("4B prefill n=4096 (fills cache)", 32, 8, 4096, 0),
    ("1.7B continuation", 16, 8, 300, 3796),
    # the launcher switches to buffer stores from 64 tokens on: both sides of that line
    ("1.7B n=63 (global stores)", 16, 8, 63, 17),
    ("1.7B n=64 (buffer stores)", 16, 8, 64, 4032),
    # one GPU's share under tensor parallelism over 8 GPUs (one kv head each)
    ("1.7B TP=8 shard n=2811", 2, 1, 2811, 0),
    ("4B TP=8 shard n=4096", 4, 1, 4096, 0),
]


@pytest.mark.parametrize("name,hq,hkv,seq,pos0", QK_CASES)
@pytest.mark.parametrize("write_k", [True, False])
def test_qk_norm_rope_kv(gpu, ora, name, hq, hkv, seq, pos0, write_k):
    import torch

    case(f"qk_norm_rope_kv {name} write_k={write_k}")
    d, max_seq = 128, 4096
    rng = np.random.default_rng(1000 + seq + pos0)
    tab = ora.build_rope_table(d, 1e6, 4096)
    q = synth.normal(rng, (seq, hq, d))
    k = synth.normal(rng, (seq, hkv, d))
    v = synth.normal(rng, (seq, hkv, d))
    qn = synth.normal(rng, d, 1.0, 0.1)
    kn = synth.normal(rng, d, 1.0, 0.1)
    qd, kd, vd = dev(q), dev(k), dev(v)
    kc = torch.full((hkv * max_seq * d,), 0x5A5A, dtype=torch.int16, device="cuda")
    vc = torch.full_like(kc, 0x5A5A)
    gpu.GpuQkNormRopeKv(qd, kd, vd, dev(qn), dev(kn), hq, hkv, d, dev(tab), 4096, pos0, seq, EPS, kc, vc, max_seq,
                        write_k_f32=write_k)
    ok, err = within(host(qd).reshape(-1), ora.norm_rope_f64(q, qn, hq, d, tab, pos0, seq, EPS))
    assert ok, ("q", err)
    kc3 = host(kc).view(np.uint16).reshape(hkv, max_seq, d)
    vc3 = host(vc).view(np.uint16).reshape(hkv, max_seq, d)
    k_ref = ora.norm_rope_f64(k, kn, hkv, d, tab, pos0, seq, EPS).reshape(seq, hkv, d)
    k_cached = kc3[:, pos0:pos0 + seq].view(np.float16).astype(np.float32).transpose(1, 0, 2)
    # fp16 store of the normalised, rotated k: the fp32 bar (1e-5 rel, 1e-6 abs) plus half an fp16 ulp
    # (2^-11 relative, 2^-25 absolute below the normal range)
    ok, err = within(k_cached, k_ref, rtol=2.0 ** -11 + 1e-5, atol=1e-6 + 2.0 ** -25)
    assert ok, ("k cache", err)
    if write_k:
        kf = host(kd)
        ok, err = within(kf.reshape(-1), k_ref.reshape(-1))
        assert ok, ("k f32", err)
        # the cache holds exactly the RNE fp16 of the fp32 k the kernel computed
        assert np.array_equal(kc3[:, pos0:pos0 + seq].transpose(1, 0, 2), ora.f32_to_f16_rne(kf))
    else:
        assert np.array_equal(bits(host(kd)), bits(k))        # k left untouched
    assert np.array_equal(vc3[:, pos0:pos0 + seq].transpose(1, 0, 2), ora.f32_to_f16_rne(v))
    outside = np.ones(max_seq, bool)
    outside[pos0:pos0 + seq] = False
    assert np.all(kc3[:, outside] == 0x5A5A) and np.all(vc3[:, outside] == 0x5A5A)


def test_qk_norm_rope_kv_matches_unfused_reference_sequence(gpu, ora):
    """The fused operator equals the reference's own op sequence run on the GPU
    (GpuRmsNorm q, k; GpuRope q, k; GpuKvWrite), src/qwen3_gpu.cu:77-91."""
    import torch

    case("qk fused vs unfused sequence n=64")
    hq, hkv, d, seq, pos0, max_seq = 16, 8, 128, 64, 17, 256
    rng = np.random.default_rng(1100)
    tab = dev(ora.build_rope_table(d, 1e6, max_seq))
    q = synth.normal(rng, (seq, hq, d))
    k = synth.normal(rng, (seq, hkv, d))
    v = synth.normal(rng, (seq, hkv, d))
    qn = dev(synth.normal(rng, d, 1.0, 0.1))
    kn = dev(synth.normal(rng, d, 1.0, 0.1))
    q1, k1, v1 = dev(q), dev(k), dev(v)
    kc1 = torch.zeros(hkv * max_seq * d, dtype=torch.int16, device="cuda")
    vc1 = torch.zeros_like(kc1)
    gpu.GpuQkNormRopeKv(q1, k1, v1, qn, kn, hq, hkv, d, tab, max_seq, pos0, seq, EPS, kc1, vc1, max_seq, True)
    q2, k2, v2 = dev(q), dev(k), dev(v)
    kc2 = torch.zeros_like(kc1)
    vc2 = torch.zeros_like(kc1)
    gpu.GpuRmsNorm(q2, qn, seq * hq, d, d, EPS, q2)
    gpu.GpuRmsNorm(k2, kn, seq * hkv, d, d, EPS, k2)
    gpu.GpuRope(q2, hq, d, tab, pos0, seq)
    gpu.GpuRope(k2, hkv, d, tab, pos0, seq)
    gpu.GpuKvWrite(k2, v2, hkv, d, pos0, seq, kc2, vc2, max_seq)
    assert np.array_equal(bits(host(q1)), bits(host(q2)))
    assert np.array_equal(bits(host(k1)), bits(host(k2)))
    assert np.array_equal(host(kc1), host(kc2)) and np.array_equal(host(vc1), host(vc2))


@pytest.mark.parametrize("cache_off", [4, 1])
def test_qk_norm_rope_kv_unaligned_cache_base(gpu, ora, cache_off):
    """Cache bases that are not 16-byte aligned (offset by `cache_off` halves) take
    the unfused sequence; the cache and q bits equal those of the fused kernel."""
    import torch

    case(f"qk cache base offset {cache_off} halves")
    hq, hkv, d, seq, pos0, max_seq = 16, 8, 128, 40, 5, 128
    rng = np.random.default_rng(1200 + cache_off)
    tab = dev(ora.build_rope_table(d, 1e6, max_seq))
    q = synth.normal(rng, (seq, hq, d))
    k = synth.normal(rng, (seq, hkv, d))
    v = synth.normal(rng, (seq, hkv, d))
    qn = dev(synth.normal(rng, d, 1.0, 0.1))
    kn = dev(synth.normal(rng, d, 1.0, 0.1))
    n_cache = hkv * max_seq * d
    q1, k1 = dev(q), dev(k)
    kc1 = torch.zeros(n_cache, dtype=torch.int16, device="cuda")
    vc1 = torch.zeros_like(kc1)
    gpu.GpuQkNormRopeKv(q1, k1, dev(v), qn, kn, hq, hkv, d, tab, max_seq, pos0, seq, EPS, kc1, vc1, max_seq, True)
    q2, k2 = dev(q), dev(k)
    kbuf = torch.zeros(n_cache + 8, dtype=torch.int16, device="cuda")
    vbuf = torch.zeros_like(kbuf)
    kc2 = kbuf[cache_off:cache_off + n_cache]
    vc2 = vbuf[cache_off:cache_off + n_cache]
    gpu.GpuQkNormRopeKv(q2, k2, dev(v), qn, kn, hq, hkv, d, tab, max_seq, pos0, seq, EPS, kc2, vc2, max_seq, True)
    assert np.array_equal(bits(host(q1)), bits(host(q2)))
    assert np.array_equal(bits(host(k1)), bits(host(k2)))
    assert np.array_equal(host(kc1), host(kc2)) and np.array_equal(host(vc1), host(vc2))
    kb, vb = host(kbuf), host(vbuf)
    assert not kb[:cache_off].any() and not kb[cache_off + n_cache:].any()
    assert not vb[:cache_off].any() and not vb[cache_off + n_cache:].any()


# ----------------------------------------------------------------------------- SwiGLU / add


@pytest.mark.parametrize("n,off", [(21 * 6144, 0), (2811 * 6144, 0), (6144, 0), (1, 0), (1001, 0), (1003, 1),
                                   (4096 * 9728, 0),
                                   # TP=8 shards of the intermediate width (1.7B: 768 columns, 4B: 1216)
                                   (2811 * 768, 0), (4096 * 1216, 0),
                                   # write-through stores from 131072 elements on; the last block partial
                                   (131071, 0), (131072, 0), (131072 + 2050, 0), (262147, 1)])
def test_silu_mul(gpu, ora, n, off):
    import torch

    case(f"silu_mul n={n} off={off}")
    rng = np.random.default_rng(1200 + n % 1000)
    g = synth.normal(rng, n + off, 0.0, 2.0)
    u = synth.normal(rng, n + off, 0.0, 2.0)
    g[off: off + 6] = [0.0, -0.0, -100.0, 100.0, -1e30, 88.0][: min(6, n)]
    gd, ud = dev(g), dev(u)
    gpu.GpuSiluMulInPlace(gd.data_ptr() + 4 * off, ud.data_ptr() + 4 * off, n)
    got = host(gd)[off:]
    ok, err = within(got, ora.silu_mul_f64(g[off:], u[off:]))
    assert ok, err


@pytest.mark.parametrize("n,off", [(2811 * 2048, 0), (1, 0), (4097, 0), (999, 3), (4096 * 2560, 0)])
def test_vec_add_bitexact(gpu, n, off):
    case(f"vec_add n={n} off={off}")
    rng = np.random.default_rng(1300 + n % 1000)
    a = synth.normal(rng, n + off)
    b = synth.normal(rng, n + off)
    ad, bd = dev(a), dev(b)
    gpu.GpuVecAddInPlace(ad.data_ptr() + 4 * off, bd.data_ptr() + 4 * off, n)
    got = host(ad)
    assert np.array_equal(bits(got[off:]), bits(a[off:] + b[off:]))
    assert np.array_equal(bits(got[:off]), bits(a[:off]))


def test_stream_copy(gpu):
    import torch

    case("stream copy 64 MiB")
    src = torch.randn(16 << 20, device="cuda")
    dst = torch.empty_like(src)
    gpu.GpuStreamCopy(src, dst, src.numel() * 4)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)


def test_stream_fill(gpu):
    import torch

    case("stream fill 64 MiB + 16 B inside a larger buffer")
    buf = torch.zeros((16 << 20) + 12, dtype=torch.int32, device="cuda")
    n = (16 << 20) + 4
    gpu.GpuStreamFill(buf[4:4 + n], n * 4, 0x89ABCDEF)
    got = buf.cpu().numpy().view(np.uint32)
    assert np.all(got[4:4 + n] == 0x89ABCDEF)
    assert not got[:4].any() and not got[4 + n:].any()


def test_stream_read(gpu):
    import torch

    case("stream read 64 MiB + 48 B: writes only when a thread's fold equals the key")
    rng = np.random.default_rng(31)
    n16 = (4 << 20) + 3                                    # a ragged last workgroup
    words = rng.integers(0, 1 << 32, 4 * n16, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).cuda()
    sink = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    gpu.GpuStreamRead(src, 4 * words.size, sink, key=0x9E3779B9)
    torch.cuda.synchronize()
    assert int(sink.item()) == 7                           # no thread folds to the key: nothing written
    # thread 0 of workgroup 0 reads float4 0, 256, 512, 768 (256 threads, 4 per thread)
    f4 = words.reshape(-1, 4)
    fold = np.bitwise_xor.reduce(f4[[0, 256, 512, 768]].ravel())
    gpu.GpuStreamRead(src, 4 * words.size, sink, key=int(fold))
    torch.cuda.synchronize()
    assert int(sink.cpu().numpy().view(np.uint32)[0]) == int(fold)
    # the last thread of the ragged tail: float4 n16 - 1 alone (its other three are past the end)
    last = n16 - 1
    blk, t = divmod(last, 1024)
    idx = [blk * 1024 + t % 256 + u * 256 for u in range(4)]
    idx = [i for i in idx if i < n16]
    tail_fold = np.bitwise_xor.reduce(f4[idx].ravel())
    sink.fill_(7)
    gpu.GpuStreamRead(src, 4 * words.size, sink, key=int(tail_fold))
    torch.cuda.synchronize()
    assert int(sink.cpu().numpy().view(np.uint32)[0]) == int(tail_fold)


# ----------------------------------------------------------------------------- graph capture


def test_graph_capture_reads_staged_pos0(gpu, ora):
    """Captured launches read pos0 from the staging scalar, so one graph serves every
    decode step (src/cuda_common.h:139-175). Each replay is checked against an eager run."""
    import torch

    case("graph capture with staged pos0")
    hq, hkv, d, max_seq = 16, 8, 128, 64
    rng = np.random.default_rng(1400)
    tab = dev(ora.build_rope_table(d, 1e6, max_seq))
    qn = dev(synth.normal(rng, d, 1.0, 0.1))
    kn = dev(synth.normal(rng, d, 1.0, 0.1))
    q0 = synth.normal(rng, (1, hq, d))
    k0 = synth.normal(rng, (1, hkv, d))
    v0 = synth.normal(rng, (1, hkv, d))
    qd, kd, vd = dev(q0), dev(k0), dev(v0)
    kc = torch.zeros(hkv * max_seq * d, dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with gpu.ScopedEngineStream(s):
            g.capture_begin()
            gpu.GpuQkNormRopeKv(qd, kd, vd, qn, kn, hq, hkv, d, tab, max_seq, 0, 1, EPS, kc, vc, max_seq, True)
            g.capture_end()
    torch.cuda.synchronize()
    for pos in (3, 40, 0, 63):
        qd.copy_(dev(q0))
        kd.copy_(dev(k0))
        torch.cuda.synchronize()
        gpu.stage_pos0(pos)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        q_graph = host(qd).copy()
        kc_graph = host(kc).reshape(hkv, max_seq, d)[:, pos].copy()
        qd.copy_(dev(q0))
        kd.copy_(dev(k0))
        kc2 = torch.zeros_like(kc)
        vc2 = torch.zeros_like(vc)
        gpu.GpuQkNormRopeKv(qd, kd, vd, qn, kn, hq, hkv, d, tab, max_seq, pos, 1, EPS, kc2, vc2, max_seq, True)
        assert np.array_equal(bits(q_graph), bits(host(qd))), pos
        assert np.array_equal(kc_graph, host(kc2).reshape(hkv, max_seq, d)[:, pos]), pos


def test_launch_profiler_counts_and_times(gpu):
    """Dispatch-attached timing: one record per launch, positive durations, names as launched."""
    import torch

    case("launch profiler")
    a = torch.randn(1 << 20, device="cuda")
    b = torch.randn(1 << 20, device="cuda")
    gpu.profile_start(8)
    for _ in range(3):
        gpu.GpuSiluMulInPlace(a, b, a.numel())
    gpu.GpuVecAddInPlace(a, b, a.numel())
    gpu.profile_stop()
    gpu.GpuVecAddInPlace(a, b, a.numel())          # not recorded: profiling stopped
    rep = gpu.profile_report()
    assert rep["SiluMulKernel"]["count"] == 3 and rep["VecAddKernel"]["count"] == 1
    for k in rep.values():
        assert 0 < k["min_us"] <= k["avg_us"] <= k["max_us"] < 1e5
