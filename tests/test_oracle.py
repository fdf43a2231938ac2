"""Pins the CPU oracle (oracle/cpu_ref.c) to the reference and to mathematics.

Every oracle function is checked against something other than its own formula:
the reference's quant.cc (golden vectors, and oracle/_ref when built here),
numpy's independent IEEE conversions, brute force over all finite halves,
closed forms and invariants. CPU only.
"""
from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest

import synth

TOL_RTOL = 1e-5
TOL_ATOL = 1e-6


def within(got, ref, rtol=TOL_RTOL, atol=TOL_ATOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.all(np.abs(got - ref) <= atol + rtol * np.abs(ref))


# ----------------------------------------------------------------------------- fp16


def test_f16_to_f32_exhaustive_vs_numpy(ora, golden):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = ora.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    finite = ~np.isnan(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.all(np.isnan(got[~finite]))
    # NaN payloads: the reference shifts the payload without quieting it.
    nan_bits = bits[~finite].astype(np.uint32)
    expect = ((nan_bits & 0x8000) << 16) | 0x7F800000 | ((nan_bits & 0x3FF) << 13)
    assert np.array_equal(got[~finite].view(np.uint32), expect)
    # The reference's own F16ToF32 over all 65536 halves (hash stored by make_golden.py).
    assert hashlib.sha256(got.tobytes()).hexdigest() == str(golden["f16_to_f32_sha256"])


def test_f16_to_f32_vs_reference_build(ora):
    ref = ora.ref_lib()
    if ref is None:
        pytest.skip("oracle/_ref not built (reference sources absent on this host)")
    got = ora.f16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    want = ora.ref_f16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _all_finite_halves():
    h = np.arange(0x7C00, dtype=np.uint32).astype(np.uint16)
    return h.view(np.float16).astype(np.float64)  # 0 .. 65504, increasing


def _brute_force_rne(x: np.ndarray) -> np.ndarray:
    """Nearest binary16 by search over every finite half; ties to the even pattern."""
    mags = _all_finite_halves()
    a = np.abs(x.astype(np.float64))
    idx = np.searchsorted(mags, a)
    lo = np.clip(idx - 1, 0, len(mags) - 1)
    hi = np.clip(idx, 0, len(mags) - 1)
    dlo = np.abs(a - mags[lo])
    dhi = np.abs(mags[hi] - a)
    pick = np.where(dlo < dhi, lo, np.where(dhi < dlo, hi, np.where(lo % 2 == 0, lo, hi)))
    # beyond the largest finite half: 65520 and above round to Inf (65504 + half an ulp of 32)
    res = pick.astype(np.uint32)
    res = np.where(a >= 65520.0, 0x7C00, res)
    sign = (np.signbit(x).astype(np.uint32)) << 15
    return (res | sign).astype(np.uint16)


def test_f32_to_f16_rne_brute_force_and_numpy(ora):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.normal(0, 1, 200000),
        rng.normal(0, 1e-5, 50000),      # subnormal halves
        rng.normal(0, 3e4, 50000),       # near overflow
        rng.uniform(-70000, 70000, 5000),
    ]).astype(np.float32)
    got = ora.f32_to_f16_rne(x)
    assert np.array_equal(got, _brute_force_rne(x))
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))


def test_f32_to_f16_rne_exact_ties(ora):
    """Midpoints between adjacent halves (exact in fp32) must round to the even pattern."""
    rng = np.random.default_rng(2)
    h = rng.integers(0, 0x7BFF, 20000).astype(np.uint16)     # finite, not the largest
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    assert np.array_equal(mid.astype(np.float64), (lo + hi) / 2)  # exact ties
    sign = rng.integers(0, 2, mid.size).astype(bool)
    mid = np.where(sign, -mid, mid).astype(np.float32)
    want = np.where(h % 2 == 0, h, h + 1).astype(np.uint16) | (sign.astype(np.uint16) << 15)
    assert np.array_equal(ora.f32_to_f16_rne(mid), want)


def test_f32_to_f16_rne_specials(ora, golden):
    x = np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, -65520.0, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25,
                  2.0 ** -25 * 1.0000001, 2.0 ** -26, 6.1e-5], dtype=np.float32)
    want = np.array([0x0000, 0x8000, 0x7BFF, 0x7BFF, 0x7C00, 0xFC00, 0x7C00, 0xFC00, 0x0001, 0x0000, 0x0001,
                     0x0000, x[-1].astype(np.float16).view(np.uint16)], dtype=np.uint16)
    assert np.array_equal(ora.f32_to_f16_rne(x), want)
    nan = ora.f32_to_f16_rne(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7C00) == 0x7C00 and (nan & 0x3FF) != 0
    # The reference helper dtypes.h F32ToF16 rounds these ties away from zero; RNE does not.
    ties = golden["ties"]
    rne = ora.f32_to_f16_rne(ties)
    assert np.array_equal(rne, ties.astype(np.float16).view(np.uint16))
    assert not np.array_equal(rne, golden["ties_dtypes_f32_to_f16"])


# ----------------------------------------------------------------------------- dequant


def test_dequant_matches_reference_golden(ora, golden):
    for t, key in ((12, "q4k"), (14, "q6k")):
        blocks = golden[f"{key}_blocks"]
        got = ora.dequantize_row(t, blocks.reshape(-1), blocks.shape[0] * 256)
        assert np.array_equal(got.view(np.uint32), golden[f"{key}_out_bits"]), key


def test_dequant_matches_reference_build(ora):
    if ora.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference sources absent on this host)")
    rng = np.random.default_rng(3)
    for t, gen in ((12, synth.q4k_blocks), (14, synth.q6k_blocks)):
        blocks = gen(rng, 512)
        raw = blocks.reshape(-1)
        n = blocks.shape[0] * 256
        a = ora.dequantize_row(t, raw, n)
        b = ora.ref_dequantize_row(t, raw, n)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert ora.row_bytes(t, 2048) == ora.ref_lib().ref_type_row_bytes(t, 2048)


def _h(b0, b1):
    return np.array([b0 | (b1 << 8)], np.uint16).view(np.float16).astype(np.float32)[0]


def _py_q4k_elem(blk: bytes, e: int) -> np.float32:
    """Element e of a Q4_K block from the GGUF layout, one element at a time."""
    f32 = np.float32
    sub, l = e // 32, e % 32
    qbyte = blk[16 + 32 * (sub // 2) + l]
    raw = (qbyte >> 4) if sub % 2 else (qbyte & 15)
    s = blk[4:16]
    if sub < 4:
        sc, m = s[sub] & 63, s[sub + 4] & 63
    else:
        sc = (s[sub + 4] & 15) | ((s[sub - 4] >> 6) << 4)
        m = (s[sub + 4] >> 4) | ((s[sub] >> 6) << 4)
    d, dmin = _h(blk[0], blk[1]), _h(blk[2], blk[3])
    return f32(f32(f32(d) * f32(sc)) * f32(raw)) - f32(f32(dmin) * f32(m))


def _py_q6k_elem(blk: bytes, e: int) -> np.float32:
    f32 = np.float32
    half, r = e // 128, e % 128
    quarter, l = r // 32, r % 32
    qlb = blk[64 * half + l + (32 if quarter % 2 else 0)]
    nib = (qlb & 15) if quarter < 2 else (qlb >> 4)
    hi = (blk[128 + 32 * half + l] >> (2 * quarter)) & 3
    q = (nib | (hi << 4)) - 32
    sc = np.array([blk[192 + 8 * half + l // 16 + 2 * quarter]], np.uint8).view(np.int8)[0]
    d = _h(blk[208], blk[209])
    return f32(f32(d) * f32(sc)) * f32(q)


@pytest.mark.parametrize("t", [12, 14])
def test_dequant_vs_per_element_restatement(ora, t):
    rng = np.random.default_rng(4)
    if t == 12:
        blocks = np.concatenate([synth.q4k_blocks(rng, 3), synth.special_q4k_blocks()])
        elem = _py_q4k_elem
    else:
        blocks = np.concatenate([synth.q6k_blocks(rng, 3), synth.special_q6k_blocks()])
        elem = _py_q6k_elem
    got = ora.dequantize_row(t, blocks.reshape(-1), blocks.shape[0] * 256).reshape(blocks.shape[0], 256)
    with np.errstate(over="ignore", invalid="ignore"):
        for b in range(blocks.shape[0]):
            raw = bytes(blocks[b])
            want = np.array([elem(raw, e) for e in range(256)], np.float32)
            assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (t, b)


def test_dequant_special_closed_forms(ora):
    q4 = synth.special_q4k_blocks()
    y = ora.dequantize_row(12, q4.reshape(-1), q4.shape[0] * 256).reshape(-1, 256)
    assert np.all(y[0].view(np.uint32) == 0)                         # all-zero block -> +0.0
    assert np.all(y[1] == np.float32(63 * 15 - 63))                 # d = dmin = 1, sc = m = 63, q = 15
    # Block 3: d = 1, dmin = 0, scale bytes 0x3F -> sc = 63 for sub-blocks 0..3 and
    # (0x3F & 15) | ((0x3F >> 6) << 4) = 15 for 4..7; qs = 0xA5 -> low nibble 5, high 10.
    sub_sc = np.repeat([63, 63, 63, 63, 15, 15, 15, 15], 32)
    sub_q = np.repeat([5, 10, 5, 10, 5, 10, 5, 10], 32)
    assert np.array_equal(y[3], (sub_sc * sub_q).astype(np.float32))
    # Block 4: d = 0, dmin = 2 -> y = 0*q - 2*m, i.e. +0.0 - 2m (+0.0 where m = 0).
    # Mins unpacked by hand from scale bytes [0,1,2,63, 0,5,6,63, 0xC1,0x72,0x0F,0xF0]:
    # j<4: m = byte[j+4] & 63; j>=4: m = (byte[j+4] >> 4) | ((byte[j] >> 6) << 4).
    m = np.repeat([0, 5, 6, 63, 12, 7, 0, 15], 32)
    want4 = np.float32(0.0) - (np.float32(2.0) * m.astype(np.float32))
    assert np.array_equal(y[4].view(np.uint32), want4.astype(np.float32).view(np.uint32))
    q6 = synth.special_q6k_blocks()
    z = ora.dequantize_row(14, q6.reshape(-1), q6.shape[0] * 256).reshape(-1, 256)
    assert np.all(z[0].view(np.uint32) == 0x80000000)                # q = 0 - 32: (0*0)*(-32) = -0.0
    sc = np.array([-1, -32, 5, -7] * 4, np.int8)
    neg = np.array([sc[e // 128 * 8 + (e % 32) // 16 + 2 * ((e % 128) // 32)] < 0 for e in range(256)])
    assert np.all(z[1] == 0.0)
    assert np.array_equal(np.signbit(z[1]), neg)                     # q = 0 with sc < 0 gives -0.0
    # Block 2: q = 31 everywhere, d = 65504, scales alternate -32, 31 -> y = (65504*sc)*31.
    sc2 = np.array([-32, 31] * 8, np.float32)
    e = np.arange(256)
    sc_e = sc2[e // 128 * 8 + (e % 32) // 16 + 2 * ((e % 128) // 32)]
    assert np.array_equal(z[2], (np.float32(65504.0) * sc_e).astype(np.float32) * np.float32(31))


def test_embedding_lookup_is_rowwise_dequant(ora):
    rng = np.random.default_rng(5)
    rows, cols = 37, 512
    for t in (0, 12, 14):
        table = synth.quant_table(rng, t, rows, cols)
        toks = np.array([0, 36, 5, 5, -1, 37, 12], np.int32)
        out = ora.embedding_lookup(t, table, rows, cols, toks)
        rb = ora.row_bytes(t, cols)
        for i, tok in enumerate(toks):
            if 0 <= tok < rows:
                want = ora.dequantize_row(t, table[tok * rb:(tok + 1) * rb], cols)
                assert np.array_equal(out[i].view(np.uint32), want.view(np.uint32))
            else:
                assert np.all(out[i].view(np.uint32) == 0)


# ----------------------------------------------------------------------------- quantized matmul


def _dequant_matrix(ora, t, w, rows, cols):
    rb = ora.row_bytes(t, cols)
    return np.stack([ora.dequantize_row(t, w[r * rb:(r + 1) * rb], cols) for r in range(rows)])


@pytest.mark.parametrize("t", [0, 12, 14])
def test_matmul_quant_f64_vs_numpy_blas(ora, t):
    """OUT = X . W^T against numpy's float64 matmul of the dequantised matrix (an
    independent BLAS summation), and absdot against |W| . |X|^T."""
    rng = np.random.default_rng(600 + t)
    rows, cols, n = 23, 768, 3
    w = synth.quant_table(rng, t, rows, cols)
    x = rng.normal(0, 1, (n, cols)).astype(np.float32)
    out, absdot = ora.matmul_quant_f64(t, w, rows, cols, x)
    wd = _dequant_matrix(ora, t, w, rows, cols).astype(np.float64)
    want = x.astype(np.float64) @ wd.T
    assert out.shape == (n, rows)
    assert np.allclose(out, want, rtol=1e-12, atol=1e-12 * np.max(np.abs(want)))
    assert np.allclose(absdot, np.abs(x.astype(np.float64)) @ np.abs(wd).T, rtol=1e-12)


def test_matmul_quant_f64_one_hot_and_linearity(ora):
    """One-hot X rows select exact matrix columns (bit-exact, no rounding is
    possible); OUT is linear in X (a dropped or doubled term breaks both)."""
    rng = np.random.default_rng(610)
    rows, cols = 9, 512
    for t in (12, 14):
        w = synth.quant_table(rng, t, rows, cols)
        wd = _dequant_matrix(ora, t, w, rows, cols)
        picks = [0, 1, 255, 256, 300, 511]
        x = np.zeros((len(picks), cols), np.float32)
        x[np.arange(len(picks)), picks] = 1.0
        out, _ = ora.matmul_quant_f64(t, w, rows, cols, x)
        assert np.array_equal(out, wd[:, picks].T.astype(np.float64))
        a = rng.normal(0, 1, (1, cols)).astype(np.float32)
        b = rng.normal(0, 1, (1, cols)).astype(np.float32)
        a[:, cols // 2:] = 0.0          # disjoint supports: a + b is exact in fp32
        b[:, :cols // 2] = 0.0
        oa, _ = ora.matmul_quant_f64(t, w, rows, cols, a)
        ob, _ = ora.matmul_quant_f64(t, w, rows, cols, b)
        oc, _ = ora.matmul_quant_f64(t, w, rows, cols, 2.0 * a + b)   # power-of-two scaling is exact
        assert np.allclose(oc, 2.0 * oa + ob, rtol=1e-13, atol=1e-13 * np.max(np.abs(oc)))


# ----------------------------------------------------------------------------- attention


def _np_attention(q, kc, vc, max_seq, nh, nkv, d, pos0, seq):
    """numpy float64 restatement used only to pin the C oracle."""
    k = kc.view(np.float16).astype(np.float64).reshape(nkv, max_seq, d)
    v = vc.view(np.float16).astype(np.float64).reshape(nkv, max_seq, d)
    qq = q.astype(np.float64).reshape(seq, nh, d)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(d)))
    out = np.zeros((seq, nh, d))
    for t in range(seq):
        for h in range(nh):
            kh = h // (nh // nkv)
            s = (k[kh, :pos0 + t + 1] @ qq[t, h]) * scale
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v[kh, :pos0 + t + 1]
    return out


def _cache(rng, nkv, max_seq, d, scale=1.0):
    return (rng.normal(0, scale, (nkv, max_seq, d)).astype(np.float16).view(np.uint16))


def test_attention_f64_vs_numpy(ora):
    rng = np.random.default_rng(900)
    nh, nkv, d, max_seq, pos0, seq = 4, 2, 16, 40, 7, 5
    q = rng.normal(0, 1, (seq, nh, d)).astype(np.float32)
    kc, vc = _cache(rng, nkv, max_seq, d), _cache(rng, nkv, max_seq, d)
    out, smag, vmax = ora.attention_f64(q, kc, vc, max_seq, nh, nkv, d, pos0, seq)
    assert np.allclose(out, _np_attention(q, kc, vc, max_seq, nh, nkv, d, pos0, seq), rtol=1e-12, atol=1e-12)
    vv = vc.view(np.float16).astype(np.float64).reshape(nkv, max_seq, d)
    for t in range(seq):
        for h in range(nh):
            assert vmax[t, h] == np.max(np.abs(vv[h // 2, :pos0 + t + 1]))
            assert smag[t, h] > 0


def test_attention_f64_closed_forms_and_causality(ora):
    rng = np.random.default_rng(901)
    nh, nkv, d, max_seq, pos0, seq = 2, 1, 8, 20, 3, 4
    q = rng.normal(0, 1, (seq, nh, d)).astype(np.float32)
    # equal keys: uniform weights, the output is the mean of the visible v rows
    kc = np.tile(_cache(rng, 1, 1, d), (1, max_seq, 1))
    vc = _cache(rng, nkv, max_seq, d)
    out, _, _ = ora.attention_f64(q, kc, vc, max_seq, nh, nkv, d, pos0, seq)
    vv = vc.view(np.float16).astype(np.float64).reshape(max_seq, d)
    for t in range(seq):
        assert np.allclose(out[t], vv[:pos0 + t + 1].mean(axis=0), rtol=1e-12, atol=1e-12)
    # a dominant score selects its v row
    kc2 = np.zeros((1, max_seq, d), np.float16)
    kc2[0, 2, 0] = 60.0
    q2 = np.zeros((seq, nh, d), np.float32)
    q2[..., 0] = 60.0
    out2, _, _ = ora.attention_f64(q2, kc2.view(np.uint16), vc, max_seq, nh, nkv, d, pos0, seq)
    assert np.allclose(out2, np.broadcast_to(vv[2], out2.shape), rtol=1e-9, atol=1e-9)
    # rows past pos0 + t never matter
    vc3 = vc.copy().reshape(max_seq, d)
    vc3[pos0 + seq:] = np.float16(1000.0).view(np.uint16)
    out3, _, _ = ora.attention_f64(q, kc, vc3, max_seq, nh, nkv, d, pos0, seq)
    assert np.array_equal(out3, out)


# ----------------------------------------------------------------------------- RMSNorm


def test_rms_norm_constant_rows_closed_form(ora):
    n = 2048
    cs = np.array([1.0, -3.5, 1e-3, 250.0], np.float32)
    x = np.repeat(cs[:, None], n, axis=1)
    w = synth.normal(np.random.default_rng(6), n, 1.0, 0.1)
    out = ora.rms_norm(x, w, 4, n, n, 1e-6)
    c = cs.astype(np.float64)[:, None]
    want = w.astype(np.float64)[None, :] * c / np.sqrt(c * c + 1e-6)
    assert within(out, want, rtol=3e-7, atol=0)


def test_rms_norm_invariants_and_f64(ora):
    rng = np.random.default_rng(7)
    rows, n = 21, 2048
    x = synth.normal(rng, (rows, n))
    ones = np.ones(n, np.float32)
    out = ora.rms_norm(x, ones, rows, n, n, 1e-6)
    rms = np.sqrt(np.mean(out.astype(np.float64) ** 2, axis=1))
    assert np.all(np.abs(rms - 1.0) < 1e-5)
    scaled = ora.rms_norm(x * np.float32(8.0), ones, rows, n, n, 1e-6)
    assert within(scaled, out, rtol=1e-5)
    w = synth.normal(rng, n, 1.0, 0.1)
    got = ora.rms_norm(x, w, rows, n, n, 1e-6)
    xd = x.astype(np.float64)
    want = xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-6) * w.astype(np.float64)
    assert within(got, want)
    assert within(ora.rms_norm_f64(x, w, rows, n, n, 1e-6), want, rtol=1e-13, atol=0)


def test_rms_norm_strided_rows_and_inplace_semantics(ora):
    rng = np.random.default_rng(8)
    rows, n, stride = 5, 100, 130
    x = synth.normal(rng, rows * stride)
    w = synth.normal(rng, n, 1.0, 0.1)
    out = ora.rms_norm(x, w, rows, n, stride, 1e-6)
    for r in range(rows):
        xr = x[r * stride:r * stride + n].astype(np.float64)
        want = xr / np.sqrt(np.mean(xr * xr) + 1e-6) * w
        assert within(out[r * stride:r * stride + n], want)
        assert np.array_equal(out[r * stride + n:(r + 1) * stride], x[r * stride + n:(r + 1) * stride])


# ----------------------------------------------------------------------------- RoPE


def test_rope_table_vs_numpy(ora):
    n_pos, d = 4096, 128
    tab = ora.build_rope_table(d, 1e6, n_pos)
    i = np.arange(d // 2, dtype=np.float64)
    inv = 1.0 / np.power(1e6, 2 * i / d)
    ang = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None, :]
    want = np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)
    ulp = np.abs(tab.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert np.mean(ulp == 0) > 0.9999
    assert np.all(tab[0, :64] == 1.0) and np.all(tab[0, 64:] == 0.0)


def test_rope_identity_norm_and_complex_form(ora):
    rng = np.random.default_rng(9)
    rows, heads, d = 21, 16, 128
    tab = ora.build_rope_table(d, 1e6, 64)
    x = synth.normal(rng, rows * heads * d)
    ident = ora.rope(x[: heads * d], heads, d, tab, 0, 1)
    assert np.array_equal(ident, x[: heads * d])                           # position 0: identity
    out = ora.rope(x, heads, d, tab, 7, rows).reshape(rows, heads, d).astype(np.float64)
    xin = x.reshape(rows, heads, d).astype(np.float64)
    # pair norms preserved
    n_in = np.hypot(xin[..., :64], xin[..., 64:])
    n_out = np.hypot(out[..., :64], out[..., 64:])
    assert within(n_out, n_in, rtol=1e-6, atol=1e-6)
    # complex form: (x_i + j x_{i+64}) * (c + j s) with the table's own c, s
    c = tab[7:7 + rows, :64].astype(np.float64)[:, None, :]
    s = tab[7:7 + rows, 64:].astype(np.float64)[:, None, :]
    z = (xin[..., :64] + 1j * xin[..., 64:]) * (c + 1j * s)
    assert within(out[..., :64], z.real) and within(out[..., 64:], z.imag)
    assert within(ora.rope_f64(x, heads, d, tab, 7, rows).reshape(rows, heads, d)[..., :64], z.real,
                  rtol=1e-14, atol=1e-15)


# ----------------------------------------------------------------------------- KV write


def test_kv_write_reference_kat(ora):
    """tools/kv_map_check.cu:51-186: value h*100 + t*10 + d (V: +1000), 3 heads x dim 8,
    capacity 12, positions [4, 9); every untouched slot stays 0."""
    heads, dim, max_seq, pos0, seq = 3, 8, 12, 4, 5
    t, h, d = np.meshgrid(np.arange(seq), np.arange(heads), np.arange(dim), indexing="ij")
    k = (h * 100 + t * 10 + d).astype(np.float32)
    v = k + np.float32(1000)
    kc = np.zeros(heads * max_seq * dim, np.uint16)
    vc = np.zeros_like(kc)
    assert ora.kv_write(k, v, heads, dim, pos0, seq, kc, vc, max_seq) == 0
    kc3 = kc.reshape(heads, max_seq, dim).view(np.float16).astype(np.float32)
    vc3 = vc.reshape(heads, max_seq, dim).view(np.float16).astype(np.float32)
    for hh in range(heads):
        for tt in range(seq):
            for dd in range(dim):
                assert kc3[hh, pos0 + tt, dd] == hh * 100 + tt * 10 + dd
                assert vc3[hh, pos0 + tt, dd] == hh * 100 + tt * 10 + dd + 1000
    untouched = np.ones(max_seq, bool)
    untouched[pos0:pos0 + seq] = False
    assert np.all(kc.reshape(heads, max_seq, dim)[:, untouched] == 0)
    assert np.all(vc.reshape(heads, max_seq, dim)[:, untouched] == 0)
    assert ora.kv_write(k, v, heads, dim, 8, seq, kc, vc, max_seq) == -1   # 8 + 5 > 12
    assert ora.kv_write(k, v, heads, dim, -1, seq, kc, vc, max_seq) == -1


def test_kv_write_rounding_is_rne(ora):
    rng = np.random.default_rng(10)
    heads, dim, max_seq, seq = 8, 128, 64, 50
    k = synth.normal(rng, (seq, heads, dim))
    v = synth.normal(rng, (seq, heads, dim))
    kc = np.zeros(heads * max_seq * dim, np.uint16)
    vc = np.zeros_like(kc)
    assert ora.kv_write(k, v, heads, dim, 3, seq, kc, vc, max_seq) == 0
    want_k = k.astype(np.float16).view(np.uint16).transpose(1, 0, 2)
    assert np.array_equal(kc.reshape(heads, max_seq, dim)[:, 3:3 + seq], want_k)


# ----------------------------------------------------------------------------- SwiGLU / add


def test_silu_mul_special_values_and_f64(ora):
    g = np.array([0.0, -0.0, -100.0, -1e30, 30.0, 88.0, 1.0, -1.0], np.float32)
    u = np.array([3.0, 3.0, 2.0, 2.0, 1.5, 1.0, 1.0, 1.0], np.float32)
    out = ora.silu_mul(g, u)
    assert out[0] == 0.0 and out[1] == 0.0
    assert out[2] == 0.0 and np.signbit(out[2]) and out[3] == 0.0       # v -> -inf gives -0
    assert out[4] == np.float32(45.0) and out[5] == np.float32(88.0)   # v >> 0 gives v * up
    assert within(out[6:], [1 / (1 + math.exp(-1)), -1 / (1 + math.exp(1))], rtol=2e-7, atol=0)
    rng = np.random.default_rng(11)
    gate = synth.normal(rng, 100000, 0.0, 2.0)
    up = synth.normal(rng, 100000, 0.0, 2.0)
    gd = gate.astype(np.float64)
    want = gd / (1 + np.exp(-gd)) * up
    assert within(ora.silu_mul(gate, up), want)
    assert within(ora.silu_mul_f64(gate, up), want, rtol=1e-14, atol=1e-300)


def test_vec_add_bitwise(ora):
    rng = np.random.default_rng(12)
    a = synth.normal(rng, 10007)
    b = synth.normal(rng, 10007)
    assert np.array_equal(ora.vec_add(a, b).view(np.uint32), (a + b).view(np.uint32))


def test_fused_compositions_vs_f64(ora):
    rng = np.random.default_rng(13)
    n, H, Hq, Hkv, d = 21, 2048, 16, 8, 128
    x = synth.normal(rng, (n, H))
    dl = synth.normal(rng, (n, H))
    w = synth.normal(rng, H, 1.0, 0.1)
    xs, h = ora.add_rms_norm(x, dl, w, n, H, 1e-6)
    assert np.array_equal(xs, x + dl)
    xd = xs.astype(np.float64)
    assert within(h, xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-6) * w)
    tab = ora.build_rope_table(d, 1e6, 64)
    q = synth.normal(rng, (n, Hq, d))
    k = synth.normal(rng, (n, Hkv, d))
    v = synth.normal(rng, (n, Hkv, d))
    qn = synth.normal(rng, d, 1.0, 0.1)
    kn = synth.normal(rng, d, 1.0, 0.1)
    kc = np.zeros(Hkv * 64 * d, np.uint16)
    vc = np.zeros_like(kc)
    q2, k2 = ora.qk_norm_rope_kv(q, k, v, qn, kn, Hq, Hkv, d, tab, 5, n, 1e-6, kc, vc, 64)
    assert within(q2.reshape(-1), ora.norm_rope_f64(q, qn, Hq, d, tab, 5, n, 1e-6))
    assert within(k2.reshape(-1), ora.norm_rope_f64(k, kn, Hkv, d, tab, 5, n, 1e-6))
    kc3 = kc.reshape(Hkv, 64, d)
    assert np.array_equal(kc3[:, 5:5 + n], k2.astype(np.float16).view(np.uint16).transpose(1, 0, 2))
