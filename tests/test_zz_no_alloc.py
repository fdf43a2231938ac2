"""The no-allocation attention entry point (rpg_op_attention_from_cache_noalloc)
against the allocating one (rpg_op_attention_from_cache), through the C ABI.

Both run the same kernels; only where the split-key partials live differs (a
fixed device array of the library instead of its grow-only buffer), so the
outputs must be identical bit for bit. Two calls in a row, the second smaller,
show that what the first call left in the shared array does not leak into the
second; a third, too large for the array, must fail before launching anything.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(name: str) -> None:
    print(f"\n[case] {name}", flush=True)


def _inputs(rng, nh, nkv, max_seq, seq):
    q = rng.normal(0, 1, (seq, nh, 128)).astype(np.float32)
    kc = rng.normal(0, 1, (nkv, max_seq, 128)).astype(np.float16).view(np.uint16)
    vc = rng.normal(0, 1, (nkv, max_seq, 128)).astype(np.float16).view(np.uint16)
    return q, kc, vc


def _run(lib, fn, nh, nkv, pos0, seq, q, kc, vc, max_seq, out):
    rc = fn(ctypes.c_void_p(q.data_ptr()), nh, nkv, 128, pos0, seq, ctypes.c_void_p(kc.data_ptr()),
            ctypes.c_void_p(vc.data_ptr()), max_seq, ctypes.c_void_p(out.data_ptr()), -1)
    return rc


def test_noalloc_attention_matches_allocating_entry(gpu):
    import torch

    lib = gpu.load_library()
    rng = np.random.default_rng(77)
    # (name, n_heads, n_kv_heads, max_seq, pos0, seq): the first call splits the
    # keys into the most chunks, the second is smaller; both use the scratch.
    # A split decode is one launch whose last workgroup per (token, kv head) merges.
    calls = [("4B shape, decode at 4095, 2 tokens (32 workgroups per pair)", 32, 8, 4096, 4094, 2),
             ("1.7B shape, decode at 3000 (24 workgroups per pair)", 16, 8, 3072, 3000, 1),
             ("1.7B shape, decode at 700", 16, 8, 4096, 700, 1),
             ("prefill of 100 tokens at 1900, 4 key chunks merged in the launch", 4, 2, 2048, 1900, 100)]
    for name, nh, nkv, max_seq, pos0, seq in calls:
        _case(f"noalloc vs allocating: {name}")
        q, kc, vc = _inputs(rng, nh, nkv, max_seq, seq)
        qd = torch.from_numpy(q).cuda()
        kd = torch.from_numpy(kc.view(np.int16)).cuda()
        vd = torch.from_numpy(vc.view(np.int16)).cuda()
        ref = torch.full((seq, nh, 128), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full_like(ref, float("nan"))
        assert _run(lib, lib.rpg_op_attention_from_cache, nh, nkv, pos0, seq, qd, kd, vd, max_seq, ref) == 0
        assert _run(lib, lib.rpg_op_attention_from_cache_noalloc, nh, nkv, pos0, seq, qd, kd, vd, max_seq,
                    got) == 0, lib.rpg_ops_last_error()
        torch.cuda.synchronize()
        a = ref.cpu().numpy()
        b = got.cpu().numpy()
        assert np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name}: outputs differ"


def test_noalloc_attention_rejects_oversized_split(gpu):
    import torch

    lib = gpu.load_library()
    _case("noalloc rejects a split beyond its fixed scratch")
    # GQA group 4 with 7 x 71 = 497 (token, kv head) pairs at 1007 positions: the
    # split takes 5 chunks, 2 workgroups per pair, 497 x 4 heads x 2 x 132 floats
    # = 524832 > 2^19.
    nh, nkv, max_seq, pos0, seq = 284, 71, 1024, 1000, 7
    q = torch.zeros((seq, nh, 128), dtype=torch.float32, device="cuda")
    kc = torch.zeros((nkv, max_seq, 128), dtype=torch.int16, device="cuda")
    vc = torch.zeros_like(kc)
    out = torch.full((seq, nh, 128), 7.0, dtype=torch.float32, device="cuda")
    rc = _run(lib, lib.rpg_op_attention_from_cache_noalloc, nh, nkv, pos0, seq, q, kc, vc, max_seq, out)
    assert rc < 0
    msg = lib.rpg_ops_last_error().decode()
    assert "no-allocation" in msg and "scratch" in msg, msg
    torch.cuda.synchronize()
    assert bool(torch.all(out == 7.0)), "a rejected call must not launch"
    # the allocating entry point takes the same call
    assert _run(lib, lib.rpg_op_attention_from_cache, nh, nkv, pos0, seq, q, kc, vc, max_seq, out) == 0
    torch.cuda.synchronize()


def _group_partials_floats(units, group, positions):
    """Partials floats of a grouped decode call: chunks of a multiple of 32 keys,
    enough for ~2048 waves over `units` (token, kv head) pairs, no split at >= 2048
    units or <= 128 positions; one launch whose workgroups take 4 chunks each and
    keep 132 floats per (token, query head, workgroup), none when one workgroup
    takes every chunk."""
    if units >= 2048 or positions <= 128:
        return 0
    want = min((2048 + units - 1) // units, 128)
    length = ((positions + want - 1) // want + 31) // 32 * 32
    chunks = (positions + length - 1) // length
    groups = (chunks + 3) // 4
    return units * group * groups * 132 if groups > 1 else 0


def test_noalloc_attention_group4_boundary(gpu):
    """GQA group 4 split 5 ways (2 workgroups per pair): 16 x 31 = 496 (token, kv
    head) pairs fit the 2^19-float scratch and match the allocating entry bit for
    bit; 7 x 71 = 497 pairs are rejected unlaunched; the same 497 pairs at 107
    positions (no split) need no partials and go through."""
    import torch

    lib = gpu.load_library()
    max_seq, pos0 = 1024, 1000
    # (seq, n_kv_heads)
    fits, over = (16, 31), (7, 71)
    assert _group_partials_floats(fits[0] * fits[1], 4, pos0 + fits[0]) == 496 * 1056 <= 1 << 19
    assert _group_partials_floats(over[0] * over[1], 4, pos0 + over[0]) == 497 * 1056 > 1 << 19
    assert _group_partials_floats(over[0] * over[1], 4, 100 + over[0]) == 0

    def inputs(seq, nh, nkv, seed):
        gen = torch.Generator(device="cuda").manual_seed(seed)
        q = torch.randn((seq, nh, 128), generator=gen, device="cuda")
        kc = torch.randn((nkv, max_seq, 128), generator=gen, device="cuda").half().view(torch.int16)
        vc = torch.randn((nkv, max_seq, 128), generator=gen, device="cuda").half().view(torch.int16)
        return q, kc, vc

    def both_equal(seq, nh, nkv, p0, q, kc, vc):
        ref = torch.full((seq, nh, 128), float("nan"), dtype=torch.float32, device="cuda")
        got = torch.full_like(ref, float("nan"))
        assert _run(lib, lib.rpg_op_attention_from_cache, nh, nkv, p0, seq, q, kc, vc, max_seq, ref) == 0
        assert _run(lib, lib.rpg_op_attention_from_cache_noalloc, nh, nkv, p0, seq, q, kc, vc, max_seq,
                    got) == 0, lib.rpg_ops_last_error()
        torch.cuda.synchronize()
        assert bool(torch.all(torch.isfinite(ref)))
        assert torch.equal(ref.view(torch.int32), got.view(torch.int32))

    seq, nkv = fits
    nh = 4 * nkv
    _case(f"noalloc group-4 boundary: seq {seq}, {nh}/{nkv} heads, 496 pairs at {pos0} (fits)")
    both_equal(seq, nh, nkv, pos0, *inputs(seq, nh, nkv, 78))

    seq, nkv = over
    nh = 4 * nkv
    _case(f"noalloc group-4 boundary: seq {seq}, {nh}/{nkv} heads, 497 pairs at {pos0} (rejected)")
    q, kc, vc = inputs(seq, nh, nkv, 79)
    out = torch.full((seq, nh, 128), 7.0, dtype=torch.float32, device="cuda")
    rc = _run(lib, lib.rpg_op_attention_from_cache_noalloc, nh, nkv, pos0, seq, q, kc, vc, max_seq, out)
    assert rc < 0
    assert "no-allocation" in lib.rpg_ops_last_error().decode()
    torch.cuda.synchronize()
    assert bool(torch.all(out == 7.0)), "a rejected call must not launch"

    _case(f"noalloc group-4: seq {seq}, {nh}/{nkv} heads, 497 pairs at 100 (no split, accepted)")
    both_equal(seq, nh, nkv, 100, q, kc, vc)
