"""Pins for the CPU oracle (no GPU).

The oracle is only trusted because these checks hold.  Each pins a function
against something other than a retyping of its own formula: the reference's
own known-answer test, an independent library routine (torch's ops and
float8_e4m3fn cast), brute force, and closed forms / invariants chosen so a
dropped term, a wrong sign or index, or a transposed operand fails.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attn_oracle as AO
from oracle import kv_oracle as KO


# ----------------------------------------------------------------- store KAT
def test_store_kat_reference():
    """pd_self/evaluation/test_kv_cache_dtype_matrix.py:61-82: Hkv=8, D=16,
    one token of ones (bf16) and twos, slot 0, fp16 cache."""
    kc = np.zeros((1, 256, 8, 16), dtype=np.float16)
    vc = np.zeros_like(kc)
    k = np.ones((1, 8, 16), dtype=np.float32)
    v = np.full((1, 8, 16), 2.0, dtype=np.float32)
    KO.store_kvcache(k, v, [0], kc, vc, 256, cast=lambda x: x.astype(np.float16))
    assert kc.dtype == np.float16
    assert np.all(kc[0, 0] == 1.0) and np.all(vc[0, 0] == 2.0)
    assert np.all(kc[0, 1:] == 0) and np.all(vc[0, 1:] == 0)


def test_store_slot_mapping_block_offset():
    """block = slot // bs, offset = slot % bs; untouched slots stay; negative
    slots are skipped."""
    bs = 4
    kc = np.zeros((3, bs, 1, 2), dtype=np.float32)
    vc = np.zeros_like(kc)
    k = np.arange(8, dtype=np.float32).reshape(4, 1, 2) + 1
    slots = [5, 2, -1, 11]
    KO.store_kvcache(k, -k, slots, kc, vc, bs, cast=lambda x: x)
    assert np.all(kc[1, 1, 0] == [1, 2])
    assert np.all(kc[0, 2, 0] == [3, 4])
    assert np.all(kc[2, 3, 0] == [7, 8])
    assert np.all(vc[2, 3, 0] == [-7, -8])
    assert np.count_nonzero(kc) == 6


# ----------------------------------------------------------------- int8 quant
def _torch_int8_reference(x32: torch.Tensor):
    # The exact tensor ops of attention.py:94-98, run by torch on the CPU.
    absmax = x32.abs().amax(dim=-1, keepdim=True)
    scale = (absmax / 127.0).clamp(min=1e-6)
    q = torch.round(x32 / scale).clamp(-127, 127).to(torch.int8)
    return q, scale


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_int8_matches_torch_ops(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(257, 8, 128, generator=g)
    x = torch.where(torch.rand(x.shape, generator=g) < 0.01, x * 8, x).to(torch.bfloat16).float()
    qo, so = KO.quantize_int8_per_token(x.numpy())
    qt, st = _torch_int8_reference(x)
    assert np.array_equal(qo, qt.numpy())
    assert np.array_equal(so.view(np.uint32), st.numpy().view(np.uint32))


def test_int8_special_cases():
    x = np.zeros((4, 1, 8), dtype=np.float32)
    # row 0: all zero -> scale 1e-6, codes 0
    # row 1: exact ties after dividing by scale 1.0 (absmax 127)
    x[1, 0] = [127, 2.5, -2.5, 3.5, 0.5, -0.5, 1.5, -126.5]
    # row 2: absmax element maps to +-127
    x[2, 0] = [-3.0, 1.0, 0.25, 0, 0, 0, 0, 2.0]
    # row 3: tiny values below the scale floor
    x[3, 0] = [1e-9, -1e-9, 0, 0, 0, 0, 0, 5e-8]
    q, s = KO.quantize_int8_per_token(x)
    assert s[0, 0, 0] == np.float32(1e-6) and np.all(q[0] == 0)
    assert s[1, 0, 0] == 1.0
    assert list(q[1, 0]) == [127, 2, -2, 4, 0, 0, 2, -126]  # half to even
    assert q[2, 0, 0] == -127 and q[2, 0, 7] == round(2.0 / (3.0 / 127))
    assert s[3, 0, 0] == np.float32(1e-6)
    assert list(q[3, 0]) == [0, 0, 0, 0, 0, 0, 0, 0]


# ----------------------------------------------------------------- fp8 e4m3
def test_e4m3_decode_all_codes_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = KO.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert list(np.nonzero(nan)[0]) == [0x7F, 0xFF]
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def _encode_inputs():
    vals = KO.e4m3_decode(np.arange(256, dtype=np.uint8))
    finite = np.sort(np.unique(vals[np.isfinite(vals)]))
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    around = np.concatenate([mids, np.nextafter(mids, np.float32(-np.inf)), np.nextafter(mids, np.float32(np.inf))])
    bf = KO.bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    bf = bf[np.isfinite(bf) & (np.abs(bf) <= 448)]
    rnd = np.random.default_rng(0).uniform(-448, 448, 200000).astype(np.float32)
    tiny = np.random.default_rng(1).uniform(-2 ** -5, 2 ** -5, 100000).astype(np.float32)
    return np.concatenate([finite, around, bf, rnd, tiny, np.float32([0.0, -0.0, 448.0, -448.0])])


def test_e4m3_encode_vs_torch_cast():
    x = _encode_inputs()
    ours = KO.e4m3_encode(x)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bad = np.nonzero(ours != ref)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={x[bad[:5]]} ours={ours[bad[:5]]} torch={ref[bad[:5]]}"


def test_e4m3_encode_brute_force_nearest_even():
    codes = np.arange(256, dtype=np.uint8)
    vals = KO.e4m3_decode(codes).astype(np.float64)
    ok = np.isfinite(vals)
    x = np.random.default_rng(2).uniform(-448, 448, 4000).astype(np.float32)
    x = np.concatenate([x, ((vals[ok][:-1] + vals[ok][1:]) / 2).astype(np.float32)])
    enc = KO.e4m3_encode(x)
    for xi, ci in zip(x, enc):
        d = np.abs(vals - float(xi))
        d[~ok] = np.inf
        best = np.nonzero(d == d.min())[0]
        # among equally near codes pick the one with an even mantissa; at +-0
        # the sign of x decides
        cand = [c for c in best if (c & 1) == 0] or list(best)
        if float(xi) == 0.0:
            cand = [0x80 if math.copysign(1.0, float(xi)) < 0 else 0x00]
        elif len(cand) > 1:
            cand = [c for c in cand if (c >> 7) == (1 if xi < 0 else 0)]
        assert ci == cand[0], (xi, ci, cand)


def test_fp8_quant_absmax_maps_to_448():
    x = np.random.default_rng(3).normal(size=(64, 8, 128)).astype(np.float32)
    q, s = KO.quantize_fp8_per_token(x)
    idx = np.abs(x).argmax(-1)
    top = np.take_along_axis(q, idx[..., None], -1)[..., 0]
    assert np.all((top & 0x7F) == 0x7E)
    deq = KO.dequantize_per_token(q, s, "fp8")
    # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 of the value's binade
    assert np.all(np.abs(deq - x) <= np.abs(x) * 2.0 ** -4 + s[..., 0:1] * 2.0 ** -9 + 1e-12)


# ----------------------------------------------------------------- gather
def test_gather_compacts_truncates_pads():
    bs, h, d = 2, 1, 1
    vals = np.arange(10, dtype=np.float32).reshape(5, bs, h, d)  # block b holds 2b, 2b+1
    bt = np.array([[3, -1, 1, -1], [4, -1, -1, -1], [-1, -1, -1, -1]])
    lens = [3, 1, 2]
    kb, vb, mask = KO.get_kv_cache(vals, -vals, bt, lens)
    assert kb.shape == (3, 3, 1, 1)
    assert list(kb[0, :, 0, 0]) == [6, 7, 2]  # blocks 3 then 1, cut to 3
    assert list(kb[1, :, 0, 0]) == [8, 0, 0]
    assert list(kb[2, :, 0, 0]) == [0, 0, 0]  # no valid block: skipped
    assert mask.tolist() == [[True, True, True], [True, False, False], [False, False, False]]
    assert np.array_equal(vb, -kb)


def test_gather_hole_compacts_like_reference():
    """A -1 inside a row's k_len (input the engine never builds: it pads -1
    only at the tail, model_runner.py:334-344).  The reference's gather keeps
    row[row != -1] (attention.py:255-275), so the keys of later blocks move
    left into the hole; the HIP kernels instead read the hole as zero K/V at
    its logical positions.  Both conventions, side by side."""
    bs, h, d = 2, 1, 1
    vals = np.arange(1, 11, dtype=np.float32).reshape(5, bs, h, d)  # block b holds 2b+1, 2b+2
    bt = np.array([[2, -1, 4, 0]])  # hole at logical block 1
    kb, _, mask = KO.get_kv_cache(vals, vals, bt, [5])
    assert list(kb[0, :, 0, 0]) == [5, 6, 9, 10, 1]  # blocks 2, 4, 0: compacted
    assert mask.tolist() == [[True] * 5]
    # the kernels' convention for the same row: logical block j at keys 2j, 2j+1
    zero_read = [5, 6, 0, 0, 9]
    assert list(kb[0, :, 0, 0]) != zero_read
    # torch's semantics the reference relies on: row[row != -1] drops only -1,
    # and a negative slot wraps (slot // bs, slot % bs: -1 -> last row of block -1)
    row = torch.tensor([2, -1, 4, -2])
    assert row[row != -1].tolist() == [2, 4, -2]
    slot = torch.tensor([-1])
    assert (slot // 256).item() == -1 and (slot % 256).item() == 255


# ----------------------------------------------------------------- attention
def _brute(q, k, v, cu_q, cu_k, Hq, Hkv):
    """float64 loops straight from the definition."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    g = Hq // Hkv
    D = q.shape[-1]
    out = np.zeros_like(q)
    for i in range(len(cu_q) - 1):
        L = cu_q[i + 1] - cu_q[i]
        K = cu_k[i + 1] - cu_k[i]
        for r in range(L):
            for h in range(Hq):
                kh = h // g
                lim = r + K - L
                sc = [sum(q[cu_q[i] + r, h, e] * k[cu_k[i] + j, kh, e] for e in range(D)) / math.sqrt(D)
                      for j in range(lim + 1)]
                if not sc:
                    continue
                m = max(sc)
                w = [math.exp(s - m) for s in sc]
                z = sum(w)
                for e in range(D):
                    out[cu_q[i] + r, h, e] = sum(w[j] * v[cu_k[i] + j, kh, e] for j in range(lim + 1)) / z
    return out


def _rand(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed))


def test_attention_cached_brute_force():
    Hq, Hkv, D = 4, 2, 8
    qlens, klens = [3, 1, 4], [5, 4, 4]
    cu_q = np.concatenate([[0], np.cumsum(qlens)]).tolist()
    cu_k = np.concatenate([[0], np.cumsum(klens)]).tolist()
    q = _rand((cu_q[-1], Hq, D), 0)
    kflat = _rand((cu_k[-1], Hkv, D), 1)
    vflat = _rand((cu_k[-1], Hkv, D), 2)
    B, M = len(qlens), max(klens)
    kb = torch.zeros(B, M, Hkv, D)
    vb = torch.zeros(B, M, Hkv, D)
    for i in range(B):
        kb[i, : klens[i]] = kflat[cu_k[i]:cu_k[i + 1]]
        vb[i, : klens[i]] = vflat[cu_k[i]:cu_k[i + 1]]
    got = AO.attention_cached(q, kb, vb, cu_q, cu_k, Hq, Hkv, D).numpy()
    ref = _brute(q.numpy(), kflat.numpy(), vflat.numpy(), cu_q, cu_k, Hq, Hkv)
    assert np.abs(got - ref).max() < 1e-5


def test_attention_local_brute_force():
    Hq, Hkv, D = 6, 3, 8
    lens = [4, 1, 3]
    cu = np.concatenate([[0], np.cumsum(lens)]).tolist()
    q, k, v = _rand((cu[-1], Hq, D), 3), _rand((cu[-1], Hkv, D), 4), _rand((cu[-1], Hkv, D), 5)
    got = AO.attention_local(q, k, v, cu, Hq, Hkv, D).numpy()
    ref = _brute(q.numpy(), k.numpy(), v.numpy(), cu, cu, Hq, Hkv)
    assert np.abs(got - ref).max() < 1e-5


def test_attention_closed_forms():
    Hq, Hkv, D = 2, 1, 4
    v = _rand((6, Hkv, D), 6)
    # identical keys -> uniform weights -> mean of the visible values
    k = torch.ones(6, Hkv, D)
    q = _rand((2, Hq, D), 7)
    out = AO.attention_cached(q, k[None], v[None], [0, 2], [0, 6], Hq, Hkv, D)
    assert torch.allclose(out[0, 0], v[:5, 0].mean(0), atol=1e-6)
    assert torch.allclose(out[1, 1], v[:6, 0].mean(0), atol=1e-6)
    # a single visible key -> its value
    out1 = AO.attention_local(q[:1], k[:1], v[:1], [0, 1], Hq, Hkv, D)
    assert torch.allclose(out1[0, 0], v[0, 0]) and torch.allclose(out1[0, 1], v[0, 0])
    # no visible key (q_len > k_len) -> 0
    out2 = AO.attention_cached(q, k[None, :1], v[None, :1], [0, 2], [0, 1], Hq, Hkv, D)
    assert torch.all(out2[0] == 0) and torch.allclose(out2[1, 0], v[0, 0])


def test_prefix_plus_suffix_equals_fresh_and_decode_row():
    Hq, Hkv, D, n, p = 4, 2, 16, 9, 5
    q, k, v = _rand((n, Hq, D), 8), _rand((n, Hkv, D), 9), _rand((n, Hkv, D), 10)
    fresh = AO.attention_local(q, k, v, [0, n], Hq, Hkv, D)
    suffix = AO.attention_cached(q[p:], k[None], v[None], [0, n - p], [0, n], Hq, Hkv, D)
    assert torch.allclose(fresh[p:], suffix, atol=1e-6)
    last = AO.attention_cached(q[n - 1:], k[None], v[None], [0, 1], [0, n], Hq, Hkv, D)
    assert torch.allclose(fresh[n - 1:], last, atol=1e-6)


def test_paged_block_permutation_invariance():
    bs, Hq, Hkv, D = 4, 4, 2, 8
    lens = [7, 10]
    nb = 8
    kv = _rand((nb, bs, Hkv, D), 11).numpy()
    vv = _rand((nb, bs, Hkv, D), 12).numpy()
    bt = np.array([[0, 1, -1], [2, 3, 4]])
    q = _rand((2, Hq, D), 13)
    cu_q, cu_k = [0, 1, 2], [0, 7, 17]
    base = AO.paged_attention(q, kv, vv, bt, cu_q, cu_k, lens, Hq, Hkv, D)
    perm = np.random.default_rng(0).permutation(nb)
    inv = np.argsort(perm)
    kv2, vv2 = kv[perm], vv[perm]  # block b now lives at inv[b]
    bt2 = np.where(bt >= 0, inv[np.maximum(bt, 0)], -1)
    moved = AO.paged_attention(q, kv2, vv2, bt2, cu_q, cu_k, lens, Hq, Hkv, D)
    assert torch.equal(base, moved)
