"""KV-cache write, per-token quantisation, dequantisation and the paged
gather on the GPU, bit-exact against the CPU oracle."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import PagedAttention
from oracle import kv_oracle as KO
from tests.gpu_util import bf16_to_np, say

pytestmark = pytest.mark.gpu

NVS_NP = {torch.bfloat16: None, torch.float16: np.float16, torch.float32: np.float32}


def _src(shape, dtype, seed, outliers=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    if outliers:
        x = torch.where(torch.rand(shape, generator=g) < 0.01, x * 8, x)
    x = x.to(dtype)
    return x


def _f32(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype == torch.bfloat16:
        return bf16_to_np(t)
    return t.float().numpy()


def _layer(hkv, d, nb, bs, cache_dtype, mode, device):
    a = PagedAttention(2 * hkv, hkv, d)
    a.block_size = bs
    a.kv_cache_quant_mode = mode
    a.k_cache = torch.zeros(nb, bs, hkv, d, dtype=cache_dtype, device=device)
    a.v_cache = torch.zeros_like(a.k_cache)
    if mode != "none":
        a.k_scale_cache = torch.ones(nb, bs, hkv, 1, dtype=torch.float32, device=device)
        a.v_scale_cache = torch.ones_like(a.k_scale_cache)
    return a


def test_store_kat_reference(device):
    """pd_self/evaluation/test_kv_cache_dtype_matrix.py:61-82 on the GPU."""
    say("store KAT fp16 cache")
    a = PagedAttention(num_heads=8, num_kv_heads=8, head_dim=16)
    a.block_size = 256
    a.k_cache = torch.zeros(1, 256, 8, 16, dtype=torch.float16, device=device)
    a.v_cache = torch.zeros_like(a.k_cache)
    k = torch.ones(1, 8, 16, dtype=torch.bfloat16, device=device)
    v = torch.ones(1, 8, 16, dtype=torch.bfloat16, device=device) * 2
    a.store_kv_cache_torch(k, v, torch.tensor([0], dtype=torch.int32, device=device))
    torch.cuda.synchronize()
    assert a.k_cache.dtype == torch.float16
    assert torch.allclose(a.k_cache[0, 0].float(), k[0].float())
    assert torch.allclose(a.v_cache[0, 0].float(), v[0].float())
    assert torch.count_nonzero(a.k_cache[0, 1:]) == 0


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dst", [torch.bfloat16, torch.float16, torch.float32])
def test_store_cast_bit_exact(device, src, dst):
    say(f"store cast {src} -> {dst}")
    T, H, D, NB, bs = 300, 8, 128, 16, 256
    a = _layer(H, D, NB, bs, dst, "none", device)
    k = _src((T, H, D), src, 1)
    v = _src((T, H, D), src, 2)
    slots = torch.randperm(NB * bs, generator=torch.Generator().manual_seed(3))[:T].to(torch.int32)
    slots[7] = -1  # padding row: skipped
    a.store_kv_cache_torch(k.to(device), v.to(device), slots.to(device))
    torch.cuda.synchronize()
    ref_k = np.zeros(tuple(a.k_cache.shape), dtype=np.float32)
    ref_v = np.zeros_like(ref_k)

    def cast(x):
        if dst == torch.bfloat16:
            return KO.round_to_bf16(x)
        return x.astype(NVS_NP[dst]).astype(np.float32)

    KO.store_kvcache(_f32(k), _f32(v), slots.numpy(), ref_k, ref_v, bs, cast=cast)
    assert np.array_equal(_f32(a.k_cache), ref_k)
    assert np.array_equal(_f32(a.v_cache), ref_v)


def _wide_src(shape, dtype, seed):
    """Random finite values of the source dtype from its bit patterns: every
    exponent, subnormals and signed zeros included; each (token, head) row
    scaled by its own power of two so that row absmaxes span the range."""
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.float32:
        bits = torch.randint(-(1 << 31), 1 << 31, shape, generator=g, dtype=torch.int64).to(torch.int32)
        x = bits.view(torch.float32).clone()
    else:
        bits = torch.randint(0, 1 << 16, shape, generator=g, dtype=torch.int32).to(torch.int16)
        x = bits.view(dtype).float()
    x = torch.where(torch.isfinite(x), x, torch.zeros_like(x))
    lim = 6.0e4 if dtype == torch.float16 else 3.0e38
    x = x.clamp(-lim, lim)
    lo = -20 if dtype == torch.float16 else -40
    shift = torch.randint(lo, 1, shape[:-1] + (1,), generator=g).float()
    return (x * torch.exp2(shift)).to(dtype)


def _store_quant_case(device, mode, T=513, H=8, D=128, NB=8, bs=256, strided=False, seed=0,
                      src=torch.bfloat16, wide=False):
    cache_dtype = torch.int8 if mode == "int8_mock" else torch.float8_e4m3fn
    a = _layer(H, D, NB, bs, cache_dtype, mode, device)
    make = (lambda sh, sd: _wide_src(sh, src, sd)) if wide else (lambda sh, sd: _src(sh, src, sd))
    k = make((T, H, D), seed + 1)
    v = make((T, H, D), seed + 2)
    k[3] = 0  # all-zero rows -> scale 1e-6, codes 0
    v[5, 2] = torch.tensor([127.0, 2.5, -2.5, 3.5] + [0.0] * (D - 4))  # exact ties
    slots = torch.randperm(NB * bs, generator=torch.Generator().manual_seed(seed + 3))[:T].to(torch.int32)
    slots[11] = -5
    kd, vd = k.to(device), v.to(device)
    if strided:
        # k and v as views of a fused [T, (2 + 2) * H, D] buffer
        fused = torch.zeros(T, 4 * H, D, dtype=torch.bfloat16, device=device)
        fused[:, H:2 * H] = kd
        fused[:, 3 * H:] = vd
        kd, vd = fused[:, H:2 * H], fused[:, 3 * H:]
        assert not kd.is_contiguous()
    a.store_kv_cache_torch(kd, vd, slots.to(device))
    torch.cuda.synchronize()
    kind = "int8" if mode == "int8_mock" else "fp8"
    npdt = np.int8 if kind == "int8" else np.uint8
    ref_k = np.zeros(tuple(a.k_cache.shape), dtype=npdt)
    ref_v = np.zeros_like(ref_k)
    ref_ks = np.ones(tuple(a.k_scale_cache.shape), dtype=np.float32)
    ref_vs = np.ones_like(ref_ks)
    KO.store_kvcache(_f32(k), _f32(v), slots.numpy(), ref_k, ref_v, bs, mode=kind, k_scale=ref_ks, v_scale=ref_vs)
    got_k = a.k_cache.cpu().view(torch.uint8).numpy().view(npdt)
    got_v = a.v_cache.cpu().view(torch.uint8).numpy().view(npdt)
    assert np.array_equal(got_k, ref_k), f"k codes differ at {np.argwhere(got_k != ref_k)[:5]}"
    assert np.array_equal(got_v, ref_v), f"v codes differ at {np.argwhere(got_v != ref_v)[:5]}"
    assert np.array_equal(a.k_scale_cache.cpu().numpy().view(np.uint32), ref_ks.view(np.uint32))
    assert np.array_equal(a.v_scale_cache.cpu().numpy().view(np.uint32), ref_vs.view(np.uint32))


@pytest.mark.parametrize("mode", ["int8_mock", "fp8_e4m3"])
def test_store_quant_bit_exact(device, mode):
    say(f"store quant {mode}")
    _store_quant_case(device, mode)


@pytest.mark.parametrize("src", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("mode", ["int8_mock", "fp8_e4m3"])
def test_store_quant_wide_exponents(device, mode, src):
    """Rows of random bit patterns (every exponent, subnormals, signed
    zeros) at row scales from 2^-40 (fp16: 2^-20) up: the bf16 / fp16 sources take the
    reciprocal-and-correction quotient, fp32 sources the divide; the codes
    and scales are bit-exact against the oracle either way."""
    say(f"store quant wide exponents {mode} {src}")
    _store_quant_case(device, mode, T=1024, src=src, wide=True, seed=90)


@pytest.mark.parametrize("mode", ["int8_mock", "fp8_e4m3"])
def test_store_quant_strided_sources(device, mode):
    say(f"store quant strided {mode}")
    _store_quant_case(device, mode, T=130, strided=True, seed=10)


@pytest.mark.parametrize("mode", ["int8_mock", "fp8_e4m3"])
@pytest.mark.parametrize("D", [16, 64, 256])
def test_store_quant_head_dims(device, mode, D):
    say(f"store quant {mode} D={D}")
    _store_quant_case(device, mode, T=97, H=4, D=D, NB=2, bs=64, seed=20 + D)


def test_fp8_hardware_decode_matches_ocp_e4m3(device):
    """gfx950's fp8 conversion (used by the decode kernels) reads OCP e4m3:
    every code through nvs_dequantize_per_token with scale 1 equals the
    format's value."""
    say("fp8 decode all codes")
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).reshape(2, 1, 128)
    a = PagedAttention(1, 1, 128)
    a.attention_compute_dtype = torch.float32
    out = a.dequantize_int8_per_token(codes.to(device), torch.ones(2, 1, 1, device=device)).cpu().numpy()
    ref = KO.e4m3_decode(np.arange(256, dtype=np.uint8)).reshape(2, 1, 128)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(out), nan)
    assert np.array_equal(out[~nan], ref[~nan])


def _e4m3_probe_values() -> np.ndarray:
    """Every finite bf16 value in [-448, 448]; every midpoint between
    neighbouring e4m3 values (a tie: round to even), the f32 values on
    either side of it, and the same around 0 and the subnormal codes; f32
    subnormals and signed zeros."""
    bf = (np.arange(0x10000, dtype=np.uint32) << 16).view(np.float32)
    bf = bf[np.isfinite(bf) & (np.abs(bf) <= 448.0)]
    pos = np.unique(KO.e4m3_decode(np.arange(0x7F, dtype=np.uint8)))  # 0 .. 448
    mid = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    near = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9)),
                           np.float32([2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11, 1e-40, 1.4e-45, 0.0])])
    near = near[near <= 448.0]
    return np.concatenate([bf, near, -near]).astype(np.float32)


def test_fp8_encode_every_value(device):
    """The fp8 store's encoder on every value that decides a code: rows of
    128 whose first element is 448 have scale 448 / 448 = 1 exactly, so each
    other element's code is its own e4m3 rounding; the codes equal the
    oracle's round-to-nearest-even encoder (pinned against torch's cast)."""
    say("fp8 encode every value")
    vals = _e4m3_probe_values()
    per = 127
    n = (vals.size + per - 1) // per
    rows = np.zeros((n, 128), dtype=np.float32)
    rows[:, 0] = 448.0
    flat = np.zeros(n * per, dtype=np.float32)
    flat[:vals.size] = vals
    rows[:, 1:] = flat.reshape(n, per)
    x = torch.from_numpy(rows).reshape(n, 1, 128)
    a = PagedAttention(1, 1, 128)
    q, s = a.quantize_fp8_per_token(x.to(device))
    assert np.all(s.cpu().numpy() == 1.0)
    rq, rs = KO.quantize_fp8_per_token(rows.reshape(n, 1, 128))
    assert np.all(rs == 1.0)
    got = q.cpu().view(torch.uint8).numpy().reshape(n, 128)
    want = rq.view(np.uint8).reshape(n, 128)
    bad = np.argwhere(got != want)
    assert bad.size == 0, (f"{len(bad)} codes differ, e.g. value {rows[tuple(bad[0])]!r}: "
                           f"got {got[tuple(bad[0])]:#04x}, want {want[tuple(bad[0])]:#04x}")


@pytest.mark.parametrize("kind", ["int8", "fp8"])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_quantize_dequantize_entry_points(device, kind, out_dtype):
    say(f"quantize/dequantize {kind} -> {out_dtype}")
    x = _src((77, 8, 128), torch.bfloat16, 30)
    a = PagedAttention(8, 8, 128)
    a.attention_compute_dtype = out_dtype
    q, s = a.quantize_int8_per_token(x.to(device)) if kind == "int8" else a.quantize_fp8_per_token(x.to(device))
    rq, rs = (KO.quantize_int8_per_token if kind == "int8" else KO.quantize_fp8_per_token)(_f32(x))
    qn = q.cpu().view(torch.uint8).numpy()
    assert np.array_equal(qn, rq.view(np.uint8))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))
    d = a.dequantize_int8_per_token(q, s)
    assert d.dtype == out_dtype
    ref = KO.dequantize_per_token(rq, rs, kind)
    if out_dtype == torch.bfloat16:
        ref = KO.round_to_bf16(ref)
    elif out_dtype == torch.float16:
        ref = ref.astype(np.float16).astype(np.float32)
    assert np.array_equal(_f32(d), ref)


@pytest.mark.parametrize("mode", ["none", "int8_mock", "fp8_e4m3"])
def test_gather_matches_oracle(device, mode):
    say(f"gather {mode}")
    H, D, NB, bs = 4, 128, 12, 64
    cache_dtype = {"none": torch.bfloat16, "int8_mock": torch.int8, "fp8_e4m3": torch.float8_e4m3fn}[mode]
    a = _layer(H, D, NB, bs, cache_dtype, mode, device)
    a.attention_compute_dtype = torch.bfloat16
    T = NB * bs
    k, v = _src((T, H, D), torch.bfloat16, 40), _src((T, H, D), torch.bfloat16, 41)
    a.store_kv_cache_torch(k.to(device), v.to(device), torch.arange(T, dtype=torch.int32, device=device))
    bt = torch.tensor([[3, -1, 7, 1], [5, 0, -1, -1], [-1, -1, -1, -1], [9, 10, 11, 2]], dtype=torch.int32)
    lens = torch.tensor([150, 64, 10, 200], dtype=torch.int32)
    from nanovllm_self_amd.utils.context import Context

    kb, vb, mask = a.get_kv_cache(Context(block_tables=bt.to(device), context_lens=lens.to(device)))
    torch.cuda.synchronize()
    from tests.gpu_util import cache_blocks_f32

    kv, vv = cache_blocks_f32(a, np.arange(NB))
    rk, rv, rm = KO.get_kv_cache(kv, vv, bt.numpy(), lens.numpy())
    assert kb.dtype == torch.bfloat16 and kb.shape == (4, 200, H, D)
    assert np.array_equal(mask.cpu().numpy(), rm)
    assert np.array_equal(_f32(kb), rk)
    assert np.array_equal(_f32(vb), rv)
