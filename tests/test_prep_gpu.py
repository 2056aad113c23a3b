"""Fused pre-attention step (nvs_qk_norm_rope_store) on the GPU against the
CPU oracle (oracle/prep_oracle.py, oracle/kv_oracle.py) and against the
reference's own torch ops.

Against the oracle, bit-exact: the rotated q and k equal the oracle's (which
fixes the order of the norm's sum, left open by the reference, to the
kernel's), and the cache holds the rotated k and the raw v cast or quantised
exactly as the store oracle does from those values; slots < 0 leave the
cache untouched.  Against RMSNorm.py:11-18 and RoPE.py:5-25 run as torch ops
on the CPU (their own summation order and division by sqrt): at least 99.9%
of the elements equal and none more than 4 bf16 steps apart.  The norm's sum
in another order can move a normed value by one step (rounded to bf16
between norm and rotation, as the reference does); where the rotation
x1 cos - x2 sin cancels, that step is several steps of the smaller result."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import PagedAttention
from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import KVCacheConfig, allocate_kv_cache, bind_kv_cache
from oracle import kv_oracle as KO
from oracle import prep_oracle as PO
from tests.gpu_util import bf16_to_np, say

pytestmark = pytest.mark.gpu

D = 128
MAX_POS = 4096
QUANT_MODE = {"bf16": "none", "int8": "int8_mock", "fp8": "fp8_e4m3"}
CACHE_DTYPE = {"bf16": torch.bfloat16, "int8": torch.int8, "fp8": torch.float8_e4m3fn}


def _layer(Hq, Hkv, kv, NB, bs, device):
    cfg = KVCacheConfig(dtype=torch.bfloat16, kv_cache_dtype=CACHE_DTYPE[kv],
                        attention_compute_dtype=torch.bfloat16, kv_cache_quant_mode=QUANT_MODE[kv],
                        block_size=bs, num_blocks=NB)
    attn = PagedAttention(Hq, Hkv, D, dtype=torch.bfloat16)
    kv_cache, scales = allocate_kv_cache(1, Hkv, D, cfg, device)
    bind_kv_cache([attn], kv_cache, scales, cfg)
    return attn


def _ulps(got: np.ndarray, ref: np.ndarray):
    """Largest distance in bf16 steps and the fraction of equal elements."""
    def line(x):
        b = KO.f32_to_bf16_bits(x).astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    d = np.abs(line(got) - line(ref))
    return int(d.max()) if d.size else 0, float(np.mean(d == 0)) if d.size else 1.0


def _inputs(T, Hq, Hkv, seed, NB, bs):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, Hq, D, generator=g).to(torch.bfloat16)
    k = (3.0 * torch.randn(T, Hkv, D, generator=g)).to(torch.bfloat16)
    v = torch.randn(T, Hkv, D, generator=g).to(torch.bfloat16)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, MAX_POS, (T,), generator=g, dtype=torch.int64)
    slots = torch.randperm(NB * bs, generator=g)[:T].to(torch.int32)
    slots[torch.rand(T, generator=g) < 0.1] = -1
    return q, k, v, qw, kw, pos, slots


def _check_cache(attn, kv, slots, k_rot, v):
    kc = attn.k_cache.reshape(-1, attn.num_kv_heads, D).cpu()
    vc = attn.v_cache.reshape(-1, attn.num_kv_heads, D).cpu()
    ok = slots >= 0
    s = slots[ok].long()
    kk, vv = k_rot[ok.numpy()], bf16_to_np(v)[ok.numpy()]
    if kv == "bf16":
        assert np.array_equal(bf16_to_np(kc[s]), kk) and np.array_equal(bf16_to_np(vc[s]), vv)
    else:
        quant = KO.quantize_int8_per_token if kv == "int8" else KO.quantize_fp8_per_token
        ks = attn.k_scale_cache.reshape(-1, attn.num_kv_heads).cpu().numpy()
        vs = attn.v_scale_cache.reshape(-1, attn.num_kv_heads).cpu().numpy()
        for cache, scales, x in ((kc, ks, kk), (vc, vs, vv)):
            codes, sc = quant(x)
            got = cache[s].view(torch.uint8).numpy()
            assert np.array_equal(got, codes.view(np.uint8)), "codes"
            assert np.array_equal(scales[s.numpy()], sc[..., 0]), "scales"
    # Slots never named keep the sentinel the cache was filled with.
    untouched = np.ones(kc.shape[0], dtype=bool)
    untouched[s.numpy()] = False
    raw = attn.k_cache.reshape(-1, attn.num_kv_heads, D).view(torch.uint8).cpu().numpy()[untouched]
    assert np.all(raw == 0x3C)


@pytest.mark.parametrize("kv", ["bf16", "int8", "fp8"])
@pytest.mark.parametrize("Hq,Hkv,T", [(32, 8, 64), (16, 8, 300), (4, 2, 1), (64, 8, 17)])
def test_prep_matches_oracle(device, kv, Hq, Hkv, T):
    say(f"qk_norm_rope_store {kv} Hq={Hq} Hkv={Hkv} T={T}")
    NB, bs = 16, 64
    attn = _layer(Hq, Hkv, kv, NB, bs, device)
    attn.k_cache.view(torch.uint8).fill_(0x3C)
    attn.v_cache.view(torch.uint8).fill_(0x3C)
    q, k, v, qw, kw, pos, slots = _inputs(T, Hq, Hkv, 100 + T, NB, bs)
    table = PO.cos_sin_table(D, MAX_POS, 1e6)
    q_rot, k_rot = attn.qk_norm_rope_store(
        q.to(device), k.to(device), v.to(device), pos.to(device), qw.to(device), kw.to(device), 1e-6,
        torch.from_numpy(table).reshape(MAX_POS, 1, D).to(device), slots.to(device), want_k=True)
    torch.cuda.synchronize()
    qo, ko = PO.qk_norm_rope(bf16_to_np(q), bf16_to_np(k), pos.numpy(), bf16_to_np(qw), bf16_to_np(kw), 1e-6, table)
    gq, gk = bf16_to_np(q_rot), bf16_to_np(k_rot)
    for name, got, ref in (("q", gq, qo), ("k", gk, ko)):
        worst, equal = _ulps(got, ref)
        assert worst == 0, f"{name}: {worst} bf16 steps from the oracle ({1 - equal:.2%} of elements differ)"
    _check_cache(attn, kv, slots, gk, v)


def _edge_rows(x: torch.Tensor, g: torch.Generator) -> torch.Tensor:
    """x [T, H, D] with rows at the edges of the norm's arithmetic: scaled by
    2^-90 (tiny, normal quotients), 2^-80 (squares underflow to 0), 2^70
    (squares overflow), and an all-zero row."""
    x = x.clone().float()
    T, H, _ = x.shape
    cells = [(t, h) for t in range(T) for h in range(H)]
    pick = torch.randperm(len(cells), generator=g)[:4 * max(1, len(cells) // 8)].tolist()
    for n, i in enumerate(pick):
        t, h = cells[i]
        x[t, h] = x[t, h] * (2.0 ** (-90), 2.0 ** (-80), 2.0 ** 70, 0.0)[n % 4]
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("eps", [0.0, 1e-6])
def test_prep_edge_rows_match_oracle(device, eps):
    """Rows whose rms is 0 or infinite take the per-element division, tiny
    rows the reciprocal path: both equal the oracle bit for bit (NaN where
    the reference's arithmetic gives NaN)."""
    say(f"qk_norm_rope_store edge rows eps={eps}")
    Hq, Hkv, T, NB, bs = 8, 2, 16, 4, 64
    attn = _layer(Hq, Hkv, "bf16", NB, bs, device)
    q, k, v, qw, kw, pos, slots = _inputs(T, Hq, Hkv, 77, NB, bs)
    g = torch.Generator().manual_seed(78)
    q, k = _edge_rows(q, g), _edge_rows(k, g)
    table = PO.cos_sin_table(D, MAX_POS, 1e6)
    q_rot, k_rot = attn.qk_norm_rope_store(
        q.to(device), k.to(device), v.to(device), pos.to(device), qw.to(device), kw.to(device), eps,
        torch.from_numpy(table).reshape(MAX_POS, 1, D).to(device), slots.to(device), want_k=True)
    torch.cuda.synchronize()
    with np.errstate(all="ignore"):
        qo, ko = PO.qk_norm_rope(bf16_to_np(q), bf16_to_np(k), pos.numpy(), bf16_to_np(qw), bf16_to_np(kw), eps,
                                 table)
    for name, got, ref in (("q", bf16_to_np(q_rot), qo), ("k", bf16_to_np(k_rot), ko)):
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan), f"{name}: NaN positions differ"
        assert np.array_equal(got[~nan], ref[~nan]), f"{name}: differs from the oracle"
        say(f"  {name}: {int(nan.sum())} NaN, {int(np.isinf(ref).sum())} inf elements, equal")


def _torch_reference(x, w, eps, cos, sin):
    """RMSNorm.py:11-18 then RoPE.py:5-25 as torch ops (CPU): the normed
    value is rounded to the input dtype between the two, as there."""
    x32 = x.float()
    normed = (w.float() * x32 / torch.sqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    x1, x2 = torch.chunk(normed.float(), 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


@pytest.mark.parametrize("Hq,Hkv,T", [(32, 8, 512), (64, 8, 97)])
def test_prep_matches_reference_torch_ops(device, Hq, Hkv, T):
    say(f"qk_norm_rope_store vs torch ops Hq={Hq} Hkv={Hkv} T={T}")
    NB, bs = 16, 64
    attn = _layer(Hq, Hkv, "bf16", NB, bs, device)
    q, k, v, qw, kw, pos, slots = _inputs(T, Hq, Hkv, 300 + T, NB, bs)
    table = torch.from_numpy(PO.cos_sin_table(D, MAX_POS, 1e6))  # [max_pos, D]: cos | sin
    q_rot, k_rot = attn.qk_norm_rope_store(
        q.to(device), k.to(device), v.to(device), pos.to(device), qw.to(device), kw.to(device), 1e-6,
        table.reshape(MAX_POS, 1, D).to(device), slots.to(device), want_k=True)
    torch.cuda.synchronize()
    cos, sin = table[pos].unsqueeze(1).chunk(2, dim=-1)  # [T, 1, D/2]
    for name, got, x, w in (("q", q_rot, q, qw), ("k", k_rot, k, kw)):
        ref = _torch_reference(x, w, 1e-6, cos, sin)
        worst, equal = _ulps(bf16_to_np(got), bf16_to_np(ref))
        say(f"  {name}: at most {worst} bf16 steps from the torch ops, {equal:.4%} of elements equal")
        assert worst <= 4 and equal >= 0.999, f"{name}: {worst} bf16 steps, {equal:.4%} equal"


def test_prep_clamps_positions_and_handles_empty_batches(device):
    say("qk_norm_rope_store clamp / empty")
    attn = _layer(8, 2, "bf16", 4, 64, device)
    q, k, v, qw, kw, _, _ = _inputs(3, 8, 2, 7, 4, 64)
    table = torch.from_numpy(PO.cos_sin_table(D, 32, 1e6)).reshape(32, 1, D).to(device)
    args = [t.to(device) for t in (q, k, v)]
    slots = torch.tensor([-1, -1, -1], dtype=torch.int32, device=device)
    a, _ = attn.qk_norm_rope_store(*args, torch.tensor([-5, 40, 31], device=device), qw.to(device),
                                   kw.to(device), 1e-6, table, slots)
    b, _ = attn.qk_norm_rope_store(*args, torch.tensor([0, 31, 31], device=device), qw.to(device),
                                   kw.to(device), 1e-6, table, slots)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    e = [t[:0].to(device) for t in (q, k, v)]
    out, _ = attn.qk_norm_rope_store(*e, torch.zeros(0, dtype=torch.int64, device=device), qw.to(device),
                                     kw.to(device), 1e-6, table, slots[:0])
    assert out.shape == (0, 8, D)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_forward_fused_equals_forward_on_prepared_inputs(device, kv):
    """forward_fused(raw q, k) == forward(rotated q, k) on the same batch."""
    say(f"forward_fused decode_small/{kv}")
    wl = W.decode_small(device, kv=kv)
    attn, ctx = wl.attn, wl.context
    g = torch.Generator().manual_seed(11)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(device)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(device)
    table = torch.from_numpy(PO.cos_sin_table(D, MAX_POS, 1e6)).reshape(MAX_POS, 1, D).to(device)
    pos = (ctx.context_lens.to(torch.int64) - 1).to(device)
    fused = attn.forward_fused(wl.q, wl.k, wl.v, pos, qw, kw, 1e-6, table, ctx)
    q_rot, k_rot = attn.qk_norm_rope_store(wl.q, wl.k, wl.v, pos, qw, kw, 1e-6, table, ctx.slot_mapping,
                                           want_k=True)
    plain = attn.forward(q_rot, k_rot, wl.v, ctx)
    torch.cuda.synchronize()
    assert torch.equal(fused, plain)
