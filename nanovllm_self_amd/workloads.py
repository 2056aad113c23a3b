"""Seeded synthetic attention batches at the shapes the path is measured on.

Each builder returns a Workload: the step's q/k/v, a bound PagedAttention
layer whose paged cache already holds every sequence's history, and the step
Context built the way the engine builds it (kv_cache.build_context).  Batch
structure (lengths, block tables, the step's q/k/v) comes from a CPU
torch.Generator with the stated seed, drawn in fp32 and cast to bf16; the
cache history is drawn on the target device from a generator with the same
seed (fast for multi-GB pools) and, for quantised caches, written through the
store kernel so codes and scales are the ones the path itself produces.

Shapes:
  decode_small   16 q / 8 kv heads, D 128, bs 256, 64 blocks, 8 seqs,
                 ctx U[128, 1024]                                (seed 0)
  decode_8b      32 q / 8 kv heads, D 128, bs 256, 4096 blocks, 64 seqs,
                 ctx U[2048, 8192], k * 0.5                      (seed 1)
  prefill_8b     32 / 8 heads, 16 seqs, new U[512, 4096], cached prefix of
                 0-8 whole blocks                                (seed 2)
  decode_quant   32 / 8 heads, 256 seqs, ctx U[1024, 4096], fp8 / int8 / bf16
                 cache, sources N(0,1) with 1% outliers x8       (seed 3)
  mixed_32b      64 / 8 heads, 128 decode seqs with ctx log-U[256, 32768]
                 followed by 4 prefill chunks of 2048 tokens over a cached
                 prefix U[0, 16384] rounded down to whole blocks, 16384
                 blocks                                          (seed 4)
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .kv_cache import KVCacheConfig, SeqSlice, allocate_kv_cache, bind_kv_cache, build_context
from .layers.attention import PagedAttention
from .utils.context import Context

QUANT_MODE = {"bf16": "none", "fp16": "none", "int8": "int8_mock", "fp8": "fp8_e4m3"}


@dataclass
class Workload:
    name: str
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    kv: str  # "bf16" | "fp16" (an fp16 model: fp16 cache and compute) | "int8" | "fp8"
    attn: PagedAttention
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    context: Context
    seqs: list = field(default_factory=list)  # SeqSlice per sequence
    kv_cache: torch.Tensor | None = None
    kv_scale_cache: torch.Tensor | None = None

    # ----------------------------------------------------------- accounting
    @property
    def num_seqs(self) -> int:
        return len(self.seqs)

    def decode_seq_ids(self):
        return [i for i, s in enumerate(self.seqs) if s.num_new_tokens == 1]

    def prefill_seq_ids(self):
        return [i for i, s in enumerate(self.seqs) if s.num_new_tokens > 1]

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of the decode rows: every visible K/V element
        (and scale) once, plus q read and o written."""
        s_kv = 2 if self.kv in ("bf16", "fp16") else 1
        s_sc = 0 if self.kv in ("bf16", "fp16") else 4
        ctx = sum(self.seqs[i].num_cached_tokens + 1 for i in self.decode_seq_ids())
        nd = len(self.decode_seq_ids())
        H, Hq, D = self.num_kv_heads, self.num_heads, self.head_dim
        return ctx * H * 2 * D * s_kv + ctx * H * 2 * s_sc + nd * Hq * D * 2 * 2

    def prefill_flops(self) -> float:
        """4 Hq D sum_i [L_i P_i + L_i (L_i + 1) / 2]: QK^T and PV over the
        pairs the bottom-right causal mask leaves visible."""
        tot = 0
        for i in self.prefill_seq_ids():
            s = self.seqs[i]
            L, P = s.num_new_tokens, s.num_cached_tokens
            tot += L * P + L * (L + 1) // 2
        return 4.0 * self.num_heads * self.head_dim * tot


def _gen(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _randn(g, shape, scale=1.0, outliers=False, dtype=torch.bfloat16):
    x = torch.randn(shape, generator=g, dtype=torch.float32) * scale
    if outliers:
        hit = torch.rand(shape, generator=g) < 0.01
        x = torch.where(hit, x * 8.0, x)
    return x.to(dtype)


def _fill_history(wl: Workload, seed: int, k_scale: float, outliers: bool) -> None:
    """Write every sequence's cached positions [0, num_cached) into the cache
    with random N(0,1) values (through the store kernel for quantised caches)."""
    dev = wl.q.device
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1000)
    slots = []
    bs = wl.block_size
    for s in wl.seqs:
        n = s.num_cached_tokens
        if n == 0:
            continue
        pos = torch.arange(n, dtype=torch.int64)
        bt = torch.tensor(s.block_table, dtype=torch.int64)
        slots.append(bt[pos // bs] * bs + pos % bs)
    if not slots:
        return
    slot_mapping = torch.cat(slots).to(torch.int32).to(dev)
    H, D = wl.num_kv_heads, wl.head_dim
    chunk = 1 << 18
    for a in range(0, slot_mapping.numel(), chunk):
        sl = slot_mapping[a:a + chunk]
        n = sl.numel()
        kk = torch.randn((n, H, D), generator=g, device=dev, dtype=torch.float32) * k_scale
        vv = torch.randn((n, H, D), generator=g, device=dev, dtype=torch.float32)
        if outliers:
            kk = torch.where(torch.rand(kk.shape, generator=g, device=dev) < 0.01, kk * 8.0, kk)
            vv = torch.where(torch.rand(vv.shape, generator=g, device=dev) < 0.01, vv * 8.0, vv)
        src = torch.float16 if wl.kv == "fp16" else torch.bfloat16
        wl.attn.store_kv_cache_torch(kk.to(src), vv.to(src), sl)


def _assemble(name, seqs, Hq, Hkv, D, bs, NB, kv, device, g, k_scale=1.0, outliers=False,
              seed=0) -> Workload:
    elem = torch.float16 if kv == "fp16" else torch.bfloat16
    cfg = KVCacheConfig(
        dtype=elem, kv_cache_dtype=elem,
        attention_compute_dtype=elem, kv_cache_quant_mode=QUANT_MODE[kv],
        block_size=bs, num_blocks=NB,
    )
    attn = PagedAttention(Hq, Hkv, D, dtype=elem)
    kv_cache, kv_scale_cache = allocate_kv_cache(1, Hkv, D, cfg, device)
    bind_kv_cache([attn], kv_cache, kv_scale_cache, cfg)
    T = sum(s.num_new_tokens for s in seqs)
    q = _randn(g, (T, Hq, D), dtype=elem).to(device)
    k = _randn(g, (T, Hkv, D), k_scale, outliers, dtype=elem).to(device)
    v = _randn(g, (T, Hkv, D), 1.0, outliers, dtype=elem).to(device)
    ctx = build_context(seqs, bs, device)
    wl = Workload(name, Hq, Hkv, D, bs, NB, kv, attn, q, k, v, ctx, list(seqs), kv_cache, kv_scale_cache)
    _fill_history(wl, seed, k_scale, outliers)
    return wl


def _tables(g, lens_total, bs, NB):
    need = [(n + bs - 1) // bs for n in lens_total]
    if sum(need) > NB:
        raise ValueError(f"pool of {NB} blocks too small for {sum(need)}")
    perm = torch.randperm(NB, generator=g).tolist()
    out, at = [], 0
    for n in need:
        out.append(perm[at:at + n])
        at += n
    return out


def _decode_seqs(g, B, lo, hi, NB, bs):
    ctx = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
    tables = _tables(g, ctx, bs, NB)
    return [SeqSlice(tables[i], ctx[i] - 1, 1) for i in range(B)]


def decode_workload(name, B, lo, hi, Hq, Hkv, NB, kv="bf16", seed=0, k_scale=1.0, outliers=False,
                    device="cuda", D=128, bs=256) -> Workload:
    g = _gen(seed)
    seqs = _decode_seqs(g, B, lo, hi, NB, bs)
    return _assemble(name, seqs, Hq, Hkv, D, bs, NB, kv, device, g, k_scale, outliers, seed)


def decode_small(device="cuda", kv="bf16") -> Workload:
    return decode_workload("decode_small", 8, 128, 1024, 16, 8, 64, kv, seed=0, device=device)


def decode_8b(device="cuda", kv="bf16") -> Workload:
    return decode_workload("decode_8b", 64, 2048, 8192, 32, 8, 4096, kv, seed=1, k_scale=0.5,
                           device=device)


def decode_quant(device="cuda", kv="fp8", B=256) -> Workload:
    return decode_workload("decode_quant", B, 1024, 4096, 32, 8, 4096, kv, seed=3, outliers=True,
                           device=device)


def _prefill_8b_seqs(g, B, NB, bs=256):
    prefix = [bs * int(x) for x in torch.randint(0, 9, (B,), generator=g).tolist()]
    new = torch.randint(512, 4097, (B,), generator=g).tolist()
    tables = _tables(g, [p + n for p, n in zip(prefix, new)], bs, NB)
    return [SeqSlice(tables[i], prefix[i], new[i]) for i in range(B)]


def prefill_8b(device="cuda", kv="bf16", B=16, NB=512) -> Workload:
    g = _gen(2)
    seqs = _prefill_8b_seqs(g, B, NB)
    return _assemble("prefill_8b", seqs, 32, 8, 128, 256, NB, kv, device, g, seed=2)


def _mixed_32b_seqs(g, n_decode, n_chunks, chunk, bs=256, NB=16384):
    lo, hi = math.log(256), math.log(32768)
    u = torch.rand((n_decode,), generator=g, dtype=torch.float64)
    dec_ctx = [int(round(math.exp(lo + (hi - lo) * float(x)))) for x in u]
    pre = torch.rand((n_chunks,), generator=g, dtype=torch.float64)
    prefix = [bs * (int(16384 * float(x)) // bs) for x in pre]
    totals = dec_ctx + [p + chunk for p in prefix]
    tables = _tables(g, totals, bs, NB)
    seqs = [SeqSlice(tables[i], dec_ctx[i] - 1, 1) for i in range(n_decode)]
    return seqs + [SeqSlice(tables[n_decode + j], prefix[j], chunk) for j in range(n_chunks)]


def mixed_32b(device="cuda", kv="bf16", n_decode=128, n_chunks=4, chunk=2048) -> Workload:
    g = _gen(4)
    seqs = _mixed_32b_seqs(g, n_decode, n_chunks, chunk)
    return _assemble("mixed_32b", seqs, 64, 8, 128, 256, 16384, kv, device, g, seed=4)


def mixed_32b_chunks(device="cuda", kv="bf16") -> Workload:
    """mixed_32b's four prefill chunks alone: the same draw (tables, prefixes,
    cache contents of those sequences) without the decode rows."""
    g = _gen(4)
    seqs = _mixed_32b_seqs(g, 128, 4, 2048)[128:]
    return _assemble("mixed_32b chunks", seqs, 64, 8, 128, 256, 16384, kv, device, g, seed=4)


def step_batches() -> dict:
    """The sequence lists (block size 256) of decode_8b, prefill_8b,
    decode_quant and mixed_32b, drawn as their builders draw them, without
    building any tensor."""
    return {
        "decode_8b": _decode_seqs(_gen(1), 64, 2048, 8192, 4096, 256),
        "prefill_8b": _prefill_8b_seqs(_gen(2), 16, 512),
        "decode_quant": _decode_seqs(_gen(3), 256, 1024, 4096, 4096, 256),
        "mixed_32b": _mixed_32b_seqs(_gen(4), 128, 4, 2048),
    }


BUILDERS = {
    "decode_small": decode_small,
    "decode_8b": decode_8b,
    "prefill_8b": prefill_8b,
    "decode_quant": decode_quant,
    "mixed_32b": mixed_32b,
}
