"""A generation loop over the whole path, engine-style, against the CPU oracle.

A tiny random "model" (embedding tables for q, k and v, the two norm
weights, a rotary table, an output projection) drives the path the way
ModelRunner.run does each step: the step's Context and positions from the
sequences (build_context_on_device, model_runner.py:461-532), the fused
q/k norm + rotary + KV store and the attention call
(PagedAttention.forward_fused; qwen3.py:100-104 and attention.py:500-550),
then greedy sampling from the last position of each sequence that needs
logits.  The oracle keeps each sequence's rotated k and raw v (bf16 values,
exactly as the cache must hold them) and attends in fp32 (oracle/
prep_oracle.py, oracle/attn_oracle.py).

Scenario (the reference's own prefix tests, tests/test_prefix_prefill_long.py:
135-156, and mixed workload, tests/test_p0_mixed_workload.py): a fresh
prompt, then a second prompt sharing the first one's first full block (a
prefix-cache hit: num_cached_tokens = floor(shared / 256) * 256, block_tables
present, more keys than queries, only the suffix computed), then decode
steps of both beside the chunked prefill of a third prompt, the third
prompt's tokens identical to the second's so its output can be checked
against the prefix-hit run.  Every step compares the attention output with
the oracle within the bf16 bars and the greedy tokens (the oracle's choice
is fed to both sides, so a near-tie cannot make the runs diverge).
"""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import PagedAttention
from nanovllm_self_amd.kv_cache import KVCacheConfig, SeqSlice, allocate_kv_cache, bind_kv_cache
from oracle import attn_oracle as AO
from oracle import prep_oracle as PO
from oracle import kv_oracle as KO
from oracle.kv_oracle import round_to_bf16
from tests.gpu_util import bf16_to_np, compare, say

pytestmark = pytest.mark.gpu

V, HQ, HKV, D, BS, NB, MAX_POS, EPS = 512, 8, 2, 128, 256, 24, 4096, 1e-6


class Model:
    def __init__(self, device, seed=0):
        g = torch.Generator().manual_seed(seed)
        self.eq = torch.randn(V, HQ, D, generator=g).to(torch.bfloat16)
        self.ek = (2 * torch.randn(V, HKV, D, generator=g)).to(torch.bfloat16)
        self.ev = torch.randn(V, HKV, D, generator=g).to(torch.bfloat16)
        self.qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
        self.kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
        self.w_out = torch.randn(HQ * D, V, generator=g) / np.sqrt(HQ * D)
        self.table = PO.cos_sin_table(D, MAX_POS, 1e6)
        self.dev = {n: getattr(self, n).to(device) for n in ("eq", "ek", "ev", "qw", "kw")}
        self.dev["table"] = torch.from_numpy(self.table).reshape(MAX_POS, 1, D).to(device)
        self.dev["w_out"] = self.w_out.to(device)


class Seq:
    """The Sequence fields the runner reads, plus the oracle's per-sequence K/V
    as the cache holds it (bf16 values, or the quantised codes' bf16(code *
    scale))."""

    def __init__(self, tokens, blocks):
        self.tokens = list(tokens)
        self.block_table = list(blocks)
        self.num_cached_tokens = 0
        self.k = np.zeros((0, HKV, D), np.float32)
        self.v = np.zeros((0, HKV, D), np.float32)

    def slice(self, n_new):
        return SeqSlice(self.block_table, self.num_cached_tokens, n_new)


def gpu_step(model, attn, batch, device):
    from nanovllm_self_amd.kv_cache import build_context_on_device

    ctx, positions = build_context_on_device([s.slice(n) for s, n in batch], BS, device)
    ids = torch.tensor([t for s, n in batch for t in s.tokens[s.num_cached_tokens:s.num_cached_tokens + n]],
                       dtype=torch.long, device=device)
    m = model.dev
    out = attn.forward_fused(m["eq"][ids], m["ek"][ids], m["ev"][ids], positions, m["qw"], m["kw"], EPS,
                             m["table"], ctx)
    torch.cuda.synchronize()
    return ctx, out


def cached_values(x, kv):
    """What the cache gives back for rows x (bf16 values): x itself, or the
    per-token quantised codes dequantised and rounded to bf16."""
    if kv == "bf16":
        return x
    quant = KO.quantize_int8_per_token if kv == "int8" else KO.quantize_fp8_per_token
    codes, sc = quant(x)
    return round_to_bf16(KO.dequantize_per_token(codes, sc, kv))


def oracle_step(model, batch, kv="bf16"):
    """The step on the CPU; extends each sequence's cached K/V as the store
    would.  A step without block tables (no sequence has cached tokens)
    attends over the raw k/v, the others over the cache (attention.py:
    401-415 against 441-498)."""
    fresh = all(s.num_cached_tokens == 0 for s, _ in batch)
    outs = []
    for s, n in batch:
        a = s.num_cached_tokens
        ids = torch.tensor(s.tokens[a:a + n], dtype=torch.long)
        pos = np.arange(a, a + n)
        q, k = PO.qk_norm_rope(bf16_to_np(model.eq[ids]), bf16_to_np(model.ek[ids]), pos, bf16_to_np(model.qw),
                               bf16_to_np(model.kw), EPS, model.table)
        v = bf16_to_np(model.ev[ids])
        s.k = np.concatenate([s.k, cached_values(k, kv)])
        s.v = np.concatenate([s.v, cached_values(v, kv)])
        kk, vv = (k, v) if fresh else (s.k, s.v)
        kb, vb = torch.from_numpy(np.ascontiguousarray(kk))[None], torch.from_numpy(np.ascontiguousarray(vv))[None]
        outs.append(AO.attention_cached(torch.from_numpy(q), kb, vb, [0, n], [0, kb.shape[1]], HQ, HKV, D).numpy())
    return np.concatenate(outs)


def greedy(model, out_rows):
    """Logits of each sequence's last row; the oracle's choice and its margin."""
    logits = torch.from_numpy(out_rows.reshape(len(out_rows), -1)) @ model.w_out
    top = torch.topk(logits, 2, dim=-1)
    return top.indices[:, 0].tolist(), (top.values[:, 0] - top.values[:, 1]).tolist(), logits


def run_step(model, attn, batch, device, what, kv="bf16"):
    say(what)
    ctx, out = gpu_step(model, attn, batch, device)
    ref = oracle_step(model, batch, kv)
    got = bf16_to_np(out)
    compare(got, ref, kv != "bf16", what)
    last = np.cumsum([n for _, n in batch]) - 1
    want, margin, _ = greedy(model, round_to_bf16(ref[last]))
    mine, _, _ = greedy(model, got[last])
    for i, (w, g_, mg) in enumerate(zip(want, mine, margin)):
        if mg > 1e-2:  # a clear choice must agree; near-ties are fed the oracle's token anyway
            assert w == g_, f"{what}: sequence {i} picked {g_}, the oracle {w} (margin {mg:.3g})"
    for (s, n), tok in zip(batch, want):
        s.num_cached_tokens += n
        if s.num_cached_tokens == len(s.tokens):
            s.tokens.append(tok)
    return ctx, got, ref


CACHE = {"bf16": (torch.bfloat16, "none"), "fp8": (torch.float8_e4m3fn, "fp8_e4m3"), "int8": (torch.int8, "int8_mock")}


@pytest.mark.parametrize("kv", ["bf16", "fp8", "int8"])
def test_generation_loop_with_prefix_hit_and_mixed_steps(device, kv):
    model = Model(device)
    cfg = KVCacheConfig(dtype=torch.bfloat16, kv_cache_dtype=CACHE[kv][0], attention_compute_dtype=torch.bfloat16,
                        kv_cache_quant_mode=CACHE[kv][1], block_size=BS, num_blocks=NB)
    attn = PagedAttention(HQ, HKV, D, dtype=torch.bfloat16)
    kv_cache, scales = allocate_kv_cache(1, HKV, D, cfg, device)
    bind_kv_cache([attn], kv_cache, scales, cfg)
    rng = np.random.default_rng(7)
    prompt_a = rng.integers(0, V, 300).tolist()

    # A: a fresh 300-token prompt (no cached tokens anywhere: block_tables None).
    a = Seq(prompt_a, [3, 9])
    ctx, _, _ = run_step(model, attn, [(a, 300)], device, f"engine {kv}: prefill A (fresh)", kv)
    assert ctx.block_tables is None

    # B: A's first 300 tokens plus 100 more; the first full block is a cache
    # hit (it shares A's block 3), so only positions 256 .. 399 are computed.
    b = Seq(prompt_a + rng.integers(0, V, 100).tolist(), [3, 5])
    shared = 300
    b.num_cached_tokens = shared // BS * BS
    assert b.num_cached_tokens == 256
    b.k, b.v = a.k[:256].copy(), a.v[:256].copy()  # the oracle's view of the shared block
    ctx, out_b, _ = run_step(model, attn, [(b, len(b.tokens) - 256)], device, f"engine {kv}: prefill B over a cached block", kv)
    assert ctx.block_tables is not None and int(ctx.cu_seqlens_k[-1]) > int(ctx.cu_seqlens_q[-1])
    assert int(ctx.cu_seqlens_q[-1]) == 144

    # C: B's 400 prompt tokens as a fresh sequence, prefilled in two chunks
    # beside decode steps of A and B (mixed batches).
    c = Seq(b.tokens[:400], [11, 12])
    run_step(model, attn, [(a, 1), (b, 1), (c, 256)], device, f"engine {kv}: decode A, B + chunk 1 of C", kv)
    _, out_c, _ = run_step(model, attn, [(a, 1), (c, 144), (b, 1)], device, f"engine {kv}: decode A, chunk 2 of C, decode B", kv)
    # C's last prompt row attends over the same 400 keys as B's last prompt row.
    np.testing.assert_allclose(out_c[1 + 143], out_b[143], rtol=0, atol=2e-2 if kv == "bf16" else 5e-2)
    for step in range(6):
        run_step(model, attn, [(a, 1), (b, 1), (c, 1)], device, f"engine {kv}: decode step {step} of A, B, C", kv)
    assert len(a.tokens) == 300 + 9 and len(c.tokens) == 400 + 7
