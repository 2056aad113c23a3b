"""HIP attention vs the fp32 CPU oracle on the measured shapes and on edge
cases.  Tolerances: bf16 KV max-abs <= 2e-2 and mean-abs <= 2e-3; int8 / fp8
KV max-abs <= 5e-2; the max-abs bound applies on top of the half-ulp
(2^-8 |ref|) that rounding the output to bf16 costs the reference itself
(tests/gpu_util.py).  Large batches are checked on a
subset of their sequences (the per-sequence math does not depend on the
others) plus size-independent properties at full size."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from nanovllm_self_amd.utils.context import Context
from oracle import attn_oracle as AO
from tests.gpu_util import bf16_to_np, cache_blocks_f32, compare, oracle_paged, say

pytestmark = pytest.mark.gpu


def _run(wl):
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    assert out.shape == wl.q.shape and out.dtype == torch.bfloat16
    return bf16_to_np(out)


def _check(wl, seq_ids=None, what=""):
    got = _run(wl)
    ids = list(range(wl.num_seqs)) if seq_ids is None else list(seq_ids)
    ref, rows = oracle_paged(wl, ids)
    return compare(got[rows], ref, wl.kv != "bf16", what or wl.name)


def _custom(seqs, Hq, Hkv, NB, kv="bf16", seed=7, bs=256, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return W._assemble("custom", seqs, Hq, Hkv, 128, bs, NB, kv, device, g, seed=seed)


def _tables(lens, NB, seed, bs=256):
    g = torch.Generator().manual_seed(seed)
    return W._tables(g, lens, bs, NB)


# ---------------------------------------------------------------- decode
@pytest.mark.parametrize("kv", ["bf16", "int8", "fp8"])
def test_decode_small_full(device, kv):
    say(f"decode_small {kv}")
    _check(W.decode_small(device, kv=kv), what=f"decode_small/{kv}")


def test_decode_8b_subset_and_permutation(device):
    say("decode_8b bf16 full size")
    wl = W.decode_8b(device)
    lens = [s.num_cached_tokens + 1 for s in wl.seqs]
    order = np.argsort(lens)
    ids = sorted(set(order[:3].tolist() + order[-3:].tolist()))
    _check(wl, ids, "decode_8b subset")
    base = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    # Physical placement must not matter: move every block, remap the tables.
    say("decode_8b block permutation")
    NB = wl.num_blocks
    perm = torch.randperm(NB, generator=torch.Generator().manual_seed(99)).to(device)
    inv = torch.argsort(perm)
    for name in ("k_cache", "v_cache"):
        old = getattr(wl.attn, name)
        new = torch.empty_like(old)
        new[inv] = old
        setattr(wl.attn, name, new)
    bt = wl.context.block_tables
    wl.context.block_tables = torch.where(bt >= 0, inv[bt.clamp(min=0).long()].int(), bt)
    sl = wl.context.slot_mapping.long()
    bs = wl.block_size
    wl.context.slot_mapping = (inv[sl // bs] * bs + sl % bs).int()
    moved = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    assert torch.equal(base, moved)


@pytest.mark.parametrize("kv", ["bf16", "int8", "fp8"])
def test_decode_quant_shape(device, kv):
    say(f"decode_quant {kv}")
    wl = W.decode_quant(device, kv=kv)
    ids = list(range(0, wl.num_seqs, 32))
    _check(wl, ids, f"decode_quant/{kv}")


@pytest.mark.parametrize("ctx", [1, 2, 31, 32, 33, 255, 256, 257, 511, 513, 1000])
def test_decode_lengths(device, ctx):
    say(f"decode ctx={ctx}")
    lens = [ctx, max(1, ctx // 2), ctx + 3]
    tabs = _tables(lens, 16, ctx)
    wl = _custom([SeqSlice(tabs[i], lens[i] - 1, 1) for i in range(3)], 8, 2, 16, seed=ctx)
    _check(wl, what=f"decode ctx={ctx}")


@pytest.mark.parametrize("g", [1, 2, 3, 5, 8, 16])
def test_decode_gqa_groups(device, g):
    say(f"decode g={g}")
    Hkv = 2
    lens = [700, 90, 1500]
    tabs = _tables(lens, 16, g)
    wl = _custom([SeqSlice(tabs[i], lens[i] - 1, 1) for i in range(3)], g * Hkv, Hkv, 16, seed=g)
    _check(wl, what=f"decode g={g}")


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_decode_missing_blocks_read_as_zero(device, kv):
    """An entry < 0 inside k_len (outside the engine's precondition: -1 only
    after a row's last needed block) reads as zero K/V at its logical
    positions.  This pins the kernels' own convention against a hand-built
    zero-padded reference; the reference's gather would compact the row
    instead (tests/test_oracle.py::test_gather_hole_compacts_like_reference)."""
    say(f"decode missing block {kv}")
    tabs = _tables([600, 300], 8, 5)
    wl = _custom([SeqSlice(tabs[0], 599, 1), SeqSlice(tabs[1], 299, 1)], 8, 2, 8, kv=kv, seed=5)
    bt = wl.context.block_tables.clone()
    bt[0, 2] = -1  # tokens 512..599 of sequence 0 (incl. the new one) are missing
    wl.context.block_tables = bt
    wl.seqs[0] = SeqSlice([tabs[0][0], tabs[0][1], -1], 599, 1)
    # the oracle gathers block -1 as padding; compare only as the eager path sees it
    got = _run(wl)
    ref, rows = oracle_paged(wl, [1])
    compare(got[rows], ref, kv != "bf16", "missing block: intact sequence")
    # sequence 0 by hand: keys 512.. are zero vectors with score 0 and value 0
    kk, vv = cache_blocks_f32(wl.attn, np.asarray(tabs[0][:2]))
    k_all = np.concatenate([kk.reshape(-1, 2, 128), np.zeros((88, 2, 128), np.float32)])
    v_all = np.concatenate([vv.reshape(-1, 2, 128), np.zeros((88, 2, 128), np.float32)])
    q0 = torch.from_numpy(bf16_to_np(wl.q[:1]))
    r0 = AO.attention_cached(q0, torch.from_numpy(k_all)[None], torch.from_numpy(v_all)[None], [0, 1],
                             [0, 600], 8, 2, 128).numpy()
    compare(got[:1], r0, kv != "bf16", "missing block: zero-padded sequence")


# ---------------------------------------------------------------- prefill
def test_prefill_8b_subset(device):
    say("prefill_8b full size")
    wl = W.prefill_8b(device)
    assert wl.context.block_tables is not None
    tot = [s.num_new_tokens * (s.num_new_tokens + s.num_cached_tokens) for s in wl.seqs]
    ids = np.argsort(tot)[:3].tolist()
    _check(wl, ids, "prefill_8b subset")


@pytest.mark.parametrize("kv", ["bf16", "int8", "fp8"])
def test_prefill_prefix_small(device, kv):
    say(f"prefill prefix small {kv}")
    spec = [(0, 130), (256, 77), (512, 300), (768, 2), (256, 64), (0, 1)]
    tabs = _tables([p + n for p, n in spec], 24, 11)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 16, 4, 24, kv=kv, seed=11)
    _check(wl, what=f"prefill prefix small/{kv}")


@pytest.mark.parametrize("g", [1, 4, 5, 8])
def test_prefill_gqa_and_ragged(device, g):
    say(f"prefill g={g}")
    spec = [(256, 129), (0, 63), (512, 200), (0, 1)]
    tabs = _tables([p + n for p, n in spec], 16, 12 + g)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 2 * g, 2, 16, seed=12 + g)
    _check(wl, what=f"prefill g={g}")


def test_local_mode_matches_oracle(device):
    """block_tables None: causal over the step's own k/v."""
    say("local mode")
    lens = [1, 37, 200, 129, 300]
    tabs = _tables(lens, 16, 13)
    wl = _custom([SeqSlice(tabs[i], 0, n) for i, n in enumerate(lens)], 8, 2, 16, seed=13)
    assert wl.context.block_tables is None
    got = _run(wl)
    ref = AO.attention_local(torch.from_numpy(bf16_to_np(wl.q)), torch.from_numpy(bf16_to_np(wl.k)),
                             torch.from_numpy(bf16_to_np(wl.v)), wl.context.cu_seqlens_q.cpu(), 8, 2, 128)
    compare(got, ref.numpy(), False, "local mode")


def test_local_mode_strided_views(device):
    """q/k/v as views of one fused projection buffer (non-contiguous)."""
    say("local mode strided")
    T, Hq, Hkv, D = 300, 8, 2, 128
    g = torch.Generator().manual_seed(14)
    fused = torch.randn(T, Hq + 2 * Hkv, D, generator=g).to(torch.bfloat16).to(device)
    q, k, v = fused[:, :Hq], fused[:, Hq:Hq + Hkv], fused[:, Hq + Hkv:]
    from nanovllm_self_amd import PagedAttention

    a = PagedAttention(Hq, Hkv, D)
    a.attention_compute_dtype = torch.bfloat16
    a.k_cache = torch.zeros(2, 256, Hkv, D, dtype=torch.bfloat16, device=device)
    a.v_cache = torch.zeros_like(a.k_cache)
    a.block_size = 256
    cu = torch.tensor([0, 100, 300], dtype=torch.int32, device=device)
    ctx = Context(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=200, max_seqlen_k=200,
                  slot_mapping=torch.arange(T, dtype=torch.int32, device=device),
                  context_lens=torch.tensor([100, 200], dtype=torch.int32, device=device))
    out = a.forward(q, k, v, ctx)
    torch.cuda.synchronize()
    ref = AO.attention_local(torch.from_numpy(bf16_to_np(q)), torch.from_numpy(bf16_to_np(k)),
                             torch.from_numpy(bf16_to_np(v)), [0, 100, 300], Hq, Hkv, D)
    compare(bf16_to_np(out), ref.numpy(), False, "local strided")


@pytest.mark.parametrize("paged", [False, True])
def test_fp16_inputs_are_cast_to_the_compute_dtype(device, paged):
    """fp16 q / k / v (an fp16 model) with bf16 compute: cast to bf16 before
    the attention, as the reference's q.to(attention_compute_dtype) does
    (attention.py:340-342, 362); the result equals the call on the cast
    inputs bit for bit."""
    say(f"fp16 inputs, bf16 compute, paged={paged}")
    spec = [(256, 100), (0, 37), (512, 1)] if paged else [(0, 100), (0, 37), (0, 1)]
    tabs = _tables([p + n for p, n in spec], 12, 17)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 8, 2, 12, seed=17)
    assert (wl.context.block_tables is not None) == paged
    q16, k16, v16 = (t.to(torch.float16) for t in (wl.q, wl.k, wl.v))
    out16 = wl.attn.forward(q16, k16, v16, wl.context)
    ref = wl.attn.forward(q16.to(torch.bfloat16), k16.to(torch.bfloat16), v16.to(torch.bfloat16), wl.context)
    torch.cuda.synchronize()
    assert out16.dtype == torch.bfloat16
    assert torch.equal(out16, ref)


def test_prefix_equals_fresh(device):
    """A sequence run as cached prefix + chunk gives the rows a fresh prefill
    of the whole sequence gives."""
    say("prefix == fresh")
    P, L = 512, 300
    tabs = _tables([P + L], 8, 15)
    wl = _custom([SeqSlice(tabs[0], P, L)], 8, 2, 8, seed=15)
    paged = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    kb, vb, _ = wl.attn.get_kv_cache(wl.context)
    qf = torch.cat([torch.randn(P, 8, 128, device=device).to(torch.bfloat16), wl.q])
    cu = torch.tensor([0, P + L], dtype=torch.int32, device=device)
    fresh_ctx = Context(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=P + L, max_seqlen_k=P + L,
                        slot_mapping=torch.full((P + L,), -1, dtype=torch.int32, device=device))
    fresh = wl.attn.forward(qf, kb[0], vb[0], fresh_ctx)
    torch.cuda.synchronize()
    compare(bf16_to_np(fresh[P:]), bf16_to_np(paged).astype(np.float32), False, "prefix vs fresh")


def test_rows_without_keys_are_zero(device):
    """q_len > k_len leaves the first rows with no visible key: output 0."""
    say("rows without keys")
    tabs = _tables([40], 4, 16)
    wl = _custom([SeqSlice(tabs[0], 0, 40)], 4, 1, 4, seed=16)
    wl.context.cu_seqlens_k = torch.tensor([0, 30], dtype=torch.int32, device=device)
    wl.context.max_seqlen_k = 30
    wl.context.block_tables = torch.tensor([tabs[0]], dtype=torch.int32, device=device)
    got = _run(wl)
    assert np.all(got[:10] == 0)
    kk, vv = [x.reshape(-1, 1, 128)[:30] for x in cache_blocks_f32(wl.attn, np.asarray(tabs[0]))]
    ref = AO.attention_cached(torch.from_numpy(bf16_to_np(wl.q)), torch.from_numpy(kk)[None],
                              torch.from_numpy(vv)[None], [0, 40], [0, 30], 4, 1, 128)
    compare(got, ref.numpy(), False, "rows without keys")


def test_rows_without_keys_multi_tile(device):
    """q_len > k_len over several 64-key tiles: rows 0 .. 99 see no key (0),
    the rest see a growing prefix; waves hold both kinds of rows."""
    say("rows without keys, multi-tile")
    tabs = _tables([300], 4, 17)
    wl = _custom([SeqSlice(tabs[0], 0, 300)], 8, 2, 4, seed=17)
    wl.context.cu_seqlens_k = torch.tensor([0, 200], dtype=torch.int32, device=device)
    wl.context.max_seqlen_k = 200
    wl.context.block_tables = torch.tensor([tabs[0]], dtype=torch.int32, device=device)
    got = _run(wl)
    assert np.all(got[:100] == 0)
    kk, vv = [x.reshape(-1, 2, 128)[:200] for x in cache_blocks_f32(wl.attn, np.asarray(tabs[0]))]
    ref = AO.attention_cached(torch.from_numpy(bf16_to_np(wl.q)), torch.from_numpy(kk)[None],
                              torch.from_numpy(vv)[None], [0, 300], [0, 200], 8, 2, 128)
    compare(got, ref.numpy(), False, "rows without keys, multi-tile")


@pytest.mark.parametrize("prefix", [0, 256])
def test_prefill_scores_jump_in_later_tiles(device, prefix):
    """Keys of later tiles scaled by 8 and 32: the running max of every row
    jumps by far more than the tile loop lets it lag, twice, after rows have
    accumulated earlier tiles (the max moves and O / l rescale mid-row)."""
    say(f"prefill score jumps, prefix {prefix}")
    L = 700
    tabs = _tables([prefix + L], 8, 18)
    wl = _custom([SeqSlice(tabs[0], prefix, L)], 8, 2, 8, seed=18)
    with torch.no_grad():
        wl.k[320:384] *= 8
        wl.k[520:600] *= 32
    _check(wl, what=f"prefill score jumps/{prefix}")


# ---------------------------------------------------------------- mixed
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_mixed_small(device, kv):
    say(f"mixed small {kv}")
    wl = W.mixed_32b(device, kv=kv, n_decode=24, n_chunks=2, chunk=384)
    _check(wl, what=f"mixed small/{kv}")


def test_mixed_32b_decode_rows(device):
    say("mixed_32b full size")
    wl = W.mixed_32b(device)
    ids = wl.decode_seq_ids()[:6]
    _check(wl, ids, "mixed_32b decode rows")


@pytest.mark.parametrize("bs", [64, 128])
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_small_blocks(device, bs, kv):
    """block_size below the 256-key decode partition: one partition spans
    several blocks (decode), and prefill key tiles cross block boundaries."""
    say(f"block_size {bs} {kv}")
    dec = [700, 1000, 1537, 63, 256]
    pre = [(bs * 3, 200), (0, 333)]
    lens = dec + [p + n for p, n in pre]
    NB = sum((n + bs - 1) // bs for n in lens) + 3
    tabs = _tables(lens, NB, 30 + bs, bs=bs)
    seqs = [SeqSlice(tabs[i], n - 1, 1) for i, n in enumerate(dec)]
    seqs += [SeqSlice(tabs[len(dec) + j], p, n) for j, (p, n) in enumerate(pre)]
    wl = _custom(seqs, 8, 2, NB, kv=kv, seed=31 + bs, bs=bs)
    _check(wl, what=f"block_size {bs}/{kv}")


def test_more_rows_than_one_plan_chunk(device):
    """More than 1024 rows: decode records are planned in chunks of rows and
    prefill tiles take the general (level by level) ordering."""
    say("1100-row batch")
    g = torch.Generator().manual_seed(40)
    n_dec, n_pre = 1080, 20
    dec = torch.randint(1, 700, (n_dec,), generator=g).tolist()
    pre = [(int(p), int(n)) for p, n in zip(torch.randint(0, 4, (n_pre,), generator=g).tolist(),
                                            torch.randint(2, 300, (n_pre,), generator=g).tolist())]
    pre = [(64 * p, n) for p, n in pre]
    lens = dec + [p + n for p, n in pre]
    bs = 64
    NB = sum((n + bs - 1) // bs for n in lens)
    tabs = _tables(lens, NB, 41, bs=bs)
    seqs = [SeqSlice(tabs[i], n - 1, 1) for i, n in enumerate(dec)]
    seqs += [SeqSlice(tabs[n_dec + j], p, n) for j, (p, n) in enumerate(pre)]
    wl = _custom(seqs, 4, 2, NB, seed=42, bs=bs)
    ids = list(range(0, n_dec, 37)) + [n_dec - 1] + list(range(n_dec, n_dec + n_pre))
    _check(wl, ids, "1100-row batch")


@pytest.mark.parametrize("kv", ["bf16", "fp8", "int8"])
def test_decode_step_graph_replay(device, kv):
    """The decode step (the token write inside the decode kernel, then the
    attention) captured in a HIP graph: every replay, with eager calls and
    synchronisations between replays, equals the eager result bit for bit
    (the same kernels on the same inputs; the write rewrites the same
    token)."""
    from nanovllm_self_amd.layers.attention import reserve_attention_workspace

    say(f"graph replay decode_small/{kv}")
    wl = W.decode_small(device, kv=kv)
    attn, ctx = wl.attn, wl.context
    reserve_attention_workspace(wl.num_seqs, 1, int(ctx.max_seqlen_k), attn.num_heads, device,
                                num_kv_heads=attn.num_kv_heads)
    eager = attn.forward(wl.q, wl.k, wl.v, ctx).clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            attn.forward(wl.q, wl.k, wl.v, ctx)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    attn.in_cuda_graph_capture = True
    try:
        with torch.cuda.graph(graph):
            out = attn.forward(wl.q, wl.k, wl.v, ctx)
    finally:
        attn.in_cuda_graph_capture = False
    for r in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager step"
        again = attn.forward(wl.q, wl.k, wl.v, ctx)
        torch.cuda.synchronize()
        assert torch.equal(again, eager), f"eager step after replay {r} differs"
    ref, rows = oracle_paged(wl, list(range(wl.num_seqs)))
    compare(bf16_to_np(out)[rows], ref, kv != "bf16", f"graph replay {kv}")


# ---------------------------------------------------------------- API
def test_forward_profile_and_decode_entry(device):
    say("profile + decode_flashattn")
    wl = W.decode_small(device)
    wl.attn.enable_profile = True
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    assert wl.attn.profile_decode["calls"] == 1 and wl.attn.profile_decode["store"] > 0
    dec = wl.attn.decode_flashattn(wl.q, wl.context)
    torch.cuda.synchronize()
    assert torch.equal(out, dec)
    wl.attn.forward_backend = "torch"
    out2 = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_decode_attention_torch_entry(device):
    """decode_attention_torch (attention.py:586-675) over get_kv_cache's
    gathered K/V equals the paged decode of the same batch; an arbitrary
    mask (holes, an empty row) matches the oracle over the kept keys."""
    say("decode_attention_torch")
    wl = W.decode_small(device)
    attn = wl.attn
    paged = attn.forward(wl.q, wl.k, wl.v, wl.context)  # also stores the step's token
    k_batch, v_batch, kv_mask = attn.get_kv_cache(wl.context)
    got = attn.decode_attention_torch(wl.q, k_batch, v_batch, kv_mask)
    torch.cuda.synchronize()
    compare(bf16_to_np(got), bf16_to_np(paged), False, "decode_attention_torch vs paged decode")

    g = torch.Generator().manual_seed(5)
    B, Lmax, Hq, Hkv, D = 5, 300, 16, 8, 128
    q = torch.randn(B, Hq, D, generator=g).to(torch.bfloat16)
    kb = torch.randn(B, Lmax, Hkv, D, generator=g).to(torch.bfloat16)
    vb = torch.randn(B, Lmax, Hkv, D, generator=g).to(torch.bfloat16)
    mask = torch.rand(B, Lmax, generator=g) < 0.7
    mask[1] = False  # no key: output 0
    mask[2, 64:] = False  # a prefix
    out = attn.decode_attention_torch(q.to(device), kb.to(device), vb.to(device), mask.to(device))
    torch.cuda.synchronize()
    ref = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        keep = mask[b]
        if keep.any():
            ref[b] = AO.attention_cached(q[b:b + 1].float(), kb[b:b + 1][:, keep].float(), vb[b:b + 1][:, keep].float(),
                                         [0, 1], [0, int(keep.sum())], Hq, Hkv, D).numpy()[0]
    compare(bf16_to_np(out), ref, False, "decode_attention_torch vs oracle")
    assert np.all(bf16_to_np(out)[1] == 0)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_determinism_and_batch_split(device, kv):
    """The same call twice gives the same bits (split rows are merged in a
    fixed order), and a sequence's output does not depend on the batch it is
    in: the mixed batch's two halves attended on their own match the whole
    batch's rows (the stream-K split points move, so within the bars)."""
    from nanovllm_self_amd.kv_cache import build_context

    say(f"determinism + batch split {kv}")
    wl = W.mixed_32b(device, kv=kv, n_decode=24, n_chunks=2, chunk=384)
    attn, ctx = wl.attn, wl.context
    first = attn.forward(wl.q, wl.k, wl.v, ctx)
    again = attn.prefill_flashattn(wl.q, wl.k, wl.v, ctx)
    torch.cuda.synchronize()
    assert torch.equal(first, again), "two identical calls differ"
    full = bf16_to_np(first)
    cu = ctx.cu_seqlens_q.cpu().tolist()
    n = len(wl.seqs)
    for part in (list(range(0, n, 2)), list(range(1, n, 2))):  # interleaved halves: decode and prefill rows in both
        sub = build_context([wl.seqs[i] for i in part], wl.block_size, device)
        rows = np.concatenate([np.arange(cu[i], cu[i + 1]) for i in part])
        idx = torch.as_tensor(rows, device=device)
        out = attn.prefill_flashattn(wl.q[idx], wl.k[idx], wl.v[idx], sub)
        torch.cuda.synchronize()
        compare(bf16_to_np(out), full[rows], kv != "bf16", f"batch half {part[:3]}... vs whole batch ({kv})")


def _cache_bytes(attn):
    out = [attn.k_cache.view(torch.uint8).clone(), attn.v_cache.view(torch.uint8).clone()]
    if attn.k_scale_cache is not None:
        out += [attn.k_scale_cache.clone(), attn.v_scale_cache.clone()]
    return out


_STORE_CASES = {
    "decode_small": lambda d: W.decode_small(d),
    "decode_8b": lambda d: W.decode_8b(d),
    "decode_small/fp8": lambda d: W.decode_small(d, kv="fp8"),
    "decode_small/int8": lambda d: W.decode_small(d, kv="int8"),
    "decode_quant/fp8": lambda d: W.decode_quant(d, kv="fp8"),
    "decode_quant/int8": lambda d: W.decode_quant(d, kv="int8"),
}


@pytest.mark.parametrize("which", list(_STORE_CASES))
def test_decode_store_in_kernel_equals_store_then_attend(device, which):
    """forward on a decode batch writes the new tokens inside the decode
    kernel (bf16 values, or fp8 / int8 codes and per-token scales); the cache
    bytes, the scales and the output equal write_kv_cache followed by the
    attention call, bit for bit."""
    say(f"store in the decode kernel: {which}")
    a, b = _STORE_CASES[which](device), _STORE_CASES[which](device)  # identical seeded workloads
    assert a.attn._store_in_decode(a.k, a.v, a.context)
    fused = a.attn.forward(a.q, a.k, a.v, a.context)
    b.attn.write_kv_cache(b.k, b.v, b.context.slot_mapping)
    plain = b.attn.prefill_flashattn(b.q, b.k, b.v, b.context)
    torch.cuda.synchronize()
    assert torch.equal(fused, plain)
    for x, y in zip(_cache_bytes(a.attn), _cache_bytes(b.attn)):
        assert torch.equal(x, y), "cache contents differ"


@pytest.mark.parametrize("kv", ["bf16", "fp8", "int8"])
def test_decode_store_in_kernel_edge_rows(device, kv):
    """A decode row with no visible key still has its token written; a
    negative slot is skipped; a wrapped write_kv_cache is still called."""
    say(f"store in the decode kernel ({kv}): keyless row, skipped slot, wrapped writer")
    tabs = _tables([300, 40, 90], 8, 21)
    seqs = [SeqSlice(tabs[0], 299, 1), SeqSlice(tabs[1], 39, 1), SeqSlice(tabs[2], 89, 1)]
    a, b = _custom(seqs, 8, 2, 8, kv=kv, seed=22), _custom(seqs, 8, 2, 8, kv=kv, seed=22)
    assert a.attn._store_in_decode(a.k, a.v, a.context)
    for wl in (a, b):
        # Row 1 sees no key (k_len 0); row 2's slot is -1.
        ctx = wl.context
        ctx.cu_seqlens_k = torch.tensor([0, 300, 300, 390], dtype=torch.int32, device=device)
        ctx.context_lens = torch.tensor([300, 0, 90], dtype=torch.int32, device=device)
        ctx.slot_mapping = ctx.slot_mapping.clone()
        ctx.slot_mapping[2] = -1
    fused = a.attn.forward(a.q, a.k, a.v, a.context)
    b.attn.write_kv_cache(b.k, b.v, b.context.slot_mapping)
    plain = b.attn.prefill_flashattn(b.q, b.k, b.v, b.context)
    torch.cuda.synchronize()
    assert torch.equal(fused, plain) and torch.all(fused[1] == 0)
    for x, y in zip(_cache_bytes(a.attn), _cache_bytes(b.attn)):
        assert torch.equal(x, y), "cache contents differ"
    calls = []
    inner = a.attn.write_kv_cache
    a.attn.write_kv_cache = lambda k, v, s: (calls.append(1), inner(k, v, s))[1]
    assert not a.attn._store_in_decode(a.k, a.v, a.context)
    again = a.attn.forward(a.q, a.k, a.v, a.context)
    torch.cuda.synchronize()
    assert calls == [1] and torch.equal(again, fused)
    # A wrapped attention method is called too (the write then runs first).
    del a.attn.write_kv_cache
    assert a.attn._store_in_decode(a.k, a.v, a.context)
    seen = []
    inner_attn = a.attn.prefill_flashattn
    a.attn.prefill_flashattn = lambda q, k, v, c: (seen.append(1), inner_attn(q, k, v, c))[1]
    assert not a.attn._store_in_decode(a.k, a.v, a.context)
    third = a.attn.forward(a.q, a.k, a.v, a.context)
    torch.cuda.synchronize()
    assert seen == [1] and torch.equal(third, fused)


def _slot_of(wl, row, pos):
    s = wl.seqs[row]
    bs = wl.block_size
    return s.block_table[pos // bs] * bs + pos % bs


def _fused_vs_plain(a, b):
    """forward() on `a` (one call, decode kernel writes) against
    write_kv_cache + the attention call on `b` (same seeded workload and
    context edits): output and every cache byte equal."""
    fused = a.attn.forward(a.q, a.k, a.v, a.context)
    b.attn.write_kv_cache(b.k, b.v, b.context.slot_mapping)
    plain = b.attn.prefill_flashattn(b.q, b.k, b.v, b.context)
    torch.cuda.synchronize()
    assert torch.equal(fused, plain), "output differs from store-then-attend"
    for x, y in zip(_cache_bytes(a.attn), _cache_bytes(b.attn)):
        assert torch.equal(x, y), "cache contents differ"
    return fused


_SLOT_CASES = ["other_row", "earlier_tile", "keyless_in_range", "missing_last_block"]


@pytest.mark.parametrize("kv", ["bf16", "fp8", "int8"])
@pytest.mark.parametrize("case", _SLOT_CASES)
def test_decode_store_slot_not_own_position(device, kv, case):
    """A decode row whose slot is not its own last position (a distinct slot
    inside another row's keys, in an earlier tile of its own row, the slot
    of a keyless row inside another row's keys, a row whose last block is
    missing) is found on the device and written by every wave of its kv head
    before any load: forward() still equals write_kv_cache followed by the
    attention, bit for bit (the reference's write-then-read,
    attention.py:516, 539)."""
    say(f"store in the decode kernel, slot not the row's own position: {case} {kv}")
    a, b = W.decode_small(device, kv=kv), W.decode_small(device, kv=kv)
    for wl in (a, b):
        ctx = wl.context
        ctx.slot_mapping = ctx.slot_mapping.clone()
        if case == "other_row":
            # row 0's token lands at position 10 of row 1 (read by row 1's waves)
            ctx.slot_mapping[0] = _slot_of(wl, 1, 10)
        elif case == "earlier_tile":
            # row 2's token lands at position 3 of its own keys (its first tile)
            ctx.slot_mapping[2] = _slot_of(wl, 2, 3)
        elif case == "keyless_in_range":
            # row 3 sees no key; its slot is position 40 of row 4
            lens = (ctx.cu_seqlens_k[1:] - ctx.cu_seqlens_k[:-1]).clone()
            lens[3] = 0
            ctx.cu_seqlens_k = torch.cat([torch.zeros(1, dtype=torch.int32, device=device),
                                          torch.cumsum(lens, 0).to(torch.int32)])
            ctx.context_lens = lens.to(torch.int32)
            ctx.slot_mapping[3] = _slot_of(wl, 4, 40)
        else:
            # row 5's last block entry is -1: its slot (position k_len - 1 of
            # the original table) is read by nobody, but is still written
            n = wl.seqs[5].num_cached_tokens
            ctx.block_tables = ctx.block_tables.clone()
            ctx.block_tables[5, n // wl.block_size] = -1
    assert a.attn._store_in_decode(a.k, a.v, a.context)
    _fused_vs_plain(a, b)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_decode_store_slot_cases_at_size(device, kv):
    """The same on the 256-row quantised-decode shape (many groups split every
    row): three rows' slots moved into other rows' keys."""
    say(f"store in the decode kernel, moved slots at size ({kv})")
    a, b = W.decode_quant(device, kv=kv), W.decode_quant(device, kv=kv)
    for wl in (a, b):
        ctx = wl.context
        ctx.slot_mapping = ctx.slot_mapping.clone()
        ctx.slot_mapping[0] = _slot_of(wl, 200, 700)
        ctx.slot_mapping[17] = _slot_of(wl, 17, 100)
        ctx.slot_mapping[255] = _slot_of(wl, 3, 1000)
    _fused_vs_plain(a, b)


def test_decode_store_shared_block_takes_store_path(device, monkeypatch):
    """A row's own last position read by another row through a shared block is
    outside what the decode kernel checks; with verify_decode_slots the layer
    finds it on the host and runs the store kernel first, so the result equals
    store-then-attend; the engine's batches pass the check."""
    say("store in the decode kernel: shared last block, verify_decode_slots")
    from nanovllm_self_amd import _lib
    a, b = W.decode_small(device), W.decode_small(device)
    assert a.attn._decode_slots_private(a.context)
    bs = a.block_size
    n0 = a.seqs[0].num_cached_tokens  # row 0's new token sits at position n0
    lens = (a.context.cu_seqlens_k[1:] - a.context.cu_seqlens_k[:-1]).tolist()
    r2 = next(r for r in range(1, a.num_seqs) if lens[r] > n0 % bs)
    for wl in (a, b):
        ctx = wl.context
        ctx.block_tables = ctx.block_tables.clone()
        # row r2's first block becomes row 0's last block: r2 reads row 0's
        # new-token position
        ctx.block_tables[r2, 0] = ctx.block_tables[0, n0 // bs]
    a.attn.verify_decode_slots = True
    assert a.attn._store_in_decode(a.k, a.v, a.context)
    assert not a.attn._decode_slots_private(a.context)
    lib = _lib.load()
    calls = []
    inner = lib.nvs_store_kvcache
    monkeypatch.setattr(lib, "nvs_store_kvcache", lambda *args: (calls.append(1), inner(*args))[1])
    _fused_vs_plain(a, b)
    assert len(calls) == 2, "the layer must run the store kernel (and b's write_kv_cache one more)"
