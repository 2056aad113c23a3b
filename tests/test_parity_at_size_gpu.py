"""Parity on the long-key paths of the measured shapes, at full size.

The oracle checks contiguous row blocks of the longest sequences
(gpu_util.oracle_seq_rows: a row block [r0, r1) of a sequence with P cached
tokens is a sequence of r1 - r0 new tokens over P + r1 keys under the same
bottom-right mask), so the CPU cost is the block's, not the sequence's.
Covered: the longest prefill_8b sequence (its first query tile, tiles
across the middle, its last, partial tile); mixed_32b's chunk over the
longest cached prefix and its longest and shortest decode rows, bf16 and
fp8; its four chunks alone (the prefill batch bench.py times on long
units); the same shape with a chunk over 16384 cached tokens and decode rows
of 24K-32K keys; a block_size-64 prefill past 32768 keys, where the prefill kernel
reloads the block-table window it stages in LDS (512 entries).  Bars as in
gpu_util: bf16 max-abs 2e-2 / mean-abs 2e-3, quantised max-abs 5e-2 (reference
attention.py:441-498)."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from tests.gpu_util import bf16_to_np, compare, oracle_paged, oracle_seq_rows, say

pytestmark = pytest.mark.gpu


def _run(wl):
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    return bf16_to_np(out)


def _check_blocks(wl, got, i, blocks, what):
    for r0, r1 in blocks:
        ref, rows = oracle_seq_rows(wl, i, r0, r1)
        compare(got[rows], ref, wl.kv != "bf16", f"{what} rows [{r0}, {r1})")


def test_prefill_8b_longest_sequence(device):
    say("prefill_8b: row blocks of the longest sequences")
    wl = W.prefill_8b(device)
    got = _run(wl)
    tot = [s.num_cached_tokens + s.num_new_tokens for s in wl.seqs]
    # the sequence with the most keys, and the one with the most new tokens
    for i in sorted({int(np.argmax(tot)), int(np.argmax([s.num_new_tokens for s in wl.seqs]))}):
        L = wl.seqs[i].num_new_tokens
        mid = (L // 2) // 64 * 64
        blocks = [(0, 64), (mid - 16, mid + 48), (L - 100, L)]
        _check_blocks(wl, got, i, blocks, f"prefill_8b seq {i} (P={wl.seqs[i].num_cached_tokens}, L={L})")


@pytest.fixture(scope="module", params=["bf16", "fp8"])
def mixed(request, device):
    wl = W.mixed_32b(device, kv=request.param)
    got = _run(wl)
    yield wl, got
    del wl
    torch.cuda.empty_cache()


def test_mixed_32b_longest_chunk(mixed):
    wl, got = mixed
    say(f"mixed_32b/{wl.kv}: chunk over the longest prefix")
    pre = wl.prefill_seq_ids()
    i = max(pre, key=lambda j: wl.seqs[j].num_cached_tokens)
    assert wl.seqs[i].num_cached_tokens >= 8 * 1024  # 8448 in the seed-4 draw
    L = wl.seqs[i].num_new_tokens
    _check_blocks(wl, got, i, [(0, 64), (1000, 1064), (L - 64, L)],
                  f"mixed_32b/{wl.kv} chunk {i} (P={wl.seqs[i].num_cached_tokens})")


def test_mixed_32b_chunks_alone(device):
    """The batch bench.py times for the prefill kernel on long units:
    mixed_32b's four chunks without the decode rows (no q_len == 1 row: the
    decode launch finds no tile).  The same prefixes and tables as in the
    full draw; row blocks of every chunk against the oracle."""
    say("mixed_32b prefill chunks alone (bf16)")
    wl = W.mixed_32b_chunks(device)
    full = W._mixed_32b_seqs(W._gen(4), 128, 4, 2048)[128:]
    assert [(s.num_cached_tokens, s.num_new_tokens) for s in wl.seqs] == \
        [(s.num_cached_tokens, s.num_new_tokens) for s in full]
    assert all(s.num_new_tokens == 2048 for s in wl.seqs)
    got = _run(wl)
    for i, s in enumerate(wl.seqs):
        _check_blocks(wl, got, i, [(0, 32), (2048 - 64, 2048)],
                      f"mixed_32b chunk {i} alone (P={s.num_cached_tokens})")
    del wl
    torch.cuda.empty_cache()


def test_mixed_32b_extreme_decode_rows(mixed):
    wl, got = mixed
    say(f"mixed_32b/{wl.kv}: longest and shortest decode rows")
    dec = wl.decode_seq_ids()
    ctx = [wl.seqs[j].num_cached_tokens + 1 for j in dec]
    order = np.argsort(ctx)
    ids = [dec[int(x)] for x in list(order[-4:]) + list(order[:2])]
    assert max(ctx) >= 24 * 1024
    ref, rows = oracle_paged(wl, ids)
    compare(got[rows], ref, wl.kv != "bf16", f"mixed_32b/{wl.kv} decode rows {ids}")


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_mixed_32b_shape_chunk_over_16k(device, kv):
    """The Qwen3-32B-like mixed shape at the top of its ranges: a 2048-token
    chunk over the largest cached prefix the shape allows (16384 tokens,
    18432 keys) beside 32 decode rows of 24K-32K keys."""
    say(f"mixed 32b shape: chunk over 16384 cached tokens ({kv})")
    g = torch.Generator().manual_seed(60)
    dec = torch.randint(24 * 1024, 32 * 1024 + 1, (32,), generator=g).tolist()
    lens = dec + [16384 + 2048]
    NB = sum((n + 255) // 256 for n in lens) + 8
    tabs = W._tables(g, lens, 256, NB)
    seqs = [SeqSlice(tabs[i], n - 1, 1) for i, n in enumerate(dec)] + [SeqSlice(tabs[-1], 16384, 2048)]
    wl = W._assemble("mixed_16k", seqs, 64, 8, 128, 256, NB, kv, device, g, seed=61)
    got = _run(wl)
    _check_blocks(wl, got, len(dec), [(0, 64), (960, 1024), (1984, 2048)], f"mixed 16k chunk/{kv}")
    ref, rows = oracle_paged(wl, [int(np.argmax(dec)), int(np.argmin(dec))])
    compare(got[rows], ref, kv != "bf16", f"mixed 16k decode rows/{kv}")


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_prefill_block_window_reload(device, kv):
    """block_size 64 and 36 140 keys (565 blocks): the prefill kernel's
    512-entry block-table window is reloaded inside the item."""
    say(f"prefill block-table window reload ({kv})")
    bs = 64
    spec = [(64 * 560, 300), (64 * 10, 100)]
    lens = [p + n for p, n in spec]
    NB = sum((n + bs - 1) // bs for n in lens) + 5
    g = torch.Generator().manual_seed(50)
    tabs = W._tables(g, lens, bs, NB)
    seqs = [SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)]
    wl = W._assemble("window", seqs, 8, 2, 128, bs, NB, kv, device, torch.Generator().manual_seed(51), seed=51)
    assert (lens[0] + bs - 1) // bs > 512
    got = _run(wl)
    _check_blocks(wl, got, 0, [(0, 64), (136, 200), (236, 300)], f"window reload/{kv}")
    ref, rows = oracle_paged(wl, [1])
    compare(got[rows], ref, kv != "bf16", f"window reload/{kv} short sequence")
