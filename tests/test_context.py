"""Step metadata (prepare_model_input, model_runner.py:461-532).

CPU: the oracle (oracle/context_oracle.py) against hand-computed vectors and
closed forms, and the host builder (kv_cache.build_context) against the
oracle.  GPU: the device builder (nvs_build_context through
kv_cache.build_context_on_device and through the C ABI) bit-exact against
the oracle."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd.kv_cache import SeqSlice, build_context
from oracle import context_oracle as CO


def _as_tuples(seqs):
    return [(s.block_table, s.num_cached_tokens, s.num_new_tokens, s.need_logits) for s in seqs]


def _random_batch(rng, B, bs, kind, pool=100000):
    """Sequences over disjoint physical blocks (a shuffled pool)."""
    ids = rng.permutation(pool)
    seqs, used = [], 0
    for i in range(B):
        if kind == "decode":
            cached, new = int(rng.integers(0, 4 * bs)), 1
        elif kind == "prefill":
            cached, new = bs * int(rng.integers(0, 9)), int(rng.integers(1, 3 * bs))
        else:  # mixed, including sequences that bring no new token
            cached, new = int(rng.integers(0, 6 * bs)), int(rng.choice([0, 1, 1, 2, 37, 2 * bs]))
        n = (cached + new + bs - 1) // bs + int(rng.integers(0, 3))
        seqs.append(SeqSlice([int(x) for x in ids[used:used + n]], cached, new, bool(rng.integers(0, 2))))
        used += n
    return seqs


# ---------------------------------------------------------------- CPU: oracle


def test_oracle_docstring_example():
    # model_runner.py:463-468: seqA = 5 tokens, seqB = 3 tokens packed as
    # positions [0, 1, 2, 3, 4, 0, 1, 2].
    r = CO.prepare_model_input([([0], 0, 5, True), ([1], 0, 3, True)], 256)
    assert r["positions"] == [0, 1, 2, 3, 4, 0, 1, 2]
    assert r["slot_mapping"] == [0, 1, 2, 3, 4, 256, 257, 258]
    assert r["cu_seqlens_q"] == r["cu_seqlens_k"] == [0, 5, 8]
    assert r["block_tables"] is None


def test_oracle_hand_computed_vectors():
    # bs 4.  seq 0: cached 5, one new token at position 5 -> block 1 (id 2),
    # offset 1 -> slot 9.  seq 1: positions 4..8 -> blocks 1,1,1,1,2 (ids
    # 3,3,3,3,0) -> 12..15, 0.  seq 2: positions 0..2 in block id 6 -> 24..26.
    seqs = [([7, 2], 5, 1, True), ([1, 3, 0], 4, 5, False), ([6], 0, 3, True)]
    r = CO.prepare_model_input(seqs, 4)
    assert r["slot_mapping"] == [9, 12, 13, 14, 15, 0, 24, 25, 26]
    assert r["positions"] == [5, 4, 5, 6, 7, 8, 0, 1, 2]
    assert r["cu_seqlens_q"] == [0, 1, 6, 9] and r["cu_seqlens_k"] == [0, 6, 15, 18]
    assert r["context_lens"] == [6, 9, 3] and (r["max_seqlen_q"], r["max_seqlen_k"]) == (5, 9)
    assert r["block_tables"] == [[7, 2, -1], [1, 3, 0], [6, -1, -1]]
    assert r["seq_need_compute_logits"] == [0, 2]


def test_oracle_contiguous_tables_give_linear_slots():
    # Sequence b owning blocks b*W .. b*W + W - 1 in order: slot = b*W*bs + pos.
    bs, W = 16, 5
    seqs = [(list(range(b * W, b * W + W)), c, n, True) for b, (c, n) in enumerate([(0, 80), (33, 1), (17, 40), (79, 1)])]
    r = CO.prepare_model_input(seqs, bs)
    want = [b * W * bs + p for b, (_, c, n, _) in enumerate(seqs) for p in range(c, c + n)]
    assert r["slot_mapping"] == want


def test_oracle_decode_batch_points_at_each_last_token():
    rng = np.random.default_rng(0)
    bs = 256
    seqs = _random_batch(rng, 64, bs, "decode")
    r = CO.prepare_model_input(_as_tuples(seqs), bs)
    for s, slot, pos in zip(seqs, r["slot_mapping"], r["positions"]):
        last = s.num_cached_tokens
        assert pos == last and slot == s.block_table[last // bs] * bs + last % bs
    assert r["context_lens"] == [s.num_cached_tokens + 1 for s in seqs]


def test_oracle_slots_are_distinct_and_decompose():
    rng = np.random.default_rng(1)
    bs = 32
    seqs = _random_batch(rng, 40, bs, "mixed")
    r = CO.prepare_model_input(_as_tuples(seqs), bs)
    slots, pos = np.array(r["slot_mapping"]), np.array(r["positions"])
    assert len(set(slots.tolist())) == len(slots)
    b_of = np.repeat(np.arange(len(seqs)), [s.num_new_tokens for s in seqs])
    assert np.array_equal(slots % bs, pos % bs)
    assert all(slots[t] // bs == seqs[b_of[t]].block_table[pos[t] // bs] for t in range(len(slots)))


@pytest.mark.parametrize("kind", ["decode", "prefill", "mixed"])
def test_host_builder_matches_oracle(kind):
    rng = np.random.default_rng({"decode": 2, "prefill": 3, "mixed": 4}[kind])
    bs = 256
    seqs = _random_batch(rng, 48, bs, kind)
    r = CO.prepare_model_input(_as_tuples(seqs), bs)
    c = build_context(seqs, bs, "cpu")
    for f in ("cu_seqlens_q", "cu_seqlens_k", "slot_mapping", "context_lens", "seq_need_compute_logits"):
        assert getattr(c, f).tolist() == r[f], f
    assert (c.max_seqlen_q, c.max_seqlen_k) == (r["max_seqlen_q"], r["max_seqlen_k"])
    assert (c.block_tables is None and r["block_tables"] is None) or c.block_tables.tolist() == r["block_tables"]


# ---------------------------------------------------------------- GPU


def _check_device(seqs, bs, device):
    from nanovllm_self_amd.kv_cache import build_context_on_device

    ctx, positions = build_context_on_device(seqs, bs, device)
    torch.cuda.synchronize()
    r = CO.prepare_model_input(_as_tuples(seqs), bs)
    for f in ("cu_seqlens_q", "cu_seqlens_k", "slot_mapping", "context_lens", "seq_need_compute_logits"):
        t = getattr(ctx, f)
        assert t.dtype == torch.int32 and t.is_cuda, f
        assert t.cpu().tolist() == r[f], f
    assert positions.dtype == torch.int64 and positions.cpu().tolist() == r["positions"]
    assert (ctx.max_seqlen_q, ctx.max_seqlen_k) == (r["max_seqlen_q"], r["max_seqlen_k"])
    if r["block_tables"] is None:
        assert ctx.block_tables is None
    else:
        assert ctx.block_tables.cpu().tolist() == r["block_tables"]


@pytest.mark.gpu
@pytest.mark.parametrize("kind,B,bs", [("decode", 256, 256), ("prefill", 16, 256), ("mixed", 131, 256),
                                        ("mixed", 300, 16), ("decode", 4096, 256), ("prefill", 1, 1)])
def test_device_builder_matches_oracle(device, kind, B, bs):
    from tests.gpu_util import say

    say(f"build_context_on_device {kind} B={B} bs={bs}")
    rng = np.random.default_rng(B * 7 + bs)
    _check_device(_random_batch(rng, B, bs, kind), bs, device)


@pytest.mark.gpu
def test_device_builder_edge_batches(device):
    from nanovllm_self_amd.kv_cache import build_context_on_device
    from tests.gpu_util import say

    say("build_context_on_device edge batches")
    # Fresh prompts only (block_tables None), a sequence with no new tokens
    # between others, and positions crossing many 4096-token work-group spans.
    _check_device([SeqSlice([0], 0, 3), SeqSlice([1], 0, 2)], 4, device)
    _check_device([SeqSlice([5, 6], 3, 2), SeqSlice([2], 1, 0), SeqSlice([9], 0, 1)], 4, device)
    _check_device([SeqSlice(list(range(100, 160)), 0, 15000), SeqSlice(list(range(0, 60)), 7, 14000)], 256, device)
    ctx, pos = build_context_on_device([], 256, device)
    torch.cuda.synchronize()
    assert ctx.cu_seqlens_q.cpu().tolist() == [0] and pos.numel() == 0 and ctx.slot_mapping.numel() == 0
    with pytest.raises(IndexError):
        build_context_on_device([SeqSlice([3], 250, 10)], 256, device)


@pytest.mark.gpu
def test_c_abi_maps_unmapped_positions_to_minus_one(device):
    """Through the C ABI without the host checks: a position past the end of
    its block list or on a -1 entry gets slot -1; tokens past the sum of
    num_new get -1 and position 0; the padded table is cut or padded to the
    width asked for."""
    from nanovllm_self_amd import _lib
    from tests.gpu_util import say

    say("nvs_build_context unmapped positions")
    bs = 4
    counts = torch.tensor([6, 0, 3, 9], dtype=torch.int32, device=device)  # cached 6, 0; new 3, 9
    offsets = torch.tensor([0, 2, 4], dtype=torch.int32, device=device)
    ids = torch.tensor([4, 5, -1, 7], dtype=torch.int32, device=device)
    T = 12 + 2
    cu = torch.full((2 * 3 + 2,), -7, dtype=torch.int32, device=device)
    slots = torch.full((T,), -7, dtype=torch.int32, device=device)
    pos = torch.full((T,), -7, dtype=torch.int64, device=device)
    lib = _lib.load()

    def call(width, table, num_seqs=2):
        _lib.check(lib.nvs_build_context(counts.data_ptr(), counts.data_ptr() + 8, num_seqs, offsets.data_ptr(),
                                         ids.data_ptr(), 4, bs, T, cu.data_ptr(), cu.data_ptr() + 12,
                                         cu.data_ptr() + 24, slots.data_ptr(), pos.data_ptr(), _lib.ptr(table),
                                         width, _lib.stream_of(cu)), "build_context")

    wide = torch.full((2, 3), -7, dtype=torch.int32, device=device)
    call(3, wide)
    torch.cuda.synchronize()
    # seq 0: positions 6, 7 in block 1 (id 5) -> 22, 23; position 8 is block 2,
    # past its list -> -1.  seq 1: positions 0-3 on the -1 entry, 4-7 in id 7,
    # position 8 past its list.
    assert slots.cpu().tolist() == [22, 23, -1, -1, -1, -1, -1, 28, 29, 30, 31, -1, -1, -1]
    assert pos.cpu().tolist() == [6, 7, 8, 0, 1, 2, 3, 4, 5, 6, 7, 8, 0, 0]
    assert cu.cpu().tolist() == [0, 3, 12, 0, 9, 18, 9, 9]
    assert wide.cpu().tolist() == [[4, 5, -1], [-1, 7, -1]]
    narrow = torch.full((2, 1), -7, dtype=torch.int32, device=device)
    call(1, narrow)
    torch.cuda.synchronize()
    assert narrow.cpu().tolist() == [[4], [-1]]
    with pytest.raises(RuntimeError, match="num_seqs"):
        call(1, narrow, num_seqs=4097)
