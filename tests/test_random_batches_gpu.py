"""Seeded random batches that vary the paths' parameters together: kv heads,
group size, block size, cache dtype and the row mix (decode rows, fresh
prefill rows, prefill rows over a cached prefix), so the kernels are
exercised in combinations the named cases do not list.  Every row of every
batch is checked against the fp32 CPU oracle (tolerances of
tests/gpu_util.py): over the cache for paged batches, over the step's own
k / v for batches without a cached prefix (no block_tables).  A case's draw
is fixed by its seed and printed before the GPU step, so a failure names
its batch."""
import random

import pytest
import torch

from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from oracle import attn_oracle as AO
from tests.gpu_util import bf16_to_np, compare, oracle_paged, say

pytestmark = pytest.mark.gpu


def _draw(seed):
    r = random.Random(1000 + seed)
    Hkv = r.choice([1, 2, 4, 8])
    g = r.choice([1, 2, 3, 4, 5, 8])
    bs = r.choice([64, 128, 256])
    kv = r.choice(["bf16", "int8", "fp8"])
    spec = []
    for _ in range(r.randint(1, 10)):
        u = r.random()
        if u < 0.35:
            spec.append((r.randint(0, 1500), 1))  # decode row
        elif u < 0.65:
            spec.append((0, r.randint(2, 600)))  # fresh prefill
        else:
            spec.append((r.randint(1, 1500), r.randint(2, 400)))  # prefill over a cached prefix
    return Hkv, g, bs, kv, spec


@pytest.mark.parametrize("seed", range(64))
def test_random_batch_matches_oracle(device, seed):
    Hkv, g, bs, kv, spec = _draw(seed)
    say(f"random batch {seed}: Hkv={Hkv} g={g} block_size={bs} cache={kv} rows (cached, new)={spec}")
    lens = [p + n for p, n in spec]
    NB = sum((n + bs - 1) // bs for n in lens) + 2
    gen = torch.Generator().manual_seed(seed)
    tabs = W._tables(gen, lens, bs, NB)
    seqs = [SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)]
    wl = W._assemble("random", seqs, g * Hkv, Hkv, 128, bs, NB, kv, device, gen, seed=seed)
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    got = bf16_to_np(out)
    if wl.context.block_tables is None:
        # No row has a cached prefix: the reference attends over the step's
        # own (unquantised) k / v, whatever the cache dtype.
        ref = AO.attention_local(torch.from_numpy(bf16_to_np(wl.q)), torch.from_numpy(bf16_to_np(wl.k)),
                                 torch.from_numpy(bf16_to_np(wl.v)), wl.context.cu_seqlens_q.cpu(),
                                 g * Hkv, Hkv, 128)
        compare(got, ref.numpy(), False, f"random batch {seed} (local)")
        return
    ref, rows = oracle_paged(wl, list(range(len(spec))))
    compare(got[rows], ref, kv != "bf16", f"random batch {seed}")


@pytest.mark.parametrize("seed", range(16))
def test_random_fp16_batch_matches_oracle(device, seed):
    """The same draws (other seeds) with an fp16 model: fp16 q / k / v and
    cache, fp16 compute and output."""
    Hkv, g, bs, _, spec = _draw(100 + seed)
    say(f"random fp16 batch {seed}: Hkv={Hkv} g={g} block_size={bs} rows (cached, new)={spec}")
    lens = [p + n for p, n in spec]
    NB = sum((n + bs - 1) // bs for n in lens) + 2
    gen = torch.Generator().manual_seed(100 + seed)
    tabs = W._tables(gen, lens, bs, NB)
    seqs = [SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)]
    wl = W._assemble("random-fp16", seqs, g * Hkv, Hkv, 128, bs, NB, "fp16", device, gen, seed=100 + seed)
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    got = bf16_to_np(out)
    if wl.context.block_tables is None:
        ref = AO.attention_local(torch.from_numpy(bf16_to_np(wl.q)), torch.from_numpy(bf16_to_np(wl.k)),
                                 torch.from_numpy(bf16_to_np(wl.v)), wl.context.cu_seqlens_q.cpu(),
                                 g * Hkv, Hkv, 128)
        compare(got, ref.numpy(), False, f"random fp16 batch {seed} (local)")
        return
    ref, rows = oracle_paged(wl, list(range(len(spec))))
    compare(got[rows], ref, False, f"random fp16 batch {seed}")
