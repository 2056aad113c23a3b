"""Batches of many short prefill rows, so that each work-group of the tile-loop
kernel runs long sequences of unit transitions: units chained into the next
(two tiles or more, followed by a unit with keys), one-tile units (which end
the pipeline: a drain, then a fresh start), and units whose rows see no key
(rows with fewer keys than new tokens: their first rows attend nothing, the
kernel writes zeros and starts the next unit afresh).  The loop's V tiles
rotate through three LDS buffers across all of these paths.  Every row of
every batch is checked against the fp32 CPU oracle (reference semantics:
attention.py:303-375 with cu_seqlens_k below cu_seqlens_q for the keyless
rows), and the rows without a visible key must be exactly zero."""
import random

import numpy as np
import pytest
import torch

from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from oracle import attn_oracle as AO
from tests.gpu_util import bf16_to_np, compare, oracle_paged_inputs, say

pytestmark = pytest.mark.gpu


def _draw(seed):
    """(cached, new, keys dropped) per row: one-tile rows, short rows over a
    prefix, and rows whose first `drop` new tokens see no key."""
    r = random.Random(500 + seed)
    rows = []
    for _ in range(r.randint(80, 120)):
        u = r.random()
        if u < 0.35:
            rows.append((0, r.randint(2, 64), 0))
        elif u < 0.75:
            rows.append((r.choice([0, 64, 192, 300]), r.randint(2, 160), 0))
        else:
            n = r.randint(70, 260)
            rows.append((0, n, r.randint(1, n - 1)))
    return rows


@pytest.mark.parametrize("seed,bs,kv", [(0, 64, "bf16"), (1, 256, "bf16"), (2, 128, "fp8")])
def test_many_short_units(device, seed, bs, kv):
    rows = _draw(seed)
    Hq, Hkv = 8, 2
    say(f"short units {seed}: block_size={bs} cache={kv} {len(rows)} rows "
        f"({sum(1 for *_, d in rows if d)} with keyless rows)")
    lens = [p + n for p, n, _ in rows]
    NB = sum((x + bs - 1) // bs for x in lens) + 2
    gen = torch.Generator().manual_seed(seed)
    tabs = W._tables(gen, lens, bs, NB)
    wl = W._assemble("units", [SeqSlice(tabs[i], p, n) for i, (p, n, _) in enumerate(rows)], Hq, Hkv, 128, bs,
                     NB, kv, device, gen, seed=seed)
    # Rows with dropped keys attend only the first cached + new - drop keys.
    klens = [p + n - d for p, n, d in rows]
    wl.context.cu_seqlens_k = torch.tensor(np.concatenate([[0], np.cumsum(klens)]), dtype=torch.int32,
                                           device=device)
    wl.context.max_seqlen_k = max(klens)
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    got = bf16_to_np(out)
    args, qrows = oracle_paged_inputs(wl, list(range(len(rows))))
    args = list(args)
    args[5] = np.concatenate([[0], np.cumsum(klens)]).tolist()  # cu_seqlens_k
    args[6] = klens                                             # context lengths
    ref = AO.paged_attention(*args).numpy()
    compare(got[qrows], ref, kv != "bf16", f"short units {seed}")
    cu_q = wl.context.cu_seqlens_q.cpu().tolist()
    for i, (p, n, d) in enumerate(rows):
        if d:  # new token r sees keys 0 .. r + (k_len - n): none while r < d - p
            blind = d - p
            assert np.all(got[cu_q[i]:cu_q[i] + blind] == 0), f"row {i}: rows without keys not zero"
