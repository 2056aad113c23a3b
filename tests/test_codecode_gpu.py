"""Decode rows streamed by the prefill launch (a paged call with prefill rows
that the tile-loop kernel serves): the plan gives the decode part a number
of work-groups in steps of 8 and of 2 Hkv, the decode waves of each XCD form
groups, and rows split across groups are merged by a launch after the
prefill.  These cases vary what that mapping depends on (kv-head counts
whose steps differ: 3 -> 24, 5 -> 40, 16 -> 32 work-groups), keyless decode
rows beside prefill rows, and a prefill-only call whose workspace last held
a decode call's partials and records, against the fp32 CPU oracle
(reference semantics: attention.py:303-375, the paged flash call over
q_len 1 and q_len > 1 rows alike)."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from tests.gpu_util import bf16_to_np, compare, oracle_paged, oracle_seq_rows, say

pytestmark = pytest.mark.gpu


def _custom(seqs, Hq, Hkv, NB, kv="bf16", seed=7, bs=256, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return W._assemble("custom", seqs, Hq, Hkv, 128, bs, NB, kv, device, g, seed=seed)


def _tables(lens, NB, seed, bs=256):
    g = torch.Generator().manual_seed(seed)
    return W._tables(g, lens, bs, NB)


def _run(wl):
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    return bf16_to_np(out)


@pytest.mark.parametrize("Hkv,g", [(3, 2), (5, 1), (16, 2)])
@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_mixed_odd_kv_heads(device, Hkv, g, kv):
    """Long decode rows (split across the decode groups of several XCDs)
    beside prefill rows of several units; every decode row and the first
    and last 64 rows of each prefill row are checked."""
    say(f"co-decode Hkv={Hkv} g={g} {kv}")
    spec = [(9000, 1), (0, 300), (12000, 1), (1024, 700), (700, 1), (256, 129), (5000, 1)]
    tabs = _tables([p + n for p, n in spec], 160, 60 + Hkv)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], g * Hkv, Hkv, 160, kv=kv,
                 seed=60 + Hkv)
    got = _run(wl)
    dec = [i for i, (_, n) in enumerate(spec) if n == 1]
    ref, rows = oracle_paged(wl, dec)
    compare(got[rows], ref, kv != "bf16", f"co-decode Hkv={Hkv} {kv}: decode rows")
    for i, (_, n) in enumerate(spec):
        if n == 1:
            continue
        for r0 in sorted({0, max(0, n - 64)}):
            ref, rows = oracle_seq_rows(wl, i, r0, min(n, r0 + 64))
            compare(got[rows], ref, kv != "bf16", f"co-decode Hkv={Hkv} {kv}: seq {i} rows {r0}..")


def test_mixed_keyless_decode_rows(device):
    """Decode rows that see no key (k_len 0) beside prefill rows: the plan
    still gives the decode part work-groups, whose waves zero those rows."""
    say("co-decode keyless decode rows")
    spec = [(0, 200), (300, 1), (512, 150), (700, 1)]
    tabs = _tables([p + n for p, n in spec], 24, 71)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 16, 4, 24, seed=71)
    # Rows 1 and 3 keep their query row and lose their keys.
    cu_k = wl.context.cu_seqlens_k.cpu().tolist()
    lens = [cu_k[i + 1] - cu_k[i] for i in range(len(spec))]
    lens[1] = lens[3] = 0
    wl.context.cu_seqlens_k = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32,
                                           device=device)
    wl.context.max_seqlen_k = max(lens)
    # The layer's output tensor starts uninitialised: the zeros are the kernel's.
    got = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    cu_q = wl.context.cu_seqlens_q.cpu().tolist()
    out = bf16_to_np(got)
    for i in (1, 3):
        assert np.all(out[cu_q[i]:cu_q[i + 1]] == 0), f"keyless decode row {i} not zero"
    for i in (0, 2):
        n = spec[i][1]
        ref, rows = oracle_seq_rows(wl, i, 0, min(n, 64))
        compare(out[rows], ref, False, f"keyless-decode batch: prefill seq {i}")


def test_prefill_call_after_decode_call(device):
    """A decode-only call (its decode launch leaves a group count and split
    rows' records in the workspace) and then a prefill-only call on the same
    workspace: that call's plan finds no decode row and clears the count, so
    the merge after its prefill launch finds nothing to merge."""
    say("prefill after decode, one workspace")
    dec = W.decode_8b(device)
    _ = dec.attn.forward(dec.q, dec.k, dec.v, dec.context)
    torch.cuda.synchronize()
    spec = [(0, 300), (512, 257), (256, 64)]
    tabs = _tables([p + n for p, n in spec], 16, 81)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 32, 8, 16, seed=81)
    got = _run(wl)
    ref, rows = oracle_paged(wl, [0, 1, 2])
    compare(got[rows], ref, False, "prefill after decode")
