"""Prefill over int8 / fp8 caches through the bf16 copy (the prefill rows'
keys and values dequantised as the reference's prefill_torch does,
attention.py:268-273, then the MFMA tile-loop kernel) and through the
classic kernel's own dequantising fill, which serves the call when the
workspace has no room for the copy or the copy would exceed its capacity.
Both against the CPU oracle (quantised-KV bar: max-abs 5e-2, mean-abs
5e-3), and the plan's decision read back from the workspace header."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import _lib
from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from nanovllm_self_amd.layers import attention as A
from oracle import attn_oracle as AO
from tests.gpu_util import bf16_to_np, cache_blocks_f32, compare, oracle_paged, say

pytestmark = pytest.mark.gpu

HDR_SHADOW_TILES, HDR_SHADOW_ON = 9, 10  # int32 words of the plan header


def _batch(spec, Hq, Hkv, kv, seed, bs=256, extra_blocks=3):
    lens = [p + n for p, n in spec]
    NB = sum((n + bs - 1) // bs for n in lens) + extra_blocks
    g = torch.Generator().manual_seed(seed)
    tabs = W._tables(g, lens, bs, NB)
    seqs = [SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)]
    return W._assemble("code prefill", seqs, Hq, Hkv, 128, bs, NB, kv, "cuda", g, seed=seed)


def _header(device):
    ws = A._workspaces[torch.device(device)]
    return ws[:256].view(torch.int32).cpu().numpy()


def _oracle_with_holes(wl, i, table):
    """Oracle rows of sequence i whose block table has entries < 0 (those
    blocks read as zero keys and values, as the eager gather pads them)."""
    s, bs, Hkv = wl.seqs[i], wl.block_size, wl.attn.num_kv_heads
    K = s.num_cached_tokens + s.num_new_tokens
    need = (K + bs - 1) // bs
    kk, vv = cache_blocks_f32(wl.attn, np.asarray([max(b, 0) for b in table[:need]]))
    hole = np.asarray([b < 0 for b in table[:need]])
    kk[hole] = 0.0
    vv[hole] = 0.0
    k_all = kk.reshape(-1, Hkv, 128)[:K]
    v_all = vv.reshape(-1, Hkv, 128)[:K]
    cu_q = wl.context.cu_seqlens_q.cpu().tolist()
    q = torch.from_numpy(bf16_to_np(wl.q[cu_q[i]:cu_q[i + 1]]))
    ref = AO.attention_cached(q, torch.from_numpy(k_all)[None], torch.from_numpy(v_all)[None],
                              [0, s.num_new_tokens], [0, K], wl.attn.num_heads, Hkv, 128).numpy()
    return ref, np.arange(cu_q[i], cu_q[i + 1])


def _run_checked(wl, ids, what, holes=None):
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    hdr = _header(wl.q.device)
    got = bf16_to_np(out)
    ref, rows = oracle_paged(wl, ids)
    compare(got[rows], ref, True, what)
    for i, table in (holes or {}).items():
        ref, rows = _oracle_with_holes(wl, i, table)
        compare(got[rows], ref, True, f"{what}: sequence {i} with a missing block")
    return got, hdr


@pytest.mark.parametrize("bs", [256, 64])
@pytest.mark.parametrize("kv", ["int8", "fp8"])
def test_copy_and_fill_paths_match_oracle(device, kv, bs, monkeypatch):
    """The same batch (fresh and prefix-cached prefill rows, decode rows, a
    missing block) through the copy, then with the workspace of the plain
    size (no room for the copy: the classic kernel's fill)."""
    say(f"code-cache prefill paths {kv} bs={bs}")
    spec = [(0, 300), (bs * 2, 257), (bs, 64), (4 * bs, 2), (bs, 1), (777, 1), (0, 130)]
    wl = _batch(spec, 16, 4, kv, seed=50 + bs, bs=bs)
    # A missing block inside sequence 1's prefix reads as zero keys and values.
    table1 = list(wl.seqs[1].block_table)
    table1[1] = -1
    bt = wl.context.block_tables.clone()
    bt[1, 1] = -1
    wl.context.block_tables = bt
    holes = {1: table1}
    ids = [i for i in range(len(spec)) if i != 1]
    copy_out, hdr = _run_checked(wl, ids, f"copy path {kv}/{bs}", holes)
    pre_rows = [i for i, (p, n) in enumerate(spec) if n > 1]
    tiles = sum((spec[i][0] + spec[i][1] + 63) // 64 for i in pre_rows)
    assert hdr[HDR_SHADOW_ON] == 1 and hdr[HDR_SHADOW_TILES] == tiles
    lib = _lib.load()
    plain = lib.nvs_attention_workspace_bytes
    monkeypatch.setattr(lib, "nvs_attention_workspace_bytes_cache", lambda *a: plain(*a[:7]))
    fill_out, hdr = _run_checked(wl, ids, f"fill path {kv}/{bs}", holes)
    assert hdr[HDR_SHADOW_ON] == 0
    # Decode rows come from the same decode waves either way (inside the
    # prefill launch with the copy, a decode launch of their own without it):
    # with this few decode tiles (T <= 34) both split them over T / 4 groups
    # alike.
    dec = [i for i, (p, n) in enumerate(spec) if n == 1]
    rows = np.concatenate([np.arange(int(wl.context.cu_seqlens_q[i]), int(wl.context.cu_seqlens_q[i + 1]))
                           for i in dec])
    assert np.array_equal(copy_out[rows], fill_out[rows])


def test_copy_over_capacity_falls_back_on_the_device(device):
    """72 prefill rows of 4000 keys need 72 x 63 copy tiles, more than the
    copy's 1 GiB holds at 8 kv heads (4096 tiles): the plan turns the copy
    off and the classic kernel serves the whole call."""
    say("code-cache prefill over the copy's capacity")
    spec = [(3998, 2)] * 72
    wl = _batch(spec, 32, 8, "fp8", seed=61)
    ids = [0, 35, 71]
    _, hdr = _run_checked(wl, ids, "copy over capacity")
    assert hdr[HDR_SHADOW_TILES] == 72 * 63 and hdr[HDR_SHADOW_ON] == 0


def test_copy_over_capacity_with_decode_rows(device):
    """The over-capacity batch with decode rows beside it: the prefill
    launch's first work-groups still stream the decode rows (the plan turned
    only its prefill part off), the classic kernel serves the prefill rows,
    and the merge after them joins the split decode rows."""
    say("code-cache prefill over capacity, decode rows")
    spec = [(3998, 2)] * 72 + [(9000, 1), (4000, 1), (12000, 1)]
    wl = _batch(spec, 32, 8, "fp8", seed=62)
    ids = [0, 71, 72, 73, 74]
    _, hdr = _run_checked(wl, ids, "copy over capacity, decode rows")
    assert hdr[HDR_SHADOW_ON] == 0


@pytest.mark.parametrize("g", [1, 2, 5, 8])
def test_copy_path_gqa_groups(device, g):
    """Group sizes whose query tiling the two prefill kernels share (1, 2, 8:
    the copy) and one they do not (5: the classic kernel's fill), fp8."""
    say(f"code-cache prefill g={g}")
    spec = [(256, 129), (0, 63), (512, 200), (0, 1)]
    wl = _batch(spec, 2 * g, 2, "fp8", seed=70 + g)
    _, hdr = _run_checked(wl, list(range(len(spec))), f"code-cache prefill g={g}")
    assert hdr[HDR_SHADOW_ON] == (0 if g == 5 else 1)
