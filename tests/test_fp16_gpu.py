"""fp16 compute (an fp16 model: fp16 q / k / v, fp16 cache, fp16 MFMA and P,
fp16 output), the reference's flash path with attention_compute_dtype
float16 (attention.py:326-336, 338-375; config.py:6-25), against the fp32
CPU oracle.  Bars: the bf16 suite's (max-abs 2e-2 beyond the output's own
rounding, mean-abs 2e-3), and a mean-abs error below what rounding the
oracle's own output to bf16 costs: no bf16 computation can get under that
floor, so it shows that the fp16 path ran."""
import numpy as np
import pytest
import torch

from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.kv_cache import SeqSlice
from oracle import attn_oracle as AO
from oracle import kv_oracle as KO
from tests.gpu_util import bf16_to_np, compare, oracle_paged, oracle_seq_rows, say

pytestmark = pytest.mark.gpu

def _custom(seqs, Hq, Hkv, NB, seed=7, bs=256, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    return W._assemble("custom-fp16", seqs, Hq, Hkv, 128, bs, NB, "fp16", device, g, seed=seed)


def _tables(lens, NB, seed, bs=256):
    g = torch.Generator().manual_seed(seed)
    return W._tables(g, lens, bs, NB)


def _run(wl):
    out = wl.attn.forward(wl.q, wl.k, wl.v, wl.context)
    torch.cuda.synchronize()
    assert out.shape == wl.q.shape and out.dtype == torch.float16
    return bf16_to_np(out)


def _check_f16(got, ref, what):
    _, mean = compare(got, ref, False, what)
    floor = float(np.abs(KO.round_to_bf16(ref) - ref.astype(np.float64)).mean())
    say(f"{what}: mean-abs {mean:.3e} against the bf16 rounding floor {floor:.3e}")
    assert mean < floor, f"{what}: mean-abs {mean:.3e} not below bf16 output rounding {floor:.3e}"


def _check(wl, seq_ids=None, what=""):
    got = _run(wl)
    ids = list(range(wl.num_seqs)) if seq_ids is None else list(seq_ids)
    ref, rows = oracle_paged(wl, ids)
    _check_f16(got[rows], ref, what or wl.name)


def test_decode_small_fp16(device):
    say("decode_small fp16")
    wl = W.decode_small(device, kv="fp16")
    assert wl.attn.k_cache.dtype == torch.float16 and wl.q.dtype == torch.float16
    _check(wl, what="decode_small/fp16")


def test_decode_split_rows_fp16(device):
    """Few long rows over the whole chip: every row is split across decode
    groups, so the merge (run in the plan launch of a call with prefill
    rows, or its own launch) writes the fp16 outputs."""
    say("decode split rows fp16")
    lens = [9000, 12000, 7000]
    tabs = _tables(lens, 160, 21)
    wl = _custom([SeqSlice(tabs[i], lens[i] - 1, 1) for i in range(3)], 32, 8, 160, seed=21)
    _check(wl, what="decode split rows/fp16")


def test_prefill_prefix_fp16(device):
    say("prefill prefix fp16")
    spec = [(0, 130), (256, 77), (512, 300), (768, 2), (256, 64), (0, 1)]
    tabs = _tables([p + n for p, n in spec], 24, 11)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 16, 4, 24, seed=11)
    _check(wl, what="prefill prefix small/fp16")


@pytest.mark.parametrize("g", [1, 4, 8])
def test_prefill_gqa_fp16(device, g):
    say(f"prefill fp16 g={g}")
    spec = [(256, 129), (0, 63), (512, 200), (0, 1)]
    tabs = _tables([p + n for p, n in spec], 16, 30 + g)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 2 * g, 2, 16, seed=30 + g)
    _check(wl, what=f"prefill fp16 g={g}")


def test_mixed_batch_fp16(device):
    """Decode rows (split, merged in the plan launch) beside prefill rows of
    many units (the tile loop's chained units) in one call."""
    say("mixed fp16")
    spec = [(5000, 1), (0, 700), (3000, 1), (1024, 900), (6000, 1), (256, 1200)]
    tabs = _tables([p + n for p, n in spec], 96, 41)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 32, 8, 96, seed=41)
    got = _run(wl)
    ref, rows = oracle_paged(wl, [0, 2, 4])
    _check_f16(got[rows], ref, "mixed fp16: decode rows")
    for i in (1, 3, 5):
        n = wl.seqs[i].num_new_tokens
        for r0 in (0, n - 64):
            ref, rows = oracle_seq_rows(wl, i, r0, r0 + 64)
            _check_f16(got[rows], ref, f"mixed fp16: seq {i} rows {r0}..")


def test_prefill_8b_shape_fp16(device):
    """The prefill_8b batch in fp16 (16 sequences, 512-4096 new tokens over
    0-8 cached blocks), checked on its three smallest sequences."""
    say("prefill_8b fp16")
    wl = W.prefill_8b(device, kv="fp16")
    tot = [s.num_new_tokens * (s.num_new_tokens + s.num_cached_tokens) for s in wl.seqs]
    ids = np.argsort(tot)[:3].tolist()
    _check(wl, ids, "prefill_8b fp16 subset")


def test_local_mode_fp16(device):
    """block_tables None: causal over the step's own fp16 k/v."""
    say("local mode fp16")
    lens = [1, 37, 200, 129, 300]
    tabs = _tables(lens, 16, 13)
    wl = _custom([SeqSlice(tabs[i], 0, n) for i, n in enumerate(lens)], 8, 2, 16, seed=13)
    assert wl.context.block_tables is None
    got = _run(wl)
    ref = AO.attention_local(torch.from_numpy(bf16_to_np(wl.q)), torch.from_numpy(bf16_to_np(wl.k)),
                             torch.from_numpy(bf16_to_np(wl.v)), wl.context.cu_seqlens_q.cpu(), 8, 2, 128)
    _check_f16(got, ref.numpy(), "local mode fp16")


def test_fp16_cache_holds_the_cast_values(device):
    """The step's k / v land in the fp16 cache as k.to(float16) (the
    reference's store, attention.py:139-189) before the attention reads
    them."""
    say("fp16 store")
    spec = [(0, 40), (256, 3)]
    tabs = _tables([p + n for p, n in spec], 8, 51)
    wl = _custom([SeqSlice(tabs[i], p, n) for i, (p, n) in enumerate(spec)], 8, 2, 8, seed=51)
    _run(wl)
    sl = wl.context.slot_mapping.long()
    bs = wl.block_size
    kc = wl.attn.k_cache.view(-1, *wl.attn.k_cache.shape[2:])
    got = kc[sl].cpu()
    assert torch.equal(got.view(torch.int16), wl.k.cpu().view(torch.int16))


def test_varlen_entry_refuses_other_dtypes(device):
    """nvs_varlen_attention_dtype serves BF16 and FP16 only; another dtype is
    refused on the host before any launch."""
    from nanovllm_self_amd import _lib

    lib = _lib.load()
    x = torch.zeros(4, 2, 128, dtype=torch.float16, device=device)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=device)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=device)
    rc = lib.nvs_varlen_attention_dtype(
        x.data_ptr(), x.stride(0), x.stride(1), x.data_ptr(), x.data_ptr(), x.stride(0), x.stride(1),
        x.stride(0), x.stride(1), cu.data_ptr(), cu.data_ptr(), 1, 4, 4, 4, 4, 2, 2, 128, 0.088,
        x.data_ptr(), x.stride(0), x.stride(1), ws.data_ptr(), ws.numel(), None, _lib.nvs_dtype(torch.float32))
    assert rc != 0 and "dtype" in lib.nvs_last_error().decode()
