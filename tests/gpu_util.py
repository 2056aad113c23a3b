"""Helpers shared by the GPU parity tests (not a test module)."""
from __future__ import annotations

import sys

import numpy as np
import torch

from oracle import attn_oracle as AO
from oracle import kv_oracle as KO

BF16_MAX_ABS, BF16_MEAN_ABS = 2e-2, 2e-3  # bf16 KV vs the fp32 oracle
QUANT_MAX_ABS = 5e-2                       # int8 / fp8 KV vs the fp32 oracle
QUANT_MEAN_ABS = 5e-3                      # int8 / fp8 KV mean (a bar of this suite's own)
# The reference returns bf16 (.to(self.dtype), attention.py:498), so every
# output, its own included, carries up to half a bf16 ulp (<= 2^-8 |x|) of
# rounding on top of the absolute bound.
BF16_HALF_ULP_REL = 2.0 ** -8
# The stated bars are raw max-abs bounds.  A bf16 output of magnitude >= 4
# carries up to 2^-7 (>= 8: 2^-6 ... ) of rounding alone, so no bf16 output,
# the reference's included, can meet a raw 2e-2 there; the raw bound is
# checked on every element below RAW_BOUND_BELOW, the rounding-adjusted bound
# on every element.
RAW_BOUND_BELOW = 4.0


def say(*args):
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print("[case]", *args, file=sys.stderr, flush=True)


def bf16_to_np(t: torch.Tensor) -> np.ndarray:
    """float32 copy of a bf16 (or fp16) tensor, exact."""
    if t.dtype == torch.float16:
        return t.detach().cpu().float().numpy()
    return KO.bf16_bits_to_f32(t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def cache_blocks_f32(attn, blocks: np.ndarray):
    """Dequantised float32 copies of the given cache blocks, as the eager
    path sees them: bf16 / fp16 caches as stored; int8 / fp8 codes * scale rounded
    to bf16 (dequantize_int8_per_token's .to(attention_compute_dtype))."""
    idx = torch.as_tensor(blocks, dtype=torch.long, device=attn.k_cache.device)
    out = []
    for cache, scale in ((attn.k_cache, attn.k_scale_cache), (attn.v_cache, attn.v_scale_cache)):
        sub = cache.index_select(0, idx).cpu()
        if sub.dtype in (torch.bfloat16, torch.float16):
            out.append(bf16_to_np(sub))
            continue
        codes = sub.view(torch.uint8).numpy()
        kind = "int8" if sub.dtype == torch.int8 else "fp8"
        if kind == "int8":
            codes = codes.view(np.int8)
        sc = scale.index_select(0, idx).cpu().numpy()
        out.append(KO.round_to_bf16(KO.dequantize_per_token(codes, sc, kind)))
    return out[0], out[1]


def oracle_paged_inputs(wl, seq_ids):
    """Host-side oracle inputs for the given sequences of a paged workload:
    only their blocks are copied from the device, block ids remapped onto that
    compact pool.  Returns (positional args of attn_oracle.paged_attention,
    the sequences' query rows)."""
    ctx = wl.context
    cu_q = ctx.cu_seqlens_q.cpu().tolist()
    bs = wl.block_size
    blocks, tables, lens, qrows, qlens = [], [], [], [], []
    for i in seq_ids:
        s = wl.seqs[i]
        n = s.num_cached_tokens + s.num_new_tokens
        need = (n + bs - 1) // bs
        tb = list(s.block_table[:need])
        tables.append(list(range(len(blocks), len(blocks) + len(tb))))
        blocks.extend(tb)
        lens.append(n)
        qrows.extend(range(cu_q[i], cu_q[i + 1]))
        qlens.append(s.num_new_tokens)
    kv, vv = cache_blocks_f32(wl.attn, np.asarray(blocks))
    width = max(len(t) for t in tables)
    bt = np.full((len(seq_ids), width), -1, dtype=np.int64)
    for r, t in enumerate(tables):
        bt[r, : len(t)] = t
    q = torch.from_numpy(bf16_to_np(wl.q[torch.as_tensor(qrows, device=wl.q.device)]))
    sub_cu_q = np.concatenate([[0], np.cumsum(qlens)]).tolist()
    sub_cu_k = np.concatenate([[0], np.cumsum(lens)]).tolist()
    args = (q, kv, vv, bt, sub_cu_q, sub_cu_k, lens, wl.num_heads, wl.num_kv_heads, wl.head_dim)
    return args, qrows


def oracle_paged(wl, seq_ids):
    """fp32 oracle output rows of the given sequences of a paged workload."""
    args, qrows = oracle_paged_inputs(wl, seq_ids)
    return AO.paged_attention(*args).numpy(), qrows


def compare(got: np.ndarray, ref: np.ndarray, quant: bool, what: str):
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    mx, mean = float(err.max()), float(err.mean())
    # error beyond the output's own bf16 rounding allowance
    mag = np.abs(ref.astype(np.float64))
    excess = float((err - BF16_HALF_ULP_REL * mag).max())
    small = mag < RAW_BOUND_BELOW
    raw = float(err[small].max()) if small.any() else 0.0
    say(f"{what}: max-abs {mx:.3e} (|ref| < {RAW_BOUND_BELOW:g}: {raw:.3e}, max |ref| {float(mag.max()):.2f}) "
        f"mean-abs {mean:.3e} max-abs beyond bf16 rounding {excess:.3e}")
    atol = QUANT_MAX_ABS if quant else BF16_MAX_ABS
    mtol = QUANT_MEAN_ABS if quant else BF16_MEAN_ABS
    assert raw <= atol, f"{what}: max-abs {raw:.3e} > {atol} where |ref| < {RAW_BOUND_BELOW:g}"
    assert excess <= atol, f"{what}: max-abs beyond bf16 output rounding {excess:.3e} > {atol}"
    assert mean <= mtol, f"{what}: mean-abs {mean:.3e} > {mtol}"
    return mx, mean


def oracle_seq_rows(wl, i, r0, r1):
    """fp32 oracle for query rows r0 .. r1-1 of sequence i of a paged workload.

    Under the bottom-right causal mask, row r of a sequence with P cached and
    L new tokens sees keys 0 .. P + r.  A contiguous row block [r0, r1) is
    therefore itself a sequence with q_len = r1 - r0 new tokens over
    k_len = P + r1 keys (its row j sees keys up to j + k_len - q_len =
    P + r0 + j), so long sequences are checked block by block at the cost of
    the block alone.  Returns (oracle rows, their indices in the batch)."""
    s = wl.seqs[i]
    bs = wl.block_size
    klen = s.num_cached_tokens + r1
    need = (klen + bs - 1) // bs
    kv, vv = cache_blocks_f32(wl.attn, np.asarray(s.block_table[:need]))
    q0 = int(wl.context.cu_seqlens_q[i].item())
    q = torch.from_numpy(bf16_to_np(wl.q[q0 + r0:q0 + r1]))
    bt = np.arange(need, dtype=np.int64)[None]
    ref = AO.paged_attention(q, kv, vv, bt, [0, r1 - r0], [0, klen], [klen], wl.num_heads,
                             wl.num_kv_heads, wl.head_dim)
    return ref.numpy(), list(range(q0 + r0, q0 + r1))
