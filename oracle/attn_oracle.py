"""CPU fp32 oracle for the attention math (torch on the CPU).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker.  It restates the eager path of the reference (nanovllm_self,
nanovllm/layers/attention.py:prefill_torch, :378-498):

  attention_local   :400-439  no cached prefix: causal over the step's k/v
  attention_cached  :441-498  per sequence: k_len = cu_k[i+1] - cu_k[i];
                              GQA by repeat_interleave (kv head = h // g);
                              fp32 QK^T / sqrt(D); mask
                              triu(ones(q_len, k_len), 1 + k_len - q_len)
                              (bottom-right causal); fp32 softmax; P V.

Outputs are returned in fp32 (before the final .to(bf16)) so tests can apply
their stated tolerances.  One deliberate choice: a query row with no visible
key (only possible when q_len > k_len) returns 0, flash-attn's convention,
where torch's softmax over an all -inf row would give NaN.  Query rows are
processed in chunks to bound memory; the math per row is unchanged.
"""
from __future__ import annotations

import math

import numpy as np
import torch

ROW_CHUNK = 512


def _attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, groups: int, scale: float) -> torch.Tensor:
    """q [Lq, Hq, D], k/v [Lk, Hkv, D] (fp32) -> [Lq, Hq, D] with the
    bottom-right causal mask of a sequence whose last Lq of Lk keys are new."""
    q_len, k_len = q.shape[0], k.shape[0]
    if q_len == 0:
        return q.new_zeros(q.shape)
    if groups > 1:
        k = k.repeat_interleave(groups, dim=1)
        v = v.repeat_interleave(groups, dim=1)
    kh = k.permute(1, 0, 2)  # [Hq, Lk, D]
    vh = v.permute(1, 0, 2)
    out = []
    for r0 in range(0, q_len, ROW_CHUNK):
        r1 = min(r0 + ROW_CHUNK, q_len)
        qh = q[r0:r1].permute(1, 0, 2)  # [Hq, r, D]
        scores = torch.matmul(qh, kh.transpose(-2, -1)) * scale
        rows = torch.arange(r0, r1).unsqueeze(1)
        cols = torch.arange(k_len).unsqueeze(0)
        masked = cols > rows + (k_len - q_len)  # triu(diagonal = 1 + k_len - q_len)
        scores = scores.masked_fill(masked, float("-inf"))
        dead = masked.all(dim=1)  # rows with no visible key
        w = torch.softmax(scores, dim=-1)
        w = torch.nan_to_num(w, nan=0.0)
        o = torch.matmul(w, vh)  # [Hq, r, D]
        if dead.any():
            o[:, dead] = 0.0
        out.append(o.permute(1, 0, 2))
    return torch.cat(out, dim=0)


def _as_f32(x) -> torch.Tensor:
    t = torch.as_tensor(x)
    return t.float()


def attention_local(q, k, v, cu_seqlens_q, num_heads, num_kv_heads, head_dim) -> torch.Tensor:
    """attention.py:400-439: each sequence attends causally over its own
    rows of the step's k/v (keys = queries)."""
    q, k, v = _as_f32(q), _as_f32(k), _as_f32(v)
    cu = [int(x) for x in torch.as_tensor(cu_seqlens_q).tolist()]
    groups = num_heads // num_kv_heads
    scale = 1.0 / math.sqrt(head_dim)
    outs = [_attend(q[a:b], k[a:b], v[a:b], groups, scale) for a, b in zip(cu[:-1], cu[1:])]
    return torch.cat(outs, dim=0) if outs else q.new_zeros(q.shape)


def attention_cached(q, k_batch, v_batch, cu_seqlens_q, cu_seqlens_k, num_heads, num_kv_heads,
                     head_dim, seqs=None) -> torch.Tensor:
    """attention.py:441-498 over gathered K/V [B, max_len, Hkv, D].

    ``seqs`` optionally restricts the computation to some sequence indices
    (rows of other sequences are left zero) to bound CPU time on large
    batches; the per-sequence math does not depend on the others.
    """
    q = _as_f32(q)
    kb, vb = _as_f32(k_batch), _as_f32(v_batch)
    cu_q = [int(x) for x in torch.as_tensor(cu_seqlens_q).tolist()]
    cu_k = [int(x) for x in torch.as_tensor(cu_seqlens_k).tolist()]
    groups = num_heads // num_kv_heads
    scale = 1.0 / math.sqrt(head_dim)
    out = q.new_zeros(q.shape)
    for i in (range(len(cu_q) - 1) if seqs is None else seqs):
        a, b = cu_q[i], cu_q[i + 1]
        k_len = cu_k[i + 1] - cu_k[i]
        out[a:b] = _attend(q[a:b], kb[i, :k_len], vb[i, :k_len], groups, scale)
    return out


def paged_attention(q, k_vals, v_vals, block_tables, cu_seqlens_q, cu_seqlens_k, context_lens,
                    num_heads, num_kv_heads, head_dim, seqs=None) -> torch.Tensor:
    """Cached-prefix path end to end: get_kv_cache over the dequantised
    caches (float32 [NB, bs, Hkv, D]) then attention_cached.  Gathers only
    the requested sequences."""
    from .kv_oracle import get_kv_cache

    bt = np.asarray(torch.as_tensor(block_tables).cpu())
    lens = np.asarray(torch.as_tensor(context_lens).cpu())
    idx = list(range(bt.shape[0])) if seqs is None else list(seqs)
    kb, vb, _ = get_kv_cache(k_vals, v_vals, bt[idx], lens[idx])
    # Re-index the gathered rows to batch positions.
    B = bt.shape[0]
    full_k = np.zeros((B,) + kb.shape[1:], dtype=np.float32)
    full_v = np.zeros_like(full_k)
    full_k[idx], full_v[idx] = kb, vb
    return attention_cached(q, torch.from_numpy(full_k), torch.from_numpy(full_v), cu_seqlens_q,
                            cu_seqlens_k, num_heads, num_kv_heads, head_dim, seqs=idx)
