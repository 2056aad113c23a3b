"""CPU oracle for the fused pre-attention step (numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only
tests/ and bench.py's cpu_baseline leg use it, as the checker.  It restates
the reference (nanovllm_self) step by step:

  rms_norm           nanovllm/layers/RMSNorm.py:11-18
                     x32 = x.float(); rms = sqrt(mean(x32^2) + eps);
                     out = (w32 * x32 / rms).to(x.dtype)
  rope               nanovllm/layers/RoPE.py:5-25 (apply_rotary_embedding):
                     x1, x2 = chunk(x.float(), 2); y1 = x1 cos - x2 sin;
                     y2 = x2 cos + x1 sin; cat(y1, y2).to(x.dtype)
  cos_sin_table      nanovllm/layers/RoPE.py:40-58 (the layer's buffer, as
                     float32 numpy arithmetic; the product takes the table as
                     an input, so the tests only need *a* table)
  qk_norm_rope       the order of nanovllm/models/qwen3.py:100-104

Every step is a float32 numpy operation, each product and sum rounded on its
own (numpy never fuses a multiply-add).  The sum inside the reference's
mean() has no specified order (torch's reduction decides it); this
restatement fixes one — sequential sums over consecutive groups of eight
squares, then a pairwise tree over the groups in index order — which is the
order the HIP kernel uses, so the two agree bit for bit.  The pin tests
check the oracle against closed forms that hold in any order.
"""
from __future__ import annotations

import numpy as np

from .kv_oracle import round_to_bf16

F32 = np.float32


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """x [..., D] (float32 holding bf16 values), w [D] (bf16 values) ->
    bf16-rounded float32 (RMSNorm.py:11-18)."""
    x32 = x.astype(F32)
    ms = (sum_squares(x32) / F32(x32.shape[-1])).astype(F32)
    rms = np.sqrt(ms + F32(eps)).astype(F32)
    return round_to_bf16((w.astype(F32) * x32) / rms)


def sum_squares(x32: np.ndarray) -> np.ndarray:
    """Sum of squares over the last axis, [..., 1]: sequential over groups of
    eight (or fewer, when the axis is shorter), then a pairwise tree over the
    groups."""
    n = x32.shape[-1]
    g = min(8, n)
    sq = (x32 * x32).astype(F32)
    parts = []
    for s in range(0, n, g):
        acc = np.zeros(x32.shape[:-1], dtype=F32)
        for i in range(s, min(s + g, n)):
            acc = (acc + sq[..., i]).astype(F32)
        parts.append(acc)
    while len(parts) > 1:
        parts = [(parts[i] + parts[i + 1]).astype(F32) if i + 1 < len(parts) else parts[i]
                 for i in range(0, len(parts), 2)]
    return parts[0][..., None]


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """x [..., D] (bf16 values), cos / sin broadcastable to [..., D / 2] ->
    bf16-rounded float32 (RoPE.py:5-25)."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h].astype(F32), x[..., h:].astype(F32)
    c, s = cos.astype(F32), sin.astype(F32)
    y1 = x1 * c - x2 * s
    y2 = x2 * c + x1 * s
    return round_to_bf16(np.concatenate([y1, y2], axis=-1))


def cos_sin_table(head_dim: int, max_position: int, base: float) -> np.ndarray:
    """[max_position, head_dim] float32: cos of the head_dim / 2 frequencies,
    then their sin (RoPE.py:40-58, the buffer without its broadcast dim)."""
    inv_freq = (F32(1.0) / (F32(base) ** (np.arange(0, head_dim, 2, dtype=F32) / F32(head_dim)))).astype(F32)
    freqs = np.outer(np.arange(max_position, dtype=F32), inv_freq).astype(F32)
    return np.concatenate([np.cos(freqs), np.sin(freqs)], axis=1).astype(F32)


def qk_norm_rope(q, k, positions, q_w, k_w, eps, table):
    """q [T, Hq, D], k [T, Hkv, D] (bf16 values), positions [T], table
    [max_position, D] -> (rotated q, rotated k), qwen3.py:100-104."""
    D = q.shape[-1]
    pos = np.clip(np.asarray(positions, dtype=np.int64), 0, table.shape[0] - 1)
    cs = table[pos][:, None, :]  # [T, 1, D]
    cos, sin = cs[..., : D // 2], cs[..., D // 2:]
    return rope(rms_norm(q, q_w, eps), cos, sin), rope(rms_norm(k, k_w, eps), cos, sin)
