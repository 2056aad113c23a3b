"""KV pool, layer binding and step-metadata builders for the paged attention.

These are the producer side of the attention boundary in the reference:

- KVCacheConfig mirrors the hot-path knobs of nanovllm/config.py:28-80
  (kv_cache_dtype, attention_compute_dtype, kv_cache_quant_mode,
  kv_cache_scale_dtype, block_size) including the rule that a quantised mode
  forces the cache dtype (config.py:78-80).  Quant modes: "none", "int8_mock"
  (reference) and "fp8_e4m3" (OCP float8_e4m3fn codes, same per-token,
  per-kv-head fp32 scale layout).
- allocate_kv_cache mirrors model_runner.py:40-73: kv_cache
  [2, L, NB, bs, Hkv, D] and, for quantised modes, kv_scale_cache
  [2, L, NB, bs, Hkv, 1].
- bind_kv_cache mirrors bind_kvcache_to_attention (model_runner.py:302-331).
  The reference pins int8 to forward_backend="torch" (:323-324) because
  flash-attn cannot read int8; the HIP kernels serve int8 and fp8 on every
  backend, so the backend is left as the caller set it.
- prepare_block_tables mirrors model_runner.py:334-344 (rows padded with -1).
- build_context mirrors prepare_model_input (model_runner.py:461-532) with the
  per-token slot loop vectorised.
- export_kv_blocks / import_kv_blocks are the KV handoff copies of the PD
  connector (pd_self/kv_connector.py:65-135, 264-311): whole cache blocks,
  codes and fp32 scales alike, moved by one launch per tensor.
- build_context_on_device forms the same Context (plus the step's positions)
  with one HIP launch (nvs_build_context): the host handles only per-sequence
  counts and the padded block table, sent in one pinned copy.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from itertools import chain
from typing import Iterable, Sequence

import numpy as np
import torch

from . import _lib
from .utils.context import Context, get_context

KV_QUANT_MODES = ("none", "int8_mock", "fp8_e4m3")

_DTYPE_ALIASES = {
    "float32": torch.float32,
    "fp32": torch.float32,
    "float16": torch.float16,
    "fp16": torch.float16,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
}


def resolve_torch_dtype(dtype):
    """String alias or torch dtype -> torch dtype; None / "auto" -> None (config.py:6-25)."""
    if isinstance(dtype, torch.dtype):
        return dtype
    if dtype in (None, "auto"):
        return None
    if dtype not in _DTYPE_ALIASES:
        raise ValueError(f"unsupported dtype: {dtype}")
    return _DTYPE_ALIASES[dtype]


@dataclass
class KVCacheConfig:
    dtype: torch.dtype | str = torch.bfloat16
    kv_cache_dtype: torch.dtype | str = torch.bfloat16
    attention_compute_dtype: torch.dtype | str = torch.bfloat16
    kv_cache_quant_mode: str = "none"
    kv_cache_scale_dtype: torch.dtype | str = "fp32"
    block_size: int = 256
    num_blocks: int = 256

    def __post_init__(self):
        self.dtype = resolve_torch_dtype(self.dtype) or torch.float16
        self.kv_cache_dtype = resolve_torch_dtype(self.kv_cache_dtype) or self.dtype
        self.attention_compute_dtype = resolve_torch_dtype(self.attention_compute_dtype) or self.dtype
        self.kv_cache_scale_dtype = resolve_torch_dtype(self.kv_cache_scale_dtype) or torch.float32
        if self.kv_cache_quant_mode not in KV_QUANT_MODES:
            raise ValueError(f"unsupported kv_cache_quant_mode: {self.kv_cache_quant_mode}")
        if self.kv_cache_quant_mode == "int8_mock":
            self.kv_cache_dtype = torch.int8
        elif self.kv_cache_quant_mode == "fp8_e4m3":
            self.kv_cache_dtype = torch.float8_e4m3fn
        if self.kv_cache_quant_mode != "none" and self.kv_cache_scale_dtype != torch.float32:
            raise ValueError("quantised KV caches keep fp32 scales")


def allocate_kv_cache(
    num_layers: int,
    num_kv_heads: int,
    head_dim: int,
    cfg: KVCacheConfig,
    device: torch.device | str,
):
    """Zeroed kv_cache [2, L, NB, bs, Hkv, D] and, when quantised, a
    kv_scale_cache [2, L, NB, bs, Hkv, 1] of ones (model_runner.py:40-73)."""
    kv_cache = torch.zeros(
        2, num_layers, cfg.num_blocks, cfg.block_size, num_kv_heads, head_dim,
        dtype=cfg.kv_cache_dtype, device=device,
    )
    kv_scale_cache = None
    if cfg.kv_cache_quant_mode != "none":
        kv_scale_cache = torch.ones(
            2, num_layers, cfg.num_blocks, cfg.block_size, num_kv_heads, 1,
            dtype=cfg.kv_cache_scale_dtype, device=device,
        )
    return kv_cache, kv_scale_cache


def bind_kv_cache(attn_layers: Iterable, kv_cache, kv_scale_cache, cfg: KVCacheConfig) -> None:
    """Bind per-layer K/V (and scale) views onto PagedAttention modules."""
    for layer_id, p_attn in enumerate(attn_layers):
        p_attn.k_cache = kv_cache[0, layer_id]
        p_attn.v_cache = kv_cache[1, layer_id]
        p_attn.block_size = cfg.block_size
        p_attn.layer_id = layer_id
        p_attn.kv_cache_quant_mode = cfg.kv_cache_quant_mode
        p_attn.kv_cache_dtype = cfg.kv_cache_dtype
        p_attn.attention_compute_dtype = cfg.attention_compute_dtype
        if kv_scale_cache is not None:
            p_attn.k_scale_cache = kv_scale_cache[0, layer_id]
            p_attn.v_scale_cache = kv_scale_cache[1, layer_id]
        else:
            p_attn.k_scale_cache = None
            p_attn.v_scale_cache = None


def prepare_block_tables(block_tables: Sequence[Sequence[int]], device) -> torch.Tensor:
    """Pad per-sequence block lists with -1 into an int32 [B, max_blocks] tensor."""
    max_len = max(len(bt) for bt in block_tables)
    rows = [list(bt) + [-1] * (max_len - len(bt)) for bt in block_tables]
    t = torch.tensor(rows, dtype=torch.int32)
    if torch.device(device).type == "cuda":
        t = t.pin_memory().to(device, non_blocking=True)
    return t


@dataclass
class SeqSlice:
    """What the step needs of one sequence (the Sequence fields the runner reads)."""

    block_table: Sequence[int]
    num_cached_tokens: int
    num_new_tokens: int
    need_logits: bool = True


def build_context(seqs: Sequence[SeqSlice], block_size: int, device) -> Context:
    """Step metadata exactly as prepare_model_input forms it.

    Query tokens of a sequence are positions [num_cached, num_cached + num_new);
    its visible KV length is num_cached + num_new; the slot of position p is
    block_table[p // block_size] * block_size + p % block_size; block_tables
    is only built when some sequence sees more keys than it brings queries.
    """
    cu_q = [0]
    cu_k = [0]
    ctx_lens, need = [], []
    slots = []
    for i, s in enumerate(seqs):
        start = s.num_cached_tokens
        end = start + s.num_new_tokens
        cu_q.append(cu_q[-1] + s.num_new_tokens)
        cu_k.append(cu_k[-1] + end)
        ctx_lens.append(end)
        if s.need_logits:
            need.append(i)
        pos = np.arange(start, end, dtype=np.int64)
        bt = np.asarray(s.block_table, dtype=np.int64)
        slots.append(bt[pos // block_size] * block_size + pos % block_size)
    slot_mapping = np.concatenate(slots) if slots else np.zeros(0, dtype=np.int64)
    max_q = max((s.num_new_tokens for s in seqs), default=0)
    max_k = max(ctx_lens, default=0)
    block_tables = None
    if cu_k[-1] > cu_q[-1]:
        block_tables = prepare_block_tables([s.block_table for s in seqs], device)

    def i32(x):
        return torch.as_tensor(np.asarray(x, dtype=np.int32)).to(device)

    return get_context(
        cu_seqlens_q=i32(cu_q),
        cu_seqlens_k=i32(cu_k),
        max_seqlen_q=max_q,
        max_seqlen_k=max_k,
        slot_mapping=i32(slot_mapping),
        context_lens=i32(ctx_lens),
        block_tables=block_tables,
        seq_need_compute_logits=i32(need),
    )


def build_context_on_device(seqs: Sequence[SeqSlice], block_size: int, device) -> tuple[Context, torch.Tensor]:
    """prepare_model_input's step metadata (model_runner.py:461-532) formed on
    the device; returns (context, positions int64 [T]).

    The host touches each sequence once and each block id once: it packs
    num_cached, num_new, the block-list offsets, the need-logits indices and
    the concatenated block lists into one pinned int32 buffer and copies it
    once; nvs_build_context expands them into cu_seqlens_q/k, context_lens,
    slot_mapping, positions and the -1-padded block_tables.  The Context
    equals build_context's, including block_tables None when no sequence has
    cached tokens (:516-518).  A block list too short for a sequence's
    positions raises IndexError, as the reference's seq.block_table[block_idx]
    does (:505).
    """
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("build_context_on_device needs a GPU device")
    B = len(seqs)
    meta = np.fromiter(
        chain.from_iterable((s.num_cached_tokens, s.num_new_tokens, len(s.block_table), s.need_logits) for s in seqs),
        dtype=np.int64, count=4 * B).reshape(B, 4)
    cached, new, nblk = meta[:, 0], meta[:, 1], meta[:, 2]
    lens = cached + new
    if np.any(cached < 0) or np.any(new < 0):
        raise ValueError("token counts must be non-negative")
    short = (new > 0) & ((lens + block_size - 1) // block_size > nblk)
    if np.any(short):
        i = int(np.argmax(short))
        raise IndexError(f"sequence {i}: block_table holds {int(nblk[i])} blocks, positions reach {int(lens[i]) - 1}")
    n_ids = int(nblk.sum())
    if int(lens.sum()) >= 2**31 or n_ids >= 2**31:
        raise ValueError("step too large for int32 metadata")
    T = int(new.sum())
    need = np.flatnonzero(meta[:, 3])
    n_need = len(need)
    # Pinned staging: [cached B | new B | offsets B+1 | need | block ids]
    o_off, o_need, o_ids = 2 * B, 3 * B + 1, 3 * B + 1 + n_need
    staging = torch.empty(o_ids + n_ids, dtype=torch.int32, pin_memory=True)
    host = staging.numpy()
    host[:B] = cached
    host[B:o_off] = new
    host[o_off] = 0
    np.cumsum(nblk, out=host[o_off + 1:o_need])
    host[o_need:o_ids] = need
    host[o_ids:] = np.fromiter(chain.from_iterable(s.block_table for s in seqs), dtype=np.int32, count=n_ids)
    inputs = staging.to(dev, non_blocking=True)
    W = max(int(nblk.max(initial=0)), 1)
    with_table = int(cached.sum()) > 0
    out = torch.empty(3 * B + 2 + T + (B * W if with_table else 0), dtype=torch.int32, device=dev)
    positions = torch.empty(T, dtype=torch.int64, device=dev)
    cu_q, cu_k = out[: B + 1], out[B + 1: 2 * B + 2]
    ctx_lens, slots = out[2 * B + 2: 3 * B + 2], out[3 * B + 2: 3 * B + 2 + T]
    table = out[3 * B + 2 + T:].view(B, W) if with_table else None
    ip = inputs.data_ptr()
    _lib.check(
        _lib.load().nvs_build_context(
            ip, ip + 4 * B, B, ip + 4 * o_off, ip + 4 * o_ids, n_ids, block_size, T,
            cu_q.data_ptr(), cu_k.data_ptr(), ctx_lens.data_ptr(), slots.data_ptr(), positions.data_ptr(),
            _lib.ptr(table), W if with_table else 0, _lib.stream_of(out),
        ),
        "build_context",
    )
    ctx = get_context(
        cu_seqlens_q=cu_q,
        cu_seqlens_k=cu_k,
        max_seqlen_q=int(new.max(initial=0)),
        max_seqlen_k=int(lens.max(initial=0)),
        slot_mapping=slots,
        context_lens=ctx_lens,
        block_tables=table,
        seq_need_compute_logits=inputs[o_need:o_ids],
    )
    return ctx, positions


def _device_ids(ids: Sequence[int], num_blocks: int, device) -> torch.Tensor:
    """Block ids as an int32 device tensor; an id outside the cache raises
    IndexError, as indexing the reference's cache tensor does."""
    host = np.asarray(list(ids), dtype=np.int64)
    if host.size and (host.min() < 0 or host.max() >= num_blocks):
        raise IndexError(f"block id out of range for a cache of {num_blocks} blocks")
    return torch.from_numpy(host.astype(np.int32)).pin_memory().to(device, non_blocking=True)


def _copy_blocks(src: torch.Tensor, src_ids, dst: torch.Tensor, dst_ids, n: int) -> None:
    """Copy n blocks of every plane between two [2, L, num_blocks, ...]
    tensors; src_ids / dst_ids are int32 device tensors or None (identity)."""
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise RuntimeError("block copies need contiguous caches and snapshots")
    if src.dtype != dst.dtype or src.shape[:2] != dst.shape[:2] or src.shape[3:] != dst.shape[3:]:
        raise RuntimeError(f"block shapes differ: {tuple(src.shape)} {src.dtype} vs {tuple(dst.shape)} {dst.dtype}")
    planes = src.shape[0] * src.shape[1]
    block_bytes = math.prod(src.shape[3:]) * src.element_size()
    _lib.check(
        _lib.load().nvs_copy_blocks(
            src.data_ptr(), src.shape[2], _lib.ptr(src_ids), dst.data_ptr(), dst.shape[2], _lib.ptr(dst_ids),
            planes, block_bytes, n, _lib.stream_of(dst),
        ),
        "copy_blocks",
    )


def export_kv_blocks(kv_cache: torch.Tensor, kv_scale_cache: torch.Tensor | None, block_ids: Sequence[int]):
    """kv_cache[:, :, block_ids].contiguous() and the same of the scale cache
    (None when there is none), formed on the device: the snapshot of
    KVConnector._export_kv_snapshot's device-direct path
    (kv_connector.py:94-110).  Quantised caches export their codes and fp32
    scales as they are stored."""
    dev = kv_cache.device
    n = len(block_ids)
    ids = _device_ids(block_ids, kv_cache.shape[2], dev)
    kv_blocks = torch.empty((*kv_cache.shape[:2], n, *kv_cache.shape[3:]), dtype=kv_cache.dtype, device=dev)
    _copy_blocks(kv_cache, ids, kv_blocks, None, n)
    scale_blocks = None
    if kv_scale_cache is not None:
        scale_blocks = torch.empty((*kv_scale_cache.shape[:2], n, *kv_scale_cache.shape[3:]),
                                   dtype=kv_scale_cache.dtype, device=dev)
        _copy_blocks(kv_scale_cache, ids, scale_blocks, None, n)
    return kv_blocks, scale_blocks


def import_kv_blocks(kv_cache: torch.Tensor, kv_scale_cache: torch.Tensor | None, kv_blocks: torch.Tensor,
                     scale_blocks: torch.Tensor | None, dst_block_ids: Sequence[int]) -> None:
    """kv_cache[:, :, dst_block_ids[i]] = kv_blocks[:, :, i] for each i, and
    the same for the scales: KVConnector.load_kv_item (kv_connector.py:264-311)
    in one launch per tensor.  Host snapshots are copied to the device first
    (non-blocking, as the reference does).  When an id repeats, the last copy
    wins, as in the reference's sequential loop."""
    if kv_blocks is None or not len(dst_block_ids):
        return
    if scale_blocks is not None and kv_scale_cache is None:
        raise RuntimeError("received scale_blocks but decode runner has no kv_scale_cache")
    dev = kv_cache.device
    ids = list(dst_block_ids)
    if len(ids) > kv_blocks.shape[2]:
        raise IndexError(f"{len(ids)} destination blocks for a snapshot of {kv_blocks.shape[2]}")
    last = {b: i for i, b in enumerate(ids)}
    src_idx = sorted(last.values())
    dst = _device_ids([ids[i] for i in src_idx], kv_cache.shape[2], dev)
    src = None if len(src_idx) == len(ids) else _device_ids(src_idx, kv_blocks.shape[2], dev)
    kv_dev = kv_blocks.to(dev, non_blocking=True)
    _copy_blocks(kv_dev, src, kv_cache, dst, len(src_idx))
    if scale_blocks is not None:
        _copy_blocks(scale_blocks.to(dev, non_blocking=True), src, kv_scale_cache, dst, len(src_idx))
