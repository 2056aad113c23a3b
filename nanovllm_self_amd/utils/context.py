"""Per-step attention metadata.

Same dataclass and fields as the reference's nanovllm/utils/context.py:5-49,
so the engine's prepare_model_input (model_runner.py:461-532) builds it
unchanged:

- cu_seqlens_q / cu_seqlens_k: int32 [B + 1] prefix sums of the new-token
  counts and of the visible KV lengths (cached prefix + new tokens).
- max_seqlen_q / max_seqlen_k: host ints.
- slot_mapping: int32 [T], the cache slot of every new token.
- context_lens: int32 [B], visible KV length per sequence.
- block_tables: int32 [B, max_blocks] padded with -1, or None when no
  sequence of the step has cached context (model_runner.py:516-518).
- seq_need_compute_logits: int32 indices of sequences that sample a token.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class Context:
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    seq_need_compute_logits: torch.Tensor | None = None


def get_context(
    cu_seqlens_q=None,
    cu_seqlens_k=None,
    max_seqlen_q=0,
    max_seqlen_k=0,
    slot_mapping=None,
    context_lens=None,
    block_tables=None,
    seq_need_compute_logits=None,
) -> Context:
    """Builder with the reference's keyword signature (context.py:39-49)."""
    return Context(
        cu_seqlens_q=cu_seqlens_q,
        cu_seqlens_k=cu_seqlens_k,
        max_seqlen_q=max_seqlen_q,
        max_seqlen_k=max_seqlen_k,
        slot_mapping=slot_mapping,
        context_lens=context_lens,
        block_tables=block_tables,
        seq_need_compute_logits=seq_need_compute_logits,
    )
