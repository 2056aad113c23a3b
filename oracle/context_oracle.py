"""CPU oracle for the step metadata (pure Python).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only
tests/ and bench.py's cpu_baseline leg use it, as the checker.  It restates
ModelRunner.prepare_model_input (nanovllm/engine/model_runner.py:461-532)
loop for loop:

  :482-488   start = num_cached, end = num_cached + num_new,
             context_lens.append(num_cached + num_new)
  :490-492   seq_need_compute_logits.append(seq_index) when the sequence
             needs logits
  :495       positions.extend(range(start, end))
  :497-501   cu_seqlens_q / cu_seqlens_k running sums, max_seqlen_q / k
  :503-507   slot = block_table[pos // block_size] * block_size
                    + pos % block_size, per token
  :511-513   block tables (padded with -1, model_runner.py:334-344) only
             when cu_seqlens_k[-1] > cu_seqlens_q[-1]

A sequence is (block_table, num_cached_tokens, num_new_tokens, need_logits).
"""
from __future__ import annotations


def prepare_model_input(seqs, block_size):
    """-> dict of plain Python lists / ints, keyed like the Context fields,
    plus "positions"."""
    positions, slot_mapping, context_lens, need = [], [], [], []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    for seq_index, (block_table, num_cached, num_new, need_logits) in enumerate(seqs):
        start = num_cached
        end = num_cached + num_new
        seqlen_q = num_new
        seqlen_k = num_cached + num_new
        context_lens.append(seqlen_k)
        if need_logits:
            need.append(seq_index)
        positions.extend(range(start, end))
        cu_q.append(cu_q[-1] + seqlen_q)
        cu_k.append(cu_k[-1] + seqlen_k)
        max_q = max(max_q, seqlen_q)
        max_k = max(max_k, seqlen_k)
        for token_pos in range(start, end):
            block_id = block_table[token_pos // block_size]
            slot_mapping.append(block_id * block_size + token_pos % block_size)
    block_tables = None
    if cu_k[-1] > cu_q[-1]:
        width = max(len(s[0]) for s in seqs)
        block_tables = [list(s[0]) + [-1] * (width - len(s[0])) for s in seqs]
    return {
        "cu_seqlens_q": cu_q,
        "cu_seqlens_k": cu_k,
        "max_seqlen_q": max_q,
        "max_seqlen_k": max_k,
        "slot_mapping": slot_mapping,
        "context_lens": context_lens,
        "block_tables": block_tables,
        "seq_need_compute_logits": need,
        "positions": positions,
    }
