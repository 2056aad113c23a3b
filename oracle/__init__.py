"""CPU oracle of the paged-KV attention path (test infrastructure only).

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, always as the checker; the product (nanovllm_self_amd) never imports it.
kv_oracle: quantisation, store and gather in numpy; attn_oracle: fp32
attention in torch on the CPU.  Every function cites the reference
(nanovllm_self) lines it restates.
"""
