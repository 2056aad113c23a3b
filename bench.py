"""Benchmark of the paged-KV attention path on one MI355X.

Headline (the JSON line's value): bf16 paged decode at the Qwen3-8B shape
(32 q / 8 kv heads, head_dim 128, block_size 256, 4096-block pool, 64
sequences with context U[2048, 8192], seed 1).  A step is one pass of the
path over the batch: the store of every sequence's new token, then the
decode.  value = algorithmic decode bytes (every visible K/V element once,
q read, o written) / step time, in GB/s.

Also reported on the same line: prefill TFLOP/s at the Qwen3-8B shape (16
sequences, new U[512, 4096] over 0-8 cached blocks, seed 2), quantised
decode tokens/s (256 sequences, ctx U[1024, 4096], fp8 / int8 / bf16, seed
3), the mixed chunked-prefill + decode step at a Qwen3-32B-like shape (seed
4), the dominant kernel's roofline fraction (HIP events on the launch
stream), the CPU eager restatement timed on the host cores beside each of
those workloads (with the CPU model and count), and the steps
either side of the path: the fused q/k norm + rotary + KV store
(`qk_prep`), the step's Context built on the device (`step_context`), the
KV handoff block copies (`kv_handoff`) and a 36-layer decode step, eager
against one HIP-graph replay (`layers36_decode_step`).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--only decode|prefill|quant|mixed|prep|context|handoff|layers]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, AMD published
BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, AMD published


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def timed_steps(fn, steps: int, warmup: int):
    """W untimed calls, then K timed calls bracketed by synchronize; returns
    (wall ms per step, ms per step from one pair of HIP events around the K
    calls on the current stream).  One pair for the whole region keeps the
    event packets' own cost out of the per-step figure."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, e0.elapsed_time(e1) / steps


def paired_steps(step_fn, attn_fn, steps: int, warmup: int, reps: int = 3):
    """A batch's attention-only call and its whole step (store + attention),
    timed in alternating blocks (attention, step, attention, ...), each block
    W untimed calls then K timed ones, `reps` blocks of each.  Returns the
    medians of (step wall ms, step event ms, attention event ms).  The first
    block after a workload is built runs several percent slower than later
    ones while the clock settles; alternating keeps that out of the
    difference between the two."""
    sw, se, ae = [], [], []
    for _ in range(reps):
        ae.append(timed_steps(attn_fn, steps, warmup)[1])
        w, e = timed_steps(step_fn, steps, warmup)
        sw.append(w)
        se.append(e)
    med = statistics.median
    return med(sw), med(se), med(ae)


def attention_only(wl):
    a = wl.attn
    fn = a.prefill_flashattn if a.forward_backend in ("flashattn", "hip") else a.prefill_torch
    return lambda: fn(wl.q, wl.k, wl.v, wl.context)


def step(wl):
    return lambda: wl.attn.forward(wl.q, wl.k, wl.v, wl.context)


def bench_decode(steps, warmup, cpu=False):
    from nanovllm_self_amd import workloads as W

    log("building decode_8b (bf16)")
    wl = W.decode_8b("cuda")
    nbytes = wl.decode_bytes()
    _, ms_attn = timed_steps(attention_only(wl), steps, warmup)
    ms_step, _ = timed_steps(step(wl), steps, warmup)
    res = {
        "bytes": nbytes,
        "ms_per_step": ms_step,
        "gbs_step": nbytes / ms_step / 1e6,
        "ms_attention": ms_attn,
        "gbs_attention": nbytes / ms_attn / 1e6,
        "tokens_per_s": wl.num_seqs / (ms_step / 1e3),
    }
    log(f"decode_8b: {ms_step:.3f} ms/step, attention {ms_attn:.3f} ms -> {res['gbs_attention']:.0f} GB/s")
    res["graph_ms_per_step"] = graph_step_ms(wl, steps, warmup)
    log(f"decode_8b: {res['graph_ms_per_step']:.3f} ms/step replayed from a HIP graph")
    # A launch-bound step: the 8-sequence decode batch, eager against replayed.
    small = W.decode_small("cuda")
    wall, ms_small = timed_steps(step(small), steps, warmup)
    res["small_step"] = {
        "workload": "decode_small: 16q/8kv heads, D128, 8 seqs ctx U[128,1024], seed 0; step = store + decode",
        "eager_ms_per_step": ms_small,
        "eager_wall_ms_per_step": wall,
        "graph_ms_per_step": graph_step_ms(small, steps, warmup),
    }
    log(f"decode_small: eager {ms_small * 1e3:.1f} us/step (wall {wall * 1e3:.1f}), "
        f"graph {res['small_step']['graph_ms_per_step'] * 1e3:.1f} us/step")
    if cpu:
        log("cpu baseline: decode_small")
        res["small_step"]["cpu_baseline"] = cpu_decode_leg(small, 3.0, "decode_small", full_passes=3)
    del small
    return wl, res


def graph_step_ms(wl, steps, warmup):
    """ms per decode step (store + attention) replayed from a captured HIP graph."""
    from nanovllm_self_amd.layers.attention import reserve_attention_workspace

    attn, ctx = wl.attn, wl.context
    reserve_attention_workspace(wl.num_seqs, int(ctx.max_seqlen_q), int(ctx.max_seqlen_k), attn.num_heads,
                                wl.q.device, num_kv_heads=attn.num_kv_heads)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attn.forward(wl.q, wl.k, wl.v, ctx)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    attn.in_cuda_graph_capture = True
    try:
        with torch.cuda.graph(graph):
            attn.forward(wl.q, wl.k, wl.v, ctx)
    finally:
        attn.in_cuda_graph_capture = False
    _, ms = timed_steps(graph.replay, steps, warmup)
    return ms


def bench_layers(steps, warmup, n_layers=36):
    """A decode step of a whole model's attention: n_layers PagedAttention
    layers (Qwen3-8B has 36), each with its own K/V in one pool, each doing
    its store + decode on the step's batch in turn; eager (one forward call
    per layer) against one replay of the whole step captured in a HIP graph.
    Wall clock and HIP events; the difference is the inter-token latency the
    graph saves at that batch size."""
    from nanovllm_self_amd import PagedAttention
    from nanovllm_self_amd import workloads as W
    from nanovllm_self_amd.kv_cache import KVCacheConfig, allocate_kv_cache, bind_kv_cache
    from nanovllm_self_amd.layers.attention import reserve_attention_workspace

    out = {"n_layers": n_layers}
    for name, build in (("decode_small", W.decode_small), ("decode_8b", W.decode_8b)):
        log(f"building {n_layers}-layer {name}")
        wl = build("cuda")
        ctx, a0 = wl.context, wl.attn
        # Every layer's own slice of one pool when it fits in 64 GiB, else
        # the layers share the workload's pool (same bytes read per layer).
        per_layer = a0.k_cache.numel() * a0.k_cache.element_size() * 2
        cfg = KVCacheConfig(dtype=torch.bfloat16, kv_cache_dtype=torch.bfloat16,
                            attention_compute_dtype=torch.bfloat16, block_size=wl.block_size,
                            num_blocks=wl.num_blocks)
        layers = [PagedAttention(wl.num_heads, wl.num_kv_heads, wl.head_dim, dtype=torch.bfloat16)
                  for _ in range(n_layers)]
        own = per_layer * n_layers <= (64 << 30)
        if own:
            pool, _ = allocate_kv_cache(n_layers, wl.num_kv_heads, wl.head_dim, cfg, "cuda")
            pool[:, :] = torch.stack([a0.k_cache, a0.v_cache]).unsqueeze(1)
            bind_kv_cache(layers, pool, None, cfg)
        else:
            pool = torch.stack([a0.k_cache, a0.v_cache]).unsqueeze(1).expand(2, n_layers, *a0.k_cache.shape)
            bind_kv_cache(layers, pool, None, cfg)

        def eager():
            for layer in layers:
                layer.forward(wl.q, wl.k, wl.v, ctx)

        wall_e, ms_e = timed_steps(eager, steps, warmup)
        reserve_attention_workspace(wl.num_seqs, int(ctx.max_seqlen_q), int(ctx.max_seqlen_k), wl.num_heads,
                                    wl.q.device, num_kv_heads=wl.num_kv_heads)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            eager()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        for layer in layers:
            layer.in_cuda_graph_capture = True
        try:
            with torch.cuda.graph(graph):
                eager()
        finally:
            for layer in layers:
                layer.in_cuda_graph_capture = False
        wall_g, ms_g = timed_steps(graph.replay, steps, warmup)
        out[name] = {
            "kv_per_layer": "own" if own else "shared pool",
            "eager_wall_ms_per_step": wall_e,
            "eager_ms_per_step": ms_e,
            "graph_wall_ms_per_step": wall_g,
            "graph_ms_per_step": ms_g,
            "itl_saved_ms": wall_e - wall_g,
        }
        log(f"{n_layers} layers {name}: eager {wall_e:.3f} ms wall ({ms_e:.3f} events), graph {wall_g:.3f} ms wall "
            f"({ms_g:.3f} events)")
        del graph, layers, pool, wl
        torch.cuda.empty_cache()
    return out


def bench_prefill(steps, warmup, cpu=False):
    from nanovllm_self_amd import workloads as W

    log("building prefill_8b")
    wl = W.prefill_8b("cuda")
    flops = wl.prefill_flops()
    ms_step, ms_step_ev, ms_attn = paired_steps(step(wl), attention_only(wl), steps, warmup)
    res = {
        "workload": "prefill_8b: 32q/8kv heads, D128, bs256, 16 seqs, new U[512,4096] over 0-8 cached blocks, seed 2",
        "flops": flops,
        "ms_per_step": ms_step,
        "ms_attention": ms_attn,
        "step_minus_attention_us": (ms_step_ev - ms_attn) * 1e3,  # both by HIP events
        "tflops": flops / ms_attn / 1e9,
        "frac_bf16_peak": flops / ms_attn / 1e9 / BF16_PEAK_TFLOPS,
        "tokens_per_s": sum(s.num_new_tokens for s in wl.seqs) / (ms_step / 1e3),
    }
    log(f"prefill_8b: attention {ms_attn:.3f} ms -> {res['tflops']:.0f} TFLOP/s")
    if cpu:
        log("cpu baseline: prefill_8b")
        res["cpu_baseline"] = cpu_prefill_leg(wl, 10.0, "prefill_8b")
    del wl
    torch.cuda.empty_cache()
    # The same batch over an fp8 cache: the prefill rows' keys and values are
    # dequantised into a bf16 copy and the tile-loop kernel runs on it.
    log("building prefill_8b (fp8 cache)")
    wl = W.prefill_8b("cuda", kv="fp8")
    ms_step8, _, ms_attn8 = paired_steps(step(wl), attention_only(wl), steps, warmup)
    res["fp8_cache"] = {
        "ms_per_step": ms_step8,
        "ms_attention": ms_attn8,
        "tflops": flops / ms_attn8 / 1e9,
        "vs_bf16_cache": ms_attn / ms_attn8,
    }
    log(f"prefill_8b/fp8 cache: attention {ms_attn8:.3f} ms -> {res['fp8_cache']['tflops']:.0f} TFLOP/s")
    del wl
    torch.cuda.empty_cache()
    return res


def bench_quant(steps, warmup, cpu=False):
    from nanovllm_self_amd import workloads as W

    out = {"workload": "decode_quant: 32q/8kv heads, D128, bs256, 256 seqs, ctx U[1024,4096], 1% outliers x8, seed 3"}
    for kv in ("bf16", "fp8", "int8"):
        log(f"building decode_quant ({kv})")
        wl = W.decode_quant("cuda", kv=kv)
        nbytes = wl.decode_bytes()
        ms_step, _, ms_attn = paired_steps(step(wl), attention_only(wl), steps, warmup)
        out[kv] = {
            "bytes": nbytes,
            "ms_per_step": ms_step,
            "ms_attention": ms_attn,
            "gbs_attention": nbytes / ms_attn / 1e6,
            "tokens_per_s": wl.num_seqs / (ms_step / 1e3),
        }
        log(f"decode_quant/{kv}: {ms_step:.3f} ms/step -> {out[kv]['tokens_per_s']:.0f} tok/s")
        if cpu and kv != "bf16":
            log(f"cpu baseline: decode_quant/{kv}")
            out[kv]["cpu_baseline"] = cpu_decode_leg(wl, 5.0, f"decode_quant/{kv}", dequant_timed=True)
        del wl
        torch.cuda.empty_cache()
    out["fp8_vs_bf16_tokens"] = out["fp8"]["tokens_per_s"] / out["bf16"]["tokens_per_s"]
    out["int8_vs_bf16_tokens"] = out["int8"]["tokens_per_s"] / out["bf16"]["tokens_per_s"]
    return out


def bench_prep(steps, warmup):
    """The fused pre-attention step (q/k RMSNorm + rotary embedding + KV
    store, one launch) against the same work as separate eager ops (the
    reference's RMSNorm and rotary formulas in torch, then the store
    kernel), at the decode_8b and prefill_8b token counts."""
    from nanovllm_self_amd import PagedAttention
    from nanovllm_self_amd.kv_cache import KVCacheConfig, allocate_kv_cache, bind_kv_cache

    Hq, Hkv, D, bs, NB, max_pos = 32, 8, 128, 256, 1024, 40960
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float, device=dev) / D))
    freqs = torch.einsum("i,j->ij", torch.arange(max_pos, device=dev).float(), inv_freq)
    table = torch.cat((freqs.cos(), freqs.sin()), dim=1).unsqueeze(1)  # [max_pos, 1, D]
    out = {"workload": "Qwen3-8B heads (32q/8kv, D128), bf16 KV, block 256; q/k/v random, positions "
                       "random in [0, 40960), every token stored"}

    def rms(x, w, eps=1e-6):  # RMSNorm.py:11-18
        x32 = x.float()
        return (w.float() * x32 / torch.sqrt(x32.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)

    def rope(x, cos, sin):  # RoPE.py:5-25
        x1, x2 = torch.chunk(x.float(), 2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)

    for name, T in (("decode_8b", 64), ("prefill_8b", 36864)):
        cfg = KVCacheConfig(dtype=torch.bfloat16, kv_cache_dtype=torch.bfloat16,
                            attention_compute_dtype=torch.bfloat16, block_size=bs, num_blocks=NB * (1 + T // 4096))
        attn = PagedAttention(Hq, Hkv, D, dtype=torch.bfloat16)
        kv_cache, scales = allocate_kv_cache(1, Hkv, D, cfg, dev)
        bind_kv_cache([attn], kv_cache, scales, cfg)
        q = torch.randn(T, Hq, D, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(T, Hkv, D, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(T, Hkv, D, generator=g, device=dev).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(D, generator=g, device=dev)).to(torch.bfloat16)
        pos = torch.randint(0, max_pos, (T,), generator=g, device=dev)
        slots = torch.randperm(cfg.num_blocks * bs, generator=g, device=dev)[:T].to(torch.int32)

        def fused():
            attn.qk_norm_rope_store(q, k, v, pos, w, w, 1e-6, table, slots)

        def unfused():
            cs = table[pos]
            cos, sin = cs.chunk(2, dim=-1)
            qr, kr = rope(rms(q, w), cos, sin), rope(rms(k, w), cos, sin)
            attn.store_kv_cache_torch(kr, v, slots)
            return qr

        nbytes = T * (2 * D * (2 * Hq + 4 * Hkv) + 4 * D)
        _, ms_f = timed_steps(fused, steps, warmup)
        _, ms_u = timed_steps(unfused, steps, warmup)
        out[name] = {"tokens": T, "bytes": nbytes, "ms_fused": ms_f, "gbs_fused": nbytes / ms_f / 1e6,
                     "ms_unfused": ms_u, "speedup": ms_u / ms_f}
        log(f"prep {name}: fused {ms_f * 1e3:.1f} us ({nbytes / ms_f / 1e6:.0f} GB/s), "
            f"eager ops {ms_u * 1e3:.1f} us")
        del attn, kv_cache, q, k, v
        torch.cuda.empty_cache()
    return out


def context_kernel_us(seqs, steps, warmup):
    """nvs_build_context alone (with the padded block table), launched back
    to back on resident inputs."""
    from nanovllm_self_amd import _lib

    B, T = len(seqs), sum(s.num_new_tokens for s in seqs)
    W = max(len(s.block_table) for s in seqs)
    counts = torch.tensor([s.num_cached_tokens for s in seqs] + [s.num_new_tokens for s in seqs],
                          dtype=torch.int32, device="cuda")
    lens = [len(s.block_table) for s in seqs]
    offsets = torch.tensor([sum(lens[:i]) for i in range(B + 1)], dtype=torch.int32, device="cuda")
    ids = torch.tensor([x for s in seqs for x in s.block_table], dtype=torch.int32, device="cuda")
    out = torch.empty(3 * B + 2 + T + B * W, dtype=torch.int32, device="cuda")
    pos = torch.empty(T, dtype=torch.int64, device="cuda")
    lib, st = _lib.load(), _lib.stream_of(out)
    p = out.data_ptr()

    def launch():
        _lib.check(lib.nvs_build_context(counts.data_ptr(), counts.data_ptr() + 4 * B, B, offsets.data_ptr(),
                                         ids.data_ptr(), ids.numel(), 256, T, p, p + 4 * (B + 1), p + 8 * (B + 1),
                                         p + 4 * (3 * B + 2), pos.data_ptr(), p + 4 * (3 * B + 2 + T), W, st),
                   "build_context")

    _, ms = timed_steps(launch, steps, warmup)
    return ms * 1e3


def bench_context(steps, warmup):
    """Step metadata for the measured batches: the device builder
    (build_context_on_device: host packing + one pinned copy + one launch)
    against the vectorised host builder (build_context), each timed to a
    synchronised device Context; the CPU baseline is the reference's
    per-token loop restated in Python plus the device tensors it makes from
    the lists."""
    from nanovllm_self_amd import workloads as W
    from nanovllm_self_amd.kv_cache import build_context, build_context_on_device
    from oracle import context_oracle as CO

    dev = torch.device("cuda")
    out = {"workload": "sequence lists of decode_8b, prefill_8b, decode_quant, mixed_32b (block 256)"}
    for name, seqs in W.step_batches().items():
        T = sum(s.num_new_tokens for s in seqs)

        def host():
            build_context(seqs, 256, dev)
            torch.cuda.synchronize()

        def device():
            build_context_on_device(seqs, 256, dev)
            torch.cuda.synchronize()

        res = {"seqs": len(seqs), "tokens": T}
        for label, fn in (("device", device), ("host", host)):
            for _ in range(warmup):
                fn()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            res[f"{label}_us"] = (time.perf_counter() - t0) * 1e6 / steps
        res["kernel_us"] = context_kernel_us(seqs, steps, warmup)
        # CPU baseline: the reference's loop (restated) plus the device tensors
        # it creates from the lists (model_runner.py:519-531, 334-344).
        tup = [(s.block_table, s.num_cached_tokens, s.num_new_tokens, s.need_logits) for s in seqs]

        def reference():
            r = CO.prepare_model_input(tup, 256)
            for f in ("cu_seqlens_q", "cu_seqlens_k", "slot_mapping", "context_lens", "seq_need_compute_logits"):
                torch.tensor(r[f], dtype=torch.int32, device=dev)
            torch.tensor(r["positions"], dtype=torch.int64, device=dev)
            if r["block_tables"] is not None:
                torch.tensor(r["block_tables"], dtype=torch.int32, pin_memory=True).to(dev)
            torch.cuda.synchronize()

        reference()
        t0 = time.perf_counter()
        reps = 0
        while reps < 3 or time.perf_counter() - t0 < 0.5:
            reference()
            reps += 1
        res["cpu_baseline_reference_us"] = (time.perf_counter() - t0) * 1e6 / reps
        out[name] = res
        log(f"context {name}: device {res['device_us']:.0f} us (kernel {res['kernel_us']:.1f}), host numpy "
            f"{res['host_us']:.0f} us, reference loop + copies {res['cpu_baseline_reference_us']:.0f} us ({T} tokens)")
    return out


def bench_handoff(steps, warmup):
    """KV handoff copies at the Qwen3-8B cache shape (36 layers, 8 kv heads,
    D 128, block 256): export of one 4096-token sequence's 16 blocks into a
    snapshot and import of the snapshot into other blocks, against the
    reference's torch expressions on the same GPU (kv_cache[:, :, ids]
    .contiguous(); a copy_ per block)."""
    from nanovllm_self_amd.kv_cache import (KVCacheConfig, allocate_kv_cache, export_kv_blocks,
                                            import_kv_blocks)

    L, Hkv, D, bs, NB, n = 36, 8, 128, 256, 128, 16
    out = {"workload": f"Qwen3-8B cache ({L} layers, {Hkv} kv heads, D{D}, block {bs}, {NB}-block pool); "
                       f"{n} blocks (one 4096-token sequence) exported and imported"}
    for kv, dt, mode in (("bf16", torch.bfloat16, "none"), ("fp8", torch.float8_e4m3fn, "fp8_e4m3")):
        cfg = KVCacheConfig(dtype=torch.bfloat16, kv_cache_dtype=dt, attention_compute_dtype=torch.bfloat16,
                            kv_cache_quant_mode=mode, block_size=bs, num_blocks=NB)
        kvc, sc = allocate_kv_cache(L, Hkv, D, cfg, "cuda")
        g = torch.Generator().manual_seed(6)
        perm = torch.randperm(NB, generator=g).tolist()
        src_ids, dst_ids = perm[:n], perm[n:2 * n]
        blocks, scales = export_kv_blocks(kvc, sc, src_ids)
        moved = 2 * (blocks.numel() * blocks.element_size() + (scales.numel() * 4 if scales is not None else 0))

        def ref_export():
            kvc[:, :, src_ids].contiguous()
            if sc is not None:
                sc[:, :, src_ids].contiguous()

        def ref_import():
            for i, b in enumerate(dst_ids):
                kvc[:, :, b].copy_(blocks[:, :, i])
                if sc is not None:
                    sc[:, :, b].copy_(scales[:, :, i])

        res = {"bytes_moved": moved}
        for label, fn in (("export", lambda: export_kv_blocks(kvc, sc, src_ids)),
                          ("import", lambda: import_kv_blocks(kvc, sc, blocks, scales, dst_ids)),
                          ("ref_export", ref_export), ("ref_import", ref_import)):
            _, ms = timed_steps(fn, steps, warmup)
            res[f"{label}_us"] = ms * 1e3
            res[f"{label}_gbs"] = moved / ms / 1e6
        out[kv] = res
        log(f"handoff {kv}: export {res['export_us']:.0f} us ({res['export_gbs']:.0f} GB/s), import "
            f"{res['import_us']:.0f} us; torch: {res['ref_export_us']:.0f} / {res['ref_import_us']:.0f} us")
        del kvc, sc, blocks, scales
        torch.cuda.empty_cache()
    return out


def bench_mixed(steps, warmup, cpu=False):
    from nanovllm_self_amd import workloads as W

    out = {"workload": "mixed_32b: 64q/8kv heads, 128 decode seqs ctx logU[256,32768] + 4 x 2048-token chunks over U[0,16384] cached, 16384 blocks, seed 4"}
    for kv in ("bf16", "fp8"):
        log(f"building mixed_32b ({kv})")
        wl = W.mixed_32b("cuda", kv=kv)
        ms_step, _, ms_attn = paired_steps(step(wl), attention_only(wl), steps, warmup)
        dec_b, pf = wl.decode_bytes(), wl.prefill_flops()
        t_roof = dec_b / (HBM_PEAK_GBS * 1e9) + pf / (BF16_PEAK_TFLOPS * 1e12)
        out[kv] = {
            "ms_per_step": ms_step,
            "ms_attention": ms_attn,
            "decode_bytes": dec_b,
            "prefill_flops": pf,
            "roofline_ms": t_roof * 1e3,
            "frac_roofline": t_roof * 1e3 / ms_step,
        }
        log(f"mixed_32b/{kv}: {ms_step:.3f} ms/step (roofline {t_roof * 1e3:.3f} ms)")
        if cpu and kv == "bf16":
            log("cpu baseline: mixed_32b")
            dec = cpu_decode_leg(wl, 6.0, "mixed_32b decode part")
            pre = cpu_prefill_leg(wl, 6.0, "mixed_32b prefill part")
            ms = (dec_b / (dec["value"] * 1e9) + pf / (pre["value"] * 1e12)) * 1e3
            out[kv]["cpu_baseline"] = dict(
                value=round(ms, 1), unit="ms per step (extrapolated from the two parts' rates)",
                cores=dec["cores"], kind="port", decode_part=dec, prefill_part=pre,
                sample="decode rows and prefill row blocks as sampled below, each rate applied to the "
                       "step's decode bytes / prefill FLOPs", **cpu_host())
        del wl
        torch.cuda.empty_cache()
        if kv == "bf16":
            # The step's four prefill chunks alone (2048 rows over 0-16 K
            # cached keys each): the prefill kernel's rate on long units.
            log("building mixed_32b prefill chunks (bf16)")
            wc = W.mixed_32b_chunks("cuda", kv=kv)
            pf_c = wc.prefill_flops()
            _, ms_c = timed_steps(attention_only(wc), steps, warmup)
            out[kv]["prefill_chunks"] = {
                "flops": pf_c,
                "ms_attention": ms_c,
                "tflops": pf_c / ms_c / 1e9,
                "frac_bf16_peak": pf_c / ms_c / 1e9 / BF16_PEAK_TFLOPS,
            }
            log(f"mixed_32b prefill chunks alone: attention {ms_c:.3f} ms -> {pf_c / ms_c / 1e9:.0f} TFLOP/s")
            del wc
            torch.cuda.empty_cache()
    return out


def cpu_threads() -> int:
    """Host threads for the CPU leg: the job's OpenMP share when set (the GPU
    host's per-GPU share), else every visible core."""
    try:
        return max(1, int(os.environ["OMP_NUM_THREADS"]))
    except (KeyError, ValueError):
        return os.cpu_count() or 1


def cpu_host():
    """The host CPU's model name (/proc/cpuinfo, as lscpu reports it) and its
    logical CPU count."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.lower().startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count()}


def _cpu_setup():
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    torch.set_num_threads(cpu_threads())


def _host_seq(wl, i, dequant_timed=False):
    """Sequence i's query rows and cache blocks in host memory (untimed: the
    CPU path, like the GPU one, starts from resident data).  With
    dequant_timed, a quantised cache stays as codes and scales and the
    returned `prepare` dequantises them (the eager path's dequantize step,
    timed with the attention); otherwise `prepare` is the identity."""
    import numpy as np
    from oracle import kv_oracle as KO
    from tests.gpu_util import bf16_to_np, oracle_paged_inputs

    args, _ = oracle_paged_inputs(wl, [i])
    if not (dequant_timed and wl.kv != "bf16"):
        return args, lambda a: a
    s = wl.seqs[i]
    n = s.num_cached_tokens + s.num_new_tokens
    idx = torch.as_tensor(s.block_table[:(n + wl.block_size - 1) // wl.block_size], dtype=torch.long,
                          device=wl.attn.k_cache.device)
    raw = []
    for cache, scale in ((wl.attn.k_cache, wl.attn.k_scale_cache), (wl.attn.v_cache, wl.attn.v_scale_cache)):
        codes = cache.index_select(0, idx).cpu().view(torch.uint8).numpy()
        if wl.kv == "int8":
            codes = codes.view(np.int8)
        raw.append((codes, scale.index_select(0, idx).cpu().numpy()))

    def prepare(a):
        kv = [KO.round_to_bf16(KO.dequantize_per_token(c, sc, wl.kv)) for c, sc in raw]
        return (a[0], kv[0], kv[1]) + tuple(a[3:])

    return args, prepare


def cpu_decode_leg(wl, budget_s, label, dequant_timed=False, full_passes=0):
    """Decode rows through the eager restatement on the host cores: per
    sequence, (dequantise,) gather and fp32 attention, in batch order, until
    about `budget_s` seconds (with full_passes > 0: whole passes over the
    batch, at least that many, the rate taken over all of them).  Units: the
    GPU figures' units, decode bytes / s and decode rows (tokens) / s."""
    from oracle import attn_oracle

    _cpu_setup()
    ids = list(wl.decode_seq_ids())
    ctx = [wl.seqs[i].num_cached_tokens + wl.seqs[i].num_new_tokens for i in ids]
    H, D, Hq = wl.num_kv_heads, wl.head_dim, wl.num_heads
    s_kv, s_sc = (2, 0) if wl.kv == "bf16" else (1, 4)
    seq_bytes = [c * H * 2 * (D * s_kv + s_sc) + Hq * D * 2 * 2 for c in ctx]
    keep = {}
    nbytes, rows, t, passes, stop = 0, 0, 0.0, 0, False
    while not stop:
        for j, i in enumerate(ids):
            args, prep = keep[i] if i in keep else _host_seq(wl, i, dequant_timed)
            if full_passes:
                keep[i] = (args, prep)
            if rows == 0:  # warm-up
                attn_oracle.paged_attention(*prep(args))
            t0 = time.perf_counter()
            attn_oracle.paged_attention(*prep(args))
            t += time.perf_counter() - t0
            nbytes += seq_bytes[j]
            rows += 1
            if t >= budget_s and not full_passes:
                stop = True
                break
        else:
            passes += 1
            stop = stop or (full_passes and passes >= full_passes and t >= budget_s)
    keep.clear()
    if full_passes:
        what = f"{passes} full passes over the batch's {len(ids)} rows"
    elif rows > len(ids):
        what = f"{rows} rows: the batch's {len(ids)} rows in order, repeated"
    else:
        what = f"the first {rows} of the batch's {len(ids)} rows"
    sample = (f"{label}: {what}, {nbytes / 1e9:.2f} GB, {t:.1f} s: per row "
              + ("dequantise + " if dequant_timed and wl.kv != "bf16" else "")
              + "gather + fp32 attention from host memory")
    return dict(value=round(nbytes / t / 1e9, 4), unit="GB/s", tokens_per_s=round(rows / t, 2),
                cores=torch.get_num_threads(), kind="port", sample=sample, **cpu_host())


def cpu_prefill_leg(wl, budget_s, label, rows_per_block=256):
    """Prefill rows through the eager restatement on the host cores, in
    blocks of query rows: a row block [r0, r1) of a sequence with P cached
    tokens is the same attention as a sequence of r1 - r0 new tokens over
    P + r1 keys, so the sample is whole row blocks of the batch's sequences,
    in order, until about `budget_s` seconds.  Unit: TFLOP/s counted as the
    GPU figure counts them (4 Hq D per visible query-key pair)."""
    from oracle import attn_oracle

    _cpu_setup()
    Hq, D = wl.num_heads, wl.head_dim
    flops, t, nblk = 0.0, 0.0, 0
    warm = False
    for i in wl.prefill_seq_ids():
        s = wl.seqs[i]
        P, L = s.num_cached_tokens, s.num_new_tokens
        args, _ = _host_seq(wl, i)
        q = args[0]
        for r0 in range(0, L, rows_per_block):
            r1 = min(L, r0 + rows_per_block)
            klen = P + r1
            blk = (q[r0:r1], args[1], args[2], args[3], [0, r1 - r0], [0, klen], [klen]) + tuple(args[7:])
            if not warm:
                attn_oracle.paged_attention(*blk)
                warm = True
            t0 = time.perf_counter()
            attn_oracle.paged_attention(*blk)
            t += time.perf_counter() - t0
            flops += 4.0 * Hq * D * ((r1 - r0) * P + (r1 * (r1 + 1) - r0 * (r0 + 1)) // 2)
            nblk += 1
            if t >= budget_s:
                break
        if t >= budget_s:
            break
    sample = (f"{label}: {nblk} blocks of up to {rows_per_block} query rows, sequences in batch order, "
              f"{flops / 1e12:.3f} TFLOP, {t:.1f} s: per block gather + fp32 attention with the "
              f"bottom-right causal mask, from host memory")
    return dict(value=round(flops / t / 1e12, 5), unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                sample=sample, **cpu_host())


def cpu_baseline(wl, budget_s: float = 10.0):
    """The headline's CPU leg: decode_8b rows through the eager restatement
    (gather + per-sequence fp32 attention, the reference's torch path) on
    the host cores.  Unit: decode bytes / s, the GPU figure's unit."""
    return cpu_decode_leg(wl, budget_s, "decode_8b")


def decode_traffic():
    """HBM bytes per decode call as measured by the committed rocprofv3 PMC
    runs (FETCH_SIZE + WRITE_SIZE, scaled by a plain copy's readings), or
    None when no measurement is committed."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "decode_8b_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["bytes_per_call"]
    except (OSError, ValueError, KeyError):
        return None


def calib_copy(nbytes: int = 1 << 30, reps: int = 5):
    """A plain device copy of known size: reads and writes `nbytes` per
    launch; its FETCH_SIZE / WRITE_SIZE readings scale the counters of the
    attention kernels to bytes."""
    src = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").normal_()
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calib_copy_bytes": nbytes, "reps": reps}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["decode", "prefill", "quant", "mixed", "prep", "context", "handoff", "layers"],
                    default=None)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run a 1 GiB device copy (for scaling PMC byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path has no multi-GPU code); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    from nanovllm_self_amd import _lib

    _lib.load()
    torch.cuda.set_device(0)
    steps, warmup = args.steps, args.warmup
    if args.calib_copy:
        calib_copy()
        return

    if args.only == "prefill":
        print(json.dumps(bench_prefill(steps, warmup)))
        return
    if args.only == "quant":
        print(json.dumps(bench_quant(steps, warmup)))
        return
    if args.only == "mixed":
        print(json.dumps(bench_mixed(steps, warmup)))
        return
    if args.only == "prep":
        print(json.dumps(bench_prep(steps, warmup)))
        return
    if args.only == "context":
        print(json.dumps(bench_context(steps, warmup)))
        return
    if args.only == "handoff":
        print(json.dumps(bench_handoff(steps, warmup)))
        return
    if args.only == "layers":
        print(json.dumps(bench_layers(steps, warmup)))
        return

    want_cpu = args.only is None and not args.no_cpu
    wl, dec = bench_decode(steps, warmup, cpu=want_cpu)
    line = {
        "metric": "paged-decode attn GB/s (%HBM peak) + prefill attn TFLOP/s, Qwen3-8B shape",
        "value": round(dec["gbs_step"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(dec["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode_8b: Qwen3-8B attention layer, 32q/8kv heads, D128, bf16 KV, block 256, "
                        "4096-block pool, 64 seqs ctx U[2048,8192] (seed 1); step = store + decode",
            "global_batch": wl.num_seqs,
            "seq_len": wl.context.max_seqlen_k,
            "parallelism": "none (1 GPU)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "paged_attention decode call (stream-K decode kernel + merge of split rows)",
            "achieved": round(dec["gbs_attention"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["gbs_attention"] / HBM_PEAK_GBS, 4),
            "traffic": decode_traffic(),
        },
        "decode_8b": dec,
    }
    if args.only is None:
        if not args.no_cpu:
            log("cpu baseline")
            line["cpu_baseline"] = cpu_baseline(wl)
        del wl
        torch.cuda.empty_cache()
        line["prefill_8b"] = bench_prefill(steps, warmup, cpu=want_cpu)
        line["decode_quant"] = bench_quant(steps, warmup, cpu=want_cpu)
        line["mixed_32b"] = bench_mixed(steps, warmup, cpu=want_cpu)
        line["qk_prep"] = bench_prep(steps, warmup)
        line["step_context"] = bench_context(steps, warmup)
        line["kv_handoff"] = bench_handoff(steps, warmup)
        line["layers36_decode_step"] = bench_layers(steps, warmup)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
