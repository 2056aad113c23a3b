"""The drop-in boundary, on the CPU: library exports, Context fields, the
KV-pool/config knobs, the step-metadata builder and the guards that fire
before any launch."""
import dataclasses
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from nanovllm_self_amd import PagedAttention, Attention, _lib
from nanovllm_self_amd.kv_cache import (
    KVCacheConfig, SeqSlice, allocate_kv_cache, bind_kv_cache, build_context, prepare_block_tables,
)
from nanovllm_self_amd.utils.context import Context, get_context

ROOT = Path(__file__).resolve().parents[1]


def test_library_exports_every_declared_symbol():
    header = (ROOT / "include" / "nvs_attention.h").read_text()
    declared = set(re.findall(r"\b(nvs_[a-z0-9_]+)\s*\(", header))
    assert declared, "no declarations parsed"
    lib = _lib.load()
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    assert lib.nvs_version() >= 100


def _declared_params(header):
    """Parameter C types of each nvs_* declaration in the header, in order."""
    out = {}
    for m in re.finditer(r"^\s*(?:int|int64_t|const char\*)\s+(nvs_[a-z0-9_]+)\s*\(([^;]*?)\)\s*;", header,
                         re.M | re.S):
        body = re.sub(r"/\*.*?\*/", "", m.group(2), flags=re.S).strip()
        params = [] if body in ("", "void") else [x.strip() for x in body.split(",")]
        out[m.group(1)] = params
    return out


def _ctype_of(decl):
    if "*" in decl:
        return ctypes.c_void_p
    t = decl.rsplit(" ", 1)[0].replace("const ", "").strip()
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "float": ctypes.c_float}[t]


def test_bindings_match_the_header():
    """The ctypes argtypes (_lib.SIGNATURES) match every header declaration
    in count and C type."""
    header = (ROOT / "include" / "nvs_attention.h").read_text()
    decls = _declared_params(header)
    assert set(decls) == set(_lib.SIGNATURES), set(decls) ^ set(_lib.SIGNATURES)
    for name, params in decls.items():
        want = [_ctype_of(p) for p in params]
        got = list(_lib.SIGNATURES[name][1])
        assert got == want, f"{name}: SIGNATURES {got} vs header {want}"


def test_context_fields_match_reference():
    # nanovllm/utils/context.py:5-36
    names = [f.name for f in dataclasses.fields(Context)]
    assert names == ["cu_seqlens_q", "cu_seqlens_k", "max_seqlen_q", "max_seqlen_k", "slot_mapping",
                     "context_lens", "block_tables", "seq_need_compute_logits"]
    c = get_context(max_seqlen_q=3)
    assert c.max_seqlen_q == 3 and c.block_tables is None


def test_attention_module_surface():
    a = Attention(32, 8, 128)
    assert isinstance(a, PagedAttention)
    assert a.groups == 4 and a.dtype == torch.bfloat16
    for attr in ("k_cache", "v_cache", "block_size", "layer_id", "kv_cache_quant_mode", "kv_cache_dtype",
                 "attention_compute_dtype", "forward_backend", "k_scale_cache", "v_scale_cache",
                 "prefill_backend", "decode_backend", "enable_profile", "profile_decode",
                 "in_cuda_graph_capture", "kv_writer_backend"):
        assert hasattr(a, attr), attr
    assert set(a.profile_decode) == {"store", "load", "attn", "gqa_expand", "permute", "qk", "softmax", "av", "calls"}
    for m in ("forward", "forward_unified", "write_kv_cache", "store_kv_cache_torch", "get_kv_cache",
              "prefill_torch", "prefill_flashattn", "quantize_int8_per_token", "dequantize_int8_per_token",
              "decode_flashattn"):
        assert callable(getattr(a, m)), m


@pytest.mark.parametrize("alias,dt", [("bf16", torch.bfloat16), ("bfloat16", torch.bfloat16),
                                      ("fp16", torch.float16), ("float16", torch.float16),
                                      ("fp32", torch.float32), ("float32", torch.float32)])
def test_config_aliases(alias, dt):
    # pd_self/evaluation/test_kv_cache_dtype_matrix.py:35-51
    c = KVCacheConfig(kv_cache_dtype=alias, attention_compute_dtype=alias)
    assert c.kv_cache_dtype == dt and c.attention_compute_dtype == dt


def test_config_quant_modes():
    assert KVCacheConfig().block_size == 256
    assert KVCacheConfig().kv_cache_dtype == torch.bfloat16
    assert KVCacheConfig(kv_cache_quant_mode="int8_mock").kv_cache_dtype == torch.int8
    assert KVCacheConfig(kv_cache_quant_mode="fp8_e4m3").kv_cache_dtype == torch.float8_e4m3fn
    with pytest.raises(ValueError, match="unsupported kv_cache_quant_mode"):
        KVCacheConfig(kv_cache_quant_mode="int4")


def test_allocate_and_bind_layout():
    cfg = KVCacheConfig(kv_cache_quant_mode="fp8_e4m3", block_size=256, num_blocks=3)
    kv, sc = allocate_kv_cache(2, 4, 128, cfg, "cpu")
    assert kv.shape == (2, 2, 3, 256, 4, 128) and kv.dtype == torch.float8_e4m3fn
    assert sc.shape == (2, 2, 3, 256, 4, 1) and sc.dtype == torch.float32 and torch.all(sc == 1)
    layers = [PagedAttention(8, 4, 128), PagedAttention(8, 4, 128)]
    bind_kv_cache(layers, kv, sc, cfg)
    assert layers[1].k_cache.data_ptr() == kv[0, 1].data_ptr() and layers[1].k_cache.is_contiguous()
    assert layers[0].v_scale_cache.data_ptr() == sc[1, 0].data_ptr()
    assert layers[1].layer_id == 1 and layers[0].kv_cache_quant_mode == "fp8_e4m3"


def test_build_context_matches_reference_formula():
    # model_runner.py:461-532 on a decode row, a chunk over a prefix and a fresh prompt
    bs = 4
    seqs = [SeqSlice([7, 2], 5, 1), SeqSlice([1, 3, 0], 4, 5), SeqSlice([6], 0, 3)]
    c = build_context(seqs, bs, "cpu")
    assert c.cu_seqlens_q.tolist() == [0, 1, 6, 9]
    assert c.cu_seqlens_k.tolist() == [0, 6, 15, 18]
    assert c.context_lens.tolist() == [6, 9, 3]
    assert (c.max_seqlen_q, c.max_seqlen_k) == (5, 9)
    ref = []
    for s in seqs:
        for p in range(s.num_cached_tokens, s.num_cached_tokens + s.num_new_tokens):
            ref.append(s.block_table[p // bs] * bs + p % bs)
    assert c.slot_mapping.tolist() == ref
    assert c.block_tables.tolist() == [[7, 2, -1], [1, 3, 0], [6, -1, -1]]
    assert c.slot_mapping.dtype == torch.int32 and c.block_tables.dtype == torch.int32
    fresh = build_context([SeqSlice([0], 0, 3), SeqSlice([1], 0, 2)], bs, "cpu")
    assert fresh.block_tables is None
    assert prepare_block_tables([[1], [2, 3]], "cpu").tolist() == [[1, -1], [2, 3]]


def test_flashattn_guard_rejects_fp32_cache():
    # pd_self/evaluation/test_kv_cache_dtype_matrix.py:124-140
    a = PagedAttention(num_heads=8, num_kv_heads=8, head_dim=16)
    a.k_cache = torch.zeros(1, 256, 8, 16, dtype=torch.float32)
    a.v_cache = torch.zeros_like(a.k_cache)
    a.attention_compute_dtype = torch.float32
    z = torch.zeros(1, 8, 16)
    with pytest.raises(RuntimeError, match="fp16/bf16 kv cache"):
        a.prefill_flashattn(z, z, z, context=None)


def test_dtype_mismatch_guard():
    a = PagedAttention(8, 8, 128)
    a.k_cache = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    a.v_cache = torch.zeros_like(a.k_cache)
    a.attention_compute_dtype = torch.float16
    z = torch.zeros(1, 8, 128)
    with pytest.raises(RuntimeError, match="same dtype"):
        a.prefill_flashattn(z, z, z, context=None)


@pytest.mark.parametrize("paged", [False, True])
def test_fp16_attention_reaches_the_kernels(paged):
    """fp16 compute is served in both modes (the reference's flash path
    computes in fp16, attention.py:326-336): with CPU tensors the call gets
    past the dtype checks and stops at the device check."""
    a = PagedAttention(8, 8, 128)
    a.block_size = 256
    a.k_cache = torch.zeros(1, 256, 8, 128, dtype=torch.float16)
    a.v_cache = torch.zeros_like(a.k_cache)
    a.kv_cache_dtype = a.attention_compute_dtype = torch.float16
    z = torch.zeros(1, 8, 128, dtype=torch.float16)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    ctx = Context(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=1, max_seqlen_k=1,
                  block_tables=torch.zeros(1, 1, dtype=torch.int32) if paged else None)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        a.prefill_flashattn(z, z, z, ctx)


def test_fp16_compute_over_codes_is_refused():
    """int8 / fp8 codes are dequantised to bf16 by these kernels, where the
    reference's eager path would round them to an fp16 compute dtype: the
    layer refuses that combination instead of computing in bf16."""
    a = PagedAttention(8, 8, 128)
    a.block_size = 256
    a.kv_cache_quant_mode = "int8_mock"
    a.k_cache = torch.zeros(1, 256, 8, 128, dtype=torch.int8)
    a.v_cache = torch.zeros_like(a.k_cache)
    a.k_scale_cache = torch.ones(1, 256, 8, 1)
    a.v_scale_cache = torch.ones(1, 256, 8, 1)
    a.attention_compute_dtype = torch.float16
    z = torch.zeros(1, 8, 128, dtype=torch.float16)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    ctx = Context(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=1, max_seqlen_k=1,
                  block_tables=torch.zeros(1, 1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="codes computes in bf16"):
        a.prefill_torch(z, z, z, ctx)


@pytest.mark.parametrize("paged", [False, True])
def test_fp32_attention_is_refused_in_both_modes(paged):
    """fp32 compute (the reference's eager path allows it) is not served
    either: the layer raises instead of computing in bf16."""
    a = PagedAttention(8, 8, 128)
    a.block_size = 256
    a.k_cache = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    a.v_cache = torch.zeros_like(a.k_cache)
    a.kv_cache_dtype = torch.bfloat16
    a.attention_compute_dtype = torch.float32
    z = torch.zeros(1, 8, 128, dtype=torch.float32)
    cu = torch.tensor([0, 1], dtype=torch.int32)
    ctx = Context(cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=1, max_seqlen_k=1,
                  block_tables=torch.zeros(1, 1, dtype=torch.int32) if paged else None)
    with pytest.raises(RuntimeError, match="fp32 attention"):
        a.prefill_torch(z, z, z, ctx)


def test_no_cpu_fallback():
    a = PagedAttention(8, 8, 128)
    a.block_size = 256
    a.k_cache = torch.zeros(1, 256, 8, 128, dtype=torch.bfloat16)
    a.v_cache = torch.zeros_like(a.k_cache)
    k = torch.zeros(1, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        a.store_kv_cache_torch(k, k, torch.zeros(1, dtype=torch.int32))
    a.kv_writer_backend = "triton"
    with pytest.raises(NotImplementedError):
        a.write_kv_cache(k, k, torch.zeros(1, dtype=torch.int32))
    a.forward_backend = "nope"
    a.kv_writer_backend = "torch"
    with pytest.raises((NotImplementedError, RuntimeError)):
        a.forward(k, k, k, Context(slot_mapping=torch.zeros(1, dtype=torch.int32)))


def test_c_abi_validates_before_launch():
    """Invalid requests are rejected on the host with a message; fake
    non-null pointers are never dereferenced."""
    lib = _lib.load()
    P = 1 << 20  # 16-byte aligned, never touched
    rc = lib.nvs_paged_attention(P, 1024, 128, P, P, 0, None, None, P, P, P, 8, 1, 1, 1, 256,
                                 4, 1, 64, 256, 8, 0.125, P, 512, 128, None, 0, None)
    assert rc == -2 and b"head_dim" in lib.nvs_last_error()
    rc = lib.nvs_paged_attention(P, 1024, 128, P, P, 0, None, None, P, P, P, 8, 1, 1, 1, 256,
                                 5, 2, 128, 256, 8, 0.125, P, 512, 128, None, 0, None)
    assert rc == -1 and b"multiple of num_kv_heads" in lib.nvs_last_error()
    rc = lib.nvs_paged_attention(P, 1024, 128, P, P, 3, None, None, P, P, P, 8, 1, 1, 1, 256,
                                 4, 1, 128, 256, 8, 0.125, P, 512, 128, None, 0, None)
    assert rc == -1 and b"k_scale" in lib.nvs_last_error()
    rc = lib.nvs_paged_attention(P, 1024, 128, P, P, 0, None, None, P, P, P, 1, 1, 1, 1, 4096,
                                 4, 1, 128, 256, 8, 0.125, P, 512, 128, None, 0, None)
    assert rc == -1 and b"too short" in lib.nvs_last_error()
    rc = lib.nvs_paged_attention(P, 1024, 128, P, P, 0, None, None, P, P, P, 32, 2, 2, 1, 4096,
                                 4, 1, 128, 256, 8, 0.125, P, 512, 128, None, 0, None)
    assert rc == -3 and b"workspace" in lib.nvs_last_error()
    rc = lib.nvs_paged_attention(P, 1024, 128, P, P, 0, None, None, P, P, P, 32, 2, 2, 1, 4096,
                                 4, 1, 128, 256, 8, 0.125, P, 512, 128, P + 16, 1 << 30, None)
    assert rc == -3 and b"256-byte aligned" in lib.nvs_last_error()
    rc = lib.nvs_store_kvcache(P, P, 0, 1024, 128, 1024, 128, P, 4, P, P, 3, None, None, 8, 256,
                               8, 128, None)
    assert rc == -1 and b"k_scale" in lib.nvs_last_error()
    rc = lib.nvs_store_kvcache(P, P, 0, 1024, 128, 1024, 128, P, 4, P, P, 0, None, None, 8, 256,
                               8, 96, None)
    assert rc == -2
    assert lib.nvs_store_kvcache(P, P, 0, 8, 8, 8, 8, P, 0, P, P, 0, None, None, 8, 256, 8, 128, None) == 0


def test_fp16_calls_the_tile_loop_cannot_serve_are_refused():
    """fp16 prefill runs on the tile-loop kernel only: a local-mode fp16 call
    whose k and v token strides differ (which that kernel does not serve) is
    refused on the host, where a bf16 call would go to the classic kernel;
    the same strides in bf16 get past the check to the launch (which the
    fake pointers never reach: the dtype is refused first)."""
    lib = _lib.load()
    P = 1 << 20  # 16-byte aligned, never touched
    ws = 1 << 21
    args = (P, 1024, 128, P, P, 1024, 128, 2048, 128, P, P, 1, 4, 4, 4, 4, 8, 8, 128, 0.088,
            P, 1024, 128, ws, 1 << 24, None)
    rc = lib.nvs_varlen_attention_dtype(*args, 1)
    assert rc == -2 and b"tile-loop" in lib.nvs_last_error()
    rc = lib.nvs_varlen_attention_dtype(*args, 2)
    assert rc == -2 and b"dtype" in lib.nvs_last_error()


def test_workspace_bytes():
    """The prefill plan (256-byte header + prefill list + a 64-byte record
    per list entry, each 256-aligned) followed by the decode partials: two slots of g x (128 + 2) floats per decode
    wave, then a 4-int header and a 4-int merge record per decode wave
    (for the 2048-wave cap).  Decode waves come in groups of Hkv: at most 2048 waves, and at
    most one group per 4 32-key tiles the batch can hold, rounded up to a
    multiple of 8 groups.  An unknown kv-head count (0) gets an upper bound."""
    lib = _lib.load()
    a256 = lambda x: (x + 255) // 256 * 256

    def expect(B, max_q, max_k, Hq, Hkv):
        known = Hkv > 0 and Hq % Hkv == 0
        g = Hq // Hkv if known else Hq  # unknown: one kv head, every query head in its group
        hk = Hkv if known else 1
        tiles = B * ((max_k + 31) // 32)
        groups = ((tiles + 3) // 4 + 7) // 8 * 8
        waves = hk * min(2048 // hk, max(1, groups))
        gg = Hq // Hkv if Hkv > 0 and Hq % Hkv == 0 else 0
        pbm = 32 * (8 // min(gg, 8)) if gg > 0 else 32
        ntq = max(1, (max_q + pbm - 1) // pbm)
        return a256(256 + a256(B * ntq * 4) + a256(B * ntq * 64)) + waves * 2 * g * 130 * 4 + 2049 * 16

    # 64 decode rows, max_k 256: 512 tiles -> 128 groups of 8 waves
    assert lib.nvs_attention_workspace_bytes(64, 1, 256, 32, 8, 128, 256) == expect(64, 1, 256, 32, 8)
    assert expect(64, 1, 256, 32, 8) == a256(256 + a256(64 * 4) + a256(64 * 64)) + 1024 * 2 * 4 * 130 * 4 + 2049 * 16
    # max_k 8192: the 2048-wave cap
    assert lib.nvs_attention_workspace_bytes(64, 1, 8192, 32, 8, 128, 256) == expect(64, 1, 8192, 32, 8)
    assert expect(64, 1, 8192, 32, 8) == a256(256 + a256(64 * 4) + a256(64 * 64)) + 2048 * 2 * 4 * 130 * 4 + 2049 * 16
    # prefill tiles: 32 positions per wave, 8 waves shared by the g query heads
    # of a kv head -> 64 positions at g = 4, 32 at g >= 8, 256 at g = 1
    for Hq, Hkv in ((32, 8), (64, 4), (8, 8), (32, 0)):
        assert lib.nvs_attention_workspace_bytes(16, 4096, 256, Hq, Hkv, 128, 256) == expect(16, 4096, 256, Hq, Hkv)
    assert expect(16, 4096, 256, 32, 8) == a256(256 + a256(16 * 64 * 4) + a256(16 * 64 * 64)) + 256 * 2 * 4 * 520 + 2049 * 16


def test_workspace_unknown_kv_heads_is_upper_bound():
    """num_kv_heads = 0 (what a caller reserving ahead of time may pass) must
    size the workspace for every kv-head count the call could have."""
    lib = _lib.load()
    for B, max_q, max_k in ((1, 1, 32), (8, 1, 1000), (64, 1, 8192), (300, 1, 4096), (16, 4096, 20000), (4, 2048, 32768)):
        for Hq in (8, 16, 32, 64):
            bound = lib.nvs_attention_workspace_bytes(B, max_q, max_k, Hq, 0, 128, 256)
            for Hkv in (h for h in (1, 2, 4, 8, 16, 32, 64) if Hq % h == 0 and Hq // h <= 16):
                need = lib.nvs_attention_workspace_bytes(B, max_q, max_k, Hq, Hkv, 128, 256)
                assert bound >= need, (B, max_q, max_k, Hq, Hkv, bound, need)
