"""The allocation-free entry point nvs_paged_attention_store_noalloc (its
workspace is the library's static per-device scratch) against
nvs_paged_attention_store with a caller workspace: the same kernels on the
same inputs, so output and cache bytes must be equal bit for bit, on two
calls in a row (a mixed prefill + decode batch, then a smaller decode
batch whose tokens the decode kernel writes), and a batch that needs more
scratch than the library holds is refused before any launch."""
import ctypes

import pytest
import torch

from nanovllm_self_amd import _lib
from nanovllm_self_amd import workloads as W
from nanovllm_self_amd.layers.attention import attention_workspace
from tests.gpu_util import say

pytestmark = pytest.mark.gpu

NVS_ERR_WORKSPACE = -3


def _noalloc():
    fn = _lib.load().nvs_paged_attention_store_noalloc
    assert list(fn.argtypes) == list(_lib.SIGNATURES["nvs_paged_attention_store"][1][:-3]) + [ctypes.c_void_p]
    return fn


def _store_args(wl, out):
    a, ctx = wl.attn, wl.context
    kc, vc = a.k_cache, a.v_cache
    quant = kc.dtype != torch.bfloat16
    bt = ctx.block_tables
    return [
        wl.q.data_ptr(), wl.q.stride(0), wl.q.stride(1),
        wl.k.data_ptr(), wl.v.data_ptr(), _lib.NVS_DTYPE_BF16, wl.k.stride(0), wl.k.stride(1),
        wl.v.stride(0), wl.v.stride(1), ctx.slot_mapping.data_ptr(),
        kc.data_ptr(), vc.data_ptr(), _lib.nvs_dtype(kc.dtype),
        a.k_scale_cache.data_ptr() if quant else None, a.v_scale_cache.data_ptr() if quant else None,
        ctx.cu_seqlens_q.data_ptr(), ctx.cu_seqlens_k.data_ptr(), bt.data_ptr(), bt.size(1),
        ctx.cu_seqlens_q.numel() - 1, wl.q.shape[0], int(ctx.max_seqlen_q), int(ctx.max_seqlen_k),
        wl.num_heads, wl.num_kv_heads, wl.head_dim, wl.block_size, kc.shape[0],
        wl.head_dim ** -0.5, out.data_ptr(), out.stride(0), out.stride(1),
    ]


def _cache_bytes(attn):
    out = [attn.k_cache.view(torch.uint8).clone(), attn.v_cache.view(torch.uint8).clone()]
    if attn.k_scale_cache is not None:
        out += [attn.k_scale_cache.clone(), attn.v_scale_cache.clone()]
    return out


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_noalloc_equals_workspace_entry(device, kv):
    lib = _lib.load()
    noalloc = _noalloc()
    stream = torch.cuda.current_stream().cuda_stream
    builders = [
        ("mixed (24 decode rows + 2 chunks of 384)",
         lambda: W.mixed_32b(device, kv=kv, n_decode=24, n_chunks=2, chunk=384)),
        ("decode_small (8 rows)", lambda: W.decode_small(device, kv=kv)),
    ]
    for what, make in builders:
        say(f"no-alloc entry vs workspace entry: {what} {kv}")
        a, b = make(), make()
        ctx = a.context
        ws_bytes = int(lib.nvs_attention_workspace_bytes(
            ctx.cu_seqlens_q.numel() - 1, int(ctx.max_seqlen_q), int(ctx.max_seqlen_k), a.num_heads,
            a.num_kv_heads, a.head_dim, 0))
        ws = attention_workspace(device, ws_bytes)
        out_a = torch.empty_like(a.q)
        out_b = torch.empty_like(b.q)
        _lib.check(lib.nvs_paged_attention_store(*_store_args(a, out_a), ws.data_ptr(), ws_bytes, stream),
                   "paged_attention_store")
        _lib.check(noalloc(*_store_args(b, out_b), stream), "paged_attention_store_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(out_a, out_b), f"{what}: outputs differ"
        for x, y in zip(_cache_bytes(a.attn), _cache_bytes(b.attn)):
            assert torch.equal(x, y), f"{what}: cache contents differ"


def test_noalloc_refuses_a_batch_beyond_its_scratch(device):
    """60000 rows of up to 8192 new tokens need a plan far above 32 MiB: the
    call returns NVS_ERR_WORKSPACE with a message and launches nothing (the
    pointers are never read)."""
    noalloc = _noalloc()
    say("no-alloc entry: oversize batch refused")
    p = 256  # a non-null stand-in; the size check returns before any use
    rc = noalloc(p, 1024, 128, p, p, 0, 256, 128, 256, 128, p, p, p, 0, None, None, p, p, p, 64,
                 60000, 60000 * 8, 8192, 8192, 32, 8, 128, 256, 4096, 0.088, p, 1024, 128,
                 torch.cuda.current_stream().cuda_stream)
    assert rc == NVS_ERR_WORKSPACE
    msg = _lib.load().nvs_last_error().decode()
    assert "scratch" in msg and "workspace" in msg, msg
