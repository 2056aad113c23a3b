"""KV handoff block copies (nvs_copy_blocks via kv_cache.export_kv_blocks /
import_kv_blocks) against the reference's own tensor expressions run on the
CPU: the snapshot kv_cache[:, :, ids] (pd_self/kv_connector.py:94-110) and
the sequential per-block copy_ loop of load_kv_item (:282-311).  Bit-exact
for every cache dtype, codes and fp32 scales alike."""
import pytest
import torch

from nanovllm_self_amd.kv_cache import KVCacheConfig, allocate_kv_cache, export_kv_blocks, import_kv_blocks
from tests.gpu_util import say

pytestmark = pytest.mark.gpu

CACHE = {"bf16": (torch.bfloat16, "none"), "int8": (torch.int8, "int8_mock"), "fp8": (torch.float8_e4m3fn, "fp8_e4m3")}


def _cache(kv, L, Hkv, D, NB, bs, device, seed):
    dt, mode = CACHE[kv]
    cfg = KVCacheConfig(dtype=torch.bfloat16, kv_cache_dtype=dt, attention_compute_dtype=torch.bfloat16,
                        kv_cache_quant_mode=mode, block_size=bs, num_blocks=NB)
    kvc, sc = allocate_kv_cache(L, Hkv, D, cfg, device)
    g = torch.Generator(device=device).manual_seed(seed)
    kvc.view(torch.uint8).copy_(torch.randint(0, 256, kvc.view(torch.uint8).shape, generator=g, device=device,
                                              dtype=torch.uint8))
    if sc is not None:
        sc.copy_(torch.rand(sc.shape, generator=g, device=device))
    return kvc, sc


def _bytes(t):
    return t.cpu().contiguous().view(torch.uint8)


@pytest.mark.parametrize("kv", ["bf16", "int8", "fp8"])
def test_export_equals_reference_indexing(device, kv):
    say(f"export_kv_blocks {kv}")
    kvc, sc = _cache(kv, 3, 2, 128, 16, 32, device, 1)
    ids = [5, 0, 11, 5, 15]
    blocks, scales = export_kv_blocks(kvc, sc, ids)
    torch.cuda.synchronize()
    assert blocks.shape == (2, 3, 5, 32, 2, 128) and blocks.dtype == kvc.dtype
    assert torch.equal(_bytes(blocks), _bytes(kvc.cpu()[:, :, ids]))
    if kv == "bf16":
        assert scales is None
    else:
        assert torch.equal(_bytes(scales), _bytes(sc.cpu()[:, :, ids]))


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
@pytest.mark.parametrize("on_host", [False, True])
def test_import_equals_reference_loop(device, kv, on_host):
    say(f"import_kv_blocks {kv} host={on_host}")
    src, src_sc = _cache(kv, 2, 8, 128, 12, 16, device, 2)
    dst, dst_sc = _cache(kv, 2, 8, 128, 20, 16, device, 3)
    blocks, scales = export_kv_blocks(src, src_sc, [1, 7, 3, 9, 4])
    if on_host:
        blocks = blocks.cpu()
        scales = scales.cpu() if scales is not None else None
    want, want_sc = dst.cpu().clone(), dst_sc.cpu().clone() if dst_sc is not None else None
    dst_ids = [19, 2, 6, 2]  # 2 repeats: the loop's later copy wins; block 4 of the snapshot is unused
    for i, b in enumerate(dst_ids):  # kv_connector.py:302-311
        want[:, :, b].copy_(blocks.cpu()[:, :, i])
        if want_sc is not None:
            want_sc[:, :, b].copy_(scales.cpu()[:, :, i])
    import_kv_blocks(dst, dst_sc, blocks, scales, dst_ids)
    torch.cuda.synchronize()
    assert torch.equal(_bytes(dst), _bytes(want))
    if want_sc is not None:
        assert torch.equal(_bytes(dst_sc), _bytes(want_sc))


def test_round_trip_and_errors(device):
    say("export/import round trip, errors")
    a, a_sc = _cache("int8", 4, 8, 128, 32, 256, device, 4)
    b, b_sc = _cache("int8", 4, 8, 128, 40, 256, device, 5)
    src_ids, dst_ids = [30, 2, 17], [0, 39, 21]
    import_kv_blocks(b, b_sc, *export_kv_blocks(a, a_sc, src_ids), dst_ids)
    torch.cuda.synchronize()
    assert torch.equal(_bytes(b[:, :, dst_ids]), _bytes(a[:, :, src_ids]))
    assert torch.equal(_bytes(b_sc[:, :, dst_ids]), _bytes(a_sc[:, :, src_ids]))
    blocks, scales = export_kv_blocks(a, a_sc, [])
    assert blocks.shape[2] == 0 and scales.shape[2] == 0
    with pytest.raises(IndexError):
        export_kv_blocks(a, a_sc, [32])
    with pytest.raises(IndexError):
        import_kv_blocks(b, b_sc, *export_kv_blocks(a, a_sc, [1]), [40])
    with pytest.raises(RuntimeError, match="no kv_scale_cache"):
        import_kv_blocks(b, None, *export_kv_blocks(a, a_sc, [1]), [3])
