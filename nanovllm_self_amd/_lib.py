"""ctypes binding of libnvs_attention.so (the C ABI in include/nvs_attention.h).

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already loaded (both carry the SONAME libamdhip64.so.7): device
pointers and stream handles from torch are then valid inside the library.
There is no fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libnvs_attention.so")

NVS_DTYPE_BF16 = 0
NVS_DTYPE_FP16 = 1
NVS_DTYPE_FP32 = 2
NVS_DTYPE_INT8 = 3
NVS_DTYPE_FP8_E4M3 = 4

_TORCH_TO_NVS = {
    torch.bfloat16: NVS_DTYPE_BF16,
    torch.float16: NVS_DTYPE_FP16,
    torch.float32: NVS_DTYPE_FP32,
    torch.int8: NVS_DTYPE_INT8,
    torch.float8_e4m3fn: NVS_DTYPE_FP8_E4M3,
}

# Every exported symbol with (restype, argtypes).
_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float
SIGNATURES = {
    "nvs_last_error": (ctypes.c_char_p, []),
    "nvs_version": (_I, []),
    "nvs_store_kvcache": (
        _I,
        [_P, _P, _I, _L, _L, _L, _L, _P, _L, _P, _P, _I, _P, _P, _L, _I, _I, _I, _P],
    ),
    "nvs_quantize_per_token": (_I, [_P, _I, _L, _L, _L, _I, _I, _P, _I, _P, _P]),
    "nvs_dequantize_per_token": (_I, [_P, _I, _P, _L, _I, _I, _P, _I, _P]),
    "nvs_gather_kvcache": (
        _I,
        [_P, _P, _I, _P, _P, _P, _L, _I, _P, _I, _I, _L, _I, _I, _I, _P, _P, _I, _P, _P],
    ),
    "nvs_attention_workspace_bytes": (_L, [_I, _I, _I, _I, _I, _I, _I]),
    "nvs_attention_workspace_bytes_cache": (_L, [_I, _I, _I, _I, _I, _I, _I, _I]),
    "nvs_paged_attention": (
        _I,
        [
            _P, _L, _L,  # q
            _P, _P, _I, _P, _P,  # caches
            _P, _P, _P, _L,  # cu_q, cu_k, block_tables, bt_stride
            _I, _L, _I, _I,  # num_seqs, num_tokens, max_q, max_k
            _I, _I, _I, _I, _L,  # heads, kv heads, head_dim, block_size, num_blocks
            _F, _P, _L, _L,  # scale, out
            _P, _L, _P,  # workspace, bytes, stream
        ],
    ),
    "nvs_paged_attention_store": (
        _I,
        [
            _P, _L, _L,  # q
            _P, _P, _I, _L, _L, _L, _L, _P,  # k, v, src dtype, strides, slot_mapping
            _P, _P, _I, _P, _P,  # caches, dtype, scales
            _P, _P, _P, _L,  # cu_q, cu_k, block_tables, bt_stride
            _I, _L, _I, _I,  # num_seqs, num_tokens, max_q, max_k
            _I, _I, _I, _I, _L,  # heads, kv heads, head_dim, block_size, num_blocks
            _F, _P, _L, _L,  # scale, out
            _P, _L, _P,  # workspace, bytes, stream
        ],
    ),
    "nvs_paged_attention_store_noalloc": (
        _I,
        [
            _P, _L, _L,  # q
            _P, _P, _I, _L, _L, _L, _L, _P,  # k, v, src dtype, strides, slot_mapping
            _P, _P, _I, _P, _P,  # caches, dtype, scales
            _P, _P, _P, _L,  # cu_q, cu_k, block_tables, bt_stride
            _I, _L, _I, _I,  # num_seqs, num_tokens, max_q, max_k
            _I, _I, _I, _I, _L,  # heads, kv heads, head_dim, block_size, num_blocks
            _F, _P, _L, _L,  # scale, out
            _P,  # stream
        ],
    ),
    "nvs_qk_norm_rope_store": (
        _I,
        [
            _P, _L, _L, _P, _L, _L, _P, _L, _L,  # q, k, v
            _P, _L,  # positions, num_tokens
            _P, _P, _F,  # q_norm weight, k_norm weight, eps
            _P, _L,  # cos_sin_cache, max_position
            _P, _P, _P, _I, _P, _P, _L, _I,  # slots, caches, dtype, scales, blocks, block_size
            _I, _I, _I,  # heads, kv heads, head_dim
            _P, _L, _L, _P, _L, _L,  # q_out, k_out
            _P,  # stream
        ],
    ),
    "nvs_varlen_attention": (
        _I,
        [
            _P, _L, _L,  # q
            _P, _P, _L, _L, _L, _L,  # k, v
            _P, _P, _I, _L, _L, _I, _I,  # cu_q, cu_k, num_seqs, num_tokens, num_kv_tokens, max_q, max_k
            _I, _I, _I, _F,  # heads, kv heads, head_dim, scale
            _P, _L, _L,  # out
            _P, _L, _P,  # workspace, bytes, stream
        ],
    ),
    "nvs_varlen_attention_dtype": (
        _I,
        [
            _P, _L, _L,  # q
            _P, _P, _L, _L, _L, _L,  # k, v
            _P, _P, _I, _L, _L, _I, _I,  # cu_q, cu_k, num_seqs, num_tokens, num_kv_tokens, max_q, max_k
            _I, _I, _I, _F,  # heads, kv heads, head_dim, scale
            _P, _L, _L,  # out
            _P, _L, _P,  # workspace, bytes, stream
            _I,  # dtype of q, k, v, out
        ],
    ),
    "nvs_build_context": (
        _I,
        [
            _P, _P, _I,  # num_cached, num_new, num_seqs
            _P, _P, _L, _I, _L,  # block_offsets, block_ids, num_block_ids, block_size, num_tokens
            _P, _P, _P, _P, _P,  # cu_q, cu_k, context_lens, slot_mapping, positions
            _P, _I, _P,  # block_tables, width, stream
        ],
    ),
    "nvs_copy_blocks": (_I, [_P, _L, _P, _P, _L, _P, _L, _L, _L, _P]),
}

_lock = threading.Lock()
_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryMissing(
                    f"{LIB_PATH.name} is not built; run `python -m nanovllm_self_amd.build`"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def nvs_dtype(dt: torch.dtype) -> int:
    try:
        return _TORCH_TO_NVS[dt]
    except KeyError:
        raise RuntimeError(f"dtype {dt} is not served by the HIP kernels") from None


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().nvs_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream
