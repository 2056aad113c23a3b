"""Drop-in PagedAttention backed by hand-written gfx950 HIP kernels.

Mirrors nanovllm/layers/attention.py:PagedAttention of the reference
(nanovllm_self): same constructor, attributes the model runner binds
(model_runner.py:302-331), method names the engine and tests call, forward
semantics and error messages.  The tensor work is done by libnvs_attention.so
(include/nvs_attention.h); there is no eager fallback, so every path fails
loudly when the library or a GPU is missing.

Backends: forward_backend "flashattn" (reference default) and "hip" run
prefill_flashattn; "torch" runs prefill_torch.  Both reach the same HIP
kernels; they differ only in the guards prefill_flashattn applies
(attention.py:319-336).  Quantised caches ("int8_mock", "fp8_e4m3") are served
by both.
"""
from __future__ import annotations

import math
import os
from time import perf_counter

import torch
import torch.nn as nn

from .. import _lib
from ..utils.context import Context

_COMPUTE_DTYPES = (torch.bfloat16, torch.float16)
_SERVED_CACHE_DTYPES = (torch.bfloat16, torch.float16, torch.int8, torch.float8_e4m3fn)
_QUANT_DTYPE = {"int8_mock": torch.int8, "fp8_e4m3": torch.float8_e4m3fn}

_workspaces: dict = {}


def _need_device(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what} must be a GPU tensor for the HIP kernels (got {t.device})")


def attention_workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """Per-device split-K workspace, grown on demand (never inside graph capture).

    Calls that share it must be ordered on one stream."""
    if nbytes <= 0:
        return None
    key = torch.device(device)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError(
                "decode workspace too small inside graph capture; call "
                "reserve_attention_workspace(...) before capturing"
            )
        buf = torch.empty(nbytes, dtype=torch.uint8, device=key)
        _workspaces[key] = buf
    return buf


def reserve_attention_workspace(num_seqs: int, max_seqlen_q: int, max_seqlen_k: int, num_heads: int,
                                device, num_kv_heads: int = 0) -> None:
    """Pre-size the workspace for batches up to these bounds (for example
    before capturing a graph, where it cannot grow).  num_kv_heads = 0 sizes
    for every kv-head count (an upper bound); passing the layer's count
    reserves exactly what its calls need."""
    n = _lib.load().nvs_attention_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads,
                                                  128, 0)
    attention_workspace(torch.device(device), int(n))


def _quantize(x: torch.Tensor, code_dtype: torch.dtype):
    """[N, H, D] -> (codes [N, H, D], fp32 scales [N, H, 1])."""
    _need_device(x, "x")
    if x.dim() != 3 or x.stride(-1) != 1:
        raise RuntimeError("quantize expects [num_tokens, num_heads, head_dim] with contiguous head_dim")
    n, h, d = x.shape
    codes = torch.empty((n, h, d), dtype=code_dtype, device=x.device)
    scales = torch.empty((n, h, 1), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    _lib.check(
        lib.nvs_quantize_per_token(
            x.data_ptr(), _lib.nvs_dtype(x.dtype), x.stride(0), x.stride(1), n, h, d,
            codes.data_ptr(), _lib.nvs_dtype(code_dtype), scales.data_ptr(), _lib.stream_of(x),
        ),
        "quantize_per_token",
    )
    return codes, scales


def _dequantize(q: torch.Tensor, scale: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    _need_device(q, "q")
    q = q.contiguous()
    scale = scale.to(torch.float32).contiguous()
    d = q.shape[-1]
    h = q.shape[-2] if q.dim() >= 2 else 1
    n = q.numel() // (h * d)
    if scale.numel() != n * h:
        raise RuntimeError("scale must hold one value per (token, head)")
    out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    lib = _lib.load()
    _lib.check(
        lib.nvs_dequantize_per_token(
            q.data_ptr(), _lib.nvs_dtype(q.dtype), scale.data_ptr(), n, h, d,
            out.data_ptr(), _lib.nvs_dtype(out_dtype), _lib.stream_of(q),
        ),
        "dequantize_per_token",
    )
    return out


class PagedAttention(nn.Module):
    """Paged-KV attention layer; call it per decoder layer with the step's
    q [T, Hq, D], k, v [T, Hkv, D] and the step Context."""

    def __init__(self, num_heads, num_kv_heads, head_dim, dtype=torch.bfloat16):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.groups = num_heads // num_kv_heads if num_kv_heads > 0 else 1
        self.dtype = dtype

        self.kv_cache_dtype = torch.float16
        self.attention_compute_dtype = torch.float16
        self.decode_backend = "paged_flash"
        self.prefill_backend = "hip"

        self.kv_cache_quant_mode = "none"
        self.k_scale_cache = None
        self.v_scale_cache = None

        # Bound per layer by the model runner.
        self.k_cache = None
        self.v_cache = None
        self.block_size = None
        self.layer_id = None

        self.enable_profile = False
        self.profile_decode = dict(
            store=0.0, load=0.0, attn=0.0, gqa_expand=0.0, permute=0.0,
            qk=0.0, softmax=0.0, av=0.0, calls=0,
        )
        # No synchronisation or host timing while a graph is being captured.
        self.in_cuda_graph_capture = False

        self.kv_writer_backend = "torch"
        self.forward_backend = "flashattn"
        # Debug check of the one-call decode write's precondition (no row of
        # the batch reads another row's new-token position); it synchronises,
        # so it is off by default and never runs during graph capture.
        self.verify_decode_slots = os.environ.get("NVS_VERIFY_DECODE_SLOTS", "0") == "1"

    def _should_profile(self):
        return self.enable_profile and (not self.in_cuda_graph_capture)

    # ------------------------------------------------------------------ quant
    def quantize_int8_per_token(self, x):
        """Symmetric per-token, per-head int8: scale = max(absmax/127, 1e-6),
        q = clamp(round_half_even(x / scale), -127, 127) (attention.py:63-98)."""
        return _quantize(x, torch.int8)

    def quantize_fp8_per_token(self, x):
        """Per-token, per-head OCP e4m3: scale = max(absmax/448, 1e-6),
        q = e4m3(clamp(x / scale, -448, 448)) with round-to-nearest-even."""
        return _quantize(x, torch.float8_e4m3fn)

    def dequantize_int8_per_token(self, q, scale):
        """(q.float() * scale) rounded to attention_compute_dtype
        (attention.py:100-117); int8 or e4m3 codes."""
        return _dequantize(q, scale, self.attention_compute_dtype)

    # ------------------------------------------------------------------ store
    def write_kv_cache(self, k, v, slot_mapping):
        """KV write entry point (attention.py:120-136)."""
        if self.kv_writer_backend in ("torch", "hip"):
            return self.store_kv_cache_torch(k, v, slot_mapping)
        raise NotImplementedError(f"unknown kv writer backend: {self.kv_writer_backend}")

    def store_kv_cache_torch(self, k, v, slot_mapping):
        """Write k, v [T, Hkv, D] to the cache slots (attention.py:139-189).

        Name kept for drop-in compatibility; runs nvs_store_kvcache.  Plain
        caches receive k.to(cache dtype); quantised modes write codes and
        per-token, per-kv-head fp32 scales.  Negative slots are skipped.
        """
        kc, vc = self.k_cache, self.v_cache
        if kc is None or vc is None:
            raise RuntimeError("k_cache / v_cache are not bound")
        for t, name in ((k, "k"), (v, "v"), (kc, "k_cache"), (vc, "v_cache"), (slot_mapping, "slot_mapping")):
            _need_device(t, name)
        mode = self.kv_cache_quant_mode
        if mode in _QUANT_DTYPE:
            if kc.dtype != _QUANT_DTYPE[mode]:
                raise RuntimeError(f"{mode} KV cache must be {_QUANT_DTYPE[mode]}, got {kc.dtype}")
            if self.k_scale_cache is None or self.v_scale_cache is None:
                raise RuntimeError(f"{mode} KV cache needs k_scale_cache / v_scale_cache")
        elif mode != "none":
            raise ValueError(f"unsupported kv_cache_quant_mode: {mode}")
        elif kc.dtype in (torch.int8, torch.float8_e4m3fn):
            raise RuntimeError(f"cache dtype {kc.dtype} needs a quantised kv_cache_quant_mode")
        if k.stride(-1) != 1 or v.stride(-1) != 1:
            raise RuntimeError("k / v need a contiguous head_dim")
        if not kc.is_contiguous() or not vc.is_contiguous():
            raise RuntimeError("k_cache / v_cache must be contiguous [num_blocks, block_size, Hkv, D]")
        if slot_mapping.dtype != torch.int32:
            slot_mapping = slot_mapping.to(torch.int32)
        slot_mapping = slot_mapping.contiguous()
        if v.dtype != k.dtype:
            v = v.to(k.dtype)
        num_blocks, block_size, hkv, d = kc.shape
        ks = self.k_scale_cache if mode in _QUANT_DTYPE else None
        vs = self.v_scale_cache if mode in _QUANT_DTYPE else None
        if ks is not None and (ks.dtype != torch.float32 or not ks.is_contiguous() or not vs.is_contiguous()):
            raise RuntimeError("scale caches must be contiguous fp32 [num_blocks, block_size, Hkv, 1]")
        lib = _lib.load()
        _lib.check(
            lib.nvs_store_kvcache(
                k.data_ptr(), v.data_ptr(), _lib.nvs_dtype(k.dtype),
                k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                slot_mapping.data_ptr(), k.shape[0],
                kc.data_ptr(), vc.data_ptr(), _lib.nvs_dtype(kc.dtype),
                _lib.ptr(ks), _lib.ptr(vs),
                num_blocks, block_size, hkv, d, _lib.stream_of(k),
            ),
            "store_kvcache",
        )

    # ----------------------------------------------------------------- gather
    def get_kv_cache(self, context):
        """Visible K/V of the batch gathered to [B, max_len, Hkv, D] plus the
        validity mask (attention.py:201-285), via nvs_gather_kvcache."""
        bt = context.block_tables.to(torch.int32).contiguous()
        seq_lens = context.context_lens.to(torch.int32).contiguous()
        batch_size = bt.size(0)
        max_len = int(seq_lens.max().item())
        mode = self.kv_cache_quant_mode
        out_dtype = self.attention_compute_dtype if mode in _QUANT_DTYPE else self.k_cache.dtype
        if mode not in _QUANT_DTYPE and self.attention_compute_dtype is not None:
            out_dtype = self.attention_compute_dtype
        dev = self.k_cache.device
        k_batch = torch.empty(batch_size, max_len, self.num_kv_heads, self.head_dim, dtype=out_dtype, device=dev)
        v_batch = torch.empty_like(k_batch)
        kv_mask = torch.empty(batch_size, max_len, dtype=torch.bool, device=dev)
        kc = self.k_cache
        num_blocks, block_size = kc.shape[0], kc.shape[1]
        ks = self.k_scale_cache if mode in _QUANT_DTYPE else None
        vs = self.v_scale_cache if mode in _QUANT_DTYPE else None
        lib = _lib.load()
        _lib.check(
            lib.nvs_gather_kvcache(
                kc.data_ptr(), self.v_cache.data_ptr(), _lib.nvs_dtype(kc.dtype),
                _lib.ptr(ks), _lib.ptr(vs), bt.data_ptr(), bt.stride(0), bt.size(1),
                seq_lens.data_ptr(), batch_size, max_len, num_blocks, block_size,
                self.num_kv_heads, self.head_dim, k_batch.data_ptr(), v_batch.data_ptr(),
                _lib.nvs_dtype(out_dtype), kv_mask.data_ptr(), _lib.stream_of(kc),
            ),
            "gather_kvcache",
        )
        return k_batch, v_batch, kv_mask

    # -------------------------------------------------------------- attention
    def _attention(self, q, k, v, context, store_slots=None):
        """One call of the HIP attention over the whole (mixed) batch; with
        store_slots the same call first writes k / v to those cache slots
        (nvs_paged_attention_store, paged mode only)."""
        # The kernels compute in bf16 or fp16 (attention_compute_dtype,
        # config.py:33-38; the reference's flash path computes in it,
        # attention.py:326-336): the local mode in attention_compute_dtype,
        # the paged mode in the dtype of a bf16 / fp16 cache, and in bf16 over
        # int8 / fp8 codes.  fp32 attention (the eager path's) is refused in
        # both modes, and so are codes with fp16 compute (the reference
        # dequantises them to fp16 there; these kernels to bf16).  q / k / v
        # of another dtype are cast to the element type, as the reference
        # casts them (attention.py:340-342, 362).
        paged = context.block_tables is not None
        if self.attention_compute_dtype not in _COMPUTE_DTYPES:
            name = {torch.float32: "fp32"}.get(self.attention_compute_dtype, str(self.attention_compute_dtype))
            raise RuntimeError(
                f"HIP attention computes in bf16 or fp16: {name} attention (attention_compute_dtype "
                f"{self.attention_compute_dtype}) is not served")
        if not paged:
            compute = self.attention_compute_dtype
        elif self.k_cache is None or self.v_cache is None:
            raise RuntimeError("k_cache / v_cache are not bound")
        elif self.k_cache.dtype in (torch.bfloat16, torch.float16):
            compute = self.k_cache.dtype
        else:
            compute = torch.bfloat16
            if self.attention_compute_dtype != torch.bfloat16:
                raise RuntimeError(
                    f"HIP attention over int8 / fp8 codes computes in bf16: attention_compute_dtype "
                    f"{self.attention_compute_dtype} is not served with a {self.k_cache.dtype} cache")
        if q.dtype != compute:
            q = q.to(compute)
        _need_device(q, "q")
        if q.stride(-1) != 1:
            q = q.contiguous()
        T = q.shape[0]
        out = torch.empty(T, self.num_heads, self.head_dim, dtype=compute, device=q.device)
        cu_q = context.cu_seqlens_q.to(torch.int32).contiguous()
        cu_k = context.cu_seqlens_k.to(torch.int32).contiguous()
        B = cu_q.numel() - 1
        scale = 1.0 / math.sqrt(self.head_dim)
        lib = _lib.load()
        stream = _lib.stream_of(q)
        max_q, max_k = int(context.max_seqlen_q), int(context.max_seqlen_k)
        if (context.block_tables is not None and self.k_cache is not None
                and self.k_cache.dtype in (torch.int8, torch.float8_e4m3fn)):
            # int8 / fp8 caches: room for the bf16 copy of the prefill rows'
            # keys and values that the tile-loop prefill kernel reads.
            ws_bytes = int(lib.nvs_attention_workspace_bytes_cache(
                B, max_q, max_k, self.num_heads, self.num_kv_heads, self.head_dim, 0,
                _lib.nvs_dtype(self.k_cache.dtype)))
        else:
            ws_bytes = int(lib.nvs_attention_workspace_bytes(
                B, max_q, max_k, self.num_heads, self.num_kv_heads, self.head_dim, 0))
        ws = attention_workspace(q.device, ws_bytes)
        if context.block_tables is None:
            k = k.to(compute) if k.dtype != compute else k
            v = v.to(compute) if v.dtype != compute else v
            if k.stride(-1) != 1:
                k = k.contiguous()
            if v.stride(-1) != 1:
                v = v.contiguous()
            _lib.check(
                lib.nvs_varlen_attention_dtype(
                    q.data_ptr(), q.stride(0), q.stride(1),
                    k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
                    cu_q.data_ptr(), cu_k.data_ptr(), B, T, k.shape[0], max_q, max_k,
                    self.num_heads, self.num_kv_heads, self.head_dim, scale,
                    out.data_ptr(), out.stride(0), out.stride(1), _lib.ptr(ws), ws_bytes, stream,
                    _lib.nvs_dtype(compute),
                ),
                "varlen_attention",
            )
        else:
            kc, vc = self.k_cache, self.v_cache
            if kc.dtype not in _SERVED_CACHE_DTYPES:
                raise RuntimeError(f"HIP attention serves bf16/fp16/int8/fp8 KV caches, got {kc.dtype}")
            mode = self.kv_cache_quant_mode
            quant = kc.dtype in (torch.int8, torch.float8_e4m3fn)
            if quant and mode not in _QUANT_DTYPE:
                raise RuntimeError(f"cache dtype {kc.dtype} needs a quantised kv_cache_quant_mode")
            ks = self.k_scale_cache if quant else None
            vs = self.v_scale_cache if quant else None
            if quant and (ks is None or vs is None):
                raise RuntimeError("quantised KV cache needs k_scale_cache / v_scale_cache")
            bt = context.block_tables
            if bt.dtype != torch.int32 or not bt.is_contiguous():
                bt = bt.to(torch.int32).contiguous()
            num_blocks, block_size = kc.shape[0], kc.shape[1]
            if store_slots is None:
                _lib.check(
                    lib.nvs_paged_attention(
                        q.data_ptr(), q.stride(0), q.stride(1),
                        kc.data_ptr(), vc.data_ptr(), _lib.nvs_dtype(kc.dtype), _lib.ptr(ks), _lib.ptr(vs),
                        cu_q.data_ptr(), cu_k.data_ptr(), bt.data_ptr(), bt.size(1),
                        B, T, max_q, max_k, self.num_heads, self.num_kv_heads, self.head_dim,
                        block_size, num_blocks, scale, out.data_ptr(), out.stride(0), out.stride(1),
                        _lib.ptr(ws), ws_bytes, stream,
                    ),
                    "paged_attention",
                )
            else:
                slots = store_slots.to(torch.int32).contiguous()
                _lib.check(
                    lib.nvs_paged_attention_store(
                        q.data_ptr(), q.stride(0), q.stride(1),
                        k.data_ptr(), v.data_ptr(), _lib.nvs_dtype(k.dtype), k.stride(0), k.stride(1),
                        v.stride(0), v.stride(1), slots.data_ptr(),
                        kc.data_ptr(), vc.data_ptr(), _lib.nvs_dtype(kc.dtype), _lib.ptr(ks), _lib.ptr(vs),
                        cu_q.data_ptr(), cu_k.data_ptr(), bt.data_ptr(), bt.size(1),
                        B, T, max_q, max_k, self.num_heads, self.num_kv_heads, self.head_dim,
                        block_size, num_blocks, scale, out.data_ptr(), out.stride(0), out.stride(1),
                        _lib.ptr(ws), ws_bytes, stream,
                    ),
                    "paged_attention_store",
                )
        return out if self.dtype == compute else out.to(self.dtype)

    def prefill(self, q, k, v, context):
        """Write KV, then attend with the selected backend (attention.py:288-301)."""
        self.write_kv_cache(k, v, context.slot_mapping)
        if self.forward_backend == "torch":
            return self.prefill_torch(q, k, v, context)
        elif self.forward_backend in ("flashattn", "hip"):
            return self.prefill_flashattn(q, k, v, context)
        raise NotImplementedError(f"unknown prefill backend: {self.forward_backend}")

    def prefill_flashattn(self, q, k, v, context):
        """Unified varlen attention (attention.py:303-375): plain varlen over
        the step's k/v when block_tables is None, otherwise paged over the
        cache (prefix prefill, chunked prefill, decode, mixed batches)."""
        if self.k_cache.dtype not in (torch.float16, torch.bfloat16, torch.int8, torch.float8_e4m3fn):
            raise RuntimeError(
                f"flashattn only supports fp16/bf16 kv cache (or int8/fp8 codes), got {self.k_cache.dtype}"
            )
        if self.kv_cache_quant_mode == "none" and self.k_cache.dtype != self.attention_compute_dtype:
            raise RuntimeError(
                f"flashattn only supports the same dtype, got {self.k_cache.dtype} and "
                f"{self.attention_compute_dtype}"
            )
        return self._attention(q, k, v, context)

    def prefill_torch(self, q, k, v, context):
        """Unified-semantics attention of the eager path (attention.py:378-498):
        no prefix -> causal over the step's k/v; with block_tables -> the
        cached (dequantised) K/V with the bottom-right causal mask."""
        return self._attention(q, k, v, context)

    def _store_in_decode(self, k, v, context) -> bool:
        """True when the write of a decode batch can ride in the decode
        kernel: bf16 sources, every row a decode row, a bf16 cache (mode
        "none") or the quantised mode's code cache with fp32 scale caches,
        and neither write_kv_cache, store_kv_cache_torch nor the attention
        method forward_unified would call replaced on this layer (the
        reference's experiments wrap them per instance, and then they must
        run)."""
        cls = type(self)
        attn_fn = "prefill_torch" if self.forward_backend == "torch" else "prefill_flashattn"
        kc, vc, mode = self.k_cache, self.v_cache, self.kv_cache_quant_mode
        if kc is None or vc is None:
            return False
        if mode == "none":
            cache_ok = kc.dtype == torch.bfloat16 and vc.dtype == torch.bfloat16
        elif mode in _QUANT_DTYPE:
            ks, vs = self.k_scale_cache, self.v_scale_cache
            cache_ok = (kc.dtype == _QUANT_DTYPE[mode] and vc.dtype == _QUANT_DTYPE[mode]
                        and ks is not None and vs is not None
                        and ks.dtype == torch.float32 and vs.dtype == torch.float32
                        and ks.is_contiguous() and vs.is_contiguous())
        else:
            return False
        return (
            cache_ok
            and "write_kv_cache" not in self.__dict__ and "store_kv_cache_torch" not in self.__dict__
            and cls.write_kv_cache is PagedAttention.write_kv_cache
            and cls.store_kv_cache_torch is PagedAttention.store_kv_cache_torch
            and attn_fn not in self.__dict__ and getattr(cls, attn_fn) is getattr(PagedAttention, attn_fn)
            and self.kv_writer_backend in ("torch", "hip")
            and self.forward_backend in ("flashattn", "hip", "torch")
            and context.block_tables is not None and int(context.max_seqlen_q) == 1
            and self.attention_compute_dtype == torch.bfloat16
            and kc.is_contiguous() and vc.is_contiguous()
            and k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16 and k.is_cuda and v.is_cuda
            and k.stride(-1) == 1 and v.stride(-1) == 1
        )

    def _decode_slots_private(self, context) -> bool:
        """Host check (one synchronisation) of what the one-call decode write
        relies on beyond what the kernel checks itself: no row of the batch
        reads the position of a row's new token except that row at its own
        last position, i.e. no (row, logical block j) with block_tables[row,
        j] == slot // bs and j * bs + slot % bs < k_len, other than the
        writer's own last block.  The engine's block manager guarantees it
        (a sequence appends only into its own last block); a batch that
        breaks it takes the store kernel first."""
        bt = context.block_tables
        slots = context.slot_mapping.to(torch.int64)
        cu_k = context.cu_seqlens_k.to(torch.int64)
        klen = cu_k[1:] - cu_k[:-1]
        bs = self.k_cache.shape[1]
        B, W = bt.shape
        if B == 0 or slots.numel() == 0:
            return True
        rows = torch.arange(B, device=bt.device)
        sblk, soff = slots // bs, slots % bs                        # [T]
        own = torch.clamp(klen - 1, min=0) // bs                    # [B] each row's last logical block
        tok = torch.arange(slots.numel(), device=bt.device)
        cu_q = context.cu_seqlens_q.to(torch.int64)
        writer = torch.searchsorted(cu_q[1:], tok, right=True).clamp(max=B - 1)  # row of token t
        j = torch.arange(W, device=bt.device)
        hit = (bt.to(torch.int64)[None, :, :] == sblk[:, None, None]) & (slots >= 0)[:, None, None]
        hit &= (j[None, None, :] * bs + soff[:, None, None]) < klen[None, :, None]
        hit &= ~((rows[None, :, None] == writer[:, None, None]) & (j[None, None, :] == own[writer][:, None, None]))
        return not bool(hit.any().item())

    def forward_unified(self, q, k, v, context):
        """Write the step's K/V, then one attention call over the whole batch
        (attention.py:500-546).  A decode batch does both in one call: the
        decode kernel writes each row's new token (bf16 values, or fp8 / int8
        codes and scales) before reading its last tile."""
        should_profile = self._should_profile()
        if not should_profile and self._store_in_decode(k, v, context) and (
                not self.verify_decode_slots or self.in_cuda_graph_capture
                or self._decode_slots_private(context)):
            return self._attention(q, k, v, context, store_slots=context.slot_mapping)
        if should_profile:
            torch.cuda.synchronize()
            t0 = perf_counter()

        self.write_kv_cache(k, v, context.slot_mapping)

        if should_profile:
            torch.cuda.synchronize()
            self.profile_decode["store"] += perf_counter() - t0

        if self.forward_backend == "torch":
            fn = self.prefill_torch
        elif self.forward_backend in ("flashattn", "hip"):
            fn = self.prefill_flashattn
        else:
            raise NotImplementedError(f"unknown decode backend: {self.decode_backend}")
        if should_profile:
            torch.cuda.synchronize()
            t0 = perf_counter()
        out = fn(q, k, v, context)
        if should_profile:
            torch.cuda.synchronize()
            self.profile_decode["attn"] += perf_counter() - t0
            self.profile_decode["calls"] += 1
        return out

    def forward(self, q, k, v, context):
        return self.forward_unified(q, k, v, context)

    # ------------------------------------------------ fused pre-attention step
    def qk_norm_rope_store(self, q, k, v, positions, q_norm_weight, k_norm_weight, eps, cos_sin_cache,
                           slot_mapping, want_k=False):
        """One launch for q_norm(q), k_norm(k), rotary_embedding(positions, q, k)
        and write_kv_cache(k, v, slot_mapping) (qwen3.py:100-104, RMSNorm.py:11-18,
        RoPE.py:5-25 and 60-74, attention.py:139-189).  q [T, Hq, 128], k, v
        [T, Hkv, 128] bf16; cos_sin_cache the rotary layer's fp32 buffer
        [max_position, 1, 128]; positions outside the table are clamped.
        Returns (rotated q, rotated k or None)."""
        kc, vc = self.k_cache, self.v_cache
        if kc is None or vc is None:
            raise RuntimeError("k_cache / v_cache are not bound")
        for t, name in ((q, "q"), (k, "k"), (v, "v"), (positions, "positions"), (cos_sin_cache, "cos_sin_cache"),
                        (slot_mapping, "slot_mapping"), (kc, "k_cache")):
            _need_device(t, name)
        for t, name in ((q, "q"), (k, "k"), (v, "v")):
            if t.dtype != torch.bfloat16 or t.stride(-1) != 1:
                raise RuntimeError(f"{name} must be bf16 with a contiguous head_dim")
        mode = self.kv_cache_quant_mode
        quant = mode in _QUANT_DTYPE
        if quant and kc.dtype != _QUANT_DTYPE[mode]:
            raise RuntimeError(f"{mode} KV cache must be {_QUANT_DTYPE[mode]}, got {kc.dtype}")
        if not quant and kc.dtype in (torch.int8, torch.float8_e4m3fn):
            raise RuntimeError(f"cache dtype {kc.dtype} needs a quantised kv_cache_quant_mode")
        if not kc.is_contiguous() or not vc.is_contiguous():
            raise RuntimeError("k_cache / v_cache must be contiguous [num_blocks, block_size, Hkv, D]")
        T, Hq, D = q.shape
        Hkv = k.shape[1]
        table = cos_sin_cache.reshape(-1, D)
        if table.dtype != torch.float32 or not table.is_contiguous():
            table = table.to(torch.float32).contiguous()
        pos = positions.reshape(-1)
        if pos.dtype != torch.int64 or not pos.is_contiguous():
            pos = pos.to(torch.int64).contiguous()
        slots = slot_mapping
        if slots.dtype != torch.int32 or not slots.is_contiguous():
            slots = slots.to(torch.int32).contiguous()
        qw = q_norm_weight.to(torch.bfloat16).contiguous()
        kw = k_norm_weight.to(torch.bfloat16).contiguous()
        q_out = torch.empty(T, Hq, D, dtype=torch.bfloat16, device=q.device)
        k_out = torch.empty(T, Hkv, D, dtype=torch.bfloat16, device=q.device) if want_k else None
        ks = self.k_scale_cache if quant else None
        vs = self.v_scale_cache if quant else None
        num_blocks, block_size = kc.shape[0], kc.shape[1]
        lib = _lib.load()
        _lib.check(
            lib.nvs_qk_norm_rope_store(
                q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1),
                v.data_ptr(), v.stride(0), v.stride(1), pos.data_ptr(), T,
                qw.data_ptr(), kw.data_ptr(), float(eps), table.data_ptr(), table.shape[0],
                slots.data_ptr(), kc.data_ptr(), vc.data_ptr(), _lib.nvs_dtype(kc.dtype), _lib.ptr(ks),
                _lib.ptr(vs), num_blocks, block_size, Hq, Hkv, D,
                q_out.data_ptr(), q_out.stride(0), q_out.stride(1),
                _lib.ptr(k_out), k_out.stride(0) if want_k else 0, k_out.stride(1) if want_k else 0,
                _lib.stream_of(q),
            ),
            "qk_norm_rope_store",
        )
        return q_out, k_out

    def forward_fused(self, q, k, v, positions, q_norm_weight, k_norm_weight, eps, cos_sin_cache, context):
        """forward() for q and k before their norms and rotary embedding: the
        fused pre-attention step (which writes the cache) and then the same
        attention call forward_unified makes."""
        local = context.block_tables is None
        q_rot, k_rot = self.qk_norm_rope_store(q, k, v, positions, q_norm_weight, k_norm_weight, eps,
                                               cos_sin_cache, context.slot_mapping, want_k=local)
        if self.forward_backend == "torch":
            return self.prefill_torch(q_rot, k_rot, v, context)
        if self.forward_backend in ("flashattn", "hip"):
            return self.prefill_flashattn(q_rot, k_rot, v, context)
        raise NotImplementedError(f"unknown backend: {self.forward_backend}")

    def decode_flashattn(self, q, context):
        """Decode-only entry (attention.py:552-584): q [B, Hq, D] against the
        cache through context.block_tables / context_lens."""
        B = q.shape[0]
        dev = q.device
        lens = context.context_lens.to(torch.int32)
        cu_q = torch.arange(B + 1, dtype=torch.int32, device=dev)
        cu_k = torch.zeros(B + 1, dtype=torch.int32, device=dev)
        cu_k[1:] = torch.cumsum(lens, 0)
        ctx = Context(
            cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=1,
            max_seqlen_k=int(context.max_seqlen_k) or int(lens.max().item()),
            context_lens=lens, block_tables=context.block_tables,
        )
        return self._attention(q, None, None, ctx)

    def decode_attention_torch(self, q, k_batch, v_batch, kv_mask):
        """Decode over gathered K/V (attention.py:586-675, an entry the
        reference keeps but never calls): q [B, Hq, D], k_batch / v_batch
        [B, max_len, Hkv, D] as get_kv_cache returns them, kv_mask
        [B, max_len] True for a real key.  The kept keys are compacted
        sequence by sequence (their order is irrelevant to the softmax) and
        served by the varlen kernel, one query per sequence seeing every kept
        key; a sequence with no key returns 0."""
        B = q.shape[0]
        dev = q.device
        _need_device(q, "q")
        mask = kv_mask.to(device=dev, dtype=torch.bool)
        lens = mask.sum(dim=1, dtype=torch.int32)
        cu_q = torch.arange(B + 1, dtype=torch.int32, device=dev)
        cu_k = torch.zeros(B + 1, dtype=torch.int32, device=dev)
        cu_k[1:] = torch.cumsum(lens, 0)
        ctx = Context(
            cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=1 if B else 0,
            max_seqlen_k=int(lens.max().item()) if B else 0, context_lens=lens, block_tables=None,
        )
        return self._attention(q, k_batch[mask], v_batch[mask], ctx)


# The name the attention layer goes by in the engine's documentation.
Attention = PagedAttention
