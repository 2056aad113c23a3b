"""CPU oracle for the KV-cache side of the attention path (numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module; only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the
checker.  Each function restates the reference (nanovllm_self,
nanovllm/layers/attention.py) step by step:

  quantize_int8_per_token  attention.py:94-98
  quantize_fp8_per_token   extension of the same recipe to OCP e4m3 (scale
                           absmax/448, same 1e-6 floor, clamp to +-448, RNE)
  dequantize_per_token     attention.py:117
  store_kvcache            attention.py:139-189
  get_kv_cache             attention.py:201-285

All floating-point steps are float32 numpy operations (IEEE, correctly
rounded division; np.rint rounds half to even like torch.round).  The e4m3
encoder is written from the format definition, independent of torch's cast;
the tests pin it against torch's float8_e4m3fn cast and against a
brute-force nearest-value search.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32

# --------------------------------------------------------------------------
# bf16 / fp16 helpers (bit-exact, RNE)
# --------------------------------------------------------------------------


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bits with round-to-nearest-even; NaN stays NaN."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


# --------------------------------------------------------------------------
# OCP float8_e4m3fn
# --------------------------------------------------------------------------


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 codes -> float32 values (exact).  1 sign, 4 exponent bits with
    bias 7, 3 mantissa bits; exponent 0 is subnormal (m * 2^-9); S.1111.111
    is NaN; there is no infinity."""
    c = codes.astype(np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3 codes, round-to-nearest-even on the 3-bit mantissa.

    |x| >= 480 (which would round past the largest finite value 448), inf and
    NaN encode as S.1111.111; values in (464, 480) round up into that code as
    well, as a non-saturating cast does.  Callers clamp to +-448 first.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    sign = ((u >> 24) & 0x80).astype(np.uint64)
    a = u & 0x7FFFFFFF
    # normal: |x| >= 2^-6 (f32 exponent >= 121)
    r = a + 0x7FFFF + ((a >> 20) & 1)
    normal = (r >> 20) - (120 << 3)
    normal = np.minimum(normal, 0x7F)
    # subnormal: m = rint(|x| * 2^9) in 0..8 (8 is the smallest normal code)
    sub = np.rint(np.abs(x).astype(np.float64) * 512.0).astype(np.uint64)
    code = np.where(a >= 0x3C800000, normal, sub)
    code = np.where(a >= 0x43F00000, 0x7F, code)
    return (sign | code).astype(np.uint8)


# --------------------------------------------------------------------------
# Per-token quantisation
# --------------------------------------------------------------------------


def _scale(x32: np.ndarray, qmax: float) -> np.ndarray:
    absmax = np.abs(x32).max(axis=-1, keepdims=True)
    scale = (absmax / F32(qmax)).astype(np.float32)
    return np.maximum(scale, F32(1e-6)).astype(np.float32)


def quantize_int8_per_token(x32: np.ndarray):
    """attention.py:94-98: absmax over head_dim, scale = clamp(absmax/127,
    min=1e-6), q = clamp(round(x / scale), -127, 127) as int8."""
    x32 = np.asarray(x32, dtype=np.float32)
    scale = _scale(x32, 127.0)
    q = np.rint((x32 / scale).astype(np.float32))
    q = np.clip(q, -127, 127).astype(np.int8)
    return q, scale


def quantize_fp8_per_token(x32: np.ndarray):
    """fp8 mode: scale = clamp(absmax/448, min=1e-6); code =
    e4m3(clamp(x / scale, -448, 448)) with round-to-nearest-even."""
    x32 = np.asarray(x32, dtype=np.float32)
    scale = _scale(x32, 448.0)
    y = np.clip((x32 / scale).astype(np.float32), F32(-448.0), F32(448.0))
    return e4m3_encode(y), scale


def dequantize_per_token(codes: np.ndarray, scale: np.ndarray, kind: str) -> np.ndarray:
    """attention.py:117 before the final cast: codes.float() * scale (fp32)."""
    vals = codes.astype(np.float32) if kind == "int8" else e4m3_decode(codes)
    return (vals * scale.astype(np.float32)).astype(np.float32)


# --------------------------------------------------------------------------
# Store and gather
# --------------------------------------------------------------------------


def store_kvcache(k32, v32, slot_mapping, k_cache, v_cache, block_size,
                  mode="none", k_scale=None, v_scale=None, cast=None):
    """attention.py:139-189 on numpy arrays (modified in place).

    k32, v32: float32 [T, Hkv, D] (the source values, exactly representable in
    the source dtype).  Caches: [NB, bs, Hkv, D]; for "none" their dtype is
    the storage representation produced by ``cast`` (float32 -> stored
    values), for "int8" int8 codes, for "fp8" uint8 codes; scales
    [NB, bs, Hkv, 1] float32.  block = slot // bs, offset = slot % bs.  Slots
    < 0 are skipped (padding), as the HIP store does.
    """
    slots = np.asarray(slot_mapping, dtype=np.int64)
    keep = slots >= 0
    slots = slots[keep]
    k32, v32 = k32[keep], v32[keep]
    blk, off = slots // block_size, slots % block_size
    if mode == "int8":
        qk, sk = quantize_int8_per_token(k32)
        qv, sv = quantize_int8_per_token(v32)
    elif mode == "fp8":
        qk, sk = quantize_fp8_per_token(k32)
        qv, sv = quantize_fp8_per_token(v32)
    else:
        k_cache[blk, off] = cast(k32)
        v_cache[blk, off] = cast(v32)
        return
    k_cache[blk, off] = qk
    v_cache[blk, off] = qv
    k_scale[blk, off] = sk
    v_scale[blk, off] = sv


def get_kv_cache(k_vals, v_vals, block_tables, context_lens):
    """attention.py:201-285 on already-dequantised float32 caches
    [NB, bs, Hkv, D].

    For sequence i: valid = row[row != -1]; tokens = cache[valid] flattened
    and cut to context_lens[i]; rows past that stay zero; the mask is True on
    gathered positions.  Returns (k_batch, v_batch, kv_mask).
    """
    bt = np.asarray(block_tables)
    lens = np.asarray(context_lens, dtype=np.int64)
    B = bt.shape[0]
    max_len = int(lens.max())
    nb, bs, h, d = k_vals.shape
    kb = np.zeros((B, max_len, h, d), dtype=np.float32)
    vb = np.zeros_like(kb)
    mask = np.zeros((B, max_len), dtype=bool)
    for i in range(B):
        row = bt[i]
        valid = row[row != -1]
        if valid.size == 0:
            continue
        n = int(lens[i])
        sk = k_vals[valid].reshape(-1, h, d)[:n]
        sv = v_vals[valid].reshape(-1, h, d)[:n]
        kb[i, : sk.shape[0]] = sk
        vb[i, : sv.shape[0]] = sv
        mask[i, : sk.shape[0]] = True
    return kb, vb, mask
