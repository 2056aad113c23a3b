"""Pins the CPU oracle of the fused pre-attention step (RMSNorm + rotary
embedding, oracle/prep_oracle.py) on what the mathematics fixes: closed-form
values, exact special cases and invariants, chosen so that a plausible
slip (a missing 1/N, interleaved instead of split-half pairs, a flipped sin
sign, the weight applied after rounding) fails one of them."""
import math

import numpy as np
import pytest
import torch

from oracle import prep_oracle as PO
from oracle.kv_oracle import round_to_bf16

D = 128
BF16_ULP_REL = 2.0 ** -7  # one bf16 ulp, relative, upper bound


def _bf16(x):
    return round_to_bf16(np.asarray(x, dtype=np.float32))


@pytest.mark.parametrize("c", [0.75, -1.5, 3.0, 0.0078125])
def test_rms_norm_of_a_constant_row_is_the_weight(c):
    x = np.full((2, D), c, dtype=np.float32)
    one = np.ones(D, dtype=np.float32)
    assert np.array_equal(PO.rms_norm(x, one, 0.0), np.full((2, D), math.copysign(1.0, c), dtype=np.float32))
    w = _bf16(np.linspace(-2, 2, D))
    assert np.array_equal(PO.rms_norm(x, w, 0.0), np.broadcast_to(w * math.copysign(1.0, c), (2, D)))


def test_rms_norm_closed_form():
    # x = (3, 4): mean of squares 12.5, so x / rms = (3, 4) / sqrt(12.5).
    x = np.array([[3.0, 4.0]], dtype=np.float32)
    got = PO.rms_norm(x, np.ones(2, dtype=np.float32), 0.0)
    want = np.array([3 / math.sqrt(12.5), 4 / math.sqrt(12.5)])
    assert np.all(np.abs(got[0] - want) <= BF16_ULP_REL * np.abs(want))
    # eps sits inside the root: zero rows stay zero, tiny rows are damped.
    assert np.array_equal(PO.rms_norm(np.zeros((1, D), np.float32), np.ones(D, np.float32), 1e-6),
                          np.zeros((1, D), np.float32))
    x = np.full((1, D), 1e-4, dtype=np.float32)
    got = PO.rms_norm(x, np.ones(D, np.float32), 1e-6)
    want = 1e-4 / math.sqrt(1e-8 + 1e-6)
    assert np.all(np.abs(got - want) <= BF16_ULP_REL * want)


def test_sum_of_squares_order_is_the_blocked_tree():
    # Exact integers: any order gives the same value...
    x = np.arange(1, 129, dtype=np.float32)
    assert PO.sum_squares(x)[0] == sum(i * i for i in range(1, 129))
    # ...and here the order shows.  Squares: one 1, then 127 of 2^-24.  The
    # first group of eight starts at 1 and loses each 2^-24 (half an ulp of
    # 1, a tie rounded to even); the other fifteen groups sum exactly to
    # 2^-21 each, and the tree adds them to 1 exactly.  A sequential sum
    # would stay at 1.
    x = np.full(128, 2.0 ** -12, dtype=np.float32)
    x[0] = 1.0
    assert float(PO.sum_squares(x)[0]) == 1.0 + 15 * 2.0 ** -21


def test_rms_norm_is_scale_invariant_without_eps():
    rng = np.random.default_rng(0)
    x = _bf16(rng.standard_normal((16, D)))
    w = _bf16(1 + 0.1 * rng.standard_normal(D))
    a = PO.rms_norm(x, w, 0.0)
    for s in (0.25, 8.0):  # powers of two scale x and rms exactly
        assert np.array_equal(PO.rms_norm(x * np.float32(s), w, 0.0), a)


def test_rope_is_the_identity_at_position_zero():
    rng = np.random.default_rng(1)
    x = _bf16(rng.standard_normal((4, 3, D)))
    table = PO.cos_sin_table(D, 8, 1e6)
    assert np.array_equal(table[0, : D // 2], np.ones(D // 2)) and np.array_equal(table[0, D // 2:], np.zeros(D // 2))
    assert np.array_equal(PO.rope(x, table[0, : D // 2], table[0, D // 2:]), x)


def test_rope_quarter_turn_pairs_the_two_halves():
    # cos = 0, sin = 1 rotates every pair (x_i, x_{i+D/2}) by 90 degrees:
    # the first half becomes -x2, the second half x1, exactly.
    rng = np.random.default_rng(2)
    x = _bf16(rng.standard_normal((5, D)))
    y = PO.rope(x, np.zeros(D // 2, np.float32), np.ones(D // 2, np.float32))
    assert np.array_equal(y[:, : D // 2], -x[:, D // 2:])
    assert np.array_equal(y[:, D // 2:], x[:, : D // 2])


def test_rope_preserves_pair_norms_and_composes():
    rng = np.random.default_rng(3)
    x = _bf16(rng.standard_normal((64, D)))
    a = rng.uniform(-math.pi, math.pi, D // 2).astype(np.float32)
    b = rng.uniform(-math.pi, math.pi, D // 2).astype(np.float32)
    y = PO.rope(x, np.cos(a), np.sin(a))
    n_x = x[:, : D // 2] ** 2 + x[:, D // 2:] ** 2
    n_y = y[:, : D // 2] ** 2 + y[:, D // 2:] ** 2
    assert np.all(np.abs(n_y - n_x) <= 4 * BF16_ULP_REL * n_x + 1e-30)
    two = PO.rope(y, np.cos(b), np.sin(b))
    one = PO.rope(x, np.cos(a + b), np.sin(a + b))
    scale = np.sqrt(np.concatenate([n_x, n_x], axis=1))
    assert np.all(np.abs(two - one) <= 4 * BF16_ULP_REL * scale)


def test_cos_sin_table_matches_the_rotary_layer_formula():
    # The rotary layer's buffer (RoPE.py:40-58), computed with torch.
    D2, max_pos, base = D, 64, 1e6
    inv_freq = 1.0 / (base ** (torch.arange(0, D2, 2, dtype=torch.float) / D2))
    freqs = torch.einsum("i,j->ij", torch.arange(0, max_pos).float(), inv_freq)
    ref = torch.cat((freqs.cos(), freqs.sin()), dim=1).numpy()
    # numpy's and torch's float32 pow differ by an ulp in some frequencies,
    # which the position multiplies: 1e-5 absolute.  (The fused kernel takes
    # the table as an input; this only checks the tests' table builder.)
    assert np.allclose(PO.cos_sin_table(D2, max_pos, base), ref, rtol=0, atol=1e-5)


def test_qk_norm_rope_order_is_norm_then_rotate():
    rng = np.random.default_rng(4)
    q = _bf16(rng.standard_normal((3, 4, D)))
    k = _bf16(rng.standard_normal((3, 2, D)))
    w = _bf16(1 + 0.1 * rng.standard_normal(D))
    table = PO.cos_sin_table(D, 16, 1e6)
    pos = np.array([0, 5, 15])
    qo, ko = PO.qk_norm_rope(q, k, pos, w, w, 1e-6, table)
    for t, p in enumerate(pos):
        c, s = table[p, : D // 2], table[p, D // 2:]
        assert np.array_equal(qo[t], PO.rope(PO.rms_norm(q[t], w, 1e-6), c, s))
        assert np.array_equal(ko[t], PO.rope(PO.rms_norm(k[t], w, 1e-6), c, s))
    assert np.array_equal(qo[0], PO.rms_norm(q[0], w, 1e-6))  # position 0: norm only
