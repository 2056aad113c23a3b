"""Exhaustive CPU check of the KV store's quantisation quotient.

The store kernel divides a bf16 / fp16 source value by the row scale with one
reciprocal per row and one FMA correction per value (csrc/store_common.h,
``quotients8``); the reference divides (nanovllm/layers/attention.py:94-98,
``x_fp32 / scale``).  ``store_quotient_check.c`` enumerates every pair
(x, absmax) of finite source values with |x| <= absmax for bf16 and fp16
sources and both code widths (int8: qmax 127, e4m3: qmax 448), and counts
pairs whose codes differ.  The arithmetic is IEEE binary32 with round to
nearest even on both sides (gcc with -ffp-contract=off; fmaf is the fused
multiply-add, as gfx950's v_fma_f32), so a zero count holds for the kernel.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "store_quotient_check.c")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not available")
    exe = str(tmp_path_factory.mktemp("sqc") / "store_quotient_check")
    subprocess.run([gcc, "-O2", "-fopenmp", "-ffp-contract=off", "-std=c99", "-o", exe, SRC, "-lm"],
                   check=True, capture_output=True, text=True)
    return exe


def _run(exe, *args):
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(8, os.cpu_count() or 1)))
    out = subprocess.run([exe, *args], check=True, capture_output=True, text=True, env=env).stdout.split()
    return {out[i]: int(out[i + 1]) for i in range(0, len(out), 2)}


def test_e4m3_encoder_against_brute_force(checker):
    # The checker's own e4m3 encoder: every bf16 value in [-448, 448] and every
    # midpoint between adjacent codes +-1 ulp against the nearest-even search.
    r = _run(checker, "encoder")
    assert r["encoder_checked"] > 30000
    assert r["encoder_errors"] == 0


# Finite non-negative bf16 values: 0x0000..0x7f7f (32640); fp16: 0x0000..0x7bff
# (31744).  Pairs with |x| <= absmax, both signs of x (+0 and -0 included):
# sum over absmax index i of 2 (i + 1) = n (n + 1).
PAIRS = {"bf16": 32640 * 32641, "fp16": 31744 * 31745}


@pytest.mark.parametrize("src", ["bf16", "fp16"])
@pytest.mark.parametrize("qmax", ["127", "448"])
def test_reciprocal_quotient_codes_equal_divide(checker, src, qmax):
    r = _run(checker, src, qmax)
    assert r["pairs"] == PAIRS[src]
    assert r["diff_codes"] == 0, r


def test_check_detects_an_uncorrected_quotient(checker):
    # Planted mistake: the quotient without its FMA correction (x * r) must
    # give different codes somewhere, or the check above proves nothing.
    assert _run(checker, "bf16", "448", "plain")["diff_codes"] > 0
    assert _run(checker, "fp16", "127", "plain")["diff_codes"] > 0
