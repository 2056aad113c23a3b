"""The prefill tile loop's LDS synchronisation and tile order, checked on the
CPU by running the generated program (csrc/check_prefill_lds.py) over random
batches, paged and local: no read of a K or V buffer before its fill is
waited for and a barrier passed, no fill over content another wave may
still read, and every QK^T / PV tile reads its unit's tile from one fill.
The last test plants a mistake in the generator (the V buffer never moves
on) and expects the check to catch it."""
import importlib.util
import random
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parents[1] / "nanovllm_self_amd" / "csrc"


def _checker():
    spec = importlib.util.spec_from_file_location("check_prefill_lds", CSRC / "check_prefill_lds.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@pytest.mark.parametrize("seed", [101, 202])
def test_generated_loop_lds_and_tile_order(seed):
    n, units = _checker().main(seed, 10)
    assert n == 20 and units > 0


def test_check_catches_a_buffer_that_never_moves():
    chk = _checker()
    chk.G.vb_advance = lambda em: None  # the mistake, in this copy of the generator only
    rng = random.Random(7)
    with pytest.raises(chk.Fail):
        for _ in range(10):
            chk.check_case(rng, True, slow_p=0.0)
