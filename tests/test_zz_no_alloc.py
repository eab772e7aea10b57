"""tatara_op_quantise_ft_noalloc (no device allocation) against tatara_op_quantise_ft.

The allocation-free entry point keeps the LEB128 tile counts and offsets in a
static device array instead of allocating them per call.  Its output must be
byte-identical to the allocating entry point's on the same table, on
consecutive calls whose second input is smaller (the array keeps the first
call's contents), for both output formats and with and without factorizer
rows.
"""
import ctypes as C

import numpy as np
import pytest

from tatara_amd import _lib
from tatara_amd.trainer import DeviceArray, check

pytestmark = pytest.mark.gpu


def entry(name):
    return getattr(_lib.load(), name)


def quantise(name, dw, rows, cols, pi, leb128):
    n = rows * cols
    cap = max(3 * n, 1)
    dout = DeviceArray.empty(cap, np.uint8)
    nbytes = C.c_uint64()
    check(entry(name)(dw.ptr, rows, cols, pi, 127.0, int(leb128), dout.ptr, cap, C.byref(nbytes)))
    out = dout.to_host()[:nbytes.value].tobytes()
    dout.free()
    return out


@pytest.mark.parametrize("leb128", [1, 0], ids=["leb128", "raw_i16"])
def test_noalloc_matches_allocating_entry_point(gpu, leb128):
    # the LS1536 halfka-hm-merged table with its factorizer rows, then a
    # smaller table without them: the second call must not see the first's
    # tile offsets
    for rows, cols, pi, seed in ((73305, 1536, 1629, 1), (1000, 256, 0, 2), (37, 96, 5, 3)):
        rng = np.random.default_rng(seed)
        w = rng.normal(0.0, 0.3, (rows + pi) * cols).astype(np.float32)
        w[:4] = [300.0, -258.5, np.nan, 0.5 / 127]
        dw = DeviceArray(w)
        want = quantise("tatara_op_quantise_ft", dw, rows, cols, pi, leb128)
        got = quantise("tatara_op_quantise_ft_noalloc", dw, rows, cols, pi, leb128)
        dw.free()
        assert len(got) == len(want) > 0, (rows, cols, pi)
        assert got == want, (rows, cols, pi)
