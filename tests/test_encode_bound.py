"""pj_encode_bound (host only, no device) is never below the exact encoded
size the CPU restatement gives: generated records of every configuration,
and random columns with every presence bit, extreme ids and strings full of
bytes that need six-byte escapes, under every inclusion mode and framing."""
import numpy as np
import pytest

import oracle_py as orc
import petjson as pj
from test_gpu_fuzz import random_columns


def bound(cols, fmt):
    import ctypes as C
    L = pj.load_lib()
    s = cols.struct()
    b = C.c_uint64(0)
    assert L.pj_encode_bound(C.byref(s), fmt, C.byref(b)) == pj.PJ_OK
    return b.value


@pytest.mark.parametrize("config", [1, 2, 3, 5])
def test_bound_covers_generated(config):
    cols = pj.generate(config, 2000)
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
        for incl in (pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS):
            assert bound(cols, fmt) >= len(orc.encode(cols, fmt, incl))


def test_bound_covers_random_and_escape_heavy():
    rng = np.random.default_rng(3)
    for _ in range(60):
        cols = random_columns(rng, int(rng.integers(0, 300)))
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
            for incl in (pj.INCLUDE_NON_EMPTY, pj.INCLUDE_ALWAYS):
                assert bound(cols, fmt) >= len(orc.encode(cols, fmt, incl, False))
    # every string byte a control character: each becomes \u00XX
    cols = pj.generate(3, 500)
    for k in ("name_bytes", "cat_name_bytes", "url_bytes", "tag_name_bytes"):
        cols.arrays[k][:] = 1
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_PRETTY):
        assert bound(cols, fmt) >= len(orc.encode(cols, fmt, pj.INCLUDE_ALWAYS))
