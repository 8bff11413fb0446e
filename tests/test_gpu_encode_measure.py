"""The nested encode's measuring pass (k_enc_measure, behind
pj_encode_size_device) and the two-pass encode built on it: the size is
exactly the length of the CPU checker's output, and the bytes written at the
measured offsets (PETJSON_ENC_TWO_PASS=1) are the checker's bytes.  The
inputs cover the bytes the measuring pass has to take back: names,
category names, urls and tag names that sit in the byte columns, hold
escapes and are not written (null name, omitted category / photoUrls /
tags, tag names flagged absent)."""
import numpy as np
import pytest

import oracle_py as orc
import petjson as pj

pytestmark = pytest.mark.gpu
MODES = [pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS]


def knock_out(cols, rng, escapes=True):
    """Random null / absent flags; with escapes, escape-needing bytes strewn
    over every byte column, so that unwritten strings hold some."""
    cols.arrays["flags"] = cols["flags"] & rng.integers(0, 32, cols.n_pets, dtype=np.uint8)
    cols.arrays["status"][rng.random(cols.n_pets) < 0.2] = pj.STATUS_NULL
    cols.arrays["tag_flags"] = rng.integers(0, 4, cols["tag_flags"].shape[0], dtype=np.uint8)
    cols.arrays["cat_flags"] = rng.integers(0, 4, cols["cat_flags"].shape[0], dtype=np.uint8)
    if escapes:
        for k in ("name_bytes", "cat_name_bytes", "url_bytes", "tag_name_bytes"):
            b = cols.arrays[k]
            hit = rng.random(b.shape[0]) < 0.05
            b[hit] = rng.choice(np.array([0x22, 0x5C, 0x0A, 0x01, 0x1F, 0x08], dtype=np.uint8), int(hit.sum()))
    return cols


def run(codec, cols, fmt, incl, fields, two_pass):
    codec.set_options(incl, True, fields)
    try:
        dev = cols.to_device()
        size = codec.encode_size(dev, fmt)
        out = codec.encode(dev, fmt, two_pass=two_pass).cpu().numpy().tobytes()
    finally:
        codec.set_options()
    return size, out


@pytest.mark.parametrize("config,n", [(1, 30_000), (3, 40_000), (5, 6_000)])
@pytest.mark.parametrize("fmt", [pj.FORMAT_ARRAY, pj.FORMAT_NDJSON])
def test_measure_size_and_two_pass_match_oracle(codec, config, n, fmt):
    print(f"[measure] config={config} n={n} fmt={fmt}", flush=True)
    cols = pj.generate(config, n)
    ref = orc.encode(cols, fmt)
    for two_pass in (False, True):
        size, out = run(codec, cols, fmt, pj.INCLUDE_NON_EMPTY, None, two_pass)
        assert size == len(ref)
        assert out == ref


@pytest.mark.parametrize("seed", range(4))
def test_measure_with_unwritten_escaped_bytes(codec, seed):
    rng = np.random.default_rng(100 + seed)
    for config, n in ((1, 8_000), (3, 12_000), (5, 3_000)):
        cols = knock_out(pj.generate(config, n), rng)
        glob = int(rng.choice(MODES))
        fields = {f: int(rng.choice(MODES)) for f in pj.FIELDS if rng.random() < 0.6}
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            print(f"[measure] seed={seed} config={config} mode={glob} fields={fields} fmt={fmt}", flush=True)
            ref = orc.encode(cols, fmt, glob, True, fields)
            size, out = run(codec, cols, fmt, glob, fields, True)
            assert size == len(ref), (config, glob, fields, fmt)
            assert out == ref, (config, glob, fields, fmt)


def test_measure_absent_groups_and_edges(codec):
    """Absent column groups, one record, a record count that leaves the last
    measuring group with fewer than four blocks."""
    for n in (1, 95, 96, 97, 383, 384, 385, 1000):
        cols = pj.generate(3, n)
        ref = orc.encode(cols, pj.FORMAT_ARRAY)
        assert run(codec, cols, pj.FORMAT_ARRAY, pj.INCLUDE_NON_EMPTY, None, True) == (len(ref), ref), n
    for absent in (("category",), ("photoUrls",), ("tags",), ("category", "photoUrls", "tags")):
        cols = pj.generate(3, 5_000)
        groups = {"category": ("cat_id", "cat_flags", "cat_name_off", "cat_name_bytes"),
                  "photoUrls": ("photo_off", "url_off", "url_bytes"),
                  "tags": ("tag_off", "tag_id", "tag_flags", "tag_name_off", "tag_name_bytes")}
        for g in absent:
            for k in groups[g]:
                cols.arrays[k] = None
        if "category" in absent:
            cols.arrays["flags"] = cols["flags"] & ~np.uint8(pj.PET_HAS_CATEGORY)
        for incl in (pj.INCLUDE_NON_EMPTY, pj.INCLUDE_ALWAYS):
            ref = orc.encode(cols, pj.FORMAT_NDJSON, incl)
            assert run(codec, cols, pj.FORMAT_NDJSON, incl, None, True) == (len(ref), ref), (absent, incl)
