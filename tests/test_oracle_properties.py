"""Property tests (Hypothesis) of the CPU restatement on arbitrary records:
- decode(encode(x)) == x column for column, in every framing (under ALWAYS,
  so that nulls and empties survive the trip);
- encode(decode(y)) == y for the canonical text y the encoder writes, under
  each inclusion mode;
- the text is the value json.loads reads back, property for property, in
  schema order.
The strings are arbitrary Unicode (surrogates excluded: the Java side would
write them as pairs of a valid code point), the ids span int64."""
import json

import numpy as np
import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle_py as orc
import petjson as pj
from model import Category, Pet, StatusEnum, Tag, from_columns, to_columns

TEXT = st.text(alphabet=st.characters(blacklist_categories=("Cs",)), max_size=24)
I64 = st.integers(min_value=-(1 << 63), max_value=(1 << 63) - 1)
SUB = st.builds(Category, id=st.none() | I64, name=st.none() | TEXT)
TAG = st.builds(Tag, id=st.none() | I64, name=st.none() | TEXT)
PET = st.builds(Pet, name=TEXT, photo_urls=st.lists(TEXT, max_size=4), id=st.none() | I64,
                category=st.none() | SUB, tags=st.none() | st.lists(TAG, max_size=4),
                status=st.none() | st.sampled_from(list(StatusEnum)))
PETS = st.lists(PET, max_size=12)
SETTINGS = settings(max_examples=300, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.too_slow])


def _decode(text: bytes, fmt):
    if fmt == pj.FORMAT_NDJSON:
        cols, _, _, res = orc.decode(text)
        return pj.PJ_OK, cols, res
    rc, cols, _, _, res = orc.decode_array(text)
    return rc, cols, res


@SETTINGS
@given(PETS, st.sampled_from([pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY]))
def test_decode_of_encode_is_identity(pets, fmt):
    cols = to_columns(pets)
    text = orc.encode(cols, fmt, pj.INCLUDE_ALWAYS)
    rc, back, res = _decode(text, fmt)
    assert rc == pj.PJ_OK and res.n_errors == 0 and res.n_pets == len(pets)
    for k in pj.COLS:
        if back[k] is not None and cols[k] is not None:
            assert np.array_equal(back[k], cols[k]), k


@SETTINGS
@given(PETS, st.sampled_from([pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS]))
def test_encode_of_decode_is_identity_on_canonical_text(pets, incl):
    text = orc.encode(to_columns(pets), pj.FORMAT_NDJSON, incl)
    cols, _, _, res = orc.decode(text)
    assert res.n_errors == 0
    assert orc.encode(cols, pj.FORMAT_NDJSON, incl) == text


def _expected(p: Pet):
    """The Pet as a dict in schema order under NON_EMPTY."""
    d = {}
    if p.id is not None:
        d["id"] = p.id
    if p.category is not None:
        c = {}
        if p.category.id is not None:
            c["id"] = p.category.id
        if p.category.name:
            c["name"] = p.category.name
        d["category"] = c
    d["name"] = p.name
    d["photoUrls"] = list(p.photo_urls)
    if p.tags:
        d["tags"] = [{**({"id": t.id} if t.id is not None else {}), **({"name": t.name} if t.name else {})}
                     for t in p.tags]
    if p.status is not None:
        d["status"] = p.status.value
    return d


@SETTINGS
@given(PETS)
def test_text_is_the_value_json_loads_reads(pets):
    text = orc.encode(to_columns(pets), pj.FORMAT_ARRAY, pj.INCLUDE_NON_EMPTY, hex_upper=False)
    got = json.loads(text, object_pairs_hook=lambda kv: ("obj", kv))
    want = [_expected(p) for p in pets]

    def plain(v):      # objects back to dicts, keeping the order they were read in
        if isinstance(v, tuple) and v[0] == "obj":
            return {k: plain(x) for k, x in v[1]}
        return [plain(x) for x in v] if isinstance(v, list) else v

    assert [plain(o) for o in got] == want
    # and in schema order
    assert [[k for k, _ in o[1]] for o in got] == [list(w.keys()) for w in want]
