"""Pins the CPU restatement's array-document decode (or_decode_array) before
it is trusted as the checker of pj_decode_array_*:
* known frame cases (intact or broken: leading / trailing bytes, '[' vs
  '{', blank elements, brackets and commas inside strings);
* a differential against Python's json module (a library routine for the
  RFC 8259 grammar) on random documents of Pet records and their mutations:
  a document json.loads reads as a list has an intact frame, one element
  per list item, and each element's code is the one the bean-binding rules
  give from the parsed value; a document it rejects has a broken frame or
  an invalid element;
* the same records as an array and as NDJSON decode to the same columns,
  which are the generated ones (round trip), also when re-serialised with
  indentation (newlines inside elements).
"""
import json
import random

import numpy as np
import pytest

import oracle_py as orc
import petjson as pj
from array_util import FRAME_CASES, join_array, mutate_doc, pretty, record_texts
from test_oracle import _has_surrogate, _no_constants, _pairs, _pet_code


@pytest.mark.parametrize("doc,status,n", FRAME_CASES, ids=[repr(c[0][:24]) for c in FRAME_CASES])
def test_array_frame_cases(doc, status, n):
    rc, cols, el, ec, res = orc.decode_array(doc)
    assert rc == status
    if status == pj.PJ_OK:
        assert res.n_lines == n
    # json.loads agrees on which frames hold a list (every element above is valid JSON)
    try:
        ok = isinstance(json.loads(doc), list)
    except ValueError:
        ok = False
    assert ok == (status == pj.PJ_OK)


def _same_cols(a, b):
    for k in pj.COLS:
        assert np.array_equal(a[k], b[k]), k


@pytest.mark.parametrize("config", [1, 3, 5])
def test_array_equals_ndjson_and_roundtrips(config):
    cols = pj.generate(config, 3000)
    arr = orc.encode(cols, pj.FORMAT_ARRAY)
    rc, dec, el, ec, res = orc.decode_array(arr)
    assert rc == pj.PJ_OK and res.n_errors == 0 and res.n_pets == cols.n_pets
    nd, _, _, nres = orc.decode(orc.encode(cols, pj.FORMAT_NDJSON))
    _same_cols(dec, nd)
    _same_cols(dec, cols.to_host())


def test_array_pretty_printed_equals_compact():
    rnd = random.Random(7)
    texts = record_texts(3, 400)
    compact = b"[" + b",".join(texts) + b"]"
    doc = join_array([pretty(t, rnd) for t in texts], rnd)
    assert b"\n" in doc
    rc1, a, _, _, r1 = orc.decode_array(compact)
    rc2, b, _, _, r2 = orc.decode_array(doc)
    assert rc1 == rc2 == pj.PJ_OK and r1.n_pets == r2.n_pets == 400
    _same_cols(a, b)


def test_array_differential_against_json_loads():
    rnd = random.Random(20261203)
    texts = record_texts(3, 600) + record_texts(1, 200)
    compared = 0
    for i in range(6000):
        k = rnd.randrange(0, 5)
        elems = [rnd.choice(texts) for _ in range(k)]
        if rnd.random() < 0.5:
            elems = [pretty(e, rnd) for e in elems]
        doc = join_array(elems, rnd)
        if i % 4:
            doc = mutate_doc(rnd, doc)
        rc, cols, el, ec, res = orc.decode_array(doc)
        try:
            text = doc.decode("utf-8")
        except UnicodeDecodeError:
            continue
        try:
            obj = json.loads(text, parse_constant=_no_constants, object_pairs_hook=_pairs)
            ok = True
        except (ValueError, RecursionError):
            ok = False
        if ok and (_has_surrogate(obj) or _has_surrogate(text)):
            continue
        compared += 1
        if ok and isinstance(obj, list):
            assert rc == pj.PJ_OK, doc
            assert res.n_lines == len(obj), doc
            want = [(j, _pet_code(v)) for j, v in enumerate(obj) if _pet_code(v)]
            assert [(int(a), int(b)) for a, b in zip(el, ec)] == want, doc
        elif ok:
            assert rc == pj.PJ_ERR_SYNTAX, doc          # a value, but not an array
        else:
            assert rc == pj.PJ_ERR_SYNTAX or res.n_errors > 0, doc
    assert compared > 4000
