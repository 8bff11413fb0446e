"""The CPU restatement of the Order and User models, pinned: hand-written
known answers (tests/golden/model_kat.json), the encoder against json.dumps
on random records, decode(encode(x)) == x in every framing, and the decoder's
accept / reject decisions and first-error codes against json.loads plus the
binding rules on mutated lines."""
import json
import random

import numpy as np
import pytest

import oracle_py as orc
import petjson as pj
from kat_util import load
from model_util import MODELS, from_model_columns, to_model_columns

INCL = {"NON_EMPTY": pj.INCLUDE_NON_EMPTY, "NON_NULL": pj.INCLUDE_NON_NULL, "ALWAYS": pj.INCLUDE_ALWAYS}
FMT = {"array": pj.FORMAT_ARRAY, "ndjson": pj.FORMAT_NDJSON, "pretty": pj.FORMAT_PRETTY}
KAT = load("model_kat.json")


@pytest.mark.parametrize("case", KAT["encode"], ids=lambda c: c["name"])
def test_model_encode_kat(case):
    cols = to_model_columns(MODELS[case["model"]], case["records"])
    out = orc.encode_model(cols, FMT[case.get("format", "array")], INCL[case.get("inclusion", "NON_EMPTY")])
    assert out == case["expected"].encode("utf-8")


@pytest.mark.parametrize("case", KAT["decode"], ids=lambda c: c["name"])
def test_model_decode_kat(case):
    model = MODELS[case["model"]]
    rc, cols, el, ec, res = orc.decode_model(model, case["line"].encode("utf-8") + b"\n")
    assert rc == pj.PJ_OK and res.n_lines == 1
    if case["code"] == 0:
        assert res.n_errors == 0 and res.n_pets == 1
        assert from_model_columns(cols) == [case["record"]]
    else:
        assert res.n_pets == 0 and list(el) == [0] and list(ec) == [case["code"]]


def _py_record(model, rec, incl):
    """The record as json.dumps would lay it out under the inclusion rules."""
    d = {}
    for name, kind in pj.MODEL_PROPS[model]:
        v = rec.get(name)
        if v is None:
            if incl == pj.INCLUDE_ALWAYS:
                d[name] = None
            continue
        if kind == "str" and v == "" and incl == pj.INCLUDE_NON_EMPTY:
            continue
        d[name] = v
    return d


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
@pytest.mark.parametrize("incl", [pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS])
def test_model_encode_matches_json_dumps(model, incl):
    cols = pj.generate_model(model, 3000, seed=model * 10 + incl, null_rate=0.2)
    # empty strings, too
    for k, (_, kind) in enumerate(cols.props):
        if kind == "str":
            lens = np.diff(cols.col[k].astype(np.int64))
            assert (lens == 0).any()
    recs = from_model_columns(cols)
    got = orc.encode_model(cols, pj.FORMAT_NDJSON, incl, hex_upper=False)
    want = "".join(json.dumps(_py_record(model, r, incl), ensure_ascii=False, separators=(",", ":")) + "\n"
                   for r in recs).encode("utf-8")
    assert got == want


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
@pytest.mark.parametrize("fmt", [pj.FORMAT_NDJSON, pj.FORMAT_ARRAY, pj.FORMAT_PRETTY])
def test_model_roundtrip(model, fmt):
    cols = pj.generate_model(model, 2000, seed=fmt, null_rate=0.2)
    text = orc.encode_model(cols, fmt, pj.INCLUDE_ALWAYS)
    rc, dec, el, ec, res = orc.decode_model(model, text, array=fmt != pj.FORMAT_NDJSON)
    assert rc == pj.PJ_OK and res.n_errors == 0 and res.n_pets == cols.n
    assert from_model_columns(dec) == from_model_columns(cols)
    assert np.array_equal(dec.present, cols.present)


class _Reject(ValueError):
    pass


def _no_constants(name):
    raise _Reject(name)


def _pairs(p):
    return ("obj", p)


def _has_surrogate(x):
    if isinstance(x, str):
        return any(0xD800 <= ord(ch) <= 0xDFFF for ch in x)
    if isinstance(x, (list, tuple)):
        return any(_has_surrogate(v) for v in x)
    return False


def _model_code(model, obj):
    """First error of a line json.loads accepted, from the binding rules."""
    if not (isinstance(obj, tuple) and obj[0] == "obj"):
        return pj.REC_TYPE
    kinds = dict(pj.MODEL_PROPS[model])
    for k, v in obj[1]:
        kind = kinds.get(k)
        if kind is None or v is None:
            continue
        if kind in ("i64", "i32"):
            if isinstance(v, bool) or not isinstance(v, (int, float)):
                return pj.REC_TYPE
            lim = 63 if kind == "i64" else 31
            if isinstance(v, float) or not (-(1 << lim) <= v < (1 << lim)):
                return pj.REC_NUMBER
        elif kind == "str":
            if not isinstance(v, str):
                return pj.REC_TYPE
        elif kind == "enum":
            if not isinstance(v, str):
                return pj.REC_TYPE
            if v not in pj.ORDER_STATUS:
                return pj.REC_BAD_STATUS
        elif not isinstance(v, bool):
            return pj.REC_TYPE
    return 0


def _mutate(rnd, line: bytes) -> bytes:
    b = bytearray(line)
    for _ in range(rnd.randrange(1, 4)):
        op = rnd.randrange(4)
        pos = rnd.randrange(len(b) + 1)
        if op == 0 and b:
            b[min(pos, len(b) - 1)] = rnd.choice(b'"\\{}[],:0aeu \t\x01\xc3\xa9/\r')
        elif op == 1:
            b[pos:pos] = bytes([rnd.choice(b'"\\{}[],:0-.eE \x00\x1f')])
        elif op == 2 and b:
            del b[min(pos, len(b) - 1)]
        else:
            b[pos:pos] = rnd.choice([b'\\u00e9', b'\\ud800', b'null', b',"x":[1,{}]', b'"', b'1.5', b'-', b'01',
                                     b'1e9', b'true', b'false', b'{}', b'[]', b'"placed"', b'"lost"',
                                     b'2147483648', b'-2147483649', b'9223372036854775808'])
    return bytes(b).replace(b"\n", b" ")


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
def test_model_decode_differential_against_json_loads(model):
    rnd = random.Random(model)
    cols = pj.generate_model(model, 2000, seed=5, null_rate=0.2)
    base = orc.encode_model(cols, pj.FORMAT_NDJSON, pj.INCLUDE_ALWAYS).split(b"\n")[:-1]
    lines = [rnd.choice(base) if i % 10 == 0 else _mutate(rnd, rnd.choice(base)) for i in range(12_000)]
    rc, _, el, ec, res = orc.decode_model(model, b"\n".join(lines) + b"\n")
    assert rc == pj.PJ_OK and res.n_lines == len(lines)
    codes = np.zeros(len(lines), np.uint8)
    codes[el.astype(np.int64)] = ec
    syntaxish = {pj.REC_SYNTAX, pj.REC_STRING, pj.REC_DEPTH, pj.REC_EMPTY}
    compared = 0
    for line, code in zip(lines, codes):
        try:
            text = line.decode("utf-8")
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
        if ok:
            assert code not in syntaxish, (line, code)
            assert code == _model_code(model, obj), (line, code)
        else:
            assert code != pj.REC_OK, line
    assert compared > 10_000
