"""Pins the CPU restatement (oracle/) before it is trusted as the checker.

Each check is chosen so that a plausible mistake fails it:
* hand-written known-answer vectors, one per rule (tests/golden/*.json);
* Long.toString brute-forced against Python's int formatting;
* string escaping cross-checked against Python's json module (a library
  routine for the RFC 8259 grammar; it writes \\u00xx in lower case, so that
  case is normalised);
* decoded values cross-checked against json.loads on valid records;
* decode(encode(x)) == x on generated records of every configuration.
"""
import json
import random
import re

import numpy as np
import pytest

import oracle_py as orc
import petjson as pj
from kat_util import expected_pet, line_bytes, load, norm_pet, pet_from_dict
from model import from_columns, to_columns

INCL = {"NON_EMPTY": pj.INCLUDE_NON_EMPTY, "NON_NULL": pj.INCLUDE_NON_NULL, "ALWAYS": pj.INCLUDE_ALWAYS}


@pytest.mark.parametrize("case", load("encode_kat.json")["cases"], ids=lambda c: c["name"])
def test_encode_kat(case):
    cols = to_columns([pet_from_dict(p) for p in case["pets"]])
    fmt = {"ndjson": pj.FORMAT_NDJSON, "pretty": pj.FORMAT_PRETTY}.get(case.get("format"), pj.FORMAT_ARRAY)
    fields = {k: INCL[v] for k, v in case.get("fields", {}).items()}
    out = orc.encode(cols, fmt, INCL[case.get("inclusion", "NON_EMPTY")], case.get("hex_upper", True), fields)
    assert out == case["expected"].encode("utf-8")


@pytest.mark.parametrize("case", load("decode_kat.json")["cases"], ids=lambda c: c["name"])
def test_decode_kat(case):
    line = line_bytes(case)
    assert orc.decode_line_code(line) == case["code"]
    cols, el, ec, res = orc.decode(line + b"\n")
    assert res.n_lines == 1
    if case["code"] == 0:
        assert res.n_errors == 0 and res.n_pets == 1
        got = from_columns(cols, as_bytes=True)[0]
        assert norm_pet(got) == norm_pet(expected_pet(case))
    else:
        assert res.n_pets == 0 and list(el) == [0] and list(ec) == [case["code"]]


def _nest(depth):
    return "{\"x\":" + "[" * (depth - 1) + "]" * (depth - 1) + ",\"name\":\"a\",\"photoUrls\":[]}"


def test_depth_limit():
    # the pet object is depth 1; jackson's default limit is 1000 open containers
    assert orc.decode_line_code(_nest(1000).encode()) == pj.REC_OK
    assert orc.decode_line_code(_nest(1001).encode()) == pj.REC_DEPTH


def test_long_format_bruteforce():
    rnd = random.Random(7)
    vals = [0, 1, -1, 9, 10, -10, 2**63 - 1, -2**63, 10**18, -10**18, 999999999999999999]
    vals += [10**k for k in range(19)] + [10**k - 1 for k in range(1, 19)] + [-(10**k) for k in range(19)]
    vals += [rnd.randrange(-2**63, 2**63) for _ in range(20000)]
    vals += [rnd.randrange(0, 10**rnd.randrange(1, 19)) for _ in range(20000)]
    for v in vals:
        assert orc.format_long(v) == str(v)


def _py_escape(b: bytes) -> bytes:
    s = json.dumps(b.decode("utf-8"), ensure_ascii=False, separators=(",", ":"))
    s = re.sub(r"\\u00([0-9a-f]{2})", lambda m: "\\u00" + m.group(1).upper(), s)
    return s.encode("utf-8")


def test_escape_matches_python_json_all_bytes():
    # every single ASCII byte and a sample of UTF-8 sequences, alone and embedded
    samples = [bytes([c]) for c in range(128)] + ["é€😀ü".encode()]
    rnd = random.Random(3)
    for _ in range(300):
        samples.append(bytes(rnd.randrange(128) for _ in range(rnd.randrange(0, 40))))
    pets = [pet_from_dict({"name": s.decode(), "photoUrls": []}) for s in samples]
    out = orc.encode(to_columns(pets), pj.FORMAT_NDJSON).split(b"\n")[:-1]
    for s, line in zip(samples, out):
        assert line == b'{"name":' + _py_escape(s) + b',"photoUrls":[]}'


def _schema_check(obj):
    """Independent Python statement of the Pet binding rules on top of json.loads."""
    assert isinstance(obj, dict)
    assert isinstance(obj.get("name"), str) and isinstance(obj.get("photoUrls"), list)
    return obj


@pytest.mark.parametrize("config", [1, 3, 5])
def test_encode_is_valid_json_and_roundtrips(config):
    cols = generate_small(config)
    out = orc.encode(cols, pj.FORMAT_NDJSON)
    pets = from_columns(cols)
    lines = out.split(b"\n")[:-1]
    assert len(lines) == len(pets)
    for p, line in zip(pets, lines):
        obj = _schema_check(json.loads(line))
        assert list(obj.keys()) == [k for k in ("id", "category", "name", "photoUrls", "tags", "status")
                                    if k in obj]
        assert obj["name"] == p.name and obj.get("id") == p.id
        assert obj["photoUrls"] == p.photo_urls
        assert obj.get("status") == (None if p.status is None else p.status.value)
        if p.category is not None:
            assert obj["category"] == {"id": p.category.id, "name": p.category.name}
        assert obj.get("tags") == ([{"id": t.id, "name": t.name} for t in p.tags] if p.tags else None)
    # array framing is the NDJSON records joined by ','
    arr = orc.encode(cols, pj.FORMAT_ARRAY)
    assert arr == b"[" + b",".join(lines) + b"]"
    # decode(encode(x)) == x, column by column
    dec, el, ec, res = orc.decode(out)
    assert res.n_errors == 0 and res.n_pets == cols.n_pets
    for k in pj.COLS:
        if cols[k] is not None:
            assert np.array_equal(dec[k], cols[k]), k


def generate_small(config, n=3000):
    return pj.generate(config, n)


def test_decode_matches_json_loads_on_valid_lines():
    cols = generate_small(3, 2000)
    out = orc.encode(cols, pj.FORMAT_NDJSON)
    dec, _, _, res = orc.decode(out)
    for line, p in zip(out.split(b"\n")[:-1], from_columns(dec)):
        obj = json.loads(line)
        assert p.name == obj["name"] and p.photo_urls == obj["photoUrls"]


def test_decode_corrupted_lines_report_expected_codes():
    cols = generate_small(3, 20000)
    buf = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), np.uint8).copy()
    lines, codes = pj.corrupt_ndjson(buf, 99, 0.01)
    assert len(lines) > 100
    dec, el, ec, res = orc.decode(buf.tobytes())
    assert list(el) == list(lines) and list(ec) == list(codes)
    assert res.n_pets == cols.n_pets - len(lines)


# ------------------------------------------------ grammar differential
def _mutate(rnd, line: bytes) -> bytes:
    """One to three random byte edits biased towards JSON syntax bytes."""
    b = bytearray(line)
    for _ in range(rnd.randrange(1, 4)):
        op = rnd.randrange(4)
        pos = rnd.randrange(len(b) + 1)
        if op == 0 and b:
            b[min(pos, len(b) - 1)] = rnd.choice(b'"\\{}[],:0aeu \t\x01\xc3\xa9\xff/\r')
        elif op == 1:
            b[pos:pos] = bytes([rnd.choice(b'"\\{}[],:0-.eE \x00\x1f\x80\xe2\xf0')])
        elif op == 2 and b:
            del b[min(pos, len(b) - 1)]
        else:
            b[pos:pos] = rnd.choice([b'\\u00e9', b'\\ud83d\\ude00', b'\\ud800', b'null', b',"x":[1,{}]', b'"', b'\\',
                                     b'1.5', b'-', b'01', b'1e9', b'true', b'{}', b'[]', b'"sold"', b'"lost"'])
    return bytes(b).replace(b"\n", b" ")


class _Reject(ValueError):
    pass


def _no_constants(name):
    raise _Reject(name)


def _has_surrogate(x):
    if isinstance(x, str):
        return any(0xD800 <= ord(ch) <= 0xDFFF for ch in x)
    if isinstance(x, list):
        return any(_has_surrogate(v) for v in x)
    if isinstance(x, tuple):
        return any(_has_surrogate(v) for v in x)
    return False


def _pairs(p):
    return ("obj", p)


def _sub_code(v):
    """Category / Tag bean binding of a value json.loads produced."""
    if v is None:
        return 0
    if not (isinstance(v, tuple) and v[0] == "obj"):
        return pj.REC_TYPE
    for k, x in v[1]:
        if k == "id":
            c = _long_code(x)
        elif k == "name":
            c = 0 if x is None or isinstance(x, str) else pj.REC_TYPE
        else:
            c = 0
        if c:
            return c
    return 0


def _long_code(x):
    if x is None:
        return 0
    if isinstance(x, bool) or not isinstance(x, (int, float)):
        return pj.REC_TYPE
    if isinstance(x, float) or not (-(1 << 63) <= x < (1 << 63)):
        return pj.REC_NUMBER
    return 0


def _pet_code(obj):
    """Expected first error of a Pet line that json.loads accepted, from the
    binding rules alone: properties in line order, then the required ones."""
    if not (isinstance(obj, tuple) and obj[0] == "obj"):
        return pj.REC_TYPE
    last = {}
    for k, v in obj[1]:
        if k == "id":
            c = _long_code(v)
        elif k == "category":
            c = _sub_code(v)
        elif k == "name":
            c = 0 if v is None or isinstance(v, str) else pj.REC_TYPE
        elif k == "photoUrls":
            c = 0 if v is None or (isinstance(v, list) and all(isinstance(u, str) for u in v)) else pj.REC_TYPE
        elif k == "tags":
            if v is None:
                c = 0
            elif not isinstance(v, list):
                c = pj.REC_TYPE
            else:
                c = next((pj.REC_TYPE if t is None else _sub_code(t) for t in v
                          if t is None or _sub_code(t)), 0)
        elif k == "status":
            c = 0 if v is None else (pj.REC_TYPE if not isinstance(v, str) else
                                     (0 if v in ("available", "pending", "sold") else pj.REC_BAD_STATUS))
        else:
            c = 0
        if c:
            return c
        last[k] = v
    if last.get("name") is None:
        return pj.REC_MISSING_NAME
    if last.get("photoUrls") is None:
        return pj.REC_MISSING_PHOTOURLS
    return 0


def test_decode_grammar_differential_against_json_loads():
    """About 50k mutated Pet lines: the restatement's accept / reject
    decision agrees with Python's json module (a library routine for the
    RFC 8259 grammar), and on lines json.loads accepts its first-error code
    equals the one the bean-binding rules give from the parsed value.
    Documented differences are set aside: lines that are not strict UTF-8
    (jackson checks lead-byte classes only) and escaped lone surrogates
    (json.loads keeps them; the restatement rejects them as STRING)."""
    rnd = random.Random(20261202)
    base = orc.encode(generate_small(3, 3000), pj.FORMAT_NDJSON).split(b"\n")[:-1]
    base += orc.encode(generate_small(1, 500), pj.FORMAT_NDJSON).split(b"\n")[:-1]
    kat = [line_bytes(c) for c in load("decode_kat.json")["cases"]]
    syntaxish = {pj.REC_SYNTAX, pj.REC_STRING, pj.REC_DEPTH, pj.REC_EMPTY}
    compared = 0
    for i in range(50_000):
        line = _mutate(rnd, rnd.choice(base + kat)) if i % 10 else rnd.choice(base)
        code = orc.decode_line_code(line)
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
            assert code == _pet_code(obj), (line, code, _pet_code(obj))
        else:
            assert code != pj.REC_OK, line
    assert compared > 40_000


# --------------------------------------------------------- pretty printing
def _strip_ws_outside_strings(b: bytes) -> bytes:
    """The bytes of a JSON text with the whitespace between tokens removed."""
    out, in_str, esc = bytearray(), False, False
    for c in b:
        if in_str:
            out.append(c)
            if esc:
                esc = False
            elif c == 0x5C:
                esc = True
            elif c == 0x22:
                in_str = False
        elif c in b" \n\r\t":
            continue
        else:
            out.append(c)
            in_str = c == 0x22
    return bytes(out)


def _pretty_py(v, level=0) -> str:
    """Jackson DefaultPrettyPrinter layout of a parsed value, as a recursion
    over the value: an object's entries on new lines at two spaces per object
    level, arrays inline."""
    if isinstance(v, list):
        return "[ " + ", ".join(_pretty_py(x, level) for x in v) + " ]" if v else "[ ]"
    if isinstance(v, dict):
        if not v:
            return "{ }"
        ind = "\n" + "  " * (level + 1)
        body = ",".join(ind + json.dumps(k) + " : " + _pretty_py(x, level + 1) for k, x in v.items())
        return "{" + body + "\n" + "  " * level + "}"
    return json.dumps(v, ensure_ascii=False)


def _knock_out(cols, seed):
    rng = np.random.default_rng(seed)
    cols.arrays["flags"] = cols["flags"] & rng.integers(0, 64, cols.n_pets, dtype=np.uint8)
    cols.arrays["status"][rng.random(cols.n_pets) < 0.2] = pj.STATUS_NULL
    if cols["tag_flags"] is not None:
        cols.arrays["tag_flags"] = rng.integers(0, 4, cols["tag_flags"].shape[0], dtype=np.uint8)
    if cols["cat_flags"] is not None:
        cols.arrays["cat_flags"] = rng.integers(0, 4, cols.n_pets, dtype=np.uint8)
    return cols


@pytest.mark.parametrize("config", [1, 3, 5])
@pytest.mark.parametrize("incl", [pj.INCLUDE_NON_EMPTY, pj.INCLUDE_ALWAYS])
def test_pretty_encode_differs_from_compact_only_in_layout(config, incl):
    cols = _knock_out(generate_small(config, 2000), config)
    # lower-case hex escapes, as json.dumps writes them
    pretty = orc.encode(cols, pj.FORMAT_PRETTY, incl, False)
    compact = orc.encode(cols, pj.FORMAT_ARRAY, incl, False)
    # the same tokens, whitespace aside (escapes are written the same way)
    assert _strip_ws_outside_strings(pretty) == compact
    # the same value, and the layout a recursion over that value gives
    val = json.loads(compact)
    assert json.loads(pretty) == val
    assert pretty.decode("utf-8") == _pretty_py(val)
    # it reads back as the same records
    # (records knocked out of name or photoUrls fail there in both layouts)
    sa, a, ela, eca, ra = orc.decode_array(pretty)
    sb, b, elb, ecb, rb = orc.decode_array(compact)
    assert sa == sb == pj.PJ_OK
    assert ra.n_lines == rb.n_lines == cols.n_pets and ra.n_pets == rb.n_pets
    assert np.array_equal(ela, elb) and np.array_equal(eca, ecb)
    for k in pj.COLS:
        if b[k] is not None:
            assert np.array_equal(a[k], b[k]), k


# ----------------------------------------------------- findPetsByStatus body
def _status_code(p):
    return 3 if p.status is None else ["available", "pending", "sold"].index(p.status.value)


@pytest.mark.parametrize("config", [1, 3, 5])
def test_encode_by_status_is_encode_of_the_selected_records(config):
    """The selection restated through the object model: filter the Pet list
    by status, rebuild columns, encode those."""
    cols = generate_small(config, 1500)
    cols.arrays["status"][::7] = pj.STATUS_NULL
    pets = from_columns(cols, as_bytes=True)
    for mask in range(16):
        chosen = [p for p in pets if (mask >> _status_code(p)) & 1]
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
            got, m = orc.encode_by_status(cols, mask, fmt)
            assert m == len(chosen)
            assert got == orc.encode(to_columns(chosen), fmt), (mask, fmt)


def test_config1_digest_is_pinned():
    """the generator and the checker together reproduce
    the committed digests (tests/golden/config1_digest.json)."""
    import hashlib
    d = load("config1_digest.json")
    cols = pj.generate(1, d["records"])
    for name, fmt in (("array", pj.FORMAT_ARRAY), ("ndjson", pj.FORMAT_NDJSON), ("pretty", pj.FORMAT_PRETTY)):
        b = orc.encode(cols, fmt)
        assert len(b) == d["digests"][name]["bytes"]
        assert hashlib.sha256(b).hexdigest() == d["digests"][name]["sha256"], name
