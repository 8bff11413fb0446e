"""Array documents for the array-decode tests: known frame cases, random
documents made of (possibly mutated) Pet records with varied whitespace,
and byte mutations of whole documents."""
import json
import random

import oracle_py as orc
import petjson as pj

# (document, expected status, expected element count when the frame is intact)
FRAME_CASES = [
    (b"[]", pj.PJ_OK, 0),
    (b" \t\r\n[ \n ]\r\n ", pj.PJ_OK, 0),
    (b'[{"name":"a","photoUrls":[]}]', pj.PJ_OK, 1),
    (b'[1,"x",null,true,{},[],[1,[2,{"a":[3]}]]]', pj.PJ_OK, 7),
    (b'["a,b","[","]","{","}","\\"",",\\\\"]', pj.PJ_OK, 7),
    (b'[ {"name":"x\\"]","photoUrls":["a,b"]} ,\n\t{"name":"y","photoUrls":[]} ]', pj.PJ_OK, 2),
    (b"", pj.PJ_ERR_SYNTAX, 0),
    (b"   ", pj.PJ_ERR_SYNTAX, 0),
    (b"[", pj.PJ_ERR_SYNTAX, 0),
    (b"[1", pj.PJ_ERR_SYNTAX, 0),
    (b"]", pj.PJ_ERR_SYNTAX, 0),
    (b"[]]", pj.PJ_ERR_SYNTAX, 0),
    (b"[}", pj.PJ_ERR_SYNTAX, 0),
    (b"[1}", pj.PJ_ERR_SYNTAX, 0),
    (b"[,]", pj.PJ_ERR_SYNTAX, 0),
    (b"[1,]", pj.PJ_ERR_SYNTAX, 0),
    (b"[,1]", pj.PJ_ERR_SYNTAX, 0),
    (b"[1,,2]", pj.PJ_ERR_SYNTAX, 0),
    (b"[1, \n ,2]", pj.PJ_ERR_SYNTAX, 0),
    (b"x[]", pj.PJ_ERR_SYNTAX, 0),
    (b"[]x", pj.PJ_ERR_SYNTAX, 0),
    (b"[] []", pj.PJ_ERR_SYNTAX, 0),
    (b'{"name":"a","photoUrls":[]}', pj.PJ_ERR_SYNTAX, 0),
    (b'"[1]"', pj.PJ_ERR_SYNTAX, 0),
    (b'["]', pj.PJ_ERR_SYNTAX, 0),
    (b'[{"a":"}]', pj.PJ_ERR_SYNTAX, 0),
]


def record_texts(config, n, seed=None):
    """Compact JSON texts of n generated records (the encoder's NDJSON lines)."""
    return orc.encode(pj.generate(config, n, seed=seed), pj.FORMAT_NDJSON).split(b"\n")[:-1]


def pretty(text: bytes, rnd: random.Random) -> bytes:
    """The same value re-serialised with random indentation and spacing."""
    obj = json.loads(text)
    indent = rnd.choice([None, 0, 1, 2, "\t"])
    seps = rnd.choice([(",", ":"), (", ", ": "), (" ,", " : ")])
    return json.dumps(obj, indent=indent, separators=seps, ensure_ascii=rnd.random() < 0.5).encode("utf-8")


def join_array(elems, rnd: random.Random) -> bytes:
    """'[' + elements separated by commas with random whitespace + ']'."""
    ws = [b"", b" ", b"\n", b"\r\n  ", b"\t"]
    out = [rnd.choice(ws), b"["]
    for i, e in enumerate(elems):
        if i:
            out.append(b",")
        out += [rnd.choice(ws), e, rnd.choice(ws)]
    out += [b"]", rnd.choice(ws)]
    return b"".join(out)


def mutate_doc(rnd: random.Random, doc: bytes) -> bytes:
    """One to three random byte edits biased towards JSON syntax bytes."""
    b = bytearray(doc)
    for _ in range(rnd.randrange(1, 4)):
        op = rnd.randrange(4)
        pos = rnd.randrange(len(b) + 1)
        if op == 0 and b:
            b[min(pos, len(b) - 1)] = rnd.choice(b'"\\{}[],:0aeu \t\n\x01\xc3\xa9\xff/\r')
        elif op == 1:
            b[pos:pos] = bytes([rnd.choice(b'"\\{}[],:0-.eE \n\x00\x1f\x80\xe2\xf0')])
        elif op == 2 and b:
            del b[min(pos, len(b) - 1)]
        else:
            b[pos:pos] = rnd.choice([b'\\u00e9', b'\\ud800', b'null', b',"x":[1,{}]', b'"', b'\\', b',', b'[]',
                                     b'{}', b'"sold"', b',{}', b'],[', b'\\\\'])
    return bytes(b)
