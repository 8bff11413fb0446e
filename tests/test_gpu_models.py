"""GPU parity of the Order and User models: pj_encode_model_device output is
byte-identical to the CPU restatement, and pj_decode_model_device gives the
restatement's columns, error indices and codes, on the hand-written vectors,
seeded random records in every framing and inclusion mode, and mutated
lines."""
import random

import numpy as np
import pytest
import torch

import oracle_py as orc
import petjson as pj
from kat_util import load
from model_util import MODELS, from_model_columns, to_model_columns
from test_oracle_models import _mutate

pytestmark = pytest.mark.gpu
INCL = {"NON_EMPTY": pj.INCLUDE_NON_EMPTY, "NON_NULL": pj.INCLUDE_NON_NULL, "ALWAYS": pj.INCLUDE_ALWAYS}
FMT = {"array": pj.FORMAT_ARRAY, "ndjson": pj.FORMAT_NDJSON, "pretty": pj.FORMAT_PRETTY}
KAT = load("model_kat.json")


def gpu_encode(codec, cols, fmt, incl=pj.INCLUDE_NON_EMPTY, hex_upper=True):
    codec.set_options(incl, hex_upper)
    try:
        return codec.encode_model(cols.to_device(), fmt).cpu().numpy().tobytes()
    finally:
        codec.set_options()


def gpu_decode(codec, model, data: bytes, array=False):
    t = torch.from_numpy(np.frombuffer(data, np.uint8).copy() if data else np.zeros(0, np.uint8)).cuda()
    cols, el, ec, res = codec.decode_model(model, t, array=array)
    return cols.to_host(), el.cpu().numpy().astype(np.uint64), ec.cpu().numpy(), res


def same_decode(codec, model, data, array=False):
    rc, rcols, rel, rec, rres = orc.decode_model(model, data, array)
    assert rc == pj.PJ_OK
    gcols, gel, gec, gres = gpu_decode(codec, model, data, array)
    assert (gres.n_lines, gres.n_pets, gres.n_errors) == (rres.n_lines, rres.n_pets, rres.n_errors)
    assert np.array_equal(gel, rel) and np.array_equal(gec, rec)
    assert gcols.n == rcols.n
    assert np.array_equal(gcols.present, rcols.present)
    for k, (_, kind) in enumerate(gcols.props):
        assert np.array_equal(gcols.col[k], rcols.col[k]), k
        if kind == "str":
            assert np.array_equal(gcols.bytes[k], rcols.bytes[k]), k
    return gres


@pytest.mark.parametrize("case", KAT["encode"], ids=lambda c: c["name"])
def test_model_encode_kat_gpu(codec, case):
    cols = to_model_columns(MODELS[case["model"]], case["records"])
    got = gpu_encode(codec, cols, FMT[case.get("format", "array")], INCL[case.get("inclusion", "NON_EMPTY")])
    assert got == case["expected"].encode("utf-8")


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
@pytest.mark.parametrize("fmt", [pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY])
def test_model_encode_matches_oracle(codec, model, fmt):
    print(f"[model encode] model={model} fmt={fmt}", flush=True)
    cols = pj.generate_model(model, 200_000, seed=fmt, null_rate=0.15)
    for incl in (pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS):
        for hx in (True, False):
            assert gpu_encode(codec, cols, fmt, incl, hx) == orc.encode_model(cols, fmt, incl, hx), (incl, hx)


def test_model_encode_capacity_and_empty(codec):
    for model in (pj.MODEL_ORDER, pj.MODEL_USER):
        empty = to_model_columns(model, [])
        assert gpu_encode(codec, empty, pj.FORMAT_ARRAY) == b"[]"
        assert gpu_encode(codec, empty, pj.FORMAT_PRETTY) == b"[ ]"
        assert gpu_encode(codec, empty, pj.FORMAT_NDJSON) == b""
    cols = pj.generate_model(pj.MODEL_USER, 20_000, seed=3)
    ref = np.frombuffer(orc.encode_model(cols, pj.FORMAT_ARRAY), np.uint8)
    out = torch.full((ref.size,), 0xEE, dtype=torch.uint8, device="cuda")
    cap = ref.size // 2
    with pytest.raises(pj.PetJsonError) as ei:
        codec.encode_model(cols.to_device(), pj.FORMAT_ARRAY, out=out[:cap])
    assert ei.value.status == pj.PJ_ERR_CAPACITY
    host = out.cpu().numpy()
    assert (host[cap:] == 0xEE).all()
    written = host[:cap] != 0xEE
    assert (host[:cap][written] == ref[:cap][written]).all()


@pytest.mark.parametrize("model", ["order", "user"])
def test_model_decode_kat_gpu(codec, model):
    cases = [c for c in KAT["decode"] if c["model"] == model]
    data = b"".join(c["line"].encode("utf-8") + b"\n" for c in cases)
    same_decode(codec, MODELS[model], data)
    cols, el, ec, res = gpu_decode(codec, MODELS[model], data)
    want_codes = [c["code"] for c in cases]
    got = [0] * len(cases)
    for i, c in zip(el, ec):
        got[int(i)] = int(c)
    assert got == want_codes
    assert from_model_columns(cols) == [c["record"] for c in cases if c["code"] == 0]


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
@pytest.mark.parametrize("fmt", [pj.FORMAT_NDJSON, pj.FORMAT_ARRAY, pj.FORMAT_PRETTY])
def test_model_decode_roundtrip_matches_oracle(codec, model, fmt):
    print(f"[model decode] model={model} fmt={fmt}", flush=True)
    cols = pj.generate_model(model, 150_000, seed=10 + fmt, null_rate=0.15)
    data = orc.encode_model(cols, fmt, pj.INCLUDE_ALWAYS)
    res = same_decode(codec, model, data, array=fmt != pj.FORMAT_NDJSON)
    assert res.n_errors == 0 and res.n_pets == cols.n


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
def test_model_decode_mutated_lines_match_oracle(codec, model):
    rnd = random.Random(100 + model)
    cols = pj.generate_model(model, 3000, seed=7, null_rate=0.2)
    base = orc.encode_model(cols, pj.FORMAT_NDJSON, pj.INCLUDE_ALWAYS).split(b"\n")[:-1]
    lines = [rnd.choice(base) if i % 5 == 0 else _mutate(rnd, rnd.choice(base)) for i in range(30_000)]
    # deep unknown values, blank lines and a final line without '\n'
    lines += [b'{"x":' + b"[" * 999 + b"]" * 999 + b',"id":1}', b'{"x":' + b"[" * 1000 + b"]" * 1000 + b"}",
              b"", b"  ", b'{"id":2}']
    res = same_decode(codec, model, b"\n".join(lines))
    assert res.n_errors > 1000 and res.n_pets > 5000


def test_model_decode_array_frames(codec):
    for model in (pj.MODEL_ORDER, pj.MODEL_USER):
        for doc in (b"[]", b" [ ] ", b'[{"id":1}]', b'[ {"id":1} , {} ,{"id":"x"}]'):
            same_decode(codec, model, doc, array=True)
        t = torch.from_numpy(np.frombuffer(b'[{"id":1},,{}]', np.uint8).copy()).cuda()
        with pytest.raises(pj.PetJsonError) as ei:
            codec.decode_model(model, t, array=True)
        assert ei.value.status == pj.PJ_ERR_SYNTAX


def test_model_decode_capacity(codec):
    cols = pj.generate_model(pj.MODEL_USER, 5000, seed=9)
    data = orc.encode_model(cols, pj.FORMAT_NDJSON, pj.INCLUDE_ALWAYS)
    t = torch.from_numpy(np.frombuffer(data, np.uint8).copy()).cuda()
    cap_n, cap_b = pj.decode_model_bounds(pj.MODEL_USER, len(data))
    cap_b = list(cap_b)
    cap_b[1] = 100                                  # username bytes
    with pytest.raises(pj.PetJsonError) as ei:
        codec.decode_model(pj.MODEL_USER, t, caps=(cap_n, cap_b))
    assert ei.value.status == pj.PJ_ERR_CAPACITY
    with pytest.raises(pj.PetJsonError) as ei:
        codec.decode_model(pj.MODEL_USER, t, caps=(100, cap_b))
    assert ei.value.status == pj.PJ_ERR_CAPACITY


@pytest.mark.parametrize("model", [pj.MODEL_ORDER, pj.MODEL_USER])
def test_model_host_entry_points_match_oracle(codec, model):
    """pj_encode_model_host / pj_decode_model_host: host columns and text,
    the device work staged by the library."""
    cols = pj.generate_model(model, 50_000, seed=21, null_rate=0.2)
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
        assert codec.encode_model_host(cols, fmt) == orc.encode_model(cols, fmt), fmt
    rnd = random.Random(model)
    lines = orc.encode_model(cols, pj.FORMAT_NDJSON).split(b"\n")[:-1]
    lines = [_mutate(rnd, x) if i % 7 == 0 else x for i, x in enumerate(lines)]
    data = b"\n".join(lines) + b"\n"
    rc, rcols, rel, rec, rres = orc.decode_model(model, data)
    gcols, gel, gec, gres = codec.decode_model_host(model, data)
    assert (gres.n_lines, gres.n_pets, gres.n_errors) == (rres.n_lines, rres.n_pets, rres.n_errors)
    assert np.array_equal(gel, rel) and np.array_equal(gec, rec)
    assert from_model_columns(gcols) == from_model_columns(rcols)
    assert np.array_equal(gcols.present, rcols.present)
    # too small a string capacity: the sizes needed come back with the error
    cap_n, cap_b = pj.decode_model_bounds(model, len(data))
    k = next(k for k, (_, kind) in enumerate(pj.MODEL_PROPS[model]) if kind == "str")
    cap_b = list(cap_b)
    cap_b[k] = 10
    with pytest.raises(pj.PetJsonError) as ei:
        codec.decode_model_host(model, data, caps=(cap_n, cap_b))
    assert ei.value.status == pj.PJ_ERR_CAPACITY


@pytest.mark.parametrize("tape", ["1", "0"])
def test_model_decode_tape_and_reparse_match_oracle(codec, monkeypatch, tape):
    """The writing pass takes each record's code, values and string positions
    from the counting pass's tape, copying escape-free strings raw and
    decoding the others again; with PETJSON_DECODE_TAPE=0 it reads every
    record again.  Both against the oracle: duplicate properties whose last
    occurrence has or lacks escapes, escapes of every kind, multi-byte UTF-8
    and mutated lines."""
    monkeypatch.setenv("PETJSON_DECODE_TAPE", tape)
    user = [b'{"username":"a\\nb","username":"plain","id":1}',
            b'{"username":"plain","username":"a\\u00e9b\\"c\\\\d\\/e","id":2}',
            b'{"email":"x\\/y","phone":"\\ud83d\\ude00 \xc3\xa9\xe2\x82\xac","password":"p\\tq\\r\\b\\f"}',
            b'{"firstName":"' + b"z" * 300 + b'\\n","lastName":"' + b"y" * 301 + b'","userStatus":-2147483648}',
            b'{"username":null,"username":"back","email":"e","email":null}']
    rnd = random.Random(5)
    cols = pj.generate_model(pj.MODEL_USER, 2000, seed=9, null_rate=0.2)
    base = orc.encode_model(cols, pj.FORMAT_NDJSON, pj.INCLUDE_ALWAYS).split(b"\n")[:-1]
    user += [_mutate(rnd, rnd.choice(base)) if i % 3 else rnd.choice(base) for i in range(6000)]
    same_decode(codec, pj.MODEL_USER, b"\n".join(user))
    order = [b'{"shipDate":"2024-01-01T00:00:00Z","shipDate":"2024\\u002d02","status":"placed"}',
             b'{"shipDate":"a\\"b","shipDate":"plain","complete":true,"quantity":7}']
    cols = pj.generate_model(pj.MODEL_ORDER, 2000, seed=8, null_rate=0.2)
    base = orc.encode_model(cols, pj.FORMAT_NDJSON, pj.INCLUDE_ALWAYS).split(b"\n")[:-1]
    order += [_mutate(rnd, rnd.choice(base)) if i % 3 else rnd.choice(base) for i in range(6000)]
    same_decode(codec, pj.MODEL_ORDER, b"\n".join(order))
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_PRETTY):
        data = orc.encode_model(cols, fmt, pj.INCLUDE_ALWAYS)
        same_decode(codec, pj.MODEL_ORDER, data, array=True)
