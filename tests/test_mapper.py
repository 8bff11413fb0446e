"""Host-side mirrors of the ObjectMapper surface: the C++ PetObjectMapper
(self-test binary) and the Python mapper.  CPU tests check packing and the
oracle known answer; GPU tests check the full write / read path."""
import os
import subprocess

import pytest

import oracle_py as orc
import petjson as pj
from kat_util import pet_from_dict, load, norm_pet
from model import StatusEnum, Pet, Tag, Category, to_columns, from_columns

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "bin", "mapper_selftest")


def test_cpp_mapper_selftest_cpu():
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "ok (cpu)" in r.stdout


def test_python_model_roundtrip():
    pets = [pet_from_dict(c) for case in load("encode_kat.json")["cases"] for c in case["pets"]]
    back = from_columns(to_columns(pets))
    assert [norm_pet(p) for p in back] == [norm_pet(p) for p in pets]
    assert StatusEnum.from_value("sold") is StatusEnum.SOLD
    with pytest.raises(ValueError):
        StatusEnum.from_value("lost")


@pytest.mark.gpu
def test_cpp_mapper_selftest_gpu():
    r = subprocess.run([BIN, "gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr + r.stdout
    assert "ok (gpu)" in r.stdout


@pytest.mark.gpu
def test_python_mapper_write_read():
    from mapper import PetObjectMapper
    m = PetObjectMapper.get_default()
    pets = [Pet(name="doggie", photo_urls=["https://x/a"], id=10, category=Category(1, "Dogs"),
                tags=[Tag(0, "t")], status=StatusEnum.AVAILABLE),
            Pet(name="é\"\n", photo_urls=[])]
    b = m.write_value_as_bytes(pets, pj.FORMAT_NDJSON)
    assert b == orc.encode(to_columns(pets), pj.FORMAT_NDJSON)
    r = m.read_value(b + b'{"name":1,"photoUrls":[]}\n')
    assert [norm_pet(p) for p in r.values] == [norm_pet(p) for p in pets]
    assert list(r.error_lines) == [2] and list(r.error_codes) == [pj.REC_TYPE]


@pytest.mark.gpu
def test_python_mapper_orders_users_and_find_by_status():
    from mapper import PetObjectMapper, _model_columns
    m = PetObjectMapper.get_default()
    orders = [{"id": 1, "petId": 7, "quantity": 2, "shipDate": "2026-01-02T03:04:05Z", "status": "approved",
               "complete": True}, {"id": 2}, {}]
    users = [{"id": 9, "username": "ué\"", "userStatus": -3}, {"email": "a@b"}]
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
        ob, ub = m.write_orders(orders, fmt), m.write_users(users, fmt)
        assert ob == orc.encode_model(_model_columns(pj.MODEL_ORDER, orders), fmt)
        assert ub == orc.encode_model(_model_columns(pj.MODEL_USER, users), fmt)
        ro = m.read_orders(ob, array=fmt != pj.FORMAT_NDJSON)
        ru = m.read_users(ub, array=fmt != pj.FORMAT_NDJSON)
        assert ro.values == orders and len(ro.error_lines) == 0
        assert ru.values == users and len(ru.error_lines) == 0
    pets = [Pet(name="a", photo_urls=[], status=StatusEnum.AVAILABLE), Pet(name="b", photo_urls=[]),
            Pet(name="c", photo_urls=["u"], status=StatusEnum.SOLD)]
    assert m.find_pets_by_status(pets) == orc.encode(to_columns(pets[:1]), pj.FORMAT_ARRAY)
    assert m.find_pets_by_status(pets, 0b1100) == orc.encode(to_columns(pets[1:]), pj.FORMAT_ARRAY)
