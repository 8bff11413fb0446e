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
