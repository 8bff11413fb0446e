"""ObjectMapper-style surface over libpetjson for Pet objects (and the
petstore's Order and User records, as dicts).

Mirrors io.micronaut.serde.ObjectMapper as the reference uses it:
ObjectMapper.getDefault() (reference service/MyEntityService.java:45),
readValue (config/MyEntityConfig.java:34), writeValueAsBytes for List<Pet>
(petstore.json:106-140).  Errors raise PetJsonError; invalid NDJSON lines are
reported, not raised, so a batch keeps going.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import List

import numpy as np

import petjson as pj
from model import Pet, from_columns, to_columns


@dataclass
class ReadResult:
    values: List[Pet] = field(default_factory=list)
    error_lines: np.ndarray = None
    error_codes: np.ndarray = None


class PetObjectMapper:
    _local = threading.local()

    def __init__(self, device: int = 0, inclusion: int = pj.INCLUDE_NON_EMPTY, hex_upper: bool = True):
        self.codec = pj.Codec(device, inclusion, hex_upper)

    @classmethod
    def get_default(cls) -> "PetObjectMapper":
        """One mapper per thread (a context owns one HIP stream)."""
        m = getattr(cls._local, "mapper", None)
        if m is None:
            m = cls._local.mapper = cls()
        return m

    def write_value_as_bytes(self, pets: List[Pet], fmt: int = pj.FORMAT_ARRAY) -> bytes:
        return self.codec.encode_host(to_columns(pets), fmt)

    def write_value_as_string(self, pets: List[Pet], fmt: int = pj.FORMAT_ARRAY) -> str:
        return self.write_value_as_bytes(pets, fmt).decode("utf-8")

    def read_value(self, ndjson: bytes, as_bytes: bool = False) -> ReadResult:
        cols, el, ec, res = self.codec.decode_host(ndjson)
        return ReadResult(from_columns(cols, as_bytes=as_bytes), el, ec)

    def read_array(self, data: bytes, as_bytes: bool = False) -> ReadResult:
        """One JSON array document, element by element (invalid elements are
        reported by index); a broken array frame raises PJ_ERR_SYNTAX."""
        cols, el, ec, res = self.codec.decode_array_host(data)
        return ReadResult(from_columns(cols, as_bytes=as_bytes), el, ec)

    def read_value_list(self, data: bytes, as_bytes: bool = False) -> List[Pet]:
        """readValue(bytes, List<Pet>): all or nothing, as jackson reads it."""
        r = self.read_array(data, as_bytes)
        if len(r.error_lines):
            raise pj.PetJsonError(pj.PJ_ERR_SYNTAX, f"element {int(r.error_lines[0])} of the array is not a valid "
                                                    f"Pet (PJ_REC code {int(r.error_codes[0])})")
        return r.values

    def find_pets_by_status(self, pets: List[Pet], status_mask: int = 1, fmt: int = pj.FORMAT_ARRAY) -> bytes:
        """GET /pet/findByStatus (petstore.json:106-140): the response body of
        the pets whose status is in the mask (bit 0 available, the query's
        default; 1 pending; 2 sold; 3 no status)."""
        body, _ = self.codec.encode_by_status_host(to_columns(pets), status_mask, fmt)
        return body

    def write_orders(self, orders: List[dict], fmt: int = pj.FORMAT_ARRAY) -> bytes:
        """writeValueAsBytes(List<Order>): records as dicts of the Order
        properties (petstore.json:937-971); a missing or None one is null."""
        return self.codec.encode_model_host(_model_columns(pj.MODEL_ORDER, orders), fmt)

    def write_users(self, users: List[dict], fmt: int = pj.FORMAT_ARRAY) -> bytes:
        """writeValueAsBytes(List<User>) (petstore.json:824-857)."""
        return self.codec.encode_model_host(_model_columns(pj.MODEL_USER, users), fmt)

    def read_orders(self, data: bytes, array: bool = False) -> ReadResult:
        return self._read_model(pj.MODEL_ORDER, data, array)

    def read_users(self, data: bytes, array: bool = False) -> ReadResult:
        return self._read_model(pj.MODEL_USER, data, array)

    def _read_model(self, model: int, data: bytes, array: bool) -> ReadResult:
        cols, el, ec, res = self.codec.decode_model_host(model, data, array)
        return ReadResult(_model_records(cols), el, ec)

    def close(self):
        self.codec.close()


def _model_columns(model: int, records: List[dict]) -> pj.ModelColumns:
    """Order / User dicts as host columns (None or missing: null)."""
    props = pj.MODEL_PROPS[model]
    n = len(records)
    present = np.zeros(n, np.uint8)
    col, byt = [], []
    for k, (name, kind) in enumerate(props):
        vals = [r.get(name) for r in records]
        for i, v in enumerate(vals):
            if v is not None:
                present[i] |= 1 << k
        if kind == "str":
            bs = [v.encode("utf-8") if isinstance(v, str) else (v or b"") for v in vals]
            off = np.zeros(n + 1, np.uint64)
            off[1:] = np.cumsum([len(b) for b in bs], dtype=np.uint64) if n else []
            col.append(off)
            byt.append(np.frombuffer(b"".join(bs), np.uint8).copy())
        else:
            if kind == "enum":
                vals = [pj.ORDER_STATUS.index(v) if v is not None else 0 for v in vals]
            col.append(np.array([int(v or 0) for v in vals], pj.KIND_DTYPE[kind]))
            byt.append(None)
    return pj.ModelColumns(model, n, present, col, byt)


def _model_records(c: pj.ModelColumns) -> List[dict]:
    """Host columns back to dicts of the non-null properties."""
    out = []
    for i in range(c.n):
        r = {}
        for k, (name, kind) in enumerate(c.props):
            if not (int(c.present[i]) >> k) & 1:
                continue
            v = c.col[k]
            if kind == "str":
                r[name] = c.bytes[k][int(v[i]): int(v[i + 1])].tobytes().decode("utf-8", "surrogateescape")
            elif kind == "enum":
                r[name] = pj.ORDER_STATUS[int(v[i])]
            elif kind == "bool":
                r[name] = bool(v[i])
            else:
                r[name] = int(v[i])
        out.append(r)
    return out
