"""ObjectMapper-style surface over libpetjson for Pet objects.

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

    def close(self):
        self.codec.close()
