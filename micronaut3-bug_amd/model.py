"""Pet / Category / Tag / StatusEnum record classes and their column packing.

Shapes follow the petstore schema of the reference (petstore.json:858-936):
Pet {id: int64, category: Category, name: string (required),
photoUrls: [string] (required), tags: [Tag], status: enum}, Category and Tag
{id: int64, name: string}.  StatusEnum carries its JSON value like the
reference's @JsonValue enums (api/EnumParam.java:15-35) and ``from_value``
rejects unknown values like VariantEnum.byId (config/data/VariantEnum.java:39-47).

Strings may be given as ``str`` (encoded as UTF-8) or ``bytes`` (raw).
"""
from __future__ import annotations

import enum
from dataclasses import dataclass, field
from typing import List, Optional, Union

import numpy as np

from petjson import (Columns, PET_HAS_CATEGORY, PET_HAS_ID, PET_HAS_NAME, PET_HAS_PHOTOURLS, PET_HAS_TAGS,
                     STATUS_NULL, SUB_HAS_ID, SUB_HAS_NAME)

Text = Union[str, bytes]


class StatusEnum(enum.Enum):
    AVAILABLE = "available"
    PENDING = "pending"
    SOLD = "sold"

    @property
    def code(self) -> int:
        return _STATUS_CODES[self]

    @classmethod
    def from_value(cls, v: str) -> "StatusEnum":
        for s in cls:
            if s.value == v:
                return s
        raise ValueError(f"Unexpected value '{v}'")

    @classmethod
    def from_code(cls, c: int) -> Optional["StatusEnum"]:
        return None if c == STATUS_NULL else list(cls)[c]


_STATUS_CODES = {StatusEnum.AVAILABLE: 0, StatusEnum.PENDING: 1, StatusEnum.SOLD: 2}


@dataclass
class Category:
    id: Optional[int] = None
    name: Optional[Text] = None


@dataclass
class Tag:
    id: Optional[int] = None
    name: Optional[Text] = None


@dataclass
class Pet:
    name: Optional[Text] = None
    photo_urls: Optional[List[Text]] = field(default_factory=list)
    id: Optional[int] = None
    category: Optional[Category] = None
    tags: Optional[List[Tag]] = None
    status: Optional[StatusEnum] = None


def _b(s: Optional[Text]) -> bytes:
    if s is None:
        return b""
    return s.encode("utf-8") if isinstance(s, str) else bytes(s)


def _u(b: bytes, as_bytes: bool) -> Text:
    return b if as_bytes else b.decode("utf-8")


def to_columns(pets: List[Pet]) -> Columns:
    """Pack pets into host (numpy) SoA columns with every group present."""
    n = len(pets)
    ids = np.zeros(n, np.int64)
    flags = np.zeros(n, np.uint8)
    status = np.full(n, STATUS_NULL, np.uint8)
    cat_id = np.zeros(n, np.int64)
    cat_flags = np.zeros(n, np.uint8)
    name_off = np.zeros(n + 1, np.uint64)
    cat_name_off = np.zeros(n + 1, np.uint64)
    photo_off = np.zeros(n + 1, np.uint64)
    tag_off = np.zeros(n + 1, np.uint64)
    names, cnames, urls, url_off, tids, tflags, tnames, tname_off = [], [], [], [0], [], [], [], [0]
    nb = cb = ub = tb = 0
    for i, p in enumerate(pets):
        f = 0
        if p.id is not None:
            f |= PET_HAS_ID
            ids[i] = p.id
        if p.category is not None:
            f |= PET_HAS_CATEGORY
            cf = 0
            if p.category.id is not None:
                cf |= SUB_HAS_ID
                cat_id[i] = p.category.id
            if p.category.name is not None:
                cf |= SUB_HAS_NAME
                b = _b(p.category.name)
                cnames.append(b)
                cb += len(b)
            cat_flags[i] = cf
        if p.name is not None:
            f |= PET_HAS_NAME
            b = _b(p.name)
            names.append(b)
            nb += len(b)
        if p.photo_urls is not None:
            f |= PET_HAS_PHOTOURLS
            for u in p.photo_urls:
                b = _b(u)
                urls.append(b)
                ub += len(b)
                url_off.append(ub)
        if p.tags is not None:
            f |= PET_HAS_TAGS
            for t in p.tags:
                tf = 0
                if t.id is not None:
                    tf |= SUB_HAS_ID
                if t.name is not None:
                    tf |= SUB_HAS_NAME
                tids.append(t.id if t.id is not None else 0)
                tflags.append(tf)
                b = _b(t.name)
                tnames.append(b)
                tb += len(b)
                tname_off.append(tb)
        if p.status is not None:
            status[i] = p.status.code
        flags[i] = f
        name_off[i + 1] = nb
        cat_name_off[i + 1] = cb
        photo_off[i + 1] = len(url_off) - 1
        tag_off[i + 1] = len(tids)
    u8 = lambda parts: np.frombuffer(b"".join(parts) + b"\0\0\0\0", np.uint8)[: sum(map(len, parts))].copy()
    arrays = {
        "id": ids, "flags": flags, "status": status, "name_off": name_off, "name_bytes": u8(names),
        "cat_id": cat_id, "cat_flags": cat_flags, "cat_name_off": cat_name_off, "cat_name_bytes": u8(cnames),
        "photo_off": photo_off, "url_off": np.array(url_off, np.uint64), "url_bytes": u8(urls),
        "tag_off": tag_off, "tag_id": np.array(tids, np.int64), "tag_flags": np.array(tflags, np.uint8),
        "tag_name_off": np.array(tname_off, np.uint64), "tag_name_bytes": u8(tnames),
    }
    return Columns(n, arrays)


def from_columns(cols: Columns, as_bytes: bool = False) -> List[Pet]:
    """Unpack host columns into Pet objects (NULL column groups = absent)."""
    a = cols.to_host().arrays
    out = []
    for i in range(cols.n_pets):
        f = int(a["flags"][i]) if a.get("flags") is not None else PET_HAS_ID | PET_HAS_NAME | PET_HAS_PHOTOURLS
        p = Pet(photo_urls=None)
        if f & PET_HAS_ID:
            p.id = int(a["id"][i])
        if f & PET_HAS_NAME:
            p.name = _u(a["name_bytes"][int(a["name_off"][i]):int(a["name_off"][i + 1])].tobytes(), as_bytes)
        if (f & PET_HAS_CATEGORY) and a.get("cat_id") is not None:
            cf = int(a["cat_flags"][i]) if a.get("cat_flags") is not None else SUB_HAS_ID | SUB_HAS_NAME
            c = Category()
            if cf & SUB_HAS_ID:
                c.id = int(a["cat_id"][i])
            if cf & SUB_HAS_NAME:
                c.name = _u(a["cat_name_bytes"][int(a["cat_name_off"][i]):int(a["cat_name_off"][i + 1])].tobytes(),
                            as_bytes)
            p.category = c
        if f & PET_HAS_PHOTOURLS:
            p.photo_urls = []
            if a.get("photo_off") is not None:
                for u in range(int(a["photo_off"][i]), int(a["photo_off"][i + 1])):
                    p.photo_urls.append(_u(a["url_bytes"][int(a["url_off"][u]):int(a["url_off"][u + 1])].tobytes(),
                                           as_bytes))
        if f & PET_HAS_TAGS:
            p.tags = []
            if a.get("tag_off") is not None:
                for t in range(int(a["tag_off"][i]), int(a["tag_off"][i + 1])):
                    tf = int(a["tag_flags"][t]) if a.get("tag_flags") is not None else SUB_HAS_ID | SUB_HAS_NAME
                    g = Tag()
                    if tf & SUB_HAS_ID:
                        g.id = int(a["tag_id"][t])
                    if tf & SUB_HAS_NAME:
                        g.name = _u(a["tag_name_bytes"][int(a["tag_name_off"][t]):int(a["tag_name_off"][t + 1])]
                                    .tobytes(), as_bytes)
                    p.tags.append(g)
        if a.get("status") is not None:
            p.status = StatusEnum.from_code(int(a["status"][i]))
        out.append(p)
    return out
