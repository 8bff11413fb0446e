"""Helpers turning fixture dictionaries into model objects and back."""
import json
import os

from model import Category, Pet, StatusEnum, Tag

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with open(os.path.join(GOLDEN, name), encoding="utf-8") as f:
        return json.load(f)


def _txt(v, latin1):
    if v is None or not latin1:
        return v
    return v.encode("latin-1")


def pet_from_dict(d, latin1=False):
    cat = d.get("category")
    tags = d.get("tags")
    st = d.get("status")
    return Pet(
        id=d.get("id"),
        category=None if cat is None else Category(cat.get("id"), _txt(cat.get("name"), latin1)),
        name=_txt(d.get("name"), latin1),
        photo_urls=None if d.get("photoUrls") is None else [_txt(u, latin1) for u in d["photoUrls"]],
        tags=None if tags is None else [Tag(t.get("id"), _txt(t.get("name"), latin1)) for t in tags],
        status=None if st is None else StatusEnum.from_value(st),
    )


def norm_pet(p):
    """Comparable tuple form of a Pet with all strings as bytes."""
    b = lambda s: None if s is None else (s.encode() if isinstance(s, str) else bytes(s))
    return (
        p.id,
        None if p.category is None else (p.category.id, b(p.category.name)),
        b(p.name),
        None if p.photo_urls is None else tuple(b(u) for u in p.photo_urls),
        None if p.tags is None else tuple((t.id, b(t.name)) for t in p.tags),
        None if p.status is None else p.status.value,
    )


def line_bytes(case):
    if "line_latin1" in case:
        return case["line_latin1"].encode("latin-1")
    return case["line"].encode("utf-8")


def expected_pet(case):
    if "pet_latin1" in case:
        return pet_from_dict(case["pet_latin1"], latin1=True)
    return pet_from_dict(case["pet"])
