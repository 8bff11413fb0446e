"""Seeded differential tests: random Pet columns (every presence bit, null
groups, ids across the int64 range, strings with every byte class, lists
long enough for the large-record paths) are encoded by libpetjson and by the
CPU restatement under random options and framings, byte for byte; the NDJSON
output, with random byte mutations, is then decoded by both and compared
column by column.  Sizes vary so that records fall on every position of the
96- and 256-record workgroups."""
import numpy as np
import pytest
import torch

import oracle_py as orc
import petjson as pj

pytestmark = pytest.mark.gpu

# byte palette: plain ASCII, every character that needs an escape, '/', DEL,
# and complete UTF-8 sequences of 2, 3 and 4 bytes
_ASCII = [bytes([c]) for c in b"abcxyzABC019 -_.:"]
_SPECIAL = [bytes([c]) for c in range(0x20)] + [b'"', b"\\", b"/", b"\x7f"]
_UTF8 = ["é".encode(), "€".encode(), "😀".encode(), "ß".encode()]


def _string(rng, long_p=0.0):
    n = int(rng.integers(1000, 3000)) if rng.random() < long_p else int(rng.geometric(0.08)) - 1
    mix = rng.random()
    out = []
    for _ in range(n):
        r = rng.random()
        if r < mix * 0.3:
            out.append(_SPECIAL[rng.integers(len(_SPECIAL))])
        elif r < mix * 0.45:
            out.append(_UTF8[rng.integers(len(_UTF8))])
        else:
            out.append(_ASCII[rng.integers(len(_ASCII))])
    return b"".join(out)


def _ids(rng, n):
    kind = rng.integers(0, 4, n)
    small = rng.integers(0, 1000, n)
    full = rng.integers(np.iinfo(np.int64).min, np.iinfo(np.int64).max, n, dtype=np.int64, endpoint=True)
    edge = rng.choice(np.array([0, -1, 1, 9, 10, 99999999, 100000000, 9999999999999999, 10000000000000000,
                                np.iinfo(np.int64).max, np.iinfo(np.int64).min], dtype=np.int64), n)
    return np.where(kind == 0, small, np.where(kind == 1, full, np.where(kind == 2, -small, edge))).astype(np.int64)


def _strings(rng, count, long_p=0.0):
    parts = [_string(rng, long_p) for _ in range(count)]
    off = np.zeros(count + 1, np.uint64)
    off[1:] = np.cumsum([len(p) for p in parts], dtype=np.uint64)
    return off, np.frombuffer(b"".join(parts) or b"\0", np.uint8).copy()


def _counts(rng, n, big_p):
    c = rng.poisson(rng.uniform(0.3, 3.0), n)
    big = rng.random(n) < big_p
    c[big] = rng.integers(17, 60, int(big.sum()))
    return c.astype(np.uint64)


def random_columns(rng, n):
    a = {}
    a["id"] = _ids(rng, n)
    a["flags"] = rng.integers(0, 32, n, dtype=np.uint8)
    st = rng.integers(0, 3, n).astype(np.uint8)
    st[rng.random(n) < 0.1] = pj.STATUS_NULL
    a["status"] = st
    a["name_off"], a["name_bytes"] = _strings(rng, n, long_p=0.01)
    a["cat_id"] = _ids(rng, n)
    a["cat_flags"] = rng.integers(0, 4, n, dtype=np.uint8)
    a["cat_name_off"], a["cat_name_bytes"] = _strings(rng, n)
    nu = _counts(rng, n, 0.005)
    a["photo_off"] = np.concatenate([[0], np.cumsum(nu)]).astype(np.uint64)
    a["url_off"], a["url_bytes"] = _strings(rng, int(nu.sum()))
    nt = _counts(rng, n, 0.005)
    a["tag_off"] = np.concatenate([[0], np.cumsum(nt)]).astype(np.uint64)
    a["tag_id"] = _ids(rng, int(nt.sum()))
    a["tag_flags"] = rng.integers(0, 4, int(nt.sum()), dtype=np.uint8)
    a["tag_name_off"], a["tag_name_bytes"] = _strings(rng, int(nt.sum()))
    # sometimes whole groups are absent
    for group, keys in (("cat", ("cat_id", "cat_flags", "cat_name_off", "cat_name_bytes")),
                        ("urls", ("photo_off", "url_off", "url_bytes")),
                        ("tags", ("tag_off", "tag_id", "tag_flags", "tag_name_off", "tag_name_bytes"))):
        if rng.random() < 0.15:
            for k in keys:
                a[k] = None
            if group == "cat":
                a["flags"] &= np.uint8(~pj.PET_HAS_CATEGORY & 0xFF)
    if rng.random() < 0.1:
        a["cat_flags"] = None if a["cat_id"] is not None else a["cat_flags"]
        a["tag_flags"] = None if a["tag_off"] is not None else a["tag_flags"]
    return pj.Columns(n, a)


SIZES = [1, 2, 95, 96, 97, 191, 255, 256, 257, 511, 767, 1000, 2049, 3001, 6000, 12000]
# decode: also line counts around the 104-line parse workgroups
SIZES_DEC = SIZES + [103, 104, 105, 207, 208, 209, 1039, 1040, 1041]


# 1074 and 1271: HAS_TAGS set with every nested column group absent (the flat
# kernel), once written as "tags":null or left out instead of an empty list
@pytest.mark.parametrize("seed", list(range(64)) + [1074, 1271])
def test_encode_random_columns_match_oracle(codec, seed):
    rng = np.random.default_rng(0xF022 + seed)
    n = SIZES[seed % len(SIZES)] + int(rng.integers(0, 3))
    cols = random_columns(rng, n)
    incl = int(rng.integers(0, 3))
    hexu = bool(rng.integers(0, 2))
    fmt = int(rng.integers(0, 2))
    codec.set_options(incl, hexu)
    try:
        got = codec.encode(cols.to_device(), fmt).cpu().numpy().tobytes()
    finally:
        codec.set_options()
    assert got == orc.encode(cols, fmt, incl, hexu), (seed, n, incl, hexu, fmt)


def _mutate(rng, data: bytes) -> bytes:
    b = bytearray(data)
    for _ in range(int(rng.integers(0, 1 + len(b) // 200))):
        k = int(rng.integers(0, len(b)))
        r = rng.random()
        if b[k] == 0x0A:
            continue                                        # keep the line structure
        if r < 0.4:
            b[k] = int(rng.choice(list(b'"\\{}[],:0a \x01\xc3\xff')))
        elif r < 0.7:
            del b[k]
        else:
            b.insert(k, int(rng.choice(list(b'"\\,}] '))))
    return bytes(b)


def _gpu_decode(codec, data: bytes):
    buf = torch.zeros(len(data) + 16, dtype=torch.uint8, device="cuda")
    if data:
        buf[: len(data)] = torch.frombuffer(bytearray(data), dtype=torch.uint8).cuda()
    cols, el, ec, res = codec.decode(buf[: len(data)])
    return cols.to_host(), el.cpu().numpy().astype(np.uint64), ec.cpu().numpy(), res


@pytest.mark.parametrize("seed", range(50))
def test_decode_random_encodings_match_oracle(codec, seed):
    rng = np.random.default_rng(0xDEC0 + seed)
    n = SIZES_DEC[seed % len(SIZES_DEC)] + int(rng.integers(0, 3))
    cols = random_columns(rng, n)
    text = orc.encode(cols, pj.FORMAT_NDJSON, int(rng.integers(0, 3)), bool(rng.integers(0, 2)))
    if seed % 2:
        text = _mutate(rng, text)
    gc, gel, gec, gres = _gpu_decode(codec, text)
    rc, rel, rec, rres = orc.decode(text)
    for f in ("n_lines", "n_pets", "n_errors", "name_bytes", "cat_name_bytes", "n_urls", "url_bytes", "n_tags",
              "tag_name_bytes"):
        assert getattr(gres, f) == getattr(rres, f), (seed, f)
    assert np.array_equal(gel, rel) and np.array_equal(gec, rec), seed
    for k in pj.COLS:
        assert np.array_equal(gc[k], rc[k]), (seed, k)
