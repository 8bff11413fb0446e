"""GPU encode parity: libpetjson (gfx950) output is byte-identical to the CPU
restatement on the same seeded records, for every configuration, both
framings and every inclusion option, plus edge cases (empty input, one
record, misaligned columns, capacity overflow)."""
import hashlib

import numpy as np
import pytest
import torch

import oracle_py as orc
import petjson as pj
from kat_util import load, pet_from_dict
from model import to_columns

pytestmark = pytest.mark.gpu
INCL = {"NON_EMPTY": pj.INCLUDE_NON_EMPTY, "NON_NULL": pj.INCLUDE_NON_NULL, "ALWAYS": pj.INCLUDE_ALWAYS}


def gpu_encode(codec, cols, fmt, incl=pj.INCLUDE_NON_EMPTY, hex_upper=True, fields=None):
    codec.set_options(incl, hex_upper, fields)
    try:
        return codec.encode(cols.to_device(), fmt).cpu().numpy().tobytes()
    finally:
        codec.set_options()


@pytest.mark.parametrize("case", load("encode_kat.json")["cases"], ids=lambda c: c["name"])
def test_encode_kat_gpu(codec, case):
    cols = to_columns([pet_from_dict(p) for p in case["pets"]])
    fmt = {"ndjson": pj.FORMAT_NDJSON, "pretty": pj.FORMAT_PRETTY}.get(case.get("format"), pj.FORMAT_ARRAY)
    incl = INCL[case.get("inclusion", "NON_EMPTY")]
    hx = case.get("hex_upper", True)
    fields = {k: INCL[v] for k, v in case.get("fields", {}).items()}
    assert gpu_encode(codec, cols, fmt, incl, hx, fields) == case["expected"].encode("utf-8")
    codec.set_options(incl, hx, fields)
    assert codec.encode_host(cols, fmt) == case["expected"].encode("utf-8")
    codec.set_options()


@pytest.mark.parametrize("config,n", [(1, 100_000), (2, 200_000), (3, 100_000), (5, 20_000)])
@pytest.mark.parametrize("fmt", [pj.FORMAT_ARRAY, pj.FORMAT_NDJSON])
def test_encode_configs_match_oracle(codec, config, n, fmt):
    print(f"[encode parity] config={config} n={n} fmt={fmt}", flush=True)
    cols = pj.generate(config, n)
    assert gpu_encode(codec, cols, fmt) == orc.encode(cols, fmt)


@pytest.mark.parametrize("incl", [pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS])
def test_encode_inclusion_options_match_oracle(codec, incl):
    cols = pj.generate(3, 30_000)
    # knock out some fields so that nulls / empties occur
    rng = np.random.default_rng(1)
    cols.arrays["flags"] = cols["flags"] & rng.integers(0, 32, cols.n_pets, dtype=np.uint8) | pj.PET_HAS_NAME
    cols.arrays["status"][rng.random(cols.n_pets) < 0.2] = pj.STATUS_NULL
    cols.arrays["tag_flags"] = rng.integers(0, 4, cols["tag_flags"].shape[0], dtype=np.uint8)
    assert gpu_encode(codec, cols, pj.FORMAT_ARRAY, incl, False) == \
        orc.encode(cols, pj.FORMAT_ARRAY, incl, False)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_encode_per_field_inclusion_matches_oracle(codec, seed):
    """Random per-property inclusion modes over records with nulls and
    empties in every optional property (configs 1, 3 and 5, both framings;
    the skewed config also goes through the hybrid and whole-workgroup
    paths)."""
    rng = np.random.default_rng(seed)
    modes = [pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS]
    for config, n in ((1, 20_000), (3, 30_000), (5, 5_000)):
        cols = pj.generate(config, n)
        cols.arrays["flags"] = cols["flags"] & rng.integers(0, 32, cols.n_pets, dtype=np.uint8) | pj.PET_HAS_NAME
        cols.arrays["status"][rng.random(cols.n_pets) < 0.2] = pj.STATUS_NULL
        cols.arrays["tag_flags"] = rng.integers(0, 4, cols["tag_flags"].shape[0], dtype=np.uint8)
        cols.arrays["cat_flags"] = rng.integers(0, 4, cols["cat_flags"].shape[0], dtype=np.uint8)
        glob = int(rng.choice(modes))
        fields = {f: int(rng.choice(modes)) for f in pj.FIELDS if rng.random() < 0.6}
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            assert gpu_encode(codec, cols, fmt, glob, True, fields) == orc.encode(cols, fmt, glob, True, fields), \
                (config, glob, fields, fmt)


def test_encode_misaligned_string_columns(codec):
    cols = pj.generate(3, 5000)
    for shift in (1, 2, 3):
        c2 = pj.Columns(cols.n_pets, dict(cols.arrays))
        for k in ("name_bytes", "cat_name_bytes", "url_bytes", "tag_name_bytes"):
            pad = np.concatenate([np.full(shift, 0x41, np.uint8), cols[k]])
            c2.arrays[k] = pad
        for k, kb in (("name_off", "name_bytes"), ("cat_name_off", "cat_name_bytes"), ("url_off", "url_bytes"),
                      ("tag_name_off", "tag_name_bytes")):
            c2.arrays[k] = cols[k] + np.uint64(shift)
        assert gpu_encode(codec, c2, pj.FORMAT_ARRAY) == orc.encode(cols, pj.FORMAT_ARRAY)


def test_encode_into_misaligned_output(codec):
    """An output buffer that starts off 16-byte alignment: the tile copy-out's
    whole-line stores then fall at unaligned addresses.  Only the output's
    bytes change, nothing before or after them."""
    for config, n, fmt in ((3, 20_000, pj.FORMAT_ARRAY), (2, 30_000, pj.FORMAT_NDJSON),
                           (5, 6_000, pj.FORMAT_NDJSON), (3, 8_000, pj.FORMAT_PRETTY)):
        cols = pj.generate(config, n)
        ref = np.frombuffer(orc.encode(cols, fmt), np.uint8)
        d = cols.to_device()
        buf = torch.full((ref.size + 64,), 0xEE, dtype=torch.uint8, device="cuda")
        for off in (1, 3, 8, 13):
            print(f"[encode misaligned out] config={config} fmt={fmt} off={off}", flush=True)
            buf.fill_(0xEE)
            got = codec.encode(d, fmt, out=buf[off:off + ref.size])
            assert got.numel() == ref.size
            host = buf.cpu().numpy()
            assert (host[:off] == 0xEE).all() and (host[off + ref.size:] == 0xEE).all(), (config, fmt, off)
            assert np.array_equal(host[off:off + ref.size], ref), (config, fmt, off)


def test_encode_long_strings_and_all_bytes(codec):
    big = bytes(range(256)) * 70 + b"x" * 3
    pets = [pet_from_dict({"name": "n", "photoUrls": []})]
    p = pets[0]
    p.name = big
    p.photo_urls = [big[: k] for k in range(0, 64)]
    cols = to_columns(pets * 3)
    assert gpu_encode(codec, cols, pj.FORMAT_NDJSON) == orc.encode(cols, pj.FORMAT_NDJSON)


def test_encode_empty_and_single(codec):
    cols = to_columns([])
    assert gpu_encode(codec, cols, pj.FORMAT_ARRAY) == b"[]"
    assert gpu_encode(codec, cols, pj.FORMAT_NDJSON) == b""
    cols = pj.generate(3, 1)
    assert gpu_encode(codec, cols, pj.FORMAT_ARRAY) == orc.encode(cols, pj.FORMAT_ARRAY)


GROUPS = {"category": ("cat_id", "cat_flags", "cat_name_off", "cat_name_bytes"),
          "photoUrls": ("photo_off", "url_off", "url_bytes"),
          "tags": ("tag_off", "tag_id", "tag_flags", "tag_name_off", "tag_name_bytes")}


@pytest.mark.parametrize("absent", [("category",), ("photoUrls",), ("tags",), ("photoUrls", "tags"),
                                    ("category", "tags"), ("category", "photoUrls")])
@pytest.mark.parametrize("incl", [pj.INCLUDE_NON_EMPTY, pj.INCLUDE_ALWAYS])
def test_encode_absent_groups_match_oracle(codec, absent, incl):
    """Nested records with whole column groups absent (NULL pointers): the
    records still go through the nested kernel, with empty lists or no
    category for every record."""
    cols = pj.generate(3, 5_000)
    for g in absent:
        for k in GROUPS[g]:
            cols.arrays[k] = None
    flags = cols["flags"].copy()
    if "category" in absent:
        flags &= ~np.uint8(pj.PET_HAS_CATEGORY)
    cols.arrays["flags"] = flags
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
        assert gpu_encode(codec, cols, fmt, incl) == orc.encode(cols, fmt, incl), (absent, fmt)


def test_encode_capacity_guard(codec):
    cols = pj.generate(2, 10_000)
    d = cols.to_device()
    need = codec.encode_size(d, pj.FORMAT_ARRAY)
    out = torch.full((need,), 0xEE, dtype=torch.uint8, device="cuda")
    cap = need // 2
    with pytest.raises(pj.PetJsonError) as ei:
        codec.encode(d, pj.FORMAT_ARRAY, out=out[:cap])
    assert ei.value.status == pj.PJ_ERR_CAPACITY
    host = out.cpu().numpy()
    assert (host[cap:] == 0xEE).all()          # nothing past the capacity
    ref = np.frombuffer(orc.encode(cols, pj.FORMAT_ARRAY), np.uint8)
    written = host[:cap] != 0xEE
    assert (host[:cap][written] == ref[:cap][written]).all()


@pytest.mark.parametrize("config", [2, 3])
def test_encode_full_size_matches_oracle(codec, config):
    """10M records (benchmark size): byte-identical to the CPU restatement."""
    print(f"[encode full] config={config}", flush=True)
    cols = pj.generate(config, 10_000_000)
    gpu = codec.encode(cols.to_device(), pj.FORMAT_ARRAY).cpu().numpy()
    ref = orc.encode(cols, pj.FORMAT_ARRAY)
    assert gpu.size == len(ref)
    assert hashlib.sha256(gpu.tobytes()).hexdigest() == hashlib.sha256(ref).hexdigest()


def _wrap_case(R, lists):
    """Records where, at the start of every R-record block, a record that owns
    list items but has that list nulled is followed by one that writes its
    list, with item lengths chosen so that the second record's item base
    (tile offset minus the items before it, modulo 2^32) is 0xFFFFFFFF."""
    from model import Pet, Tag, StatusEnum
    key = "photoUrls" if lists == "urls" else "tags"
    flag = pj.PET_HAS_PHOTOURLS if lists == "urls" else pj.PET_HAS_TAGS

    def build(fill):
        pets = [Pet(name="p", photo_urls=["u"], id=j, status=StatusEnum.SOLD) for j in range(2 * R)]
        for k in (0, R):
            if lists == "urls":
                pets[k] = Pet(name="a", photo_urls=["x" * fill], id=k)
                pets[k + 1] = Pet(name="b", photo_urls=["u"], id=k + 1)
            else:
                pets[k] = Pet(name="a", photo_urls=[], tags=[Tag(name="x" * fill)], id=k)
                pets[k + 1] = Pet(name="b", photo_urls=[], tags=[Tag(id=1, name="t")], id=k + 1)
        cols = to_columns(pets)
        for k in (0, R):
            cols.arrays["flags"][k] &= ~np.uint8(flag)
        return cols

    cols = build(1)
    recs = orc.encode(cols, pj.FORMAT_NDJSON).split(b"\n")
    pre = len(recs[0]) + 1                          # the block's first record with its separator
    ustart = 1 + recs[1].index(b'"' + key.encode() + b'":[') + len(key) + 4
    item_overhead = 3 if lists == "urls" else len(b'{"name":""},')
    fill = pre + ustart + 1 - item_overhead
    assert fill > 0
    return build(fill)


@pytest.mark.parametrize("lists", ["urls", "tags"])
def test_encode_item_base_wrap(codec, lists):
    """Regression: an item base equal to the no-items sentinel must still be
    written (whatever the records-per-block of the build)."""
    for R in (32, 48, 64, 80, 96, 112, 128, 160, 192, 256):
        cols = _wrap_case(R, lists)
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            assert gpu_encode(codec, cols, fmt) == orc.encode(cols, fmt), (R, lists, fmt)


def _hybrid_pets():
    """Nested records where some blocks (96 records each) hold large records
    (names over 512 bytes, or more than 16 tags) at the block's start, end,
    side by side and alone, the rest ordinary."""
    import random
    from model import Tag, from_columns
    rnd = random.Random(7)
    pets = from_columns(pj.generate(3, 96 * 12), as_bytes=True)
    frag = [b"a", b"\"", b"\\", b"\n", b"\x01", b"\xc3\xa9", b"\xf0\x9f\x98\x80", b"xyz"]
    big_at = [0, 95, 96, 97, 98, 200, 287, 288, 383, 500, 501, 600, 700, 701, 702, 703, 1100, 1151]
    for k, i in enumerate(big_at):
        p = pets[i]
        if k % 3 != 2:
            p.name = b"".join(rnd.choice(frag) for _ in range(rnd.randrange(300, 3000)))
        if k % 3 != 0:
            p.tags = [Tag(id=rnd.randrange(-10**15, 10**15), name=b"t%d" % j) for j in range(rnd.randrange(17, 220))]
    return pets


def test_encode_hybrid_blocks_match_oracle(codec):
    """Blocks holding large records keep their other records in the LDS tile
    and leave as segments between the large ones, which the workgroup writes
    directly: against the oracle in both framings, and under a capacity cut
    inside such a block."""
    cols = to_columns(_hybrid_pets())
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
        assert gpu_encode(codec, cols, fmt) == orc.encode(cols, fmt)
    d = cols.to_device()
    ref = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), np.uint8)
    for cap in (len(ref) // 3, len(ref) - 5):
        out = torch.full((len(ref),), 0xEE, dtype=torch.uint8, device="cuda")
        with pytest.raises(pj.PetJsonError):
            codec.encode(d, pj.FORMAT_NDJSON, out=out[:cap])
        host = out.cpu().numpy()
        assert (host[cap:] == 0xEE).all()
        written = host[:cap] != 0xEE
        assert (host[:cap][written] == ref[:cap][written]).all()


def _offtile_cases():
    """Blocks (96 records) that do not fit the tile path whole: medium names
    past the staging buffer with a large record now and then, many large
    records, a url larger than the staging buffer, control-byte names whose
    output overflows the tile, large records side by side with ordinary
    ones."""
    import random
    from model import Tag, from_columns
    rnd = random.Random(11)
    frag = [b"a", b"bc", b"\"", b"\\", b"\n", b"\x01", b"\x1f", b"\xc3\xa9", b"\xf0\x9f\x98\x80", b"xyz0123"]

    def name(lo, hi):
        out = b"".join(rnd.choice(frag) for _ in range(rnd.randrange(lo, hi)))
        return out

    cases = {}
    # medium names everywhere, a large record now and then
    pets = from_columns(pj.generate(3, 96 * 8), as_bytes=True)
    for k, p in enumerate(pets):
        p.name = name(20, 160)
        if k % 53 == 7:
            p.name = name(900, 2000)
        if k % 71 == 3:
            p.tags = [Tag(id=rnd.randrange(-10**15, 10**15), name=b"t%d" % j) for j in range(rnd.randrange(17, 40))]
    cases["medium_names"] = pets
    # a large record every 8th record
    pets = from_columns(pj.generate(3, 96 * 3), as_bytes=True)
    for k, p in enumerate(pets):
        if k % 8 == 0:
            p.name = name(600, 700)
    cases["many_large"] = pets
    # a record whose url alone overflows the staging buffer
    pets = from_columns(pj.generate(3, 96 * 3), as_bytes=True)
    pets[100].photo_urls = [b"https://" + b"u" * 20000]
    pets[101].name = name(900, 1000)
    cases["huge_url"] = pets
    # names of control bytes (6 output bytes each): the output overflows the tile
    pets = from_columns(pj.generate(3, 96 * 3), as_bytes=True)
    for k, p in enumerate(pets[96:192]):
        p.name = b"\x01" * 120
    pets[150].name = name(900, 1000)
    cases["tile_overflow"] = pets
    # single ordinary records between large records
    pets = from_columns(pj.generate(3, 96 * 2), as_bytes=True)
    for k in range(0, 96 * 2, 2):
        if k % 96 < 12:
            pets[k].name = name(600, 700)
    cases["alternating"] = pets
    return cases


@pytest.mark.parametrize("two_pass", [False, True])
def test_encode_offtile_blocks_match_oracle(codec, two_pass):
    """Blocks that do not fit the tile path whole (hybrid blocks, and blocks
    written one record per thread): against the oracle in both framings,
    single pass and at measured offsets, with a capacity cut inside such a
    block."""
    for label, pets in _offtile_cases().items():
        cols = to_columns(pets)
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            print(f"[offtile] {label} fmt={fmt} two_pass={two_pass}", flush=True)
            ref = orc.encode(cols, fmt)
            codec.set_options()
            d = cols.to_device()
            assert codec.encode_size(d, fmt) == len(ref), label
            assert codec.encode(d, fmt, two_pass=two_pass).cpu().numpy().tobytes() == ref, (label, fmt)
        if label == "medium_names" and not two_pass:
            ref = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), np.uint8)
            for cap in (len(ref) // 2, len(ref) - 7):
                out = torch.full((len(ref),), 0xEE, dtype=torch.uint8, device="cuda")
                with pytest.raises(pj.PetJsonError):
                    codec.encode(d, pj.FORMAT_NDJSON, out=out[:cap])
                host = out.cpu().numpy()
                assert (host[cap:] == 0xEE).all()
                written = host[:cap] != 0xEE
                assert (host[:cap][written] == ref[:cap][written]).all()


def test_encode_lookback_redo_in_ticket_order(codec, monkeypatch):
    """Flat blocks take their records in launch order and bound their
    look-back waits; a launch in which some wait ran out is redone with
    ticket-ordered blocks.  A one-tick bound forces that path: the output is
    still exact (nested records, on persistent ticket-ordered workgroups,
    have no bound and ignore it)."""
    monkeypatch.setenv("PETJSON_SPIN_LIMIT_TICKS", "1")
    for config, n in ((2, 300_000), (3, 100_000), (5, 20_000)):
        cols = pj.generate(config, n)
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            assert gpu_encode(codec, cols, fmt) == orc.encode(cols, fmt)


@pytest.mark.parametrize("big_cap", ["0", "1", "5"])
def test_encode_large_record_list_limits(codec, monkeypatch, big_cap):
    """Large records of nested blocks are listed for a second kernel to
    write (k_enc_big); those past the list's room are written by the pass
    itself.  With no list, a list of one and of five slots (the default
    holds 2^20) the bytes equal the oracle's, in blocks on and off the tile
    path, in both framings and at measured offsets."""
    monkeypatch.setenv("PETJSON_ENC_BIG_CAP", big_cap)
    cases = dict(_offtile_cases())
    cases["hybrid"] = _hybrid_pets()
    for label, pets in cases.items():
        cols = to_columns(pets)
        d = cols.to_device()
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            print(f"[big_cap] {big_cap} {label} fmt={fmt}", flush=True)
            ref = orc.encode(cols, fmt)
            for two_pass in (False, True):
                assert codec.encode(d, fmt, two_pass=two_pass).cpu().numpy().tobytes() == ref, (label, fmt, two_pass)
    cols = pj.generate(5, 20_000)
    assert gpu_encode(codec, cols, pj.FORMAT_NDJSON) == orc.encode(cols, pj.FORMAT_NDJSON)


def test_encode_persistent_workgroups_many_rounds(codec):
    """Nested records run on persistent workgroups (as many as the device
    holds at once: 768 on one MI355X) that claim blocks of 96 records by
    ticket until none is left; flat records one block of 256 per workgroup.
    Block counts below, at and far above one round give the oracle's bytes."""
    for config, n in ((3, 96 * 767 + 5), (3, 96 * 768), (3, 96 * 2305 + 1), (2, 256 * 1280 + 17), (2, 256 * 3900)):
        cols = pj.generate(config, n)
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
            assert gpu_encode(codec, cols, fmt) == orc.encode(cols, fmt), (config, n, fmt)


def test_encode_flat_long_records_switch_to_wide_tile(codec):
    """Flat records longer than the compact tile allows: the first call's
    blocks fall back, and later calls use the wide tile; every call's output
    equals the oracle's."""
    rnd = np.random.default_rng(3)
    base = pj.generate(2, 40_000)
    n = base.n_pets
    lens = rnd.integers(40, 120, size=n)
    off = np.zeros(n + 1, np.uint64)
    off[1:] = np.cumsum(lens)
    alnum = np.frombuffer(b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789", np.uint8)
    nb = alnum[rnd.integers(0, len(alnum), size=int(off[-1]))]
    cols = pj.Columns(n, dict(base.arrays))
    cols.arrays["name_off"] = off
    cols.arrays["name_bytes"] = nb
    ref = orc.encode(cols, pj.FORMAT_ARRAY)
    for _ in range(3):
        assert gpu_encode(codec, cols, pj.FORMAT_ARRAY) == ref


# ------------------------------------------------------------ pretty output
@pytest.mark.parametrize("config,n", [(1, 50_000), (2, 100_000), (3, 60_000), (5, 10_000)])
def test_encode_pretty_matches_oracle(codec, config, n):
    print(f"[encode pretty] config={config} n={n}", flush=True)
    cols = pj.generate(config, n)
    assert gpu_encode(codec, cols, pj.FORMAT_PRETTY) == orc.encode(cols, pj.FORMAT_PRETTY)
    assert codec.encode_size(cols.to_device(), pj.FORMAT_PRETTY) == len(orc.encode(cols, pj.FORMAT_PRETTY))


@pytest.mark.parametrize("seed", [0, 1])
def test_encode_pretty_inclusion_modes_match_oracle(codec, seed):
    cols = pj.generate(3, 20_000)
    rng = np.random.default_rng(seed)
    cols.arrays["flags"] = cols["flags"] & rng.integers(0, 64, cols.n_pets, dtype=np.uint8)
    cols.arrays["status"][rng.random(cols.n_pets) < 0.2] = pj.STATUS_NULL
    cols.arrays["tag_flags"] = rng.integers(0, 4, cols["tag_flags"].shape[0], dtype=np.uint8)
    cols.arrays["cat_flags"] = rng.integers(0, 4, cols.n_pets, dtype=np.uint8)
    for incl in (pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS):
        fields = {f: int(rng.integers(0, 3)) for f in pj.FIELDS if rng.random() < 0.5}
        assert gpu_encode(codec, cols, pj.FORMAT_PRETTY, incl, bool(seed), fields) == \
            orc.encode(cols, pj.FORMAT_PRETTY, incl, bool(seed), fields), (incl, fields)


def test_encode_pretty_flat_absent_groups_and_skew(codec):
    """The flat layout, absent column groups and records with long lists and
    long names (one thread still writes each record)."""
    cols = pj.generate(2, 30_000)
    assert gpu_encode(codec, cols, pj.FORMAT_PRETTY) == orc.encode(cols, pj.FORMAT_PRETTY)
    cols = pj.generate(3, 5_000)
    for g in ("photoUrls", "tags"):
        for k in GROUPS[g]:
            cols.arrays[k] = None
    assert gpu_encode(codec, cols, pj.FORMAT_PRETTY, pj.INCLUDE_ALWAYS) == \
        orc.encode(cols, pj.FORMAT_PRETTY, pj.INCLUDE_ALWAYS)
    cols = to_columns(_hybrid_pets())
    assert gpu_encode(codec, cols, pj.FORMAT_PRETTY) == orc.encode(cols, pj.FORMAT_PRETTY)


def test_encode_pretty_empty_single_and_capacity(codec):
    assert gpu_encode(codec, to_columns([]), pj.FORMAT_PRETTY) == b"[ ]"
    cols = pj.generate(3, 1)
    assert gpu_encode(codec, cols, pj.FORMAT_PRETTY) == orc.encode(cols, pj.FORMAT_PRETTY)
    cols = pj.generate(3, 10_000)
    d = cols.to_device()
    ref = np.frombuffer(orc.encode(cols, pj.FORMAT_PRETTY), np.uint8)
    out = torch.full((ref.size,), 0xEE, dtype=torch.uint8, device="cuda")
    cap = ref.size // 2
    with pytest.raises(pj.PetJsonError) as ei:
        codec.encode(d, pj.FORMAT_PRETTY, out=out[:cap])
    assert ei.value.status == pj.PJ_ERR_CAPACITY
    host = out.cpu().numpy()
    assert (host[cap:] == 0xEE).all()
    written = host[:cap] != 0xEE
    assert (host[:cap][written] == ref[:cap][written]).all()
    assert codec.encode_host(cols, pj.FORMAT_PRETTY) == ref.tobytes()


def test_encode_pretty_decodes_back_on_gpu(codec):
    """readValue of what the pretty writer produced: the array decoder gives
    the records the compact output gives."""
    cols = pj.generate(3, 40_000)
    data = torch.from_numpy(np.frombuffer(gpu_encode(codec, cols, pj.FORMAT_PRETTY), np.uint8).copy()).cuda()
    dec, el, ec, res = codec.decode(data, array=True)
    assert res.n_errors == 0 and res.n_pets == cols.n_pets
    dec = dec.to_host()
    _, ref, _, _, _ = orc.decode_array(orc.encode(cols, pj.FORMAT_ARRAY))
    for k in pj.COLS:
        if ref[k] is not None:
            assert np.array_equal(dec[k], ref[k]), k


# ----------------------------------------------------- findPetsByStatus body
@pytest.mark.parametrize("config,n", [(1, 60_000), (2, 100_000), (3, 50_000), (5, 8_000)])
def test_encode_by_status_matches_oracle(codec, config, n):
    print(f"[encode by status] config={config} n={n}", flush=True)
    cols = pj.generate(config, n)
    cols.arrays["status"][::11] = pj.STATUS_NULL
    d = cols.to_device()
    for mask in (1, 0b0101, 0b1000, 0xF, 0):
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
            got, m = codec.encode_by_status(d, mask, fmt)
            want, wm = orc.encode_by_status(cols, mask, fmt)
            assert m == wm and got.cpu().numpy().tobytes() == want, (mask, fmt)


def test_encode_by_status_capacity_and_no_status_column(codec):
    cols = pj.generate(3, 20_000)
    d = cols.to_device()
    want, _ = orc.encode_by_status(cols, 0b011, pj.FORMAT_ARRAY)
    ref = np.frombuffer(want, np.uint8)
    out = torch.full((ref.size,), 0xEE, dtype=torch.uint8, device="cuda")
    cap = ref.size // 3
    with pytest.raises(pj.PetJsonError) as ei:
        codec.encode_by_status(d, 0b011, pj.FORMAT_ARRAY, out=out[:cap])
    assert ei.value.status == pj.PJ_ERR_CAPACITY
    host = out.cpu().numpy()
    assert (host[cap:] == 0xEE).all()
    written = host[:cap] != 0xEE
    assert (host[:cap][written] == ref[:cap][written]).all()
    cols.arrays["status"] = None                   # no status column: every record has none
    d = cols.to_device()
    got, m = codec.encode_by_status(d, 0b1000, pj.FORMAT_ARRAY)
    assert m == cols.n_pets and got.cpu().numpy().tobytes() == orc.encode(cols, pj.FORMAT_ARRAY)
    got, m = codec.encode_by_status(d, 0b0111, pj.FORMAT_ARRAY)
    assert m == 0 and got.cpu().numpy().tobytes() == b"[]"


def test_encode_by_status_host_matches_oracle(codec):
    cols = pj.generate(3, 40_000)
    cols.arrays["status"][::5] = pj.STATUS_NULL
    for mask, fmt in ((1, pj.FORMAT_ARRAY), (0b1010, pj.FORMAT_PRETTY), (0xF, pj.FORMAT_NDJSON)):
        got, m = codec.encode_by_status_host(cols, mask, fmt)
        want, wm = orc.encode_by_status(cols, mask, fmt)
        assert m == wm and got == want, (mask, fmt)


def test_config1_gpu_output_matches_committed_digest(codec):
    """BASELINE configs[0] on the GPU hashes to the committed digests."""
    d = load("config1_digest.json")
    dev = pj.generate(1, d["records"]).to_device()
    for name, fmt in (("array", pj.FORMAT_ARRAY), ("ndjson", pj.FORMAT_NDJSON), ("pretty", pj.FORMAT_PRETTY)):
        b = codec.encode(dev, fmt).cpu().numpy().tobytes()
        assert len(b) == d["digests"][name]["bytes"]
        assert hashlib.sha256(b).hexdigest() == d["digests"][name]["sha256"], name


def _with_names(cols, lens, rng, esc_rate):
    """cols with its names replaced: lengths from lens (cycled), bytes drawn
    from letters, every byte that needs an escape and UTF-8 bytes."""
    n = cols.n_pets
    L = np.array([lens[i % len(lens)] for i in range(n)], np.uint64)
    off = np.zeros(n + 1, np.uint64)
    np.cumsum(L, out=off[1:])
    letters = np.frombuffer(b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789 ", np.uint8)
    special = np.array([0x22, 0x5C, 0x0A, 0x09, 0x08, 0x0C, 0x0D, 0x01, 0x1F, 0x1A, 0x00, 0x7F, 0xC3, 0xA9], np.uint8)
    tot = int(off[-1])
    b = rng.choice(letters, tot)
    hit = rng.random(tot) < esc_rate
    b[hit] = rng.choice(special, int(hit.sum()))
    cols.arrays["name_off"] = off
    cols.arrays["name_bytes"] = b
    return cols


@pytest.mark.parametrize("esc_rate", [0.0, 0.05, 0.3, 1.0])
def test_encode_long_names_written_by_waves(codec, esc_rate):
    """Names over 48 bytes in tile-path blocks have their escapes counted and
    their bodies written by a whole wave, 8 bytes per lane, in 512-byte
    steps: lengths around 48, 64 and 512, names past one step, null names
    whose bytes still sit in the column, escapes at every offset."""
    rng = np.random.default_rng(7 + int(esc_rate * 100))
    lens = [0, 3, 47, 48, 49, 50, 55, 56, 57, 63, 64, 65, 71, 72, 100, 200, 20, 33]
    cols = _with_names(pj.generate(3, 6_000), lens, rng, esc_rate)
    flags = cols["flags"].copy()
    flags[rng.random(cols.n_pets) < 0.05] &= ~np.uint8(pj.PET_HAS_NAME)
    cols.arrays["flags"] = flags
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
        ref = orc.encode(cols, fmt)
        assert codec.encode_size(cols.to_device(), fmt) == len(ref)
        assert gpu_encode(codec, cols, fmt) == ref, fmt
    # a few names of one and two 512-byte steps among short ones
    lens = [10] * 40 + [511, 512, 513, 700, 1023, 1024, 1025, 1100]
    cols = _with_names(pj.generate(3, 3_000), lens, rng, esc_rate)
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
        assert gpu_encode(codec, cols, fmt) == orc.encode(cols, fmt), fmt
