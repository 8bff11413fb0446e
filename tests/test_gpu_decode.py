"""GPU decode parity: libpetjson's NDJSON decode yields bit-identical columns,
error line indices and error codes to the CPU restatement on the same input:
hand-written known answers, generated records of every configuration with
seeded corruption, byte-level mutations, alignment and 64-byte block
boundary cases, and the round trip decode(encode(x)) == x."""
import random

import numpy as np
import pytest
import torch

import oracle_py as orc
import petjson as pj
from kat_util import expected_pet, line_bytes, load, norm_pet
from model import from_columns

pytestmark = pytest.mark.gpu


def gpu_decode(codec, data: bytes, shift=0, caps=None):
    buf = torch.zeros(len(data) + shift + 16, dtype=torch.uint8, device="cuda")
    if data:
        buf[shift: shift + len(data)] = torch.frombuffer(bytearray(data), dtype=torch.uint8).cuda()
    view = buf[shift: shift + len(data)]
    cols, el, ec, res = codec.decode(view, caps=caps)
    return cols.to_host(), el.cpu().numpy().astype(np.uint64), ec.cpu().numpy(), res


def assert_same(gpu, ref):
    gc, gel, gec, gres = gpu
    rc, rel, rec, rres = ref
    for f in ("n_lines", "n_pets", "n_errors", "name_bytes", "cat_name_bytes", "n_urls", "url_bytes", "n_tags",
              "tag_name_bytes"):
        assert getattr(gres, f) == getattr(rres, f), f
    assert np.array_equal(gel, rel) and np.array_equal(gec, rec)
    for k in pj.COLS:
        assert np.array_equal(gc[k], rc[k]), k


def test_decode_kat_each_line(codec):
    for case in load("decode_kat.json")["cases"]:
        line = line_bytes(case)
        cols, el, ec, res = gpu_decode(codec, line + b"\n")
        assert res.n_lines == 1, case["name"]
        if case["code"] == 0:
            assert res.n_errors == 0 and res.n_pets == 1, case["name"]
            got = from_columns(cols, as_bytes=True)[0]
            assert norm_pet(got) == norm_pet(expected_pet(case)), case["name"]
        else:
            assert list(ec) == [case["code"]], (case["name"], list(ec))


def test_decode_kat_file_matches_oracle(codec):
    lines = [line_bytes(c) for c in load("decode_kat.json")["cases"]]
    data = b"\n".join(lines)          # last line without a trailing newline
    assert_same(gpu_decode(codec, data), orc.decode(data))
    assert_same(gpu_decode(codec, data + b"\n"), orc.decode(data + b"\n"))


def test_depth_limit_gpu(codec):
    def nest(d):
        return ("{\"x\":" + "[" * (d - 1) + "]" * (d - 1) + ",\"name\":\"a\",\"photoUrls\":[]}").encode()
    mixed = ("{\"x\":" + "[{\"a\":" * 40 + "1" + "}]" * 40 + ",\"name\":\"a\",\"photoUrls\":[]}").encode()
    bad = ("{\"x\":" + "[{\"a\":" * 40 + "1" + "]}" * 40 + ",\"name\":\"a\",\"photoUrls\":[]}").encode()
    data = b"\n".join([nest(10), nest(64), nest(65), nest(200), nest(1000), nest(1001), mixed, bad]) + b"\n"
    assert_same(gpu_decode(codec, data), orc.decode(data))


@pytest.mark.parametrize("config,n", [(1, 20_000), (3, 30_000), (5, 4_000)])
def test_decode_roundtrip(codec, config, n):
    cols = pj.generate(config, n)
    text = orc.encode(cols, pj.FORMAT_NDJSON)
    gc, el, ec, res = gpu_decode(codec, text)
    assert res.n_errors == 0 and res.n_pets == n
    for k in pj.COLS:
        if cols[k] is not None:
            assert np.array_equal(gc[k], cols[k]), k


@pytest.mark.parametrize("shift", [0, 1, 3, 7, 13])
def test_decode_corrupted_matches_oracle(codec, shift):
    cols = pj.generate(3, 20_000, seed=0x5EED0004 + shift)
    buf = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), np.uint8).copy()
    lines, codes = pj.corrupt_ndjson(buf, 5 + shift, 0.01)
    data = buf.tobytes()
    ref = orc.decode(data)
    assert list(ref[1]) == list(lines)
    assert_same(gpu_decode(codec, data, shift=shift), ref)


def _mutate(rnd, line: bytes) -> bytes:
    b = bytearray(line)
    for _ in range(rnd.randrange(1, 4)):
        op = rnd.randrange(4)
        pos = rnd.randrange(len(b) + 1)
        if op == 0 and b:
            b[min(pos, len(b) - 1)] = rnd.choice(b'"\\{}[],:0aeu \t\x01\xc3\xa9\xff/\r')
        elif op == 1:
            b[pos:pos] = bytes([rnd.choice(b'"\\{}[],:0-.eE \x00\x1f\x80\xe2\xf0')])
        elif op == 2 and b:
            del b[min(pos, len(b) - 1)]
        else:
            b[pos:pos] = rnd.choice([b'\\u00e9', b'\\ud83d\\ude00', b'\\ud800', b'null', b',"x":[1,{}]', b'"', b'\\'])
    return bytes(b).replace(b"\n", b" ")


def test_decode_mutation_fuzz_matches_oracle(codec):
    rnd = random.Random(1234)
    base = orc.encode(pj.generate(3, 3000), pj.FORMAT_NDJSON).split(b"\n")[:-1]
    kat = [line_bytes(c) for c in load("decode_kat.json")["cases"]]
    lines = [_mutate(rnd, rnd.choice(base + kat)) for _ in range(30_000)]
    data = b"\n".join(lines) + b"\n"
    assert_same(gpu_decode(codec, data), orc.decode(data))


def test_decode_block_boundaries(codec):
    """Escapes, backslash runs, multi-byte UTF-8 and quotes placed across
    64-byte block edges, with blank and CRLF lines around them."""
    lines = []
    for pad in range(0, 70):
        for frag in ('\\\\\\"', '\\u00e9', 'é€😀', '\\\\', '\\"\\\\\\"'):
            name = "x" * pad + frag + "y"
            lines.append(('{"name":"%s","photoUrls":["%s"]}' % (name, frag)).encode())
    lines += [b"", b"\r", b'{"name":"a","photoUrls":[]}\r', b"   "]
    data = b"\n".join(lines) + b"\n"
    for shift in (0, 5):
        assert_same(gpu_decode(codec, data, shift=shift), orc.decode(data))


def test_decode_long_lines(codec):
    big = "a" * 70_000
    lines = [('{"name":"%s","photoUrls":["%s"]}' % (big, big[:1000])).encode(),
             ('{"name":"%s\\n","photoUrls":[]}' % big).encode(),
             ('{"name":"%s\t","photoUrls":[]}' % big).encode(),
             ('{"name":"%s' % big).encode()]
    data = b"\n".join(lines)
    assert_same(gpu_decode(codec, data), orc.decode(data))


def test_decode_empty_and_tiny(codec):
    for data in (b"", b"\n", b"\n\n", b"{", b'{"name":"a","photoUrls":[]}'):
        assert_same(gpu_decode(codec, data), orc.decode(data))


def test_decode_host_entry_point(codec):
    cols = pj.generate(3, 5000)
    text = orc.encode(cols, pj.FORMAT_NDJSON)
    assert_same(codec.decode_host(text), orc.decode(text))


def test_decode_capacity_error(codec):
    text = orc.encode(pj.generate(3, 1000), pj.FORMAT_NDJSON)
    caps = pj.decode_bounds(len(text))
    caps["cap_pets"] = 10
    with pytest.raises(pj.PetJsonError) as ei:
        gpu_decode(codec, text, caps=caps)
    assert ei.value.status == pj.PJ_ERR_CAPACITY


def test_decode_in_string_carry_reset_at_word_edge(codec):
    """A line ending inside an unterminated string, whose newline falls on
    every possible byte of a 64-byte word, followed by a line whose only
    fault (a stray UTF-8 continuation byte in a key) sits inside a string:
    the in-string state must restart at the newline."""
    victim = b'{"id":1,"catego\xa9y":{"id":2},"name":"x","photoUrls":[],"status":"sold","x":tru}'
    lines = []
    for k in range(0, 130):
        lines.append(b'{"name":"' + b"a" * k)          # unterminated string
        lines.append(victim)
    data = b"\n".join(lines) + b"\n"
    for shift in (0, 1, 9):
        assert_same(gpu_decode(codec, data, shift=shift), orc.decode(data))


def _insert_unknown(rnd, line: bytes) -> bytes:
    """Insert properties the Pet does not declare (and, now and then, known
    keys in a non-canonical shape) before a random top-level key."""
    vals = [b'"v"', b'""', b'"a\\"b\\u00e9"', b'0', b'-17', b'123456789012345678901234', b'true', b'false',
            b'null', b'1.5', b'{"a":1}', b'[1,2]', b'"\\q"', b'01', b'tru', b'"open']
    keys = [b'"x"', b'"idx"', b'"nam"', b'"names"', b'"category2"', b'"statusX"', b'"n\\u0061me"', b'"id"',
            b'"tags"', b'"\xc3\xa9"']
    # top-level key starts: after '{' or ',' at depth 1, outside strings
    starts, depth, instr, esc = [], 0, False, False
    for i, c in enumerate(line):
        if instr:
            if esc: esc = False
            elif c == 0x5C: esc = True
            elif c == 0x22: instr = False
            continue
        if c == 0x22:
            if depth == 1 and line[i - 1] in (0x7B, 0x2C): starts.append(i)
            instr = True
        elif c in (0x7B, 0x5B): depth += 1
        elif c in (0x7D, 0x5D): depth -= 1
    if not starts:
        return line
    at = rnd.choice(starts + [len(line) - 1])
    prop = rnd.choice(keys) + b":" + rnd.choice(vals)
    if at == len(line) - 1:
        return line[:at] + (b"," if line[at - 1] != 0x7B else b"") + prop + line[at:]
    return line[:at] + prop + b"," + line[at:]


def test_decode_unknown_properties_match_oracle(codec):
    rnd = random.Random(77)
    cols = pj.generate(3, 6000)
    lines = orc.encode(cols, pj.FORMAT_NDJSON).split(b"\n")[:-1]
    out = []
    for ln in lines:
        for _ in range(rnd.choice([0, 1, 1, 2, 3])):
            ln = _insert_unknown(rnd, ln)
        out.append(ln)
    data = b"\n".join(out) + b"\n"
    ref = orc.decode(data)
    assert ref[3].n_pets > 2000 and ref[3].n_errors > 200
    for shift in (0, 5):
        assert_same(gpu_decode(codec, data, shift=shift), ref)


def test_decode_null_after_value_writes_nothing(codec):
    """A property set and then nulled later in the line is absent: the
    writing pass must not copy the earlier value into the next record's
    slots."""
    lines = [b'{"name":"a","photoUrls":["u"],"tags":[{"id":1,"name":"t"}],"tags":null}',
             b'{"name":"b","photoUrls":[],"category":{"id":2,"name":"c"},"category":null}',
             b'{"name":"c","photoUrls":["x"],"photoUrls":null}',
             b'{"name":"d","photoUrls":["v"],"tags":[{"id":3,"name":"s"}],"category":{"id":4,"name":"k"}}']
    data = b"\n".join(lines * 50) + b"\n"
    assert_same(gpu_decode(codec, data), orc.decode(data))


def test_decode_blocks_over_the_tile(codec):
    """Blocks of lines whose bytes exceed one LDS tile are cut into several
    sub-tiles (and single lines longer than the tile read from global
    memory): skewed records with corruption, against the oracle."""
    cols = pj.generate(5, 12_000)
    text = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), dtype=np.uint8).copy()
    pj.corrupt_ndjson(text, 77, 0.01)
    data = text.tobytes()
    lens = np.diff(np.flatnonzero(text == 10))
    assert lens.max() > 8_000                       # the generator's long records are in
    ref = orc.decode(data)
    assert ref[3].n_errors > 50
    for shift in (0, 3):
        assert_same(gpu_decode(codec, data, shift=shift), ref)
    # every line as long as possible around the tile size (31 KiB; 40 KiB in
    # an earlier shape)
    big = [b'{"name":"' + b"x" * k + b'","photoUrls":[]}'
           for k in (31_680, 31_715, 31_744, 31_800, 40_900, 40_960, 41_000, 20_000, 39_000)]
    data2 = b"\n".join(big * 3) + b"\n"
    assert_same(gpu_decode(codec, data2), orc.decode(data2))


def _long_name(rnd, length, errors=False):
    frags = ["a", "b", "\\\\", "\\\"", "\\n", "\\t", "\\/", "\\u00e9", "\\u20AC", "\\u0001", "\\ud83d\\ude00",
             "\\\\\\\\\\\\", "é", "\U0001F600", "€"]
    bad = ["\\x", "\\u12G4", "\\ud800x", "\\udc00", "\\ud800\\u0041", "\\u00", "\\ud83d\\ud83d"]
    out, n = [], 0
    while n < length:
        f = rnd.choice(frags) if rnd.random() < 0.5 else "x" * rnd.randrange(1, 70)
        out.append(f)
        n += len(f.encode())
    if errors:
        out.insert(rnd.randrange(len(out) + 1), rnd.choice(bad))
    return "".join(out)


def test_decode_long_lines_wave_parallel(codec):
    """Lines longer than the per-thread limit are read by a whole wave, with
    long strings decoded lane-parallel: escapes, backslash runs and
    surrogate pairs at every offset around 64-byte words and 4 KiB steps,
    malformed escapes inside long strings, long URLs and tag names, and
    mutated long lines, against the oracle."""
    rnd = random.Random(99)
    lines = []
    for i in range(400):
        name = _long_name(rnd, rnd.choice([1100, 2000, 4090, 4100, 8200, 12000]), errors=i % 7 == 3)
        urls = ",".join('"%s"' % _long_name(rnd, rnd.randrange(10, 3000)) for _ in range(rnd.randrange(0, 3)))
        tags = ",".join('{"id":%d,"name":"%s"}' % (rnd.randrange(-9, 10**12), _long_name(rnd, rnd.randrange(1, 900)))
                        for _ in range(rnd.randrange(0, 40)))
        line = '{"id":%d,"name":"%s","photoUrls":[%s],"tags":[%s],"status":"sold"}' % (i, name, urls, tags)
        lines.append(line.encode())
    # backslash runs and pairs that end exactly at a word or step edge
    for pad in range(1100, 1100 + 130):
        for frag in ("\\\\", "\\\\\\\"", "\\ud83d\\ude00", "\\u00e9", "\\\""):
            lines.append(('{"name":"%s%s%s","photoUrls":[]}' % ("y" * pad, frag, "z" * 3000)).encode())
    for pad in range(4096 - 80, 4096 + 20, 3):
        lines.append(('{"name":"%s\\\\\\"\\ud83d\\ude00q","photoUrls":[]}' % ("y" * pad)).encode())
    mut = [_mutate(rnd, rnd.choice(lines[:400])) for _ in range(300)]
    data = b"\n".join(lines + mut + [b'{"name":"' + b"w" * 5000]) + b"\n"
    ref = orc.decode(data)
    assert ref[3].n_errors > 40
    for shift in (0, 11):
        assert_same(gpu_decode(codec, data, shift=shift), ref)


def test_decode_tape_full_lines_hand_over(codec):
    """Short lines with more url and tag words than a line's tape holds (27)
    go to the wave path: the bitmap-free validating pass defers them after
    writing part of their tape, also when such a line sits in a block's
    second sub-tile (blocks of 104 lines of about 400 bytes), and next to
    lines the general parser reads.  Against the oracle."""
    rnd = random.Random(7)

    def rec(i, nu, nt, pad):
        urls = ",".join('"u%d"' % k for k in range(nu))
        tags = ",".join('{"id":%d,"name":"t%d"}' % (k, k) for k in range(nt))
        return ('{"id":%d,"name":"%s","photoUrls":[%s],"tags":[%s],"status":"available"}'
                % (i, "n" * pad, urls, tags)).encode()

    lines = []
    for blk in range(48):
        full_at = {(blk * 37) % 104, (blk * 61 + 5) % 104} if blk % 3 else set()
        for j in range(104):
            if j in full_at:
                lines.append(rec(len(lines), rnd.choice([14, 20, 27]), rnd.choice([7, 12]), rnd.randrange(0, 40)))
            else:
                lines.append(rec(len(lines), rnd.randrange(0, 3), rnd.randrange(0, 3), 330 if blk % 2 else 20))
        if blk % 5 == 4:
            lines[-7] = b'{"name":"g", "photoUrls":[], "id":7}'      # the general parser (spaces)
    mut = [_mutate(rnd, lines[rnd.randrange(len(lines))]) for _ in range(200)]
    data = b"\n".join(lines + mut) + b"\n"
    ref = orc.decode(data)
    for shift in (0, 5):
        assert_same(gpu_decode(codec, data, shift=shift), ref)


def test_decode_deferred_lines_fix_offsets(codec):
    """Long lines deferred by the bitmap-free pass, at every kind of place in
    their blocks (first, last, several in a row, one per block, most of a
    block), and of every kind: valid, valid with escapes and many tags, a bad
    byte inside a string, a status outside the enum, whitespace the wave walk
    leaves to the general parser, longer than the tile, an unknown key.  The
    short lines after them take their offsets from k_dec_fixup; the error
    slots too.  Against the oracle, with the input at two alignments."""
    rnd = random.Random(11)

    def short(i):
        return ('{"id":%d,"name":"s%d","photoUrls":["p"],"tags":[{"id":%d,"name":"x"}],"status":"sold"}'
                % (i, i, i)).encode()

    def long_line(i, kind):
        name = "L" * rnd.randrange(1100, 4000)
        tags = ",".join('{"id":%d,"name":"t\\u00e9%d"}' % (k, k) for k in range(rnd.randrange(0, 60)))
        body = '"id":%d,"name":"%s","photoUrls":["a\\nb"],"tags":[%s],"status":"pending"' % (i, name, tags)
        if kind == 1:
            body = body.replace("LLLL", "L\x01LL", 1)                # a raw control byte in a string
        elif kind == 2:
            body = body.replace('"pending"', '"lost"')                # not in the enum
        elif kind == 3:
            body = body.replace('"tags":', '"tags" : ')              # whitespace: the general parser
        elif kind == 4:
            body = body.replace(name, "W" * 40000)                     # over the tile
        elif kind == 5:
            body = '"extra":{"k":[1,2,{"z":null}]},' + body           # an unknown key
        return ("{" + body + "}").encode()

    lines = []
    for blk in range(40):
        pat = blk % 5
        for j in range(104):
            i = len(lines)
            longp = (pat == 0 and j in (0, 103)) or (pat == 1 and 10 <= j < 14) or (pat == 2 and j == 50) \
                or (pat == 3 and j % 3 != 1)
            lines.append(long_line(i, rnd.randrange(6)) if longp else short(i))
    data = b"\n".join(lines) + b"\n"
    ref = orc.decode(data)
    assert ref[3].n_errors > 20
    for shift in (0, 7):
        assert_same(gpu_decode(codec, data, shift=shift), ref)


def test_roundtrip_beyond_4gib(codec):
    """16M nested records: the NDJSON passes 2^32 bytes, so every 64-bit
    offset path (line starts, column offsets, look-back sums) is exercised;
    decode(encode(x)) == x column for column, on the device."""
    n = 16_000_000
    cols = pj.generate(3, n)
    dev = cols.to_device()
    del cols
    text = codec.encode(dev, pj.FORMAT_NDJSON)
    assert text.numel() > 2 ** 32
    # the array framing of the same records: '[' + the lines joined by ',' + ']'
    arr = codec.encode(dev, pj.FORMAT_ARRAY)
    assert arr.numel() == text.numel() + 1
    assert arr[0].item() == ord("[") and arr[-1].item() == ord("]")
    body = text[:-1].clone()
    body[body == ord("\n")] = ord(",")
    assert torch.equal(arr[1:-1], body)
    del arr, body
    dcols, el, ec, res = codec.decode(text)
    assert res.n_lines == n and res.n_errors == 0 and res.n_pets == n
    for k in pj.COLS:
        if dev[k] is not None:
            assert torch.equal(dev[k].contiguous().view(torch.uint8), dcols[k].contiguous().view(torch.uint8)), k
    del text, dcols, dev
    torch.cuda.empty_cache()


def test_decode_without_line_tape(codec, monkeypatch):
    """The writing walk reads each line's tape (positions and values recorded
    by the validating walk); with the tape turned off it parses the line
    again.  Both give the oracle's columns."""
    monkeypatch.setenv("PETJSON_DECODE_TAPE", "0")
    cols = pj.generate(3, 40_000, seed=0x5EED0009)
    buf = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), np.uint8).copy()
    pj.corrupt_ndjson(buf, 11, 0.01)
    data = buf.tobytes()
    assert_same(gpu_decode(codec, data), orc.decode(data))
    skew = orc.encode(pj.generate(5, 4_000), pj.FORMAT_NDJSON)
    assert_same(gpu_decode(codec, skew), orc.decode(skew))


def test_decode_lookback_redo_in_ticket_order(codec, monkeypatch):
    """The index and parse kernels take blocks in launch order with bounded
    look-back waits; a kernel whose wait ran out is redone in ticket order.
    A one-tick bound forces that path: results still equal the oracle's."""
    monkeypatch.setenv("PETJSON_SPIN_LIMIT_TICKS", "1")
    cols = pj.generate(3, 60_000, seed=0x5EED0007)
    buf = np.frombuffer(orc.encode(cols, pj.FORMAT_NDJSON), np.uint8).copy()
    pj.corrupt_ndjson(buf, 9, 0.01)
    data = buf.tobytes()
    assert_same(gpu_decode(codec, data), orc.decode(data))
    skew = orc.encode(pj.generate(5, 6_000), pj.FORMAT_NDJSON)
    assert_same(gpu_decode(codec, skew), orc.decode(skew))


def test_decode_many_invalid_lines_retry_error_capacity(codec):
    """More invalid lines than the first error-list guess (one per 16 input
    bytes): both entry points retry with the count the call reported."""
    data = b"{}\n" * 1000 + b"\n" * 500 + b'{"name":"a","photoUrls":[]}\n'
    ref = orc.decode(data)
    assert ref[3].n_errors == 1500
    assert_same(gpu_decode(codec, data), ref)
    assert_same(codec.decode_host(data), ref)


def _sentinel_columns(caps, dev="cuda"):
    """Device columns of exactly the capacities (offset arrays cap + 1) with a
    64-byte 0xEE tail behind each, to catch stores past a capacity."""
    cp, cu, ct = caps["cap_pets"], caps["cap_urls"], caps["cap_tags"]
    sizes = {"id": cp, "flags": cp, "status": cp, "name_off": cp + 1, "name_bytes": caps["cap_name_bytes"],
             "cat_id": cp, "cat_flags": cp, "cat_name_off": cp + 1, "cat_name_bytes": caps["cap_cat_name_bytes"],
             "photo_off": cp + 1, "url_off": cu + 1, "url_bytes": caps["cap_url_bytes"], "tag_off": cp + 1,
             "tag_id": ct, "tag_flags": ct, "tag_name_off": ct + 1, "tag_name_bytes": caps["cap_tag_name_bytes"]}
    raw, arrays = {}, {}
    for k, v in sizes.items():
        isz = np.dtype(pj.DTYPES[k]).itemsize
        b = torch.full((v * isz + 64,), 0xEE, dtype=torch.uint8, device=dev)
        raw[k] = (b, v * isz)
        arrays[k] = b
    return pj.Columns(0, arrays, dict(caps)), raw


def test_decode_capacity_guard_no_store_past_cap(codec):
    """Each column capacity cut below what the input needs, in turn: the call
    reports PJ_ERR_CAPACITY and no byte behind any capacity is written."""
    cols = pj.generate(3, 3000)
    text = orc.encode(cols, pj.FORMAT_NDJSON)
    need = orc.decode(text)[3]
    full = {"cap_pets": need.n_pets, "cap_name_bytes": need.name_bytes, "cap_cat_name_bytes": need.cat_name_bytes,
            "cap_urls": need.n_urls, "cap_url_bytes": need.url_bytes, "cap_tags": need.n_tags,
            "cap_tag_name_bytes": need.tag_name_bytes}
    data = torch.frombuffer(bytearray(text), dtype=torch.uint8).cuda()
    for cut in [None] + list(full):
        for frac in ((0.5, 0.999) if cut else (1.0,)):
            caps = dict(full)
            if cut:
                caps[cut] = int(full[cut] * frac)
            dc, raw = _sentinel_columns(caps)
            el = torch.empty(16, dtype=torch.int64, device="cuda")
            ec = torch.empty(16, dtype=torch.uint8, device="cuda")
            if cut:
                with pytest.raises(pj.PetJsonError) as ei:
                    codec.decode(data, out=(dc, el, ec))
                assert ei.value.status == pj.PJ_ERR_CAPACITY, (cut, frac)
            else:
                codec.decode(data, out=(dc, el, ec))
            torch.cuda.synchronize()
            for k, (b, n) in raw.items():
                tail = b[n:].cpu().numpy()
                assert (tail == 0xEE).all(), (cut, frac, k)


def test_destroy_releases_device_memory():
    """A context that decoded (line tape, index, staging) gives all of its
    device memory back when destroyed."""
    cols = pj.generate(3, 200_000)
    text = orc.encode(cols, pj.FORMAT_NDJSON)
    data = torch.frombuffer(bytearray(text), dtype=torch.uint8).cuda()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        c = pj.Codec(0)
        c.decode_host(text[: len(text) // 4])
        out = c.decode(data)
        del out
        c.close()
        torch.cuda.synchronize()
    torch.cuda.empty_cache()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 >= free0 - (64 << 20), (free0, free1)


def _keep_rows(dev, keep):
    """The columns of `dev` (device tensors of a generated batch) restricted
    to the rows where `keep` is true: what a decode that drops those lines
    as invalid must produce."""
    i64 = lambda t: t.contiguous().view(torch.int64)  # offsets stay below 2^63
    exp = {k: dev[k][keep] for k in ("id", "flags", "status", "cat_id", "cat_flags")}

    def seg(off_key, data_key, keep_items):
        off = i64(dev[off_key])
        lens = off[1:] - off[:-1]
        data = dev[data_key][torch.repeat_interleave(keep_items, lens)]
        new_off = torch.cat([torch.zeros(1, dtype=torch.int64, device=off.device), torch.cumsum(lens[keep_items], 0)])
        return new_off, data, lens

    exp["name_off"], exp["name_bytes"], _ = seg("name_off", "name_bytes", keep)
    exp["cat_name_off"], exp["cat_name_bytes"], _ = seg("cat_name_off", "cat_name_bytes", keep)
    photo = i64(dev["photo_off"])
    nu = photo[1:] - photo[:-1]
    exp["photo_off"] = torch.cat([photo[:1] * 0, torch.cumsum(nu[keep], 0)])
    exp["url_off"], exp["url_bytes"], _ = seg("url_off", "url_bytes", torch.repeat_interleave(keep, nu))
    toff = i64(dev["tag_off"])
    nt = toff[1:] - toff[:-1]
    tkeep = torch.repeat_interleave(keep, nt)
    exp["tag_off"] = torch.cat([toff[:1] * 0, torch.cumsum(nt[keep], 0)])
    exp["tag_id"], exp["tag_flags"] = dev["tag_id"][tkeep], dev["tag_flags"][tkeep]
    exp["tag_name_off"], exp["tag_name_bytes"], _ = seg("tag_name_off", "tag_name_bytes", tkeep)
    return exp


def test_config5_full_size_roundtrip_and_corruption(codec):
    """BASELINE configs[4] at full size: 2M skewed records (log-normal
    names, 1% with 8-16 KiB names and 200 tags, 30% escape-heavy UTF-8 with
    4-byte code points).  The encode is byte-identical to the CPU checker in
    both framings (SHA-256); decode(encode(x)) == x column for column on the
    device; with 0.1% of the lines corrupted, the error lines and codes equal
    the generator's list and every other line decodes to its record."""
    import hashlib
    n = 2_000_000
    cols = pj.generate(5, n)
    sz = cols.sizes()
    dev = cols.to_device()
    nd = None
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
        print(f"[config5 full] encode fmt={fmt}", flush=True)
        gpu = codec.encode(dev, fmt).cpu().numpy()
        ref = orc.encode(cols, fmt)
        assert gpu.size == len(ref)
        assert hashlib.sha256(gpu.tobytes()).hexdigest() == hashlib.sha256(ref).hexdigest(), fmt
        del ref
        if fmt == pj.FORMAT_NDJSON:
            nd = gpu.copy()
    del cols
    caps = {"cap_pets": n, "cap_name_bytes": sz["name_bytes"], "cap_cat_name_bytes": sz["cat_name_bytes"],
            "cap_urls": sz["n_urls"], "cap_url_bytes": sz["url_bytes"], "cap_tags": sz["n_tags"],
            "cap_tag_name_bytes": sz["tag_name_bytes"]}
    print("[config5 full] round trip", flush=True)
    dcols, el, ec, res = codec.decode(torch.from_numpy(nd).cuda(), caps=caps, err_cap=16)
    assert res.n_lines == n and res.n_errors == 0 and res.n_pets == n
    for k in pj.COLS:
        assert torch.equal(dcols[k].contiguous().view(torch.uint8), dev[k].contiguous().view(torch.uint8)), k
    del dcols
    print("[config5 full] corrupted", flush=True)
    lines, codes = pj.corrupt_ndjson(nd, 0x5EED5, 0.001)
    assert len(lines) > 1_000
    dcols, el, ec, res = codec.decode(torch.from_numpy(nd).cuda(), caps=caps, err_cap=2 * len(lines))
    assert res.n_lines == n and res.n_errors == len(lines) and res.n_pets == n - len(lines)
    assert np.array_equal(el.cpu().numpy().astype(np.uint64), lines)
    assert np.array_equal(ec.cpu().numpy(), codes)
    keep = torch.ones(n, dtype=torch.bool, device="cuda")
    keep[torch.from_numpy(lines.astype(np.int64)).cuda()] = False
    exp = _keep_rows(dev, keep)
    for k, v in exp.items():
        assert torch.equal(dcols[k].contiguous().view(torch.uint8), v.contiguous().view(torch.uint8)), k
    del dcols, dev, exp
    torch.cuda.empty_cache()


def test_config4_full_size_with_corruption(codec):
    """BASELINE configs[3] at full size: ~4 GB of NDJSON from 14.6M nested
    records with 0.1% of lines corrupted (missing name, unknown status,
    truncated string).  The error line indices and codes equal the
    generator's own list of what it corrupted, and every valid line decodes
    to its original record (the columns equal the generated ones with the
    corrupted rows removed), checked on the device."""
    n = 14_600_000
    cols = pj.generate(4, n)
    sz = cols.sizes()
    dev = cols.to_device()
    del cols
    host = codec.encode(dev, pj.FORMAT_NDJSON).cpu().numpy().copy()
    lines, codes = pj.corrupt_ndjson(host, 0xBAD, 0.001)
    assert len(lines) > 10_000
    data = torch.from_numpy(host).cuda()
    del host
    caps = {"cap_pets": n, "cap_name_bytes": sz["name_bytes"], "cap_cat_name_bytes": sz["cat_name_bytes"],
            "cap_urls": sz["n_urls"], "cap_url_bytes": sz["url_bytes"], "cap_tags": sz["n_tags"],
            "cap_tag_name_bytes": sz["tag_name_bytes"]}
    dcols, el, ec, res = codec.decode(data, caps=caps, err_cap=2 * len(lines))
    assert res.n_lines == n and res.n_errors == len(lines) and res.n_pets == n - len(lines)
    assert np.array_equal(el.cpu().numpy().astype(np.uint64), lines)
    assert np.array_equal(ec.cpu().numpy(), codes)
    del data
    keep = torch.ones(n, dtype=torch.bool, device="cuda")
    keep[torch.from_numpy(lines.astype(np.int64)).cuda()] = False
    exp = _keep_rows(dev, keep)
    for k, v in exp.items():
        got = dcols[k].contiguous().view(torch.uint8)
        assert torch.equal(got, v.contiguous().view(torch.uint8)), k
    del dcols, dev, exp
    torch.cuda.empty_cache()
