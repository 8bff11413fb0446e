"""GPU array-document decode parity (pj_decode_array_device / _host):
status, element error indices and codes, and columns bit-identical to the
CPU restatement (or_decode_array) on the same documents: the frame cases,
round trips of encoded arrays of every configuration, indented documents
(newlines inside elements), separators and string bytes placed around the
64-byte words and the 64 KiB blocks of the frame scan, byte mutations, and
a document of a million records."""
import random

import numpy as np
import pytest
import torch

import oracle_py as orc
import petjson as pj
from array_util import FRAME_CASES, join_array, mutate_doc, pretty, record_texts

pytestmark = pytest.mark.gpu


def gpu_array(codec, doc: bytes, shift=0):
    buf = torch.zeros(len(doc) + shift + 16, dtype=torch.uint8, device="cuda")
    if doc:
        buf[shift: shift + len(doc)] = torch.frombuffer(bytearray(doc), dtype=torch.uint8).cuda()
    try:
        cols, el, ec, res = codec.decode_array(buf[shift: shift + len(doc)])
    except pj.PetJsonError as e:
        assert e.status == pj.PJ_ERR_SYNTAX, e
        return pj.PJ_ERR_SYNTAX, None, None, None, None
    return pj.PJ_OK, cols.to_host(), el.cpu().numpy().astype(np.uint64), ec.cpu().numpy(), res


def assert_same(doc, gpu, ref):
    rc, gc, gel, gec, gres = gpu
    rrc, rc_, rel, rec, rres = ref
    assert rc == rrc, doc[:200]
    if rc != pj.PJ_OK:
        return
    for f in ("n_lines", "n_pets", "n_errors", "name_bytes", "cat_name_bytes", "n_urls", "url_bytes", "n_tags",
              "tag_name_bytes"):
        assert getattr(gres, f) == getattr(rres, f), (f, doc[:200])
    assert np.array_equal(gel, rel) and np.array_equal(gec, rec), doc[:200]
    for k in pj.COLS:
        assert np.array_equal(gc[k], rc_[k]), (k, doc[:200])


@pytest.mark.parametrize("doc,status,n", FRAME_CASES, ids=[repr(c[0][:24]) for c in FRAME_CASES])
def test_array_frame_cases_gpu(codec, doc, status, n):
    got = gpu_array(codec, doc)
    assert got[0] == status
    if status == pj.PJ_OK:
        assert got[4].n_lines == n
    assert_same(doc, got, orc.decode_array(doc))


@pytest.mark.parametrize("config", [1, 2, 3, 5])
def test_array_roundtrip_gpu(codec, config):
    cols = pj.generate(config, 20_000 if config != 5 else 4_000)
    dev = cols.to_device()
    arr = codec.encode(dev, pj.FORMAT_ARRAY)
    dcols, el, ec, res = codec.decode_array(arr)
    assert res.n_errors == 0 and res.n_pets == cols.n_pets
    for k in pj.COLS:
        if dev[k] is not None:
            assert torch.equal(dev[k].contiguous().view(torch.uint8), dcols[k].contiguous().view(torch.uint8)), k
    doc = arr.cpu().numpy().tobytes()
    assert_same(doc, gpu_array(codec, doc), orc.decode_array(doc))


def test_array_deferred_long_elements(codec):
    """Elements over 1 KiB among short ones, so the validating pass defers
    them to the one-wave kernels: valid ones (escapes, many tags), a raw
    control byte in a string, a status outside the enum, whitespace the
    wave walk leaves to the general parser, one longer than the tile.  The
    separators around them vary.  Against the oracle."""
    rnd = random.Random(23)

    def elem(i):
        if rnd.random() < 0.8:
            return ('{"id":%d,"name":"s%d","photoUrls":[],"status":"sold"}' % (i, i)).encode()
        kind = rnd.randrange(5)
        name = "N" * rnd.randrange(1100, 3000)
        tags = ",".join('{"id":%d,"name":"t\\t%d"}' % (k, k) for k in range(rnd.randrange(0, 40)))
        body = '"id":%d,"name":"%s","photoUrls":["x"],"tags":[%s],"status":"available"' % (i, name, tags)
        if kind == 1:
            body = body.replace("NNNN", "N\x02NN", 1)
        elif kind == 2:
            body = body.replace('"available"', '"gone"')
        elif kind == 3:
            body = body.replace('"photoUrls":', '"photoUrls" :')
        elif kind == 4:
            body = body.replace(name, "Z" * 36000)
        return ("{" + body + "}").encode()

    doc = join_array([elem(i) for i in range(700)], rnd)
    ref = orc.decode_array(doc)
    assert ref[0] == pj.PJ_OK and ref[4].n_errors > 10
    for shift in (0, 3):
        assert_same(doc, gpu_array(codec, doc, shift=shift), ref)


def test_array_host_entry_point(codec):
    doc = orc.encode(pj.generate(3, 3000), pj.FORMAT_ARRAY)
    cols, el, ec, res = codec.decode_array_host(doc)
    rrc, rc_, rel, rec, rres = orc.decode_array(doc)
    assert res.n_pets == rres.n_pets == 3000
    for k in pj.COLS:
        assert np.array_equal(cols[k], rc_[k]), k
    with pytest.raises(pj.PetJsonError) as e:
        codec.decode_array_host(doc[:-1])
    assert e.value.status == pj.PJ_ERR_SYNTAX


def test_array_indented_and_spaced(codec):
    rnd = random.Random(11)
    for rep in range(6):
        texts = record_texts(3, 300, seed=0x5EED0100 + rep)
        doc = join_array([pretty(t, rnd) for t in texts], rnd)
        assert_same(doc, gpu_array(codec, doc, shift=rep % 5), orc.decode_array(doc))


def test_array_separators_around_words_and_blocks(codec):
    """Elements padded so that commas, quotes, backslash runs and brackets
    inside strings land on every offset around 64-byte words and around the
    frame scan's 64 KiB blocks."""
    rnd = random.Random(5)
    base = record_texts(3, 64, seed=0x5EED0200)
    for pad in range(0, 70, 3):
        elems = []
        for j, t in enumerate(base):
            fill = b" " * ((pad + j) % 67)
            s = [b'"a,b]', b'"\\\\\\"[', b'"{}', b'"\\\\"', b'"x'][j % 5]
            elems.append(fill + t[:-1] + b',"z":' + s + b'"}')
        doc = b"[" + b",".join(elems) + b"]"
        assert_same(doc, gpu_array(codec, doc), orc.decode_array(doc))
    # around 64 KiB blocks: one big document, elements of ragged sizes
    texts = record_texts(3, 2000, seed=0x5EED0300)
    doc = join_array([b" " * rnd.randrange(0, 200) + t for t in texts], rnd)
    assert len(doc) > 3 * 65536
    for shift in (0, 7):
        assert_same(doc, gpu_array(codec, doc, shift=shift), orc.decode_array(doc))


@pytest.mark.parametrize("seed", range(40))
def test_array_mutations_match_oracle(codec, seed):
    rnd = random.Random(0xA11A + seed)
    texts = record_texts(3, 200, seed=0x5EED0400 + seed % 4)
    elems = [rnd.choice(texts) for _ in range(rnd.randrange(0, 60))]
    if seed % 3 == 0:
        elems = [pretty(e, rnd) for e in elems]
    doc = join_array(elems, rnd)
    for _ in range(5):
        m = mutate_doc(rnd, doc)
        assert_same(m, gpu_array(codec, m), orc.decode_array(m))


def test_array_million_records(codec):
    n = 1_000_000
    cols = pj.generate(3, n)
    dev = cols.to_device()
    arr = codec.encode(dev, pj.FORMAT_ARRAY)
    dcols, el, ec, res = codec.decode_array(arr)
    assert res.n_lines == n and res.n_errors == 0 and res.n_pets == n
    for k in pj.COLS:
        assert torch.equal(dev[k].contiguous().view(torch.uint8), dcols[k].contiguous().view(torch.uint8)), k
