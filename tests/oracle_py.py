"""ctypes binding of the CPU restatement (oracle/liboracle.so).

Test infrastructure: used by tests/ as the checker and by bench.py's
cpu_baseline leg only.
"""
import ctypes as C
import os
import subprocess

import numpy as np

import petjson as pj

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "oracle", "liboracle.so")
_L = None


def lib():
    global _L
    if _L is None:
        if not os.path.exists(SO):
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        L = C.CDLL(SO)
        L.or_encode.argtypes = [C.POINTER(pj.PetColumnsStruct), C.POINTER(pj.Options), C.c_int, C.c_void_p,
                                C.c_uint64, C.POINTER(C.c_uint64)]
        L.or_decode.argtypes = [C.c_void_p, C.c_uint64, C.POINTER(pj.PetColumnsStruct), C.c_void_p, C.c_void_p,
                                C.c_uint64, C.POINTER(pj.DecodeResult)]
        L.or_decode_line.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]
        L.or_decode_array.argtypes = L.or_decode.argtypes
        L.or_format_long.argtypes = [C.c_int64, C.c_char_p]
        L.or_encode_by_status.argtypes = [C.POINTER(pj.PetColumnsStruct), C.POINTER(pj.Options), C.c_uint32, C.c_int,
                                          C.c_void_p, C.c_uint64, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
        L.or_encode_model.argtypes = [C.c_int, C.POINTER(pj.ModelColumnsStruct), C.POINTER(pj.Options), C.c_int,
                                      C.c_void_p, C.c_uint64, C.POINTER(C.c_uint64)]
        L.or_decode_model.argtypes = [C.c_int, C.c_void_p, C.c_uint64, C.c_int, C.POINTER(pj.ModelColumnsStruct),
                                      C.c_void_p, C.c_void_p, C.c_uint64, C.POINTER(pj.DecodeResult)]
        _L = L
    return _L


def encode(cols: pj.Columns, fmt=pj.FORMAT_ARRAY, inclusion=pj.INCLUDE_NON_EMPTY, hex_upper=True, fields=None) -> bytes:
    L = lib()
    s = cols.struct()
    o = pj.make_options(inclusion, hex_upper, fields)
    n = C.c_uint64(0)
    L.or_encode(C.byref(s), C.byref(o), fmt, None, 0, C.byref(n))
    out = np.empty(max(1, n.value), dtype=np.uint8)
    rc = L.or_encode(C.byref(s), C.byref(o), fmt, C.c_void_p(out.ctypes.data), out.size, C.byref(n))
    assert rc == 0
    return out[: n.value].tobytes()


def alloc_decode_columns(caps):
    """Host numpy column set sized by `caps` (dict of cap_* values)."""
    cp = caps["cap_pets"]
    arrays = {
        "id": np.zeros(cp, np.int64), "flags": np.zeros(cp, np.uint8), "status": np.zeros(cp, np.uint8),
        "name_off": np.zeros(cp + 1, np.uint64), "name_bytes": np.zeros(max(1, caps["cap_name_bytes"]) + 4, np.uint8),
        "cat_id": np.zeros(cp, np.int64), "cat_flags": np.zeros(cp, np.uint8),
        "cat_name_off": np.zeros(cp + 1, np.uint64),
        "cat_name_bytes": np.zeros(max(1, caps["cap_cat_name_bytes"]) + 4, np.uint8),
        "photo_off": np.zeros(cp + 1, np.uint64), "url_off": np.zeros(caps["cap_urls"] + 1, np.uint64),
        "url_bytes": np.zeros(max(1, caps["cap_url_bytes"]) + 4, np.uint8),
        "tag_off": np.zeros(cp + 1, np.uint64), "tag_id": np.zeros(max(1, caps["cap_tags"]), np.int64),
        "tag_flags": np.zeros(max(1, caps["cap_tags"]), np.uint8),
        "tag_name_off": np.zeros(caps["cap_tags"] + 1, np.uint64),
        "tag_name_bytes": np.zeros(max(1, caps["cap_tag_name_bytes"]) + 4, np.uint8),
    }
    return pj.Columns(0, arrays, dict(caps))


def trim(cols: pj.Columns, res) -> pj.Columns:
    """Cut a decoded column set down to the sizes in a DecodeResult."""
    a = cols.to_host().arrays
    n, nu, nt = res.n_pets, res.n_urls, res.n_tags
    out = {
        "id": a["id"][:n], "flags": a["flags"][:n], "status": a["status"][:n],
        "name_off": a["name_off"][: n + 1], "name_bytes": a["name_bytes"][: res.name_bytes],
        "cat_id": a["cat_id"][:n], "cat_flags": a["cat_flags"][:n], "cat_name_off": a["cat_name_off"][: n + 1],
        "cat_name_bytes": a["cat_name_bytes"][: res.cat_name_bytes], "photo_off": a["photo_off"][: n + 1],
        "url_off": a["url_off"][: nu + 1], "url_bytes": a["url_bytes"][: res.url_bytes],
        "tag_off": a["tag_off"][: n + 1], "tag_id": a["tag_id"][:nt], "tag_flags": a["tag_flags"][:nt],
        "tag_name_off": a["tag_name_off"][: nt + 1], "tag_name_bytes": a["tag_name_bytes"][: res.tag_name_bytes],
    }
    return pj.Columns(n, {k: np.ascontiguousarray(v) for k, v in out.items()})


def decode(data: bytes, caps=None):
    """Returns (columns trimmed to size, error lines, error codes, result)."""
    L = lib()
    buf = np.frombuffer(data, dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    if caps is None:
        caps = pj.decode_bounds(len(data)) if pj._LIB is not None or os.path.exists(pj.lib_path()) else None
    if caps is None:
        n = len(data)
        caps = {"cap_pets": n // 27 + 1, "cap_name_bytes": n, "cap_cat_name_bytes": n, "cap_urls": n // 3 + 1,
                "cap_url_bytes": n, "cap_tags": n // 3 + 1, "cap_tag_name_bytes": n}
    cols = alloc_decode_columns(caps)
    s = cols.struct()
    nl = data.count(b"\n") + 1
    el = np.zeros(nl, np.uint64)
    ec = np.zeros(nl, np.uint8)
    res = pj.DecodeResult()
    rc = L.or_decode(C.c_void_p(buf.ctypes.data), len(data), C.byref(s), C.c_void_p(el.ctypes.data),
                     C.c_void_p(ec.ctypes.data), nl, C.byref(res))
    assert rc == 0, rc
    return trim(cols, res), el[: res.n_errors].copy(), ec[: res.n_errors].copy(), res


def decode_array(data: bytes, caps=None):
    """One array document.  Returns (status, columns trimmed to size, error
    element indices, error codes, result); status is pj.PJ_OK or
    pj.PJ_ERR_SYNTAX (a broken frame: columns and lists then empty)."""
    L = lib()
    buf = np.frombuffer(data, dtype=np.uint8) if len(data) else np.zeros(1, np.uint8)
    if caps is None:
        caps = pj.decode_bounds(len(data)) if pj._LIB is not None or os.path.exists(pj.lib_path()) else None
    if caps is None:
        n = len(data)
        caps = {"cap_pets": n // 27 + 1, "cap_name_bytes": n, "cap_cat_name_bytes": n, "cap_urls": n // 3 + 1,
                "cap_url_bytes": n, "cap_tags": n // 3 + 1, "cap_tag_name_bytes": n}
    cols = alloc_decode_columns(caps)
    s = cols.struct()
    ne = data.count(b",") + 2
    el = np.zeros(ne, np.uint64)
    ec = np.zeros(ne, np.uint8)
    res = pj.DecodeResult()
    rc = L.or_decode_array(C.c_void_p(buf.ctypes.data), len(data), C.byref(s), C.c_void_p(el.ctypes.data),
                           C.c_void_p(ec.ctypes.data), ne, C.byref(res))
    assert rc in (pj.PJ_OK, pj.PJ_ERR_SYNTAX), rc
    if rc != pj.PJ_OK:
        res = pj.DecodeResult()
    return rc, trim(cols, res), el[: res.n_errors].copy(), ec[: res.n_errors].copy(), res


def decode_line_code(line: bytes) -> int:
    buf = np.frombuffer(line, dtype=np.uint8) if line else np.zeros(1, np.uint8)
    return lib().or_decode_line(C.c_void_p(buf.ctypes.data), len(line), None, None)


def format_long(v: int) -> str:
    b = C.create_string_buffer(32)
    n = lib().or_format_long(v, b)
    return b.raw[:n].decode()


def encode_model(cols: "pj.ModelColumns", fmt=pj.FORMAT_ARRAY, inclusion=pj.INCLUDE_NON_EMPTY, hex_upper=True) -> bytes:
    """Order / User records (host columns) through the CPU restatement."""
    L = lib()
    s = cols.struct()
    o = pj.make_options(inclusion, hex_upper)
    n = C.c_uint64(0)
    L.or_encode_model(cols.model, C.byref(s), C.byref(o), fmt, None, 0, C.byref(n))
    out = np.empty(max(1, n.value), dtype=np.uint8)
    rc = L.or_encode_model(cols.model, C.byref(s), C.byref(o), fmt, C.c_void_p(out.ctypes.data), out.size,
                           C.byref(n))
    assert rc == 0
    return out[: n.value].tobytes()


def decode_model(model: int, data: bytes, array=False):
    """Returns (status, host columns trimmed to size, error indices, error
    codes, result)."""
    L = lib()
    n = len(data)
    buf = np.frombuffer(data, dtype=np.uint8) if n else np.zeros(1, np.uint8)
    cap_bytes = [n] * pj.MODEL_MAX_PROPS
    cols = pj.alloc_model_columns(model, n // 3 + 1, cap_bytes)
    s = cols.struct()
    ne = n + 1
    el = np.zeros(ne, np.uint64)
    ec = np.zeros(ne, np.uint8)
    res = pj.DecodeResult()
    rc = L.or_decode_model(model, C.c_void_p(buf.ctypes.data), n, int(array), C.byref(s),
                           C.c_void_p(el.ctypes.data), C.c_void_p(ec.ctypes.data), ne, C.byref(res))
    assert rc in (pj.PJ_OK, pj.PJ_ERR_SYNTAX), rc
    cols.n = int(s.n) if rc == pj.PJ_OK else 0
    cols.n_bytes = [int(s.n_bytes[k]) for k in range(pj.MODEL_MAX_PROPS)]
    if rc != pj.PJ_OK:
        res = pj.DecodeResult()
    return rc, cols.to_host(), el[: res.n_errors].copy(), ec[: res.n_errors].copy(), res


def encode_by_status(cols: pj.Columns, mask: int, fmt=pj.FORMAT_ARRAY, inclusion=pj.INCLUDE_NON_EMPTY):
    """(bytes, selected count) of the records whose status is in mask."""
    L = lib()
    s = cols.struct()
    o = pj.make_options(inclusion, True)
    n, m = C.c_uint64(0), C.c_uint64(0)
    L.or_encode_by_status(C.byref(s), C.byref(o), mask, fmt, None, 0, C.byref(n), C.byref(m))
    out = np.empty(max(1, n.value), dtype=np.uint8)
    rc = L.or_encode_by_status(C.byref(s), C.byref(o), mask, fmt, C.c_void_p(out.ctypes.data), out.size,
                               C.byref(n), C.byref(m))
    assert rc == 0
    return out[: n.value].tobytes(), m.value
