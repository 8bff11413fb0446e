"""The C-ABI library loads and exports every function include/*.h declares
(no compute calls: this runs without a GPU)."""
import ctypes
import glob
import os
import re

import petjson as pj

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"^[A-Za-z_][\w \*]*?\b(pj_\w+)\s*\(", txt, flags=re.M))
    return names


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert set(pj.EXPORTS) <= names, set(pj.EXPORTS) - names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(pj.lib_path())
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_load_lib_sets_signatures():
    L = pj.load_lib()
    assert L.pj_last_error.restype is ctypes.c_char_p


def test_decode_bounds_are_safe_upper_bounds():
    b = pj.decode_bounds(1000)
    assert b["cap_pets"] >= 1000 // 27 and b["cap_name_bytes"] == 1000 and b["cap_urls"] >= 333
