"""ctypes binding of libpetjson (include/petjson.h) and of the record generator.

Host columns are numpy arrays; device columns are torch tensors on the
context's GPU (torch is only the device allocator here).  The product path
always runs the gfx950 kernels of libpetjson.so: when that library is missing
or no gfx950 device is present the calls raise, they never fall back to CPU.

Reference interface mirrored: io.micronaut.serde.ObjectMapper
(reference src/main/java/com/micronaut/bug/config/MyEntityConfig.java:8,34 and
service/MyEntityService.java:45) — see ``mapper.py`` for the object surface.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)

# ----------------------------------------------------------------- constants
PJ_OK, PJ_ERR_INVALID_ARG, PJ_ERR_CAPACITY, PJ_ERR_DEVICE, PJ_ERR_NO_DEVICE, PJ_ERR_OUT_OF_MEMORY, \
    PJ_ERR_SYNTAX = range(7)
STATUS_NAMES = {0: "PJ_OK", 1: "PJ_ERR_INVALID_ARG", 2: "PJ_ERR_CAPACITY", 3: "PJ_ERR_DEVICE",
                4: "PJ_ERR_NO_DEVICE", 5: "PJ_ERR_OUT_OF_MEMORY", 6: "PJ_ERR_SYNTAX"}
FORMAT_ARRAY, FORMAT_NDJSON, FORMAT_PRETTY = 0, 1, 2
INCLUDE_NON_EMPTY, INCLUDE_NON_NULL, INCLUDE_ALWAYS = 0, 1, 2
STATUS_AVAILABLE, STATUS_PENDING, STATUS_SOLD, STATUS_NULL = 0, 1, 2, 255
PET_HAS_ID, PET_HAS_CATEGORY, PET_HAS_NAME, PET_HAS_PHOTOURLS, PET_HAS_TAGS = 1, 2, 4, 8, 16
PET_DEFAULT_FLAGS = PET_HAS_ID | PET_HAS_NAME | PET_HAS_PHOTOURLS
SUB_HAS_ID, SUB_HAS_NAME = 1, 2
SUB_DEFAULT_FLAGS = SUB_HAS_ID | SUB_HAS_NAME
REC_OK, REC_SYNTAX, REC_STRING, REC_NUMBER, REC_TYPE, REC_MISSING_NAME, REC_MISSING_PHOTOURLS, \
    REC_BAD_STATUS, REC_DEPTH, REC_EMPTY = range(10)
MAX_DEPTH = 1000
SEED_BASE = 0x5EED0000

COLS = ["id", "flags", "status", "name_off", "name_bytes", "cat_id", "cat_flags", "cat_name_off",
        "cat_name_bytes", "photo_off", "url_off", "url_bytes", "tag_off", "tag_id", "tag_flags",
        "tag_name_off", "tag_name_bytes"]
DTYPES = {"id": np.int64, "flags": np.uint8, "status": np.uint8, "name_off": np.uint64,
          "name_bytes": np.uint8, "cat_id": np.int64, "cat_flags": np.uint8, "cat_name_off": np.uint64,
          "cat_name_bytes": np.uint8, "photo_off": np.uint64, "url_off": np.uint64, "url_bytes": np.uint8,
          "tag_off": np.uint64, "tag_id": np.int64, "tag_flags": np.uint8, "tag_name_off": np.uint64,
          "tag_name_bytes": np.uint8}
CAPS = ["cap_pets", "cap_name_bytes", "cap_cat_name_bytes", "cap_urls", "cap_url_bytes", "cap_tags",
        "cap_tag_name_bytes"]


class PetColumnsStruct(C.Structure):
    _fields_ = [("n_pets", C.c_uint64)] + [(n, C.c_void_p) for n in COLS] + [(n, C.c_uint64) for n in CAPS]


# optional properties with an inclusion mode of their own (pj_field)
FIELDS = ("pet_id", "pet_category", "pet_tags", "pet_status", "category_id", "category_name", "tag_id", "tag_name")
INCLUDE_DEFAULT = -1


class Options(C.Structure):
    _fields_ = [("inclusion", C.c_int32), ("hex_upper", C.c_int32), ("field_inclusion", C.c_int32 * len(FIELDS))]


def make_options(inclusion=0, hex_upper=True, fields=None) -> "Options":
    """pj_options: the mapper-wide inclusion mode, the hex case, and per-property
    modes {field name: mode} that override it (the rest follow `inclusion`)."""
    per = [INCLUDE_DEFAULT] * len(FIELDS)
    for k, m in (fields or {}).items():
        per[FIELDS.index(k)] = int(m)
    return Options(inclusion, 1 if hex_upper else 0, (C.c_int32 * len(FIELDS))(*per))


class DecodeResult(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("n_lines", "n_pets", "n_errors", "name_bytes", "cat_name_bytes",
                                          "n_urls", "url_bytes", "n_tags", "tag_name_bytes", "n_general")]


class PetJsonError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


# -------------------------------------------------------------------- loader
# ------------------------------------------------ Order and User models
MODEL_ORDER, MODEL_USER = 1, 2
MODEL_MAX_PROPS = 8
# property name and kind, in schema order (petstore.json:937-971 Order,
# :824-857 User)
MODEL_PROPS = {
    MODEL_ORDER: (("id", "i64"), ("petId", "i64"), ("quantity", "i32"), ("shipDate", "str"), ("status", "enum"),
                  ("complete", "bool")),
    MODEL_USER: (("id", "i64"), ("username", "str"), ("firstName", "str"), ("lastName", "str"), ("email", "str"),
                 ("password", "str"), ("phone", "str"), ("userStatus", "i32")),
}
ORDER_STATUS = ("placed", "approved", "delivered")
KIND_DTYPE = {"i64": np.int64, "i32": np.int32, "enum": np.uint8, "bool": np.uint8, "str": np.uint64}


class ModelColumnsStruct(C.Structure):
    _fields_ = [("n", C.c_uint64), ("present", C.c_void_p), ("col", C.c_void_p * MODEL_MAX_PROPS),
                ("bytes", C.c_void_p * MODEL_MAX_PROPS), ("cap_n", C.c_uint64),
                ("cap_bytes", C.c_uint64 * MODEL_MAX_PROPS), ("n_bytes", C.c_uint64 * MODEL_MAX_PROPS)]


_LIB = None
_GEN = None

EXPORTS = ["pj_create", "pj_destroy", "pj_default_options", "pj_set_options", "pj_last_error",
           "pj_last_timings", "pj_encode_device", "pj_encode_size_device", "pj_encode_host",
           "pj_decode_device", "pj_decode_host", "pj_decode_bounds", "pj_encode_device_noalloc",
           "pj_decode_array_device", "pj_decode_array_host", "pj_encode_bound", "pj_host_alloc", "pj_host_free"]
NOALLOC_SCRATCH_WORDS = 1 << 20


def noalloc_max_records(nested: bool) -> int:
    """Largest n_pets pj_encode_device_noalloc accepts (PJ_NOALLOC_MAX_RECORDS)."""
    return (NOALLOC_SCRATCH_WORDS - 132) * (96 if nested else 256)


def lib_path() -> str:
    """The in-tree library, or the file named by $PETJSON_LIB."""
    return os.environ.get("PETJSON_LIB") or os.path.join(PKG_DIR, "libpetjson.so")


def load_lib():
    """Load libpetjson.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not os.path.exists(p):
            raise FileNotFoundError(f"{p} missing: run __graft_entry__.build() (no CPU fallback exists)")
        # torch bundles its own HIP runtime under the same soname as
        # /opt/rocm's; whichever loads first is the one both use, and torch
        # only finds the GPU through its own.  So torch is loaded first.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(p)
        vp, u64, i32 = C.c_void_p, C.c_uint64, C.c_int
        L.pj_create.restype = vp
        L.pj_create.argtypes = [i32, C.POINTER(i32)]
        L.pj_destroy.argtypes = [vp]
        L.pj_default_options.argtypes = [C.POINTER(Options)]
        L.pj_set_options.argtypes = [vp, C.POINTER(Options)]
        L.pj_set_options.restype = i32
        L.pj_last_error.restype = C.c_char_p
        L.pj_last_timings.argtypes = [vp, C.POINTER(C.c_float), i32]
        L.pj_last_timings.restype = i32
        for f in ("pj_encode_device", "pj_encode_host", "pj_encode_device_noalloc"):
            getattr(L, f).argtypes = [vp, C.POINTER(PetColumnsStruct), i32, vp, u64, C.POINTER(u64)]
            getattr(L, f).restype = i32
        L.pj_encode_bound.argtypes = [C.POINTER(PetColumnsStruct), i32, C.POINTER(u64)]
        L.pj_encode_bound.restype = i32
        L.pj_encode_size_device.argtypes = [vp, C.POINTER(PetColumnsStruct), i32, C.POINTER(u64)]
        L.pj_encode_size_device.restype = i32
        for f in ("pj_decode_device", "pj_decode_host", "pj_decode_array_device", "pj_decode_array_host"):
            getattr(L, f).argtypes = [vp, vp, u64, C.POINTER(PetColumnsStruct), vp, vp, u64,
                                      C.POINTER(DecodeResult)]
            getattr(L, f).restype = i32
        L.pj_decode_bounds.argtypes = [u64, C.POINTER(PetColumnsStruct)]
        L.pj_host_alloc.argtypes = [u64]
        L.pj_host_alloc.restype = vp
        L.pj_host_free.argtypes = [vp]
        L.pj_encode_by_status_device.argtypes = [vp, C.POINTER(PetColumnsStruct), C.c_uint32, i32, vp, u64,
                                                 C.POINTER(u64), C.POINTER(u64)]
        L.pj_encode_by_status_device.restype = i32
        L.pj_encode_by_status_host.argtypes = L.pj_encode_by_status_device.argtypes
        L.pj_encode_by_status_host.restype = i32
        L.pj_encode_model_host.argtypes = [vp, i32, C.POINTER(ModelColumnsStruct), i32, vp, u64, C.POINTER(u64)]
        L.pj_encode_model_host.restype = i32
        L.pj_decode_model_host.argtypes = [vp, i32, vp, u64, i32, C.POINTER(ModelColumnsStruct), vp, vp, u64,
                                           C.POINTER(DecodeResult)]
        L.pj_decode_model_host.restype = i32
        L.pj_encode_model_device.argtypes = [vp, i32, C.POINTER(ModelColumnsStruct), i32, vp, u64, C.POINTER(u64)]
        L.pj_encode_model_device.restype = i32
        L.pj_decode_model_device.argtypes = [vp, i32, vp, u64, i32, C.POINTER(ModelColumnsStruct), vp, vp, u64,
                                             C.POINTER(DecodeResult)]
        L.pj_decode_model_device.restype = i32
        L.pj_decode_model_bounds.argtypes = [i32, u64, C.POINTER(ModelColumnsStruct)]
        _LIB = L
    return _LIB


def host_array(n: int, dtype) -> np.ndarray:
    """A numpy array of n elements in pinned host memory (pj_host_alloc),
    freed when the array is collected: inputs and outputs of the *_host
    entry points placed in it move by DMA with no bounce copy."""
    L = load_lib()
    nbytes = max(1, int(n) * np.dtype(dtype).itemsize)
    p = L.pj_host_alloc(nbytes)
    if not p:
        raise MemoryError(f"pj_host_alloc({nbytes}) failed")
    buf = (C.c_uint8 * nbytes).from_address(p)
    arr = np.frombuffer(buf, dtype=np.uint8, count=nbytes).view(dtype)[: int(n)]
    import weakref
    weakref.finalize(buf, L.pj_host_free, p)
    return arr


def load_gen():
    global _GEN
    if _GEN is None:
        p = os.path.join(PKG_DIR, "libpjgen.so")
        if not os.path.exists(p):
            raise FileNotFoundError(f"{p} missing: run __graft_entry__.build()")
        G = C.CDLL(p)
        G.pjg_generate.argtypes = [C.c_int, C.c_uint64, C.c_uint64, C.c_int, C.POINTER(PetColumnsStruct)]
        G.pjg_generate.restype = C.c_int
        G.pjg_free.argtypes = [C.POINTER(PetColumnsStruct)]
        G.pjg_corrupt_ndjson.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_double, C.c_void_p,
                                         C.c_void_p, C.c_uint64]
        G.pjg_corrupt_ndjson.restype = C.c_uint64
        _GEN = G
    return _GEN


# ------------------------------------------------------------------- columns
def _ptr(a) -> Optional[int]:
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        return a.ctypes.data
    return a.data_ptr()  # torch tensor


def _len(a) -> int:
    return 0 if a is None else (a.shape[0] if isinstance(a, np.ndarray) else a.numel())


@dataclass
class Columns:
    """SoA Pet columns (numpy on the host or torch tensors on a GPU).  A
    missing group is None, with the meaning given in include/petjson.h."""
    n_pets: int
    arrays: Dict[str, object] = field(default_factory=dict)
    caps: Dict[str, int] = field(default_factory=dict)
    # logical lengths of device arrays that carry tail padding
    lengths: Dict[str, int] = field(default_factory=dict)

    def __getitem__(self, k):
        v = self.arrays.get(k)
        if v is not None and k in self.lengths:
            v = v[: self.lengths[k]]
        return v

    def struct(self) -> PetColumnsStruct:
        s = PetColumnsStruct()
        s.n_pets = self.n_pets
        for n in COLS:
            setattr(s, n, _ptr(self.arrays.get(n)))
        for n in CAPS:
            setattr(s, n, int(self.caps.get(n, 0)))
        return s

    def to_device(self, device="cuda"):
        import torch

        def up(v):
            # never a zero-size allocation (its data pointer would be NULL,
            # which means "column group absent"), plus a few tail bytes
            v = np.ascontiguousarray(v)
            pad = max(1, 8 // v.itemsize)
            buf = torch.empty(v.shape[0] + pad, dtype=torch.from_numpy(v[:0]).dtype, device=device)
            if v.shape[0]:
                buf[: v.shape[0]].copy_(torch.from_numpy(v))
            return buf

        arr, lens = {}, {}
        for k in self.arrays:
            v = self[k]
            arr[k] = up(v) if v is not None else None
            if v is not None:
                lens[k] = v.shape[0]
        return Columns(self.n_pets, arr, dict(self.caps), lens)

    def to_host(self):
        arr = {}
        for k in self.arrays:
            v = self[k]
            arr[k] = v if isinstance(v, np.ndarray) or v is None else v.cpu().numpy()
        return Columns(self.n_pets, arr, dict(self.caps))

    # sizes implied by the offset arrays
    def sizes(self):
        h = self.to_host()
        n = self.n_pets
        get = lambda k, i: int(h.arrays[k][i]) if h.arrays.get(k) is not None else 0
        nu, nt = get("photo_off", n), get("tag_off", n)
        return {"n_pets": n, "name_bytes": get("name_off", n), "cat_name_bytes": get("cat_name_off", n),
                "n_urls": nu, "url_bytes": get("url_off", nu) if nu or h.arrays.get("url_off") is not None else 0,
                "n_tags": nt, "tag_name_bytes": get("tag_name_off", nt) if h.arrays.get("tag_name_off") is not None else 0}

    def input_bytes(self) -> int:
        """Bytes of all columns an encode reads (algorithmic input bytes)."""
        tot = 0
        for k in self.arrays:
            v = self[k]
            if v is None:
                continue
            tot += v.nbytes if isinstance(v, np.ndarray) else v.numel() * v.element_size()
        return tot


def columns_from_struct(s: PetColumnsStruct, copy=True) -> Columns:
    """Copy columns described by a host struct into numpy arrays."""
    n = s.n_pets
    arrays = {}

    def grab(name, count):
        p = getattr(s, name)
        if not p:
            return None
        dt = np.dtype(DTYPES[name])
        if count == 0:
            return np.zeros(0, dtype=dt)
        buf = (C.c_uint8 * (count * dt.itemsize)).from_address(p)
        a = np.frombuffer(buf, dtype=dt, count=count)
        return a.copy() if copy else a

    for k in ("id", "flags", "status", "cat_id", "cat_flags"):
        arrays[k] = grab(k, n)
    for k in ("name_off", "cat_name_off", "photo_off", "tag_off"):
        arrays[k] = grab(k, n + 1)
    arrays["name_bytes"] = grab("name_bytes", int(arrays["name_off"][n]) if arrays["name_off"] is not None else 0)
    arrays["cat_name_bytes"] = grab("cat_name_bytes", int(arrays["cat_name_off"][n]) if arrays["cat_name_off"] is not None else 0)
    nu = int(arrays["photo_off"][n]) if arrays["photo_off"] is not None else 0
    nt = int(arrays["tag_off"][n]) if arrays["tag_off"] is not None else 0
    arrays["url_off"] = grab("url_off", nu + 1)
    arrays["url_bytes"] = grab("url_bytes", int(arrays["url_off"][nu]) if arrays["url_off"] is not None else 0)
    arrays["tag_id"] = grab("tag_id", nt)
    arrays["tag_flags"] = grab("tag_flags", nt)
    arrays["tag_name_off"] = grab("tag_name_off", nt + 1)
    arrays["tag_name_bytes"] = grab("tag_name_bytes", int(arrays["tag_name_off"][nt]) if arrays["tag_name_off"] is not None else 0)
    return Columns(n, arrays)


def generate(config: int, n: int, seed: Optional[int] = None, threads: int = 0) -> Columns:
    """Seeded synthetic records of a benchmark configuration (1..5)."""
    G = load_gen()
    s = PetColumnsStruct()
    if seed is None:
        seed = SEED_BASE + config
    rc = G.pjg_generate(config, n, seed, threads, C.byref(s))
    if rc != 0:
        raise ValueError(f"pjg_generate({config}, {n}) failed")
    try:
        return columns_from_struct(s)
    finally:
        G.pjg_free(C.byref(s))


def corrupt_ndjson(buf: np.ndarray, seed: int, rate: float):
    """Corrupt ~rate of the lines of an NDJSON uint8 array in place; returns
    (line indices, expected codes)."""
    G = load_gen()
    cap = max(16, int(len(buf) // 20 * rate * 4) + 16)
    lines = np.zeros(cap, dtype=np.uint64)
    codes = np.zeros(cap, dtype=np.uint8)
    k = G.pjg_corrupt_ndjson(buf.ctypes.data, len(buf), seed, rate, lines.ctypes.data, codes.ctypes.data, cap)
    if k > cap:
        raise RuntimeError("corruption list overflow")
    return lines[:k].copy(), codes[:k].copy()


def default_err_cap(length: int) -> int:
    """First guess at the error-list capacity for `length` input bytes.  The
    list can hold at most one entry per line (at most `length` lines), but
    sizing for that would cost 9 bytes per input byte; the decode calls
    retry once with the count a PJ_ERR_CAPACITY result reports."""
    return length // 16 + 16


def decode_bounds(length: int) -> Dict[str, int]:
    s = PetColumnsStruct()
    load_lib().pj_decode_bounds(length, C.byref(s))
    return {k: int(getattr(s, k)) for k in CAPS}


# --------------------------------------------------------------------- codec
class Codec:
    """One libpetjson context (one HIP stream on one gfx950 device)."""

    def __init__(self, device: int = 0, inclusion: int = INCLUDE_NON_EMPTY, hex_upper: bool = True):
        self.L = load_lib()
        st = C.c_int(0)
        self.ctx = self.L.pj_create(device, C.byref(st))
        if not self.ctx:
            raise PetJsonError(st.value, self.L.pj_last_error().decode())
        self.device = device
        self.set_options(inclusion, hex_upper)

    def close(self):
        if self.ctx:
            self.L.pj_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != PJ_OK:
            raise PetJsonError(rc, self.L.pj_last_error().decode())

    def set_options(self, inclusion=INCLUDE_NON_EMPTY, hex_upper=True, fields=None):
        o = make_options(inclusion, hex_upper, fields)
        self._check(self.L.pj_set_options(self.ctx, C.byref(o)))

    def timings(self):
        buf = (C.c_float * 16)()
        k = self.L.pj_last_timings(self.ctx, buf, 16)
        return [buf[i] for i in range(k)]

    # ---- encode
    def encode_size(self, cols: Columns, fmt: int = FORMAT_ARRAY) -> int:
        import torch
        torch.cuda.synchronize()
        s = cols.struct()
        n = C.c_uint64(0)
        self._check(self.L.pj_encode_size_device(self.ctx, C.byref(s), fmt, C.byref(n)))
        return n.value

    def encode(self, cols: Columns, fmt: int = FORMAT_ARRAY, out=None, two_pass=False):
        """Encode device columns; returns a uint8 torch tensor (a view of `out`
        when given) holding exactly the JSON bytes.  two_pass: nested records
        are written at the offsets of the measuring pass rather than by the
        single pass (the library reads PETJSON_ENC_TWO_PASS on every call)."""
        import torch
        if out is None:
            need = self.encode_size(cols, fmt)
            out = torch.empty(need + 4, dtype=torch.uint8, device=f"cuda:{self.device}")
        torch.cuda.synchronize()
        s = cols.struct()
        n = C.c_uint64(0)
        cap = out.numel()
        old = os.environ.get("PETJSON_ENC_TWO_PASS")
        if two_pass:
            os.environ["PETJSON_ENC_TWO_PASS"] = "1"
        try:
            self._check(self.L.pj_encode_device(self.ctx, C.byref(s), fmt, C.c_void_p(out.data_ptr()), cap,
                                                C.byref(n)))
        finally:
            if two_pass:
                if old is None:
                    del os.environ["PETJSON_ENC_TWO_PASS"]
                else:
                    os.environ["PETJSON_ENC_TWO_PASS"] = old
        return out[: n.value]

    def encode_noalloc(self, cols: Columns, out, fmt: int = FORMAT_ARRAY):
        """pj_encode_device_noalloc into the caller's device tensor `out`
        (the call itself allocates nothing); returns the view of `out`
        holding the JSON bytes."""
        import torch
        torch.cuda.synchronize()
        s = cols.struct()
        n = C.c_uint64(0)
        self._check(self.L.pj_encode_device_noalloc(self.ctx, C.byref(s), fmt, C.c_void_p(out.data_ptr()),
                                                    out.numel(), C.byref(n)))
        return out[: n.value]

    def encode_host(self, cols: Columns, fmt: int = FORMAT_ARRAY, as_array: bool = False):
        """Encode host columns in one call, into a buffer sized by
        pj_encode_bound.  Returns bytes (or, with as_array, the numpy uint8
        view of the buffer, which saves a copy)."""
        s = cols.struct()
        bound = C.c_uint64(0)
        self._check(self.L.pj_encode_bound(C.byref(s), fmt, C.byref(bound)))
        out = np.empty(max(1, bound.value), dtype=np.uint8)
        n = C.c_uint64(0)
        self._check(self.L.pj_encode_host(self.ctx, C.byref(s), fmt, C.c_void_p(out.ctypes.data), out.size,
                                          C.byref(n)))
        return out[: n.value] if as_array else out[: n.value].tobytes()

    # ---- decode
    def _alloc_decode(self, caps, device):
        import torch
        dev = f"cuda:{self.device}" if device is None else device
        cp, cu, ct = caps["cap_pets"], caps["cap_urls"], caps["cap_tags"]
        sizes = {"id": cp, "flags": cp, "status": cp, "name_off": cp + 1, "name_bytes": caps["cap_name_bytes"],
                 "cat_id": cp, "cat_flags": cp, "cat_name_off": cp + 1, "cat_name_bytes": caps["cap_cat_name_bytes"],
                 "photo_off": cp + 1, "url_off": cu + 1, "url_bytes": caps["cap_url_bytes"], "tag_off": cp + 1,
                 "tag_id": ct, "tag_flags": ct, "tag_name_off": ct + 1, "tag_name_bytes": caps["cap_tag_name_bytes"]}
        tdt = {np.int64: torch.int64, np.uint8: torch.uint8, np.uint64: torch.int64}
        arrays = {k: torch.empty(max(1, v) + 8, dtype=tdt[DTYPES[k]], device=dev) for k, v in sizes.items()}
        return Columns(0, arrays, dict(caps), {k: 0 for k in arrays})

    def decode_buffers(self, caps, err_cap, device=None):
        """Preallocated outputs for decode(..., out=...): (columns, err lines, err codes)."""
        import torch
        cols = self._alloc_decode(caps, device)
        dev = cols.arrays["id"].device
        el = torch.empty(max(1, err_cap), dtype=torch.int64, device=dev)
        ec = torch.empty(max(1, err_cap), dtype=torch.uint8, device=dev)
        return cols, el, ec

    def decode(self, data, caps=None, err_cap=None, device=None, out=None, array=False):
        """Decode NDJSON (or, with array=True, one JSON array document) held in
        a uint8 device tensor.  Returns (columns on the device trimmed to
        size, error line / element indices, error codes, DecodeResult).
        `out` = decode_buffers(...) reuses preallocated outputs.  A broken
        array frame raises PetJsonError(PJ_ERR_SYNTAX)."""
        import torch
        fn = self.L.pj_decode_array_device if array else self.L.pj_decode_device
        n = data.numel()
        own = out is None
        if own:
            caps = caps or decode_bounds(n)
            if err_cap is None:
                err_cap = default_err_cap(n)
            out = self.decode_buffers(caps, err_cap, device)
        cols, el, ec = out
        err_cap = el.numel() if err_cap is None else err_cap
        torch.cuda.synchronize()
        s = cols.struct()
        res = DecodeResult()
        ptr = C.c_void_p(data.data_ptr()) if n else C.c_void_p(el.data_ptr())
        rc = fn(self.ctx, ptr, n, C.byref(s), C.c_void_p(el.data_ptr()), C.c_void_p(ec.data_ptr()), err_cap,
                C.byref(res))
        if rc == PJ_ERR_CAPACITY and own and res.n_errors > err_cap:
            # more invalid lines than the first guess: the call reported how
            # many there are, so one retry with that capacity suffices
            err_cap = int(res.n_errors)
            el = torch.empty(max(1, err_cap), dtype=torch.int64, device=el.device)
            ec = torch.empty(max(1, err_cap), dtype=torch.uint8, device=ec.device)
            s = cols.struct()
            res = DecodeResult()
            rc = fn(self.ctx, ptr, n, C.byref(s), C.c_void_p(el.data_ptr()), C.c_void_p(ec.data_ptr()), err_cap,
                    C.byref(res))
        self._check(rc)
        return self._trim(cols, res), el[: res.n_errors], ec[: res.n_errors], res

    @staticmethod
    def _trim(cols, res):
        np_, nu, nt = res.n_pets, res.n_urls, res.n_tags
        lens = {"id": np_, "flags": np_, "status": np_, "name_off": np_ + 1, "name_bytes": res.name_bytes,
                "cat_id": np_, "cat_flags": np_, "cat_name_off": np_ + 1, "cat_name_bytes": res.cat_name_bytes,
                "photo_off": np_ + 1, "url_off": nu + 1, "url_bytes": res.url_bytes, "tag_off": np_ + 1,
                "tag_id": nt, "tag_flags": nt, "tag_name_off": nt + 1, "tag_name_bytes": res.tag_name_bytes}
        return Columns(np_, cols.arrays, dict(cols.caps), lens)

    def decode_array(self, data, caps=None, err_cap=None, device=None, out=None):
        """decode(..., array=True): one JSON array document on the device."""
        return self.decode(data, caps, err_cap, device, out, array=True)

    def decode_array_host(self, data: bytes, caps=None, err_cap=None):
        """decode_host(..., array=True): one JSON array document from host bytes."""
        return self.decode_host(data, caps, err_cap, array=True)

    def decode_host(self, data: bytes, caps=None, err_cap=None, array=False):
        """Decode NDJSON bytes (or one array document) through the host entry
        point; numpy results."""
        fn = self.L.pj_decode_array_host if array else self.L.pj_decode_host
        n = len(data)
        caps = caps or decode_bounds(n)
        cp, cu, ct = caps["cap_pets"], caps["cap_urls"], caps["cap_tags"]
        sizes = {"id": cp, "flags": cp, "status": cp, "name_off": cp + 1, "name_bytes": caps["cap_name_bytes"],
                 "cat_id": cp, "cat_flags": cp, "cat_name_off": cp + 1, "cat_name_bytes": caps["cap_cat_name_bytes"],
                 "photo_off": cp + 1, "url_off": cu + 1, "url_bytes": caps["cap_url_bytes"], "tag_off": cp + 1,
                 "tag_id": ct, "tag_flags": ct, "tag_name_off": ct + 1, "tag_name_bytes": caps["cap_tag_name_bytes"]}
        arrays = {k: np.zeros(max(1, v), dtype=DTYPES[k]) for k, v in sizes.items()}
        cols = Columns(0, arrays, dict(caps))
        guessed = err_cap is None
        if guessed:
            err_cap = default_err_cap(n)
        buf = np.frombuffer(data, np.uint8) if n else np.zeros(1, np.uint8)
        for _ in range(2):
            el = np.zeros(max(1, err_cap), np.uint64)
            ec = np.zeros(max(1, err_cap), np.uint8)
            s = cols.struct()
            res = DecodeResult()
            rc = fn(self.ctx, C.c_void_p(buf.ctypes.data), n, C.byref(s), C.c_void_p(el.ctypes.data),
                    C.c_void_p(ec.ctypes.data), err_cap, C.byref(res))
            if not (rc == PJ_ERR_CAPACITY and guessed and res.n_errors > err_cap):
                break
            err_cap = int(res.n_errors)     # one retry with the count the call reported
        self._check(rc)
        t = self._trim(cols, res).to_host()
        return t, el[: res.n_errors].copy(), ec[: res.n_errors].copy(), res


# ------------------------------------------------------ Order / User columns
@dataclass
class ModelColumns:
    """SoA columns of Order or User records (numpy on the host or torch
    tensors on a GPU): per property k, col[k] holds the values (string
    properties: n + 1 offsets into bytes[k]); bit k of present[i] marks
    property k of record i non-null (present None: all non-null)."""
    model: int
    n: int
    present: object = None
    col: list = field(default_factory=list)
    bytes: list = field(default_factory=list)
    cap_n: int = 0
    cap_bytes: list = field(default_factory=lambda: [0] * MODEL_MAX_PROPS)
    n_bytes: list = field(default_factory=lambda: [0] * MODEL_MAX_PROPS)

    @property
    def props(self):
        return MODEL_PROPS[self.model]

    def struct(self) -> ModelColumnsStruct:
        s = ModelColumnsStruct()
        s.n = self.n
        s.present = _ptr(self.present)
        for k in range(len(self.props)):
            s.col[k] = _ptr(self.col[k])
            s.bytes[k] = _ptr(self.bytes[k]) if k < len(self.bytes) else None
        s.cap_n = self.cap_n
        for k in range(MODEL_MAX_PROPS):
            s.cap_bytes[k] = int(self.cap_bytes[k])
        return s

    def to_device(self, device="cuda"):
        import torch

        def up(v):
            if v is None:
                return None
            v = np.ascontiguousarray(v)
            buf = torch.empty(v.shape[0] + max(1, 8 // v.itemsize), dtype=torch.from_numpy(v[:0]).dtype,
                              device=device)
            if v.shape[0]:
                buf[: v.shape[0]].copy_(torch.from_numpy(v))
            return buf

        return ModelColumns(self.model, self.n, up(self.present), [up(c) for c in self.col],
                            [up(b) for b in self.bytes], self.cap_n, list(self.cap_bytes), list(self.n_bytes))

    def to_host(self):
        """numpy copies trimmed to the record count and string sizes."""
        def dn(v, count):
            if v is None:
                return None
            v = v if isinstance(v, np.ndarray) else v.cpu().numpy()
            return v[:count].copy()
        col, byt = [], []
        for k, (_, kind) in enumerate(self.props):
            c = dn(self.col[k], self.n + 1 if kind == "str" else self.n)
            col.append(c)
            byt.append(dn(self.bytes[k], int(c[self.n])) if kind == "str" and self.bytes[k] is not None else None)
        return ModelColumns(self.model, self.n, dn(self.present, self.n), col, byt)


def _rand_text(rng, n, lo, hi, fancy):
    """Offsets and bytes of n strings of lo..hi bytes: ASCII word bytes,
    and (fancy) one record in 20 with escapes and multi-byte UTF-8."""
    pool = np.frombuffer(b"abz09-_.@ ", np.uint8)
    lens = rng.integers(lo, hi + 1, n).astype(np.int64)
    odd = [b'"', b"\\", b"\n", b"\x01", b"\x1f", b"\xc3\xa9", b"\xe2\x82\xac", b"\xf0\x9f\x98\x80", b"/"]
    special = {}
    if fancy:
        for i in np.nonzero(rng.random(n) < 0.05)[0]:
            b = bytearray()
            while len(b) < lens[i]:
                b += odd[int(rng.integers(len(odd)))] if rng.random() < 0.3 else bytes([pool[int(rng.integers(10))]])
            special[int(i)] = bytes(b)
            lens[i] = len(b)
    off = np.zeros(n + 1, np.uint64)
    off[1:] = np.cumsum(lens, dtype=np.uint64)
    data = pool[rng.integers(0, pool.size, int(off[-1]))]
    for i, b in special.items():
        data[int(off[i]): int(off[i + 1])] = np.frombuffer(b, np.uint8)
    return off, data


def generate_model(model: int, n: int, seed: int = 0, null_rate: float = 0.1, fancy: bool = True) -> ModelColumns:
    """Seeded random Order or User records (host columns): extreme and
    ordinary integers, every enum value, strings with escapes and UTF-8,
    nulls and empty strings."""
    rng = np.random.default_rng(seed)
    props = MODEL_PROPS[model]
    present = np.zeros(n, np.uint8)
    col, byt = [], []
    for k, (name, kind) in enumerate(props):
        present |= ((rng.random(n) >= null_rate).astype(np.uint8) << k)
        if kind == "i64":
            v = rng.integers(-2**63, 2**63 - 1, n, dtype=np.int64, endpoint=True)
            small = rng.random(n) < 0.5
            v[small] = rng.integers(-1000, 10**6, int(small.sum()))
            v[:4] = [0, -1, -2**63, 2**63 - 1][: min(4, n)]
            col.append(v); byt.append(None)
        elif kind == "i32":
            v = rng.integers(-2**31, 2**31 - 1, n, dtype=np.int64, endpoint=True).astype(np.int32)
            small = rng.random(n) < 0.5
            v[small] = rng.integers(0, 100, int(small.sum()))
            v[:3] = [-2**31, 2**31 - 1, 0][: min(3, n)]
            col.append(v); byt.append(None)
        elif kind in ("enum", "bool"):
            col.append(rng.integers(0, 3 if kind == "enum" else 2, n).astype(np.uint8)); byt.append(None)
        else:
            if name == "shipDate":
                y = rng.integers(1970, 2100, n); mo = rng.integers(1, 13, n); d = rng.integers(1, 29, n)
                hh = rng.integers(0, 24, n); mm = rng.integers(0, 60, n); ms = rng.integers(0, 1000, n)
                empty = rng.random(n) < 0.05
                strs = [b"" if empty[i] else
                        b"%04d-%02d-%02dT%02d:%02d:%02d.%03dZ" % (y[i], mo[i], d[i], hh[i], mm[i], mm[i], ms[i])
                        for i in range(n)]
                off = np.zeros(n + 1, np.uint64)
                off[1:] = np.cumsum([len(x) for x in strs], dtype=np.uint64)
                data = np.frombuffer(b"".join(strs), np.uint8).copy() if off[-1] else np.zeros(0, np.uint8)
            else:
                off, data = _rand_text(rng, n, 0, 24, fancy)
            col.append(off)
            byt.append(data)
    return ModelColumns(model, n, present, col, byt)


def decode_model_bounds(model: int, length: int):
    """(cap_n, cap_bytes) that always suffice for `length` input bytes."""
    L = load_lib()
    s = ModelColumnsStruct()
    L.pj_decode_model_bounds(model, length, C.byref(s))
    return int(s.cap_n), [int(s.cap_bytes[k]) for k in range(MODEL_MAX_PROPS)]


def alloc_model_columns(model: int, cap_n: int, cap_bytes, device=None) -> ModelColumns:
    """Empty decode outputs (numpy, or torch on `device`)."""
    def mk(count, dt):
        if device is None:
            return np.zeros(count, dt)
        import torch
        return torch.zeros(count, dtype=torch.from_numpy(np.zeros(0, dt)).dtype, device=device)
    col, byt = [], []
    for k, (_, kind) in enumerate(MODEL_PROPS[model]):
        col.append(mk(cap_n + 1 if kind == "str" else max(cap_n, 1), KIND_DTYPE[kind]))
        byt.append(mk(max(int(cap_bytes[k]), 1), np.uint8) if kind == "str" else None)
    return ModelColumns(model, 0, mk(max(cap_n, 1), np.uint8), col, byt, cap_n, list(cap_bytes))


def _model_encode(self, cols: ModelColumns, fmt: int = FORMAT_ARRAY, out=None):
    """writeValueAsBytes(List<Order|User>) of device columns: a uint8 torch
    tensor holding exactly the JSON bytes (a view of `out` when given)."""
    import torch
    torch.cuda.synchronize()
    s = cols.struct()
    n = C.c_uint64(0)
    if out is None:
        rc = self.L.pj_encode_model_device(self.ctx, cols.model, C.byref(s), fmt, None, 0, C.byref(n))
        if rc not in (PJ_OK, PJ_ERR_CAPACITY):
            self._check(rc)
        out = torch.empty(n.value + 4, dtype=torch.uint8, device=f"cuda:{self.device}")
    self._check(self.L.pj_encode_model_device(self.ctx, cols.model, C.byref(s), fmt, C.c_void_p(out.data_ptr()),
                                              out.numel(), C.byref(n)))
    return out[: n.value]


def _model_decode(self, model: int, data, array: bool = False, caps=None, err_cap=None):
    """readValue of NDJSON (or one array document) of Orders / Users held in
    a uint8 device tensor.  Returns (device columns, error indices, error
    codes, DecodeResult)."""
    import torch
    n = data.numel()
    cap_n, cap_bytes = caps or decode_model_bounds(model, n)
    dev = f"cuda:{self.device}"
    cols = alloc_model_columns(model, cap_n, cap_bytes, device=dev)
    if err_cap is None:
        err_cap = n + 1
    el = torch.zeros(max(err_cap, 1), dtype=torch.int64, device=dev)
    ec = torch.zeros(max(err_cap, 1), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    s = cols.struct()
    res = DecodeResult()
    self._check(self.L.pj_decode_model_device(self.ctx, model, C.c_void_p(data.data_ptr()), n, int(array),
                                              C.byref(s), C.c_void_p(el.data_ptr()), C.c_void_p(ec.data_ptr()),
                                              err_cap, C.byref(res)))
    cols.n = int(s.n)
    cols.n_bytes = [int(s.n_bytes[k]) for k in range(MODEL_MAX_PROPS)]
    ne = int(res.n_errors)
    return cols, el[:ne], ec[:ne], res


def _encode_by_status(self, cols: Columns, mask: int, fmt: int = FORMAT_ARRAY, out=None):
    """findPetsByStatus body: the records of device columns whose status is in
    mask (bit s: status s, bit 3: none).  Returns (uint8 tensor, count)."""
    import torch
    torch.cuda.synchronize()
    s = cols.struct()
    n, m = C.c_uint64(0), C.c_uint64(0)
    if out is None:
        rc = self.L.pj_encode_by_status_device(self.ctx, C.byref(s), mask, fmt, None, 0, C.byref(n), C.byref(m))
        if rc not in (PJ_OK, PJ_ERR_CAPACITY):
            self._check(rc)
        out = torch.empty(n.value + 4, dtype=torch.uint8, device=f"cuda:{self.device}")
    self._check(self.L.pj_encode_by_status_device(self.ctx, C.byref(s), mask, fmt, C.c_void_p(out.data_ptr()),
                                                  out.numel(), C.byref(n), C.byref(m)))
    return out[: n.value], m.value


def _encode_by_status_host(self, cols: Columns, mask: int, fmt: int = FORMAT_ARRAY):
    """pj_encode_by_status_host: host columns in, (bytes, count) out."""
    s = cols.struct()
    n, m = C.c_uint64(0), C.c_uint64(0)
    rc = self.L.pj_encode_by_status_host(self.ctx, C.byref(s), mask, fmt, None, 0, C.byref(n), C.byref(m))
    if rc not in (PJ_OK, PJ_ERR_CAPACITY):
        self._check(rc)
    out = np.empty(max(1, n.value), np.uint8)
    self._check(self.L.pj_encode_by_status_host(self.ctx, C.byref(s), mask, fmt, C.c_void_p(out.ctypes.data),
                                                out.size, C.byref(n), C.byref(m)))
    return out[: n.value].tobytes(), m.value


def _model_encode_host(self, cols: ModelColumns, fmt: int = FORMAT_ARRAY) -> bytes:
    """pj_encode_model_host: host columns in, the JSON bytes out."""
    s = cols.struct()
    n = C.c_uint64(0)
    rc = self.L.pj_encode_model_host(self.ctx, cols.model, C.byref(s), fmt, None, 0, C.byref(n))
    if rc not in (PJ_OK, PJ_ERR_CAPACITY):
        self._check(rc)
    out = np.empty(max(1, n.value), np.uint8)
    self._check(self.L.pj_encode_model_host(self.ctx, cols.model, C.byref(s), fmt, C.c_void_p(out.ctypes.data),
                                            out.size, C.byref(n)))
    return out[: n.value].tobytes()


def _model_decode_host(self, model: int, data: bytes, array: bool = False, caps=None, err_cap=None):
    """pj_decode_model_host: bytes in, (host columns, error indices, error
    codes, DecodeResult) out."""
    n = len(data)
    cap_n, cap_bytes = caps or decode_model_bounds(model, n)
    cols = alloc_model_columns(model, cap_n, cap_bytes)
    if err_cap is None:
        err_cap = n + 1
    el = np.zeros(max(err_cap, 1), np.uint64)
    ec = np.zeros(max(err_cap, 1), np.uint8)
    buf = np.frombuffer(data, np.uint8) if n else np.zeros(1, np.uint8)
    s = cols.struct()
    res = DecodeResult()
    self._check(self.L.pj_decode_model_host(self.ctx, model, C.c_void_p(buf.ctypes.data), n, int(array), C.byref(s),
                                            C.c_void_p(el.ctypes.data), C.c_void_p(ec.ctypes.data), err_cap,
                                            C.byref(res)))
    cols.n = int(s.n)
    cols.n_bytes = [int(s.n_bytes[k]) for k in range(MODEL_MAX_PROPS)]
    ne = int(res.n_errors)
    return cols.to_host(), el[:ne].copy(), ec[:ne].copy(), res


Codec.encode_by_status = _encode_by_status
Codec.encode_by_status_host = _encode_by_status_host
Codec.encode_model_host = _model_encode_host
Codec.decode_model_host = _model_decode_host
Codec.encode_model = _model_encode
Codec.decode_model = _model_decode
