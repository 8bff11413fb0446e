"""pj_encode_device_noalloc (encode with the per-GPU fixed scratch array,
no allocation inside the call) gives byte-identical output to
pj_encode_device, on two calls in a row with the second input smaller, and
rejects inputs beyond the fixed scratch with a clear error."""
import ctypes as C

import pytest
import torch

import petjson as pj

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("config,fmt", [(3, pj.FORMAT_ARRAY), (3, pj.FORMAT_NDJSON), (2, pj.FORMAT_ARRAY),
                                        (5, pj.FORMAT_NDJSON), (3, pj.FORMAT_PRETTY)])
def test_noalloc_matches_encode_device_twice(config, fmt):
    codec = pj.Codec(0)
    try:
        for n in (60_000, 7_000):            # the second call is smaller
            cols = pj.generate(config, n).to_device()
            ref = codec.encode(cols, fmt).cpu().numpy().tobytes()
            out = torch.full((len(ref) + 64,), 0xEE, dtype=torch.uint8, device="cuda")
            got = codec.encode_noalloc(cols, out, fmt).cpu().numpy().tobytes()
            assert got == ref, (config, fmt, n)
            assert (out[len(ref):].cpu() == 0xEE).all()
    finally:
        codec.close()


def test_noalloc_capacity_and_size_limit():
    codec = pj.Codec(0)
    try:
        cols = pj.generate(3, 1000).to_device()
        need = codec.encode_size(cols, pj.FORMAT_ARRAY)
        out = torch.empty(need // 2, dtype=torch.uint8, device="cuda")
        with pytest.raises(pj.PetJsonError) as ei:
            codec.encode_noalloc(cols, out)
        assert ei.value.status == pj.PJ_ERR_CAPACITY
        # more records than the fixed scratch holds: rejected before any launch
        s = cols.struct()
        s.n_pets = pj.noalloc_max_records(True) + 1
        n = C.c_uint64(0)
        rc = codec.L.pj_encode_device_noalloc(codec.ctx, C.byref(s), pj.FORMAT_ARRAY, C.c_void_p(out.data_ptr()),
                                              out.numel(), C.byref(n))
        assert rc == pj.PJ_ERR_INVALID_ARG
        assert b"fixed scratch" in codec.L.pj_last_error()
        # still usable afterwards
        full = torch.empty(need + 8, dtype=torch.uint8, device="cuda")
        assert codec.encode_noalloc(cols, full).numel() == need
    finally:
        codec.close()
