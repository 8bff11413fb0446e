"""Hypothesis-generated records through the GPU codec: encode equals the CPU
restatement byte for byte in every framing and inclusion mode, and the GPU
decode of that text gives the restatement's columns."""
import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import oracle_py as orc
import petjson as pj
from model import to_columns
from test_oracle_properties import PETS

pytestmark = pytest.mark.gpu
SETTINGS = settings(max_examples=60, deadline=None, derandomize=True,
                    suppress_health_check=[HealthCheck.too_slow, HealthCheck.function_scoped_fixture])


@SETTINGS
@given(PETS, st.sampled_from([pj.INCLUDE_NON_EMPTY, pj.INCLUDE_NON_NULL, pj.INCLUDE_ALWAYS]))
def test_gpu_encode_decode_match_oracle(codec, pets, incl):
    cols = to_columns(pets)
    dev = cols.to_device()
    codec.set_options(incl)
    try:
        for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON, pj.FORMAT_PRETTY):
            want = orc.encode(cols, fmt, incl)
            assert codec.encode(dev, fmt).cpu().numpy().tobytes() == want, fmt
    finally:
        codec.set_options()
    text = orc.encode(cols, pj.FORMAT_NDJSON, incl)
    if not text:
        return
    data = torch.from_numpy(np.frombuffer(text, np.uint8).copy()).cuda()
    g, gel, gec, gres = codec.decode(data)
    r, rel, rec, rres = orc.decode(text)
    assert (gres.n_pets, gres.n_errors) == (rres.n_pets, rres.n_errors)
    g = g.to_host()
    for k in pj.COLS:
        if r[k] is not None:
            assert np.array_equal(g[k], r[k]), k
