"""The host entry points copy through two pinned bounce buffers, chunk by
chunk, overlapping the host copies with the DMA.  With small odd chunk sizes
(PETJSON_XFER_CHUNK, read when a context first copies) every copy crosses
many chunk boundaries: pj_encode_host's output equals pj_encode_device's,
and pj_decode_host's / pj_decode_array_host's columns equal the device
decode's, byte for byte, on records of every configuration."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

SCRIPT = r"""
import sys
import numpy as np, torch
import petjson as pj
codec = pj.Codec(0)
for cfg, n in ((1, 20000), (3, 30000), (5, 3000)):
    cols = pj.generate(cfg, n)
    dev = cols.to_device()
    for fmt in (pj.FORMAT_ARRAY, pj.FORMAT_NDJSON):
        want = codec.encode(dev, fmt).cpu().numpy().tobytes()
        got = codec.encode_host(cols, fmt)
        assert got == want, (cfg, fmt, len(got), len(want))
        d = torch.from_numpy(np.frombuffer(want, np.uint8).copy()).cuda()
        ref = codec.decode(d, array=fmt == pj.FORMAT_ARRAY)[0].to_host()
        host = (codec.decode_array_host if fmt == pj.FORMAT_ARRAY else codec.decode_host)(want)[0]
        for k in pj.COLS:
            assert np.array_equal(host[k], ref[k]), (cfg, fmt, k)
codec.close()
print("host pipeline ok")
"""


@pytest.mark.parametrize("chunk", [4099, 65537, 1 << 20])
def test_host_entry_points_across_chunks(chunk):
    env = dict(os.environ, PETJSON_XFER_CHUNK=str(chunk),
               PYTHONPATH=os.pathsep.join([os.path.join(ROOT, "micronaut3-bug_amd"), os.path.join(ROOT, "tests")]))
    r = subprocess.run([sys.executable, "-c", SCRIPT], capture_output=True, text=True, env=env, timeout=240)
    assert r.returncode == 0 and "host pipeline ok" in r.stdout, r.stdout[-2000:] + r.stderr[-3000:]
