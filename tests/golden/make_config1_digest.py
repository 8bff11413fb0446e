"""Writes config1_digest.json: SHA-256 and size of the CPU checker's output
for BASELINE configs[0] (100k Pets from the seeded generator) in each framing.
Run from the repo root after __graft_entry__.build()."""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "micronaut3-bug_amd"), os.path.join(ROOT, "tests")]
import oracle_py as orc  # noqa: E402
import petjson as pj  # noqa: E402

cols = pj.generate(1, 100_000)
digests = {}
for name, fmt in (("array", pj.FORMAT_ARRAY), ("ndjson", pj.FORMAT_NDJSON), ("pretty", pj.FORMAT_PRETTY)):
    b = orc.encode(cols, fmt)
    digests[name] = {"bytes": len(b), "sha256": hashlib.sha256(b).hexdigest()}
doc = {"_about": ("BASELINE configs[0] (CPU plumbing): 100k Pets from the seeded generator (seed 0x5EED0001), "
                  "encoded by the CPU checker in each framing under the default options. A regression pin of the "
                  "generator and the checker together (written by tests/golden/make_config1_digest.py); the GPU "
                  "output must hash the same."), "records": 100000, "digests": digests}
with open(os.path.join(HERE, "config1_digest.json"), "w") as f:
    json.dump(doc, f, indent=1)
    f.write("\n")
