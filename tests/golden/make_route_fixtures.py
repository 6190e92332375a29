"""Extract the reference's recorded router traces into compact fixtures.

Reads notes/route-trace.json, notes/route-trace-512.json and
notes/route-trace-direct.json from the reference checkout (written by
bin/offload.py:716-808, records {"phase", "layer", "ids"}), and the per-layer
expert censuses notes/census-*.json, and writes tests/golden/route_traces.npz:

  <name>_decode_layer  int16 [N]      layer of each decode record, in order
  <name>_decode_ids    int16 [N, 8]   the 8 expert ids of that record
  trace_prefill_layer  int16 [P]      layer of each prefill record of route-trace.json
  trace_prefill_rows   int32 [P]      rows of each prefill record
  trace_prefill_ids    int16 [sum rows, 8]  all prefill ids, records concatenated

These are data the reference's own notes hold (real routing of the Drama 3
model); no reference code is copied or run.  Run from the repo root:

    python tests/golden/make_route_fixtures.py /root/reference
"""
import json
import sys
from pathlib import Path

import numpy as np

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
out = {}
for name, fn in (("trace", "route-trace.json"), ("t512", "route-trace-512.json"),
                 ("direct", "route-trace-direct.json")):
    recs = json.loads((ref / "notes" / fn).read_text())["records"]
    dec = [r for r in recs if r["phase"] == "decode"]
    out[f"{name}_decode_layer"] = np.array([r["layer"] for r in dec], np.int16)
    out[f"{name}_decode_ids"] = np.array([r["ids"][0] for r in dec], np.int16)
    if name == "trace":
        pre = [r for r in recs if r["phase"] == "prefill"]
        out["trace_prefill_layer"] = np.array([r["layer"] for r in pre], np.int16)
        out["trace_prefill_rows"] = np.array([len(r["ids"]) for r in pre], np.int32)
        out["trace_prefill_ids"] = np.concatenate([np.array(r["ids"], np.int16) for r in pre])
dest = Path(__file__).resolve().parent / "route_traces.npz"
np.savez_compressed(dest, **out)
for k, v in out.items():
    print(k, v.shape, v.dtype)
print(dest, dest.stat().st_size, "bytes")
