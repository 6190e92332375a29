"""Writes tests/golden/drama3_mlp_headers.json.gz: the MoE-block entries
(routed experts, router gate, shared expert and its gate) of layers 0 and 39
from the reference's recorded safetensors headers
(notes/drama3-safetensors-headers.json.gz, data only), with the shard each
entry lives in and the shard's header length.

    python tests/golden/make_header_fixture.py /root/reference
"""
import gzip
import json
import sys
from pathlib import Path

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
headers = json.load(gzip.open(ref / "notes" / "drama3-safetensors-headers.json.gz"))
keep = {}
for shard, hdr in headers.items():
    for name, meta in hdr.items():
        if name == "__metadata__":
            continue
        if ".layers.0.mlp." in name or ".layers.39.mlp." in name:
            keep[name] = {"shard": shard, **meta}
out = Path(__file__).resolve().parent / "drama3_mlp_headers.json.gz"
with gzip.open(out, "wt") as f:
    json.dump({"entries": keep, "n_shards": len(headers)}, f, sort_keys=True)
print(f"{len(keep)} entries -> {out} ({out.stat().st_size} bytes)")
