"""MI355X (gfx950) expert-offload MoE path for Drama 3: drop-in for the
reference's bin/offload.py and bin/devcache.py hook surface.

The modules are imported by their plain names, exactly as the reference's
`bin/` modules are (`import devcache`, `import offload`): put this directory
on sys.path, or import this package, which does that and re-exports them.

  hipfetch  loader of libmoeoffload.so (the HIP kernels), cppfetch's contract
  fp8_moe   fp8_moe_forward, the W8A8 block-FP8 expert FFN
  moe       MoEExperts / SparseMoE / route / select_fp8
  devcache  device-resident slot table + zero-copy fetch (decode path)
  offload   host pool, gather/LRU dispatch hooks, router trace and census
  hostpool  one packed page-locked pool of expert records per set of layers
  decode    the 40-layer decode step captured in one hipGraph
  synth     seeded Drama-3-shaped synthetic inputs
"""
import os as _os
import sys as _sys

_HERE = _os.path.dirname(_os.path.abspath(__file__))
if _HERE not in _sys.path:
    _sys.path.insert(0, _HERE)

import hipfetch  # noqa: E402,F401
import fp8_moe  # noqa: E402,F401
import moe  # noqa: E402,F401
import devcache  # noqa: E402,F401
import offload  # noqa: E402,F401
import synth  # noqa: E402,F401
