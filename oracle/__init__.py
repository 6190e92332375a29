"""CPU oracle for the expert-offload MoE path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (the package directory and
its HIP library) imports this. The only permitted callers are `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`, and they
use it as the checker, never as the thing being measured or shipped.

Each module restates one part of the reference's algorithm in numpy (or, for
small sequential cases, plain Python loops) and cites the reference file:line
it follows. Modules:

  fp8        OCP e4m3fn codec, 128x128 weight block quantisation, per-token
             per-128 activation quantisation
  moe        the expert FFN in two numerics: W8A8 (dynamic activation quant,
             the GPU kernel's contract) and W8A16 (dequantise + matmul, the
             reference's CPU path)
  router     linear -> softmax -> top-k -> renormalise
  slots      device LRU slot table, the host-side OrderedDict LRU, the offline
             LRU/LFU/static simulator
  permute    torch.unique-style id remap and the token->expert stable sort
  fetch      the self-identifying host pool pattern
  cpu_moe    the timed CPU baseline (torch on host cores)

Where a function's parity rests only on this restatement (no golden vector,
closed form or brute-force cross-check pins it), its docstring says
"parity unpinned".
"""
